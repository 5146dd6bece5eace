// Autograd.hpp -- grad mode, saved tensors and the backward nodes of the GEMM family.
//
// GradMode / NoGradGuard / SavedTensor / AutogradNode follow the reference
// (include/Autograd.hpp:1-60).  The nodes:
//   MatmulBackward    dA = dC·Bᵀ, dB = Aᵀ·dC through transpose views
//                     (reference include/Autograd.hpp:117-147); on the GPU a
//                     gradient that already exists is accumulated by the GEMM
//                     epilogue (beta = 1) instead of a separate add_.
//   BmmBackward       the same per batch entry (the reference's bmm attaches
//                     MatmulBackward, which cannot handle 3-D tensors).
//   LinearBackward    dX = dY·W, dW = dYᵀ·X, db = Σ_rows dY for F::linear
//                     (W [out,in]) and for Linear's W_ref [in,out] layout.
//   AddBackward       broadcast add: unbroadcast of the gradient
//                     (reference include/Autograd.hpp:55-82).
//   Conv2DBackward    input / weight / bias gradients (reference
//                     include/Autograd.hpp:470-512).
#pragma once

#include <memory>
#include <stdexcept>
#include <vector>

#include "Tensor.hpp"

struct GradMode {
    static bool& is_enabled() {
        thread_local bool enabled = true;
        return enabled;
    }
};

class NoGradGuard {
public:
    NoGradGuard() : prev_(GradMode::is_enabled()) { GradMode::is_enabled() = false; }
    ~NoGradGuard() { GradMode::is_enabled() = prev_; }
    NoGradGuard(const NoGradGuard&) = delete;
    NoGradGuard& operator=(const NoGradGuard&) = delete;

private:
    bool prev_;
};

template <typename T>
class SavedTensor {
public:
    SavedTensor() = default;
    SavedTensor(const Tensor<T>& t) : t_(t), version_(t.defined() ? t.version() : 0) {}
    Tensor<T> unpack() const {
        if (t_.defined() && t_.version() != version_)
            throw std::runtime_error(
                "RuntimeError: one of the variables needed for gradient computation "
                "has been modified by an inplace operation.");
        return t_;
    }

private:
    Tensor<T> t_;
    uint32_t version_ = 0;
};

template <typename T>
struct AutogradNode {
    virtual ~AutogradNode() = default;
    virtual void apply(const Tensor<T>& grad_output) = 0;
    virtual std::vector<Tensor<T>> get_inputs() const = 0;
};

// Operations the nodes call (defined in TensorOps.hpp).
template <typename T> Tensor<T> matmul(const Tensor<T>& A, const Tensor<T>& B);
template <typename T> Tensor<T> bmm(const Tensor<T>& A, const Tensor<T>& B);
template <typename T> Tensor<T> unbroadcast(Tensor<T> grad, const std::vector<size_t>& shape);
template <typename T>
void accumulate_product(Tensor<T>& target, const Tensor<T>& A, const Tensor<T>& B);
template <typename T>
void linear_backward_into(const Tensor<T>& dY, const Tensor<T>& X, const Tensor<T>& W, bool w_ref,
                          Tensor<T>* x_t, Tensor<T>* w_t, Tensor<T>* b_t);
template <typename T>
void conv2d_backward_input(const Tensor<T>& grad_output, const Tensor<T>& weight,
                           Tensor<T>& grad_input, size_t stride, size_t padding);
template <typename T>
void conv2d_backward_weight(const Tensor<T>& grad_output, const Tensor<T>& input,
                            Tensor<T>& grad_weight, size_t stride, size_t padding);
template <typename T>
void conv2d_backward_bias(const Tensor<T>& grad_output, Tensor<T>& grad_bias);
template <typename T>
void conv2d_backward_weight_bias(const Tensor<T>& grad_output, const Tensor<T>& input,
                                 Tensor<T>& grad_weight, Tensor<T>& grad_bias, size_t stride,
                                 size_t padding);

template <typename T>
struct AddBackward : AutogradNode<T> {
    SavedTensor<T> a, b;
    AddBackward(const Tensor<T>& x, const Tensor<T>& y) : a(x), b(y) {}
    void apply(const Tensor<T>& g) override {
        NoGradGuard guard;
        Tensor<T> x = a.unpack(), y = b.unpack();
        if (x.requires_grad()) x.accumulate_grad(unbroadcast(g, x.shape()));
        if (y.requires_grad()) y.accumulate_grad(unbroadcast(g, y.shape()));
    }
    std::vector<Tensor<T>> get_inputs() const override { return {a.unpack(), b.unpack()}; }
};

template <typename T>
struct MatmulBackward : AutogradNode<T> {
    SavedTensor<T> a, b;
    MatmulBackward(const Tensor<T>& x, const Tensor<T>& y) : a(x), b(y) {}
    void apply(const Tensor<T>& g) override {
        NoGradGuard guard;
        Tensor<T> A = a.unpack(), B = b.unpack();
        if (A.requires_grad()) accumulate_product(A, g, B.transpose(0, 1));   // dA = dC·Bᵀ
        if (B.requires_grad()) accumulate_product(B, A.transpose(0, 1), g);   // dB = Aᵀ·dC
    }
    std::vector<Tensor<T>> get_inputs() const override { return {a.unpack(), b.unpack()}; }
};

template <typename T>
struct BmmBackward : AutogradNode<T> {
    SavedTensor<T> a, b;
    BmmBackward(const Tensor<T>& x, const Tensor<T>& y) : a(x), b(y) {}
    void apply(const Tensor<T>& g) override {
        NoGradGuard guard;
        Tensor<T> A = a.unpack(), B = b.unpack();
        if (A.requires_grad()) accumulate_product(A, g, B.transpose(1, 2));
        if (B.requires_grad()) accumulate_product(B, A.transpose(1, 2), g);
    }
    std::vector<Tensor<T>> get_inputs() const override { return {a.unpack(), b.unpack()}; }
};

template <typename T>
struct LinearBackward : AutogradNode<T> {
    SavedTensor<T> x, w, b;
    bool w_ref;  // true: W is the reference's [in,out] layout; false: [out,in]
    LinearBackward(const Tensor<T>& x_, const Tensor<T>& w_, const Tensor<T>& b_, bool ref)
        : x(x_), w(w_), b(b_), w_ref(ref) {}
    void apply(const Tensor<T>& g) override {
        NoGradGuard guard;
        Tensor<T> X = x.unpack(), W = w.unpack(), Bb = b.unpack();
        const bool has_b = Bb.defined() && !Bb.empty() && Bb.requires_grad();
        linear_backward_into(g, X, W, w_ref, X.requires_grad() ? &X : nullptr,
                             W.requires_grad() ? &W : nullptr, has_b ? &Bb : nullptr);
    }
    std::vector<Tensor<T>> get_inputs() const override {
        return {x.unpack(), w.unpack(), b.unpack()};
    }
};

template <typename T>
struct Conv2DBackward : AutogradNode<T> {
    SavedTensor<T> in, w, b;
    size_t stride, padding;
    Conv2DBackward(const Tensor<T>& i, const Tensor<T>& w_, const Tensor<T>& b_, size_t s, size_t p)
        : in(i), w(w_), b(b_), stride(s), padding(p) {}
    void apply(const Tensor<T>& g) override {
        NoGradGuard guard;
        Tensor<T> input = in.unpack(), weight = w.unpack(), bias = b.unpack();
        Tensor<T> go = g.contiguous();
        if (input.requires_grad()) {
            Tensor<T> gi(input.shape(), input.device());
            conv2d_backward_input(go, weight.contiguous(), gi, stride, padding);
            input.accumulate_grad(gi);
        }
        const bool want_b = bias.defined() && !bias.empty() && bias.requires_grad();
        if (weight.requires_grad() && want_b) {   // one library call for both
            Tensor<T> gw(weight.shape(), weight.device()), gb(bias.shape(), bias.device());
            conv2d_backward_weight_bias(go, input.contiguous(), gw, gb, stride, padding);
            weight.accumulate_grad(gw);
            bias.accumulate_grad(gb);
        } else if (weight.requires_grad()) {
            Tensor<T> gw(weight.shape(), weight.device());
            conv2d_backward_weight(go, input.contiguous(), gw, stride, padding);
            weight.accumulate_grad(gw);
        } else if (want_b) {
            Tensor<T> gb(bias.shape(), bias.device());
            conv2d_backward_bias(go, gb);
            bias.accumulate_grad(gb);
        }
    }
    std::vector<Tensor<T>> get_inputs() const override {
        return {in.unpack(), w.unpack(), b.unpack()};
    }
};

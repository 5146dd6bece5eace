// Dispatch.hpp -- the op registry of the reference (include/Dispatch.hpp:12-70):
// OpType, OpRegistry<T> keyed by op, AutoRegistrar, dispatch_{unary,binary}_op.
// The reference declares it but registers nothing; here the GEMM family is
// registered for float so OpType::Matmul and OpType::Conv2D reach the same
// device routing as matmul() and conv2d().
#pragma once

#include <cstdint>
#include <functional>
#include <stdexcept>
#include <unordered_map>

#include "TensorOps.hpp"

enum class OpType : uint8_t { Add, Sub, Mul, Div, Matmul, Relu, Sigmoid, Softmax, Sum, Conv2D };

template <typename T>
using UnaryOpFn = std::function<void(const Tensor<T>&, Tensor<T>&)>;
template <typename T>
using BinaryOpFn = std::function<void(const Tensor<T>&, const Tensor<T>&, Tensor<T>&)>;

template <typename T>
class OpRegistry {
public:
    static OpRegistry& instance() {
        static OpRegistry reg;
        return reg;
    }
    void register_unary(OpType op, UnaryOpFn<T> fn) { unary_[op] = std::move(fn); }
    void register_binary(OpType op, BinaryOpFn<T> fn) { binary_[op] = std::move(fn); }
    UnaryOpFn<T>* lookup_unary(OpType op) {
        auto it = unary_.find(op);
        return it == unary_.end() ? nullptr : &it->second;
    }
    BinaryOpFn<T>* lookup_binary(OpType op) {
        auto it = binary_.find(op);
        return it == binary_.end() ? nullptr : &it->second;
    }

private:
    OpRegistry() = default;
    std::unordered_map<OpType, UnaryOpFn<T>> unary_;
    std::unordered_map<OpType, BinaryOpFn<T>> binary_;
};

template <typename T>
struct AutoRegistrar {
    AutoRegistrar(OpType op, UnaryOpFn<T> fn) { OpRegistry<T>::instance().register_unary(op, std::move(fn)); }
    AutoRegistrar(OpType op, BinaryOpFn<T> fn) { OpRegistry<T>::instance().register_binary(op, std::move(fn)); }
};

template <typename T>
void dispatch_unary_op(OpType op, const Tensor<T>& a, Tensor<T>& out) {
    if (auto* fn = OpRegistry<T>::instance().lookup_unary(op)) (*fn)(a, out);
}

template <typename T>
void dispatch_binary_op(OpType op, const Tensor<T>& a, const Tensor<T>& b, Tensor<T>& out) {
    if (auto* fn = OpRegistry<T>::instance().lookup_binary(op)) (*fn)(a, b, out);
}

namespace mt_detail {

// out = a·b into a caller-provided [M,N] tensor (any strides), routed by device.
template <typename T>
void matmul_into(const Tensor<T>& a, const Tensor<T>& b, Tensor<T>& out) {
    if (a.device() != b.device() || a.device() != out.device())
        throw std::invalid_argument("Tensors must be on the same device for matmul.");
    if (a.shape().size() != 2 || b.shape().size() != 2 || out.shape().size() != 2 ||
        a.shape()[1] != b.shape()[0] || out.shape()[0] != a.shape()[0] || out.shape()[1] != b.shape()[1])
        throw std::invalid_argument("Dimension mismatch: A columns must match B rows.");
    if (a.device().is_gpu()) matmul_gpu(a, b, out);
    else matmul_cpu_strided(a, b, out);
}

// out = conv2d(input, weight) into out's shape.  The registry's binary
// signature carries no stride or padding (include/Dispatch.hpp:21-22), so they
// are inferred from the shapes: stride 1 with the padding that gives out's
// size, else the "same" padding (kh-1)/2 of ResNet-style layers with the
// smallest stride that gives it.  Any other shape throws std::invalid_argument.
template <typename T>
void conv2d_into(const Tensor<T>& input, const Tensor<T>& weight, Tensor<T>& out) {
    if (input.shape().size() != 4 || weight.shape().size() != 4 || out.shape().size() != 4)
        throw std::invalid_argument("conv2d expects NCHW input and OIHW weight.");
    const size_t H = input.shape()[2], W = input.shape()[3];
    const size_t kh = weight.shape()[2], kw = weight.shape()[3];
    const size_t Ho = out.shape()[2], Wo = out.shape()[3];
    auto fits = [&](size_t s, size_t p) {
        return safe_out_size(H, p, kh, s) == Ho && safe_out_size(W, p, kw, s) == Wo;
    };
    size_t stride = 0, pad = 0;
    const long twice = (long)Ho - (long)H + (long)kh - 1;
    if (twice >= 0 && twice % 2 == 0 && fits(1, (size_t)twice / 2)) {
        stride = 1;
        pad = (size_t)twice / 2;
    } else {
        pad = (kh - 1) / 2;
        for (size_t s = 2; s <= std::max(H, W) + 2 * pad; ++s)
            if (fits(s, pad)) {
                stride = s;
                break;
            }
    }
    if (stride == 0)
        throw std::invalid_argument("conv2d: no stride and padding give the output shape");
    Tensor<T> r = conv2d(input, weight, Tensor<T>(), stride, pad);
    if (r.shape() != out.shape()) throw std::invalid_argument("conv2d: output shape mismatch");
    copy_strided(r, out);
}

inline const AutoRegistrar<float> kRegisterMatmul{
    OpType::Matmul, BinaryOpFn<float>(
                        [](const Tensor<float>& a, const Tensor<float>& b, Tensor<float>& out) {
                            matmul_into(a, b, out);
                        })};
inline const AutoRegistrar<float> kRegisterConv2D{
    OpType::Conv2D, BinaryOpFn<float>(
                        [](const Tensor<float>& a, const Tensor<float>& b, Tensor<float>& out) {
                            conv2d_into(a, b, out);
                        })};

}  // namespace mt_detail

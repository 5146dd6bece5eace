// Dispatch.hpp -- the op registry of the reference (include/Dispatch.hpp:12-70):
// OpType, OpRegistry<T> keyed by op, AutoRegistrar, dispatch_{unary,binary}_op.
// The reference declares it but registers nothing; here the GEMM family is
// registered for float so OpType::Matmul and OpType::Conv2D reach the same
// device routing as matmul() and conv2d().
#pragma once

#include <cstdint>
#include <functional>
#include <stdexcept>
#include <string>
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
// signature carries no stride or padding (include/Dispatch.hpp:18-21), so they
// are inferred from the shapes: every stride s >= 1 and padding
// 0 <= p < max(kh, kw) whose output size is out's is a candidate; two
// candidates compute the same thing when their paddings are equal and their
// strides are too (or the output is 1x1, where the stride is never used).
// Exactly one distinct candidate must remain: none, or several (a 9x9 input
// with a 3x3 kernel gives 3x3 at stride 3 with padding 0 or 1, and at stride
// 4 with padding 1), throws std::invalid_argument naming them; such callers
// call conv2d(input, weight, bias, stride, pad) with the values they mean.
template <typename T>
void conv2d_into(const Tensor<T>& input, const Tensor<T>& weight, Tensor<T>& out) {
    if (input.shape().size() != 4 || weight.shape().size() != 4 || out.shape().size() != 4)
        throw std::invalid_argument("conv2d expects NCHW input and OIHW weight.");
    const size_t H = input.shape()[2], W = input.shape()[3];
    const size_t kh = weight.shape()[2], kw = weight.shape()[3];
    const size_t Ho = out.shape()[2], Wo = out.shape()[3];
    const bool one = Ho == 1 && Wo == 1;
    size_t stride = 0, pad = 0, distinct = 0;
    std::string found;
    for (size_t p = 0; p < std::max<size_t>(std::max(kh, kw), 1); ++p) {
        // beyond the padded extent every stride gives one output position
        const size_t s_max = std::max(H, W) + 2 * p + 1;
        for (size_t s = 1; s <= s_max; ++s) {
            if (safe_out_size(H, p, kh, s) != Ho || safe_out_size(W, p, kw, s) != Wo) continue;
            if (distinct < 4)
                found += (distinct ? ", " : "") + std::string("stride ") + std::to_string(s) +
                         " pad " + std::to_string(p);
            if (distinct++ == 0) {
                stride = s;
                pad = p;
            }
            if (one) break;   // the other strides compute the same 1x1 output
        }
    }
    if (distinct == 0)
        throw std::invalid_argument("conv2d: no stride and padding give the output shape");
    if (distinct > 1)
        throw std::invalid_argument("conv2d: the output shape fits " + std::to_string(distinct) +
                                    " stride/padding pairs (" + found + (distinct > 4 ? ", ..." : "") +
                                    "); call conv2d(input, weight, bias, stride, pad)");
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

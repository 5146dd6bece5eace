// Functional.hpp -- F::linear and F::conv2d.
// F::conv2d forwards to conv2d as the reference does (include/Functional.hpp:28-32).
// F::linear does not exist in the reference (its Functional.hpp has no linear);
// it is added here with PyTorch's layout -- x [B,in], w [out,in], b [out] --
// as one GEMM with the bias fused into the epilogue.
#pragma once

#include "TensorOps.hpp"

namespace F {

template <typename T>
Tensor<T> linear(const Tensor<T>& x, const Tensor<T>& w, const Tensor<T>& b = Tensor<T>()) {
    return linear_impl(x, w, b, /*w_ref=*/false);
}

template <typename T>
Tensor<T> conv2d(const Tensor<T>& input, const Tensor<T>& weight, const Tensor<T>& bias,
                 size_t stride, size_t padding) {
    return ::conv2d(input, weight, bias, stride, padding);
}

}  // namespace F

// ref_driver.cpp -- TEST INFRASTRUCTURE ONLY.  A C-ABI shim, written for this
// repository, around the reference's own CPU code: it is compiled against
// the reference headers where they lie (/root/reference/include, see
// oracle/Makefile) into oracle/_ref/libref.so, so the tests can check the C
// restatement (oracle.c) against the real reference on identical inputs.
// None of the reference's source is copied here; only its public API is
// called.  The reference's tensors are CPU tensors (DeviceType::CPU), so
// everything below runs the reference's CPU kernels:
//   matmul -> matmul_cpu / matmul_cpu_strided   include/TensorOps.hpp:993-1045
//   conv2d -> conv2d_cpu                          include/TensorOps.hpp:1076-1110
//   Linear graph (matmul + broadcast add, backward through MatmulBackward /
//   AddBackward / unbroadcast)                   include/Module.hpp:112-114,
//                                                include/Autograd.hpp:55-147
#include <cstring>
#include <memory>
#include <vector>

#include "Tensor.hpp"
#include "TensorOps.hpp"

namespace {

Tensor<float> from_buffer(const float* src, size_t len) {
    Tensor<float> t({len});
    std::memcpy(t.data(), src, len * sizeof(float));
    return t;
}

// A strided 2-D view over a copy of `src` (len elements of storage).
Tensor<float> view2d(const float* src, size_t len, size_t offset, size_t rows, size_t cols,
                     size_t rs, size_t cs) {
    auto storage = std::make_shared<TensorStorage<float>>(len, Device{});
    std::memcpy(storage->data(), src, len * sizeof(float));
    return Tensor<float>(std::make_shared<TensorImpl<float>>(
        storage, std::vector<size_t>{rows, cols}, std::vector<size_t>{rs, cs}, offset));
}

Tensor<float> dense(const float* src, std::vector<size_t> shape) {
    Tensor<float> t(shape);
    std::memcpy(t.data(), src, t.total_elements() * sizeof(float));
    return t;
}

void copy_out(const Tensor<float>& t, float* dst) {
    // Results of matmul/conv2d are fresh contiguous tensors with offset 0.
    std::memcpy(dst, t.data() + t.offset(), t.total_elements() * sizeof(float));
}

}  // namespace

extern "C" {

int ref_matmul_f32(const float* a, const float* b, float* c, size_t M, size_t K, size_t N) {
    Tensor<float> A = dense(a, {M, K});
    Tensor<float> B = dense(b, {K, N});
    copy_out(matmul(A, B), c);
    return 0;
}

int ref_matmul_view_f32(const float* a, size_t a_len, size_t a_off, size_t a_rs, size_t a_cs,
                        const float* b, size_t b_len, size_t b_off, size_t b_rs, size_t b_cs,
                        size_t M, size_t K, size_t N, float* c) {
    Tensor<float> A = view2d(a, a_len, a_off, M, K, a_rs, a_cs);
    Tensor<float> B = view2d(b, b_len, b_off, K, N, b_rs, b_cs);
    copy_out(matmul(A, B), c);
    return 0;
}

int ref_conv2d_f32(const float* in, const float* w, const float* bias, float* out, size_t N,
                   size_t C, size_t H, size_t W, size_t Cout, size_t kh, size_t kw, size_t stride,
                   size_t pad) {
    Tensor<float> I = dense(in, {N, C, H, W});
    Tensor<float> Wt = dense(w, {Cout, C, kh, kw});
    Tensor<float> Bt;
    if (bias) Bt = dense(bias, {Cout});
    copy_out(conv2d(I, Wt, Bt, stride, pad), out);
    return 0;
}

// conv2d backward through the reference's autograd (Conv2DBackward ->
// conv2d_backward_{input,weight,bias}_cpu), with dY installed as the output gradient.
int ref_conv2d_bwd_f32(const float* in, const float* w, const float* dy, float* dx, float* dw,
                       float* db, size_t N, size_t C, size_t H, size_t W, size_t Cout, size_t kh,
                       size_t kw, size_t stride, size_t pad) {
    Tensor<float> I = dense(in, {N, C, H, W});
    Tensor<float> Wt = dense(w, {Cout, C, kh, kw});
    Tensor<float> Bt({Cout});
    I.set_requires_grad(true);
    Wt.set_requires_grad(true);
    Bt.set_requires_grad(true);
    Tensor<float> Y = conv2d(I, Wt, Bt, stride, pad);
    Y.grad() = dense(dy, Y.shape());
    Y.backward();
    copy_out(I.grad().contiguous(), dx);
    copy_out(Wt.grad().contiguous(), dw);
    copy_out(Bt.grad().contiguous(), db);
    return 0;
}

// The reference Linear: W_ref [in,out], bias [1,out]; Y = matmul(X, W_ref) + bias.
// The upstream gradient dY is installed as Y's gradient before backward().
int ref_linear_f32(const float* x, const float* w_ref, const float* bias, const float* dy,
                   size_t B, size_t in_f, size_t out_f, float* y, float* dx, float* dw_ref,
                   float* db) {
    Tensor<float> X = dense(x, {B, in_f});
    Tensor<float> W = dense(w_ref, {in_f, out_f});
    Tensor<float> b = dense(bias, {1, out_f});
    X.set_requires_grad(true);
    W.set_requires_grad(true);
    b.set_requires_grad(true);
    Tensor<float> Y = matmul(X, W) + b;
    copy_out(Y, y);
    Y.grad() = dense(dy, {B, out_f});
    Y.backward();
    copy_out(X.grad().contiguous(), dx);
    copy_out(W.grad().contiguous(), dw_ref);
    copy_out(b.grad().contiguous(), db);
    return 0;
}

}  // extern "C"

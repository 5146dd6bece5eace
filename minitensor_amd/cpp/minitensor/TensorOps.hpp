// TensorOps.hpp -- matmul / bmm / conv2d / broadcast add and their device routing.
//
// Public API as the reference's include/TensorOps.hpp:
//   matmul(A, B)         993-1045  2-D, A.cols == B.rows, fresh contiguous C [M,N]
//   bmm(A, B)            933-991   [B,M,K]·[B,K,N] -> [B,M,N]
//   conv2d(x, w, b, s, p) 1076-1110 NCHW, output size via safe_out_size (17-20)
//   operator+ / add_     735-833   broadcast add (the reference Linear's bias add)
//   sum / unbroadcast    1047-1070, 1304-1346
// Routing follows the reference's switch on the device type: CPU tensors run
// the host loops below (the reference CPU kernels' semantics, 139-189,
// 235-317); GPU tensors go through the C ABI of libmtgemm (include/mtgemm.h)
// and nothing else -- every view (transpose, slice with offset, expand) is
// handed to the kernels by descriptor, never copied, and the offset is always
// applied (the reference's contiguous GPU path drops it).
// GPU launchers keep the reference's names and signatures
// (include/TensorOps.hpp:697-728) for the GEMM path and what it needs:
// matmul_gpu, matmul_gpu_strided, matmul_gpu_v2, matmul_gpu_bk16 (A, B, C&);
// sum_gpu(input, axis, keepdims) -> Tensor; conv2d_gpu, conv2d_gpu_strided,
// conv2d_backward_{input,weight,bias}_gpu; fill_gpu(T*, T, size_t);
// copy_gpu_strided(const Tensor<T> src, T* dst).  (Additions: a beta argument
// defaulting to 0 on the backward weight/bias launchers, for gradient
// accumulation, and a Tensor-to-Tensor copy_gpu_strided overload.)  The
// reference's other launchers (elementwise, pooling, losses, optimizers,
// batch norm) are outside this backend.
#pragma once

#include <cmath>
#include <stdexcept>
#include <type_traits>
#include <vector>

#include "Autograd.hpp"
#include "Tensor.hpp"
#include "mtgemm.h"

inline size_t safe_out_size(size_t in, size_t pad, size_t k, size_t stride) noexcept {
    if (in + 2 * pad < k) return 0;
    return (in + 2 * pad - k) / stride + 1;
}

namespace mt_detail {

template <typename T>
void require_float_gpu() {
    static_assert(std::is_same_v<T, float>, "the GPU backend computes in float32");
}

// Descriptor of a 2-D view, or of a 3-D view as (batch, rows, cols).
inline mt_mat_f32 mat(const Tensor<float>& t) {
    const auto& sh = t.shape();
    const auto& st = t.strides();
    if (sh.size() == 2)
        return mt_mat_f32{t.data(), (int64_t)t.offset(), (int64_t)sh[0], (int64_t)sh[1],
                          (int64_t)st[0], (int64_t)st[1], 1, 0};
    if (sh.size() == 3)
        return mt_mat_f32{t.data(), (int64_t)t.offset(), (int64_t)sh[1], (int64_t)sh[2],
                          (int64_t)st[1], (int64_t)st[2], (int64_t)sh[0], (int64_t)st[0]};
    throw std::invalid_argument("GEMM operands are 2-D or 3-D");
}

// Device scratch memory from the MemoryPool for the duration of one call.
class Workspace {
public:
    Workspace(size_t bytes, Device d) : bytes_(bytes), dev_(d) {
        ptr_ = bytes ? MemoryPool::get().allocate(bytes, d) : nullptr;
    }
    ~Workspace() { MemoryPool::get().free(ptr_, bytes_, dev_); }
    Workspace(const Workspace&) = delete;
    Workspace& operator=(const Workspace&) = delete;
    void* get() const { return ptr_; }
    size_t size() const { return bytes_; }

private:
    void* ptr_;
    size_t bytes_;
    Device dev_;
};

// Collapses a (shape, x-strides, y-strides) triple into as few dims as
// possible (size-1 dims dropped, mergeable neighbours merged); outer first.
struct Dim { size_t n; size_t xs; size_t ys; };
inline std::vector<Dim> collapse(const std::vector<size_t>& shape, const std::vector<size_t>& xs,
                                 const std::vector<size_t>& ys) {
    std::vector<Dim> d;
    for (size_t i = 0; i < shape.size(); ++i)
        if (shape[i] != 1) d.push_back({shape[i], xs[i], ys[i]});
    std::vector<Dim> out;
    for (auto& cur : d) {
        if (!out.empty()) {
            Dim& prev = out.back();
            if (prev.xs == cur.n * cur.xs && prev.ys == cur.n * cur.ys) {
                prev = {prev.n * cur.n, cur.xs, cur.ys};
                continue;
            }
        }
        out.push_back(cur);
    }
    return out;
}

// Y = alpha·X + beta·Y over same-shape GPU views (X may broadcast), in slabs
// of at most three dims per mt_axpby_f32 launch.  Y is given as raw device
// memory: element i of Y is ybase[yoff + Σ idx·ystrides].
inline void axpby_raw(const Tensor<float>& X, float alpha, float* ybase, size_t yoff,
                      const std::vector<size_t>& ystrides, float beta) {
    auto dims = collapse(X.shape(), X.strides(), ystrides);
    if (dims.empty()) dims.push_back({1, 0, 0});
    while (dims.size() < 3) dims.insert(dims.begin(), Dim{1, 0, 0});
    const size_t outer = dims.size() - 3;
    size_t n_outer = 1;
    for (size_t i = 0; i < outer; ++i) n_outer *= dims[i].n;
    for (size_t o = 0; o < n_outer; ++o) {
        size_t xo = X.offset(), yo = yoff, rem = o;
        for (size_t i = outer; i-- > 0;) {
            const size_t c = rem % dims[i].n;
            rem /= dims[i].n;
            xo += c * dims[i].xs;
            yo += c * dims[i].ys;
        }
        const Dim& b = dims[outer];
        const Dim& r = dims[outer + 1];
        const Dim& c = dims[outer + 2];
        mt_mat_f32 mx{X.data(), (int64_t)xo, (int64_t)r.n, (int64_t)c.n, (int64_t)r.xs,
                      (int64_t)c.xs, (int64_t)b.n, (int64_t)b.xs};
        mt_mat_f32 my{ybase, (int64_t)yo, (int64_t)r.n, (int64_t)c.n, (int64_t)r.ys,
                      (int64_t)c.ys, (int64_t)b.n, (int64_t)b.ys};
        if (b.n > 1 && b.xs == 0) mx.batch = 1;  // broadcast over the batch dim
        mt_check_status(mt_axpby_f32(&mx, alpha, &my, beta, active_stream()), "axpby");
    }
}

inline void axpby(const Tensor<float>& X, float alpha, Tensor<float>& Y, float beta) {
    if (X.shape() != Y.shape()) throw std::invalid_argument("axpby: shape mismatch");
    axpby_raw(X, alpha, Y.data(), Y.offset(), Y.strides(), beta);
}

template <typename T>
void check_same_device(const Tensor<T>& a, const Tensor<T>& b, const char* what) {
    if (a.device() != b.device()) throw std::invalid_argument(what);
}

inline mt_conv2d_desc conv_desc(const std::vector<size_t>& in, const std::vector<size_t>& w,
                                size_t stride, size_t padding) {
    return mt_conv2d_desc{(int64_t)in[0], (int64_t)in[1], (int64_t)in[2], (int64_t)in[3],
                          (int64_t)w[0],  (int64_t)w[2],  (int64_t)w[3],  (int64_t)stride,
                          (int64_t)padding};
}

}  // namespace mt_detail

// ======================================================================
// CPU kernels (CPU tensors only)
// ======================================================================
template <typename T>
void matmul_cpu(const Tensor<T>& A, const Tensor<T>& B, Tensor<T>& C) {
    matmul_cpu_strided(A, B, C);
}

// C[i][j] = Σ_k A[i][k]·B[k][j]: i -> j -> k, T accumulator from 0.
template <typename T>
void matmul_cpu_strided(const Tensor<T>& A, const Tensor<T>& B, Tensor<T>& C, T beta = T(0)) {
    const size_t M = A.shape()[0], K = A.shape()[1], N = B.shape()[1];
    const T* a = A.data() + A.offset();
    const T* b = B.data() + B.offset();
    T* c = C.data() + C.offset();
    const size_t am = A.strides()[0], ak = A.strides()[1];
    const size_t bk = B.strides()[0], bn = B.strides()[1];
    const size_t cm = C.strides()[0], cn = C.strides()[1];
    for (size_t i = 0; i < M; ++i)
        for (size_t j = 0; j < N; ++j) {
            T sum = 0;
            for (size_t k = 0; k < K; ++k) sum += a[i * am + k * ak] * b[k * bk + j * bn];
            T& dst = c[i * cm + j * cn];
            dst = beta != T(0) ? sum + beta * dst : sum;
        }
}

template <typename T>
void copy_strided_cpu(const Tensor<T>& src, Tensor<T>& dst) {
    const size_t n = src.total_elements(), nd = src.shape().size();
    std::vector<size_t> idx(nd, 0);
    for (size_t e = 0; e < n; ++e) {
        size_t so = src.offset(), d = dst.offset();
        for (size_t i = 0; i < nd; ++i) {
            so += idx[i] * src.strides()[i];
            d += idx[i] * dst.strides()[i];
        }
        dst.data()[d] = src.data()[so];
        for (size_t i = nd; i-- > 0;) {
            if (++idx[i] < src.shape()[i]) break;
            idx[i] = 0;
        }
    }
}

// Element (n, c, y, x) of a 4-D view.
template <typename T>
inline size_t at4(const Tensor<T>& t, size_t a, size_t b, size_t c, size_t d) {
    const auto& s = t.strides();
    return t.offset() + a * s[0] + b * s[1] + c * s[2] + d * s[3];
}

template <typename T>
void conv2d_cpu(const Tensor<T>& in, const Tensor<T>& w, const Tensor<T>& bias, Tensor<T>& out,
                size_t stride, size_t pad) {
    const size_t N = in.shape()[0], Ci = in.shape()[1], H = in.shape()[2], W = in.shape()[3];
    const size_t Co = w.shape()[0], kh = w.shape()[2], kw = w.shape()[3];
    const size_t Ho = out.shape()[2], Wo = out.shape()[3];
    const bool has_b = bias.defined() && !bias.empty();
    for (size_t n = 0; n < N; ++n)
        for (size_t co = 0; co < Co; ++co)
            for (size_t y = 0; y < Ho; ++y)
                for (size_t x = 0; x < Wo; ++x) {
                    T v = has_b ? bias.data()[bias.offset() + co * bias.strides()[0]] : T(0);
                    for (size_t ci = 0; ci < Ci; ++ci)
                        for (size_t r = 0; r < kh; ++r)
                            for (size_t s = 0; s < kw; ++s) {
                                const long iy = (long)(y * stride + r) - (long)pad;
                                const long ix = (long)(x * stride + s) - (long)pad;
                                if (iy < 0 || iy >= (long)H || ix < 0 || ix >= (long)W) continue;
                                v += in.data()[at4(in, n, ci, iy, ix)] * w.data()[at4(w, co, ci, r, s)];
                            }
                    out.data()[at4(out, n, co, y, x)] = v;
                }
}

template <typename T>
void conv2d_backward_input_cpu(const Tensor<T>& go, const Tensor<T>& w, Tensor<T>& gi,
                               size_t stride, size_t pad) {
    const size_t N = gi.shape()[0], Ci = gi.shape()[1], H = gi.shape()[2], W = gi.shape()[3];
    const size_t Co = w.shape()[0], kh = w.shape()[2], kw = w.shape()[3];
    const size_t Ho = go.shape()[2], Wo = go.shape()[3];
    for (size_t n = 0; n < N; ++n)
        for (size_t ci = 0; ci < Ci; ++ci)
            for (size_t y = 0; y < H; ++y)
                for (size_t x = 0; x < W; ++x) gi.data()[at4(gi, n, ci, y, x)] = T(0);
    for (size_t n = 0; n < N; ++n)
        for (size_t co = 0; co < Co; ++co)
            for (size_t oy = 0; oy < Ho; ++oy)
                for (size_t ox = 0; ox < Wo; ++ox) {
                    const T g = go.data()[at4(go, n, co, oy, ox)];
                    for (size_t ci = 0; ci < Ci; ++ci)
                        for (size_t r = 0; r < kh; ++r)
                            for (size_t s = 0; s < kw; ++s) {
                                const long iy = (long)(oy * stride + r) - (long)pad;
                                const long ix = (long)(ox * stride + s) - (long)pad;
                                if (iy < 0 || iy >= (long)H || ix < 0 || ix >= (long)W) continue;
                                gi.data()[at4(gi, n, ci, iy, ix)] += g * w.data()[at4(w, co, ci, r, s)];
                            }
                }
}

template <typename T>
void conv2d_backward_weight_cpu(const Tensor<T>& go, const Tensor<T>& in, Tensor<T>& gw,
                                size_t stride, size_t pad) {
    const size_t N = in.shape()[0], Ci = in.shape()[1], H = in.shape()[2], W = in.shape()[3];
    const size_t Co = gw.shape()[0], kh = gw.shape()[2], kw = gw.shape()[3];
    const size_t Ho = go.shape()[2], Wo = go.shape()[3];
    // per image: a partial sum over the output positions, added to the
    // gradient image by image -- the reference's order (include/TensorOps.hpp:356-394)
    for (size_t co = 0; co < Co; ++co)
        for (size_t ci = 0; ci < Ci; ++ci)
            for (size_t r = 0; r < kh; ++r)
                for (size_t s = 0; s < kw; ++s) gw.data()[at4(gw, co, ci, r, s)] = T(0);
    for (size_t n = 0; n < N; ++n)
        for (size_t co = 0; co < Co; ++co)
            for (size_t ci = 0; ci < Ci; ++ci)
                for (size_t r = 0; r < kh; ++r)
                    for (size_t s = 0; s < kw; ++s) {
                        T v = 0;
                        for (size_t oy = 0; oy < Ho; ++oy)
                            for (size_t ox = 0; ox < Wo; ++ox) {
                                const long iy = (long)(oy * stride + r) - (long)pad;
                                const long ix = (long)(ox * stride + s) - (long)pad;
                                if (iy < 0 || iy >= (long)H || ix < 0 || ix >= (long)W) continue;
                                v += in.data()[at4(in, n, ci, iy, ix)] * go.data()[at4(go, n, co, oy, ox)];
                            }
                        gw.data()[at4(gw, co, ci, r, s)] += v;
                    }
}

template <typename T>
void conv2d_backward_bias_cpu(const Tensor<T>& go, Tensor<T>& gb) {
    const size_t N = go.shape()[0], Co = go.shape()[1], Ho = go.shape()[2], Wo = go.shape()[3];
    // per image, then added: the reference's order (include/TensorOps.hpp:396-415)
    for (size_t co = 0; co < Co; ++co) gb.data()[gb.offset() + co * gb.strides()[0]] = T(0);
    for (size_t n = 0; n < N; ++n)
        for (size_t co = 0; co < Co; ++co) {
            T v = 0;
            for (size_t y = 0; y < Ho; ++y)
                for (size_t x = 0; x < Wo; ++x) v += go.data()[at4(go, n, co, y, x)];
            gb.data()[gb.offset() + co * gb.strides()[0]] += v;
        }
}

// ======================================================================
// GPU launchers (reference names), all through libmtgemm's C ABI
// ======================================================================
// C = A·B (+ bias) (+ beta·C) for 2-D or 3-D (batched) views of any strides.
template <typename T>
void gemm_gpu(const Tensor<T>& A, const Tensor<T>& B, Tensor<T>& C,
              const std::type_identity_t<Tensor<T>>* bias = nullptr, int bias_axis = MT_BIAS_NONE,
              float beta = 0.f) {
    mt_detail::require_float_gpu<T>();
    if (C.total_elements() == 0) return;
    const mt_mat_f32 a = mt_detail::mat(A), b = mt_detail::mat(B), c = mt_detail::mat(C);
    mt_epilogue_f32 ep{nullptr, 0, MT_BIAS_NONE, beta};
    if (bias && bias->defined() && !bias->empty() && bias_axis != MT_BIAS_NONE) {
        ep.bias = bias->data() + bias->offset();
        ep.bias_stride = (int64_t)bias->strides().back();
        ep.bias_axis = bias_axis;
    }
    mt_detail::Workspace ws(mt_gemm_workspace_f32(&a, &b, &c), C.device());
    mt_check_status(mt_gemm_f32(&a, &b, &c, &ep, ws.get(), ws.size(), active_stream()), "matmul");
}

template <typename T> void matmul_gpu(const Tensor<T>& A, const Tensor<T>& B, Tensor<T>& C) { gemm_gpu(A, B, C); }
template <typename T> void matmul_gpu_strided(const Tensor<T>& A, const Tensor<T>& B, Tensor<T>& C) { gemm_gpu(A, B, C); }
template <typename T> void matmul_gpu_v2(const Tensor<T>& A, const Tensor<T>& B, Tensor<T>& C) { gemm_gpu(A, B, C); }
template <typename T> void matmul_gpu_bk16(const Tensor<T>& A, const Tensor<T>& B, Tensor<T>& C) { gemm_gpu(A, B, C); }

template <typename T>
void fill_gpu(T* data, T val, size_t n) {
    mt_detail::require_float_gpu<T>();
    mt_check_status(mt_fill_f32(data, (int64_t)n, val, active_stream()), "fill_gpu");
}

// The reference's launcher (include/TensorOps.hpp:717): src (any strides)
// into dense row-major memory at dst.
template <typename T>
void copy_gpu_strided(const Tensor<T> src, T* dst) {
    mt_detail::require_float_gpu<T>();
    if (src.total_elements() == 0) return;
    mt_detail::axpby_raw(src, 1.f, dst, 0, contiguous_strides(src.shape()), 0.f);
}

// src into dst, both any strides (dst's shape = src's).
template <typename T>
void copy_gpu_strided(const Tensor<T>& src, Tensor<T>& dst) {
    mt_detail::require_float_gpu<T>();
    mt_detail::axpby(src, 1.f, dst, 0.f);
}

template <typename T>
void copy_strided(const Tensor<T>& src, Tensor<T>& dst) {
    if (src.device().is_gpu()) copy_gpu_strided(src, dst);
    else copy_strided_cpu(src, dst);
}

// The input is read in place through its strides (any NCHW view); weight,
// bias and output are dense.  Covers conv2d_gpu and conv2d_gpu_strided
// (reference src/gpu_ops.cpp:2237-2325, 2367-2399).
template <typename T>
void conv2d_gpu(const Tensor<T>& in, const Tensor<T>& w, const Tensor<T>& bias, Tensor<T>& out,
                size_t stride, size_t padding) {
    mt_detail::require_float_gpu<T>();
    Tensor<T> wt = w.contiguous();
    const bool has_b = bias.defined() && !bias.empty();
    Tensor<T> b = has_b ? bias.contiguous() : bias;
    Tensor<T> o = out.is_contiguous() ? out : Tensor<T>(out.shape(), out.device());
    const mt_conv2d_desc d = mt_detail::conv_desc(in.shape(), wt.shape(), stride, padding);
    const int64_t st[4] = {(int64_t)in.strides()[0], (int64_t)in.strides()[1],
                           (int64_t)in.strides()[2], (int64_t)in.strides()[3]};
    mt_detail::Workspace ws(mt_conv2d_workspace_f32(&d), out.device());
    mt_check_status(mt_conv2d_fwd_strided_f32(&d, in.data() + in.offset(), st,
                                              wt.data() + wt.offset(),
                                              has_b ? b.data() + b.offset() : nullptr,
                                              o.data() + o.offset(), ws.get(), ws.size(),
                                              active_stream()),
                    "conv2d");
    if (!out.is_contiguous()) copy_gpu_strided(o, out);
}

template <typename T>
void conv2d_gpu_strided(const Tensor<T>& in, const Tensor<T>& w, const Tensor<T>& bias,
                        Tensor<T>& out, size_t stride, size_t padding) {
    conv2d_gpu(in, w, bias, out, stride, padding);
}

// The backward kernels take dense tensors: views are copied in (and a strided
// output is produced densely, then copied out; with beta != 0 its current
// contents are copied in first).
namespace mt_detail {
template <typename T>
Tensor<T> dense_out(const Tensor<T>& out, float beta) {
    if (out.is_contiguous()) return out;
    Tensor<T> o(out.shape(), out.device());
    if (beta != 0.f) copy_gpu_strided(out, o);
    return o;
}
}  // namespace mt_detail

template <typename T>
void conv2d_backward_input_gpu(const Tensor<T>& go, const Tensor<T>& w, Tensor<T>& gi,
                               size_t stride, size_t padding) {
    mt_detail::require_float_gpu<T>();
    const Tensor<T> g = go.contiguous(), wd = w.contiguous();
    Tensor<T> o = mt_detail::dense_out(gi, 0.f);
    const mt_conv2d_desc d = mt_detail::conv_desc(gi.shape(), wd.shape(), stride, padding);
    mt_detail::Workspace ws(mt_conv2d_bwd_workspace_f32(&d), gi.device());
    mt_check_status(mt_conv2d_bwd_input_f32(&d, g.data() + g.offset(), wd.data() + wd.offset(),
                                            o.data() + o.offset(), ws.get(), ws.size(),
                                            active_stream()),
                    "conv2d backward input");
    if (!gi.is_contiguous()) copy_gpu_strided(o, gi);
}

template <typename T>
void conv2d_backward_weight_gpu(const Tensor<T>& go, const Tensor<T>& in, Tensor<T>& gw,
                                size_t stride, size_t padding, float beta = 0.f) {
    mt_detail::require_float_gpu<T>();
    const Tensor<T> g = go.contiguous(), x = in.contiguous();
    Tensor<T> o = mt_detail::dense_out(gw, beta);
    const mt_conv2d_desc d = mt_detail::conv_desc(x.shape(), gw.shape(), stride, padding);
    mt_detail::Workspace ws(mt_conv2d_bwd_workspace_f32(&d), gw.device());
    mt_check_status(mt_conv2d_bwd_weight_f32(&d, x.data() + x.offset(), g.data() + g.offset(),
                                             o.data() + o.offset(), beta, ws.get(), ws.size(),
                                             active_stream()),
                    "conv2d backward weight");
    if (!gw.is_contiguous()) copy_gpu_strided(o, gw);
}

// dW and db in one library call (mt_conv2d_bwd_weight_bias_f32): db can ride
// on the reduction launch of the dW GEMM.
template <typename T>
void conv2d_backward_weight_bias_gpu(const Tensor<T>& go, const Tensor<T>& in, Tensor<T>& gw,
                                     Tensor<T>& gb, size_t stride, size_t padding) {
    mt_detail::require_float_gpu<T>();
    const Tensor<T> g = go.contiguous(), x = in.contiguous();
    Tensor<T> ow = mt_detail::dense_out(gw, 0.f), ob = mt_detail::dense_out(gb, 0.f);
    const mt_conv2d_desc d = mt_detail::conv_desc(x.shape(), gw.shape(), stride, padding);
    mt_detail::Workspace ws(mt_conv2d_bwd_workspace_f32(&d), gw.device());
    mt_check_status(mt_conv2d_bwd_weight_bias_f32(&d, x.data() + x.offset(), g.data() + g.offset(),
                                                  ow.data() + ow.offset(), 0.f,
                                                  ob.data() + ob.offset(), 0.f, ws.get(),
                                                  ws.size(), active_stream()),
                    "conv2d backward weight and bias");
    if (!gw.is_contiguous()) copy_gpu_strided(ow, gw);
    if (!gb.is_contiguous()) copy_gpu_strided(ob, gb);
}

template <typename T>
void conv2d_backward_bias_gpu(const Tensor<T>& go, Tensor<T>& gb, float beta = 0.f) {
    mt_detail::require_float_gpu<T>();
    const Tensor<T> g = go.contiguous();
    Tensor<T> o = mt_detail::dense_out(gb, beta);
    const auto& s = g.shape();
    mt_conv2d_desc d{(int64_t)s[0], 1, (int64_t)s[2], (int64_t)s[3], (int64_t)s[1], 1, 1, 1, 0};
    mt_check_status(mt_conv2d_bwd_bias_f32(&d, g.data() + g.offset(), o.data() + o.offset(),
                                           beta, active_stream()),
                    "conv2d backward bias");
    if (!gb.is_contiguous()) copy_gpu_strided(o, gb);
}

// ======================================================================
// Public operations
// ======================================================================
inline std::vector<size_t> compute_broadcast_shape(const std::vector<size_t>& a,
                                                   const std::vector<size_t>& b) {
    const size_t n = std::max(a.size(), b.size());
    std::vector<size_t> out(n);
    for (size_t i = 0; i < n; ++i) {
        const size_t da = i < n - a.size() ? 1 : a[i - (n - a.size())];
        const size_t db = i < n - b.size() ? 1 : b[i - (n - b.size())];
        if (da != db && da != 1 && db != 1)
            throw std::invalid_argument("Incompatible shapes for broadcasting.");
        out[i] = std::max(da, db);
    }
    return out;
}

template <typename T>
Tensor<T> matmul(const Tensor<T>& A, const Tensor<T>& B) {
    if (A.device() != B.device())
        throw std::invalid_argument("Tensors must be on the same device for matmul.");
    if (A.shape().size() != 2 || B.shape().size() != 2)
        throw std::invalid_argument("matmul currently only supports 2D tensors.");
    if (A.shape()[1] != B.shape()[0])
        throw std::invalid_argument("Dimension mismatch: A columns must match B rows.");
    Tensor<T> C({A.shape()[0], B.shape()[1]}, A.device());
    switch (A.device().type) {
        case DeviceType::CPU: matmul_cpu_strided(A, B, C); break;
        case DeviceType::CUDA: matmul_gpu(A, B, C); break;
        default: throw std::runtime_error("Unknown device type.");
    }
    if (GradMode::is_enabled() && (A.requires_grad() || B.requires_grad())) {
        C.set_requires_grad(true);
        C.set_grad_fn(std::make_shared<MatmulBackward<T>>(A, B));
    }
    return C;
}

template <typename T>
Tensor<T> bmm(const Tensor<T>& A, const Tensor<T>& B) {
    if (A.device() != B.device())
        throw std::invalid_argument("Tensors must be on the same device for bmm.");
    if (A.shape().size() != 3 || B.shape().size() != 3)
        throw std::invalid_argument("bmm requires 3D tensors.");
    if (A.shape()[0] != B.shape()[0]) throw std::invalid_argument("bmm: batch dimension mismatch.");
    if (A.shape()[2] != B.shape()[1])
        throw std::invalid_argument("bmm: inner dimension mismatch (A.K != B.K).");
    const size_t nb = A.shape()[0], M = A.shape()[1], K = A.shape()[2], N = B.shape()[2];
    Tensor<T> C({nb, M, N}, A.device());
    if (A.device().is_gpu()) {
        gemm_gpu(A, B, C);  // one batched launch over the leading dim, views in place
    } else {
        for (size_t z = 0; z < nb; ++z) {
            auto a = A.as_strided({M, K}, {A.strides()[1], A.strides()[2]}, A.offset() + z * A.strides()[0]);
            auto b = B.as_strided({K, N}, {B.strides()[1], B.strides()[2]}, B.offset() + z * B.strides()[0]);
            auto c = C.as_strided({M, N}, {N, 1}, z * M * N);
            matmul_cpu_strided(a, b, c);
        }
    }
    if (GradMode::is_enabled() && (A.requires_grad() || B.requires_grad())) {
        C.set_requires_grad(true);
        C.set_grad_fn(std::make_shared<BmmBackward<T>>(A, B));
    }
    return C;
}

// target.grad (+)= A·B.  A GPU gradient that already exists is accumulated by
// the GEMM epilogue (beta = 1) in place -- the reference's add_ without the
// extra launch and the extra read/write of the product.
template <typename T>
void accumulate_product(Tensor<T>& target, const Tensor<T>& A, const Tensor<T>& B) {
    Tensor<T>& g = target.grad();
    const bool gpu = target.device().is_gpu();
    if (gpu && g.defined() && !g.empty() && g.shape() == target.shape()) {
        gemm_gpu(A, B, g, nullptr, MT_BIAS_NONE, 1.f);
        return;
    }
    target.accumulate_grad(A.shape().size() == 3 ? bmm(A, B) : matmul(A, B));
}

template <typename T>
void add_(Tensor<T>& A, const Tensor<T>& B) {
    mt_detail::check_same_device(A, B, "Device mismatch.");
    Tensor<T> b = B.expand(A.shape());
    if (A.device().is_gpu()) {
        mt_detail::require_float_gpu<T>();
        mt_detail::axpby(b, 1.f, A, 1.f);
    } else {
        Tensor<T> tmp(A.shape(), A.device());
        copy_strided_cpu(b, tmp);
        Tensor<T> ac = A;
        const size_t n = A.total_elements(), nd = A.shape().size();
        std::vector<size_t> idx(nd, 0);
        for (size_t e = 0; e < n; ++e) {
            size_t o = A.offset();
            for (size_t i = 0; i < nd; ++i) o += idx[i] * A.strides()[i];
            ac.data()[o] += tmp.data()[e];
            for (size_t i = nd; i-- > 0;) {
                if (++idx[i] < A.shape()[i]) break;
                idx[i] = 0;
            }
        }
    }
    A.bump_version();
}

template <typename T>
Tensor<T> operator+(const Tensor<T>& A, const Tensor<T>& B) {
    mt_detail::check_same_device(A, B, "Device mismatch.");
    const auto shape = compute_broadcast_shape(A.shape(), B.shape());
    Tensor<T> C(shape, A.device());
    copy_strided(A.expand(shape), C);
    {
        NoGradGuard g;
        add_(C, B.expand(shape));
    }
    if (GradMode::is_enabled() && (A.requires_grad() || B.requires_grad())) {
        C.set_requires_grad(true);
        C.set_grad_fn(std::make_shared<AddBackward<T>>(A, B));
    }
    return C;
}

// Sum over one axis on the GPU: the reference's launcher
// (include/TensorOps.hpp:707, src/gpu_ops.cpp:1306-1348), with the same
// output shape (keepdims: the axis kept with extent 1).  The view is read in
// place through its strides: one mt_colsum_f32 launch per slab of the
// remaining dims that does not collapse into a single strided run.
template <typename T>
Tensor<T> sum_gpu(const Tensor<T>& A, size_t axis, bool keepdims) {
    mt_detail::require_float_gpu<T>();
    if (axis >= A.shape().size()) throw std::out_of_range("sum: axis out of range");
    std::vector<size_t> out_shape = A.shape();
    if (keepdims) out_shape[axis] = 1;
    else out_shape.erase(out_shape.begin() + axis);
    Tensor<T> out(out_shape, A.device());
    std::vector<size_t> rshape, rstr;   // remaining dims of A in order: (extent, stride)
    for (size_t i = 0; i < A.shape().size(); ++i)
        if (i != axis) { rshape.push_back(A.shape()[i]); rstr.push_back(A.strides()[i]); }
    const size_t R = A.shape()[axis], rs = A.strides()[axis];
    const size_t n_out = numel_of(rshape);
    if (n_out == 0) return out;
    auto dims = mt_detail::collapse(rshape, rstr, contiguous_strides(rshape));
    if (dims.empty()) dims.push_back({1, 0, 0});
    const mt_detail::Dim inner = dims.back();
    const size_t n_outer = n_out / inner.n;
    for (size_t o = 0; o < n_outer; ++o) {
        size_t xo = A.offset(), yo = 0, rem = o;
        for (size_t i = dims.size() - 1; i-- > 0;) {
            const size_t c = rem % dims[i].n;
            rem /= dims[i].n;
            xo += c * dims[i].xs;
            yo += c * dims[i].ys;
        }
        mt_mat_f32 x{A.data(), (int64_t)xo, (int64_t)R, (int64_t)inner.n, (int64_t)rs,
                     (int64_t)inner.xs, 1, 0};
        mt_check_status(mt_colsum_f32(&x, out.data() + yo, (int64_t)inner.ys, 0.f, active_stream()),
                        "sum");
    }
    return out;
}

// Sum over one axis of a CPU tensor, sequential over the reduced axis (the
// reference's sum_cpu order, include/TensorOps.hpp:190-233).
template <typename T>
Tensor<T> sum_cpu(const Tensor<T>& A, size_t axis, bool keepdims) {
    if (axis >= A.shape().size()) throw std::out_of_range("sum: axis out of range");
    std::vector<size_t> out_shape = A.shape();
    if (keepdims) out_shape[axis] = 1;
    else out_shape.erase(out_shape.begin() + axis);
    Tensor<T> out(out_shape, A.device());
    std::vector<size_t> rshape, rstr;
    for (size_t i = 0; i < A.shape().size(); ++i)
        if (i != axis) { rshape.push_back(A.shape()[i]); rstr.push_back(A.strides()[i]); }
    const size_t R = A.shape()[axis], rs = A.strides()[axis];
    const size_t n_out = numel_of(rshape);
    std::vector<size_t> idx(rshape.size(), 0);
    for (size_t e = 0; e < n_out; ++e) {
        size_t base = A.offset();
        for (size_t i = 0; i < rshape.size(); ++i) base += idx[i] * rstr[i];
        T s = 0;
        for (size_t j = 0; j < R; ++j) s += A.data()[base + j * rs];
        out.data()[e] = s;
        for (size_t i = rshape.size(); i-- > 0;) {
            if (++idx[i] < rshape[i]) break;
            idx[i] = 0;
        }
    }
    return out;
}

// Sum over one axis (no autograd node: used by unbroadcast under NoGradGuard),
// routed by device as the reference's sum (include/TensorOps.hpp:1047-1070).
template <typename T>
Tensor<T> sum(const Tensor<T>& A, size_t axis, bool keepdims) {
    return A.device().is_gpu() ? sum_gpu(A, axis, keepdims) : sum_cpu(A, axis, keepdims);
}

template <typename T>
Tensor<T> unbroadcast(Tensor<T> grad, const std::vector<size_t>& target) {
    NoGradGuard guard;
    if (grad.shape() == target) return grad;
    Tensor<T> r = grad;
    const size_t lead = grad.shape().size() - target.size();
    for (size_t i = 0; i < lead; ++i) r = sum(r, 0, false);
    for (size_t i = 0; i < target.size(); ++i)
        if (target[i] == 1 && r.shape()[i] > 1) r = sum(r, i, true);
    return r;
}

template <typename T>
Tensor<T> conv2d(const Tensor<T>& input, const Tensor<T>& weight, const Tensor<T>& bias,
                 size_t stride, size_t padding) {
    const bool has_b = bias.defined() && !bias.empty();
    if (input.device() != weight.device() || (has_b && input.device() != bias.device()))
        throw std::invalid_argument("Device mismatch.");
    if (input.shape().size() != 4 || weight.shape().size() != 4)
        throw std::invalid_argument("conv2d expects NCHW input and OIHW weight.");
    if (input.shape()[1] != weight.shape()[1])
        throw std::invalid_argument("conv2d: input channels do not match the weight.");
    if (stride == 0) throw std::invalid_argument("conv2d: stride must be positive.");
    if (has_b && (bias.shape().size() != 1 || bias.shape()[0] != weight.shape()[0]))
        throw std::invalid_argument("conv2d: bias must be [C_out].");
    const size_t Ho = safe_out_size(input.shape()[2], padding, weight.shape()[2], stride);
    const size_t Wo = safe_out_size(input.shape()[3], padding, weight.shape()[3], stride);
    Tensor<T> out({input.shape()[0], weight.shape()[0], Ho, Wo}, input.device());
    if (input.device().is_gpu()) conv2d_gpu(input, weight, bias, out, stride, padding);
    else conv2d_cpu(input, weight, bias, out, stride, padding);
    if (GradMode::is_enabled() &&
        (input.requires_grad() || weight.requires_grad() || (has_b && bias.requires_grad()))) {
        out.set_requires_grad(true);
        out.set_grad_fn(std::make_shared<Conv2DBackward<T>>(input, weight, bias, stride, padding));
    }
    return out;
}

template <typename T>
void conv2d_backward_input(const Tensor<T>& go, const Tensor<T>& w, Tensor<T>& gi, size_t stride,
                           size_t padding) {
    if (gi.device().is_gpu()) conv2d_backward_input_gpu(go, w, gi, stride, padding);
    else conv2d_backward_input_cpu(go, w, gi, stride, padding);
}

template <typename T>
void conv2d_backward_weight(const Tensor<T>& go, const Tensor<T>& in, Tensor<T>& gw, size_t stride,
                            size_t padding) {
    if (gw.device().is_gpu()) conv2d_backward_weight_gpu(go, in, gw, stride, padding);
    else conv2d_backward_weight_cpu(go, in, gw, stride, padding);
}

template <typename T>
void conv2d_backward_bias(const Tensor<T>& go, Tensor<T>& gb) {
    if (gb.device().is_gpu()) conv2d_backward_bias_gpu(go, gb);
    else conv2d_backward_bias_cpu(go, gb);
}

// Both parameter gradients: one library call on the GPU, the two CPU paths
// otherwise.
template <typename T>
void conv2d_backward_weight_bias(const Tensor<T>& go, const Tensor<T>& in, Tensor<T>& gw,
                                 Tensor<T>& gb, size_t stride, size_t padding) {
    if (gw.device().is_gpu() && gb.device().is_gpu()) {
        conv2d_backward_weight_bias_gpu(go, in, gw, gb, stride, padding);
    } else {
        conv2d_backward_weight(go, in, gw, stride, padding);
        conv2d_backward_bias(go, gb);
    }
}

// ---- Linear ---------------------------------------------------------------
// Y = X·Wᵀ + b (W [out,in], F::linear) or Y = X·W_ref + b (W_ref [in,out], the
// reference Linear), one GEMM with the bias fused into its epilogue.
template <typename T>
Tensor<T> linear_impl(const Tensor<T>& x, const Tensor<T>& w, const Tensor<T>& b, bool w_ref) {
    const bool has_b = b.defined() && !b.empty();
    if (x.device() != w.device() || (has_b && x.device() != b.device()))
        throw std::invalid_argument("Device mismatch.");
    if (x.shape().size() != 2 || w.shape().size() != 2)
        throw std::invalid_argument("linear: expected 2-D input and weight.");
    const Tensor<T> wm = w_ref ? w : w.transpose(0, 1);  // [in,out] view either way
    if (x.shape()[1] != wm.shape()[0])
        throw std::invalid_argument("linear: input features do not match the weight.");
    const size_t out_f = wm.shape()[1];
    if (has_b && b.total_elements() != out_f)
        throw std::invalid_argument("linear: bias must have out_features elements.");
    Tensor<T> y({x.shape()[0], out_f}, x.device());
    if (x.device().is_gpu()) {
        gemm_gpu(x, wm, y, has_b ? &b : nullptr, MT_BIAS_COL);
    } else {
        matmul_cpu_strided(x, wm, y);
        if (has_b) {
            const size_t bs = b.strides().back();
            for (size_t i = 0; i < y.shape()[0]; ++i)
                for (size_t j = 0; j < out_f; ++j) y.data()[i * out_f + j] += b.data()[b.offset() + j * bs];
        }
    }
    if (GradMode::is_enabled() && (x.requires_grad() || w.requires_grad() || (has_b && b.requires_grad()))) {
        y.set_requires_grad(true);
        y.set_grad_fn(std::make_shared<LinearBackward<T>>(x, w, b, w_ref));
    }
    return y;
}

// dX = dY·Wᵀ(view), dW = dYᵀ·X (or Xᵀ·dY for W_ref), db = Σ_rows dY; existing
// GPU gradients are accumulated in the epilogues (beta = 1).
template <typename T>
void linear_backward_into(const Tensor<T>& dY, const Tensor<T>& X, const Tensor<T>& W, bool w_ref,
                          Tensor<T>* x_t, Tensor<T>* w_t, Tensor<T>* b_t) {
    const Tensor<T> wm = w_ref ? W.transpose(0, 1) : W;  // [out,in] view
    if (x_t) accumulate_product(*x_t, dY, wm);                                   // [B,in]
    if (w_t) {
        if (w_ref) accumulate_product(*w_t, X.transpose(0, 1), dY);              // [in,out]
        else accumulate_product(*w_t, dY.transpose(0, 1), X);                   // [out,in]
    }
    if (b_t) {
        Tensor<T>& g = b_t->grad();
        if (dY.device().is_gpu() && g.defined() && !g.empty()) {
            mt_detail::require_float_gpu<T>();
            const mt_mat_f32 d = mt_detail::mat(dY);
            mt_check_status(mt_colsum_f32(&d, g.data() + g.offset(), (int64_t)g.strides().back(), 1.f,
                                          active_stream()),
                            "linear bias gradient");
        } else {
            Tensor<T> db = sum(dY, 0, false);  // [out]
            b_t->accumulate_grad(db.reshape(b_t->shape()));
        }
    }
}

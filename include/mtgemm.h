/*
 * mtgemm.h -- C ABI of the MI355X (gfx950) fp32 GEMM backend for miniTensor.
 *
 * Every entry point takes plain pointers, element strides and sizes; no C++
 * or torch types cross this boundary, so the library can be bound from the
 * reference's C++ launchers, from ctypes, or from any other FFI.
 *
 * Conventions (they follow the reference's launch contract):
 *   - Device pointers only.  `base` is the storage base (the reference's
 *     Tensor::data(), include/Tensor.hpp:80) and `offset` is added inside the
 *     library (Tensor::offset(), include/Tensor.hpp:83).  Strides are in
 *     elements, may be 0 (a broadcast / expand view, include/TensorImpl.hpp:204-228)
 *     and are never materialised.
 *   - All work is enqueued asynchronously on `stream` (a hipStream_t; NULL is
 *     the legacy default stream), like the reference's active_stream()
 *     (include/GpuUtils.hpp:61-64).  No entry point synchronises the device or
 *     allocates memory: scratch space is passed in by the caller
 *     (`workspace`, sized by the matching *_workspace_* query), as the
 *     reference takes it from its MemoryPool (src/gpu_ops.cpp:2264-2266).
 *   - Return value 0 on success, a negative mt_status otherwise; nothing
 *     throws across the ABI.  MT_ERR_INVALID maps to the reference's
 *     std::invalid_argument, every other code to std::runtime_error
 *     (include/GpuUtils.hpp:47-55).
 *   - C must not overlap A, B or bias.
 */
#ifndef MTGEMM_H
#define MTGEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MTGEMM_VERSION 1

typedef enum mt_status {
    MT_OK = 0,
    MT_ERR_INVALID = -1,     /* bad shape / stride / pointer argument        */
    MT_ERR_WORKSPACE = -2,   /* workspace missing or smaller than required   */
    MT_ERR_HIP = -3,         /* a HIP runtime call or kernel launch failed   */
    MT_ERR_UNSUPPORTED = -4, /* valid request this build does not implement  */
    MT_ERR_SCRATCH_LIMIT = -5 /* mt_gemm_noalloc_f32: the problem needs more
                                 scratch than MT_NOALLOC_SCRATCH_BYTES        */
} mt_status;

/* A (possibly batched) strided fp32 matrix view.
 * Element (b, r, c) lives at base[offset + b*batch_stride + r*row_stride + c*col_stride]. */
typedef struct mt_mat_f32 {
    const float* base;
    int64_t offset;
    int64_t rows, cols;
    int64_t row_stride, col_stride;
    int64_t batch;          /* >= 0 (0: an empty stack) */
    int64_t batch_stride;   /* 0: the same matrix for every batch entry */
} mt_mat_f32;

typedef enum mt_bias_axis {
    MT_BIAS_NONE = 0,
    MT_BIAS_ROW = 1,   /* bias[m * bias_stride] added to row m    (conv, per output channel) */
    MT_BIAS_COL = 2    /* bias[n * bias_stride] added to column n (Linear, per output feature) */
} mt_bias_axis;

/* Fused epilogue: C = A·B + bias + beta·C_old.  beta == 0 never reads C. */
typedef struct mt_epilogue_f32 {
    const float* bias;      /* device pointer, element 0 of the bias vector (offset applied) */
    int64_t bias_stride;
    int32_t bias_axis;      /* mt_bias_axis */
    float beta;
} mt_epilogue_f32;

/* C[b] = A[b]·B[b] (+ epilogue) for b in [0, batch).
 * A: [M,K], B: [K,N], C: [M,N] per batch entry; C->base is written.
 * batch = C->batch; A->batch and B->batch must be 1 or equal to it.
 * `ep` may be NULL (no bias, beta 0).  K == 0 writes bias (or zeros).
 * Replaces matmul_gpu / matmul_gpu_v2 / matmul_gpu_bk16 / matmul_gpu_strided
 * (reference src/gpu_ops.cpp:1103-1144, 1167-1223; declared in
 * include/TensorOps.hpp:703-706) and the per-batch loop of bmm
 * (include/TensorOps.hpp:933-991). */
int mt_gemm_f32(const mt_mat_f32* A, const mt_mat_f32* B, const mt_mat_f32* C,
                const mt_epilogue_f32* ep, void* workspace, size_t ws_bytes,
                void* stream);

/* Workspace bytes mt_gemm_f32 needs for these operands (0 if none). */
size_t mt_gemm_workspace_f32(const mt_mat_f32* A, const mt_mat_f32* B, const mt_mat_f32* C);

/* mt_gemm_f32 without a workspace argument.  No counterpart in the reference;
 * it is for callers that cannot allocate device memory: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Its scratch
 * (split-K partials) is a static device buffer of MT_NOALLOC_SCRATCH_BYTES
 * that the library holds on each GPU it runs on until the process ends.
 *   - Same plan and the same results, bit for bit, as mt_gemm_f32 with a
 *     workspace of mt_gemm_workspace_f32 bytes.
 *   - A problem whose mt_gemm_workspace_f32 exceeds MT_NOALLOC_SCRATCH_BYTES
 *     returns MT_ERR_SCRATCH_LIMIT and launches nothing.
 *   - Allocates nothing and calls no allocating routine; the first call on
 *     each GPU looks up that GPU's copy of the buffer (hipGetSymbolAddress).
 *   - Every call on a GPU uses that GPU's one buffer: calls that may overlap
 *     on one GPU (other streams, other threads) race, and the caller must
 *     serialise them.  Nothing in the buffer needs to start at zero: a split-K
 *     launch writes every partial before it sums them. */
#define MT_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int mt_gemm_noalloc_f32(const mt_mat_f32* A, const mt_mat_f32* B, const mt_mat_f32* C,
                        const mt_epilogue_f32* ep, void* stream);

/* out[c] = beta*out[c] + sum_r X[r][c]: the bias gradient of Linear.
 * Replaces the reference's unbroadcast -> sum_gpu(dY, 0, keepdims) path
 * (include/TensorOps.hpp:1304-1346, src/gpu_ops.cpp:1306-1348). */
int mt_colsum_f32(const mt_mat_f32* X, float* out, int64_t out_stride, float beta,
                  void* stream);

/* ---- Linear -------------------------------------------------------------
 * PyTorch layout, as F::linear: X [B,in], W [out,in], bias [out], Y [B,out].
 * The reference's Linear keeps W_ref = Wᵀ as [in,out] (include/Module.hpp:92-114);
 * a caller holding W_ref passes it with row/col strides swapped.
 * Forward:  Y = X·Wᵀ + b (bias fused into the GEMM epilogue).
 * Backward: dX = dY·W, dW = dYᵀ·X (+ beta_w·dW_old), db = Σ_rows dY (+ beta_b·db_old).
 * Any of dX, dW, db may be NULL to skip that gradient. */
int mt_linear_forward_f32(const mt_mat_f32* X, const mt_mat_f32* W, const float* bias,
                          int64_t bias_stride, const mt_mat_f32* Y,
                          void* workspace, size_t ws_bytes, void* stream);
size_t mt_linear_workspace_f32(int64_t batch_rows, int64_t in_features, int64_t out_features);
int mt_linear_backward_f32(const mt_mat_f32* dY, const mt_mat_f32* X, const mt_mat_f32* W,
                           const mt_mat_f32* dX, const mt_mat_f32* dW, float beta_w,
                           float* db, int64_t db_stride, float beta_b,
                           void* workspace, size_t ws_bytes, void* stream);

/* ---- Conv2D forward as a GEMM ---------------------------------------------
 * NCHW input [n,c_in,h,w], OIHW weight [c_out,c_in,kh,kw], bias [c_out] or NULL,
 * output [n,c_out,h_out,w_out] with h_out = (h + 2*pad - kh)/stride + 1
 * (0 when h + 2*pad < kh), as the reference's safe_out_size
 * (include/TensorOps.hpp:17-20).  Weight and output are dense (element
 * offsets applied by the caller).  The GEMM is C[c_out, n*h_out*w_out] =
 * W[c_out, c_in*kh*kw] · col[c_in*kh*kw, n*h_out*w_out] with the row bias fused
 * and the output scattered straight into NCHW.  col is never formed when
 *   c_in % 16 == 0: the input is copied to channels-last in the workspace
 *     (unless it already is channels-last), the weights to OHWI, and the GEMM
 *     kernel gathers the im2col operand from that copy with 16-byte loads;
 *   else c_in*kh*kw % 4 == 0: the GEMM kernel builds the im2col operand
 *     from the NCHW input itself, with the K order of the OIHW weights,
 *     which it reads in place (a weight pointer that is not 16-byte aligned
 *     is first copied to the workspace): from halo patches of the input in
 *     LDS where they pay, else gathered per K-chunk, 4 bytes per load.
 * (Implicit GEMM; the workspace holds the copies and any split-K partials.)
 * Otherwise (or when h or w plus twice the padding reaches 2^30) an im2col
 * pass fills a column buffer in the workspace first.  mt_conv2d_workspace_f32
 * reports the size of whichever path the geometry takes; a workspace that is
 * missing or too small returns MT_ERR_WORKSPACE.  Replaces conv2d_gpu +
 * im2col_kernel + batched_sgemm_kernel_v2 (reference src/gpu_ops.cpp:2237-2325,
 * 1748-1825, 683-859; declared include/TensorOps.hpp:708). */
typedef struct mt_conv2d_desc {
    int64_t n, c_in, h, w;
    int64_t c_out, kh, kw;
    int64_t stride, pad;
} mt_conv2d_desc;

/* A 1x1 kernel with stride 1 and no padding, c_in and h*w multiples of 4:
 * one product per image, Y_b[c_out][h*w] = W · X_b[c_in][h*w], over the NCHW
 * tensors themselves.  c_in 3, 6, 7, ... with a kernel of at least 25 taps
 * (the RGB stem) and a dense input: the input and weights padded with zero
 * channels in the workspace, then the implicit GEMM over the NCHW view. */
int mt_conv2d_fwd_f32(const mt_conv2d_desc* d, const float* input, const float* weight,
                      const float* bias, float* output, void* workspace, size_t ws_bytes,
                      void* stream);
size_t mt_conv2d_workspace_f32(const mt_conv2d_desc* d);
/* Same, for an input given as any NCHW view: in_strides = element strides of
 * (n, c, h, w), e.g. a channel slice or an NHWC-stored tensor, read in place
 * (weight and output stay dense).  The 1x1 product above takes views whose
 * (h, w) fold into one index (in_strides[2] == w * in_strides[3]); other
 * views of such a layer take the NCHW-view kernel, and the workspace query
 * covers both.  Replaces conv2d_gpu_strided +
 * conv2d_forward_kernel_strided (reference src/gpu_ops.cpp:2328-2399;
 * declared include/TensorOps.hpp:709), which conv2d() takes for
 * non-contiguous operands (include/TensorOps.hpp:1088-1097). */
int mt_conv2d_fwd_strided_f32(const mt_conv2d_desc* d, const float* input,
                              const int64_t in_strides[4], const float* weight,
                              const float* bias, float* output, void* workspace,
                              size_t ws_bytes, void* stream);

/* Conv2D backward as GEMMs (dense NCHW tensors, same descriptor as forward).
 * 1x1, stride 1, no padding, c_in and h_out*w_out multiples of 4: dX_b =
 * Wᵀ · dY_b per image, and dW = Σ_b dY_b · X_bᵀ as per-image partial
 * products in the workspace, summed (with beta·dW, and db as the channel
 * sums of dY) by the split-K reduction launch; at strides 2-4 the dW takes
 * the same product on the input pixels the stride reads, copied out into
 * the workspace.  Other geometries:
 *   weight: dW[c_out, c_in*kh*kw] = dY[c_out, n*h_out*w_out] · colᵀ (+ beta·dW);
 *           when c_in % 4 == 0 and n*h_out*w_out % 4 == 0, colᵀ is gathered by
 *           the kernel from a channels-last copy of the input (no column
 *           buffer); c_in 3, 6, 7, 10, ... (rounding up to 4 adds at most a
 *           third) the same on the input padded with zero channels in the
 *           workspace; otherwise im2col fills one first
 *           replaces conv2d_backward_weight_gpu (reference src/gpu_ops.cpp:2623-2713)
 *   input:  stride 1, square kernel, pad <= kh-1, c_out*kh*kw % 4 == 0: the
 *           implicit-GEMM forward convolution of dY with the weights
 *           transposed to [c_in][c_out] and flipped, padding kh-1-pad (no
 *           column buffer; channels-last when c_out % 16 == 0, else from
 *           the NCHW dY); a strided 1x1 kernel without padding (c_in and
 *           h_out*w_out multiples of 4): Wᵀ · dY_b per image into the
 *           workspace, then one launch writes dX (zeros where no tap
 *           reaches); other strides up to 4 (and other stride-1 kernels):
 *           one implicit GEMM per stride phase (ih % s, iw % s) of dX, a
 *           stride-1 convolution of dY with that phase's flipped sub-kernel
 *           into the workspace, then one launch interleaves the phases into
 *           dX (channels-last dY when c_out % 16 == 0, else dY read in
 *           place when every phase's c_out*taps % 4 == 0); otherwise
 *           dcol = Wᵀ · dY, then a deterministic col2im gather into dX
 *           replaces conv2d_backward_input_gpu + fused_backward_input_kernel
 *           (reference src/gpu_ops.cpp:2499-2550, 861-907)
 *   bias:   db[c] = Σ_{n,y,x} dY[n,c,y,x] (+ beta·db)
 *           replaces conv2d_backward_bias_gpu (reference src/gpu_ops.cpp:2483-2497)
 * One workspace query covers weight and input: the larger of what the two
 * paths the geometry takes use, for 16-byte-aligned tensors.  (A dY that is
 * not 16-byte aligned cannot be read in place by the implicit weight
 * gradient, which then copies it: c_out*n*h_out*w_out floats, rounded up to
 * 256 bytes, more; with less the call returns MT_ERR_WORKSPACE.) */
int mt_conv2d_bwd_weight_f32(const mt_conv2d_desc* d, const float* input, const float* grad_out,
                             float* grad_weight, float beta, void* workspace, size_t ws_bytes,
                             void* stream);
int mt_conv2d_bwd_input_f32(const mt_conv2d_desc* d, const float* grad_out, const float* weight,
                            float* grad_input, void* workspace, size_t ws_bytes, void* stream);
int mt_conv2d_bwd_bias_f32(const mt_conv2d_desc* d, const float* grad_out, float* grad_bias,
                           float beta, void* stream);
/* dW (+ beta_w·dW) and db (+ beta_b·db) in one call; grad_bias may be NULL
 * (then as mt_conv2d_bwd_weight_f32).  When the implicit weight path runs
 * with split-K, the reduction launch of its GEMM also sums db (one workgroup
 * per output channel, fixed order), so db needs no launch of its own;
 * otherwise the two run as above.  Same workspace as the weight gradient.
 * Replaces conv2d_backward_weight_gpu followed by conv2d_backward_bias_gpu
 * (reference src/gpu_ops.cpp:2623-2713 and 2483-2497; called in turn by
 * Conv2DBackward, include/Autograd.hpp:471-505). */
int mt_conv2d_bwd_weight_bias_f32(const mt_conv2d_desc* d, const float* input,
                                  const float* grad_out, float* grad_weight, float beta_w,
                                  float* grad_bias, float beta_b, void* workspace,
                                  size_t ws_bytes, void* stream);
size_t mt_conv2d_bwd_workspace_f32(const mt_conv2d_desc* d);

/* ---- support kernels the Tensor layer needs around the GEMMs --------------- */
/* p[i] = value for i in [0, n).  Replaces fill_gpu (reference
 * src/gpu_ops.cpp:1149-1161; declared include/TensorOps.hpp:721), which the
 * reference's Tensor::fill and backward()'s ones_like seed call. */
int mt_fill_f32(float* p, int64_t n, float value, void* stream);

/* Y = alpha·X + beta·Y elementwise over matching (batch, rows, cols) views.
 * X may broadcast (stride 0); beta == 0 never reads Y; Y must not alias X
 * unless X and Y are the same view.  Replaces copy_gpu_strided behind
 * Tensor::contiguous() (reference src/gpu_ops.cpp:2940-2972), the add_ of
 * accumulate_grad (include/Tensor.hpp:96-102) and the unfused broadcast bias
 * add (binary_gpu_strided with AddOp, src/gpu_ops.cpp:192-213). */
int mt_axpby_f32(const mt_mat_f32* X, float alpha, const mt_mat_f32* Y, float beta,
                 void* stream);

/* ---- diagnostics ---------------------------------------------------------- */
const char* mt_strerror(int status);
int mt_version(void);
/* Name of the kernel configuration the last mt_gemm_f32 call on this thread
 * selected (tile, operand layouts, split-K), for tests and benchmarks. */
const char* mt_last_config(void);

/* Tuning and test hooks; no counterpart in the reference (its launcher has one
 * fixed kernel per case, src/gpu_ops.cpp:1103-1144).  Kernel families: */
enum {
    MT_FAMILY_AUTO = 0,  /* the cost model chooses (default)                   */
    MT_FAMILY_RS = 1,    /* register-staged kernel: any operand layout          */
    MT_FAMILY_DL = 2,    /* direct-to-LDS kernel: k- or mn-contiguous operands;
                            configurations 0-3 gemm_f32_dl, 4-6 with fragment
                            prefetch (not the channels-last convolution
                            operand), 7 the channels-last convolution operand
                            only (64x112 tiles of 16x16 MFMA blocks)          */
    MT_FAMILY_KSW = 3,   /* wave-split kernel: small tiles, K split across the
                            waves of a workgroup; any operand layout;
                            configurations 0-3 on 32x32 MFMA blocks, 4-8 on
                            16x16 blocks (32x16, 16x32, 32x16 with 8 waves,
                            64x32, 32x64)                                    */
    MT_FAMILY_SKINNY = 4 /* vector-ALU kernels of the HBM-bound shapes:
                            configuration 0 GEMV (at most 8 rows of A against a
                            k- or mn-contiguous B, or at most 8 columns of B
                            against such an A; `splits` K splits; unforced,
                            4 against a k-contiguous operand), 1 rank-k
                            (K <= 16, at least 256 columns); no implicit
                            convolution operands, no fused row sums          */
};
/* Number of tile configurations of a family (0 for MT_FAMILY_AUTO). */
int mt_gemm_config_count(int family);
/* Forces tile configuration `cfg` of `family`, asked for `splits` K splits
 * (1..64; fewer when K is short), on every later GEMM launch of the calling
 * thread whose operands that family takes; the others keep the cost model.
 * (Direct-to-LDS configurations 4-6, the fragment-prefetching kernel with
 * 256x256, 64x64 and 128x128 tiles, take the convolution weight gradient's
 * implicit operand and the fused row sums but not the forward convolution's
 * implicit im2col operand.)
 * A forced direct-to-LDS configuration also builds the im2col operand of a
 * convolution over an NCHW view from halo patches in LDS whenever the patches
 * fit, without the rule that otherwise keeps the per-chunk gather where the
 * patches would not pay.
 * MT_FAMILY_AUTO clears it.  While it is set, workspace queries include its
 * split-K partials and a launch given less returns MT_ERR_WORKSPACE.
 * Returns MT_ERR_INVALID for an unknown family, configuration or split count. */
int mt_gemm_force_config(int family, int cfg, int splits);

#ifdef __cplusplus
}
#endif

#endif /* MTGEMM_H */

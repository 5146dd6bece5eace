// gemm_kernel.hpp -- fp32 GEMM on CDNA4 matrix cores (gfx950).
//
// One templated kernel computes C[b] = A[b]·B[b] (+ bias + beta·C) for every
// operand layout the reference's matmul can hand over: row-major tensors,
// transpose views (reference include/TensorImpl.hpp:194-202), row slices with
// an offset (include/Tensor.hpp:52-74) and stride-0 expand views
// (include/TensorImpl.hpp:204-228).  It replaces the reference's FMA kernels
// sgemm_kernel_v2 (src/gpu_ops.cpp:932-1101), matmul_kernel_strided
// (909-930) and batched_sgemm_kernel_v2 (683-859) with one MFMA design.
//
// Design (wave64, v_mfma_f32_32x32x2_f32):
//   * A block tile BM x BN is split over (BM/WM) x (BN/WN) waves; each wave
//     owns (WM/32) x (WN/32) accumulators of 32x32 fp32 (16 VGPR/AGPR each).
//   * K advances in chunks of BK, double-buffered in LDS: chunk k+1 is fetched
//     from HBM into registers while chunk k is multiplied, then written to the
//     other LDS buffer; one barrier per chunk.
//   * Each operand tile is stored in LDS in the layout that matches its
//     contiguous global dimension, so every global load is a coalesced
//     16-byte vector (or a scalar gather for unaligned / doubly strided views)
//     and no view is ever materialised:
//        k-contiguous operands  -> LDS [mn][BK+4]   (A row-major, Bᵀ views)
//        mn-contiguous operands -> LDS [BK][BMN+4]  (B row-major, Aᵀ views)
//   * K is permuted inside every 16-wide sub-chunk: at MFMA step s lanes 0-31
//     contract k = 8h + s with h = lane/32 instead of 2s + h.  A sum does not
//     depend on its order of terms, and both operands use the same
//     permutation, so the product is unchanged; the gain is that a lane's 8
//     k-values of one row are contiguous, one pair of ds_read_b128 for
//     k-contiguous LDS tiles.
//   * MFMA operand layout (v_mfma_f32_32x32x2_f32, CDNA3/CDNA4 ISA):
//        src0: lane l holds X[i = l%32][k = l/32];  src1: lane l holds Y[k = l/32][j = l%32]
//        D: lane l, register r holds D[8*(r/4) + 4*(l/32) + r%4][l%32].
//     The kernels pass B's fragment as src0 and A's as src1, i.e. they
//     accumulate the transposed block, so each lane owns four consecutive
//     columns of one output row per register quad (one 16-byte LDS write
//     when the epilogue stages the tile, store_tile_lds).
//   * Work decomposition: one workgroup per (tile, split, batch) in a 1-D grid.
//     Consecutive workgroup ids are dealt round-robin to the 8 XCDs, so ids
//     are remapped to give each XCD a contiguous range of tiles, which are
//     then ordered in groups of `group_m` tile rows for L2 reuse.
//   * Split-K writes fp32 partials to a workspace that a second kernel sums
//     in a fixed order (deterministic; no float atomics).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mtk {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Operand layout modes, in (mn, k) coordinates of the operand.
enum : int {
    L_KV = 0,  // k contiguous (stride 1), 16-byte vector loads
    L_MV = 1,  // mn contiguous (stride 1), 16-byte vector loads
    L_KS = 2,  // k-contiguous LDS tile, scalar gathers (any strides)
    L_MS = 3,  // mn-contiguous LDS tile, scalar gathers (any strides)
    L_IM = 4,  // B only, direct-to-LDS kernel: implicit im2col of a channels-last input
    L_IMW = 5, // B only, direct-to-LDS kernel: implicit im2colᵀ (conv weight gradient)
    L_IMR = 6, // B only, direct-to-LDS kernel: implicit im2col of an NCHW view, K order
               // (ci, r, s), gathered by 4-byte DMA
    L_IMH = 7, // B only (gemm_f32_dlh): L_IMR's operand built in LDS from a halo
               // patch of the input
    L_KVI = 8  // A only, direct-to-LDS kernels: k-contiguous rows split into images,
               // A(m, k) = A[(k / a_hw)*a_img + m*a_mn + k % a_hw] (dY of a
               // convolution read in NCHW as [c_out][n*h_out*w_out])
};

// Geometry of an implicit-im2col B operand over a channels-last input
// xt[img][ih][iw][ci] (image stride img_stride, dense within an image):
//   L_IM:  B(k, n) with k = (r*kw + s)*c + ci and n = (img*ho + oh)*wo + ow
//          (forward convolution; c % 16 == 0, so a 16-deep K-chunk is 16
//          consecutive channels of one filter tap);
//   L_IMW: B(k, n) with k = (img*ho + oh)*wo + ow and n = (r*kw + s)*c + ci
//          (weight gradient; c % 4 == 0, so 4 consecutive n are 4
//          consecutive channels of one tap);
// both read xt[img][oh*stride - pad + r][ow*stride - pad + s][ci], zero
// outside the image.
//   L_IMR: B(k, n) with k = (ci*kh + r)*kw + s -- the OIHW weights' own K
//          order, so they need no reorder -- and n as for L_IM, read from an
//          NCHW view of any strides (img_stride, sc, sh, sw) of the input.
struct ConvGeom {
    int64_t img_stride;
    int c, h, w, kh, kw, stride, pad, ho, wo;
    int pad_w;            // padding of the w axis (pad: the h axis); either may be
                          // negative (a window that starts inside the input)
    int64_t sc, sh, sw;   // L_IMR: element strides of a channel, a row, a column
    int hp, pw;           // L_IMH: padded rows per image, (ho-1)*stride + kh, and
                          // padded columns, (wo-1)*stride + kw
};

// Padded input rows a tile of bn consecutive output pixels can touch: at
// most ceil((bn-1)/wo) row steps, each +stride within an image and +kh across
// an image boundary (at most ceil(steps/ho) of those), plus the kh rows of the
// last window.
__host__ __device__ inline int halo_rows(const ConvGeom& g, int bn) {
    const int steps = (bn - 1 + g.wo - 1) / g.wo;
    const int cross = (steps + g.ho - 1) / g.ho;
    return steps * g.stride + (g.kh > g.stride ? cross * (g.kh - g.stride) : 0) + g.kh;
}

// Floats between consecutive channels of a patch: one channel's band
// (halo_rows x pw) rounded up to whole 64-element DMA instructions, at most
// kHaloIpcMax of them.
constexpr int kHaloIpcMax = 12;
__host__ __device__ inline int halo_chan_stride(const ConvGeom& g, int bn) {
    return (halo_rows(g, bn) * g.pw + 63) & ~63;
}

// Patch offsets of the 16*kh*kw k of a patch (k = ch*kh*kw + r*kw + s ->
// ch*halo_chan_stride + r*pw + s), passed to gemm_f32_dlh as a kernel
// argument so that a chunk's offsets are wave-uniform scalar loads.
constexpr int kHaloMaxTaps = 25;
struct HaloTable {
    int off[16 * kHaloMaxTaps];
};
inline void halo_table(const ConvGeom& g, int bn, HaloTable* t) {
    const int khw = g.kh * g.kw, cst = halo_chan_stride(g, bn);
    for (int e = 0; e < 16 * khw; ++e) {
        const int ch = e / khw, tap = e - ch * khw, r = tap / g.kw;
        t->off[e] = ch * cst + r * g.pw + (tap - r * g.kw);
    }
}

// LDS of one gemm_f32_dlh workgroup, in floats: the A ring and two patches
// of 16 channels, or the epilogue's staging if that is larger.
template <int BM, int BN, int WM, int WN>
__host__ __device__ inline int dlh_lds_floats(const ConvGeom& g) {
    constexpr int NW = (BM / WM) * (BN / WN);
    const int need = 2 * BM * 16 + 2 * 16 * halo_chan_stride(g, BN);
    return need > 1024 * NW ? need : 1024 * NW;
}


struct GemmParams {
    const float* A; int64_t a_mn, a_k, a_b;   // A(m,k) = A[m*a_mn + k*a_k + b*a_b]
    int64_t a_img; int a_hw;                  // L_KVI: image stride, k per image
    const float* B; int64_t b_mn, b_k, b_b;   // B(k,n) = B[n*b_mn + k*b_k + b*b_b]
    float* C; int64_t c_m, c_n, c_b;          // C(m,n) = C[m*c_m + col(n) + b*c_b]
    // col(n) = n*c_n when c_n_inner >= N, otherwise
    // (n / c_n_inner)*c_n_outer + (n % c_n_inner)*c_n (NCHW scatter of a conv GEMM),
    // and with c_n_inner2 > 0 (a multiple of c_n_inner) one more level:
    // (n / c_n_inner2)*c_n_outer2 + col(n % c_n_inner2) (a stride phase of a
    // strided convolution's input gradient: image, row, column).
    int64_t c_n_inner, c_n_outer;
    int64_t c_n_inner2, c_n_outer2;
    const float* bias; int64_t bias_stride; int bias_axis;  // 0 none, 1 per row m, 2 per column n
    float beta;
    float* ws;                                // split-K partials [splits][batch][M][N]
    int M, N, K, batch;
    int splits, k_per_split;                  // k_per_split is a multiple of BK
    int c_vec;    // C takes 16-byte stores of 4 consecutive columns (c_n == 1, aligned)
    int ws_vec;   // the split-K workspace takes 16-byte stores (N % 4 == 0, aligned)
    // Raw partials into ws even with one split: a batch-summed product
    // C = sum_b A_b·B_b, whose reduction launch sums all splits x batch slabs.
    int part;
    ConvGeom cv;  // B = implicit im2col of the input at B (layout L_IM only)
    // Optional fused row sums of A (direct-to-LDS kernels):
    // rowsum[m*rowsum_stride] = rowsum_beta*rowsum[...] + sum_k A(m, k).  In
    // dW = dYᵀ·X this is the bias gradient db = sum over the batch of dY.
    // With split-K or part, each (split, batch entry) writes its row sums to
    // rowsum[(split*batch + b)*M + m] instead, for the reduction (csum_rows).
    float* rowsum; int64_t rowsum_stride; float rowsum_beta;
    // Optional channel sums (the convolution bias gradient db from dY [n][M][hw]),
    // computed by the vector split-K reduction, one workgroup per row m:
    // csum[m] = csum_beta*csum[m] + sum over img < csum_n, q < csum_hw of
    // csum_src[(img*M + m)*csum_hw + q].  The launcher clears csum when the
    // plan has no such reduction (the caller then sums separately).
    const float* csum_src; float* csum; int csum_n; int64_t csum_hw; float csum_beta;
    // With csum_rows set, the channel sums are csum_beta*csum[m] + the sum over
    // slabs of csum_rows[slab*M + m] (the GEMM's row-sum partials) instead.
    const float* csum_rows;
    int tiles_m, tiles_n, group_m;
};

template <int L>
struct LayoutTraits {
    static constexpr bool kc = (L == L_KV || L == L_KS);
    static constexpr bool vec = (L == L_KV || L == L_MV);
};

// Geometry of one operand tile (BMN rows of the mn dimension by BK of k).
template <int L, int BMN, int BK, int NT>
struct TileGeom {
    static constexpr bool kc = LayoutTraits<L>::kc;
    static constexpr bool vec = LayoutTraits<L>::vec;
    static constexpr int pitch = kc ? (BK + 4) : (BMN + 4);
    static constexpr int lds_floats = kc ? BMN * pitch : BK * pitch;
    static constexpr int items = vec ? (BMN * BK / 4) / NT : (BMN * BK) / NT;
    static_assert(items >= 1, "tile too small for the thread count");
    static_assert(vec ? ((BMN * BK / 4) % NT == 0) : ((BMN * BK) % NT == 0),
                  "tile elements must divide evenly over the threads");
    static_assert(pitch % 4 == 0, "LDS rows must stay 16-byte aligned");
};

// Global -> register -> LDS mover for one operand tile.
template <int L, int BMN, int BK, int NT>
struct TileLoader {
    using G = TileGeom<L, BMN, BK, NT>;
    static constexpr int NI = G::items;
    using Reg = typename std::conditional<G::vec, f32x4, float>::type;

    const float* ptr[NI];
    int kofs[NI];
    int lds_off[NI];
    bool mn_ok[NI];
    int64_t kstep;
    Reg reg[NI];

    __device__ __forceinline__ void init(const float* X, int64_t s_mn, int64_t s_k, int MN,
                                         int mn0, int k0, int t) {
        kstep = (int64_t)BK * s_k;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int v = t + i * NT;
            int mn, kk, off;
            if constexpr (G::vec && G::kc) {
                const int kq = v % (BK / 4), r = v / (BK / 4);
                mn = mn0 + r; kk = kq * 4; off = r * G::pitch + kk;
            } else if constexpr (G::vec) {
                const int mq = v % (BMN / 4), kr = v / (BMN / 4);
                mn = mn0 + mq * 4; kk = kr; off = kr * G::pitch + mq * 4;
            } else if constexpr (G::kc) {
                const int k = v % BK, r = v / BK;
                mn = mn0 + r; kk = k; off = r * G::pitch + k;
            } else {
                const int c = v % BMN, k = v / BMN;
                mn = mn0 + c; kk = k; off = k * G::pitch + c;
            }
            mn_ok[i] = mn < MN;
            kofs[i] = kk;
            lds_off[i] = off;
            ptr[i] = X + (int64_t)(mn_ok[i] ? mn : 0) * s_mn + (int64_t)(k0 + kk) * s_k;
        }
    }

    // Fetch the chunk whose first k index is kbase; k >= kend reads as zero.
    __device__ __forceinline__ void load(int kbase, int kend) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const bool ok = mn_ok[i] && (kbase + kofs[i] < kend);
            if constexpr (G::vec) {
                f32x4 z = {0.f, 0.f, 0.f, 0.f};
                reg[i] = ok ? *reinterpret_cast<const f32x4*>(ptr[i]) : z;
            } else {
                reg[i] = ok ? *ptr[i] : 0.f;
            }
            ptr[i] += kstep;
        }
    }

    __device__ __forceinline__ void store(float* lds) const {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if constexpr (G::vec) {
                *reinterpret_cast<f32x4*>(lds + lds_off[i]) = reg[i];
            } else {
                lds[lds_off[i]] = reg[i];
            }
        }
    }
};

// The 8 k-values (sub-chunk q, permuted order) of one 32-row MFMA block.
template <int L, int BMN, int BK, int NT>
__device__ __forceinline__ void read_frag(const float* lds, int row0, int q, int lane,
                                          float (&f)[8]) {
    using G = TileGeom<L, BMN, BK, NT>;
    const int h = lane >> 5, c = lane & 31;
    if constexpr (G::kc) {
        const float* p = lds + (row0 + c) * G::pitch + q * 16 + h * 8;
        const f32x4 x = *reinterpret_cast<const f32x4*>(p);
        const f32x4 y = *reinterpret_cast<const f32x4*>(p + 4);
        f[0] = x[0]; f[1] = x[1]; f[2] = x[2]; f[3] = x[3];
        f[4] = y[0]; f[5] = y[1]; f[6] = y[2]; f[7] = y[3];
    } else {
        const float* p = lds + (q * 16 + h * 8) * G::pitch + row0 + c;
#pragma unroll
        for (int s = 0; s < 8; ++s) f[s] = p[s * G::pitch];
    }
}

__device__ __forceinline__ int xcd_remap(int bid, int nblk) {
    // Hardware deals workgroup ids round-robin over the 8 XCDs; give each XCD
    // a contiguous range of logical ids instead (only when it divides evenly).
    if ((nblk & 7) == 0) return (bid & 7) * (nblk >> 3) + (bid >> 3);
    return bid;
}

// Workgroup -> (tile row, tile column, K split, batch) of a 1-D grid laid out
// as [batch][split][tile].  Tiles are visited in groups of group_m tile rows so
// that concurrently running workgroups share A and B panels in L2.
struct TileId { int tm, tn, split, bz; };

__device__ __forceinline__ TileId tile_id(const GemmParams& p) {
    const int bid = xcd_remap(blockIdx.x, gridDim.x);
    const int ntiles = p.tiles_m * p.tiles_n;
    const int tile = bid % ntiles;
    const int rest = bid / ntiles;
    TileId id;
    id.split = rest % p.splits;
    id.bz = rest / p.splits;
    const int per_group = p.group_m * p.tiles_n;
    const int g = tile / per_group;
    const int first = g * p.group_m;
    const int gsz = min(p.tiles_m - first, p.group_m);
    const int in_g = tile - g * per_group;
    id.tm = first + in_g % gsz;
    id.tn = in_g / gsz;
    return id;
}

// One 32x32 accumulator of a wave: the MFMA is issued with B's fragment as
// its first operand and A's as its second, so it computes the transposed
// block and lane l, register r holds C(m, n) with
//     m = m_blk + l%32,   n = n_blk + 8*(r/4) + 4*(l/32) + r%4.
// Registers 4q..4q+3 of a lane are four consecutive columns of one row: the
// epilogue writes them to LDS as one 16-byte group.
__device__ __forceinline__ f32x16 mfma_32x32x2(float a, float b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(b, a, c, 0, 0, 0);
}

// Column offset col(n) of the output (see GemmParams).
// (c_n_inner < N < 2^31 when the scatter applies: a 32-bit division.)
__device__ __forceinline__ int64_t col_offset(const GemmParams& p, int n) {
    if (p.c_n_inner >= p.N) return (int64_t)n * p.c_n;
    int64_t base = 0;
    unsigned u = (unsigned)n;
    if (p.c_n_inner2 > 0) {
        const unsigned inner2 = (unsigned)p.c_n_inner2;
        const unsigned nb = u / inner2;
        base = (int64_t)nb * p.c_n_outer2;
        u -= nb * inner2;
    }
    const unsigned inner = (unsigned)p.c_n_inner;
    const unsigned no = u / inner, ni = u - no * inner;
    return base + (int64_t)no * p.c_n_outer + (int64_t)ni * p.c_n;
}

// s_waitcnt immediate (gfx9 encoding): vmcnt(n), lgkmcnt(0), expcnt unconstrained.
constexpr int waitcnt_vm_lgkm0(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4); }

// ---- Epilogue through LDS ---------------------------------------------------
// The accumulators leave through LDS, one pass per (block row i, group of JP
// block columns): every wave writes its JP 32x32 blocks acc[i][j0..j0+JP-1]
// as 16-byte groups, then all threads store the staged rows, four consecutive
// columns per thread and consecutive threads along a row (32*JP floats of a
// row are contiguous in C).  The store loop is not unrolled, so the whole
// epilogue -- bounds, bias, beta, split-K partials, scattered columns and the
// element-wise form -- stays a few hundred instructions: a fully unrolled
// epilogue over 128-256 accumulator registers is 30-200 KB of code that runs
// once per tile, every line of it an instruction-cache miss.
//
// Staged row r of a wave block is RG = 8*JP groups of 16 bytes; group g sits
// at g ^ stage_swz(r).  A ds_write_b128 covers rows c = 0..15 at one group
// (lanes 0-15) per LDS cycle: for RG >= 16 the XOR with r & 15 spreads them
// over all 16 four-bank groups; for RG == 8 rows 2 apart differ by 8 groups
// and the XOR with (r >> 1) & 7 separates the rest.
template <int RG>
__device__ __forceinline__ int stage_swz(int r) {
    if constexpr (RG >= 16) return r & 15;
    else return (r >> 1) & 7;
}

// Block columns per pass: the most (dividing NB) whose staging fits the ring.
template <int NB, int NW, int RING>
constexpr int stage_blocks() {
    int jp = NB;
    while (jp > 1 && 1024 * NW * jp > RING) jp /= 2;
    return jp;
}

// The epilogue operands of four consecutive output columns n..n+3 of row m:
// the row bias, the column biases and the old C (for beta), loaded ahead of
// the stores.  (On gfx950 vmcnt also counts stores in flight, so a load
// between two stores makes the second wait for the first to complete: an
// epilogue loop that loads and stores in each pass runs one store round trip
// per pass.  Loading every pass's operands first keeps the stores back to
// back.)  Columns past N read nothing (element-wise form).
struct Epi4 {
    float brow;
    f32x4 bcol, cold;
};
__device__ __forceinline__ Epi4 epi_load4(const GemmParams& p, const float* base, int64_t rs,
                                          bool part, bool vec, int bias_axis, float beta, int m,
                                          int n) {
    Epi4 e;
    e.brow = bias_axis == 1 ? p.bias[(int64_t)m * p.bias_stride] : 0.f;
    e.bcol = f32x4{0.f, 0.f, 0.f, 0.f};
    e.cold = f32x4{0.f, 0.f, 0.f, 0.f};
    if (bias_axis == 2)
#pragma unroll
        for (int x = 0; x < 4; ++x)
            if (vec || n + x < p.N) e.bcol[x] = p.bias[(int64_t)(n + x) * p.bias_stride];
    if (beta != 0.f) {
        const float* const row = base + (int64_t)m * rs;
        if (vec) {
            e.cold = *reinterpret_cast<const f32x4*>(row + (part ? (int64_t)n : col_offset(p, n)));
        } else {
#pragma unroll
            for (int x = 0; x < 4; ++x)
                if (n + x < p.N) e.cold[x] = row[part ? (int64_t)(n + x) : col_offset(p, n + x)];
        }
    }
    return e;
}

// Stores four consecutive output columns n..n+3 of row m (v, the bare sums):
// C = v + bias + beta*C through col(n), 16-byte when `vec`, element by element
// otherwise (columns past N skipped); or, for a split-K launch (`part`), the
// raw partial into the split's workspace slab at `base` (row stride rs).  The
// operands come from epi_load4 with the same arguments.
__device__ __forceinline__ void epi_store4(const GemmParams& p, float* base, int64_t rs,
                                           bool part, bool vec, int bias_axis, float beta, int m,
                                           int n, f32x4 v, const Epi4& e) {
    float* const row = base + (int64_t)m * rs;
    if (vec) {
        f32x4 o;
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            o[x] = v[x] + e.brow;
            if (bias_axis == 2) o[x] += e.bcol[x];
        }
        if (beta != 0.f) o += beta * e.cold;
        *reinterpret_cast<f32x4*>(row + (part ? (int64_t)n : col_offset(p, n))) = o;
    } else {
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            if (n + x >= p.N) break;
            float o = v[x] + e.brow;
            if (bias_axis == 2) o += e.bcol[x];
            if (beta != 0.f) o += beta * e.cold[x];
            row[part ? (int64_t)(n + x) : col_offset(p, n + x)] = o;
        }
    }
}

// epi_load4 then epi_store4: one group's loads and store together.
__device__ __forceinline__ void store_group4(const GemmParams& p, float* base, int64_t rs,
                                             bool part, bool vec, int bias_axis, float beta,
                                             int m, int n, f32x4 v) {
    epi_store4(p, base, rs, part, vec, bias_axis, beta, m, n, v,
               epi_load4(p, base, rs, part, vec, bias_axis, beta, m, n));
}

// Epilogue of a workgroup of NW waves (wave tiles WM x WN, WAVES_N per tile
// row) whose first output element is (m0, n0).  `lds` is the kernel's ring of
// RING floats; the main loop must be finished with it (the first pass waits
// for every wave's outstanding DMA and LDS reads before writing).  Writes
// C(m, n) = acc + bias + beta*C, or the raw partial into split `split`'s
// workspace slab.
template <int MB, int NB, int NW, int WAVES_N, int WM, int WN, int RING>
__device__ __forceinline__ void store_tile_lds(const GemmParams& p, const f32x16 (&acc)[MB][NB],
                                               float* lds, int m0, int n0, int wave, int lane,
                                               int split, int bz) {
    constexpr int NT = NW * 64;
    constexpr int JP = stage_blocks<NB, NW, RING>();
    static_assert(1024 * NW * JP <= RING, "the staging must fit the ring");
    constexpr int RG = 8 * JP;
    constexpr int PER = 4 * JP;   // 16-byte groups per thread per pass
    constexpr int U = 4;
    const int t = threadIdx.x;
    const int h = lane >> 5, c = lane & 31;
    const bool part = p.splits > 1 || p.part;
    float* const base = part ? p.ws + ((int64_t)split * p.batch + bz) * (int64_t)p.M * p.N
                             : p.C + (int64_t)bz * p.c_b;
    const int64_t rs = part ? (int64_t)p.N : p.c_m;
    const int bias_axis = part ? 0 : p.bias_axis;
    const float beta = part ? 0.f : p.beta;
    const bool vec = part ? p.ws_vec : p.c_vec;
    // 16-byte stores of the bare sums to unscattered columns: the common case,
    // with a loop of its own that batches its LDS reads.
    const bool plain = vec && bias_axis == 0 && beta == 0.f && (part || p.c_n_inner >= p.N);
    f32x4* const sl = reinterpret_cast<f32x4*>(lds);
    // Every wave's DMA has landed and its fragment reads are done before any
    // wave overwrites the ring.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j0 = 0; j0 < NB; j0 += JP) {
            __syncthreads();
#pragma unroll
            for (int jj = 0; jj < JP; ++jj)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int g = 8 * jj + 2 * q + h;
                    const f32x4 v = {acc[i][j0 + jj][4 * q], acc[i][j0 + jj][4 * q + 1],
                                     acc[i][j0 + jj][4 * q + 2], acc[i][j0 + jj][4 * q + 3]};
                    sl[(wave * 32 + c) * RG + (g ^ stage_swz<RG>(c))] = v;
                }
            __syncthreads();
            auto where = [&](int k, int* m, int* n, int* idx) {
                const int e = k * NT + t;
                const int w = e / (32 * RG), r = (e / RG) & 31, g = e % RG;
                *idx = (w * 32 + r) * RG + (g ^ stage_swz<RG>(r));
                *m = m0 + (w / WAVES_N) * WM + 32 * i + r;
                *n = n0 + (w % WAVES_N) * WN + 32 * j0 + 4 * g;
            };
            if (plain) {
                // U groups per iteration, their LDS reads issued together
#pragma unroll 1
                for (int k0 = 0; k0 < PER; k0 += U) {
                    f32x4 vs[U];
                    int ms[U], ns[U];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        int idx;
                        where(k0 + u, &ms[u], &ns[u], &idx);
                        vs[u] = sl[idx];
                    }
#pragma unroll
                    for (int u = 0; u < U; ++u)
                        if (ms[u] < p.M && ns[u] < p.N)
                            *reinterpret_cast<f32x4*>(base + (int64_t)ms[u] * rs + ns[u]) =
                                vs[u] + 0.f;
                }
                continue;
            }
#pragma unroll 1
            for (int k = 0; k < PER; ++k) {
                int m, n, idx;
                where(k, &m, &n, &idx);
                const f32x4 v = sl[idx];
                if (m >= p.M || n >= p.N) continue;
                store_group4(p, base, rs, part, vec, bias_axis, beta, m, n, v);
            }
        }
}

// MINW: minimum resident waves per SIMD the register allocation must allow
// (2 lets two 4-wave workgroups share a CU and hide each other's barriers).
template <int BM, int BN, int BK, int WM, int WN, int LA, int LB, int MINW = 1>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64, MINW)
gemm_f32_mfma(GemmParams p) {
    constexpr int WAVES_N = BN / WN;
    constexpr int NT = (BM / WM) * WAVES_N * 64;
    constexpr int MB = WM / 32, NB = WN / 32;
    static_assert(BK % 16 == 0, "BK must be a multiple of 16");
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be 32-aligned");
    using GA = TileGeom<LA, BM, BK, NT>;
    using GB = TileGeom<LB, BN, BK, NT>;

    __shared__ __attribute__((aligned(16))) float smem[2 * (GA::lds_floats + GB::lds_floats)];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    const TileId id = tile_id(p);
    const int tm = id.tm, tn = id.tn, split = id.split, bz = id.bz;
    const int m0 = tm * BM, n0 = tn * BN;
    const int k_begin = split * p.k_per_split;
    const int k_end = min(p.K, k_begin + p.k_per_split);
    const int nk = k_end > k_begin ? (k_end - k_begin + BK - 1) / BK : 0;

    TileLoader<LA, BM, BK, NT> la;
    TileLoader<LB, BN, BK, NT> lb;
    la.init(p.A + (int64_t)bz * p.a_b, p.a_mn, p.a_k, p.M, m0, k_begin, t);
    lb.init(p.B + (int64_t)bz * p.b_b, p.b_mn, p.b_k, p.N, n0, k_begin, t);

    f32x16 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    float* const As0 = smem;
    float* const Bs0 = smem + GA::lds_floats;
    float* const As1 = Bs0 + GB::lds_floats;
    float* const Bs1 = As1 + GA::lds_floats;

    if (nk > 0) {
        la.load(k_begin, k_end);
        lb.load(k_begin, k_end);
        la.store(As0);
        lb.store(Bs0);
        __syncthreads();

        for (int kt = 0; kt < nk; ++kt) {
            const bool more = kt + 1 < nk;
            const float* Acur = (kt & 1) ? As1 : As0;
            const float* Bcur = (kt & 1) ? Bs1 : Bs0;
            if (more) {
                la.load(k_begin + (kt + 1) * BK, k_end);
                lb.load(k_begin + (kt + 1) * BK, k_end);
            }
#pragma unroll
            for (int q = 0; q < BK / 16; ++q) {
                float fa[MB][8], fb[NB][8];
#pragma unroll
                for (int i = 0; i < MB; ++i)
                    read_frag<LA, BM, BK, NT>(Acur, wm * WM + i * 32, q, lane, fa[i]);
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    read_frag<LB, BN, BK, NT>(Bcur, wn * WN + j * 32, q, lane, fb[j]);
#pragma unroll
                for (int s = 0; s < 8; ++s)
#pragma unroll
                    for (int i = 0; i < MB; ++i)
#pragma unroll
                        for (int j = 0; j < NB; ++j)
                            acc[i][j] = mfma_32x32x2(fa[i][s], fb[j][s], acc[i][j]);
            }
            if (more) {
                la.store((kt & 1) ? As0 : As1);
                lb.store((kt & 1) ? Bs0 : Bs1);
            }
            __syncthreads();
        }
    }

    store_tile_lds<MB, NB, (BM / WM) * WAVES_N, WAVES_N, WM, WN,
                   2 * (GA::lds_floats + GB::lds_floats)>(p, acc, smem, m0, n0, wave, lane, split,
                                                          bz);
}

}  // namespace mtk

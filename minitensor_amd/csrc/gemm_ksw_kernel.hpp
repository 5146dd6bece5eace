// gemm_ksw_kernel.hpp -- small-tile fp32 MFMA GEMM whose waves split K.
//
// For GEMMs with too few output tiles to fill 256 CUs with the LDS-tiled
// kernels (the MLP-Linear and Linear-layer shapes: 256 x 512 x 512,
// 256 x 1000 x 2048), those kernels need split-K across workgroups: partials
// in HBM and a second reduction launch, about a third of the time at these
// sizes.  Here the K split stays inside one workgroup instead:
//   * a workgroup computes one (32*MB) x (32*NB) output tile with W waves;
//     wave w takes the 16-deep K-chunks w, w+W, w+2W, ... of the tile's K
//     range (the W waves read neighbouring 64-byte pieces of the same rows at
//     about the same time), and keeps accumulators for the whole tile;
//   * operands are not shared between the waves, so there is no LDS staging
//     and no barrier in the K loop: every wave loads its MFMA fragments
//     straight from global memory (L2) into registers, in the fragment
//     layout and K permutation of gemm_kernel.hpp (lane l: row l%32, the
//     k-values 8h..8h+7 of a chunk, h = l/32).  A k-contiguous operand with
//     16-byte rows takes two 16-byte loads per 32-row block; any other
//     layout takes 8 scalar loads, and for an mn-contiguous operand each
//     such load instruction reads 32 consecutive floats per half-wave;
//   * a ring of D register sets keeps D chunks in flight per wave; loads past
//     the wave's last chunk re-fetch that chunk (always in bounds) so the
//     loop has no branches; a partial last chunk (K % 16) is fetched with
//     bounds checks by the wave it falls to;
//   * at the end the W partial tiles meet in LDS and are summed in wave
//     order (deterministic), then the shared epilogue (store_group4) adds
//     bias and beta*C, or writes a split-K partial when the plan also splits
//     K across workgroups.
// Rows beyond M or N read a clamped, valid row (their products reach only
// outputs that are never written), as in the other kernels.
#pragma once

#include "gemm_dl_kernel.hpp"

namespace mtk {

// One operand's fragments for the wave-split kernel: NBLK blocks of 32 rows.
// VEC: k-contiguous rows with 16-byte alignment (k stride 1, row stride and
// the K range's start multiples of 4).
template <int NBLK, bool VEC>
struct KswFrag {
    const float* row[NBLK];   // this lane's row at k = k0 + 8h
    int64_t s_k;

    __device__ __forceinline__ void init(const float* X, int64_t s_mn, int64_t sk, int MN, int mn0,
                                         int k0, int lane) {
        s_k = sk;
        const int h = lane >> 5, c = lane & 31;
#pragma unroll
        for (int i = 0; i < NBLK; ++i) {
            const int64_t r = min((int64_t)mn0 + 32 * i + c, (int64_t)MN - 1);
            row[i] = X + r * s_mn + (int64_t)(k0 + 8 * h) * sk;
        }
    }

    // The whole chunk whose first k is k0 + kc.
    __device__ __forceinline__ void load(float (&f)[NBLK][8], int kc) const {
#pragma unroll
        for (int i = 0; i < NBLK; ++i) {
            const float* q = row[i] + (int64_t)kc * s_k;
            if constexpr (VEC) {
                const f32x4 x = *reinterpret_cast<const f32x4*>(q);
                const f32x4 y = *reinterpret_cast<const f32x4*>(q + 4);
                f[i][0] = x[0]; f[i][1] = x[1]; f[i][2] = x[2]; f[i][3] = x[3];
                f[i][4] = y[0]; f[i][5] = y[1]; f[i][6] = y[2]; f[i][7] = y[3];
            } else {
#pragma unroll
                for (int s = 0; s < 8; ++s) f[i][s] = q[(int64_t)s * s_k];
            }
        }
    }

    // A partial chunk: k-values at or past klen (from k0) read as zero.
    __device__ __forceinline__ void load_tail(float (&f)[NBLK][8], int kc, int klen,
                                              int lane) const {
        const int kb = kc + 8 * (lane >> 5);
#pragma unroll
        for (int i = 0; i < NBLK; ++i)
#pragma unroll
            for (int s = 0; s < 8; ++s)
                f[i][s] = kb + s < klen ? row[i][(int64_t)(kc + s) * s_k] : 0.f;
    }
};

// LDS of the cross-wave reduction: W partial tiles, rows padded by 4 floats.
template <int MB, int NB, int W>
constexpr int ksw_lds_floats() {
    return W * (32 * MB) * (32 * NB + 4);
}

// The end of both wave-split kernels: the W partial BM x BN tiles in LDS
// (rows of BN + 4 floats) are summed in wave order and stored through the
// shared epilogue (bias and beta*C, or a split-K partial) by the NT threads
// of the workgroup.
template <int BM, int BN, int W, int NT = 64 * W>
__device__ __forceinline__ void ksw_store(const GemmParams& p, const TileId& id,
                                          const float* red, int m0, int n0) {
    constexpr int PITCH = BN + 4;
    const bool part = p.splits > 1 || p.part;
    float* const base = part ? p.ws + ((int64_t)id.split * p.batch + id.bz) * (int64_t)p.M * p.N
                             : p.C + (int64_t)id.bz * p.c_b;
    const int64_t rs = part ? (int64_t)p.N : p.c_m;
    const int bias_axis = part ? 0 : p.bias_axis;
    const float beta = part ? 0.f : p.beta;
    const bool vec = part ? p.ws_vec : p.c_vec;
    constexpr int GN = BN / 4;
    constexpr int IT = (BM * GN + NT - 1) / NT;   // groups per thread
    // Every group's epilogue loads (biases, beta*C) before the first store:
    // a load behind a store waits for that store (vmcnt counts both).
    int ms[IT], ns[IT], rr[IT], cc[IT];
    bool ok[IT];
    Epi4 es[IT];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
        const int g = threadIdx.x + i * NT;
        rr[i] = g / GN;
        cc[i] = 4 * (g - rr[i] * GN);
        ms[i] = m0 + rr[i];
        ns[i] = n0 + cc[i];
        ok[i] = g < BM * GN && ms[i] < p.M && ns[i] < p.N;
        if (ok[i]) es[i] = epi_load4(p, base, rs, part, vec, bias_axis, beta, ms[i], ns[i]);
    }
    // those loads landed before the first store (none is in flight yet), so
    // that the compiler places no wait between two stores
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
#pragma unroll
    for (int i = 0; i < IT; ++i) {
        if (!ok[i]) continue;
        f32x4 v = *reinterpret_cast<const f32x4*>(red + rr[i] * PITCH + cc[i]);
#pragma unroll
        for (int w = 1; w < W; ++w)
            v += *reinterpret_cast<const f32x4*>(red + (w * BM + rr[i]) * PITCH + cc[i]);
        epi_store4(p, base, rs, part, vec, bias_axis, beta, ms[i], ns[i], v, es[i]);
    }
}

template <int MB, int NB, int W, bool VA, bool VB, int D>
__global__ void __launch_bounds__(W * 64) gemm_f32_ksw(GemmParams p) {
    constexpr int BM = 32 * MB, BN = 32 * NB;
    constexpr int PITCH = BN + 4;
    static_assert(D >= 1, "at least one chunk in flight");
    __shared__ __attribute__((aligned(16))) float red[ksw_lds_floats<MB, NB, W>()];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const TileId id = tile_id(p);
    const int m0 = id.tm * BM, n0 = id.tn * BN;
    const int k_begin = id.split * p.k_per_split;
    const int k_end = min(p.K, k_begin + p.k_per_split);
    const int klen = max(k_end - k_begin, 0);
    const int nfull = klen >> 4;
    // this wave's whole chunks: wave, wave + W, ...
    const int nkw = nfull > wave ? (nfull - 1 - wave) / W + 1 : 0;

    KswFrag<MB, VA> fa;
    KswFrag<NB, VB> fb;
    fa.init(p.A + (int64_t)id.bz * p.a_b, p.a_mn, p.a_k, p.M, m0, k_begin, lane);
    fb.init(p.B + (int64_t)id.bz * p.b_b, p.b_mn, p.b_k, p.N, n0, k_begin, lane);

    f32x16 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    if ((klen & 15) != 0 && wave == nfull % W) {   // the partial last chunk
        float a[MB][8], b[NB][8];
        fa.load_tail(a, nfull * 16, klen, lane);
        fb.load_tail(b, nfull * 16, klen, lane);
        mfma_chunk<MB, NB>(acc, a, b);
    }

    if (nkw > 0) {
        // k offset of this wave's j-th whole chunk (clamped to its last one)
        auto koff = [&](int j) { return (wave + min(j, nkw - 1) * W) * 16; };
        float ra[D][MB][8], rb[D][NB][8];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            fa.load(ra[d], koff(d));
            fb.load(rb[d], koff(d));
        }
        int j = 0;
        for (; j + D <= nkw; j += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                mfma_chunk<MB, NB>(acc, ra[d], rb[d]);
                fa.load(ra[d], koff(j + d + D));
                fb.load(rb[d], koff(j + d + D));
            }
        }
#pragma unroll
        for (int d = 0; d < D - 1; ++d)
            if (j + d < nkw) mfma_chunk<MB, NB>(acc, ra[d], rb[d]);
    }

    // Cross-wave reduction.  Lane l, register 4q+e of block (i, j) holds
    // C(32i + l%32, 32j + 8q + 4(l/32) + e): one 16-byte LDS write per quad.
    {
        const int h = lane >> 5, c = lane & 31;
        float* const mine = red + wave * BM * PITCH;
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int jb = 0; jb < NB; ++jb)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4 v = {acc[i][jb][4 * q], acc[i][jb][4 * q + 1],
                                     acc[i][jb][4 * q + 2], acc[i][jb][4 * q + 3]};
                    *reinterpret_cast<f32x4*>(mine + (32 * i + c) * PITCH + 32 * jb + 8 * q +
                                              4 * h) = v;
                }
    }
    __syncthreads();
    ksw_store<BM, BN, W>(p, id, red, m0, n0);
}


// The same wave split on 16 x 16 MFMA blocks (v_mfma_f32_16x16x4_f32, the
// same rate per SIMD as the 32 x 32 form), so that half-size tiles
// (32 x 16, 16 x 32) give a small output twice the workgroups: 256 x 512 is
// 128 tiles of 32 x 32, half the CUs, but 256 tiles of 32 x 16.
//   * Fragments: lane l takes row l%16 of a 16-row block and, for the four
//     4-deep MFMAs of a 16-deep chunk, the k-values 4g..4g+3 (g = l/16), one
//     per MFMA: one 16-byte load per block for a k-contiguous operand, four
//     scalar loads (16 consecutive floats per quarter-wave) otherwise.  The
//     same k order on both operands leaves the sum unchanged.
//   * The MFMA takes B's fragment first, so it computes the transposed block
//     and lane l, register r of block (i, j) holds
//     C(16i + l%16, 16j + 4(l/16) + r): four consecutive columns, one 16-byte
//     LDS write for the cross-wave reduction.
template <int NBLK, bool VEC>
struct KswFrag16 {
    const float* row[NBLK];   // this lane's row at k = k0 + 4g
    int64_t s_k;

    __device__ __forceinline__ void init(const float* X, int64_t s_mn, int64_t sk, int MN, int mn0,
                                         int k0, int lane) {
        s_k = sk;
        const int g = lane >> 4, c = lane & 15;
#pragma unroll
        for (int i = 0; i < NBLK; ++i) {
            const int64_t r = min((int64_t)mn0 + 16 * i + c, (int64_t)MN - 1);
            row[i] = X + r * s_mn + (int64_t)(k0 + 4 * g) * sk;
        }
    }

    __device__ __forceinline__ void load(float (&f)[NBLK][4], int kc) const {
#pragma unroll
        for (int i = 0; i < NBLK; ++i) {
            const float* q = row[i] + (int64_t)kc * s_k;
            if constexpr (VEC) {
                const f32x4 x = *reinterpret_cast<const f32x4*>(q);
                f[i][0] = x[0]; f[i][1] = x[1]; f[i][2] = x[2]; f[i][3] = x[3];
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) f[i][s] = q[(int64_t)s * s_k];
            }
        }
    }

    __device__ __forceinline__ void load_tail(float (&f)[NBLK][4], int kc, int klen,
                                              int lane) const {
        const int kb = kc + 4 * (lane >> 4);
#pragma unroll
        for (int i = 0; i < NBLK; ++i)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                f[i][s] = kb + s < klen ? row[i][(int64_t)(kc + s) * s_k] : 0.f;
    }
};

template <int MB, int NB>
__device__ __forceinline__ void mfma16_chunk(f32x4 (&acc)[MB][NB], const float (&fa)[MB][4],
                                             const float (&fb)[NB][4]) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fb[j][s], fa[i][s], acc[i][j], 0,
                                                                 0, 0);
}

template <int MB, int NB, int W>
constexpr int ksw16_lds_floats() {
    return W * (16 * MB) * (16 * NB + 4);
}

template <int MB, int NB, int W, bool VA, bool VB, int D>
__global__ void __launch_bounds__(W * 64) gemm_f32_ksw16(GemmParams p) {
    constexpr int BM = 16 * MB, BN = 16 * NB;
    constexpr int PITCH = BN + 4;
    static_assert(D >= 1, "at least one chunk in flight");
    __shared__ __attribute__((aligned(16))) float red[ksw16_lds_floats<MB, NB, W>()];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const TileId id = tile_id(p);
    const int m0 = id.tm * BM, n0 = id.tn * BN;
    const int k_begin = id.split * p.k_per_split;
    const int k_end = min(p.K, k_begin + p.k_per_split);
    const int klen = max(k_end - k_begin, 0);
    const int nfull = klen >> 4;
    const int nkw = nfull > wave ? (nfull - 1 - wave) / W + 1 : 0;

    KswFrag16<MB, VA> fa;
    KswFrag16<NB, VB> fb;
    fa.init(p.A + (int64_t)id.bz * p.a_b, p.a_mn, p.a_k, p.M, m0, k_begin, lane);
    fb.init(p.B + (int64_t)id.bz * p.b_b, p.b_mn, p.b_k, p.N, n0, k_begin, lane);

    f32x4 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    if ((klen & 15) != 0 && wave == nfull % W) {   // the partial last chunk
        float a[MB][4], b[NB][4];
        fa.load_tail(a, nfull * 16, klen, lane);
        fb.load_tail(b, nfull * 16, klen, lane);
        mfma16_chunk<MB, NB>(acc, a, b);
    }

    if (nkw > 0) {
        auto koff = [&](int j) { return (wave + min(j, nkw - 1) * W) * 16; };
        float ra[D][MB][4], rb[D][NB][4];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            fa.load(ra[d], koff(d));
            fb.load(rb[d], koff(d));
        }
        int j = 0;
        for (; j + D <= nkw; j += D) {
            if (j + D < nkw) {   // more chunks follow: refill each slot after its MFMAs
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    mfma16_chunk<MB, NB>(acc, ra[d], rb[d]);
                    fa.load(ra[d], koff(j + d + D));
                    fb.load(rb[d], koff(j + d + D));
                }
            } else {
#pragma unroll
                for (int d = 0; d < D; ++d) mfma16_chunk<MB, NB>(acc, ra[d], rb[d]);
            }
        }
#pragma unroll
        for (int d = 0; d < D - 1; ++d)
            if (j + d < nkw) mfma16_chunk<MB, NB>(acc, ra[d], rb[d]);
    }

    {
        const int g = lane >> 4, c = lane & 15;
        float* const mine = red + wave * BM * PITCH;
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int jb = 0; jb < NB; ++jb)
                *reinterpret_cast<f32x4*>(mine + (16 * i + c) * PITCH + 16 * jb + 4 * g) =
                    acc[i][jb];
    }
    __syncthreads();
    ksw_store<BM, BN, W>(p, id, red, m0, n0);
}

}  // namespace mtk

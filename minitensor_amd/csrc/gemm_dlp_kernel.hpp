// gemm_dlp_kernel.hpp -- direct-to-LDS fp32 MFMA GEMM whose waves read the
// next K-chunk's fragments while the current chunk's MFMAs issue.
//
// Three tile shapes (direct-to-LDS configurations 4, 5 and 6):
//   * 256x256 block tile, four waves of 128x128 (one wave per SIMD, 256
//     accumulator registers).  Per 16-deep K-chunk a wave reads 16 KB of
//     fragments from LDS for 128 MFMAs, against 12 KB for 64 MFMAs with the
//     8-wave 128x64 split of gemm_f32_dl: two thirds of the LDS read traffic
//     per flop.  The headline kernel.
//   * 64x64 block tile, four waves of 32x32: the small GEMMs that run about
//     one workgroup per CU, where each SIMD again holds a single wave and the
//     fragment-read latency after every barrier is exposed.
//   * 128x128 block tile, eight waves of 64x32 (two per SIMD), for K ranges
//     of at least 512 per split (256 when every workgroup has a CU).
// Structure:
//   * With no second wave on the SIMD to cover the LDS latency, chunk kt+1's
//     fragments are read while chunk kt's MFMAs issue: two register sets
//     alternate (the loop is unrolled by two so that each set is a fixed set
//     of registers).  The body has no branches, so the scheduler can spread
//     the fragment reads and the next DMA over the MFMA stream (the
//     sched_group_barrier patterns in dlp_interleave for the 256x256 tile
//     and dlp_interleave_reads for the 128x128 one; the 64x64 tile's 8
//     MFMAs per step do best left to the compiler).
//   * Ring of STAGES LDS slots, one s_barrier per chunk.  At the barrier of
//     step kt, chunk kt+1 has landed (each wave waited for its own DMA) and
//     every wave has retired its reads of chunk kt's slot, which the step then
//     refills with chunk kt+STAGES.  Refills past the last chunk re-fetch the
//     last chunk (always in bounds) into slots nobody reads again, so the DMA
//     count per step, and hence every vmcnt, is the same on every step.
//   * TAIL: a K range that is not a multiple of 16 ends in a partial chunk,
//     fetched by the same DMA with the lanes past the end reading a zero page
//     (DlLoader::issue_bounded), so the loop has no tail step.  A separate
//     instantiation: the bounds test costs the whole-chunk case about 4 %.
//   * The epilogue is store_tile_lds, as in gemm_f32_dl.
// Host contract (checked in the dispatcher): operand layouts L_KV / L_MV (B
// also the implicit im2col-transpose operand L_IMW of the convolution weight
// gradient; A and B both L_MV for the row-sum form) and a non-empty K range.
// Rows or columns beyond M or N read clamped, valid rows, as in gemm_f32_dl.
#pragma once

#include "gemm_dl_kernel.hpp"

namespace mtk {

// Spread the instructions that follow a step's barrier over its NM MFMAs:
// the DMA of the refill (up to 8 wave instructions) first, one per MFMA, then
// the fragment reads of the next chunk (up to 40 LDS instructions), one per
// one or two MFMAs.  Groups without instructions of their kind stay empty.
template <int NM>
__device__ __forceinline__ void dlp_interleave() {
    constexpr int kMfma = 0x008, kVmemRead = 0x020, kDsRead = 0x100;
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        __builtin_amdgcn_sched_group_barrier(kVmemRead, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    }
#pragma unroll
    for (int g = 0; g < 40; ++g) {
        __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kMfma, NM >= 100 ? 2 : 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kMfma, NM, 0);
}

// The 64x32 wave tile (configuration 6): the refill's DMA first, then one
// fragment read (up to 24 LDS instructions) per MFMA.  Left to itself the
// scheduler packs the reads behind the MFMAs: 16 % slower with an
// n-contiguous B (2048^2 x 1024), 2-4 % with the other layouts.
template <int LOADS>
__device__ __forceinline__ void dlp_interleave_reads() {
    constexpr int kMfma = 0x008, kVmemRead = 0x020, kDsRead = 0x100;
    __builtin_amdgcn_sched_group_barrier(kVmemRead, LOADS, 0);
#pragma unroll
    for (int g = 0; g < 24; ++g) {
        __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    }
}

// The MFMAs of k-steps S0..S1-1 of one chunk.
template <int MB, int NB, int S0, int S1>
__device__ __forceinline__ void mfma_steps(f32x16 (&acc)[MB][NB], const float (&fa)[MB][8],
                                           const float (&fb)[NB][8]) {
#pragma unroll
    for (int s = S0; s < S1; ++s)
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j)
                acc[i][j] = mfma_32x32x2(fa[i][s], fb[j][s], acc[i][j]);
}

// WPE: waves per SIMD the register allocation targets (1 lets the 128x128
// wave tile keep its 256 accumulators in AGPRs beside 256 VGPRs).
// RS: also produce the row sums of A (GemmParams::rowsum), as gemm_f32_dl's
// row-sum form does: same waves, same order of additions.
template <int BM, int BN, int WM, int WN, int LA, int LB, int STAGES, int WPE, bool TAIL,
          bool RS = false>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64)
__attribute__((amdgpu_waves_per_eu(WPE, WPE)))
gemm_f32_dlp(GemmParams p) {
    constexpr int WAVES_N = BN / WN;
    constexpr int NW = (BM / WM) * WAVES_N;
    constexpr int MB = WM / 32, NB = WN / 32;
    static_assert(STAGES >= 2, "the ring needs at least two slots");
    static_assert((LA == L_KV || LA == L_MV || LA == L_KVI) &&
                      (LB == L_KV || LB == L_MV || LB == L_IMW),
                  "vector operand layouts or the implicit im2col-transpose operand");
    constexpr bool imw = (LB == L_IMW);
    constexpr int LBF = imw ? L_MV : LB;     // LDS layout of B's tile
    constexpr bool kvi = (LA == L_KVI);      // A split into images (no partial chunks)
    static_assert(!(kvi && TAIL), "the image-split A operand's K ranges hold whole chunks");
    constexpr int LAF = kvi ? L_KV : LA;     // LDS layout of A's tile
    using TA = DlTile<LAF, BM, NW>;
    using TB = DlTile<LB, BN, NW>;
    constexpr int STAGE = TA::floats + TB::floats;
    constexpr int LOADS = TA::per_wave + TB::per_wave;   // wave instructions per chunk
    static_assert(LOADS * (STAGES - 1) < 64, "vmcnt holds at most 63");
    __shared__ __attribute__((aligned(1024))) float smem[STAGES * STAGE];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int ra = (wave / WAVES_N) * WM, rb = (wave % WAVES_N) * WN;

    const TileId id = tile_id(p);
    const int m0 = id.tm * BM, n0 = id.tn * BN;
    const int k_begin = id.split * p.k_per_split;
    const int k_end = min(p.K, k_begin + p.k_per_split);
    const int klen = k_end - k_begin;        // >= 1 by the host contract
    const int nk = TAIL ? (klen + 15) >> 4 : klen >> 4;   // host: !TAIL => klen % 16 == 0
    const float* Ab = p.A + (int64_t)id.bz * p.a_b;
    const float* Bb = p.B + (int64_t)id.bz * p.b_b;

    f32x16 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Fused row sums of A: the waves of the first wave column of the first
    // tile column see every A fragment of their rows exactly once (a partial
    // last chunk holds zeros past K; re-fetched chunks are not multiplied).
    static_assert(!RS || (LA == L_MV && LB == L_MV) || (LA == L_KV && LB == L_KV),
                  "row sums: two mn-contiguous or two k-contiguous operands");
    const bool do_rs = RS && id.tn == 0 && (wave % WAVES_N) == 0;
    float rsum[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) rsum[i] = 0.f;
    auto add_rows = [&](const float (&fa)[MB][8]) {
        if (RS && do_rs)
#pragma unroll
            for (int i = 0; i < MB; ++i)
#pragma unroll
                for (int s = 0; s < 8; ++s) rsum[i] += fa[i][s];
    };

    std::conditional_t<kvi, DlKviLoader<BM, NW>, DlLoader<LA, BM, NW>> la;
    std::conditional_t<imw, DlImwLoader<BN, NW>, DlLoader<LB, BN, NW>> lb;
    if constexpr (kvi) la.init(p, Ab, p.M, m0, k_begin, wave, lane);
    else la.init(Ab, p.a_mn, p.a_k, p.M, m0, k_begin, wave, lane);
    if constexpr (imw) lb.init(p, Bb, n0, k_begin, k_end, wave, lane);
    else lb.init(Bb, p.b_mn, p.b_k, p.N, n0, k_begin, wave, lane);
    // (The implicit operand's loader tests k < k_end itself, on every chunk.)
    auto issue = [&](float* slot, int chunk) {
        if constexpr (TAIL && !kvi) la.issue_bounded(slot, chunk, wave, klen);
        else la.issue(slot, chunk, wave);
        if constexpr (TAIL && !imw) lb.issue_bounded(slot + TA::floats, chunk, wave, klen);
        else lb.issue(slot + TA::floats, chunk, wave);
    };
#pragma unroll
    for (int c = 0; c < STAGES; ++c) {
        const int cc = min(c, nk - 1);
        issue(smem + c * STAGE, cc);
    }
    // chunk 0 landed (own DMA), then everyone's
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(LOADS * (STAGES - 1)));
    __builtin_amdgcn_s_barrier();
    float fa0[MB][8], fb0[NB][8], fa1[MB][8], fb1[NB][8];
    dl_frags<LAF, BM, MB>(smem, ra, lane, fa0);
    dl_frags<LBF, BN, NB>(smem + TA::floats, rb, lane, fb0);

    // Step kt: multiply chunk kt (registers ca/cb) while reading chunk kt+1
    // into na/nb and refilling chunk kt's slot with chunk kt+STAGES.  The
    // barrier guards only the refill and the reads, so the first PRE k-steps
    // of MFMAs issue before it: the MFMA pipe has work queued while the waves
    // synchronize (about 1 % at 4096^3, 3-9 % for the 64x64 tile).  Three
    // k-steps for the 64x32 wave tile (8 waves of the 128x128 tile): about
    // 1 % more at 2048^2 x 1024; equal or slower for the other two.
    constexpr int PRE = (MB == 2 && NB == 1) ? 3 : 2;
    auto step = [&](int kt, const float (&ca)[MB][8], const float (&cb)[NB][8],
                    float (&na)[MB][8], float (&nb)[NB][8]) {
        if constexpr (PRE > 0) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));   // ca/cb landed
            mfma_steps<MB, NB, 0, PRE>(acc, ca, cb);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(LOADS * (STAGES - 2)));
        __builtin_amdgcn_s_barrier();
        float* const refill = smem + (kt % STAGES) * STAGE;
        const int cn = min(kt + STAGES, nk - 1);
        issue(refill, cn);
        const float* const next = smem + ((kt + 1) % STAGES) * STAGE;
        dl_frags<LAF, BM, MB>(next, ra, lane, na);
        dl_frags<LBF, BN, NB>(next + TA::floats, rb, lane, nb);
        mfma_steps<MB, NB, PRE, 8>(acc, ca, cb);
        if constexpr (MB * NB * 8 >= 128) dlp_interleave<(8 - PRE) * MB * NB>();
        else if constexpr (MB == 2 && NB == 1) dlp_interleave_reads<LOADS>();
        add_rows(ca);
    };

    int kt = 0;
    for (; kt + 2 < nk; kt += 2) {
        step(kt, fa0, fb0, fa1, fb1);
        step(kt + 1, fa1, fb1, fa0, fb0);
    }
    if (kt + 1 < nk) {
        // one more step leaves the last chunk in set 1; moving it to set 0
        // keeps a single final MFMA block (an MFMA block per branch arm makes
        // the compiler copy the accumulators out of their registers)
        step(kt, fa0, fb0, fa1, fb1);
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int s = 0; s < 8; ++s) fa0[i][s] = fa1[i][s];
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int s = 0; s < 8; ++s) fb0[j][s] = fb1[j][s];
    }
    mfma_chunk<MB, NB>(acc, fa0, fb0);
    add_rows(fa0);
    if (RS && do_rs) {
        // lanes c and c+32 hold the two k-halves of row c: combine, then
        // the lower lane writes (same order for every row: deterministic)
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const float tot = rsum[i] + __shfl_xor(rsum[i], 32);
            const int m = m0 + ra + i * 32 + (lane & 31);
            if (lane < 32 && m < p.M) {
                if (p.splits > 1 || p.part) {   // this (split, batch entry)'s partial
                    p.rowsum[((int64_t)id.split * p.batch + id.bz) * p.M + m] = tot;
                } else {
                    float* d = p.rowsum + (int64_t)m * p.rowsum_stride;
                    *d = (p.rowsum_beta != 0.f ? p.rowsum_beta * *d : 0.f) + tot;
                }
            }
        }
    }
    // (store_tile_lds first waits for the re-fetches past the last chunk.)
    store_tile_lds<MB, NB, NW, WAVES_N, WM, WN, STAGES * STAGE>(p, acc, smem, m0, n0, wave, lane,
                                                                id.split, id.bz);
}

}  // namespace mtk

// gemm_dl16_kernel.hpp -- the direct-to-LDS convolution GEMM on 16x16 MFMA
// blocks (v_mfma_f32_16x16x4_f32), for tile widths that are multiples of 16
// but not of 32.
//
// Why: a ResNet layer's pixel count N*H*W is a multiple of 7*7*16 = 784 at
// every even batch, so 112 pixels (7 blocks of 16) divide it where the
// 32-multiple tiles do not: 28x28 with 128 output channels at batch 32
// (M = 128, N = 25088) is 2 x 224 = 448 tiles of 64x112, two per CU, where
// the 32-aligned tiles give 196 of 128x128 or 1568 of 64x64.  The tile
// moves about twice the operand bytes per flop of the 256x128 one, so the
// cost model offers it only where two or more workgroups share each CU.
//
// Structure (the ring and loaders of gemm_f32_dl, the fragment prefetch of
// gemm_f32_dlp, the fragments and cross-wave reduction of gemm_f32_ksw16):
//   * KG groups of GW waves; group g multiplies the 16-deep K-chunks g,
//     g + KG, g + 2*KG, ... of the tile's K range, so each SIMD holds KG
//     waves that hide each other's waits on the LDS and the barrier.  Every
//     group has its own part of each ring slot and moves its own chunks into
//     it by DMA (global_load_lds_dwordx4; the chunk's A and B tiles split
//     evenly over the group's waves), STAGES chunks in flight per group, one
//     s_barrier per step (a chunk per group).
//   * While a step's MFMAs issue, each wave reads its fragments of the
//     group's next chunk (two register sets, the loop unrolled by two), and
//     the first PRE k-steps issue before the barrier.  Refills past a
//     group's last chunk DMA the zero page: every step issues the same DMA
//     (constant vmcnt waits) and a group with one chunk fewer multiplies a
//     zero chunk, with no branch around the MFMAs.
//   * A (k-contiguous weights) and B (the implicit im2col of a channels-last
//     input, DlImLoader) land in the swizzled k-contiguous tile [rows][16];
//     B's tile is padded to whole DMA instructions (rows at or past BN read
//     zeros and are never multiplied).
//   * Fragments: lane l reads row l%16 of a 16-row block at the k-group
//     l/16 (one ds_read_b128, the tiles swizzled by kswz16 for these reads),
//     and the four 4-deep MFMAs of the chunk take its four k-values, in the
//     same order on both operands.
//   * At the end the KG partial tiles meet in LDS and are summed in group
//     order (deterministic), then stored by the shared epilogue (bias, beta,
//     the scattered NCHW output, or a split-K partial).
// Host contract (launch_gemm): B = L_IM, c % 16 == 0 (whole chunks), the grid
// tiles_m x tiles_n x splits x batch.
#pragma once

#include "gemm_ksw_kernel.hpp"

namespace mtk {

template <int BM, int BN, int WM, int WN, int KG>
struct Dl16Geom {
    static constexpr int WAVES_N = BN / WN;
    static constexpr int GW = (BM / WM) * WAVES_N;   // waves per K-group
    static constexpr int NW = KG * GW;
    static constexpr int MB = WM / 16, NB = WN / 16;
    // B's tile rows: whole DMA instructions (16 rows each) for every wave
    static constexpr int BNP = (BN + 16 * GW - 1) / (16 * GW) * (16 * GW);
    using TA = DlTile<L_KV, BM, GW>;
    using TB = DlTile<L_IM, BNP, GW>;
    static constexpr int CHUNK = TA::floats + TB::floats;   // one group's chunk
    static constexpr int LOADS = TA::per_wave + TB::per_wave;
    static constexpr int PITCH = BN + 4;
    static_assert(WM % 16 == 0 && WN % 16 == 0 && BM % WM == 0 && BN % WN == 0,
                  "wave tiles of whole 16x16 blocks");
};

template <int BM, int BN, int WM, int WN, int KG, int STAGES>
constexpr int dl16_lds_floats() {
    using G = Dl16Geom<BM, BN, WM, WN, KG>;
    constexpr int ring = STAGES * KG * G::CHUNK;
    constexpr int red = KG * BM * G::PITCH;
    return ring > red ? ring : red;
}

// The 4 k-values of one 16-row block for this lane from a k-contiguous tile.
__device__ __forceinline__ void dl16_frag(const float* tile, int row0, int lane, float (&f)[4]) {
    const int r = row0 + (lane & 15);
    const f32x4 x =
        *reinterpret_cast<const f32x4*>(tile + r * 16 + (((lane >> 4) ^ kswz16(r)) << 2));
    f[0] = x[0]; f[1] = x[1]; f[2] = x[2]; f[3] = x[3];
}

// The MFMAs of k-steps S0..S1-1 (4 k each) of one chunk.
template <int MB, int NB, int S0, int S1>
__device__ __forceinline__ void mfma16_steps(f32x4 (&acc)[MB][NB], const float (&fa)[MB][4],
                                             const float (&fb)[NB][4]) {
#pragma unroll
    for (int s = S0; s < S1; ++s)
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fb[j][s], fa[i][s], acc[i][j], 0,
                                                                 0, 0);
}

// One DMA per instruction slot of a chunk from the zero page: the refills
// past a group's last chunk (same instruction count, so every vmcnt holds).
template <int INSTS, int GW>
__device__ __forceinline__ void dl16_issue_zero(float* tile, int gw) {
#pragma unroll
    for (int j = 0; j < INSTS / GW; ++j)
        __builtin_amdgcn_global_load_lds(
            (const void __attribute__((address_space(1)))*)dl_zero_page,
            (void __attribute__((address_space(3)))*)(tile + (j * GW + gw) * 256), 16, 0, 0);
}

template <int BM, int BN, int WM, int WN, int KG, int STAGES, int PRE>
__global__ void __launch_bounds__(KG * (BM / WM) * (BN / WN) * 64)
gemm_f32_dl16(GemmParams p) {
    using G = Dl16Geom<BM, BN, WM, WN, KG>;
    using TA = typename G::TA;
    using TB = typename G::TB;
    constexpr int GW = G::GW, NW = G::NW, MB = G::MB, NB = G::NB;
    constexpr int CHUNK = G::CHUNK, LOADS = G::LOADS, PITCH = G::PITCH;
    constexpr int SLOT = KG * CHUNK;   // one ring slot: a chunk per group
    static_assert(STAGES >= 2, "the ring needs at least two slots");
    static_assert(LOADS * (STAGES - 1) < 64, "vmcnt holds at most 63");
    __shared__ __attribute__((aligned(1024))) float smem[dl16_lds_floats<BM, BN, WM, WN, KG, STAGES>()];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = wave / GW, gw = wave - grp * GW;     // K-group, wave within it
    const int wm = gw / G::WAVES_N, wn = gw - wm * G::WAVES_N;
    const int ra = wm * WM, rb = wn * WN;

    const TileId id = tile_id(p);
    const int m0 = id.tm * BM, n0 = id.tn * BN;
    const int k_begin = id.split * p.k_per_split;
    const int k_end = min(p.K, k_begin + p.k_per_split);
    const int nk = max(k_end - k_begin, 0) >> 4;          // whole chunks (c % 16 == 0), >= 1
    const int ng = nk > grp ? (nk - 1 - grp) / KG + 1 : 0;  // this group's chunks
    // Every group runs npass steps (one barrier each); a group with fewer
    // chunks multiplies zero chunks (refills past its last chunk DMA the
    // zero page), which leaves its sums unchanged.
    const int npass = (nk + KG - 1) / KG;

    // group grp's j-th chunk is chunk grp + KG*j of the range
    DlLoader<L_KV, BM, GW, 1> la;
    DlImLoader<G::BNP, GW, BN, KG, 1> lb;
    la.init(p.A + (int64_t)id.bz * p.a_b, p.a_mn, p.a_k, p.M, m0, k_begin + 16 * grp, gw, lane);
    lb.init(p, p.B + (int64_t)id.bz * p.b_b, n0, k_begin + 16 * grp, k_end, gw, lane);
    la.kstep *= KG;
    float* const mine = smem + grp * CHUNK;   // this group's chunk of slot 0
    // chunks in order 0, 1, 2, ... (the implicit operand's loader steps itself)
    auto issue = [&](int j) {
        float* const st = mine + (j % STAGES) * SLOT;
        if (j < ng) {
            la.issue(st, j, gw);
            lb.issue(st + TA::floats, j, gw);
        } else {
            dl16_issue_zero<TA::insts, GW>(st, gw);
            dl16_issue_zero<TB::insts, GW>(st + TA::floats, gw);
        }
    };

    f32x4 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int c = 0; c < STAGES; ++c) issue(c);
    // chunk 0 landed (own DMA), then everyone's
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(LOADS * (STAGES - 1)));
    __builtin_amdgcn_s_barrier();
    float fa0[MB][4], fb0[NB][4], fa1[MB][4], fb1[NB][4];
    auto frags = [&](int j, float (&fa)[MB][4], float (&fb)[NB][4]) {
        const float* const At = mine + (j % STAGES) * SLOT;
#pragma unroll
        for (int i = 0; i < MB; ++i) dl16_frag(At, ra + 16 * i, lane, fa[i]);
#pragma unroll
        for (int jb = 0; jb < NB; ++jb) dl16_frag(At + TA::floats, rb + 16 * jb, lane, fb[jb]);
    };
    frags(0, fa0, fb0);

    // Step j: multiply chunk j (registers ca/cb) while reading chunk j+1 into
    // na/nb and refilling chunk j's slot with chunk j+STAGES.  The first PRE
    // k-steps issue before the barrier, which guards only the refill and the
    // reads.
    static_assert(PRE >= 0 && PRE <= 4, "PRE k-steps of four");
    auto step = [&](int j, const float (&ca)[MB][4], const float (&cb)[NB][4], float (&na)[MB][4],
                    float (&nb)[NB][4]) {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));   // ca/cb landed
        mfma16_steps<MB, NB, 0, PRE>(acc, ca, cb);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(LOADS * (STAGES - 2)));
        __builtin_amdgcn_s_barrier();
        issue(j + STAGES);
        frags(j + 1, na, nb);
        mfma16_steps<MB, NB, PRE, 4>(acc, ca, cb);
    };
    int j = 0;
    for (; j + 2 < npass; j += 2) {
        step(j, fa0, fb0, fa1, fb1);
        step(j + 1, fa1, fb1, fa0, fb0);
    }
    if (j + 1 < npass) {
        step(j, fa0, fb0, fa1, fb1);
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int s = 0; s < 4; ++s) fa0[i][s] = fa1[i][s];
#pragma unroll
        for (int jb = 0; jb < NB; ++jb)
#pragma unroll
            for (int s = 0; s < 4; ++s) fb0[jb][s] = fb1[jb][s];
    }
    mfma16_steps<MB, NB, 0, 4>(acc, fa0, fb0);

    // The KG partial tiles in LDS, lane l, register r of block (i, jb)
    // holding C(16i + l%16, 16jb + 4(l/16) + r).  The refills past the end
    // must have landed and every wave must be past its fragment reads before
    // the ring is overwritten.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    __syncthreads();
    {
        const int g = lane >> 4, c = lane & 15;
        float* const red = smem + grp * BM * PITCH;
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int jb = 0; jb < NB; ++jb)
                *reinterpret_cast<f32x4*>(red + (ra + 16 * i + c) * PITCH + rb + 16 * jb + 4 * g) =
                    acc[i][jb];
    }
    __syncthreads();
    ksw_store<BM, BN, KG, NW * 64>(p, id, smem, m0, n0);
}

}  // namespace mtk

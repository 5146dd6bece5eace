// gemm_dlh_kernel.hpp -- implicit-GEMM convolution over an NCHW view whose
// im2col operand is built in LDS from a halo patch of the input (L_IMH).
//
// C[c_out, n*ho*wo] = W[c_out, kg] · im2col(x)[kg, n*ho*wo] with the OIHW
// weights' own K order k = (ci*kh + r)*kw + s, so A is the weight tensor as it
// lies (16-byte DMA ring of k-contiguous rows, as in gemm_f32_dl).  B is never
// gathered per K-chunk: the BN output pixels of a tile (consecutive in
// n*ho*wo order) read a band of input rows, the same band for every filter
// tap, so the workgroup copies that band -- 16 channels at a time, all padded
// columns, the padding and the rows between images as zeros -- into LDS once
// (4-byte DMA, one element per lane) and reads every tap's B fragment from
// it.  16 channels are 16*kh*kw consecutive k, i.e. kh*kw whole 16-deep
// chunks, so a patch serves kh*kw chunks; two patch buffers alternate, the
// next one loading while the current one is multiplied.
//
// Patch geometry (ConvGeom::hp, pw): padded row P(img, oh) = img*hp +
// oh*stride with hp = (ho-1)*stride + kh, padded column ow*stride, the
// window's element (r, s) at (P + r, ow*stride + s).  A tile's first output
// row fixes the band's first padded row R0; halo_rows() bounds its height
// for any tile, so a patch is 16 channel bands of halo_rows * pw floats
// (each rounded up to whole 64-element DMA instructions), at the same offset
// for every tile.  A lane's pixel has a fixed base (its window's top-left in
// the patch) and each k of a chunk an offset ch*plane + r*pw + s that is the
// same for every pixel, so a fragment read is one ds_read_b32 at base +
// offset.  The offsets come from a table in the kernel arguments (scalar
// loads): an LDS table read is ordered by the compiler after every DMA in
// flight, which serialised the A prefetch with the multiply, and decoding
// them per lane cost more vector instructions than the multiply hides.
//
// Reads the same operands and writes the same output and split-K partials as
// gemm_f32_dl with B = L_IMR, in 16-deep chunks with the permuted K order of
// gemm_kernel.hpp.  The order of the chunks differs when the K range ends in
// a partial chunk (c*kh*kw % 16 != 0): gemm_f32_dl multiplies that chunk
// first, this kernel last.  The two paths are therefore not bitwise equal in
// general (each is deterministic, and both are within the parity bound); the
// planner may switch between them (LDS limit, cost rule, forced
// configurations), and nothing relies on their bits agreeing.
#pragma once

#include "gemm_dl_kernel.hpp"

namespace mtk {

template <int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64)
gemm_f32_dlh(GemmParams p, HaloTable ht) {
    constexpr int WAVES_N = BN / WN;
    constexpr int NW = (BM / WM) * WAVES_N;
    constexpr int MB = WM / 32, NB = WN / 32;
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be 32-aligned");
    static_assert(16 % NW == 0, "a patch's 16 channels must split evenly over the waves");
    using TA = DlTile<L_KV, BM, NW>;
    constexpr int RING = 2 * TA::floats;   // two slots
    constexpr int STAGING = 1024 * NW;     // the epilogue: one block column per pass
    extern __shared__ float smem[];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int ra = wm * WM, rb = wn * WN;

    const TileId id = tile_id(p);
    const int m0 = id.tm * BM, n0 = id.tn * BN;
    const int k_begin = id.split * p.k_per_split;
    const int k_end = min(p.K, k_begin + p.k_per_split);
    const int klen = k_end > k_begin ? k_end - k_begin : 0;
    const int nk = (klen + 15) >> 4;          // chunks, the last one possibly partial
    const float* Ab = p.A + (int64_t)id.bz * p.a_b;

    const ConvGeom& g = p.cv;
    const int khw = g.kh * g.kw;
    const int pw = g.pw, hp = g.hp;
    const int plane = halo_rows(g, BN) * pw;  // floats of one channel's band
    const int cst = halo_chan_stride(g, BN);  // floats between channels in a patch
    const int ipc = cst >> 6;                 // DMA instructions per channel
    const int pst = 16 * cst;                 // floats between the two patches
    const int nimg = p.N / (g.ho * g.wo);
    float* const patch = smem + RING;

    // the band's first padded row: that of the tile's first output row
    const int gr0 = n0 / g.wo;
    const int img0 = gr0 / g.ho;
    const int R0 = img0 * hp + (gr0 - img0 * g.ho) * g.stride;
    const float* Xb = p.B + (int64_t)id.bz * p.b_b + (int64_t)img0 * g.img_stride;

    // this lane's window origin in the patch, per block column (pixels past N
    // read the last pixel's window: their columns are never stored)
    int base[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int n = min(n0 + rb + 32 * j + (lane & 31), p.N - 1);
        const int gr = n / g.wo, ow = n - gr * g.wo;
        const int img = gr / g.ho, oh = gr - img * g.ho;
        base[j] = (img * hp + oh * g.stride - R0) * pw + ow * g.stride;
    }

    // Element i*64 + lane of a channel's band: its offset from Xb in channel
    // 0 (32-bit: the host bounds the images a band spans), or -1 for the
    // padding, the rows between images, rows past the last image and the
    // surplus past the band.
    int soff[kHaloIpcMax];
#pragma unroll
    for (int i = 0; i < kHaloIpcMax; ++i) {
        soff[i] = -1;
        const int e = i * 64 + lane;
        if (i < ipc && e < plane) {
            const int prow = e / pw, pcol = e - prow * pw;
            const int R = R0 + prow;
            const int img = R / hp;
            const int ih = R - img * hp - g.pad, iw = pcol - g.pad_w;
            if (img < nimg && (unsigned)ih < (unsigned)g.h && (unsigned)iw < (unsigned)g.w)
                soff[i] = (img - img0) * (int)g.img_stride + ih * (int)g.sh + iw * (int)g.sw;
        }
    }

    f32x16 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Patch of channels 16*G .. 16*G+15 into dst, channel ch at dst + ch*cst,
    // moved by wave ch % NW: one 4-byte DMA per lane and band row of 64,
    // the zero page where soff says so or past c.
    auto issue_patch = [&](int G, float* dst) {
#pragma unroll
        for (int jj = 0; jj < 16 / NW; ++jj) {
            const int ch = wave + NW * jj;
            const int c = G * 16 + ch;
            const bool cok = c < g.c;
            const float* xc = Xb + (int64_t)(cok ? c : 0) * g.sc;
            float* d = dst + ch * cst;
#pragma unroll
            for (int i = 0; i < kHaloIpcMax; ++i)
                if (i < ipc) {
                    const float* src = cok && soff[i] >= 0 ? xc + soff[i] : dl_zero_page;
                    __builtin_amdgcn_global_load_lds(
                        (const void __attribute__((address_space(1)))*)src,
                        (void __attribute__((address_space(3)))*)(d + i * 64), 4, 0, 0);
                }
        }
    };

    // B fragments of the chunk at position q of patch buffer pb: the 8 k of
    // this lane are 16*q + 8*(lane/32) + s in the patch, at the offsets of
    // the argument table (scalar loads; each half of the wave selects its
    // eight).  No k needs masking: a split's K range ends on a chunk
    // boundary except at K itself, and the k of the last chunk past K are
    // channels past c, which the patch holds as zeros (A is zero there too).
    const bool hi = lane >= 32;
    auto frag_b = [&](int q, const float* pb, float (&fb)[NB][8]) {
        const int* tq = ht.off + 16 * q;
        int off[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            // both halves' offsets as scalars, then a per-lane select (a
            // select of the addresses would turn the loads into vector ones)
            const int lo = __builtin_amdgcn_readfirstlane(tq[s]);
            const int up = __builtin_amdgcn_readfirstlane(tq[8 + s]);
            off[s] = hi ? up : lo;
        }
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int s = 0; s < 8; ++s) fb[j][s] = pb[base[j] + off[s]];
    };

    DlLoader<L_KV, BM, NW> la;
    la.init(Ab, p.a_mn, p.a_k, p.M, m0, k_begin, wave, lane);
    auto issue_a = [&](int chunk) {
        float* st = smem + (chunk & 1) * TA::floats;
        if (klen - chunk * 16 >= 16) la.issue(st, chunk, wave);
        else la.issue_bounded(st, chunk, wave, klen);
    };

    const int J0 = k_begin >> 4;              // global index of the first chunk
    const int Gf = J0 / khw;                  // its patch
    const int Gl = nk > 0 ? (J0 + nk - 1) / khw : Gf;
    // APF: the A fragments are also read a chunk ahead (A's DMA then runs two
    // chunks ahead, in the slot whose fragments are already in registers).
    // It pays for wave tiles of at most two 32x32 blocks, whose few MFMAs per
    // chunk cannot cover the A reads after the barrier (128x128 tiles: 53.1
    // against 55.3 us for a c_in 120 3x3 layer); for four blocks it was
    // slower (256x128: 84.9 against 84.2 us, c_in 252).
    constexpr bool APF = MB * NB <= 2;
    if (nk > 0) {
        issue_patch(Gf, patch);
        if (Gl > Gf) issue_patch(Gf + 1, patch + pst);
        issue_a(0);
        if (APF && nk > 1) issue_a(1);
    }

    // The B fragments of chunk kt+1 are read while chunk kt is multiplied:
    // with kh*kw >= 2 (the host's condition) the patch of chunk kt+1 is the
    // current one, or the next one, issued at the first chunk of the current
    // patch (at least one barrier ago) or in the prologue; and the buffer a
    // patch DMA refills (that of patch G-1, at the first chunk of G) was last
    // read before that chunk's barrier.  After the last chunk the read is of
    // no use but stays inside the buffers.  Two fragment sets alternate.
    int q_in = J0 - Gf * khw;                 // chunk index within its patch
    int G = Gf;
    constexpr int NMF = 8 * MB * NB, NRA = 2 * MB, NRB = 8 * NB;
    float fa0[MB][8], fa1[MB][8], fb0[NB][8], fb1[NB][8];
    if constexpr (APF) {
        // chunk 0's fragments; A(1) has landed too, for the first step
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
        __builtin_amdgcn_s_barrier();
        dl_frags<L_KV, BM, MB>(smem, ra, lane, fa0);
        frag_b(q_in, patch, fb0);
    }
    auto step = [&](int kt, float (&fac)[MB][8], float (&fbc)[NB][8], float (&fan)[MB][8],
                    float (&fbn)[NB][8]) {
        // Everything issued so far has landed (nothing newer is in flight),
        // then everyone's; the barrier also retires every wave's reads of the
        // A slot and of the patch buffer refilled below.
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
        __builtin_amdgcn_s_barrier();
        if constexpr (APF) {
            if (kt + 2 < nk) issue_a(kt + 2);
        } else {
            if (kt + 1 < nk) issue_a(kt + 1);
        }
        if (kt > 0 && q_in == 0 && G < Gl) issue_patch(G + 1, patch + ((G + 1 - Gf) & 1) * pst);
        if constexpr (!APF) {
            if (kt == 0) frag_b(q_in, patch, fbc);
            dl_frags<L_KV, BM, MB>(smem + (kt & 1) * TA::floats, ra, lane, fac);
        }
        if (++q_in == khw) {
            q_in = 0;
            ++G;
        }
        if constexpr (APF) dl_frags<L_KV, BM, MB>(smem + ((kt + 1) & 1) * TA::floats, ra, lane, fan);
        frag_b(q_in, patch + ((G - Gf) & 1) * pst, fbn);
        mfma_chunk<MB, NB>(acc, fac, fbc);
        // Interleave the next chunk's fragment reads (and their address
        // arithmetic) with this chunk's MFMAs, after this chunk's own A reads
        // (without APF), so that they run in the MFMAs' shadow.
        if constexpr (APF && NMF >= NRA + NRB) {
#pragma unroll
            for (int i = 0; i < NRA; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        } else {
            __builtin_amdgcn_sched_group_barrier(0x100, NRA, 0);
        }
#pragma unroll
        for (int i = 0; i < NRB; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        constexpr int rest = NMF - NRB - (APF && NMF >= NRA + NRB ? NRA : 0);
        if constexpr (rest > 0) __builtin_amdgcn_sched_group_barrier(0x008, rest, 0);
    };
    for (int kt = 0; kt < nk; kt += 2) {
        step(kt, fa0, fb0, fa1, fb1);
        if (kt + 1 < nk) step(kt + 1, fa1, fb1, fa0, fb0);
    }

    store_tile_lds<MB, NB, NW, WAVES_N, WM, WN, STAGING>(p, acc, smem, m0, n0, wave, lane,
                                                          id.split, id.bz);
}

}  // namespace mtk

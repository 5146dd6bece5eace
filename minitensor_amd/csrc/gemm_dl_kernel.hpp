// gemm_dl_kernel.hpp -- fp32 MFMA GEMM whose operand tiles travel from HBM
// straight into LDS (gfx950 global_load_lds_dwordx4), for operands with a
// 16-byte vector layout (L_KV or L_MV).
//
// Same mathematics, tile mapping and epilogue as gemm_f32_mfma; the difference
// is the data path:
//   * No VGPR staging.  Each wave instruction moves 64 lanes x 16 B = 1 KB of
//     one operand tile into LDS asynchronously, so the loads cost neither
//     registers nor the issue slots of a register -> ds_write round trip, and
//     the number of K-chunks in flight is limited only by LDS.
//   * K advances in chunks of 16 through a ring of STAGES LDS slots: while
//     chunk kt is multiplied, chunks kt+1 .. kt+STAGES-1 are in flight.  One
//     s_barrier per chunk; each wave first waits (vmcnt) only for its own
//     instructions of chunk kt, since the later ones may still be landing.
//   * LDS tiles are unpadded (the DMA writes 1 KB contiguous per
//     instruction):  k-contiguous operands -> [BMN][16], with the four 16-B
//     k-groups of row r stored at position g ^ ((r >> 2) & 3), so that the
//     fragment reads (two ds_read_b128 per lane, 16 rows per LDS cycle at
//     stride 64 B) hit every bank once;  mn-contiguous operands -> [16][BMN].
//   * Rows beyond M (or N) read a clamped, valid row: their products only
//     reach output rows/columns that the epilogue never writes.
//   * A K range that is not a multiple of 16 ends in a partial chunk.  It is
//     fetched first, with bounds-checked scalar loads that write zeros past
//     k_end, into the last ring slot (which the prologue leaves free), and
//     multiplied before the pipelined loop starts; the prologue's DMA
//     overlaps it.
// K permutation, MFMA operand layouts and the accumulator layout are the ones
// documented in gemm_kernel.hpp.
#pragma once

#include <type_traits>

#include "gemm_kernel.hpp"

namespace mtk {

// Geometry of one 16-deep K-chunk of an operand tile with BMN rows, moved by
// NW waves: 16 B per lane (global_load_lds_dwordx4), 256 floats per wave
// instruction.  The implicit-im2col operand uses the k-contiguous tile.
template <int L, int BMN, int NW>
struct DlTile {
    static_assert(L == L_KV || L == L_MV || L == L_IM || L == L_IMW || L == L_IMR,
                  "direct-to-LDS needs a DMA layout");
    static constexpr bool kc = (L == L_KV || L == L_IM);
    static constexpr int floats = BMN * 16;
    static constexpr int insts = floats / 256;
    static_assert(insts % NW == 0, "tile must split evenly over the waves");
    static constexpr int per_wave = insts / NW;
};

// Position (in 16-B groups) of k-group g of row r inside a k-contiguous tile
// is g ^ kswz(r).  The 32x32-block fragment read (lane l: row l%32, k-group
// 2*(l/32) or 2*(l/32)+1) then takes 4 LDS cycles per ds_read_b128 on gfx950,
// the conflict-free rate (64 lanes x 16 B at 256 B per cycle); without the
// swizzle it takes 8.
__device__ __forceinline__ int kswz(int r) { return (r >> 2) & 3; }
// The 16x16-block fragment read of gemm_f32_dl16 (lane l: row l%16 of a
// block, k-group l/16: the four 16-lane groups read the four k-groups of the
// same 16 rows) takes 8 cycles with kswz and 4 with kswz16.  Measured with
// SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE on read patterns in isolation;
// no plain bank model (lanes served in fixed groups of 8 or 16, 32 or 64
// banks) reproduces both results, so the swizzles are chosen by measurement.
// SW selects kswz16 in the loaders.
__device__ __forceinline__ int kswz16(int r) { return (r >> 1) & 3; }
template <int SW>
__device__ __forceinline__ int kswz_sel(int r) { return SW == 0 ? kswz(r) : kswz16(r); }

// Zero source for lanes whose 16 bytes fall in the padding, beyond N, or past
// the end of the K range: the DMA writes every lane, so those lanes read 16
// bytes of zeros.
static __device__ const float __attribute__((aligned(16))) dl_zero_page[4] = {0.f, 0.f, 0.f,
                                                                              0.f};

// n / d for 0 <= n < 2^31 and d >= 1 with a double reciprocal rd = 1/d and
// one upward correction (the product is within 2^-52 relative of n/d, so its
// truncation is the quotient or one less, never more): a few vector
// instructions where the integer division costs about thirty.
__device__ __forceinline__ int div_by(int n, int d, double rd) {
    int q = (int)((double)n * rd);
    q += n - q * d >= d;
    return q;
}

template <int L, int BMN, int NW, int SW = 0>
struct DlLoader {
    using T = DlTile<L, BMN, NW>;
    const float* src[T::per_wave];   // this lane's source for each instruction, chunk 0
    int kofs[T::per_wave];            // k of this lane's 16 bytes within a chunk
    int64_t kstep;                    // elements between consecutive K-chunks

    // X points at element (0, 0) of the operand (batch applied); mn0/k0 are the
    // tile's first row and first k.  MN % 4 == 0 for L_MV (checked on the host).
    __device__ __forceinline__ void init(const float* X, int64_t s_mn, int64_t s_k, int MN,
                                         int mn0, int k0, int wave, int lane) {
        kstep = 16 * s_k;
#pragma unroll
        for (int j = 0; j < T::per_wave; ++j) {
            const int q = j * NW + wave;                  // instruction index within the chunk
            if constexpr (T::kc) {
                // 16 rows x 4 groups of 4 k per instruction; lane -> (row, slot).
                const int r = q * 16 + (lane >> 2);
                const int g = (lane & 3) ^ kswz_sel<SW>(r);   // k-group that lands in slot lane&3
                const int64_t row = min((int64_t)mn0 + r, (int64_t)MN - 1);
                src[j] = X + row * s_mn + (int64_t)(k0 + g * 4) * s_k;
                kofs[j] = g * 4;
            } else {
                const int e = q * 256 + lane * 4;         // float index within [16][BMN]
                const int kr = e / BMN, mn = e - kr * BMN;
                const int64_t col = min((int64_t)mn0 + mn, (int64_t)MN - 4);
                src[j] = X + (int64_t)(k0 + kr) * s_k + col;
                kofs[j] = kr;
            }
        }
    }

    // Issue the DMA of K-chunk `chunk` into the LDS tile at `tile`.
    __device__ __forceinline__ void issue(float* tile, int chunk, int wave) const {
#pragma unroll
        for (int j = 0; j < T::per_wave; ++j) {
            const int q = j * NW + wave;
            __builtin_amdgcn_global_load_lds(
                (const void __attribute__((address_space(1)))*)(src[j] + chunk * kstep),
                (void __attribute__((address_space(3)))*)(tile + q * 256), 16, 0, 0);
        }
    }

    // As issue(), for a chunk that may reach past the end of the K range
    // (klen elements from the k0 given to init): lanes whose 16 bytes start at
    // or past klen load zeros.  A lane's 16 bytes never straddle the end: an
    // L_KV operand has K % 4 == 0 and splits start at multiples of 16, and an
    // L_MV lane reads one k.
    __device__ __forceinline__ void issue_bounded(float* tile, int chunk, int wave, int klen) const {
#pragma unroll
        for (int j = 0; j < T::per_wave; ++j) {
            const int q = j * NW + wave;
            // chunk * 16 < klen for every chunk issued, so this cannot overflow
            const float* s = kofs[j] < klen - chunk * 16 ? src[j] + chunk * kstep : dl_zero_page;
            __builtin_amdgcn_global_load_lds(
                (const void __attribute__((address_space(1)))*)s,
                (void __attribute__((address_space(3)))*)(tile + q * 256), 16, 0, 0);
        }
    }
};

// A operand of layout L_KVI (the convolution weight gradient's dY, read in
// NCHW): k-contiguous rows that restart every a_hw k at the next image, in
// the L_KV tile layout.  A lane's 16 bytes are four consecutive k of one
// image (the host guarantees a_hw % 4 == 0, K % 16 == 0 and 16-byte aligned
// rows and images), so its source is the image (div_by) plus the row plus
// k % a_hw, recomputed from the chunk index on every issue (a re-fetched
// chunk reads the same bytes).
template <int BMN, int NW>
struct DlKviLoader {
    using T = DlTile<L_KV, BMN, NW>;
    const float* row[T::per_wave];   // X + row*a_mn of each instruction's row
    int kofs[T::per_wave];           // k of this lane's 16 bytes within a chunk
    int k0, hw;
    double rhw;
    int64_t img;

    __device__ __forceinline__ void init(const GemmParams& p, const float* X, int MN, int mn0,
                                         int kb, int wave, int lane) {
        k0 = kb;
        hw = p.a_hw;
        rhw = 1.0 / (double)p.a_hw;
        img = p.a_img;
#pragma unroll
        for (int j = 0; j < T::per_wave; ++j) {
            const int q = j * NW + wave;
            const int r = q * 16 + (lane >> 2);
            const int g = (lane & 3) ^ kswz(r);
            const int64_t rr = min((int64_t)mn0 + r, (int64_t)MN - 1);
            row[j] = X + rr * p.a_mn;
            kofs[j] = g * 4;
        }
    }

    __device__ __forceinline__ void issue(float* tile, int chunk, int wave) const {
#pragma unroll
        for (int j = 0; j < T::per_wave; ++j) {
            const int q = j * NW + wave;
            const int k = k0 + chunk * 16 + kofs[j];
            const int im = div_by(k, hw, rhw);
            const float* src = row[j] + (int64_t)im * img + (k - im * hw);
            __builtin_amdgcn_global_load_lds(
                (const void __attribute__((address_space(1)))*)src,
                (void __attribute__((address_space(3)))*)(tile + q * 256), 16, 0, 0);
        }
    }
};

// Bounds-checked fetch of the partial chunk [kt0, k_end) of one operand tile,
// zero past k_end, in the same LDS layout as the DMA path.
template <int L, int BMN, int NT>
struct DlTail {
    static constexpr int NI = BMN * 16 / NT;
    static_assert(NI * NT == BMN * 16, "tail must split evenly over the threads");
    float v[NI];

    __device__ __forceinline__ void load(const float* X, int64_t s_mn, int64_t s_k, int MN,
                                         int mn0, int kt0, int k_end, int t) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int e = t + i * NT;
            int r, kk;
            if constexpr (L == L_KV) { r = e >> 4; kk = e & 15; }
            else { kk = e / BMN; r = e - kk * BMN; }
            const int64_t row = min((int64_t)mn0 + r, (int64_t)MN - 1);
            v[i] = (kt0 + kk < k_end) ? X[row * s_mn + (int64_t)(kt0 + kk) * s_k] : 0.f;
        }
    }

    __device__ __forceinline__ void store(float* tile, int t) const {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int e = t + i * NT;
            if constexpr (L == L_KV) {
                const int r = e >> 4, kk = e & 15;
                tile[r * 16 + ((((kk >> 2) ^ kswz(r))) << 2) + (kk & 3)] = v[i];
            } else {
                tile[e] = v[i];
            }
        }
    }
};

// Implicit im2col of a channels-last input as the B operand, in the
// k-contiguous tile layout of L_KV ([BMN][16], k-groups swizzled).  Lane
// (row r, group g) of an instruction loads channels ci0 + 4g' .. +3 (g' the
// k-group stored at g) of output pixel n0 + r at the chunk's filter tap
// (rt, st): 16 contiguous, 16-byte aligned bytes of xt, or the zero page when
// the tap falls in the padding or n >= N.  The tap and channel offset are the
// same for every lane (scalar registers, the wave index is uniform) and step
// through (rt, st, ci0) once per chunk; per lane only the bounds test and one
// address add remain.  Chunks must be issued in order 0, 1, 2, ... (STEP > 1:
// each issue advances STEP chunks, for a loader that takes every STEP-th
// chunk).  Rows at or past VR (a tile padded to whole DMA instructions) read
// zeros.
template <int BMN, int NW, int VR = BMN, int STEP = 1, int SW = 0>
struct DlImLoader {
    using T = DlTile<L_IM, BMN, NW>;
    const float* pix[T::per_wave];   // xt + img*img_stride + (ih0*w + iw0)*c + 4g
    int ih0[T::per_wave], iw0[T::per_wave];
    int rt, st, ci0;                 // filter tap and first channel of the next chunk
    int c, h, w, kw;

    __device__ __forceinline__ void init(const GemmParams& p, const float* X, int n0, int k0,
                                         int /*kend*/, int wave, int lane) {
        const ConvGeom& g = p.cv;
        c = g.c; h = g.h; w = g.w; kw = g.kw;
        const int hw = g.ho * g.wo;
#pragma unroll
        for (int j = 0; j < T::per_wave; ++j) {
            const int r = (j * NW + wave) * 16 + (lane >> 2);
            const int grp = (lane & 3) ^ kswz_sel<SW>(r);
            const int n = n0 + r;
            const int img = n / hw, rem = n - img * hw;
            const int oh = rem / g.wo, ow = rem - oh * g.wo;
            ih0[j] = n < p.N && r < VR ? oh * g.stride - g.pad : -(1 << 30);   // past N: zeros
            iw0[j] = ow * g.stride - g.pad_w;
            pix[j] = X + (int64_t)img * g.img_stride +
                     ((int64_t)ih0[j] * g.w + iw0[j]) * g.c + grp * 4;
        }
        const int tap = k0 / g.c;
        ci0 = k0 - tap * g.c;
        rt = tap / g.kw;
        st = tap - rt * g.kw;
    }

    __device__ __forceinline__ void issue(float* tile, int /*chunk*/, int wave) {
        const int64_t toff = ((int64_t)rt * w + st) * c + ci0;
#pragma unroll
        for (int j = 0; j < T::per_wave; ++j) {
            const int q = j * NW + wave;
            const bool ok = (unsigned)(ih0[j] + rt) < (unsigned)h &&
                            (unsigned)(iw0[j] + st) < (unsigned)w;
            const float* src = ok ? pix[j] + toff : dl_zero_page;
            __builtin_amdgcn_global_load_lds(
                (const void __attribute__((address_space(1)))*)src,
                (void __attribute__((address_space(3)))*)(tile + q * 256), 16, 0, 0);
        }
#pragma unroll
        for (int a = 0; a < STEP; ++a) {   // next chunk (c % 16 == 0)
            ci0 += 16;
            if (ci0 == c) {
                ci0 = 0;
                if (++st == kw) { st = 0; ++rt; }
            }
        }
    }
};

// Implicit im2col of an NCHW view (any strides) as the B operand (L_IMR), in
// the K order (ci, r, s) of OIHW weights, so that A is the weight tensor
// itself.  The tile is the n-contiguous [16][BN] one of L_MV, filled by 4-byte
// DMA (global_load_lds_dword): one wave instruction moves one k-row of 64
// consecutive output pixels, which read mostly contiguous runs of an input
// row.  Each lane keeps the same pixel for all its instructions (NW is a
// multiple of BN/64), so the per-lane state is that pixel's window; the k-row
// of an instruction is wave-uniform, so its tap (r, s) and element offset
// c*sc + r*sh + s*sw are scalar state, stepped by 16 k per chunk with
// additions (chunks are issued in order 0, 1, 2, ...; issue_tail decodes the
// partial last chunk).  Per instruction a lane only tests its window against
// the image and selects its address; a tap in the padding, a pixel past N or
// (tail) a k past the K range reads the zero page.
template <int BN, int NW>
struct DlImrLoader {
    static constexpr int INSTS = BN * 16 / 64;   // 4-byte DMA instructions per chunk
    static constexpr int per_wave = INSTS / NW;
    static_assert(per_wave * NW == INSTS, "instructions must split evenly over the waves");
    static_assert(NW % (BN / 64) == 0, "a lane keeps one pixel for all its instructions");
    const float* pix;        // input + img*img_stride + ih0*sh + iw0*sw of the lane's pixel
    int ih0, iw0;            // the window's top-left input row / column (far negative past N)
    int kr[per_wave];        // k-row of each instruction within a chunk: wave-uniform
    int r[per_wave], s[per_wave];   // tap of each instruction's k in the next chunk
    int64_t off[per_wave];          // c*sc + r*sh + s*sw of that k
    int k0, k_end, kh, kw, h, w, dr, ds;
    int64_t sc, sh, sw;
    int64_t step, carry_s, carry_r;   // offset steps: 16 k; s wraps; r wraps

    __device__ __forceinline__ void decode(int k, int& c_, int& r_, int& s_) const {
        const int khw = kh * kw;
        c_ = k / khw;
        const int tap = k - c_ * khw;
        r_ = tap / kw;
        s_ = tap - r_ * kw;
    }

    __device__ __forceinline__ void init(const GemmParams& p, const float* X, int n0, int kbegin,
                                         int kend, int wave, int lane) {
        const ConvGeom& g = p.cv;
        kh = g.kh; kw = g.kw; h = g.h; w = g.w;
        sc = g.sc; sh = g.sh; sw = g.sw;
        k0 = kbegin;
        k_end = kend;
        // one chunk (16 k) in mixed radix (c, r, s)
        const int khw = kh * kw;
        const int dci = 16 / khw;
        dr = (16 - dci * khw) / kw;
        ds = 16 - dci * khw - dr * kw;
        step = dci * sc + dr * sh + ds * sw;
        carry_s = sh - kw * sw;
        carry_r = sc - kh * sh;
        int n = n0 + 64 * (wave % (BN / 64)) + lane;
        const bool nok = n < p.N;
        if (!nok) n = p.N - 1;
        const int hw = g.ho * g.wo;
        const int img = n / hw, rem = n - img * hw;
        const int oh = rem / g.wo, ow = rem - oh * g.wo;
        ih0 = nok ? oh * g.stride - g.pad : -(1 << 29);
        iw0 = ow * g.stride - g.pad_w;
        pix = X + (int64_t)img * g.img_stride + (int64_t)(oh * g.stride - g.pad) * sh +
              (int64_t)iw0 * sw;
#pragma unroll
        for (int j = 0; j < per_wave; ++j) {
            kr[j] = (j * NW + wave) / (BN / 64);
            int c_;
            decode(k0 + kr[j], c_, r[j], s[j]);
            off[j] = c_ * sc + r[j] * sh + s[j] * sw;
        }
    }

    __device__ __forceinline__ const float* source(int r_, int s_, int64_t o) const {
        const bool ok = (unsigned)(ih0 + r_) < (unsigned)h && (unsigned)(iw0 + s_) < (unsigned)w;
        return ok ? pix + o : dl_zero_page;
    }

    __device__ __forceinline__ static void dma(const float* src, float* dst) {
        __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)src,
                                         (void __attribute__((address_space(3)))*)dst, 4, 0, 0);
    }

    // Issue the DMA of the next whole chunk in order (every k inside the K
    // range), then step the taps and offsets by 16 k.
    __device__ __forceinline__ void issue(float* tile, int /*chunk*/, int wave) {
#pragma unroll
        for (int j = 0; j < per_wave; ++j) {
            dma(source(r[j], s[j], off[j]), tile + (j * NW + wave) * 64);
            // carries as masks (all-ones when s or r wraps): scalar arithmetic
            int s2 = s[j] + ds, r2 = r[j] + dr;
            const int ms = (kw - 1 - s2) >> 31;
            s2 -= kw & ms;
            r2 -= ms;
            const int mr = (kh - 1 - r2) >> 31;
            r2 -= kh & mr;
            s[j] = s2; r[j] = r2;
            off[j] += step + (carry_s & (int64_t)ms) + (carry_r & (int64_t)mr);
        }
    }

    // The DMA of chunk `chunk` (the partial last one): k past k_end reads
    // zeros.  The stepped state is untouched.
    __device__ __forceinline__ void issue_tail(float* tile, int chunk, int wave) const {
#pragma unroll
        for (int j = 0; j < per_wave; ++j) {
            const int k = k0 + chunk * 16 + kr[j];
            int c_, r_, s_;
            decode(k, c_, r_, s_);
            const float* src = source(r_, s_, c_ * sc + r_ * sh + s_ * sw);
            dma(k < k_end ? src : dl_zero_page, tile + (j * NW + wave) * 64);
        }
    }
};

// Implicit im2colᵀ of a channels-last input as the B operand of the
// convolution weight gradient (L_IMW), tile [16][BMN] (n contiguous, the L_MV
// LDS layout).  A lane of instruction q covers k-row kr = (q*256 + 4*lane) / BMN
// and the four columns n .. n+3 at (q*256 + 4*lane) % BMN: four consecutive
// channels of one filter tap, i.e. 16 contiguous, 16-byte aligned bytes of xt
// at the output pixel k, or the zero page when the tap falls in the padding,
// n >= N or k >= k_end.  The column part (tap offsets, channel) is decoded
// once; the output pixel (img, oh, ow) of k is decoded per chunk.
template <int BMN, int NW>
struct DlImwLoader {
    using T = DlTile<L_IMW, BMN, NW>;
    const float* X;
    int kr[T::per_wave];          // k-row of each instruction within a chunk
    int dr[T::per_wave], ds[T::per_wave], ci[T::per_wave];   // tap - pad, channel
    bool nok[T::per_wave];        // column inside N
    int k0, k_end;
    double rhw, rwo;              // 1 / (ho*wo), 1 / wo
    ConvGeom g;

    __device__ __forceinline__ void init(const GemmParams& p, const float* Xt, int n0, int kb,
                                         int kend, int wave, int lane) {
        g = p.cv;
        X = Xt;
        k0 = kb;
        k_end = kend;
        rhw = 1.0 / (double)(g.ho * g.wo);
        rwo = 1.0 / (double)g.wo;
#pragma unroll
        for (int j = 0; j < T::per_wave; ++j) {
            const int e = (j * NW + wave) * 256 + lane * 4;
            kr[j] = e / BMN;
            const int n = n0 + (e - kr[j] * BMN);
            nok[j] = n < p.N;
            const int tap = n / g.c;
            ci[j] = n - tap * g.c;
            const int r = tap / g.kw;
            dr[j] = r - g.pad;
            ds[j] = (tap - r * g.kw) - g.pad_w;
        }
    }

    __device__ __forceinline__ void issue(float* tile, int chunk, int wave) const {
        const int hw = g.ho * g.wo;
#pragma unroll
        for (int j = 0; j < T::per_wave; ++j) {
            const int q = j * NW + wave;
            const int k = k0 + chunk * 16 + kr[j];
            const int img = div_by(k, hw, rhw), rem = k - img * hw;
            const int oh = div_by(rem, g.wo, rwo), ow = rem - oh * g.wo;
            const int ih = oh * g.stride + dr[j], iw = ow * g.stride + ds[j];
            const bool ok = nok[j] && k < k_end && (unsigned)ih < (unsigned)g.h &&
                            (unsigned)iw < (unsigned)g.w;
            const float* src =
                ok ? X + (int64_t)img * g.img_stride + ((int64_t)ih * g.w + iw) * g.c + ci[j]
                   : dl_zero_page;
            __builtin_amdgcn_global_load_lds(
                (const void __attribute__((address_space(1)))*)src,
                (void __attribute__((address_space(3)))*)(tile + q * 256), 16, 0, 0);
        }
    }
};

// Bounds-checked fetch of the partial chunk [kt0, k_end) of the L_IMW operand
// into the [16][BMN] layout.
template <int BMN, int NT>
struct DlImwTail {
    static constexpr int NI = BMN * 16 / NT;
    static_assert(NI * NT == BMN * 16, "tail must split evenly over the threads");
    float v[NI];

    __device__ __forceinline__ void load(const GemmParams& p, const float* X, int n0, int kt0,
                                         int k_end, int t) {
        const ConvGeom& g = p.cv;
        const int hw = g.ho * g.wo;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int e = t + i * NT;
            const int kk = e / BMN, n = n0 + (e - kk * BMN), k = kt0 + kk;
            float x = 0.f;
            if (k < k_end && n < p.N) {
                const int img = k / hw, rem = k - img * hw;
                const int oh = rem / g.wo, ow = rem - oh * g.wo;
                const int tap = n / g.c, c = n - tap * g.c;
                const int r = tap / g.kw, s = tap - r * g.kw;
                const int ih = oh * g.stride - g.pad + r, iw = ow * g.stride - g.pad_w + s;
                if ((unsigned)ih < (unsigned)g.h && (unsigned)iw < (unsigned)g.w)
                    x = X[(int64_t)img * g.img_stride + ((int64_t)ih * g.w + iw) * g.c + c];
            }
            v[i] = x;
        }
    }

    __device__ __forceinline__ void store(float* tile, int t) const {
#pragma unroll
        for (int i = 0; i < NI; ++i) tile[t + i * NT] = v[i];
    }
};

// The 8 k-values (permuted order) of one 32-row MFMA block from a chunk tile.
template <int L, int BMN>
__device__ __forceinline__ void dl_frag(const float* tile, int row0, int lane, float (&f)[8]) {
    const int h = lane >> 5, c = lane & 31;
    if constexpr (L == L_KV) {
        const int r = row0 + c;
        const float* rp = tile + r * 16;
        const f32x4 x = *reinterpret_cast<const f32x4*>(rp + (((2 * h) ^ kswz(r)) * 4));
        const f32x4 y = *reinterpret_cast<const f32x4*>(rp + (((2 * h + 1) ^ kswz(r)) * 4));
        f[0] = x[0]; f[1] = x[1]; f[2] = x[2]; f[3] = x[3];
        f[4] = y[0]; f[5] = y[1]; f[6] = y[2]; f[7] = y[3];
    } else {
        const float* q = tile + (h * 8) * BMN + row0 + c;
#pragma unroll
        for (int s = 0; s < 8; ++s) f[s] = q[s * BMN];
    }
}

template <int MB, int NB>
__device__ __forceinline__ void mfma_chunk(f32x16 (&acc)[MB][NB], const float (&fa)[MB][8],
                                           const float (&fb)[NB][8]) {
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j)
                acc[i][j] = mfma_32x32x2(fa[i][s], fb[j][s], acc[i][j]);
}

template <int L, int BMN, int MB>
__device__ __forceinline__ void dl_frags(const float* tile, int row0, int lane, float (&f)[MB][8]) {
#pragma unroll
    for (int i = 0; i < MB; ++i) dl_frag<L, BMN>(tile, row0 + i * 32, lane, f[i]);
}

// RS: also produce the row sums of A (GemmParams::rowsum); a separate
// instantiation so the other kernels do not pay its registers.
template <int BM, int BN, int WM, int WN, int LA, int LB, int STAGES, bool RS = false>
__global__ void __launch_bounds__((BM / WM) * (BN / WN) * 64)
gemm_f32_dl(GemmParams p) {
    constexpr int WAVES_N = BN / WN;
    constexpr int NW = (BM / WM) * WAVES_N;
    constexpr int NT = NW * 64;
    constexpr int MB = WM / 32, NB = WN / 32;
    static_assert(STAGES >= 2, "the ring needs at least two slots");
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be 32-aligned");
    constexpr bool kvi = (LA == L_KVI);   // A split into images (no partial chunks)
    constexpr int LAF = kvi ? L_KV : LA;  // LDS layout of A's tile
    using TA = DlTile<LAF, BM, NW>;
    using TB = DlTile<LB, BN, NW>;
    constexpr bool imr = (LB == L_IMR);   // B moved by 4-byte DMA
    constexpr int STAGE = TA::floats + TB::floats;
    // DMA instructions per wave per chunk
    constexpr int LOADS = TA::per_wave + (imr ? DlImrLoader<BN, NW>::per_wave : TB::per_wave);
    static_assert(LOADS * (STAGES - 2) < 64, "vmcnt holds at most 63");
    __shared__ __attribute__((aligned(1024))) float smem[STAGES * STAGE];

    const int t = threadIdx.x;
    const int lane = t & 63;
    // Uniform across the wave: keeps per-wave loader state and LDS (M0)
    // addresses in scalar registers.
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int ra = wm * WM, rb = wn * WN;     // this wave's first row in the A / B tile

    const TileId id = tile_id(p);
    const int m0 = id.tm * BM, n0 = id.tn * BN;
    const int k_begin = id.split * p.k_per_split;
    const int k_end = min(p.K, k_begin + p.k_per_split);
    const int klen = k_end > k_begin ? k_end - k_begin : 0;
    const int nk = klen >> 4;                 // full chunks
    // The channels-last implicit operand has c % 16 == 0, so its K ranges
    // hold whole chunks.
    const bool tail = LB != L_IM && (klen & 15) != 0;
    const float* Ab = p.A + (int64_t)id.bz * p.a_b;
    const float* Bb = p.B + (int64_t)id.bz * p.b_b;

    f32x16 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    constexpr bool im = (LB == L_IM);
    constexpr bool imw = (LB == L_IMW);
    constexpr int LBF = im ? L_KV : (imw || imr) ? L_MV : LB;   // LDS layout of B's tile
    // Fused row sums of A: the waves of the first wave column of the first
    // tile column see every A fragment of their rows exactly once.
    const bool do_rs = RS && id.tn == 0 && wn == 0;
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

    DlTail<LAF, BM, NT> ta;
    std::conditional_t<imw, DlImwTail<BN, NT>, DlTail<LBF, BN, NT>> tb;
    std::conditional_t<kvi, DlKviLoader<BM, NW>, DlLoader<LA, BM, NW>> la;
    std::conditional_t<
        im, DlImLoader<BN, NW>,
        std::conditional_t<imw, DlImwLoader<BN, NW>,
                           std::conditional_t<imr, DlImrLoader<BN, NW>, DlLoader<LBF, BN, NW>>>>
        lb;
    if constexpr (kvi) la.init(p, Ab, p.M, m0, k_begin, wave, lane);
    else la.init(Ab, p.a_mn, p.a_k, p.M, m0, k_begin, wave, lane);
    if constexpr (im || imw || imr) lb.init(p, Bb, n0, k_begin, k_end, wave, lane);
    else lb.init(Bb, p.b_mn, p.b_k, p.N, n0, k_begin, wave, lane);
    if (tail) {
        const int kt0 = k_begin + nk * 16;
        ta.load(Ab, p.a_mn, p.a_k, p.M, m0, kt0, k_end, t);
        // (L_IMR: by DMA into the last ring slot, free until the first
        // loop iteration's barrier; waited for below)
        if constexpr (imr) lb.issue_tail(smem + (STAGES - 1) * STAGE + TA::floats, nk, wave);
        else if constexpr (imw) tb.load(p, Bb, n0, kt0, k_end, t);
        else tb.load(Bb, p.b_mn, p.b_k, p.N, n0, kt0, k_end, t);
    }

#pragma unroll
    for (int c = 0; c < STAGES - 1; ++c)
        if (c < nk) {
            la.issue(smem + c * STAGE, c, wave);
            lb.issue(smem + c * STAGE + TA::floats, c, wave);
        }

    if (tail) {
        // Slot STAGES-1 is free until the first loop iteration's barrier.
        float* const st = smem + (STAGES - 1) * STAGE;
        ta.store(st, t);
        if constexpr (imr) {
            // the tail DMA was issued before the prologue's chunks
            if (nk >= STAGES - 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(LOADS * (STAGES - 1)));
            else __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
        } else {
            tb.store(st + TA::floats, t);
            __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
        }
        __builtin_amdgcn_s_barrier();
        float fa[MB][8], fb[NB][8];
        dl_frags<LAF, BM, MB>(st, ra, lane, fa);
        dl_frags<LBF, BN, NB>(st + TA::floats, rb, lane, fb);
        mfma_chunk<MB, NB>(acc, fa, fb);
        add_rows(fa);
    }
    for (int kt = 0; kt < nk; ++kt) {
        // Chunk kt must have landed (own instructions, then everyone's).
        // The barrier also retires every wave's reads of the slot refilled
        // below.
        if (kt + STAGES - 1 <= nk) __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(LOADS * (STAGES - 2)));
        else __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
        __builtin_amdgcn_s_barrier();
        const int cn = kt + STAGES - 1;
        if (cn < nk) {
            float* st = smem + (cn % STAGES) * STAGE;
            la.issue(st, cn, wave);
            lb.issue(st + TA::floats, cn, wave);
        }
        const float* At = smem + (kt % STAGES) * STAGE;
        float fa[MB][8], fb[NB][8];
        dl_frags<LAF, BM, MB>(At, ra, lane, fa);
        dl_frags<LBF, BN, NB>(At + TA::floats, rb, lane, fb);
        mfma_chunk<MB, NB>(acc, fa, fb);
        add_rows(fa);
    }

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

    store_tile_lds<MB, NB, NW, WAVES_N, WM, WN, STAGES * STAGE>(p, acc, smem, m0, n0, wave, lane,
                                                               id.split, id.bz);
}

}  // namespace mtk

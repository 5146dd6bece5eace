// gemm_configs.hpp -- the tile configurations the dispatcher chooses from and
// the launcher table each instantiation unit (gemm_instances.hip) exports.
#pragma once

#include <hip/hip_runtime.h>

#include "gemm_kernel.hpp"

namespace mtk {

// Block tile BM x BN x BK, wave tile WM x WN.  Threads = (BM/WM)*(BN/WN)*64.
template <int CFG> struct TileCfg;
// 256x256: one workgroup (8 waves, 2 per SIMD) fills a CU; 4096^2 -> 256 tiles.
template <> struct TileCfg<0> { static constexpr int BM = 256, BN = 256, BK = 16, WM = 128, WN = 64; };
// 128x128: 4 waves; several workgroups share a CU.
template <> struct TileCfg<1> { static constexpr int BM = 128, BN = 128, BK = 16, WM = 64, WN = 64; };
// 64x64: 4 waves of 32x32, for small and skinny problems (usually with split-K).
template <> struct TileCfg<2> { static constexpr int BM = 64, BN = 64, BK = 16, WM = 32, WN = 32; };

constexpr int kNumCfg = 3;
constexpr int kNumLayout = 4;

template <int CFG>
constexpr int cfg_threads() {
    return (TileCfg<CFG>::BM / TileCfg<CFG>::WM) * (TileCfg<CFG>::BN / TileCfg<CFG>::WN) * 64;
}

using GemmLaunchFn = hipError_t (*)(const GemmParams&, unsigned nblocks, hipStream_t);

// Launcher of configuration CFG for (layout of A, layout of B); defined in the
// instantiation unit built with MT_CFG == CFG.
GemmLaunchFn launcher_cfg0(int la, int lb);
GemmLaunchFn launcher_cfg1(int la, int lb);
GemmLaunchFn launcher_cfg2(int la, int lb);

// Direct-to-LDS kernel (gemm_dl_kernel.hpp) for operands whose layouts are both
// L_KV or L_MV: block tile BM x BN, wave tile WM x WN, STAGES-deep LDS ring of
// 16-deep K-chunks.  Same tile sizes, in the same order, as TileCfg.
template <int CFG> struct DlCfg;
// 8 waves of 128x64; 2 x 32 KB ring.
template <> struct DlCfg<0> { static constexpr int BM = 256, BN = 256, WM = 128, WN = 64, STAGES = 2; };
// 8 waves of 64x32; 2 x 16 KB ring, up to four workgroups per CU.
template <> struct DlCfg<1> { static constexpr int BM = 128, BN = 128, WM = 64, WN = 32, STAGES = 2; };
// 4 waves of 32x32; 2 x 8 KB ring, up to eight workgroups per CU.  (Deeper
// rings measured slower for these tiles: occupancy hides more latency.)
template <> struct DlCfg<2> { static constexpr int BM = 64, BN = 64, WM = 32, WN = 32, STAGES = 2; };
// 8 waves of 64x64; 2 x 24 KB ring.  Fills the chip where M is about 256
// (e.g. convolutions with 256 output channels: 49 tiles x split 5 = 245).
template <> struct DlCfg<3> { static constexpr int BM = 256, BN = 128, WM = 64, WN = 64, STAGES = 2; };
// Configurations 4-6 are the fragment-prefetching kernel gemm_f32_dlp
// (gemm_dlp_kernel.hpp): vector layouts, the weight-gradient operand L_IMW
// and the row-sum form; no implicit-im2col (L_IM) form.  4: 4 waves of
// 128x128 (one per SIMD); 5: 4 waves of 32x32; 6: 8 waves of 64x32 (two per
// SIMD), the 128x128 tile for K ranges of 512 and more.
// WPE: waves per SIMD its registers are sized for.
template <> struct DlCfg<4> { static constexpr int BM = 256, BN = 256, WM = 128, WN = 128, STAGES = 2, WPE = 1; };
template <> struct DlCfg<5> { static constexpr int BM = 64, BN = 64, WM = 32, WN = 32, STAGES = 2, WPE = 8; };
template <> struct DlCfg<6> { static constexpr int BM = 128, BN = 128, WM = 64, WN = 32, STAGES = 2, WPE = 2; };

// Configuration 7 is the convolution kernel on 16x16 MFMA blocks
// gemm_f32_dl16 (gemm_dl16_kernel.hpp), B = L_IM only: block tile BM x BN,
// wave tile WM x WN, KG groups of waves splitting the tile's K-chunks, a
// STAGES-slot ring per group, PRE of a chunk's four MFMA k-steps issued
// before each barrier.  112 = 7 blocks of 16 divides the pixel count of
// ResNet layers (multiples of 7*7*16 at even batch sizes).  8 waves: two
// groups of four 16x112 waves, two waves per SIMD; 72 KB of LDS, two
// workgroups per CU.
template <int CFG> struct Dl16Cfg;
template <> struct Dl16Cfg<0> { static constexpr int BM = 64, BN = 112, WM = 16, WN = 112, KG = 2, STAGES = 3, PRE = 2; };
constexpr int kNumDl16Cfg = 1;

constexpr int kDlpFirstCfg = 4;    // configurations kDlpFirstCfg.. are gemm_f32_dlp
constexpr int kDl16FirstCfg = 7;   // configurations kDl16FirstCfg.. are gemm_f32_dl16
constexpr int kNumDlCfg = kDl16FirstCfg + kNumDl16Cfg;
constexpr bool is_dlp_cfg(int cfg) { return cfg >= kDlpFirstCfg && cfg < kDl16FirstCfg; }
constexpr bool is_dl16_cfg(int cfg) { return cfg >= kDl16FirstCfg; }

template <int CFG>
constexpr int dl_threads() {
    return (DlCfg<CFG>::BM / DlCfg<CFG>::WM) * (DlCfg<CFG>::BN / DlCfg<CFG>::WN) * 64;
}

// la, lb in {L_KV, L_MV}.
GemmLaunchFn dl_launcher_cfg0(int la, int lb);
GemmLaunchFn dl_launcher_cfg1(int la, int lb);
GemmLaunchFn dl_launcher_cfg2(int la, int lb);
GemmLaunchFn dl_launcher_cfg3(int la, int lb);
// Configurations 4-6 (gemm_f32_dlp); la, lb in {L_KV, L_MV}; tail: K is
// not a multiple of 16.
GemmLaunchFn dlp_launcher(int cfg, bool tail, int la, int lb);
// Configurations 4-6 with the row sums of A (GemmParams::rowsum); A and B L_MV.
GemmLaunchFn dlp_rowsum_launcher(int cfg, bool tail, bool kv);
// Configurations 4-6 for the convolution weight gradient (A L_KV, B L_IMW).
GemmLaunchFn dlp_convw_launcher(int cfg, bool tail);
// Configurations 4-6 for the weight gradient with A = dY in NCHW (L_KVI).
GemmLaunchFn dlp_convwi_launcher(int cfg);
// Implicit-im2col convolution: A = weights (L_KV), B = L_IM (GemmParams::cv).
GemmLaunchFn dl16_conv_launcher(int cfg16);   // gemm_f32_dl16, Dl16Cfg<cfg16>
void dl16_tile(int cfg16, int* bm, int* bn);
GemmLaunchFn dl_conv_launcher_cfg0();
GemmLaunchFn dl_conv_launcher_cfg1();
GemmLaunchFn dl_conv_launcher_cfg2();
GemmLaunchFn dl_conv_launcher_cfg3();
// Implicit-im2col convolution from an NCHW view: A = OIHW weights (L_KV), B = L_IMR.
GemmLaunchFn dl_convr_launcher_cfg0();
GemmLaunchFn dl_convr_launcher_cfg1();
GemmLaunchFn dl_convr_launcher_cfg2();
GemmLaunchFn dl_convr_launcher_cfg3();
// The same convolution with B built in LDS from a halo patch (L_IMH,
// gemm_dlh_kernel.hpp): ConvGeom::hp and pw set, LDS per workgroup
// dlh_lds_floats of the configuration's tile.
GemmLaunchFn dl_convh_launcher_cfg0();
GemmLaunchFn dl_convh_launcher_cfg1();
GemmLaunchFn dl_convh_launcher_cfg2();
GemmLaunchFn dl_convh_launcher_cfg3();
// Convolution weight gradient: A = dY [c_out][n*h_out*w_out] (L_KV), B = L_IMW.
GemmLaunchFn dl_convw_launcher_cfg0();
GemmLaunchFn dl_convw_launcher_cfg1();
GemmLaunchFn dl_convw_launcher_cfg2();
GemmLaunchFn dl_convw_launcher_cfg3();
// The same with A = dY in NCHW (L_KVI; K a multiple of 16).
GemmLaunchFn dl_convwi_launcher_cfg0();
GemmLaunchFn dl_convwi_launcher_cfg1();
GemmLaunchFn dl_convwi_launcher_cfg2();
GemmLaunchFn dl_convwi_launcher_cfg3();
// A and B mn-contiguous, with the row sums of A (GemmParams::rowsum).
GemmLaunchFn dl_rowsum_launcher_cfg0(bool kv);
GemmLaunchFn dl_rowsum_launcher_cfg1(bool kv);
GemmLaunchFn dl_rowsum_launcher_cfg2(bool kv);
GemmLaunchFn dl_rowsum_launcher_cfg3(bool kv);

// Wave-split kernel (gemm_ksw_kernel.hpp): tile (R*MB) x (R*NB) of R x R
// MFMA blocks (R = 32: gemm_f32_ksw, R = 16: gemm_f32_ksw16), W waves
// splitting the tile's K range, D chunks in flight per wave.  Any operand
// layout: VA / VB select 16-byte fragment loads for k-contiguous operands
// (L_KV) or scalar ones (every other layout).
template <int CFG> struct KswCfg;
template <> struct KswCfg<0> { static constexpr int R = 32, MB = 1, NB = 1, W = 4, D = 6; };
template <> struct KswCfg<1> { static constexpr int R = 32, MB = 1, NB = 1, W = 8, D = 4; };
template <> struct KswCfg<2> { static constexpr int R = 32, MB = 2, NB = 1, W = 4, D = 4; };
template <> struct KswCfg<3> { static constexpr int R = 32, MB = 1, NB = 2, W = 4, D = 4; };
template <> struct KswCfg<4> { static constexpr int R = 16, MB = 2, NB = 1, W = 4, D = 8; };
template <> struct KswCfg<5> { static constexpr int R = 16, MB = 1, NB = 2, W = 4, D = 8; };
template <> struct KswCfg<6> { static constexpr int R = 16, MB = 2, NB = 1, W = 8, D = 4; };
// 7, 8: the 64x32 and 32x64 tiles again on 16x16 blocks (eight accumulator
// chains per wave where configurations 2 and 3 have two).
template <> struct KswCfg<7> { static constexpr int R = 16, MB = 4, NB = 2, W = 4, D = 4; };
template <> struct KswCfg<8> { static constexpr int R = 16, MB = 2, NB = 4, W = 4, D = 4; };
constexpr int kNumKswCfg = 9;
template <int CFG> struct KswTile {
    static constexpr int bm = KswCfg<CFG>::R * KswCfg<CFG>::MB;
    static constexpr int bn = KswCfg<CFG>::R * KswCfg<CFG>::NB;
};

// Configuration cfg of the wave-split kernel; va / vb: A / B is L_KV.
GemmLaunchFn ksw_launcher(int cfg, bool va, bool vb);
void ksw_tile(int cfg, int* bm, int* bn);

// Vector-ALU kernels of the HBM-bound shapes (gemm_skinny_kernel.hpp):
// GEMV for M <= rows <= 8 (B k-contiguous when kv, else mn-contiguous;
// nullptr for more rows), rank-k for 1 <= K <= 16, and the reduction of the
// GEMV kernels' split-K partials (16-byte workspace, grid over groups of
// 16 column quads x M*batch rows).
constexpr int kGemvMaxRows = 8;    // rows of A the GEMV kernels take
constexpr int kRankKMax = 16;      // K the rank-k kernel takes
constexpr int kGemvMvCols = 256;   // columns per GEMV workgroup, B mn-contiguous
constexpr int kGemvKvCols = 16;    // columns per GEMV workgroup, B k-contiguous
constexpr int kRankKCols = 1024;   // columns per rank-k workgroup
constexpr int kRankKRows = 16;     // rows per rank-k workgroup
GemmLaunchFn gemv_launcher(bool kv, int rows);
GemmLaunchFn rankk_launcher(int K);
hipError_t launch_skinny_reduce(const GemmParams& p, hipStream_t s);

}  // namespace mtk

// mtgemm_api.hip -- the C ABI of include/mtgemm.h: argument checking, operand
// layout classification, the tile / split-K plan, and the small companion
// kernels (split-K reduction, column sums, im2col).
//
// Reference interfaces replaced (all reference citations are paths inside
// dionkadi/miniTensor):
//   mt_gemm_f32      <- matmul_gpu / matmul_gpu_v2 / matmul_gpu_bk16 /
//                       matmul_gpu_strided (src/gpu_ops.cpp:1103-1144, 1167-1223)
//                       and bmm's per-batch loop (include/TensorOps.hpp:933-991)
//   mt_colsum_f32    <- sum_gpu over axis 0 used by unbroadcast for the Linear
//                       bias gradient (src/gpu_ops.cpp:1306-1348)
//   mt_linear_*      <- Linear::forward (include/Module.hpp:112-114) and
//                       MatmulBackward (include/Autograd.hpp:117-147)
//   mt_conv2d_fwd_f32 <- conv2d_gpu (src/gpu_ops.cpp:2237-2325)
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <mutex>
#include <cstdint>
#include <algorithm>
#include <cstdio>
#include <cstring>

#include "gemm_configs.hpp"
#include "mtgemm.h"

using namespace mtk;

// Scratch of mt_gemm_noalloc_f32 (split-K partials), one copy per GPU, part of
// this code object and so loaded with the library: nothing is allocated for
// it at call time.  Host code must never use this name as a device address
// (on the host it is only a stand-in): kernels get the address that
// hipGetSymbolAddress returns for the current device (noalloc_scratch).
static __device__ __align__(256) unsigned char scratch[MT_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int64_t kMaxDim = (int64_t)1 << 31;  // M, N, K and batch are 32-bit inside kernels

thread_local char g_last_config[160] = "none";

hipError_t capture_safe_last_error() {
    // A launch inside stream capture reports hipErrorStreamCaptureUnsupported
    // from hipGetLastError even when it was recorded correctly (the reference
    // treats it the same way, include/GpuUtils.hpp:69-73).
    hipError_t e = hipGetLastError();
    return e == hipErrorStreamCaptureUnsupported ? hipSuccess : e;
}

int device_cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
        cus = 256;
    cache[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

// LDS a workgroup may take on the current device (bytes).
int device_lds_limit() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 65536;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    int b = 0;
    if (hipDeviceGetAttribute(&b, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
        b <= 0)
        b = 65536;
    cache[dev].store(b, std::memory_order_relaxed);
    return b;
}

bool valid_mat(const mt_mat_f32* X) {
    if (!X) return false;
    if (X->rows < 0 || X->cols < 0 || X->batch < 0) return false;
    if (X->row_stride < 0 || X->col_stride < 0 || X->batch_stride < 0 || X->offset < 0) return false;
    if (X->rows >= kMaxDim || X->cols >= kMaxDim || X->batch >= kMaxDim) return false;
    return true;
}

// Layout mode of one operand in (mn, k) coordinates; see gemm_kernel.hpp.
int classify(const float* p, int64_t s_mn, int64_t s_k, int64_t MN, int64_t K, int64_t s_b,
             bool batched) {
    const bool aligned = ((uintptr_t)p & 15u) == 0 && (!batched || (s_b & 3) == 0);
    const bool kc = (s_k == 1) || (K == 1);
    const bool mc = (s_mn == 1) || (MN == 1);
    if (kc && aligned && (K & 3) == 0 && (MN == 1 || (s_mn & 3) == 0)) return L_KV;
    if (mc && aligned && (MN & 3) == 0 && (K == 1 || (s_k & 3) == 0)) return L_MV;
    if (s_k == 1) return L_KS;
    if (s_mn == 1) return L_MS;
    return s_k <= s_mn ? L_KS : L_MS;
}

const char* layout_name(int l) {
    switch (l) {
        case L_KV: return "kv";
        case L_MV: return "mv";
        case L_IM: return "im2col";
        case L_IMW: return "im2colT";
        case L_IMR: return "im2col_nchw";
        case L_IMH: return "im2col_halo";
        case L_KVI: return "kv_nchw";
        case L_KS: return "ks";
        default: return "ms";
    }
}

struct Plan {
    bool dl = false;   // direct-to-LDS kernel (both operands in a vector layout)
    bool ksw = false;  // wave-split kernel (K split across the waves of a workgroup)
    int cfg = 0;       // TileCfg index (register-staged) or DlCfg index (direct-to-LDS)
    int bm = 0, bn = 0;
    int splits = 1;
    int kps = 0;
    int tiles_m = 0, tiles_n = 0;
    size_t ws_bytes = 0;
    double cycles = 0;  // the cost model's CU cycles for the plan
};

constexpr int kBK = 16;
static_assert(TileCfg<0>::BK == kBK && TileCfg<1>::BK == kBK && TileCfg<2>::BK == kBK,
              "split-K granularity assumes one BK for all configurations");

// One tile configuration as the cost model sees it.
struct CfgCost {
    int bm, bn;
    double eff;   // sustained fraction of the CU's MFMA rate inside a workgroup
    int occ;      // resident workgroups per CU
};

// Cost model (in CU cycles) used to pick the tile configuration and split-K
// factor.  Work per workgroup is priced at the CU's fp32 MFMA rate (256
// flop/clk) with a per-configuration efficiency; the epilogue's store of a
// tile overlaps the work of the other workgroups resident on the CU, so it is
// shared out over the occupancy; each round of resident workgroups pays a
// fixed latency; split-K pays for its partial traffic and the reduction
// launch.  The constants are fitted (log-time error plus selection regret) to
// the measured times of every configuration and split factor on 29 shapes --
// the benchmark shapes, square, ragged, tall, wide, skinny, batched and
// convolution GEMMs -- on one MI355X.  The efficiencies of the prefetching
// configurations 4-6 come from same-box comparisons with configurations 0, 2
// and 1, which have the same tiles.
constexpr CfgCost kRsCost[kNumCfg] = {      // register-staged kernel, any layout
    {TileCfg<0>::BM, TileCfg<0>::BN, 0.86, 1},
    {TileCfg<1>::BM, TileCfg<1>::BN, 0.75, 2},
    {TileCfg<2>::BM, TileCfg<2>::BN, 0.57, 4}};
// Configuration 7 (the convolution kernel on 16x16 blocks, 64x112 tiles,
// channels-last operand only): 0.78 with two workgroups per CU, from graph
// timings of ResNet-like layers at batch 32 against the plans of
// configurations 0-3 (28x28x128 3x3: 88.9 against 96.3 us, 56x56x64:
// 94.2 against 97.0, 14x14 1x1 256 -> 1024: 55.7 against 57.9); never
// offered where its workgroups would run one per CU (make_plan_uncached).
constexpr CfgCost kDlCost[kNumDlCfg] = {    // direct-to-LDS kernel, vector layouts
    {DlCfg<0>::BM, DlCfg<0>::BN, 0.90, 1},
    {DlCfg<1>::BM, DlCfg<1>::BN, 0.86, 4},
    {DlCfg<2>::BM, DlCfg<2>::BN, 0.68, 8},
    {DlCfg<3>::BM, DlCfg<3>::BN, 0.87, 3},
    {DlCfg<4>::BM, DlCfg<4>::BN, 0.98, 1},
    {DlCfg<5>::BM, DlCfg<5>::BN, 0.72, 8},
    {DlCfg<6>::BM, DlCfg<6>::BN, 0.90, 3},
    {Dl16Cfg<0>::BM, Dl16Cfg<0>::BN, 0.78, 2}};
// The same kernels with the convolution weight gradient's gathered B operand
// (L_IMW): its 16-byte gathers cost per chunk whatever the tile's height, so
// the 256-row tile of configuration 3 amortises them over twice the MFMA work
// of the 128-row ones.  Forced sweeps of every configuration and split on
// five ResNet-like dW shapes (c_out 64-512, one MI355X): configuration 3 at
// its best split is 3-4 % faster than the plain table's picks where M >= 256
// (5a layer: split 14, 86.9 vs 89.4 us at configuration 6 split 7;
// 512 x 4608 x 1568: 99.7 vs 103.7 us at configuration 1), and the 64-row
// shapes keep configuration 5.  Only configurations 3 and 6 differ.
constexpr CfgCost kDlCostImw[kNumDlCfg] = {
    {DlCfg<0>::BM, DlCfg<0>::BN, 0.90, 1},
    {DlCfg<1>::BM, DlCfg<1>::BN, 0.86, 4},
    {DlCfg<2>::BM, DlCfg<2>::BN, 0.68, 8},
    {DlCfg<3>::BM, DlCfg<3>::BN, 0.93, 3},
    {DlCfg<4>::BM, DlCfg<4>::BN, 0.98, 1},
    {DlCfg<5>::BM, DlCfg<5>::BN, 0.72, 8},
    {DlCfg<6>::BM, DlCfg<6>::BN, 0.86, 3},
    {Dl16Cfg<0>::BM, Dl16Cfg<0>::BN, 0.78, 2}};   // (configuration 7: L_IM only)
// Wave-split kernel (configurations of KswCfg): efficiencies from
// graph-replay timings of every configuration at 1, 2 and 4 K splits on the
// benchmark's small GEMMs and four neighbouring shapes (one MI355X).  It is
// L2-bandwidth-bound -- no operand is shared between its waves, about 8 flop
// per byte read for a 32x32 tile -- so it is offered without split-K only,
// where the alternative is a split-K plan and its reduction launch: config 1
// 6.7 vs 9.4 us, the Linear dX GEMM 14.7 vs 18.4 us, 512^3 6.9 vs 11.2 us.
// (The model prices the split-K reduction from eager timings, above its cost
// under graph replay; 0.38 for the 32x32 tile keeps the Linear forward GEMM,
// 17.1 us with split-K against 18.4 us here, on the split-K plan.)  The
// 16x16-block tiles (configurations 4-6, half the work per workgroup) pay
// where the 32x32 tiles leave CUs idle and the half tiles still fit one
// round: config 1 (256 x 512 x 512, 256 workgroups) 4.87 us for 16x32
// against 6.60 for 32x32 on 128, 128 x 512 x 1024 6.47 against 9.53,
// 256^3 4.17 against 4.51; at 512^3 (512 half tiles, two per CU) 8.3
// against 6.7, which the per-CU sum of the model reproduces.  The 64x32 and
// 32x64 tiles on 16x16 blocks (configurations 7, 8: eight accumulator
// chains per wave where configurations 2, 3 have two): the Linear dX GEMM
// 13.2-13.6 us against 14.2, 512 x 1024 x 1024 13.6 against 15.6.  (A 32x32
// tile of 16x16 blocks, four chains, gained 3-10 % over configuration 0 on
// some shapes but lost on the Linear forward GEMM, 18.8 against 18.4, where
// the model then preferred it to the 16.2 us split-K plan: left out.)
constexpr CfgCost kKswCost[kNumKswCfg] = {
    {KswTile<0>::bm, KswTile<0>::bn, 0.38, 8},
    {KswTile<1>::bm, KswTile<1>::bn, 0.37, 4},
    {KswTile<2>::bm, KswTile<2>::bn, 0.45, 4},
    {KswTile<3>::bm, KswTile<3>::bn, 0.45, 4},
    {KswTile<4>::bm, KswTile<4>::bn, 0.28, 8},
    {KswTile<5>::bm, KswTile<5>::bn, 0.325, 8},
    {KswTile<6>::bm, KswTile<6>::bn, 0.27, 4},
    {KswTile<7>::bm, KswTile<7>::bn, 0.47, 4},
    {KswTile<8>::bm, KswTile<8>::bn, 0.49, 4}};
// Its waves split the K-chunks, so a K range of fewer chunks than waves
// leaves some idle and pays the cross-wave sum for nothing: not offered there
// (512 x 1024 x 16: 4.1 us on the 32x64 wave-split tile against 3.1 on the
// 64x64 prefetching one).
constexpr int kKswWaves[kNumKswCfg] = {KswCfg<0>::W, KswCfg<1>::W, KswCfg<2>::W,
                                       KswCfg<3>::W, KswCfg<4>::W, KswCfg<5>::W,
                                       KswCfg<6>::W, KswCfg<7>::W, KswCfg<8>::W};

// Configuration 6 pays off only over long K ranges (short ones, such as the
// 64-deep batched GEMM of the benchmark, run up to 20 % slower than
// configuration 1): the planner offers it for K per split >= kDlp6MinK, or
// >= kDlp6MinKOneRound when every workgroup gets a CU of its own (about 4 %
// faster than configuration 1 at 2048^2 x 256; with several rounds the four
// co-resident workgroups of configuration 1 win).
constexpr int kDlp6MinK = 512;
constexpr int kDlp6MinKOneRound = 256;
struct CostModel {
    double round_latency = 6200.0;           // cycles of fill/drain per round
    double epilogue_bytes_per_cycle = 7.9;   // one workgroup's tile store
    double bytes_per_cycle = 6400.0;         // device HBM bytes per CU-clock
    double launch_cycles = 17700.0;          // second (reduce) launch
};
constexpr int kMaxSplits = 256;
// The cost model was fitted on splits 1-16.  Beyond 16, a split must keep at
// least kMinKpsBeyondFit of K: on random GEMMs (K <= 4700) the model's picks
// of 19-59 splits at 64-208 per split ran 2-12 % slower than 16 splits (it
// misses a per-workgroup cost of short K ranges), while the weight gradients
// of 64- and 128-channel convolutions (K = n*h_out*w_out = 25088-401408,
// 496-2368 per split) ran 1.2-3.4x faster than at 16.
constexpr int kFittedSplits = 16;
constexpr int kMinKpsBeyondFit = 256;
constexpr int kDlpSmallCfg = 5;          // the 64x64 prefetching configuration
constexpr int kDlSmallCfg = 2;           // the 64x64 direct-to-LDS configuration
constexpr double kCoresidentPair = 0.75;
constexpr int kAloneMinK = 1024;
constexpr double kAlonePenalty = 1.3;
constexpr int kMaxForcedSplits = 64;
constexpr bool kOfferDl16 = true;

// Tile grid and K split of configuration `cfg` asked for `s` splits (the
// split count can come out lower: every split takes whole 16-deep chunks).
Plan cfg_plan(const CfgCost& cc, int cfg, bool dl, int64_t M, int64_t N, int64_t K,
              int64_t batch, int s) {
    Plan pl;
    pl.dl = dl;
    pl.cfg = cfg;
    pl.bm = cc.bm;
    pl.bn = cc.bn;
    pl.tiles_m = (int)((M + cc.bm - 1) / cc.bm);
    pl.tiles_n = (int)((N + cc.bn - 1) / cc.bn);
    const int64_t kps = K > 0 ? ((K + s - 1) / s + kBK - 1) / kBK * kBK : kBK;
    pl.kps = (int)kps;
    pl.splits = K > 0 ? (int)((K + kps - 1) / kps) : 1;
    pl.ws_bytes = pl.splits > 1 ? (size_t)pl.splits * batch * M * N * sizeof(float) : 0;
    return pl;
}

// Workspace of a batch-summed launch (GemmParams::part): one M x N slab per
// split and batch entry, one split included, then M row sums per slab (the
// fused bias gradient's partials).
size_t part_ws_bytes(const Plan& pl, int64_t M, int64_t N, int64_t batch) {
    return (size_t)std::max(pl.splits, 1) * batch * M * (N + 1) * sizeof(float);
}

// Modelled cycles of one plan (see CostModel).
double plan_cycles(const CostModel& cm, const CfgCost& cc, const Plan& pl, int64_t M, int64_t N,
                   int64_t batch, int cus) {
    const int64_t wgs = (int64_t)pl.tiles_m * pl.tiles_n * batch * pl.splits;
    const double per_cu = std::ceil((double)wgs / cus);
    const double rounds = std::ceil((double)wgs / ((double)cus * cc.occ));
    const double work = (double)cc.bm * cc.bn * (double)std::max<int64_t>(pl.kps, kBK) * 2.0 /
                        (256.0 * cc.eff);
    const double epi = (double)cc.bm * cc.bn * 4.0 / cm.epilogue_bytes_per_cycle;
    // One tile row (M <= 64) on the 4-wave 64x64 prefetching tile, two
    // workgroups per CU: each SIMD then holds two waves that hide each other's
    // waits, which the fitted per-workgroup efficiency (mostly from one
    // workgroup per CU) does not see.  Measured, 63 x 4096 x 4096: split 8
    // (two per CU) 26.2 us against 29.4 us at split 4; 8-16 rows 24.4 against
    // 27.2.
    const double pair = (pl.dl && pl.cfg == kDlpSmallCfg && pl.tiles_m == 1 && per_cu == 2)
                            ? kCoresidentPair
                            : 1.0;
    // A 64x64 tile alone on its CU over a long K range (one wave per SIMD,
    // one accumulator chain per wave): slower than its fitted efficiency,
    // which comes from CUs holding several.  Measured on random shapes
    // (bench.py --audit): 1456 x 532 x 2500 at split 1 (207 workgroups) 64.6 us
    // against 48.0 at split 6; the factor moves such shapes to split-K.
    const double alone = (pl.dl && (pl.cfg == kDlSmallCfg || pl.cfg == kDlpSmallCfg) &&
                          per_cu == 1 && pl.kps >= kAloneMinK)
                             ? kAlonePenalty
                             : 1.0;
    double t = per_cu * work * pair * alone + per_cu * epi / cc.occ + rounds * cm.round_latency;
    if (pl.splits > 1) {
        const double bytes = (double)(2 * pl.splits + 1) * M * N * batch * 4.0;
        t += bytes / (cm.bytes_per_cycle) + cm.launch_cycles;
    }
    return t;
}

// wide: the prefetching direct-to-LDS configurations (is_dlp_cfg) may be
// chosen (see wide_ok in launch_gemm); ksw: the wave-split kernel may be;
// imw: B is the weight-gradient operand (priced by kDlCostImw); im16: the
// convolution kernel on 16x16 blocks (is_dl16_cfg, B = L_IM) may be.
Plan make_plan_uncached(int64_t M, int64_t N, int64_t K, int64_t batch, int cus,
                        bool allow_split, bool dl, bool wide, bool ksw, bool imw, bool im16) {
    static const CostModel cm;
    const CfgCost* cfgs = dl ? (imw ? kDlCostImw : kDlCost) : kRsCost;
    const int ncfg = dl ? kNumDlCfg : kNumCfg;
    Plan best;
    best.dl = dl;
    double best_t = 1e300;
    for (int cfg = 0; cfg < ncfg; ++cfg) {
        if (dl && is_dlp_cfg(cfg) && !wide) continue;
        if (dl && is_dl16_cfg(cfg) && !im16) continue;
        const CfgCost& cc = cfgs[cfg];
        for (int s = 1; s <= kMaxSplits; ++s) {
            if (s > 1 && !allow_split) break;
            const Plan pl = cfg_plan(cc, cfg, dl, M, N, K, batch, s);
            if (s > 1 && pl.kps < 64) break;
            if (s > kFittedSplits && pl.kps < kMinKpsBeyondFit) break;
            const int64_t k6 = std::min<int64_t>(pl.kps, K);
            if (dl && cfg == 6 && k6 < kDlp6MinKOneRound) break;
            if (pl.splits != s) continue;
            const int64_t wgs = (int64_t)pl.tiles_m * pl.tiles_n * batch * pl.splits;
            if (dl && cfg == 6 && k6 < kDlp6MinK && wgs > cus) continue;
            if (wgs * 512 >= ((int64_t)1 << 32)) continue;
            // The 64x112 tile of 16x16 blocks moves about twice the operand
            // bytes per flop of the 256x128 one; with one workgroup per CU
            // (nothing co-resident to hide the fetches) it lost everywhere it
            // was measured (the 5a layer: 93.2 us against 80.2 at split 5).
            if (dl && is_dl16_cfg(cfg) && wgs <= cus) continue;
            const double t = plan_cycles(cm, cc, pl, M, N, batch, cus);
            if (t < best_t) {
                best_t = t;
                best = pl;
                best.cycles = t;
            }
        }
    }
    if (ksw) {
        for (int cfg = 0; cfg < kNumKswCfg; ++cfg) {
            if (K < (int64_t)kBK * kKswWaves[cfg]) continue;
            Plan pl = cfg_plan(kKswCost[cfg], cfg, false, M, N, K, batch, 1);
            pl.ksw = true;
            const int64_t wgs = (int64_t)pl.tiles_m * pl.tiles_n * batch;
            if (wgs * 512 >= ((int64_t)1 << 32)) continue;
            const double t = plan_cycles(cm, kKswCost[cfg], pl, M, N, batch, cus);
            if (t < best_t) {
                best_t = t;
                best = pl;
                best.cycles = t;
            }
        }
    }
    return best;
}

// The cost model is a pure function of its arguments; a training loop asks
// for the same few shapes again and again (workspace query, then launch), so
// each thread keeps its last kEntries plans.  A workspace query of one GEMM
// visits up to 10 keys (both families, with and without the prefetching
// configurations and the wave-split kernel, the weight-gradient table), and
// one convolution backward query four such shapes (about 34 keys): the cache
// holds several layers' worth, so the launch that follows a query finds its
// plan instead of rerunning the cost model.
Plan make_plan(int64_t M, int64_t N, int64_t K, int64_t batch, int cus, bool allow_split,
               bool dl, bool wide, bool ksw, bool imw = false, bool im16 = false) {
    struct Entry {
        int64_t M = -1, N = -1, K = -1, batch = -1;
        int cus = 0;
        bool allow_split = false, dl = false, wide = false, ksw = false, imw = false, im16 = false;
        Plan plan;
    };
    constexpr int kEntries = 128;
    thread_local Entry cache[kEntries];
    thread_local int next = 0;
    for (const Entry& e : cache)
        if (e.M == M && e.N == N && e.K == K && e.batch == batch && e.cus == cus &&
            e.allow_split == allow_split && e.dl == dl && e.wide == wide && e.ksw == ksw &&
            e.imw == imw && e.im16 == im16)
            return e.plan;
    Entry& e = cache[next];
    next = (next + 1) % kEntries;
    e = Entry{M, N, K, batch, cus, allow_split, dl, wide, ksw, imw, im16,
              make_plan_uncached(M, N, K, batch, cus, allow_split, dl, wide, ksw, imw, im16)};
    return e.plan;
}

// Configuration forced on this thread's launches by mt_gemm_force_config.
struct ForcedConfig {
    int family = MT_FAMILY_AUTO;
    int cfg = 0;
    int splits = 1;
};
thread_local ForcedConfig g_forced;

// The plan of the forced configuration, when one is set and its family can
// take these operands (dl_ok: both operands have direct-to-LDS layouts;
// rs_ok: no implicit-im2col operand; wide_ok: the prefetching configurations
// can take them too; im16_ok: B is L_IM, which the 16x16-block convolution
// configurations take).
bool forced_plan(int64_t M, int64_t N, int64_t K, int64_t batch, bool dl_ok, bool rs_ok,
                 bool wide_ok, Plan* out, bool im16_ok = false) {
    const ForcedConfig f = g_forced;
    if (f.family == MT_FAMILY_KSW && rs_ok) {
        int bm, bn;
        ksw_tile(f.cfg, &bm, &bn);
        *out = cfg_plan(CfgCost{bm, bn, 1.0, 1}, f.cfg, false, M, N, K, batch, f.splits);
        out->ksw = true;
        return true;
    }
    if (f.family == MT_FAMILY_DL && dl_ok && (!is_dlp_cfg(f.cfg) || wide_ok) &&
        (!is_dl16_cfg(f.cfg) || im16_ok)) {
        *out = cfg_plan(kDlCost[f.cfg], f.cfg, true, M, N, K, batch, f.splits);
        return true;
    }
    if (f.family == MT_FAMILY_RS && rs_ok) {
        *out = cfg_plan(kRsCost[f.cfg], f.cfg, false, M, N, K, batch, f.splits);
        return true;
    }
    return false;
}

// The implicit-im2col form (L_IM) exists for DlCfg 0..3 only; the planner
// never picks the prefetching configurations for it (nullptr is a safety
// net).  The row-sum form and the weight-gradient operand (L_IMW) exist for
// all.
// kv: two k-contiguous operands (else two mn-contiguous ones).
GemmLaunchFn rowsum_launcher(int cfg, bool tail, bool kv) {
    switch (cfg) {
        case 0: return dl_rowsum_launcher_cfg0(kv);
        case 1: return dl_rowsum_launcher_cfg1(kv);
        case 2: return dl_rowsum_launcher_cfg2(kv);
        case 3: return dl_rowsum_launcher_cfg3(kv);
        default: return dlp_rowsum_launcher(cfg, tail, kv);
    }
}

// kvi: A is dY read in NCHW (L_KVI, whole chunks only).
GemmLaunchFn convw_launcher(int cfg, bool ktail, bool kvi) {
    if (kvi) {
        if (ktail) return nullptr;
        switch (cfg) {
            case 0: return dl_convwi_launcher_cfg0();
            case 1: return dl_convwi_launcher_cfg1();
            case 2: return dl_convwi_launcher_cfg2();
            case 3: return dl_convwi_launcher_cfg3();
            default: return dlp_convwi_launcher(cfg);
        }
    }
    switch (cfg) {
        case 0: return dl_convw_launcher_cfg0();
        case 1: return dl_convw_launcher_cfg1();
        case 2: return dl_convw_launcher_cfg2();
        case 3: return dl_convw_launcher_cfg3();
        default: return dlp_convw_launcher(cfg, ktail);
    }
}

// LDS floats of the halo-patch kernel of dl configuration cfg (0-3).
int halo_lds_floats(int cfg, const ConvGeom& g) {
    switch (cfg) {
        case 0: return dlh_lds_floats<DlCfg<0>::BM, DlCfg<0>::BN, DlCfg<0>::WM, DlCfg<0>::WN>(g);
        case 1: return dlh_lds_floats<DlCfg<1>::BM, DlCfg<1>::BN, DlCfg<1>::WM, DlCfg<1>::WN>(g);
        case 2: return dlh_lds_floats<DlCfg<2>::BM, DlCfg<2>::BN, DlCfg<2>::WM, DlCfg<2>::WN>(g);
        case 3: return dlh_lds_floats<DlCfg<3>::BM, DlCfg<3>::BN, DlCfg<3>::WM, DlCfg<3>::WN>(g);
        default: return -1;
    }
}

// Whether the halo-patch kernel of configuration cfg takes the L_IMR
// geometry g (hp and pw set) with K ranges of kps: at least two taps (a patch
// then serves two or more chunks, which the kernel's B prefetch relies on),
// taps, stride and padded extents small enough for its 32-bit patch
// arithmetic, a channel's band at most kHaloIpcMax DMA instructions, the
// images one band spans addressable with 32-bit offsets, and the workgroup's
// LDS within the device's limit.  It pays only when a patch is small next to
// the per-chunk B tiles it replaces and a workgroup multiplies at least one
// whole patch: patch (16 bands) at most 0.3 of kh*kw tiles of BN x 16, and
// kps >= 16*kh*kw (smaller ratios or K ranges measured slower than the
// per-chunk gather, e.g. 45 against 30 us for c_in 8 at 56x56); cost = false
// skips that rule (a forced configuration: the test hook of the kernel).
bool halo_fits(const ConvGeom& g, int n_img, int cfg, int kps, bool cost) {
    static constexpr int kBn[4] = {DlCfg<0>::BN, DlCfg<1>::BN, DlCfg<2>::BN, DlCfg<3>::BN};
    if (cfg < 0 || cfg > 3) return false;
    if (g.kh < 1 || g.kw < 1 || g.kh * g.kw < 2 || g.kh * g.kw > kHaloMaxTaps || g.stride < 1 ||
        g.stride > 16)
        return false;
    if (g.ho < 1 || g.wo < 1 || g.pw < 1 || g.pw > 4096 || g.hp < 1) return false;
    if ((int64_t)n_img * g.hp + 512 * (int64_t)g.stride >= ((int64_t)1 << 31)) return false;
    const int rows = halo_rows(g, kBn[cfg]);
    const int cst = halo_chan_stride(g, kBn[cfg]);
    if (cst > 64 * kHaloIpcMax) return false;
    const int khw = g.kh * g.kw;
    if (cost && (kps < 16 * khw || 10 * cst > 3 * khw * kBn[cfg])) return false;
    const int64_t span = (rows + g.hp - 1) / g.hp + 1;   // images one band can touch
    if (span * g.img_stride + (int64_t)(g.h - 1) * g.sh + (int64_t)(g.w - 1) * g.sw >=
        ((int64_t)1 << 31))
        return false;
    const int f = halo_lds_floats(cfg, g);
    return f > 0 && (int64_t)f * 4 <= device_lds_limit();
}

// The ConvGeom patch extents of an L_IMR convolution.
void set_halo_geometry(ConvGeom& g) {
    g.hp = (g.ho - 1) * g.stride + g.kh;
    g.pw = (g.wo - 1) * g.stride + g.kw;
}

GemmLaunchFn convh_launcher(int cfg) {
    switch (cfg) {
        case 0: return dl_convh_launcher_cfg0();
        case 1: return dl_convh_launcher_cfg1();
        case 2: return dl_convh_launcher_cfg2();
        case 3: return dl_convh_launcher_cfg3();
        default: return nullptr;
    }
}

GemmLaunchFn conv_launcher(int cfg, bool nchw) {
    if (is_dl16_cfg(cfg)) return nchw ? nullptr : dl16_conv_launcher(cfg - kDl16FirstCfg);
    switch (cfg) {
        case 0: return nchw ? dl_convr_launcher_cfg0() : dl_conv_launcher_cfg0();
        case 1: return nchw ? dl_convr_launcher_cfg1() : dl_conv_launcher_cfg1();
        case 2: return nchw ? dl_convr_launcher_cfg2() : dl_conv_launcher_cfg2();
        case 3: return nchw ? dl_convr_launcher_cfg3() : dl_conv_launcher_cfg3();
        default: return nullptr;
    }
}

// ---- HBM-bound shapes on the vector ALUs (gemm_skinny_kernel.hpp) ----------
// GEMV: at most kGemvMaxRows rows of A against a B that is k- or
// mn-contiguous (or, transposed, at most that many columns of B against such
// an A), K >= kGemvMinK; rank-k: 1 <= K <= 2 (4) with at least kRankKMinN
// columns and 2^22 (2^24) output elements, or forced with K <= kRankKMax.  No implicit convolution operand and no fused row or
// channel sums: those shapes keep the MFMA kernels.
enum { SK_NONE = 0, SK_GEMV = 1, SK_RANKK = 2 };
constexpr int kGemvMinK = 16;
constexpr int kGemvKvMaxRows = 4;
constexpr int kRankKMinN = 256;
constexpr int64_t kRankKAutoMn2 = int64_t(1) << 22;   // outputs taking rank-k at K <= 2
constexpr int64_t kRankKAutoMn4 = int64_t(1) << 24;   // ... and at K <= 4
constexpr int kGemvMaxSplits = 64;
constexpr int kGemvWgsPerCu = 4;
// An mn-contiguous B of more than 64 MiB: about six workgroups per CU with
// shorter splits (down to 32 k), up to 128 splits.  Graph-timed: 1 x 4096 x
// 8192 24.7 against 28.0 us, 1 x 8192 x 4096 24.7 against 26.4; at 64 MiB
// and below four per CU stay faster (1 x 4096 x 4096 14.9 against 16.1).
constexpr int64_t kGemvLargeBytes = int64_t(64) << 20;
constexpr int kGemvWgsPerCuLarge = 6, kGemvMaxSplitsLarge = 128, kGemvMinKpsLarge = 32;

struct SkinnyPlan {
    int kind = SK_NONE;
    bool transpose = false;  // computes Cᵀ = Bᵀ·Aᵀ (the few columns of B become rows)
    bool kv = false;         // GEMV: the large operand is k-contiguous
    int rows = 0;            // GEMV: rows of the kernel's instantiation (1, 2, 4, 8)
    int splits = 1, kps = 0;
    int tiles_m = 1, tiles_n = 1;
    size_t ws_bytes = 0;
    unsigned blocks = 0;
};

// GEMV of m <= kGemvMaxRows rows against an n-column operand, K = k.  The
// split count aims at kGemvWgsPerCu workgroups per CU (every workgroup
// resident at once: the kernels are bound by the loads in flight), with at
// least 64 k per split (mn-contiguous B) or four 64-deep steps per lane
// (k-contiguous B), at most kGemvMaxSplits (the ...Large figures for an
// mn-contiguous B of more than kGemvLargeBytes); forced_splits > 0 asks for
// that many.
SkinnyPlan gemv_plan(int64_t m, int64_t n, int64_t k, int64_t batch, bool kv, int cus,
                     int forced_splits) {
    SkinnyPlan s;
    s.kind = SK_GEMV;
    s.kv = kv;
    s.rows = m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8;
    const int64_t cols = kv ? kGemvKvCols : kGemvMvCols;
    s.tiles_n = (int)((n + cols - 1) / cols);
    const bool large = !kv && k * n * batch * (int64_t)sizeof(float) > kGemvLargeBytes;
    const int64_t gran = kv ? 64 : 4;
    const int64_t min_kps = kv ? 256 : large ? kGemvMinKpsLarge : 64;
    const int64_t per_cu = large ? kGemvWgsPerCuLarge : kGemvWgsPerCu;
    const int64_t max_splits = large ? kGemvMaxSplitsLarge : kGemvMaxSplits;
    int64_t want = forced_splits;
    if (want <= 0) {
        const int64_t base = (int64_t)s.tiles_n * batch;
        want = std::max<int64_t>(1, (per_cu * (int64_t)cus + base - 1) / base);
        want = std::min<int64_t>({want, std::max<int64_t>(1, k / min_kps), max_splits});
    }
    int64_t kps = (k + want - 1) / want;
    kps = (kps + gran - 1) / gran * gran;
    s.kps = (int)kps;
    s.splits = (int)((k + kps - 1) / kps);
    s.ws_bytes = s.splits > 1 ? (size_t)s.splits * batch * m * n * sizeof(float) : 0;
    s.blocks = (unsigned)((int64_t)s.tiles_n * s.splits * batch);
    return s;
}

SkinnyPlan rankk_plan(int64_t m, int64_t n, int64_t k, int64_t batch) {
    SkinnyPlan s;
    s.kind = SK_RANKK;
    s.kps = (int)k;
    s.tiles_n = (int)((n + kRankKCols - 1) / kRankKCols);
    s.tiles_m = (int)((m + kRankKRows - 1) / kRankKRows);
    s.blocks = (unsigned)((int64_t)s.tiles_n * s.tiles_m * batch);
    return s;
}

// Which vector-ALU kernel, if any, takes this GEMM (`scatter`: C's columns are
// scattered, which the transposed form cannot take).  A forced configuration
// of another family keeps the shape on that family; a forced MT_FAMILY_SKINNY
// configuration applies where its kernel takes the operands.
SkinnyPlan skinny_plan(int64_t M, int64_t N, int64_t K, int64_t batch, int la, int lb,
                       bool scatter, int cus) {
    const ForcedConfig f = g_forced;
    SkinnyPlan none;
    if (K <= 0 || (f.family != MT_FAMILY_AUTO && f.family != MT_FAMILY_SKINNY)) return none;
    const bool forced = f.family == MT_FAMILY_SKINNY;
    const int splits = forced ? f.splits : 0;
    const bool vec_b = lb == L_MV || lb == L_KV, vec_a = la == L_MV || la == L_KV;
    // The rank-k kernel only writes C (its cost is the store stream), the MFMA
    // kernels also stage a 16-deep chunk: it wins on large outputs with the
    // smallest K.  Graph-timed against the best forced MFMA plan: 4096^2 K = 1,
    // 2, 4: 12.3, 12.6, 13.5 against 14.5, 15.7, 14.7 us; 2048^2 K = 1, 2: 5.6,
    // 6.2 against 7.0, 7.3, but K = 4: 8.0 against 7.1; 256 x 8192 K = 1: 4.9
    // against 4.5; K >= 8 the MFMA kernels on every shape (4096^2 K = 8: 15.7
    // against 14.7).  A forced configuration 1 takes any K <= kRankKMax.
    const int64_t mn = M * N * batch;
    const bool rk_auto = (K <= 2 && mn >= kRankKAutoMn2) || (K <= 4 && mn >= kRankKAutoMn4);
    if ((forced ? f.cfg == 1 : rk_auto) && K <= kRankKMax && N >= kRankKMinN)
        return rankk_plan(M, N, K, batch);
    if (forced && f.cfg != 0) return none;
    if (K < kGemvMinK) return none;
    // With a k-contiguous B the GEMV kernel reads A's rows from LDS beside
    // every load of B; past 4 rows that LDS traffic makes it slower than the
    // MFMA kernels (4096^2: 4 rows 20.7 against 22.8 us, 6 rows 24.4 against
    // 23.2, 8 rows 26.9 against 23.8), so those shapes keep them (a forced
    // configuration still reaches the 8-row kernel).
    const auto rows_ok = [&](int64_t rows, int layout) {
        return rows <= (layout == L_KV && !forced ? kGemvKvMaxRows : kGemvMaxRows);
    };
    if (vec_b && rows_ok(M, lb)) return gemv_plan(M, N, K, batch, lb == L_KV, cus, splits);
    if (vec_a && rows_ok(N, la) && !scatter) {
        SkinnyPlan s = gemv_plan(N, M, K, batch, la == L_KV, cus, splits);
        s.transpose = true;
        return s;
    }
    return none;
}

// Workspace the GEMV plans of this shape may need (layouts unknown).
size_t skinny_ws(int64_t M, int64_t N, int64_t K, int64_t batch, int cus) {
    if (K < kGemvMinK) return 0;
    const ForcedConfig f = g_forced;
    const int splits = f.family == MT_FAMILY_SKINNY ? f.splits : 0;
    size_t ws = 0;
    for (bool kv : {false, true}) {
        const int64_t rows = kv && f.family != MT_FAMILY_SKINNY ? kGemvKvMaxRows : kGemvMaxRows;
        if (M <= rows) ws = std::max(ws, gemv_plan(M, N, K, batch, kv, cus, splits).ws_bytes);
        if (N <= rows) ws = std::max(ws, gemv_plan(N, M, K, batch, kv, cus, splits).ws_bytes);
    }
    return ws;
}

// Workspace that covers the plan of either kernel family (for sizes queried
// before the operand pointers, and hence the layouts, are known).
size_t plan_ws(int64_t M, int64_t N, int64_t K, int64_t batch, int cus, bool imw = false) {
    size_t ws = 0;
    for (bool dl : {false, true})
        for (bool wide : {false, true})
            for (bool ksw : {false, true})
                ws = std::max(ws, make_plan(M, N, K, batch, cus, true, dl, wide, ksw).ws_bytes);
    if (imw)   // the weight-gradient operand's own table
        for (bool wide : {false, true})
            ws = std::max(ws, make_plan(M, N, K, batch, cus, true, true, wide, false, true).ws_bytes);
    Plan forced;
    if (forced_plan(M, N, K, batch, true, true, true, &forced)) ws = std::max(ws, forced.ws_bytes);
    return std::max(ws, skinny_ws(M, N, K, batch, cus));
}

GemmLaunchFn pick_launcher(const Plan& plan, int la, int lb, bool ktail) {
    if (plan.ksw) return ksw_launcher(plan.cfg, la == L_KV, lb == L_KV);
    if (plan.dl) {
        switch (plan.cfg) {
            case 0: return dl_launcher_cfg0(la, lb);
            case 1: return dl_launcher_cfg1(la, lb);
            case 2: return dl_launcher_cfg2(la, lb);
            case 3: return dl_launcher_cfg3(la, lb);
            default: return dlp_launcher(plan.cfg, ktail, la, lb);
        }
    }
    switch (plan.cfg) {
        case 0: return launcher_cfg0(la, lb);
        case 1: return launcher_cfg1(la, lb);
        default: return launcher_cfg2(la, lb);
    }
}

// Checks the three operands and derives the problem sizes.
int check_gemm(const mt_mat_f32* A, const mt_mat_f32* B, const mt_mat_f32* C,
               int64_t* M, int64_t* N, int64_t* K, int64_t* batch) {
    if (!valid_mat(A) || !valid_mat(B) || !valid_mat(C)) return MT_ERR_INVALID;
    if (A->cols != B->rows || C->rows != A->rows || C->cols != B->cols) return MT_ERR_INVALID;
    *M = A->rows; *N = B->cols; *K = A->cols; *batch = C->batch;
    if ((A->batch != 1 && A->batch != *batch) || (B->batch != 1 && B->batch != *batch))
        return MT_ERR_INVALID;
    const bool c_empty = (*M == 0 || *N == 0 || *batch == 0);
    // Two output elements must never share an address.
    if (!c_empty && ((*M > 1 && C->row_stride == 0) || (*N > 1 && C->col_stride == 0) ||
                     (*batch > 1 && C->batch_stride == 0)))
        return MT_ERR_INVALID;
    if (!c_empty && !C->base) return MT_ERR_INVALID;
    if (!c_empty && *K > 0 && (!A->base || !B->base)) return MT_ERR_INVALID;
    return MT_OK;
}

// Split-K partials are summed in split order, then bias and beta are applied:
// deterministic.  Up to kReduceBatch partial loads (and the loads of the bias
// and of beta*C) are issued before the first add: a loop bounded by the
// runtime split count would wait for each load before issuing the next.
constexpr int kReduceBatch = 8;

template <class T>
__device__ __forceinline__ T sum_partials(const float* src, int64_t split_stride, int splits,
                                          T v) {
    for (int s0 = 0; s0 < splits; s0 += kReduceBatch) {
        T t[kReduceBatch];
#pragma unroll
        for (int j = 0; j < kReduceBatch; ++j)
            if (s0 + j < splits)
                t[j] = *reinterpret_cast<const T*>(src + (int64_t)(s0 + j) * split_stride);
#pragma unroll
        for (int j = 0; j < kReduceBatch; ++j)
            if (s0 + j < splits) v += t[j];
    }
    return v;
}

// Scalar form, for outputs that do not take 16-byte stores.
__global__ void __launch_bounds__(256) splitk_reduce_f32(GemmParams p) {
    const int64_t MN = (int64_t)p.M * p.N;
    const int64_t total = MN * p.batch;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t bz = e / MN;
        const int64_t mn = e - bz * MN;
        const int m = (int)(mn / p.N);
        const int n = (int)(mn - (int64_t)m * p.N);
        const float b = p.bias_axis == 1   ? p.bias[(int64_t)m * p.bias_stride]
                        : p.bias_axis == 2 ? p.bias[(int64_t)n * p.bias_stride]
                                           : 0.f;
        float* dst = p.C + bz * p.c_b + (int64_t)m * p.c_m + col_offset(p, n);
        const float old = p.beta != 0.f ? *dst : 0.f;
        float v = sum_partials<float>(p.ws + bz * MN + mn, p.batch * MN, p.splits, 0.f);
        if (p.bias_axis != 0) v += b;
        if (p.beta != 0.f) v += p.beta * old;
        *dst = v;
    }
}

// One thread's share of Σ_{img < n, q < hw} src[(img·C + c)·hw + q] in a
// workgroup of NT threads: a fixed set of positions (item i: image i / per,
// position i % per, of 16-byte vectors when VEC), U loads in flight; 32-bit
// indices (n·per + U·NT < 2^31).
template <int NT, int U, bool VEC>
__device__ __forceinline__ float channel_part(const float* src, int64_t C, int c, int per, int total,
                                              int64_t hw) {
    float s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) s[u] = 0.f;
    for (int i0 = threadIdx.x; i0 < total; i0 += U * NT) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = i0 + u * NT < total ? i0 + u * NT : 0;
            const int img = i / per, j = i - img * per;
            const float* q = src + ((int64_t)img * C + c) * hw;
            if constexpr (VEC) {
                const f32x4 x = *reinterpret_cast<const f32x4*>(q + 4 * (int64_t)j);
                v[u] = (x[0] + x[1]) + (x[2] + x[3]);
            } else {
                v[u] = q[j];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (i0 + u * NT < total) s[u] += v[u];
    }
#pragma unroll
    for (int w = U / 2; w > 0; w >>= 1)
#pragma unroll
        for (int u = 0; u < w; ++u) s[u] += s[u + w];
    return s[0];
}

// channel_part for n·per >= 2^31 items: image by image, no 64-bit division.
template <int NT, bool VEC>
__device__ __forceinline__ float channel_part_wide(const float* src, int64_t C, int c, int64_t n,
                                                   int64_t per, int64_t hw) {
    float s = 0.f;
    for (int64_t img = 0; img < n; ++img) {
        const float* q = src + (img * C + c) * hw;
#pragma unroll 4
        for (int64_t j = threadIdx.x; j < per; j += NT) {
            if constexpr (VEC) {
                const f32x4 x = *reinterpret_cast<const f32x4*>(q + 4 * j);
                s += (x[0] + x[1]) + (x[2] + x[3]);
            } else {
                s += q[j];
            }
        }
    }
    return s;
}

// Σ_{img < n, q < hw} src[(img·C + c)·hw + q] by one workgroup of NT threads
// (16-byte loads when hw % 4 == 0 and src is aligned), returned to every
// thread: each thread sums a fixed set of positions, then a fixed-order tree
// over red[NT], so the result is deterministic.  One channel of a 64-channel
// layer is 0.4-1.6 MB; a workgroup needs about 100 KB of loads in flight to
// pull it at more than a few GB/s, hence 1024 threads x 8 16-byte loads.
template <int NT, int U>
__device__ float block_channel_sum(const float* src, int64_t C, int c, int64_t n, int64_t hw,
                                   float* red) {
    const int t = threadIdx.x;
    const bool vec = (hw & 3) == 0 && ((uintptr_t)src & 15u) == 0;
    const int64_t per = vec ? hw / 4 : hw;
    const int64_t total = n * per;
    float s;
    if (total < ((int64_t)1 << 31) - (int64_t)U * NT) {   // 32-bit index arithmetic
        s = vec ? channel_part<NT, U, true>(src, C, c, (int)per, (int)total, hw)
                : channel_part<NT, U, false>(src, C, c, (int)per, (int)total, hw);
    } else {
        s = vec ? channel_part_wide<NT, true>(src, C, c, n, per, hw)
                : channel_part_wide<NT, false>(src, C, c, n, per, hw);
    }
    red[t] = s;
    __syncthreads();
    for (int w = NT / 2; w > 0; w >>= 1) {
        if (t < w) red[t] += red[t + w];
        __syncthreads();
    }
    const float r = red[0];
    __syncthreads();   // red is reused by the caller's next channel
    return r;
}

// Channel sums run on 1024-thread workgroups when a channel holds at least
// half a pass of them (1024 x 8 x 4 / 2 floats), else on 256 threads.
// Measured, dW + db: the 256-channel 14x14 layer (6272 floats a channel)
// 84.0-84.3 us on 256 threads against 87.0 on 1024; 128-channel 28x28 layers
// (25088 floats) about 1 us faster on 1024.
constexpr int kCsumLoads = 8;
constexpr int64_t kCsumWideItems = 1024 * kCsumLoads * 4 / 2;
inline int csum_threads(int64_t per_channel) { return per_channel >= kCsumWideItems ? 1024 : 256; }

// csum[m] of GemmParams (the convolution, or Linear, bias gradient).
template <int NT>
__device__ __forceinline__ void channel_sum(const GemmParams& p, int m, float* red) {
    float r;
    if (p.csum_rows) {   // the GEMM's row-sum partials: splits slabs of M, fixed order
        float v = 0.f;
        for (int sl = threadIdx.x; sl < p.splits; sl += NT)
            v += p.csum_rows[(int64_t)sl * p.M + m];
        red[threadIdx.x] = v;
        __syncthreads();
        for (int w = NT / 2; w > 0; w >>= 1) {
            if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
            __syncthreads();
        }
        r = red[0];
        __syncthreads();
    } else {
        r = block_channel_sum<NT, kCsumLoads>(p.csum_src, p.M, m, p.csum_n, p.csum_hw, red);
    }
    if (threadIdx.x == 0) p.csum[m] = (p.csum_beta != 0.f ? p.csum_beta * p.csum[m] : 0.f) + r;
}

// Vector form (ws_vec: N % 4 == 0, 16-byte partials): blockIdx.y walks output
// rows (batch-major), threads walk 4-column groups; the group is stored as one
// 16-byte vector when C allows (c_vec), else element by element through
// col(n).  Same per-element summation order as the scalar form.
// CSUM: also the channel sums of GemmParams::csum (a separate instantiation,
// so that the plain reduction carries neither its code nor its LDS).
template <bool CSUM, int NT = 256>
__global__ void __launch_bounds__(NT) splitk_reduce_vec_f32(GemmParams p) {
    __shared__ float red[CSUM ? NT : 1];
    const int64_t MN = (int64_t)p.M * p.N;
    const int64_t rows = (int64_t)p.M * p.batch;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    for (int64_t row = blockIdx.y; row < rows; row += gridDim.y) {
        const int bz = (int)(row / p.M);
        const int m = (int)(row - (int64_t)bz * p.M);
        if constexpr (CSUM)
            if (blockIdx.x == 0) channel_sum<NT>(p, m, red);
        const float brow = p.bias_axis == 1 ? p.bias[(int64_t)m * p.bias_stride] : 0.f;
        const float* src = p.ws + (int64_t)bz * MN + (int64_t)m * p.N;
        float* crow = p.C + (int64_t)bz * p.c_b + (int64_t)m * p.c_m;
        for (int n = (blockIdx.x * blockDim.x + threadIdx.x) * 4; n < p.N;
             n += gridDim.x * blockDim.x * 4) {
            f32x4 bcol = zero, old = zero;
            if (p.bias_axis == 2)
                for (int e = 0; e < 4; ++e) bcol[e] = p.bias[(int64_t)(n + e) * p.bias_stride];
            if (p.beta != 0.f) {
                if (p.c_vec) old = *reinterpret_cast<const f32x4*>(crow + col_offset(p, n));
                else
                    for (int e = 0; e < 4; ++e) old[e] = crow[col_offset(p, n + e)];
            }
            f32x4 v = sum_partials<f32x4>(src + n, p.batch * MN, p.splits, zero);
            v += brow;
            if (p.bias_axis == 2) v += bcol;
            if (p.beta != 0.f) v += p.beta * old;
            if (p.c_vec) {
                *reinterpret_cast<f32x4*>(crow + col_offset(p, n)) = v;
            } else {
                for (int e = 0; e < 4; ++e) crow[col_offset(p, n + e)] = v[e];
            }
        }
    }
}

// The transposed problem Cᵀ = Bᵀ·Aᵀ: the operands swap roles, C's row and
// column strides swap, a per-row bias becomes a per-column one.  Only for
// unscattered outputs.
GemmParams transposed_params(const GemmParams& p) {
    GemmParams q = p;
    q.A = p.B; q.a_mn = p.b_mn; q.a_k = p.b_k; q.a_b = p.b_b;
    q.B = p.A; q.b_mn = p.a_mn; q.b_k = p.a_k; q.b_b = p.a_b;
    q.c_m = p.c_n; q.c_n = p.c_m;
    q.M = p.N; q.N = p.M;
    q.c_n_inner = q.N;
    q.c_n_outer = 0;
    q.bias_axis = p.bias_axis == MT_BIAS_ROW   ? MT_BIAS_COL
                  : p.bias_axis == MT_BIAS_COL ? MT_BIAS_ROW
                                               : p.bias_axis;
    q.c_vec = q.c_n == 1 && (q.N & 3) == 0 && ((uintptr_t)q.C & 15u) == 0 && (q.c_m & 3) == 0 &&
              (q.batch == 1 || (q.c_b & 3) == 0);
    return q;
}

// Launches a vector-ALU plan (and, for a split GEMV, the reduction of its
// partials).  A GEMV plan whose partials the workspace cannot hold runs
// unsplit, unless the configuration is forced (MT_ERR_WORKSPACE).
int launch_skinny(const GemmParams& p0, SkinnyPlan sp, void* workspace, size_t ws_bytes,
                  hipStream_t stream) {
    if (sp.splits > 1 && (workspace == nullptr || ws_bytes < sp.ws_bytes)) {
        if (g_forced.family == MT_FAMILY_SKINNY) return MT_ERR_WORKSPACE;
        const bool t = sp.transpose;
        sp = t ? gemv_plan(p0.N, p0.M, p0.K, p0.batch, sp.kv, device_cu_count(), 1)
               : gemv_plan(p0.M, p0.N, p0.K, p0.batch, sp.kv, device_cu_count(), 1);
        sp.transpose = t;
    }
    GemmParams p = sp.transpose ? transposed_params(p0) : p0;
    p.splits = sp.splits;
    p.k_per_split = sp.kps;
    p.tiles_m = sp.tiles_m;
    p.tiles_n = sp.tiles_n;
    p.group_m = 1;
    p.ws = sp.splits > 1 ? static_cast<float*>(workspace) : nullptr;
    p.ws_vec = p.ws != nullptr && ((uintptr_t)p.ws & 15u) == 0 && (p.N & 3) == 0;
    std::snprintf(g_last_config, sizeof g_last_config, "sk %s%s rows=%d split=%d wgs=%u cfg=%d",
                  sp.kind == SK_RANKK ? "rankk" : sp.kv ? "gemv_kv" : "gemv_mv",
                  sp.transpose ? "_t" : "", sp.kind == SK_GEMV ? sp.rows : 0, sp.splits,
                  sp.blocks, sp.kind == SK_RANKK ? 1 : 0);
    const GemmLaunchFn fn =
        sp.kind == SK_RANKK ? rankk_launcher(p.K) : gemv_launcher(sp.kv, sp.rows);
    if (fn == nullptr || sp.blocks == 0) return MT_ERR_UNSUPPORTED;
    hipError_t e = fn(p, sp.blocks, stream);
    if (e == hipErrorStreamCaptureUnsupported) e = hipSuccess;
    if (e != hipSuccess) return MT_ERR_HIP;
    if (sp.splits > 1) {
        if (p.ws_vec && (int64_t)p.M * p.batch <= 65535) {
            e = launch_skinny_reduce(p, stream);
        } else {
            const int64_t total = (int64_t)p.M * p.N * p.batch;
            const int64_t blocks = std::min<int64_t>((total + 255) / 256, 65536);
            hipLaunchKernelGGL(splitk_reduce_f32, dim3((unsigned)blocks), dim3(256), 0, stream, p);
            e = hipGetLastError();
        }
        if (e == hipErrorStreamCaptureUnsupported) e = hipSuccess;
        if (e != hipSuccess) return MT_ERR_HIP;
    }
    return MT_OK;
}

// Completes the plan-dependent fields of p (tile grid, split-K, vector
// epilogue flags), then launches the GEMM kernel and, for split-K, the
// deterministic reduction.  lb == L_IM selects the implicit-im2col kernel.
int launch_gemm(GemmParams& p, bool dl, int la, int lb, void* workspace, size_t ws_bytes,
                hipStream_t stream) {
    const int64_t M = p.M, N = p.N, K = p.K, batch = p.batch;
    const bool implicit = lb == L_IM || lb == L_IMW || lb == L_IMR;
    // 16-byte epilogue stores: four consecutive columns must be contiguous,
    // aligned, and (for a scattered output) never straddle a column group.
    p.c_vec = p.c_n == 1 && (N & 3) == 0 && ((uintptr_t)p.C & 15u) == 0 && (p.c_m & 3) == 0 &&
              (batch == 1 || (p.c_b & 3) == 0) &&
              (p.c_n_inner >= N || ((p.c_n_inner & 3) == 0 && (p.c_n_outer & 3) == 0 &&
                                    (p.c_n_inner2 <= 0 ||
                                     ((p.c_n_inner2 & 3) == 0 && (p.c_n_outer2 & 3) == 0))));
    // Row sums of A are fused only into a direct-to-LDS launch of two
    // mn-contiguous operands without split-K (the caller sees p.rowsum cleared
    // and computes them separately).
    // A batch-summed product of two k-contiguous operands fuses them too, as
    // partials per (split, batch entry) that its reduction sums for csum.
    const bool rs_part = p.part && la == L_KV && lb == L_KV && p.csum != nullptr;
    if (!rs_part && (batch != 1 || la != L_MV || lb != L_MV || p.part)) p.rowsum = nullptr;
    // The HBM-bound shapes (few rows or columns, or K <= 16) on the vector ALUs.
    if (!implicit && la != L_KVI && p.rowsum == nullptr && p.csum == nullptr && !p.part) {
        const SkinnyPlan sp =
            skinny_plan(M, N, K, batch, la, lb, p.c_n_inner < N, device_cu_count());
        if (sp.kind != SK_NONE) return launch_skinny(p, sp, workspace, ws_bytes, stream);
    }
    // The prefetching configurations' contract: vector layouts or the
    // weight-gradient operand (not the implicit-im2col one), a non-empty K
    // range.
    const bool wide_ok = dl && lb != L_IM && lb != L_IMR && K > 0;
    Plan plan;
    const bool im16_ok = dl && lb == L_IM;
    const bool forced = forced_plan(M, N, K, batch, dl, !implicit, wide_ok, &plan, im16_ok);
    // workspace a plan writes: split-K partials, or with p.part a slab per
    // split and batch entry even at one split
    auto need = [&](const Plan& pl) {
        return p.part ? part_ws_bytes(pl, M, N, batch) : pl.splits > 1 ? pl.ws_bytes : 0;
    };
    if (forced) {
        if (need(plan) > 0 && (workspace == nullptr || ws_bytes < need(plan)))
            return MT_ERR_WORKSPACE;
    } else {
        // the wave-split kernel takes every operand form but the implicit
        // convolution operands and the fused row sums
        const bool ksw_ok = !implicit && p.rowsum == nullptr;
        plan = make_plan(M, N, K, batch, device_cu_count(), true, dl, wide_ok, ksw_ok,
                         lb == L_IMW, im16_ok && kOfferDl16);
        if (need(plan) > 0 && (workspace == nullptr || ws_bytes < need(plan)))
            plan = make_plan(M, N, K, batch, device_cu_count(), false, dl, wide_ok, ksw_ok,
                             lb == L_IMW, im16_ok && kOfferDl16);
        if (need(plan) > 0 && (workspace == nullptr || ws_bytes < need(plan)))
            return MT_ERR_WORKSPACE;
    }
    if (!plan.dl || (plan.splits > 1 && !rs_part) || is_dl16_cfg(plan.cfg)) p.rowsum = nullptr;
    p.splits = plan.splits;
    p.k_per_split = plan.splits > 1 ? plan.kps : (int)std::max<int64_t>(K, 1);
    p.tiles_m = plan.tiles_m;
    p.tiles_n = plan.tiles_n;
    p.group_m = 4;
    const bool reduce = plan.splits > 1 || p.part;
    p.ws = reduce ? static_cast<float*>(workspace) : nullptr;
    p.ws_vec = p.ws != nullptr && ((uintptr_t)p.ws & 15u) == 0 && (N & 3) == 0;
    // Channel sums ride on the vector reduction only (one row per workgroup
    // row; a batch-summed product reduces to a single matrix)
    if (!p.ws_vec || (batch != 1 && !p.part)) p.csum = nullptr;
    // The fused row sums of a batch-summed product: partials after the slabs,
    // summed by the reduction in place of a second pass over csum_src.
    if (rs_part && p.rowsum != nullptr && p.csum != nullptr) {
        float* rows = p.ws + (int64_t)plan.splits * batch * M * N;
        p.rowsum = rows;
        p.csum_rows = rows;
    } else if (rs_part) {
        p.rowsum = nullptr;
    }

    const int64_t nblocks = (int64_t)plan.tiles_m * plan.tiles_n * plan.splits * batch;
    if (nblocks >= ((int64_t)1 << 31)) return MT_ERR_UNSUPPORTED;
    // The NCHW-view operand is built from halo patches in LDS when the
    // configuration's patches fit (same K order, operands and output).
    const bool halo = lb == L_IMR && p.cv.hp > 0 &&
                      halo_fits(p.cv, (int)(N / ((int64_t)p.cv.ho * p.cv.wo)), plan.cfg,
                                p.k_per_split, !forced);
    std::snprintf(g_last_config, sizeof g_last_config,
                  "%s %dx%d a=%s b=%s split=%d wgs=%lld cfg=%d%s",
                  plan.ksw ? "ksw" : plan.dl ? "dl" : "rs", plan.bm,
                  plan.bn, layout_name(la), layout_name(halo ? L_IMH : lb), plan.splits,
                  (long long)nblocks, plan.cfg,
                  p.part ? (p.csum_rows ? " batch-summed rows" : " batch-summed") : "");

    GemmLaunchFn fn = halo ? convh_launcher(plan.cfg)
                      : lb == L_IM || lb == L_IMR ? conv_launcher(plan.cfg, lb == L_IMR)
                      : lb == L_IMW ? convw_launcher(plan.cfg, (K & 15) != 0, la == L_KVI)
                      : p.rowsum != nullptr ? rowsum_launcher(plan.cfg, (K & 15) != 0, la == L_KV)
                                            : pick_launcher(plan, la, lb, (K & 15) != 0);
    if (fn == nullptr) return MT_ERR_UNSUPPORTED;
    hipError_t e = fn(p, (unsigned)nblocks, stream);
    if (e == hipErrorStreamCaptureUnsupported) e = hipSuccess;
    if (e != hipSuccess) return MT_ERR_HIP;
    if (reduce) {
        // A batch-summed product reduces splits x batch slabs into one C.
        GemmParams q = p;
        if (p.part) {
            q.splits = plan.splits * (int)batch;
            q.batch = 1;
            q.c_b = 0;
        }
        if (q.ws_vec) {
            const int nt =
                q.csum && !q.csum_rows ? csum_threads((int64_t)q.csum_n * q.csum_hw) : 256;
            const dim3 grid((unsigned)std::min<int64_t>((N / 4 + nt - 1) / nt, 64),
                            (unsigned)std::min<int64_t>(M * q.batch, 65535));
            if (q.csum && nt == 1024)
                hipLaunchKernelGGL((splitk_reduce_vec_f32<true, 1024>), grid, dim3(nt), 0, stream,
                                   q);
            else if (q.csum)
                hipLaunchKernelGGL(splitk_reduce_vec_f32<true>, grid, dim3(nt), 0, stream, q);
            else
                hipLaunchKernelGGL(splitk_reduce_vec_f32<false>, grid, dim3(nt), 0, stream, q);
        } else {
            const int64_t total = M * N * q.batch;
            const int64_t blocks = std::min<int64_t>((total + 255) / 256, 65536);
            hipLaunchKernelGGL(splitk_reduce_f32, dim3((unsigned)blocks), dim3(256), 0, stream, q);
        }
        if (capture_safe_last_error() != hipSuccess) return MT_ERR_HIP;
    }
    return MT_OK;
}

// Optional fused row sums of A (see GemmParams::rowsum); `done` reports
// whether the GEMM launch produced them.
struct RowSums {
    float* out;
    int64_t stride;
    float beta;
    bool done;
};

int run_gemm(const mt_mat_f32* A, const mt_mat_f32* B, const mt_mat_f32* C, int64_t c_n_inner,
             int64_t c_n_outer, const mt_epilogue_f32* ep, void* workspace, size_t ws_bytes,
             hipStream_t stream, RowSums* rows = nullptr) {
    int64_t M, N, K, batch;
    int rc = check_gemm(A, B, C, &M, &N, &K, &batch);
    if (rc != MT_OK) return rc;
    if (ep && ep->bias_axis != MT_BIAS_NONE) {
        if (ep->bias_axis != MT_BIAS_ROW && ep->bias_axis != MT_BIAS_COL) return MT_ERR_INVALID;
        if (!ep->bias || ep->bias_stride < 0) return MT_ERR_INVALID;
    }
    if (M == 0 || N == 0 || batch == 0) {
        std::snprintf(g_last_config, sizeof g_last_config, "empty");
        return MT_OK;
    }

    GemmParams p{};
    p.A = A->base ? A->base + A->offset : nullptr;
    p.a_mn = A->row_stride; p.a_k = A->col_stride; p.a_b = A->batch == 1 ? 0 : A->batch_stride;
    p.B = B->base ? B->base + B->offset : nullptr;
    p.b_mn = B->col_stride; p.b_k = B->row_stride; p.b_b = B->batch == 1 ? 0 : B->batch_stride;
    p.C = const_cast<float*>(C->base) + C->offset;
    p.c_m = C->row_stride; p.c_n = C->col_stride; p.c_b = C->batch_stride;
    p.c_n_inner = c_n_inner > 0 ? c_n_inner : N;
    p.c_n_outer = c_n_outer;
    p.bias = ep ? ep->bias : nullptr;
    p.bias_stride = ep ? ep->bias_stride : 0;
    p.bias_axis = ep ? ep->bias_axis : MT_BIAS_NONE;
    p.beta = ep ? ep->beta : 0.f;
    p.M = (int)M; p.N = (int)N; p.K = (int)K; p.batch = (int)batch;

    if (K == 0) {  // nothing to load: a K-free pass writes bias (+beta*C) or zeros
        p.A = p.B = nullptr;
    }
    const int la = K == 0 ? L_KS : classify(p.A, p.a_mn, p.a_k, M, K, p.a_b, p.a_b != 0);
    const int lb = K == 0 ? L_KS : classify(p.B, p.b_mn, p.b_k, N, K, p.b_b, p.b_b != 0);

    const bool dl = (la == L_KV || la == L_MV) && (lb == L_KV || lb == L_MV);
    if (rows && K > 0) {
        p.rowsum = rows->out;
        p.rowsum_stride = rows->stride;
        p.rowsum_beta = rows->beta;
        // A split-K plan cannot fuse them into the GEMM; its reduction launch
        // sums them instead when A is a transposed contiguous matrix (the
        // Linear dW = dYᵀ·X with dY [K][M]): the channel sums with K images of
        // one position.  (A separate column sum had one workgroup per 64
        // columns: 216 us for db of an 8192 x 512 dY.)
        if (batch == 1 && p.a_mn == 1 && p.a_k == M && rows->stride == 1) {
            p.csum_src = p.A;
            p.csum = rows->out;
            p.csum_n = (int)K;
            p.csum_hw = 1;
            p.csum_beta = rows->beta;
        }
    }
    rc = launch_gemm(p, dl, la, lb, workspace, ws_bytes, stream);
    if (rows) rows->done = rc == MT_OK && (p.rowsum != nullptr || p.csum != nullptr);
    return rc;
}

// Device address of the current GPU's copy of `scratch`, looked up on the
// first call on that GPU (with that GPU current) and kept per GPU.
constexpr int kMaxDevices = 64;
struct NoallocScratch {
    std::once_flag once;
    void* ptr = nullptr;
    hipError_t err = hipSuccess;
};
NoallocScratch g_noalloc[kMaxDevices];

int noalloc_scratch(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MT_ERR_HIP;
    NoallocScratch& sc = g_noalloc[dev];
    std::call_once(sc.once, [&sc] { sc.err = hipGetSymbolAddress(&sc.ptr, HIP_SYMBOL(scratch)); });
    if (sc.err != hipSuccess || sc.ptr == nullptr) return MT_ERR_HIP;
    *out = sc.ptr;
    return MT_OK;
}

size_t gemm_ws(const mt_mat_f32* A, const mt_mat_f32* B, const mt_mat_f32* C) {
    int64_t M, N, K, batch;
    if (check_gemm(A, B, C, &M, &N, &K, &batch) != MT_OK || M == 0 || N == 0 || batch == 0)
        return 0;
    return plan_ws(M, N, K, batch, device_cu_count());
}

// ---- column sums (Linear bias gradient) ------------------------------------
// A workgroup takes 64 columns as 16 groups of 4 (16-byte loads when the
// columns are contiguous and aligned) and 16 row slices; slice g sums the
// rows g, g+16, ... with four accumulators in flight (rows g + 16*(4i + u)
// into accumulator u), then the accumulators and the slices are added in a
// fixed order: deterministic.  (One load in flight per thread and 4 slices
// had taken 216 us for an 8192 x 512 input.)
__global__ void __launch_bounds__(256)
colsum_f32(const float* X, int64_t rs, int64_t cs, int R, int Cn, float* out, int64_t os,
           float beta) {
    __shared__ f32x4 part[16][16];
    const int cq = threadIdx.x & 15, g = threadIdx.x >> 4;
    const int c0 = blockIdx.x * 64 + 4 * cq;
    const bool vec = cs == 1 && c0 + 3 < Cn && (rs & 3) == 0 && ((uintptr_t)(X + c0) & 15u) == 0;
    auto row = [&](int r) {
        const float* q = X + (int64_t)r * rs;
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
        if (vec) {
            x = *reinterpret_cast<const f32x4*>(q + c0);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (c0 + e < Cn) x[e] = q[(int64_t)(c0 + e) * cs];
        }
        return x;
    };
    f32x4 acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (c0 < Cn) {
        int r = g;
        for (; r + 48 < R; r += 64) {
            f32x4 x[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) x[u] = row(r + 16 * u);
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[u] += x[u];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (r + 16 * u < R) acc[u] += row(r + 16 * u);
    }
    part[g][cq] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    __syncthreads();
    if (g == 0 && c0 < Cn) {
        f32x4 v = part[0][cq];
#pragma unroll
        for (int w = 1; w < 16; ++w) v += part[w][cq];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (c0 + e >= Cn) break;
            float* d = out + (int64_t)(c0 + e) * os;
            *d = (beta != 0.f ? beta * *d : 0.f) + v[e];
        }
    }
}

// ---- im2col: col[k][np], k = (c*kh + r)*kw + s, np = (img*Ho + oh)*Wo + ow --
// Each thread owns one np column and walks KCHUNK consecutive k rows, so the
// np decomposition is done once and the stores are coalesced along np.
constexpr int kIm2colK = 32;
__global__ void __launch_bounds__(256)
im2col_f32(const float* in, int64_t sn, int64_t sc, int64_t sh, int64_t sw, float* col, int H,
           int W, int kh, int kw, int st, int pad, int Ho, int Wo, int64_t NP, int64_t Kg) {
    const int64_t np = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (np >= NP) return;
    const int64_t hw = (int64_t)Ho * Wo;
    const int64_t img = np / hw;
    const int rem = (int)(np - img * hw);
    const int oh = rem / Wo, ow = rem - oh * Wo;
    const int iy0 = oh * st - pad, ix0 = ow * st - pad;
    const float* src = in + img * sn;
    int64_t k = (int64_t)blockIdx.y * kIm2colK;
    const int64_t kend = std::min<int64_t>(Kg, k + kIm2colK);
    int s = (int)(k % kw);
    int r = (int)((k / kw) % kh);
    int c = (int)(k / ((int64_t)kw * kh));
    for (; k < kend; ++k) {
        const int iy = iy0 + r, ix = ix0 + s;
        float v = 0.f;
        if (iy >= 0 && iy < H && ix >= 0 && ix < W) v = src[c * sc + iy * sh + ix * sw];
        col[k * NP + np] = v;
        if (++s == kw) { s = 0; if (++r == kh) { r = 0; ++c; } }
    }
}

// a*b for a, b >= 0, or -1 once the product would reach 2^62 (or an operand
// is already -1): sizes built from it never wrap.
int64_t mul_capped(int64_t a, int64_t b) {
    constexpr int64_t cap = (int64_t)1 << 62;
    if (a < 0 || b < 0) return -1;
    if (a != 0 && b >= cap / a) return -1;
    return a * b;
}

bool conv_dims(const mt_conv2d_desc* d, int64_t* Ho, int64_t* Wo) {
    if (!d) return false;
    for (int64_t v : {d->n, d->c_in, d->h, d->w, d->c_out, d->kh, d->kw, d->stride, d->pad})
        if (v < 0 || v >= kMaxDim) return false;
    if (d->kh < 1 || d->kw < 1 || d->stride < 1) return false;
    *Ho = (d->h + 2 * d->pad < d->kh) ? 0 : (d->h + 2 * d->pad - d->kh) / d->stride + 1;
    *Wo = (d->w + 2 * d->pad < d->kw) ? 0 : (d->w + 2 * d->pad - d->kw) / d->stride + 1;
    // GEMM extents are 32-bit inside the kernels; tensor sizes must not wrap.
    const int64_t kg = mul_capped(mul_capped(d->c_in, d->kh), d->kw);
    const int64_t np = mul_capped(mul_capped(d->n, *Ho), *Wo);
    const int64_t in_elems = mul_capped(mul_capped(mul_capped(d->n, d->c_in), d->h), d->w);
    if (kg < 0 || np < 0 || in_elems < 0 || mul_capped(np, d->c_out) < 0 ||
        mul_capped(kg, d->c_out) < 0)
        return false;
    return kg < kMaxDim && np < kMaxDim;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

void conv_gemm_views(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo, const float* weight,
                     const float* col, float* output, mt_mat_f32* A, mt_mat_f32* B,
                     mt_mat_f32* C) {
    const int64_t kg = d->c_in * d->kh * d->kw, np = d->n * Ho * Wo;
    *A = mt_mat_f32{weight, 0, d->c_out, kg, kg, 1, 1, 0};
    *B = mt_mat_f32{col, 0, kg, np, np, 1, 1, 0};
    // C(m = c_out, n = np) -> output[img][c_out][hw]; the column scatter is
    // passed separately (inner extent Ho*Wo, outer stride c_out*Ho*Wo).
    *C = mt_mat_f32{output, 0, d->c_out, np, Ho * Wo, 1, 1, 0};
}


// The implicit-GEMM convolution gathers 16 consecutive channels per K-chunk
// from a channels-last copy of the input, so it needs c_in % 16 == 0.
bool implicit_geometry(const mt_conv2d_desc* d) {
    return d->c_in > 0 && (d->c_in & 15) == 0;
}

// Workspace of the implicit path: channels-last input, OHWI weights, split-K.
struct ImplicitWs {
    size_t xt, wt;
};
ImplicitWs implicit_ws(const mt_conv2d_desc* d) {
    return {align_up((size_t)d->n * d->c_in * d->h * d->w * sizeof(float), 256),
            align_up((size_t)d->c_out * d->c_in * d->kh * d->kw * sizeof(float), 256)};
}

// ---- support kernels ---------------------------------------------------------
__global__ void __launch_bounds__(256) fill_f32(float* p, int64_t n, float v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// Y = alpha*X + beta*Y over (batch, rows, cols) views.  Grid-stride over
// items of one row: four columns (16-byte loads and stores) when vec says both
// rows are unit-stride and aligned, else one column.  Index math is 32-bit
// when the item count allows (I = int or int64_t).
template <typename I>
__device__ __forceinline__ void axpby_items(const float* X, int64_t xb, int64_t xr, int64_t xc,
                                            float alpha, float* Y, int64_t yb, int64_t yr,
                                            int64_t yc, float beta, I rows, I per_row, I total,
                                            bool vec) {
    for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (I)gridDim.x * blockDim.x) {
        const I row = i / per_row, c = i - row * per_row;
        const I b = row / rows, r = row - b * rows;
        const float* x = X + b * xb + r * xr;
        float* y = Y + b * yb + r * yr;
        if (vec) {
            f32x4 v = alpha * *reinterpret_cast<const f32x4*>(x + 4 * (int64_t)c);
            f32x4* d = reinterpret_cast<f32x4*>(y + 4 * (int64_t)c);
            if (beta != 0.f) v += beta * *d;
            *d = v;
        } else {
            const float v = alpha * x[c * xc];
            float* d = y + c * yc;
            *d = beta != 0.f ? v + beta * *d : v;
        }
    }
}

__global__ void __launch_bounds__(256)
axpby_f32(const float* X, int64_t xb, int64_t xr, int64_t xc, float alpha, float* Y, int64_t yb,
          int64_t yr, int64_t yc, float beta, int64_t rows, int64_t per_row, int64_t total,
          int vec) {
    if (total < ((int64_t)1 << 31))
        axpby_items<int>(X, xb, xr, xc, alpha, Y, yb, yr, yc, beta, (int)rows, (int)per_row,
                         (int)total, vec != 0);
    else
        axpby_items<int64_t>(X, xb, xr, xc, alpha, Y, yb, yr, yc, beta, rows, per_row, total,
                             vec != 0);
}

unsigned grid_for(int64_t total) {
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>((total + 255) / 256, 8192));
}

hipError_t launch_axpby(const float* X, int64_t xb, int64_t xr, int64_t xc, float alpha,
                        float* Y, int64_t yb, int64_t yr, int64_t yc, float beta, int64_t batch,
                        int64_t rows, int64_t cols, hipStream_t s) {
    const int64_t nrows = batch * rows;
    if (nrows == 0 || cols == 0) return hipSuccess;
    const bool vec = xc == 1 && yc == 1 && (cols & 3) == 0 && (xr & 3) == 0 && (yr & 3) == 0 &&
                     (batch == 1 || ((xb & 3) == 0 && (yb & 3) == 0)) &&
                     ((uintptr_t)X & 15u) == 0 && ((uintptr_t)Y & 15u) == 0;
    const int64_t per_row = vec ? cols / 4 : cols;
    const int64_t total = nrows * per_row;
    hipLaunchKernelGGL(axpby_f32, dim3(grid_for(total)), dim3(256), 0, s, X, xb, xr, xc, alpha,
                       Y, yb, yr, yc, beta, rows, per_row, total, vec ? 1 : 0);
    return capture_safe_last_error();
}


// dX[img][c][y][x] = Σ_{r,s} dcol[(c*kh + r)*kw + s][(img*Ho + oh)*Wo + ow] over the
// (r, s) whose window position (oh, ow) covers (y, x): a gather, so every input
// element is written once, in a fixed (r, s) order -- no atomics.
__global__ void __launch_bounds__(256)
col2im_gather_f32(const float* dcol, float* dx, int C, int H, int W, int kh, int kw, int st,
                  int pad, int Ho, int Wo, int64_t NP, int64_t total) {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int x = (int)(e % W);
        const int64_t t1 = e / W;
        const int y = (int)(t1 % H);
        const int64_t t2 = t1 / H;
        const int c = (int)(t2 % C);
        const int64_t img = t2 / C;
        float acc = 0.f;
        for (int r = 0; r < kh; ++r) {
            const int ty = y + pad - r;
            if (ty < 0 || ty % st) continue;
            const int oh = ty / st;
            if (oh >= Ho) continue;
            for (int s = 0; s < kw; ++s) {
                const int tx = x + pad - s;
                if (tx < 0 || tx % st) continue;
                const int ow = tx / st;
                if (ow >= Wo) continue;
                const int64_t k = ((int64_t)c * kh + r) * kw + s;
                acc += dcol[k * NP + (img * Ho + oh) * Wo + ow];
            }
        }
        dx[e] = acc;
    }
}

// out[img][c][q] = c < C ? in[img][c][q] : 0 for c < CP (dense NCHW both):
// blockIdx.y walks the output planes, threads the positions, V floats each
// (16-byte accesses when V == 4: HW % 4 == 0 and both tensors aligned).
template <int V>
__global__ void __launch_bounds__(256)
pad_channels_f32(const float* in, float* out, int C, int CP, int64_t planes, int64_t HW) {
    const int64_t items = HW / V;
    for (int64_t pl = blockIdx.y; pl < planes; pl += gridDim.y) {
        const int64_t img = pl / CP;
        const int c = (int)(pl - img * CP);
        float* o = out + pl * HW;
        const float* i = c < C ? in + (img * C + c) * HW : nullptr;
        for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < items;
             q += (int64_t)gridDim.x * blockDim.x) {
            if constexpr (V == 4) {
                const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
                reinterpret_cast<f32x4*>(o)[q] = i ? reinterpret_cast<const f32x4*>(i)[q] : zero;
            } else {
                o[q] = i ? i[q] : 0.f;
            }
        }
    }
}

hipError_t launch_pad_channels(const float* in, float* out, int64_t n, int C, int CP, int64_t HW,
                               hipStream_t s) {
    const bool vec = (HW & 3) == 0 && ((uintptr_t)in & 15u) == 0 && ((uintptr_t)out & 15u) == 0;
    const int64_t items = vec ? HW / 4 : HW, planes = n * CP;
    const dim3 grid((unsigned)std::max<int64_t>(1, std::min<int64_t>((items + 255) / 256, 256)),
                    (unsigned)std::max<int64_t>(1, std::min<int64_t>(planes, 65535)));
    if (vec)
        hipLaunchKernelGGL(pad_channels_f32<4>, grid, dim3(256), 0, s, in, out, C, CP, planes, HW);
    else
        hipLaunchKernelGGL(pad_channels_f32<1>, grid, dim3(256), 0, s, in, out, C, CP, planes, HW);
    return capture_safe_last_error();
}

// db[c] = beta*db[c] + Σ_{img, hw} dY[img][c][hw]; one workgroup per channel
// (block_channel_sum: fixed order, deterministic).
template <int NT>
__global__ void __launch_bounds__(NT)
conv_bias_grad_f32(const float* dy, float* db, int N, int C, int64_t HW, float beta) {
    __shared__ float red[NT];
    const int c = blockIdx.x;
    const float r = block_channel_sum<NT, kCsumLoads>(dy, C, c, N, HW, red);
    if (threadIdx.x == 0) db[c] = (beta != 0.f ? beta * db[c] : 0.f) + r;
}

// dY [n][c_out][hw] -> dYt [c_out][n][hw] (contiguous), through the axpby kernel
// (batch = channel, rows = images, cols = positions).
hipError_t transpose_dy(const mt_conv2d_desc* d, int64_t hw, const float* dy, float* dyt,
                        hipStream_t s) {
    return launch_axpby(dy, hw, d->c_out * hw, 1, 1.0f, dyt, d->n * hw, hw, 1, 0.0f, d->c_out,
                        d->n, hw, s);
}

// One layout change: out[b][j][i] = in[b*sb + i*si + (j / jw)*sj1 + (j % jw)*sj0],
// out dense [B][J][I], moved in TI x TJ tiles (2048 elements, 8 per thread)
// through LDS.  Reads run along j (coalesced when sj0 == 1), or along i when
// ri is set (si == 1: a batched copy that only reorders the outer
// dimensions); writes run along i.  Where rows are dense and 16-byte aligned
// (vec) the accesses are 16 bytes wide, and a batched copy skips LDS.  With b = image, i = channel, j = pixel it
// turns an NCHW view into channels-last; with b = c_out, i = c_in, j = filter
// tap it turns OIHW weights into OHWI.  Tiles are TI x TJ = 32 x 64, or
// 64 x 32 when J <= 32, or 128 x 16 when J <= 16 (filter taps), so that few
// threads idle.
struct TJob {
    const float* in;
    float* out;
    int64_t sb, si, sj1, sj0;
    int jw, I, J, B;
    int lti, ltj;      // log2 of the tile's extent along i and j
    int ti, tj;        // tiles along i and j
    int ri;            // read along i
    int vec;           // 16-byte accesses: 1 tiled transpose, 2 flat row copy (ri, jw == 1)
    int64_t blocks;    // ti * tj * B, or 512-vector blocks of the flat copy
};

TJob tjob(const float* in, int64_t sb, int64_t si, int64_t sj1, int64_t sj0, int64_t jw,
          int64_t I, int64_t J, int64_t B, float* out) {
    TJob t{};
    t.in = in; t.out = out;
    t.sb = sb; t.si = si; t.sj1 = sj1; t.sj0 = sj0;
    t.jw = (int)jw; t.I = (int)I; t.J = (int)J; t.B = (int)B;
    t.ltj = J <= 16 ? 4 : J <= 32 ? 5 : 6;
    t.lti = 11 - t.ltj;
    t.ti = (int)((I + (1 << t.lti) - 1) >> t.lti);
    t.tj = (int)((J + (1 << t.ltj) - 1) >> t.ltj);
    t.ri = si == 1 && sj0 != 1;
    // 16-byte loads and stores: every row start of the input and the output
    // 16-byte aligned and the rows whole multiples of 4 floats
    const bool aligned = ((uintptr_t)in & 15u) == 0 && ((uintptr_t)out & 15u) == 0 &&
                         (I & 3) == 0 && (sb & 3) == 0;
    if (aligned && !t.ri && J > 32 && sj0 == 1 && sj1 == jw && (J & 3) == 0 && (si & 3) == 0) {
        // j is linear and contiguous in the input: 64 x 32 or 32 x 64 tiles,
        // whichever covers I x J with fewer
        t.vec = 1;
        const int64_t n32 = ((I + 63) >> 6) * ((J + 31) >> 5), n64 = ((I + 31) >> 5) * ((J + 63) >> 6);
        t.ltj = n32 < n64 ? 5 : 6;
        t.lti = 11 - t.ltj;
        t.ti = (int)((I + (1 << t.lti) - 1) >> t.lti);
        t.tj = (int)((J + (1 << t.ltj) - 1) >> t.ltj);
    } else if (aligned && t.ri && jw == 1 && (sj1 & 3) == 0) {
        t.vec = 2;   // a copy of i-contiguous rows
    }
    t.blocks = (I == 0 || J == 0) ? 0
               : t.vec == 2      ? ((I >> 2) * J * B + 511) >> 9
                                 : (int64_t)t.ti * t.tj * B;
    return t;
}

// Up to two independent layout changes in one launch (the blocks of job 0,
// then those of job 1), so that a convolution's input and weight transforms
// cost one launch.  xcd: the grid is 8 * (ceil(blocks0 / 8) + ceil(blocks1 / 8))
// and block ids are remapped so that each XCD (which takes every 8th id) runs
// a contiguous eighth of each job's tiles: neighbouring tiles share the cache
// lines at their edges, and then share them in one L2.  Otherwise a
// grid-stride loop over the tiles.
__global__ void __launch_bounds__(256) transpose_f32(TJob j0, TJob j1, int xcd) {
    __shared__ float tile[128 * 17];   // [i - i0][j - j0], row pitch TJ + 1
    const int t = threadIdx.x;
    const int64_t total = j0.blocks + j1.blocks;
    int64_t first = blockIdx.x, stride = gridDim.x;
    if (xcd) {
        const int64_t per0 = (j0.blocks + 7) >> 3, per1 = (j1.blocks + 7) >> 3;
        const int64_t x = blockIdx.x & 7, q = blockIdx.x >> 3;
        first = q < per0 ? (x * per0 + q < j0.blocks ? x * per0 + q : total)
                         : (x * per1 + q - per0 < j1.blocks ? j0.blocks + x * per1 + q - per0
                                                             : total);
        stride = total;
    }
    for (int64_t blk = first; blk < total; blk += stride) {
        const bool second = blk >= j0.blocks;
        const TJob jb = second ? j1 : j0;
        int64_t r = second ? blk - j0.blocks : blk;
        if (jb.vec == 2) {
            // flat copy of I-float rows, row = b * J + j: 512 16-byte groups
            // per block, two per thread
            const int64_t q4 = jb.I >> 2, n4 = q4 * jb.J * jb.B;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int64_t g = r * 512 + k * 256 + t;
                if (g >= n4) break;
                int64_t row, iq, b, j;
                if (n4 <= INT32_MAX) {
                    const uint32_t rw = (uint32_t)g / (uint32_t)q4;
                    const uint32_t bb = rw / (uint32_t)jb.J;
                    row = rw; iq = (uint32_t)g - rw * (uint32_t)q4;
                    b = bb; j = rw - bb * (uint32_t)jb.J;
                } else {
                    row = g / q4; iq = g - row * q4; b = row / jb.J; j = row - b * jb.J;
                }
                *reinterpret_cast<f32x4*>(jb.out + row * jb.I + 4 * iq) =
                    *reinterpret_cast<const f32x4*>(jb.in + b * jb.sb + j * jb.sj1 + 4 * iq);
            }
            continue;
        }
        const int per_b = jb.ti * jb.tj;
        const int b = (int)(r / per_b);
        r -= (int64_t)b * per_b;
        const int TI = 1 << jb.lti, TJ = 1 << jb.ltj, pitch = TJ + 1;
        const int i0 = (int)(r / jb.tj) << jb.lti, jt0 = (int)(r % jb.tj) << jb.ltj;
        const float* src = jb.in + (int64_t)b * jb.sb;
        if (jb.vec == 1) {
            // two 16-byte loads along j and two 16-byte stores along i per
            // thread (TI x TJ = 64 x 32 or 32 x 64)
            const int jq = t & ((TJ >> 2) - 1), ir = t >> (jb.ltj - 2), rstep = 256 >> (jb.ltj - 2);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int il = ir + k * rstep, i = i0 + il, j = jt0 + 4 * jq;
                f32x4 x = {0.f, 0.f, 0.f, 0.f};
                if (i < jb.I && j < jb.J)
                    x = *reinterpret_cast<const f32x4*>(src + (int64_t)i * jb.si + j);
#pragma unroll
                for (int e = 0; e < 4; ++e) tile[il * pitch + 4 * jq + e] = x[e];
            }
            __syncthreads();
            const int iq = t & ((TI >> 2) - 1), jr = t >> (jb.lti - 2), jstep = 256 >> (jb.lti - 2);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int jl = jr + k * jstep, j = jt0 + jl, i = i0 + 4 * iq;
                if (i < jb.I && j < jb.J) {
                    const float* c = tile + (4 * iq) * pitch + jl;
                    const f32x4 x = {c[0], c[pitch], c[2 * pitch], c[3 * pitch]};
                    *reinterpret_cast<f32x4*>(jb.out + ((int64_t)b * jb.J + j) * jb.I + i) = x;
                }
            }
            __syncthreads();
            continue;
        }
        // i-major lanes (consecutive i) for ri reads and for the writes;
        // j-major lanes (consecutive j) for the other reads
        const int im_i = t & (TI - 1), im_j = t >> jb.lti, im_step = 256 >> jb.lti;
        const int jm_j = t & (TJ - 1), jm_i = t >> jb.ltj, jm_step = 256 >> jb.ltj;
        float v[8];
        if (!jb.ri) {
            // this thread's j (and its offset) is fixed; i steps by jm_step
            const int j = jt0 + jm_j;
            const bool jok = j < jb.J;
            const int jh = jok ? j / jb.jw : 0;
            const float* q = src + (int64_t)(i0 + jm_i) * jb.si + (int64_t)jh * jb.sj1 +
                             (int64_t)(j - jh * jb.jw) * jb.sj0;
            const int64_t qstep = (int64_t)jm_step * jb.si;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                v[k] = jok && i0 + jm_i + k * jm_step < jb.I ? q[k * qstep] : 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) tile[(jm_i + k * jm_step) * pitch + jm_j] = v[k];
        } else {
            // this thread's i is fixed (si == 1); j steps by im_step
            const int i = i0 + im_i;
            const bool iok = i < jb.I;
            if (jb.jw == 1) {   // j -> offset j * sj1, no division
                const float* q = src + i + (int64_t)(jt0 + im_j) * jb.sj1;
                const int64_t qstep = (int64_t)im_step * jb.sj1;
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    v[k] = iok && jt0 + im_j + k * im_step < jb.J ? q[k * qstep] : 0.f;
            } else {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const int j = jt0 + im_j + k * im_step;
                    v[k] = 0.f;
                    if (iok && j < jb.J) {
                        const int jh = j / jb.jw;
                        v[k] = src[i + (int64_t)jh * jb.sj1 + (int64_t)(j - jh * jb.jw) * jb.sj0];
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) tile[im_i * pitch + im_j + k * im_step] = v[k];
        }
        __syncthreads();
        {
            const int i = i0 + im_i;
            float* o = jb.out + ((int64_t)b * jb.J + jt0 + im_j) * jb.I + i;
            const int64_t ostep = (int64_t)im_step * jb.I;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (i < jb.I && jt0 + im_j + k * im_step < jb.J)
                    o[k * ostep] = tile[im_i * pitch + im_j + k * im_step];
        }
        __syncthreads();
    }
}

hipError_t launch_transposes(const TJob& a, const TJob& b, hipStream_t s) {
    const int64_t total = a.blocks + b.blocks;
    if (total == 0) return hipSuccess;
    const int64_t xgrid = 8 * (((a.blocks + 7) >> 3) + ((b.blocks + 7) >> 3));
    const bool xcd = xgrid <= ((int64_t)1 << 20);
    const unsigned grid = (unsigned)(xcd ? xgrid : (int64_t)1 << 20);
    hipLaunchKernelGGL(transpose_f32, dim3(grid), dim3(256), 0, s, a, b, xcd ? 1 : 0);
    return capture_safe_last_error();
}

hipError_t launch_transpose(const float* in, int64_t sb, int64_t si, int64_t sj1, int64_t sj0,
                            int64_t jw, int64_t I, int64_t J, int64_t B, float* out,
                            hipStream_t s) {
    return launch_transposes(tjob(in, sb, si, sj1, sj0, jw, I, J, B, out), TJob{}, s);
}

// Element strides of a dense NCHW tensor.
void dense_strides(const mt_conv2d_desc* d, int64_t st[4]) {
    st[3] = 1; st[2] = d->w; st[1] = d->h * d->w; st[0] = d->c_in * d->h * d->w;
}

hipError_t launch_im2col(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo, const float* input,
                         const int64_t in_st[4], float* col, hipStream_t s) {
    const int64_t kg = d->c_in * d->kh * d->kw, np = d->n * Ho * Wo;
    dim3 grid((unsigned)((np + 255) / 256), (unsigned)((kg + kIm2colK - 1) / kIm2colK));
    hipLaunchKernelGGL(im2col_f32, grid, dim3(256), 0, s, input, in_st[0], in_st[1], in_st[2],
                       in_st[3], col, (int)d->h, (int)d->w, (int)d->kh, (int)d->kw,
                       (int)d->stride, (int)d->pad, (int)Ho, (int)Wo, np, kg);
    return capture_safe_last_error();
}

// Implicit-GEMM convolution: C[c_out, np] = Wt[c_out, kg] · im2col(xt)[kg, np]
// with k = (r*kw + s)*c_in + ci, the im2col operand gathered by the kernel
// from a channels-last input xt (the input itself when it already is one,
// else a transposed copy in the workspace) and Wt the OHWI weights, which
// wjob writes to wsp + implicit_ws(d).xt in the same launch as the input's
// transpose.  Needs implicit_geometry(d) and ws_bytes >= xt + wt.
int run_conv_implicit(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo, const float* input,
                      const int64_t in_strides[4], const float* bias, float* output, char* wsp,
                      size_t ws_bytes, const TJob& wjob, hipStream_t s) {
    const ImplicitWs iw = implicit_ws(d);
    const int64_t c = d->c_in, kg = c * d->kh * d->kw, hw = Ho * Wo, np = d->n * hw;
    const bool nhwc = in_strides[1] == 1 && in_strides[3] == c && in_strides[2] == d->w * c &&
                      (in_strides[0] & 3) == 0 && ((uintptr_t)input & 15u) == 0;
    const float* xt = input;
    int64_t img_stride = in_strides[0];
    TJob xjob{};
    if (!nhwc) {
        float* buf = reinterpret_cast<float*>(wsp);
        xjob = tjob(input, in_strides[0], in_strides[1], in_strides[2], in_strides[3], d->w, c,
                    d->h * d->w, d->n, buf);
        xt = buf;
        img_stride = d->h * d->w * c;
    }
    if (launch_transposes(xjob, wjob, s) != hipSuccess) return MT_ERR_HIP;
    GemmParams p{};
    p.A = reinterpret_cast<const float*>(wsp + iw.xt); p.a_mn = kg; p.a_k = 1; p.a_b = 0;
    p.B = xt;
    p.C = output; p.c_m = hw; p.c_n = 1; p.c_b = 0;
    p.c_n_inner = hw; p.c_n_outer = d->c_out * hw;
    p.bias = bias; p.bias_stride = 1; p.bias_axis = bias ? MT_BIAS_ROW : MT_BIAS_NONE;
    p.beta = 0.f;
    p.M = (int)d->c_out; p.N = (int)np; p.K = (int)kg; p.batch = 1;
    ConvGeom& g = p.cv;
    g.img_stride = img_stride;
    g.c = (int)c; g.h = (int)d->h; g.w = (int)d->w;
    g.kh = (int)d->kh; g.kw = (int)d->kw; g.stride = (int)d->stride; g.pad = g.pad_w = (int)d->pad;
    g.ho = (int)Ho; g.wo = (int)Wo;
    return launch_gemm(p, true, L_KV, L_IM, wsp + iw.xt + iw.wt, ws_bytes - iw.xt - iw.wt, s);
}

// The implicit-GEMM convolution over an NCHW view (L_IMR) reads the OIHW
// weights as its A operand in 16-byte rows: kg % 4 == 0 (weights that are not
// 16-byte aligned are first copied to the workspace, nchw_weight_ws bytes).
// Its window test adds a tap to the window origin in 32-bit arithmetic, so
// the padded extents stay below 2^30 (a tap never exceeds them when an
// output exists).
// 1x1 kernel, stride 1, no padding, c_in and the positions per image
// multiples of 4: the convolution is one product per image over the NCHW
// tensors themselves (Y_b = W·X_b, dX_b = Wᵀ·dY_b, dW = Σ_b dY_b·X_bᵀ), with
// no layout copy and no scattered output.  Against the channels-last implicit
// path (which transposes the input or dY first), graph-timed at batch 32:
// 56x56 256->64 forward 38.1 against 74.3 us, dX 41.0 against 62.2, dW +
// db about 37 against 92.4.
bool pointwise(const mt_conv2d_desc* d) {
    return d->kh == 1 && d->kw == 1 && d->stride == 1 && d->pad == 0 && d->c_in > 0 &&
           (d->c_in & 3) == 0 && ((d->h * d->w) & 3) == 0 && d->h * d->w < kMaxDim;
}

// Workspace of a batch-summed product (GemmParams::part) under any plan the
// launcher can take for it.
size_t part_plan_ws(int64_t M, int64_t N, int64_t K, int64_t batch, int cus) {
    size_t ws = 0;
    for (bool dl : {false, true})
        for (bool wide : {false, true})
            for (bool ksw : {false, true})
                ws = std::max(ws, part_ws_bytes(make_plan(M, N, K, batch, cus, true, dl, wide, ksw),
                                                M, N, batch));
    Plan forced;
    if (forced_plan(M, N, K, batch, true, true, true, &forced))
        ws = std::max(ws, part_ws_bytes(forced, M, N, batch));
    return align_up(ws, 256);
}

bool nchw_implicit(const mt_conv2d_desc* d) {
    const int64_t kg = d->c_in * d->kh * d->kw;
    constexpr int64_t kWin = (int64_t)1 << 30;
    return kg > 0 && (kg & 3) == 0 && d->h * d->w < kMaxDim && d->h + 2 * d->pad < kWin &&
           d->w + 2 * d->pad < kWin;
}
size_t nchw_weight_ws(const mt_conv2d_desc* d) {
    return align_up((size_t)d->c_out * d->c_in * d->kh * d->kw * sizeof(float), 256);
}

// Implicit-GEMM convolution of an NCHW view (any strides): C[c_out, np] =
// W[c_out, kg] · im2col(x)[kg, np] with k = (ci*kh + r)*kw + s, the weights'
// own order, so neither operand is copied: the kernel gathers the im2col
// operand from the view through in_strides.  The workspace holds only split-K
// partials.  Needs nchw_implicit(d) and a 16-byte-aligned weight.
int run_conv_nchw(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo, const float* input,
                  const int64_t in_strides[4], const float* weight, const float* bias,
                  float* output, void* workspace, size_t ws_bytes, hipStream_t s) {
    const int64_t kg = d->c_in * d->kh * d->kw, hw = Ho * Wo, np = d->n * hw;
    GemmParams p{};
    p.A = weight; p.a_mn = kg; p.a_k = 1; p.a_b = 0;
    p.B = input;
    p.C = output; p.c_m = hw; p.c_n = 1; p.c_b = 0;
    p.c_n_inner = hw; p.c_n_outer = d->c_out * hw;
    p.bias = bias; p.bias_stride = 1; p.bias_axis = bias ? MT_BIAS_ROW : MT_BIAS_NONE;
    p.beta = 0.f;
    p.M = (int)d->c_out; p.N = (int)np; p.K = (int)kg; p.batch = 1;
    ConvGeom& g = p.cv;
    g.img_stride = in_strides[0];
    g.sc = in_strides[1]; g.sh = in_strides[2]; g.sw = in_strides[3];
    g.c = (int)d->c_in; g.h = (int)d->h; g.w = (int)d->w;
    g.kh = (int)d->kh; g.kw = (int)d->kw; g.stride = (int)d->stride; g.pad = g.pad_w = (int)d->pad;
    g.ho = (int)Ho; g.wo = (int)Wo;
    set_halo_geometry(g);
    return launch_gemm(p, true, L_KV, L_IMR, workspace, ws_bytes, s);
}

// The implicit weight gradient reads 4 channels of one tap per 16-byte vector
// (c_in % 4 == 0) and dYt [c_out][np] rows as 16-byte vectors (np % 4 == 0).
bool implicit_dw(const mt_conv2d_desc* d, int64_t np) {
    return np > 0 && (d->c_in & 3) == 0 && (np & 3) == 0 && d->h * d->w < kMaxDim;
}

// A layer whose c_in is not a multiple of 4 (the RGB stem) takes the implicit
// weight gradient on its input padded with zero channels to c_in rounded up
// to 4 (d4), where that adds at most a third of the work (c_in 3, 6, 7, 10,
// 11, ...); the real channels of the padded gradient are then copied out.
// The 7x7 stride-2 stem at batch 32: dW + db 231.8 against 288 us on the
// column path.
bool dw_padded(const mt_conv2d_desc* d, int64_t np, mt_conv2d_desc* d4) {
    if (d->c_in <= 0 || (d->c_in & 3) == 0) return false;
    const int64_t cp = (d->c_in + 3) / 4 * 4;
    if (3 * cp > 4 * d->c_in) return false;
    *d4 = *d;
    d4->c_in = cp;
    int64_t ho, wo;
    return conv_dims(d4, &ho, &wo) && implicit_dw(d4, np);
}
struct DwPadWs {
    size_t xp, dw4;   // the padded input, the padded weight gradient
};
DwPadWs dw_pad_ws(const mt_conv2d_desc* d4) {
    return {align_up((size_t)d4->n * d4->c_in * d4->h * d4->w * sizeof(float), 256),
            align_up((size_t)d4->c_out * d4->c_in * d4->kh * d4->kw * sizeof(float), 256)};
}

// The forward of a layer that would take the column path because c_in*kh*kw
// % 4 != 0, with a kernel of at least 25 taps (the 7x7 RGB stem) and c_in
// rounded up to 4 adding at most a third of the work: the NCHW-view kernel on
// the input and weights padded with zero channels (d4).  The stem at batch 32:
// 178.5 us against 187.5 on the column path.
bool fwd_padded(const mt_conv2d_desc* d, mt_conv2d_desc* d4) {
    if (d->c_in <= 0 || (d->c_in & 3) == 0 || d->kh * d->kw < 25) return false;
    const int64_t cp = (d->c_in + 3) / 4 * 4;
    if (3 * cp > 4 * d->c_in) return false;
    *d4 = *d;
    d4->c_in = cp;
    int64_t ho, wo;
    return conv_dims(d4, &ho, &wo) && nchw_implicit(d4);
}

// dX of a stride-1 convolution with a square kernel and pad <= kh - 1 is the
// forward convolution of dY (c_out channels, h_out x w_out) with the weights
// transposed to [c_in][c_out] and flipped in both spatial axes, padding
// kh - 1 - pad: dX[ci][ih][iw] = sum_{co,r,s} W[co][ci][r][s]·dY[co][ih+pad-r][iw+pad-s].
// Returns the descriptor of that convolution, or false when it does not apply:
// it runs on the channels-last kernel when c_out % 16 == 0, else on the NCHW
// kernel, whose flipped weights (written densely to the workspace) must take
// 16-byte rows (c_out*kh*kw % 4 == 0).
bool dx_as_forward(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo, mt_conv2d_desc* t) {
    if (d->stride != 1 || d->kh != d->kw || d->pad > d->kh - 1) return false;
    *t = mt_conv2d_desc{d->n, d->c_out, Ho, Wo, d->c_in, d->kh, d->kw, 1, d->kh - 1 - d->pad};
    return ((d->c_out * d->kh * d->kw) & 3) == 0 && d->c_out > 0 && Ho * Wo < kMaxDim;
}

// Bytes of the flipped, transposed weights of the implicit dX.
size_t flipped_ws(const mt_conv2d_desc* d) {
    return align_up((size_t)d->c_in * d->c_out * d->kh * d->kw * sizeof(float), 256);
}

// ---- input gradient by stride phase ---------------------------------------------
// dX[ci][ih][iw] = sum over co and the taps (r, t) with ih + pad - r and
// iw + pad - t multiples of the stride s of W[co][ci][r][t] ·
// dY[co][(ih + pad - r)/s][(iw + pad - t)/s].  Split the input pixels by
// phase (ih % s, iw % s) = (ph, pw).  The taps that reach phase row ph are
// r = rh0 + s*j, rh0 = (ph + pad) % s, j < jh = ceil((kh - rh0)/s), and for
// the phase row i' (ih = ph + s*i') they read dY row i' + qh - j, qh =
// (ph + pad) / s: a stride-1 convolution of dY with the phase's flipped
// sub-kernel (a = jh - 1 - j), padding jh - 1 - qh -- negative, or unequal
// between the axes, for some geometries (ConvGeom::pad, pad_w) -- whose
// hp x wp output pixels (hp = ceil((h - ph)/s)) go to every s-th pixel of dX
// (the three-level column scatter of GemmParams).  Each phase is one
// implicit GEMM, C[c_in, n*hp*wp] = Wph[c_in, c_out*jh*jw] · im2col(dY):
// no column buffer (col2im), and dY is read once per tap, as in the forward
// convolution.  A phase no tap reaches (jh or jw = 0, e.g. the odd pixels of
// a 1x1 stride-2 layer) is zero.
constexpr int kDxMaxStride = 4;
struct DxPhase {
    int ph, pw;          // the phase
    int rh0, rw0;        // its first taps
    int jh, jw;          // taps of its sub-kernel per axis (0: no tap reaches it)
    int pad_h, pad_w;    // padding of its stride-1 sub-convolution
    int hp, wp;          // its output rows / columns
    int k;               // c_out * jh * jw
    int64_t woff;        // its weights in the phase-weight block (floats)
};
struct DxPhases {
    int s, n;            // stride, s * s phases
    DxPhase f[kDxMaxStride * kDxMaxStride];
};

DxPhases dx_phases(const mt_conv2d_desc* d) {
    DxPhases t{};
    const int s = (int)d->stride;
    t.s = s;
    t.n = s * s;
    int64_t woff = 0;
    for (int ph = 0; ph < s; ++ph)
        for (int pw = 0; pw < s; ++pw) {
            DxPhase& f = t.f[ph * s + pw];
            f.ph = ph; f.pw = pw;
            f.rh0 = (int)((ph + d->pad) % s);
            f.rw0 = (int)((pw + d->pad) % s);
            f.jh = f.rh0 < d->kh ? (int)((d->kh - f.rh0 + s - 1) / s) : 0;
            f.jw = f.rw0 < d->kw ? (int)((d->kw - f.rw0 + s - 1) / s) : 0;
            f.pad_h = f.jh - 1 - (int)((ph + d->pad) / s);
            f.pad_w = f.jw - 1 - (int)((pw + d->pad) / s);
            f.hp = d->h > ph ? (int)((d->h - ph + s - 1) / s) : 0;
            f.wp = d->w > pw ? (int)((d->w - pw + s - 1) / s) : 0;
            f.k = (int)(d->c_out * f.jh * f.jw);
            f.woff = woff;
            woff += d->c_in * f.k;   // every tap is in exactly one phase: sum = c_in*c_out*kh*kw
        }
    return t;
}

// A strided 1x1 kernel without padding (strides 2-4, c_in and h_out*w_out
// multiples of 4): only the pixels of phase (0, 0) see a tap, and there
// dX_b = Wᵀ·dY_b per image, over dY in NCHW.  The product runs batched into
// the compact phase buffer and the interleave writes dX (zeros elsewhere):
// no dY copy, no phase weights, and the batch fills the chip where the
// phase's single implicit GEMM had 196 workgroups of 256x128 (56x56,
// 256 -> 512 channels).
bool pointwise_strided(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo) {
    return d->kh == 1 && d->kw == 1 && d->pad == 0 && d->stride >= 2 &&
           d->stride <= kDxMaxStride && d->c_in > 0 && (d->c_in & 3) == 0 &&
           ((Ho * Wo) & 3) == 0 && Ho * Wo < kMaxDim && d->h * d->w < kMaxDim;
}
size_t pointwise_strided_zb(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo) {
    return align_up((size_t)d->n * d->c_in * Ho * Wo * sizeof(float), 256);
}

// The phased dX applies for strides up to kDxMaxStride.  Channels-last
// (cl): c_out % 16 == 0, dY copied to channels-last once.  Otherwise the
// NCHW kernel reads dY in place, and every phase's weight rows must be
// 16-byte vectors (c_out*jh*jw % 4 == 0).  Extents stay inside the 32-bit
// window arithmetic of the implicit loaders.
bool dx_phased(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo, bool* cl) {
    if (d->stride > kDxMaxStride || d->c_out <= 0 || d->c_in <= 0 || Ho * Wo >= kMaxDim ||
        d->c_out * d->kh * d->kw >= kMaxDim ||
        d->h * d->w >= kMaxDim || d->kh + Ho >= ((int64_t)1 << 29) || d->kw + Wo >= ((int64_t)1 << 29))
        return false;
    *cl = (d->c_out & 15) == 0;
    if (*cl) return true;
    const DxPhases t = dx_phases(d);
    for (int i = 0; i < t.n; ++i)
        if ((t.f[i].k & 3) != 0) return false;
    return true;
}

// Sub-kernel weights of every phase from the OIHW weights, one thread per
// weight: W[co][ci][r][t] belongs to phase ((r - pad) mod s, (t - pad) mod s),
// tap a = jh - 1 - (r - rh0)/s, b = jw - 1 - (t - rw0)/s of its flipped
// sub-kernel, stored at f.woff + ci*f.k + k with k = (a*jw + b)*c_out + co for
// the channels-last kernel (its K order: tap, channel) or (co*jh + a)*jw + b
// for the NCHW one (OIHW of the sub-convolution).
__global__ void __launch_bounds__(256)
dx_phase_weights_f32(const float* W, float* out, DxPhases t, int c_out, int c_in, int kh, int kw,
                     int pad, int cl) {
    const int64_t total = (int64_t)c_out * c_in * kh * kw;
    const int s = t.s;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int tt = (int)(e % kw);
        const int64_t e1 = e / kw;
        const int r = (int)(e1 % kh);
        const int64_t e2 = e1 / kh;
        const int ci = (int)(e2 % c_in), co = (int)(e2 / c_in);
        const int ph = ((r - pad) % s + s) % s, pw = ((tt - pad) % s + s) % s;
        const DxPhase& f = t.f[ph * s + pw];
        const int a = f.jh - 1 - (r - f.rh0) / s, b = f.jw - 1 - (tt - f.rw0) / s;
        const int k = cl ? (a * f.jw + b) * c_out + co : (co * f.jh + a) * f.jw + b;
        out[f.woff + (int64_t)ci * f.k + k] = W[e];
    }
}

// The compact outputs of the phased dX: phase f = ph*s + pw holds the pixels
// ih = ph + s*i, iw = pw + s*j as z[f][img*c_in + ci][i][j] (hp[f] x wp[f]);
// null where no tap reaches the phase (its pixels are zero).
struct DxPhaseOut {
    const float* z[kDxMaxStride * kDxMaxStride];
    int hp[kDxMaxStride * kDxMaxStride], wp[kDxMaxStride * kDxMaxStride];
};

// dX[plane][ih][iw] = z[(ih%S)*S + iw%S][plane][ih/S][iw/S], plane = img*c_in
// + ci: blockIdx.y walks planes, threads walk items of V pixels of one row,
// stored as one 16-byte vector when V == 4 (W % 4 == 0, aligned).  The phase
// is chosen by compares against every index (an indexed read of the argument
// arrays would go through scratch).  Reads and writes dX's bytes once each.
template <int S, int V>
__global__ void __launch_bounds__(256)
dx_interleave_f32(DxPhaseOut o, float* dx, int64_t planes, int H, int W) {
    const int wq = W / V;
    const int per = H * wq;
    for (int64_t plane = blockIdx.y; plane < planes; plane += gridDim.y) {
        float* dplane = dx + plane * H * W;
        for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < per; q += gridDim.x * blockDim.x) {
            const int ih = q / wq, iw0 = (q - ih * wq) * V;
            const int ph = ih % S, i = ih / S;
            float v[V];
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const int iw = iw0 + e;
                const int f = ph * S + iw % S;
                const float* z = o.z[0];
                int hp = o.hp[0], wp = o.wp[0];
#pragma unroll
                for (int c = 1; c < S * S; ++c)
                    if (f == c) {
                        z = o.z[c];
                        hp = o.hp[c];
                        wp = o.wp[c];
                    }
                v[e] = z ? z[(plane * hp + i) * wp + iw / S] : 0.f;
            }
            float* dst = dplane + (int64_t)ih * W + iw0;
            if constexpr (V == 4)
                *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
            else
                dst[0] = v[0];
        }
    }
}

// For strides 2-4 (at stride 1 the one phase is dX itself).
hipError_t launch_dx_interleave(const DxPhaseOut& o, int s, float* dx, int64_t planes, int H,
                                int W, hipStream_t st) {
    if (s < 2 || s > kDxMaxStride) return hipErrorInvalidValue;
    const bool vec = (W & 3) == 0 && ((uintptr_t)dx & 15u) == 0;
    const int per = H * (vec ? W / 4 : W);
    const dim3 grid((unsigned)std::min<int64_t>((per + 255) / 256, 1024),
                    (unsigned)std::min<int64_t>(planes, 65535));
    if (planes == 0 || per == 0) return hipSuccess;
    auto k = s == 2 ? (vec ? dx_interleave_f32<2, 4> : dx_interleave_f32<2, 1>)
             : s == 3 ? (vec ? dx_interleave_f32<3, 4> : dx_interleave_f32<3, 1>)
                      : (vec ? dx_interleave_f32<4, 4> : dx_interleave_f32<4, 1>);
    hipLaunchKernelGGL(k, grid, dim3(256), 0, st, o, dx, planes, H, W);
    return capture_safe_last_error();
}

// Whether the phased dX is expected to beat dcol = Wᵀ·dY + col2im for d.
// Both run the same flops; the phased GEMMs have c_in rows and a phase's
// pixels as columns (small when c_in is small or the image is), the column
// GEMM kg = c_in*kh*kw rows, but its column buffer is written and gathered
// again.  The cost model prices the GEMMs; measured on seven ResNet layers
// (3x3 stride 2 at 56/28/14, 1x1 stride 2 at 56/28/14, the 7x7 c_in 3
// stem; batch 32, graph replay), the phase GEMMs ran 1.4-1.9x their modelled
// time (short K ranges per phase), so they are priced at kDxPhasedFactor
// times it, plus the dY copy and zero fill at kDxStreamBytes per CU cycle
// (5 TB/s); the column path's buffer, dY copy and gather ran at about
// 2 TB/s (kDxGatherBytes).  This picks the faster path on five of the seven
// layers and loses 5 and 8 % on the two near-ties (the 3x3 at 28, the 1x1
// at 28), where "always phased" loses up to 4.5x (the stem: 3 rows).
// Re-checked after the phases moved to compact outputs and one interleave
// (priced as 2 x dX bytes in the stream term), on eight layers (3x3 stride 2
// at 112/56/28/14 with 64-512 channels, the 1x1 at 14, the stem): 1.7 picks
// the faster path on seven and loses 9 % on the 3x3 at 28 with 256 channels
// (151.6 against 138.8 us); factors 1.0-1.4 lose on two.
constexpr double kDxPhasedFactor = 1.7;
constexpr double kDxStreamBytes = 2083.0;   // device bytes per CU cycle at 5 TB/s, 2.4 GHz
constexpr double kDxGatherBytes = 833.0;    // ... at 2 TB/s
bool dx_prefer_phased(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo, bool cl) {
    // a forced direct-to-LDS configuration skips the rule (the tests' hook
    // onto the phase GEMMs, as for the halo kernel)
    if (g_forced.family == MT_FAMILY_DL) return true;
    const int cus = device_cu_count();
    const DxPhases t = dx_phases(d);
    const int64_t kg = d->c_in * d->kh * d->kw, np = d->n * Ho * Wo;
    const double dx_bytes = 4.0 * d->n * d->c_in * d->h * d->w;
    // the dY copy, and for strides above 1 the interleave (compact phase
    // outputs read, every dX pixel written, zeros included)
    double phased = 0, stream = (cl ? 8.0 * d->c_out * np : 0.0) + (t.s > 1 ? 2.0 * dx_bytes : 0.0);
    for (int i = 0; i < t.n; ++i) {
        const DxPhase& f = t.f[i];
        if (f.hp == 0 || f.wp == 0 || f.k == 0) continue;
        phased += make_plan(d->c_in, d->n * f.hp * f.wp, f.k, 1, cus, true, true, false, false)
                      .cycles;
    }
    phased = kDxPhasedFactor * phased + stream / kDxStreamBytes;
    const double col = make_plan(kg, np, d->c_out, 1, cus, true, true, true, true).cycles +
                       (8.0 * d->c_out * np + 8.0 * kg * np + dx_bytes) / kDxGatherBytes;
    return phased < col;
}

// Workspace of one implicit-operand GEMM (L_IM / L_IMR: the direct-to-LDS
// configurations 0-3; L_IMW, imw: all of them, its own efficiency table),
// including a forced configuration's partials: what launch_gemm may use.
size_t implicit_gemm_ws(int64_t M, int64_t N, int64_t K, bool imw) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const int cus = device_cu_count();
    size_t ws = make_plan(M, N, K, 1, cus, true, true, imw, false, imw).ws_bytes;
    if (!imw && kOfferDl16)   // the channels-last operand may take the 16x16-block kernel
        ws = std::max(ws, make_plan(M, N, K, 1, cus, true, true, false, false, false, true).ws_bytes);
    Plan f;
    if (forced_plan(M, N, K, 1, true, false, imw, &f, !imw)) ws = std::max(ws, f.ws_bytes);
    return ws;
}

// Layout of the phased dX workspace: [channels-last dY (cl)][phase weights]
// [compact phase outputs (strides 2-4)][GEMM].  zoff: each phase's output, in
// floats from the start of its block (aligned to 256 bytes).
struct DxPhasedWs {
    size_t dyt, wph, z, gemm;
    int64_t zoff[kDxMaxStride * kDxMaxStride];
};
DxPhasedWs dx_phased_ws(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo, bool cl) {
    DxPhasedWs w{};
    w.dyt = cl ? align_up((size_t)d->n * d->c_out * Ho * Wo * sizeof(float), 256) : 0;
    w.wph = flipped_ws(d);
    const DxPhases t = dx_phases(d);
    for (int i = 0; i < t.n; ++i) {
        const DxPhase& f = t.f[i];
        w.zoff[i] = (int64_t)(w.z / sizeof(float));
        if (f.k > 0 && f.hp > 0 && f.wp > 0) {
            // stride 1: the one phase is dX itself, written in place
            if (t.s > 1)
                w.z += align_up((size_t)d->n * d->c_in * f.hp * f.wp * sizeof(float), 256);
            w.gemm = std::max(w.gemm, implicit_gemm_ws(d->c_in, d->n * f.hp * f.wp, f.k, false));
        }
    }
    return w;
}

// Workspace of the path mt_conv2d_bwd_input_f32 takes for d.
size_t dx_ws(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo) {
    const int64_t kg = d->c_in * d->kh * d->kw, np = d->n * Ho * Wo;
    if (np == 0 || d->c_out == 0 || d->n * d->c_in * d->h * d->w == 0) return 0;
    const int64_t nx = d->n * d->h * d->w, kx = d->c_out * d->kh * d->kw;
    if (pointwise(d)) return plan_ws(d->c_in, d->h * d->w, d->c_out, d->n, device_cu_count());
    if (pointwise_strided(d, Ho, Wo))
        return pointwise_strided_zb(d, Ho, Wo) +
               plan_ws(d->c_in, Ho * Wo, d->c_out, d->n, device_cu_count());
    mt_conv2d_desc t;
    if (dx_as_forward(d, Ho, Wo, &t) && implicit_geometry(&t)) {
        const ImplicitWs iw = implicit_ws(&t);
        return iw.xt + iw.wt + implicit_gemm_ws(d->c_in, nx, kx, false);
    }
    if (dx_as_forward(d, Ho, Wo, &t) && nchw_implicit(&t))
        return flipped_ws(d) + implicit_gemm_ws(d->c_in, nx, kx, false);
    bool cl = false;
    if (dx_phased(d, Ho, Wo, &cl) && dx_prefer_phased(d, Ho, Wo, cl)) {
        const DxPhasedWs w = dx_phased_ws(d, Ho, Wo, cl);
        return w.dyt + w.wph + w.z + w.gemm;
    }
    return align_up((size_t)kg * np * sizeof(float), 256) +
           align_up((size_t)d->c_out * np * sizeof(float), 256) +
           plan_ws(kg, np, d->c_out, 1, device_cu_count());
}

// Whether the implicit weight gradient reads dY in NCHW (L_KVI) rather than a
// [c_out][n*hw] copy: whole 16-byte groups of one image per row (and a
// 16-byte-aligned dY, checked at the call).
bool dw_reads_dy_nchw(int64_t np, int64_t hw) {
    return (np & 15) == 0 && (hw & 3) == 0 && np < ((int64_t)1 << 24);
}

// Workspace of the path of the weight gradient (and the bias gradient it
// carries) for d, for a 16-byte-aligned dY.
size_t dw_ws(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo) {
    const int64_t kg = d->c_in * d->kh * d->kw, np = d->n * Ho * Wo;
    if (np == 0 || d->c_out == 0 || kg == 0) return 0;
    if (pointwise(d)) return part_plan_ws(d->c_out, d->c_in, Ho * Wo, d->n, device_cu_count());
    if (pointwise_strided(d, Ho, Wo))   // the input's output positions, then the 1x1 product
        return pointwise_strided_zb(d, Ho, Wo) +
               part_plan_ws(d->c_out, d->c_in, Ho * Wo, d->n, device_cu_count());
    mt_conv2d_desc d4;
    if (!implicit_dw(d, np) && dw_padded(d, np, &d4)) {
        const DwPadWs pw = dw_pad_ws(&d4);
        return pw.xp + pw.dw4 + dw_ws(&d4, Ho, Wo);
    }
    const size_t dyt_b = align_up((size_t)d->c_out * np * sizeof(float), 256);
    if (implicit_dw(d, np)) {
        const size_t xt_b = align_up((size_t)d->n * d->c_in * d->h * d->w * sizeof(float), 256);
        return xt_b + (dw_reads_dy_nchw(np, Ho * Wo) ? 0 : dyt_b) +
               implicit_gemm_ws(d->c_out, kg, np, true);
    }
    return align_up((size_t)kg * np * sizeof(float), 256) + dyt_b +
           plan_ws(d->c_out, kg, np, 1, device_cu_count());
}

int run_dx_phased(const mt_conv2d_desc* d, int64_t Ho, int64_t Wo, bool cl,
                  const float* grad_out, const float* weight, float* grad_input, void* workspace,
                  size_t ws_bytes, hipStream_t s) {
    const DxPhasedWs w = dx_phased_ws(d, Ho, Wo, cl);
    if (!workspace || ws_bytes < w.dyt + w.wph + w.z || ((uintptr_t)workspace & 15u) != 0)
        return MT_ERR_WORKSPACE;
    char* wsp = static_cast<char*>(workspace);
    const DxPhases t = dx_phases(d);
    const int64_t hw = Ho * Wo;
    float* dyt = reinterpret_cast<float*>(wsp);
    float* wph = reinterpret_cast<float*>(wsp + w.dyt);
    if (cl &&
        launch_transposes(tjob(grad_out, d->c_out * hw, hw, Wo, 1, Wo, d->c_out, hw, d->n, dyt),
                          TJob{}, s) != hipSuccess)
        return MT_ERR_HIP;
    const int64_t nw = d->c_out * d->c_in * d->kh * d->kw;
    hipLaunchKernelGGL(dx_phase_weights_f32, dim3(grid_for(nw)), dim3(256), 0, s, weight, wph, t,
                       (int)d->c_out, (int)d->c_in, (int)d->kh, (int)d->kw, (int)d->pad,
                       cl ? 1 : 0);
    if (capture_safe_last_error() != hipSuccess) return MT_ERR_HIP;
    // Each phase's GEMM writes its pixels compactly, [img][c_in][hp][wp] (whole
    // 16-byte stores where hp*wp % 4 == 0), and one launch interleaves the
    // phases into dX, zeros where no tap reaches.  Storing straight into dX
    // at stride s cost more than the GEMM (4-byte stores s floats apart: the
    // 1-tap phase of a 3x3 stride-2 layer at 56x56, 128 channels, 32 us).
    float* zb = reinterpret_cast<float*>(wsp + w.dyt + w.wph);
    DxPhaseOut o{};
    char* gws = wsp + w.dyt + w.wph + w.z;
    const size_t gws_b = ws_bytes - w.dyt - w.wph - w.z;
    for (int i = 0; i < t.n; ++i) {
        const DxPhase& f = t.f[i];
        o.hp[i] = f.hp;
        o.wp[i] = f.wp;
        if (f.k == 0 || f.hp == 0 || f.wp == 0) continue;
        float* z = t.s == 1 ? grad_input : zb + w.zoff[i];
        o.z[i] = z;
        const int64_t php = (int64_t)f.hp * f.wp;
        GemmParams p{};
        p.A = wph + f.woff; p.a_mn = f.k; p.a_k = 1; p.a_b = 0;
        p.B = cl ? dyt : grad_out;
        p.C = z;
        p.c_m = php; p.c_n = 1; p.c_b = 0;
        p.c_n_inner = php; p.c_n_outer = d->c_in * php;
        p.bias = nullptr; p.bias_stride = 0; p.bias_axis = MT_BIAS_NONE;
        p.beta = 0.f;
        p.M = (int)d->c_in; p.N = (int)(d->n * f.hp * f.wp); p.K = f.k; p.batch = 1;
        ConvGeom& g = p.cv;
        g.img_stride = d->c_out * hw;
        g.c = (int)d->c_out; g.h = (int)Ho; g.w = (int)Wo;
        g.kh = f.jh; g.kw = f.jw; g.stride = 1; g.pad = f.pad_h; g.pad_w = f.pad_w;
        g.ho = f.hp; g.wo = f.wp;
        if (!cl) {
            g.sc = hw; g.sh = Wo; g.sw = 1;
            set_halo_geometry(g);
        }
        const int rc = launch_gemm(p, true, L_KV, cl ? L_IM : L_IMR, gws, gws_b, s);
        if (rc != MT_OK) return rc;
    }
    if (t.s == 1) return MT_OK;
    return launch_dx_interleave(o, t.s, grad_input, d->n * d->c_in, (int)d->h, (int)d->w, s) ==
                   hipSuccess
               ? MT_OK
               : MT_ERR_HIP;
}

}  // namespace

extern "C" {

int mt_gemm_f32(const mt_mat_f32* A, const mt_mat_f32* B, const mt_mat_f32* C,
                const mt_epilogue_f32* ep, void* workspace, size_t ws_bytes, void* stream) {
    return run_gemm(A, B, C, 0, 0, ep, workspace, ws_bytes, static_cast<hipStream_t>(stream));
}

size_t mt_gemm_workspace_f32(const mt_mat_f32* A, const mt_mat_f32* B, const mt_mat_f32* C) {
    return gemm_ws(A, B, C);
}

int mt_gemm_noalloc_f32(const mt_mat_f32* A, const mt_mat_f32* B, const mt_mat_f32* C,
                        const mt_epilogue_f32* ep, void* stream) {
    int64_t M, N, K, batch;
    const int rc = check_gemm(A, B, C, &M, &N, &K, &batch);
    if (rc != MT_OK) return rc;
    // The workspace mt_gemm_f32 would be given covers the plan it picks, so
    // with at least that much scratch the plan (and every bit of C) is the same.
    const size_t need = gemm_ws(A, B, C);
    if (need > MT_NOALLOC_SCRATCH_BYTES) return MT_ERR_SCRATCH_LIMIT;
    void* ws = nullptr;
    if (need > 0) {
        const int r = noalloc_scratch(&ws);
        if (r != MT_OK) return r;
    }
    return run_gemm(A, B, C, 0, 0, ep, ws, need > 0 ? MT_NOALLOC_SCRATCH_BYTES : 0,
                    static_cast<hipStream_t>(stream));
}

int mt_colsum_f32(const mt_mat_f32* X, float* out, int64_t out_stride, float beta, void* stream) {
    if (!valid_mat(X) || X->batch != 1 || out_stride < 0) return MT_ERR_INVALID;
    if (X->cols == 0) return MT_OK;
    if (!out || (X->cols > 1 && out_stride == 0)) return MT_ERR_INVALID;
    if (X->rows > 0 && !X->base) return MT_ERR_INVALID;
    const unsigned blocks = (unsigned)((X->cols + 63) / 64);
    hipLaunchKernelGGL(colsum_f32, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       X->base ? X->base + X->offset : nullptr, X->row_stride, X->col_stride,
                       (int)X->rows, (int)X->cols, out, out_stride, beta);
    return capture_safe_last_error() == hipSuccess ? MT_OK : MT_ERR_HIP;
}

// Linear views: X [B,in], W [out,in].  Wᵀ is W with its strides swapped.
static mt_mat_f32 transposed(const mt_mat_f32& X) {
    mt_mat_f32 t = X;
    t.rows = X.cols; t.cols = X.rows;
    t.row_stride = X.col_stride; t.col_stride = X.row_stride;
    return t;
}

int mt_linear_forward_f32(const mt_mat_f32* X, const mt_mat_f32* W, const float* bias,
                          int64_t bias_stride, const mt_mat_f32* Y, void* workspace,
                          size_t ws_bytes, void* stream) {
    if (!valid_mat(X) || !valid_mat(W) || !valid_mat(Y)) return MT_ERR_INVALID;
    const mt_mat_f32 Wt = transposed(*W);
    mt_epilogue_f32 ep{bias, bias_stride, bias ? MT_BIAS_COL : MT_BIAS_NONE, 0.f};
    return run_gemm(X, &Wt, Y, 0, 0, &ep, workspace, ws_bytes, static_cast<hipStream_t>(stream));
}

size_t mt_linear_workspace_f32(int64_t rows, int64_t in_f, int64_t out_f) {
    if (rows < 0 || in_f < 0 || out_f < 0) return 0;
    const int cus = device_cu_count();
    size_t ws = 0;
    if (rows > 0 && out_f > 0) ws = std::max(ws, plan_ws(rows, out_f, in_f, 1, cus));
    if (rows > 0 && in_f > 0) ws = std::max(ws, plan_ws(rows, in_f, out_f, 1, cus));
    if (out_f > 0 && in_f > 0) ws = std::max(ws, plan_ws(out_f, in_f, rows, 1, cus));
    return ws;
}

int mt_linear_backward_f32(const mt_mat_f32* dY, const mt_mat_f32* X, const mt_mat_f32* W,
                           const mt_mat_f32* dX, const mt_mat_f32* dW, float beta_w, float* db,
                           int64_t db_stride, float beta_b, void* workspace, size_t ws_bytes,
                           void* stream) {
    if (!valid_mat(dY) || !valid_mat(X) || !valid_mat(W)) return MT_ERR_INVALID;
    if (dY->rows != X->rows || dY->cols != W->rows || X->cols != W->cols) return MT_ERR_INVALID;
    if (db && db_stride < 0) return MT_ERR_INVALID;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dX) {  // dX[B,in] = dY[B,out] · W[out,in]
        int rc = run_gemm(dY, W, dX, 0, 0, nullptr, workspace, ws_bytes, s);
        if (rc != MT_OK) return rc;
    }
    bool db_done = false;
    if (dW) {  // dW[out,in] = dYᵀ[out,B] · X[B,in] (+ beta_w·dW); db = row sums of dYᵀ
        const mt_mat_f32 dYt = transposed(*dY);
        mt_epilogue_f32 ep{nullptr, 0, MT_BIAS_NONE, beta_w};
        RowSums rows{db, db_stride, beta_b, false};
        const bool fuse = db != nullptr && (dW->rows <= 1 || db_stride != 0);
        int rc = run_gemm(&dYt, X, dW, 0, 0, &ep, workspace, ws_bytes, s, fuse ? &rows : nullptr);
        if (rc != MT_OK) return rc;
        db_done = fuse && rows.done;
    }
    if (db && !db_done) {
        int rc = mt_colsum_f32(dY, db, db_stride, beta_b, stream);
        if (rc != MT_OK) return rc;
    }
    return MT_OK;
}

size_t mt_conv2d_workspace_f32(const mt_conv2d_desc* d) {
    int64_t Ho, Wo;
    if (!conv_dims(d, &Ho, &Wo)) return 0;
    const int64_t kg = d->c_in * d->kh * d->kw, np = d->n * Ho * Wo;
    if (np == 0 || d->c_out == 0) return 0;
    // one product per image; a strided input whose (h, w) do not fold into one
    // index takes the NCHW-view kernel instead
    if (pointwise(d))
        return std::max(plan_ws(d->c_out, d->h * d->w, d->c_in, d->n, device_cu_count()),
                        nchw_weight_ws(d) + implicit_gemm_ws(d->c_out, np, kg, false));
    if (implicit_geometry(d) && d->h * d->w < kMaxDim) {   // channels-last kernel
        const ImplicitWs iw = implicit_ws(d);
        return iw.xt + iw.wt + implicit_gemm_ws(d->c_out, np, kg, false);
    }
    // the NCHW-view kernel: split-K partials, and room for an aligned copy of
    // the weights (used only when the caller's are not 16-byte aligned)
    if (nchw_implicit(d)) return nchw_weight_ws(d) + implicit_gemm_ws(d->c_out, np, kg, false);
    const size_t col = align_up((size_t)kg * np * sizeof(float), 256) +
                       plan_ws(d->c_out, np, kg, 1, device_cu_count());
    // a dense input takes the padded NCHW-view path; other views the column one
    mt_conv2d_desc d4;
    if (fwd_padded(d, &d4)) {
        const DwPadWs pw = dw_pad_ws(&d4);
        return std::max(col, pw.xp + pw.dw4 +
                                 implicit_gemm_ws(d->c_out, np, d4.c_in * d->kh * d->kw, false));
    }
    return col;
}

int mt_conv2d_fwd_strided_f32(const mt_conv2d_desc* d, const float* input,
                              const int64_t in_strides[4], const float* weight, const float* bias,
                              float* output, void* workspace, size_t ws_bytes, void* stream) {
    int64_t Ho, Wo;
    if (!conv_dims(d, &Ho, &Wo) || !in_strides) return MT_ERR_INVALID;
    for (int i = 0; i < 4; ++i)
        if (in_strides[i] < 0) return MT_ERR_INVALID;
    const int64_t kg = d->c_in * d->kh * d->kw, np = d->n * Ho * Wo, hw = Ho * Wo;
    if (np == 0 || d->c_out == 0) return MT_OK;
    if (!output || (kg > 0 && (!input || !weight))) return MT_ERR_INVALID;
    hipStream_t s = static_cast<hipStream_t>(stream);

    // 1x1, stride 1, no padding: Y_b[c_out][hw] = W[c_out][c_in] · X_b[c_in][hw]
    // for each image b, over the input view itself when its (h, w) fold into
    // one position index (NCHW, NHWC, channel slices).
    if (pointwise(d) && (d->h == 1 || in_strides[2] == d->w * in_strides[3])) {
        const mt_mat_f32 A{weight, 0, d->c_out, d->c_in, d->c_in, 1, d->n, 0};
        const mt_mat_f32 B{input, 0, d->c_in, hw, in_strides[1], in_strides[3], d->n,
                           in_strides[0]};
        const mt_mat_f32 C{output, 0, d->c_out, hw, hw, 1, d->n, d->c_out * hw};
        const mt_epilogue_f32 ep{bias, 1, bias ? MT_BIAS_ROW : MT_BIAS_NONE, 0.f};
        return run_gemm(&A, &B, &C, 0, 0, &ep, workspace, ws_bytes, s);
    }

    // c_in % 16 == 0: the channels-last kernel (16-byte DMA gathers) on a
    // channels-last copy of the input (the input itself when it is one) and
    // OHWI weights.  Its 16-byte gathers beat the NCHW-view kernels (4-byte
    // gathers or halo patches) by more than the layout launch costs
    // (benchmark layer, forward: 79.5 us against 84.5 with halo patches).
    if (implicit_geometry(d) && d->h * d->w < kMaxDim && !pointwise(d)) {
        const ImplicitWs iw = implicit_ws(d);
        if (!workspace || ws_bytes < iw.xt + iw.wt || ((uintptr_t)workspace & 15u) != 0)
            return MT_ERR_WORKSPACE;
        char* wsp = static_cast<char*>(workspace);
        float* wt = reinterpret_cast<float*>(wsp + iw.xt);      // OIHW -> OHWI
        const TJob wjob = tjob(weight, kg, d->kh * d->kw, d->kw, 1, d->kw, d->c_in,
                               d->kh * d->kw, d->c_out, wt);
        return run_conv_implicit(d, Ho, Wo, input, in_strides, bias, output, wsp, ws_bytes, wjob,
                                 s);
    }
    // other channel counts with kg % 4 == 0: the implicit GEMM over the NCHW
    // view, no copy of either operand and no column buffer
    if (nchw_implicit(d)) {
        const size_t wb = nchw_weight_ws(d);
        if (!workspace || ws_bytes < wb || ((uintptr_t)workspace & 15u) != 0)
            return MT_ERR_WORKSPACE;
        char* wsp = static_cast<char*>(workspace);
        if (((uintptr_t)weight & 15u) != 0) {
            if (hipMemcpyAsync(wsp, weight, (size_t)d->c_out * kg * sizeof(float),
                               hipMemcpyDeviceToDevice, s) != hipSuccess)
                return MT_ERR_HIP;
            weight = reinterpret_cast<const float*>(wsp);
        }
        return run_conv_nchw(d, Ho, Wo, input, in_strides, weight, bias, output, wsp + wb,
                             ws_bytes - wb, s);
    }

    // A dense input of a padded geometry (fwd_padded): the input and the
    // weights padded with zero channels, then the NCHW-view kernel.
    mt_conv2d_desc d4;
    int64_t dst[4];
    dense_strides(d, dst);
    if (fwd_padded(d, &d4) && std::equal(dst, dst + 4, in_strides)) {
        const DwPadWs pw = dw_pad_ws(&d4);   // the padded input and weights
        if (!workspace || ws_bytes < pw.xp + pw.dw4 || ((uintptr_t)workspace & 15u) != 0)
            return MT_ERR_WORKSPACE;
        char* wsp = static_cast<char*>(workspace);
        float* xp = reinterpret_cast<float*>(wsp);
        float* wp = reinterpret_cast<float*>(wsp + pw.xp);
        if (launch_pad_channels(input, xp, d->n, (int)d->c_in, (int)d4.c_in, d->h * d->w, s) !=
                hipSuccess ||
            launch_pad_channels(weight, wp, d->c_out, (int)d->c_in, (int)d4.c_in,
                                d->kh * d->kw, s) != hipSuccess)
            return MT_ERR_HIP;
        int64_t st4[4];
        dense_strides(&d4, st4);
        return run_conv_nchw(&d4, Ho, Wo, xp, st4, wp, bias, output, wsp + pw.xp + pw.dw4,
                             ws_bytes - pw.xp - pw.dw4, s);
    }
    // Explicit im2col into the workspace, then the GEMM on the column buffer.
    const size_t col_bytes = align_up((size_t)kg * np * sizeof(float), 256);
    if (kg > 0 && (!workspace || ws_bytes < col_bytes)) return MT_ERR_WORKSPACE;
    float* col = static_cast<float*>(workspace);
    if (kg > 0 && launch_im2col(d, Ho, Wo, input, in_strides, col, s) != hipSuccess)
        return MT_ERR_HIP;
    mt_mat_f32 A, B, C;
    conv_gemm_views(d, Ho, Wo, weight, col, output, &A, &B, &C);
    mt_epilogue_f32 ep{bias, 1, bias ? MT_BIAS_ROW : MT_BIAS_NONE, 0.f};
    char* gws = static_cast<char*>(workspace) + (kg > 0 ? col_bytes : 0);
    const size_t gws_bytes = ws_bytes > col_bytes ? ws_bytes - col_bytes : 0;
    return run_gemm(&A, &B, &C, hw, d->c_out * hw, &ep, gws, gws_bytes, s);
}

int mt_conv2d_fwd_f32(const mt_conv2d_desc* d, const float* input, const float* weight,
                      const float* bias, float* output, void* workspace, size_t ws_bytes,
                      void* stream) {
    if (!d) return MT_ERR_INVALID;
    int64_t st[4];
    dense_strides(d, st);
    return mt_conv2d_fwd_strided_f32(d, input, st, weight, bias, output, workspace, ws_bytes,
                                     stream);
}

size_t mt_conv2d_bwd_workspace_f32(const mt_conv2d_desc* d) {
    int64_t Ho, Wo;
    if (!conv_dims(d, &Ho, &Wo)) return 0;
    // the paths the dX and the dW (+ db) calls take, one after the other
    return std::max(dx_ws(d, Ho, Wo), dw_ws(d, Ho, Wo));
}

}  // extern "C"

namespace {

// dW (+ beta·dW).  With grad_bias, the implicit path also hands db
// (+ beta_b·db) to the split-K reduction of its GEMM when the plan has one
// (GemmParams::csum); *db_done reports whether it did.
int conv_bwd_weight(const mt_conv2d_desc* d, const float* input, const float* grad_out,
                    float* grad_weight, float beta, float* grad_bias, float beta_b,
                    void* workspace, size_t ws_bytes, hipStream_t s, bool* db_done) {
    *db_done = false;
    int64_t Ho, Wo;
    if (!conv_dims(d, &Ho, &Wo)) return MT_ERR_INVALID;
    const int64_t kg = d->c_in * d->kh * d->kw, np = d->n * Ho * Wo, hw = Ho * Wo;
    if (kg == 0 || d->c_out == 0) return MT_OK;
    if (!grad_weight) return MT_ERR_INVALID;
    const size_t col_b = align_up((size_t)kg * np * sizeof(float), 256);
    const size_t dyt_b = align_up((size_t)d->c_out * np * sizeof(float), 256);
    if (np > 0 && (!input || !grad_out)) return MT_ERR_INVALID;
    if (pointwise_strided(d, Ho, Wo)) {
        // A strided 1x1 layer reads only x[oh*s][ow*s]: those pixels copied
        // out (n*c_in*Ho*Wo floats), then the batch-summed 1x1 product on
        // them.  The 56x56 256 -> 512 shortcut at batch 32: dW + db 81 against
        // 118 us through the channels-last copy of the whole input.
        const size_t xs_b = pointwise_strided_zb(d, Ho, Wo);
        if (!workspace || ws_bytes < xs_b || ((uintptr_t)workspace & 15u) != 0)
            return MT_ERR_WORKSPACE;
        float* xs = static_cast<float*>(workspace);
        if (launch_axpby(input, d->h * d->w, d->stride * d->w, d->stride, 1.f, xs, hw, Wo, 1, 0.f,
                         d->n * d->c_in, Ho, Wo, s) != hipSuccess)
            return MT_ERR_HIP;
        mt_conv2d_desc d1 = *d;
        d1.h = Ho; d1.w = Wo; d1.stride = 1;
        return conv_bwd_weight(&d1, xs, grad_out, grad_weight, beta, grad_bias, beta_b,
                               static_cast<char*>(workspace) + xs_b, ws_bytes - xs_b, s, db_done);
    }
    if (pointwise(d) && np > 0) {
        // dW[c_out][c_in] = Σ_b dY_b[c_out][hw] · X_b[c_in][hw]ᵀ: one product per
        // image into the workspace, summed (with beta·dW, and db as the channel
        // sums of dY) by the reduction launch.
        GemmParams p{};
        p.A = grad_out; p.a_mn = hw; p.a_k = 1; p.a_b = d->c_out * hw;
        p.B = input; p.b_mn = hw; p.b_k = 1; p.b_b = d->c_in * hw;
        p.C = grad_weight; p.c_m = d->c_in; p.c_n = 1; p.c_b = 0;
        p.c_n_inner = d->c_in; p.c_n_outer = 0;
        p.bias = nullptr; p.bias_stride = 0; p.bias_axis = MT_BIAS_NONE;
        p.beta = beta;
        p.M = (int)d->c_out; p.N = (int)d->c_in; p.K = (int)hw; p.batch = (int)d->n;
        p.part = 1;
        if (grad_bias) {
            p.csum_src = grad_out; p.csum = grad_bias; p.csum_n = (int)d->n;
            p.csum_hw = hw; p.csum_beta = beta_b;
            // the GEMM's A is dY itself: its fused row sums give db without a
            // second pass over dY where the plan can take them
            p.rowsum = grad_bias;
        }
        const int la = classify(p.A, p.a_mn, p.a_k, p.M, p.K, p.a_b, p.batch > 1);
        const int lb = classify(p.B, p.b_mn, p.b_k, p.N, p.K, p.b_b, p.batch > 1);
        const bool dl = (la == L_KV || la == L_MV) && (lb == L_KV || lb == L_MV);
        const int rc = launch_gemm(p, dl, la, lb, workspace, ws_bytes, s);
        *db_done = rc == MT_OK && p.csum != nullptr;
        return rc;
    }
    mt_conv2d_desc d4;
    if (!implicit_dw(d, np) && dw_padded(d, np, &d4)) {
        const DwPadWs pw = dw_pad_ws(&d4);
        if (!workspace || ws_bytes < pw.xp + pw.dw4 || ((uintptr_t)workspace & 15u) != 0)
            return MT_ERR_WORKSPACE;
        char* wsp = static_cast<char*>(workspace);
        float* xp = reinterpret_cast<float*>(wsp);
        float* dw4 = reinterpret_cast<float*>(wsp + pw.xp);
        if (launch_pad_channels(input, xp, d->n, (int)d->c_in, (int)d4.c_in, d->h * d->w, s) !=
            hipSuccess)
            return MT_ERR_HIP;
        const int rc = conv_bwd_weight(&d4, xp, grad_out, dw4, 0.f, grad_bias, beta_b,
                                       wsp + pw.xp + pw.dw4, ws_bytes - pw.xp - pw.dw4, s, db_done);
        if (rc != MT_OK) return rc;
        // dW[co][ci*khw + t] = beta*dW + dW4[co][ci*khw + t] for the real channels ci
        const int64_t khw = d->kh * d->kw;
        return launch_axpby(dw4, d4.c_in * khw, 0, 1, 1.f, grad_weight, d->c_in * khw, 0, 1, beta,
                            d->c_out, 1, d->c_in * khw, s) == hipSuccess
                   ? MT_OK
                   : MT_ERR_HIP;
    }
    if (implicit_dw(d, np)) {
        // Implicit GEMM dW[c_out, (r,s,ci)] = dYt[c_out, np] · im2colᵀ(xt)[np, (r,s,ci)],
        // the B operand gathered from a channels-last copy of the input and the
        // columns scattered to OIHW by the epilogue: col(n) = tap + ci*kh*kw.
        const size_t xt_b = align_up((size_t)d->n * d->c_in * d->h * d->w * sizeof(float), 256);
        // dY is read in NCHW by the GEMM (L_KVI) when every 16-byte group of a
        // row is four pixels of one image and K holds whole chunks; else it is
        // copied to dYt [c_out][n][hw] (not counted by the workspace query
        // when only dY's alignment prevents the NCHW read).  x ->
        // channels-last in the same launch.
        const bool kvi = dw_reads_dy_nchw(np, hw) && ((uintptr_t)grad_out & 15u) == 0;
        const size_t dyb = kvi ? 0 : dyt_b;
        if (!workspace || ws_bytes < xt_b + dyb || ((uintptr_t)workspace & 15u) != 0)
            return MT_ERR_WORKSPACE;
        char* wsp = static_cast<char*>(workspace);
        float* xt = reinterpret_cast<float*>(wsp);
        float* dyt = reinterpret_cast<float*>(wsp + xt_b);
        int64_t st[4];
        dense_strides(d, st);
        if (launch_transposes(tjob(input, st[0], st[1], st[2], st[3], d->w, d->c_in, d->h * d->w,
                                   d->n, xt),
                              kvi ? TJob{}
                                  : tjob(grad_out, hw, 1, d->c_out * hw, 0, 1, hw, d->n, d->c_out,
                                         dyt),
                              s) != hipSuccess)
            return MT_ERR_HIP;
        GemmParams p{};
        if (kvi) {
            p.A = grad_out; p.a_mn = hw; p.a_k = 1; p.a_b = 0;
            p.a_img = d->c_out * hw; p.a_hw = (int)hw;
        } else {
            p.A = dyt; p.a_mn = np; p.a_k = 1; p.a_b = 0;
        }
        p.B = xt;
        p.C = grad_weight; p.c_m = kg; p.c_n = d->kh * d->kw; p.c_b = 0;
        p.c_n_inner = d->c_in; p.c_n_outer = 1;
        p.bias = nullptr; p.bias_stride = 0; p.bias_axis = MT_BIAS_NONE;
        p.beta = beta;
        p.M = (int)d->c_out; p.N = (int)kg; p.K = (int)np; p.batch = 1;
        ConvGeom& g = p.cv;
        g.img_stride = d->h * d->w * d->c_in;
        g.c = (int)d->c_in; g.h = (int)d->h; g.w = (int)d->w;
        g.kh = (int)d->kh; g.kw = (int)d->kw; g.stride = (int)d->stride; g.pad = g.pad_w = (int)d->pad;
        g.ho = (int)Ho; g.wo = (int)Wo;
        if (grad_bias) {
            p.csum_src = grad_out; p.csum = grad_bias; p.csum_n = (int)d->n;
            p.csum_hw = hw; p.csum_beta = beta_b;
        }
        const int rc = launch_gemm(p, true, kvi ? L_KVI : L_KV, L_IMW, wsp + xt_b + dyb,
                                   ws_bytes - xt_b - dyb, s);
        *db_done = rc == MT_OK && p.csum != nullptr;
        return rc;
    }
    if (np > 0 && (!workspace || ws_bytes < col_b + dyt_b)) return MT_ERR_WORKSPACE;
    float* col = static_cast<float*>(workspace);
    float* dyt = reinterpret_cast<float*>(static_cast<char*>(workspace) + col_b);
    if (np > 0) {
        int64_t st[4];
        dense_strides(d, st);
        if (launch_im2col(d, Ho, Wo, input, st, col, s) != hipSuccess) return MT_ERR_HIP;
        if (transpose_dy(d, hw, grad_out, dyt, s) != hipSuccess) return MT_ERR_HIP;
    }
    // dW[c_out, kg] = dYt[c_out, np] · colᵀ[np, kg]
    const mt_mat_f32 A{dyt, 0, d->c_out, np, np, 1, 1, 0};
    const mt_mat_f32 B{col, 0, np, kg, 1, np, 1, 0};
    const mt_mat_f32 C{grad_weight, 0, d->c_out, kg, kg, 1, 1, 0};
    const mt_epilogue_f32 ep{nullptr, 0, MT_BIAS_NONE, beta};
    char* gws = static_cast<char*>(workspace) + col_b + dyt_b;
    const size_t gws_b = ws_bytes > col_b + dyt_b ? ws_bytes - col_b - dyt_b : 0;
    return run_gemm(&A, &B, &C, 0, 0, &ep, np > 0 ? gws : nullptr, np > 0 ? gws_b : 0, s);
}

}  // namespace

extern "C" {

int mt_conv2d_bwd_weight_f32(const mt_conv2d_desc* d, const float* input, const float* grad_out,
                             float* grad_weight, float beta, void* workspace, size_t ws_bytes,
                             void* stream) {
    bool db_done;
    return conv_bwd_weight(d, input, grad_out, grad_weight, beta, nullptr, 0.f, workspace,
                           ws_bytes, static_cast<hipStream_t>(stream), &db_done);
}

int mt_conv2d_bwd_weight_bias_f32(const mt_conv2d_desc* d, const float* input,
                                  const float* grad_out, float* grad_weight, float beta_w,
                                  float* grad_bias, float beta_b, void* workspace,
                                  size_t ws_bytes, void* stream) {
    int64_t Ho, Wo;
    if (!conv_dims(d, &Ho, &Wo)) return MT_ERR_INVALID;
    if (grad_bias && d->n * Ho * Wo > 0 && !grad_out) return MT_ERR_INVALID;
    bool db_done = false;
    const int rc = conv_bwd_weight(d, input, grad_out, grad_weight, beta_w, grad_bias, beta_b,
                                   workspace, ws_bytes, static_cast<hipStream_t>(stream),
                                   &db_done);
    if (rc != MT_OK || !grad_bias || db_done) return rc;
    return mt_conv2d_bwd_bias_f32(d, grad_out, grad_bias, beta_b, stream);
}

int mt_conv2d_bwd_input_f32(const mt_conv2d_desc* d, const float* grad_out, const float* weight,
                            float* grad_input, void* workspace, size_t ws_bytes, void* stream) {
    int64_t Ho, Wo;
    if (!conv_dims(d, &Ho, &Wo)) return MT_ERR_INVALID;
    const int64_t kg = d->c_in * d->kh * d->kw, np = d->n * Ho * Wo, hw = Ho * Wo;
    const int64_t total = d->n * d->c_in * d->h * d->w;
    if (total == 0) return MT_OK;
    if (!grad_input) return MT_ERR_INVALID;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (np == 0 || d->c_out == 0) {  // no output position touches the input
        hipLaunchKernelGGL(fill_f32, dim3(grid_for(total)), dim3(256), 0, s, grad_input, total, 0.f);
        return capture_safe_last_error() == hipSuccess ? MT_OK : MT_ERR_HIP;
    }
    if (!grad_out || !weight) return MT_ERR_INVALID;
    if (pointwise(d)) {   // dX_b[c_in][hw] = Wᵀ[c_in][c_out] · dY_b[c_out][hw]
        const mt_mat_f32 A{weight, 0, d->c_in, d->c_out, 1, d->c_in, d->n, 0};
        const mt_mat_f32 B{grad_out, 0, d->c_out, hw, hw, 1, d->n, d->c_out * hw};
        const mt_mat_f32 C{grad_input, 0, d->c_in, hw, hw, 1, d->n, d->c_in * hw};
        return run_gemm(&A, &B, &C, 0, 0, nullptr, workspace, ws_bytes, s);
    }
    if (pointwise_strided(d, Ho, Wo)) {   // phase (0, 0): Z_b = Wᵀ · dY_b, then interleave
        const size_t zb = pointwise_strided_zb(d, Ho, Wo);
        if (!workspace || ws_bytes < zb || ((uintptr_t)workspace & 15u) != 0)
            return MT_ERR_WORKSPACE;
        float* z = static_cast<float*>(workspace);
        const mt_mat_f32 A{weight, 0, d->c_in, d->c_out, 1, d->c_in, d->n, 0};
        const mt_mat_f32 B{grad_out, 0, d->c_out, hw, hw, 1, d->n, d->c_out * hw};
        const mt_mat_f32 C{z, 0, d->c_in, hw, hw, 1, d->n, d->c_in * hw};
        const int rc = run_gemm(&A, &B, &C, 0, 0, nullptr, static_cast<char*>(workspace) + zb,
                                ws_bytes - zb, s);
        if (rc != MT_OK) return rc;
        const DxPhases t = dx_phases(d);
        DxPhaseOut o{};
        for (int i = 0; i < t.n; ++i) {
            o.hp[i] = t.f[i].hp;
            o.wp[i] = t.f[i].wp;
        }
        o.z[0] = z;
        return launch_dx_interleave(o, t.s, grad_input, d->n * d->c_in, (int)d->h, (int)d->w,
                                    s) == hipSuccess
                   ? MT_OK
                   : MT_ERR_HIP;
    }
    mt_conv2d_desc t;
    if (dx_as_forward(d, Ho, Wo, &t) && implicit_geometry(&t)) {
        // Channels-last implicit GEMM of dY with the weights transposed to
        // [c_in][c_out] and flipped (OHWI of the dX convolution): no dcol buffer.
        int64_t th, tw;
        if (!conv_dims(&t, &th, &tw) || th != d->h || tw != d->w) return MT_ERR_INVALID;
        const ImplicitWs iw = implicit_ws(&t);
        if (!workspace || ws_bytes < iw.xt + iw.wt || ((uintptr_t)workspace & 15u) != 0)
            return MT_ERR_WORKSPACE;
        char* wsp = static_cast<char*>(workspace);
        // Wt[ci][r'][s'][co] = W[co][ci][kh-1-r'][kw-1-s'] (negative tap strides)
        const int64_t khw = d->kh * d->kw;
        const TJob wjob = tjob(weight + (khw - 1), khw, d->c_in * khw, -d->kw, -1, d->kw,
                               d->c_out, khw, d->c_in, reinterpret_cast<float*>(wsp + iw.xt));
        const int64_t st[4] = {d->c_out * hw, hw, Wo, 1};   // dense dY
        return run_conv_implicit(&t, d->h, d->w, grad_out, st, nullptr, grad_input, wsp, ws_bytes,
                                 wjob, s);
    }
    if (dx_as_forward(d, Ho, Wo, &t) && nchw_implicit(&t)) {
        // Other c_out: the implicit GEMM of dY (NCHW, read in place) with the
        // flipped, transposed weights in OIHW order: no dcol buffer, no copy of dY.
        int64_t th, tw;
        if (!conv_dims(&t, &th, &tw) || th != d->h || tw != d->w) return MT_ERR_INVALID;
        const size_t fb = flipped_ws(d);
        if (!workspace || ws_bytes < fb || ((uintptr_t)workspace & 15u) != 0)
            return MT_ERR_WORKSPACE;
        char* wsp = static_cast<char*>(workspace);
        float* wf = reinterpret_cast<float*>(wsp);
        // wf[ci][co][r'][s'] = W[co][ci][kh-1-r'][kw-1-s'] (OIHW of the dX convolution)
        const int64_t khw = d->kh * d->kw;
        if (launch_transpose(weight + (khw - 1), khw, -1, 0, d->c_in * khw, d->c_out, khw,
                             d->c_out, d->c_in, wf, s) != hipSuccess)
            return MT_ERR_HIP;
        const int64_t st[4] = {d->c_out * hw, hw, Wo, 1};   // dense dY
        return run_conv_nchw(&t, d->h, d->w, grad_out, st, wf, nullptr, grad_input, wsp + fb,
                             ws_bytes - fb, s);
    }
    bool cl = false;
    if (dx_phased(d, Ho, Wo, &cl) && dx_prefer_phased(d, Ho, Wo, cl))
        // strided or non-square: one implicit GEMM per stride phase
        return run_dx_phased(d, Ho, Wo, cl, grad_out, weight, grad_input, workspace, ws_bytes, s);
    const size_t col_b = align_up((size_t)kg * np * sizeof(float), 256);
    const size_t dyt_b = align_up((size_t)d->c_out * np * sizeof(float), 256);
    if (!workspace || ws_bytes < col_b + dyt_b) return MT_ERR_WORKSPACE;
    float* dcol = static_cast<float*>(workspace);
    float* dyt = reinterpret_cast<float*>(static_cast<char*>(workspace) + col_b);
    if (transpose_dy(d, hw, grad_out, dyt, s) != hipSuccess) return MT_ERR_HIP;
    // dcol[kg, np] = Wᵀ[kg, c_out] · dYt[c_out, np]
    const mt_mat_f32 A{weight, 0, kg, d->c_out, 1, kg, 1, 0};
    const mt_mat_f32 B{dyt, 0, d->c_out, np, np, 1, 1, 0};
    const mt_mat_f32 C{dcol, 0, kg, np, np, 1, 1, 0};
    char* gws = static_cast<char*>(workspace) + col_b + dyt_b;
    const size_t gws_b = ws_bytes - col_b - dyt_b;
    int rc = run_gemm(&A, &B, &C, 0, 0, nullptr, gws, gws_b, s);
    if (rc != MT_OK) return rc;
    hipLaunchKernelGGL(col2im_gather_f32, dim3(grid_for(total)), dim3(256), 0, s, dcol, grad_input,
                       (int)d->c_in, (int)d->h, (int)d->w, (int)d->kh, (int)d->kw, (int)d->stride,
                       (int)d->pad, (int)Ho, (int)Wo, np, total);
    return capture_safe_last_error() == hipSuccess ? MT_OK : MT_ERR_HIP;
}

int mt_conv2d_bwd_bias_f32(const mt_conv2d_desc* d, const float* grad_out, float* grad_bias,
                           float beta, void* stream) {
    int64_t Ho, Wo;
    if (!conv_dims(d, &Ho, &Wo)) return MT_ERR_INVALID;
    if (d->c_out == 0) return MT_OK;
    if (!grad_bias || (d->n * Ho * Wo > 0 && !grad_out)) return MT_ERR_INVALID;
    const auto kern = csum_threads(d->n * Ho * Wo) == 1024 ? conv_bias_grad_f32<1024>
                                                           : conv_bias_grad_f32<256>;
    hipLaunchKernelGGL(kern, dim3((unsigned)d->c_out), dim3(csum_threads(d->n * Ho * Wo)), 0,
                       static_cast<hipStream_t>(stream), grad_out, grad_bias, (int)d->n,
                       (int)d->c_out, Ho * Wo, beta);
    return capture_safe_last_error() == hipSuccess ? MT_OK : MT_ERR_HIP;
}

int mt_fill_f32(float* p, int64_t n, float value, void* stream) {
    if (n < 0 || (n > 0 && !p)) return MT_ERR_INVALID;
    if (n == 0) return MT_OK;
    hipLaunchKernelGGL(fill_f32, dim3(grid_for(n)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       p, n, value);
    return capture_safe_last_error() == hipSuccess ? MT_OK : MT_ERR_HIP;
}

int mt_axpby_f32(const mt_mat_f32* X, float alpha, const mt_mat_f32* Y, float beta, void* stream) {
    if (!valid_mat(X) || !valid_mat(Y)) return MT_ERR_INVALID;
    if (X->rows != Y->rows || X->cols != Y->cols || (X->batch != 1 && X->batch != Y->batch))
        return MT_ERR_INVALID;
    const int64_t total = Y->batch * Y->rows * Y->cols;
    if (total == 0) return MT_OK;
    if (!X->base || !Y->base) return MT_ERR_INVALID;
    if ((Y->rows > 1 && Y->row_stride == 0) || (Y->cols > 1 && Y->col_stride == 0) ||
        (Y->batch > 1 && Y->batch_stride == 0))
        return MT_ERR_INVALID;
    float* const y = const_cast<float*>(Y->base) + Y->offset;
    // A plain copy of a transposed view (X's rows adjacent, its columns
    // strided) into dense rows: the LDS-tiled layout change, whose reads run
    // down X's columns and writes along Y's rows, where the element-wise form
    // reads one column element per lane (a 2048 x 1024 Bᵀ: 15.7 -> 8.6 us).
    // alpha = 1 and beta = 0 make it an exact copy, as that form's.
    if (alpha == 1.f && beta == 0.f && X->row_stride == 1 && X->col_stride > 1 &&
        Y->col_stride == 1 && Y->row_stride == Y->cols &&
        (Y->batch == 1 || Y->batch_stride == Y->rows * Y->cols) && Y->rows >= 32 &&
        Y->cols >= 32 && Y->rows < kMaxDim && Y->cols < kMaxDim && Y->batch < kMaxDim) {
        const TJob j = tjob(X->base + X->offset, X->batch == 1 ? 0 : X->batch_stride,
                            X->col_stride, Y->rows, 1, Y->rows, Y->cols, Y->rows, Y->batch, y);
        return launch_transposes(j, TJob{}, static_cast<hipStream_t>(stream)) == hipSuccess
                   ? MT_OK
                   : MT_ERR_HIP;
    }
    const hipError_t e =
        launch_axpby(X->base + X->offset, X->batch == 1 ? 0 : X->batch_stride, X->row_stride,
                     X->col_stride, alpha, y, Y->batch_stride, Y->row_stride, Y->col_stride, beta,
                     Y->batch, Y->rows, Y->cols, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? MT_OK : MT_ERR_HIP;
}

const char* mt_strerror(int status) {
    switch (status) {
        case MT_OK: return "success";
        case MT_ERR_INVALID: return "invalid argument";
        case MT_ERR_WORKSPACE: return "workspace missing or too small";
        case MT_ERR_HIP: return "HIP runtime error";
        case MT_ERR_UNSUPPORTED: return "unsupported request";
        case MT_ERR_SCRATCH_LIMIT:
            return "problem needs more scratch than mt_gemm_noalloc_f32's static buffer "
                   "(MT_NOALLOC_SCRATCH_BYTES); use mt_gemm_f32 with a workspace";
        default: return "unknown status";
    }
}

int mt_version(void) { return MTGEMM_VERSION; }

const char* mt_last_config(void) { return g_last_config; }

int mt_gemm_config_count(int family) {
    return family == MT_FAMILY_RS       ? kNumCfg
           : family == MT_FAMILY_DL     ? kNumDlCfg
           : family == MT_FAMILY_KSW    ? kNumKswCfg
           : family == MT_FAMILY_SKINNY ? 2
                                        : 0;
}

int mt_gemm_force_config(int family, int cfg, int splits) {
    if (family == MT_FAMILY_AUTO) {
        g_forced = ForcedConfig{};
        return MT_OK;
    }
    if ((family != MT_FAMILY_RS && family != MT_FAMILY_DL && family != MT_FAMILY_KSW &&
         family != MT_FAMILY_SKINNY) || cfg < 0 ||
        cfg >= mt_gemm_config_count(family) || splits < 1 || splits > kMaxForcedSplits)
        return MT_ERR_INVALID;
    g_forced = ForcedConfig{family, cfg, splits};
    return MT_OK;
}

}  // extern "C"

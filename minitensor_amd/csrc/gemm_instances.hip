// gemm_instances.hip -- instantiates gemm_f32_mfma for one tile configuration
// (selected with -DMT_CFG=<n>) and all 4x4 operand layouts.  Built once per
// configuration so the instantiations compile in parallel.
#include "gemm_configs.hpp"

#ifndef MT_CFG
#error "build with -DMT_CFG=<tile configuration index>"
#endif

namespace mtk {
namespace {

template <int CFG, int LA, int LB>
hipError_t launch(const GemmParams& p, unsigned nblocks, hipStream_t s) {
    using C = TileCfg<CFG>;
    hipLaunchKernelGGL((gemm_f32_mfma<C::BM, C::BN, C::BK, C::WM, C::WN, LA, LB>),
                       dim3(nblocks), dim3(cfg_threads<CFG>()), 0, s, p);
    return hipGetLastError();
}

#define MT_ROW(CFG, LA) \
    { launch<CFG, LA, 0>, launch<CFG, LA, 1>, launch<CFG, LA, 2>, launch<CFG, LA, 3> }
#define MT_TABLE(CFG) { MT_ROW(CFG, 0), MT_ROW(CFG, 1), MT_ROW(CFG, 2), MT_ROW(CFG, 3) }

}  // namespace

// The tables live inside host functions so the device pass never sees them.
#if MT_CFG == 0
GemmLaunchFn launcher_cfg0(int la, int lb) {
    static const GemmLaunchFn table[kNumLayout][kNumLayout] = MT_TABLE(0);
    return table[la][lb];
}
#elif MT_CFG == 1
GemmLaunchFn launcher_cfg1(int la, int lb) {
    static const GemmLaunchFn table[kNumLayout][kNumLayout] = MT_TABLE(1);
    return table[la][lb];
}
#elif MT_CFG == 2
GemmLaunchFn launcher_cfg2(int la, int lb) {
    static const GemmLaunchFn table[kNumLayout][kNumLayout] = MT_TABLE(2);
    return table[la][lb];
}
#else
#error "unknown MT_CFG"
#endif

}  // namespace mtk

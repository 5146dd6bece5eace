// gemm_ksw_instances.hip -- instantiates gemm_f32_ksw (the wave-split kernel)
// for its tile configurations and the 2x2 choices of 16-byte or scalar
// fragment loads for A and B.
#include "gemm_configs.hpp"
#include "gemm_ksw_kernel.hpp"

namespace mtk {
namespace {

template <int CFG, bool VA, bool VB>
hipError_t launch_ksw(const GemmParams& p, unsigned nblocks, hipStream_t s) {
    using C = KswCfg<CFG>;
    hipLaunchKernelGGL((gemm_f32_ksw<C::MB, C::NB, C::W, VA, VB, C::D>), dim3(nblocks),
                       dim3(C::W * 64), 0, s, p);
    return hipGetLastError();
}

#define MT_KSW_TABLE(CFG) \
    { { launch_ksw<CFG, false, false>, launch_ksw<CFG, false, true> }, \
      { launch_ksw<CFG, true, false>, launch_ksw<CFG, true, true> } }

}  // namespace

GemmLaunchFn ksw_launcher(int cfg, bool va, bool vb) {
    static const GemmLaunchFn table[kNumKswCfg][2][2] = {MT_KSW_TABLE(0), MT_KSW_TABLE(1),
                                                          MT_KSW_TABLE(2), MT_KSW_TABLE(3)};
    return table[cfg][va][vb];
}

void ksw_tile(int cfg, int* bm, int* bn) {
    static const int tiles[kNumKswCfg][2] = {{32 * KswCfg<0>::MB, 32 * KswCfg<0>::NB},
                                             {32 * KswCfg<1>::MB, 32 * KswCfg<1>::NB},
                                             {32 * KswCfg<2>::MB, 32 * KswCfg<2>::NB},
                                             {32 * KswCfg<3>::MB, 32 * KswCfg<3>::NB}};
    *bm = tiles[cfg][0];
    *bn = tiles[cfg][1];
}

}  // namespace mtk

// gemm_ksw_instances.hip -- instantiates the wave-split kernels
// (gemm_f32_ksw, gemm_f32_ksw16) for their tile configurations and the 2x2 choices of 16-byte or scalar
// fragment loads for A and B.
#include "gemm_configs.hpp"
#include "gemm_ksw_kernel.hpp"

namespace mtk {
namespace {

template <int CFG, bool VA, bool VB>
hipError_t launch_ksw(const GemmParams& p, unsigned nblocks, hipStream_t s) {
    using C = KswCfg<CFG>;
    if constexpr (C::R == 32)
        hipLaunchKernelGGL((gemm_f32_ksw<C::MB, C::NB, C::W, VA, VB, C::D>), dim3(nblocks),
                           dim3(C::W * 64), 0, s, p);
    else
        hipLaunchKernelGGL((gemm_f32_ksw16<C::MB, C::NB, C::W, VA, VB, C::D>), dim3(nblocks),
                           dim3(C::W * 64), 0, s, p);
    return hipGetLastError();
}

#define MT_KSW_TABLE(CFG) \
    { { launch_ksw<CFG, false, false>, launch_ksw<CFG, false, true> }, \
      { launch_ksw<CFG, true, false>, launch_ksw<CFG, true, true> } }

}  // namespace

GemmLaunchFn ksw_launcher(int cfg, bool va, bool vb) {
    static const GemmLaunchFn table[kNumKswCfg][2][2] = {
        MT_KSW_TABLE(0), MT_KSW_TABLE(1), MT_KSW_TABLE(2), MT_KSW_TABLE(3),
        MT_KSW_TABLE(4), MT_KSW_TABLE(5), MT_KSW_TABLE(6), MT_KSW_TABLE(7), MT_KSW_TABLE(8)};
    return table[cfg][va][vb];
}

void ksw_tile(int cfg, int* bm, int* bn) {
    static const int tiles[kNumKswCfg][2] = {
        {KswTile<0>::bm, KswTile<0>::bn}, {KswTile<1>::bm, KswTile<1>::bn},
        {KswTile<2>::bm, KswTile<2>::bn}, {KswTile<3>::bm, KswTile<3>::bn},
        {KswTile<4>::bm, KswTile<4>::bn}, {KswTile<5>::bm, KswTile<5>::bn},
        {KswTile<6>::bm, KswTile<6>::bn}, {KswTile<7>::bm, KswTile<7>::bn},
        {KswTile<8>::bm, KswTile<8>::bn}};
    *bm = tiles[cfg][0];
    *bn = tiles[cfg][1];
}

}  // namespace mtk

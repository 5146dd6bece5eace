// gemm_dl_instances.hip -- instantiates gemm_f32_dl for one tile
// configuration (selected with -DMT_CFG=<n>): the 2x2 vector operand layouts
// (k-contiguous / mn-contiguous for A and for B), the implicit-im2col
// convolution (A k-contiguous weights, B = L_IM from a channels-last input or
// L_IMR from an NCHW view) and its weight gradient
// (A = dY as [c_out][n*h_out*w_out], B = L_IMW), and the mn-contiguous pair
// with fused row sums of A (the Linear dW GEMM with its bias gradient), the
// weight gradient with dY read in NCHW (A = L_KVI); and
// the halo-patch convolution kernel gemm_f32_dlh of the same tile.
#include "gemm_configs.hpp"
#include "gemm_dl_kernel.hpp"
#include "gemm_dlh_kernel.hpp"

#ifndef MT_CFG
#error "build with -DMT_CFG=<tile configuration index>"
#endif

namespace mtk {
namespace {

template <int CFG, int LA, int LB, bool RS = false>
hipError_t launch_dl(const GemmParams& p, unsigned nblocks, hipStream_t s) {
    using C = DlCfg<CFG>;
    hipLaunchKernelGGL((gemm_f32_dl<C::BM, C::BN, C::WM, C::WN, LA, LB, C::STAGES, RS>),
                       dim3(nblocks), dim3(dl_threads<CFG>()), 0, s, p);
    return hipGetLastError();
}

// The halo-patch kernel's LDS depends on the convolution's geometry.
template <int CFG>
hipError_t launch_dlh(const GemmParams& p, unsigned nblocks, hipStream_t s) {
    using C = DlCfg<CFG>;
    const size_t bytes = sizeof(float) * dlh_lds_floats<C::BM, C::BN, C::WM, C::WN>(p.cv);
    HaloTable t;
    halo_table(p.cv, C::BN, &t);
    hipLaunchKernelGGL((gemm_f32_dlh<C::BM, C::BN, C::WM, C::WN>), dim3(nblocks),
                       dim3(dl_threads<CFG>()), bytes, s, p, t);
    return hipGetLastError();
}

#define MT_DL_TABLE(CFG) \
    { { launch_dl<CFG, L_KV, L_KV>, launch_dl<CFG, L_KV, L_MV> }, \
      { launch_dl<CFG, L_MV, L_KV>, launch_dl<CFG, L_MV, L_MV> } }

}  // namespace

#if MT_CFG == 0
GemmLaunchFn dl_launcher_cfg0(int la, int lb) {
    static const GemmLaunchFn table[2][2] = MT_DL_TABLE(0);
    return table[la][lb];
}
GemmLaunchFn dl_conv_launcher_cfg0() { return launch_dl<0, L_KV, L_IM>; }
GemmLaunchFn dl_convr_launcher_cfg0() { return launch_dl<0, L_KV, L_IMR>; }
GemmLaunchFn dl_convh_launcher_cfg0() { return launch_dlh<0>; }
GemmLaunchFn dl_convw_launcher_cfg0() { return launch_dl<0, L_KV, L_IMW>; }
GemmLaunchFn dl_convwi_launcher_cfg0() { return launch_dl<0, L_KVI, L_IMW>; }
GemmLaunchFn dl_rowsum_launcher_cfg0(bool kv) {
    return kv ? launch_dl<0, L_KV, L_KV, true> : launch_dl<0, L_MV, L_MV, true>;
}
#elif MT_CFG == 1
GemmLaunchFn dl_launcher_cfg1(int la, int lb) {
    static const GemmLaunchFn table[2][2] = MT_DL_TABLE(1);
    return table[la][lb];
}
GemmLaunchFn dl_conv_launcher_cfg1() { return launch_dl<1, L_KV, L_IM>; }
GemmLaunchFn dl_convr_launcher_cfg1() { return launch_dl<1, L_KV, L_IMR>; }
GemmLaunchFn dl_convh_launcher_cfg1() { return launch_dlh<1>; }
GemmLaunchFn dl_convw_launcher_cfg1() { return launch_dl<1, L_KV, L_IMW>; }
GemmLaunchFn dl_convwi_launcher_cfg1() { return launch_dl<1, L_KVI, L_IMW>; }
GemmLaunchFn dl_rowsum_launcher_cfg1(bool kv) {
    return kv ? launch_dl<1, L_KV, L_KV, true> : launch_dl<1, L_MV, L_MV, true>;
}
#elif MT_CFG == 2
GemmLaunchFn dl_launcher_cfg2(int la, int lb) {
    static const GemmLaunchFn table[2][2] = MT_DL_TABLE(2);
    return table[la][lb];
}
GemmLaunchFn dl_conv_launcher_cfg2() { return launch_dl<2, L_KV, L_IM>; }
GemmLaunchFn dl_convr_launcher_cfg2() { return launch_dl<2, L_KV, L_IMR>; }
GemmLaunchFn dl_convh_launcher_cfg2() { return launch_dlh<2>; }
GemmLaunchFn dl_convw_launcher_cfg2() { return launch_dl<2, L_KV, L_IMW>; }
GemmLaunchFn dl_convwi_launcher_cfg2() { return launch_dl<2, L_KVI, L_IMW>; }
GemmLaunchFn dl_rowsum_launcher_cfg2(bool kv) {
    return kv ? launch_dl<2, L_KV, L_KV, true> : launch_dl<2, L_MV, L_MV, true>;
}
#elif MT_CFG == 3
GemmLaunchFn dl_launcher_cfg3(int la, int lb) {
    static const GemmLaunchFn table[2][2] = MT_DL_TABLE(3);
    return table[la][lb];
}
GemmLaunchFn dl_conv_launcher_cfg3() { return launch_dl<3, L_KV, L_IM>; }
GemmLaunchFn dl_convr_launcher_cfg3() { return launch_dl<3, L_KV, L_IMR>; }
GemmLaunchFn dl_convh_launcher_cfg3() { return launch_dlh<3>; }
GemmLaunchFn dl_convw_launcher_cfg3() { return launch_dl<3, L_KV, L_IMW>; }
GemmLaunchFn dl_convwi_launcher_cfg3() { return launch_dl<3, L_KVI, L_IMW>; }
GemmLaunchFn dl_rowsum_launcher_cfg3(bool kv) {
    return kv ? launch_dl<3, L_KV, L_KV, true> : launch_dl<3, L_MV, L_MV, true>;
}
#else
#error "unknown MT_CFG"
#endif

}  // namespace mtk

// gemm_dlp_instances.hip -- instantiates gemm_f32_dlp (direct-to-LDS with
// fragment prefetch) for direct-to-LDS configurations 4-6, with and
// without a partial last K-chunk, for the 2x2 vector operand layouts (and the
// row-sum form of two mn-contiguous operands) and the convolution weight
// gradient (A = dY k-contiguous or read in NCHW, B = L_IMW).
#include "gemm_configs.hpp"
#include "gemm_dlp_kernel.hpp"

namespace mtk {
namespace {

template <int CFG, bool TAIL, int LA, int LB, bool RS = false>
hipError_t launch_dlp(const GemmParams& p, unsigned nblocks, hipStream_t s) {
    using C = DlCfg<CFG>;
    hipLaunchKernelGGL(
        (gemm_f32_dlp<C::BM, C::BN, C::WM, C::WN, LA, LB, C::STAGES, C::WPE, TAIL, RS>),
        dim3(nblocks), dim3(dl_threads<CFG>()), 0, s, p);
    return hipGetLastError();
}

#define MT_DLP_TABLE(CFG, TAIL) \
    { { launch_dlp<CFG, TAIL, L_KV, L_KV>, launch_dlp<CFG, TAIL, L_KV, L_MV> }, \
      { launch_dlp<CFG, TAIL, L_MV, L_KV>, launch_dlp<CFG, TAIL, L_MV, L_MV> } }

}  // namespace

GemmLaunchFn dlp_convw_launcher(int cfg, bool tail) {
    static const GemmLaunchFn table[3][2] = {
        {launch_dlp<4, false, L_KV, L_IMW>, launch_dlp<4, true, L_KV, L_IMW>},
        {launch_dlp<5, false, L_KV, L_IMW>, launch_dlp<5, true, L_KV, L_IMW>},
        {launch_dlp<6, false, L_KV, L_IMW>, launch_dlp<6, true, L_KV, L_IMW>}};
    return table[cfg - 4][tail];
}

GemmLaunchFn dlp_convwi_launcher(int cfg) {
    static const GemmLaunchFn table[3] = {launch_dlp<4, false, L_KVI, L_IMW>,
                                          launch_dlp<5, false, L_KVI, L_IMW>,
                                          launch_dlp<6, false, L_KVI, L_IMW>};
    return table[cfg - 4];
}

GemmLaunchFn dlp_rowsum_launcher(int cfg, bool tail, bool kv) {
    static const GemmLaunchFn table[3][2][2] = {
        {{launch_dlp<4, false, L_MV, L_MV, true>, launch_dlp<4, true, L_MV, L_MV, true>},
         {launch_dlp<4, false, L_KV, L_KV, true>, launch_dlp<4, true, L_KV, L_KV, true>}},
        {{launch_dlp<5, false, L_MV, L_MV, true>, launch_dlp<5, true, L_MV, L_MV, true>},
         {launch_dlp<5, false, L_KV, L_KV, true>, launch_dlp<5, true, L_KV, L_KV, true>}},
        {{launch_dlp<6, false, L_MV, L_MV, true>, launch_dlp<6, true, L_MV, L_MV, true>},
         {launch_dlp<6, false, L_KV, L_KV, true>, launch_dlp<6, true, L_KV, L_KV, true>}}};
    if (cfg < 4 || cfg > 6) return nullptr;
    return table[cfg - 4][kv][tail];
}

GemmLaunchFn dlp_launcher(int cfg, bool tail, int la, int lb) {
    static const GemmLaunchFn table[3][2][2][2] = {
        {MT_DLP_TABLE(4, false), MT_DLP_TABLE(4, true)},
        {MT_DLP_TABLE(5, false), MT_DLP_TABLE(5, true)},
        {MT_DLP_TABLE(6, false), MT_DLP_TABLE(6, true)}};
    return table[cfg - 4][tail][la][lb];
}

}  // namespace mtk

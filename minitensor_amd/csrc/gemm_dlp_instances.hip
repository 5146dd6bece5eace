// gemm_dlp_instances.hip -- instantiates gemm_f32_dlp (direct-to-LDS, one
// 128x128 wave tile per SIMD, fragment prefetch) for the 2x2 vector operand
// layouts: direct-to-LDS tile configuration kDlpCfg.
#include "gemm_configs.hpp"
#include "gemm_dlp_kernel.hpp"

namespace mtk {
namespace {

template <int LA, int LB>
hipError_t launch_dlp(const GemmParams& p, unsigned nblocks, hipStream_t s) {
    using C = DlCfg<kDlpCfg>;
    hipLaunchKernelGGL((gemm_f32_dlp<LA, LB, C::STAGES>), dim3(nblocks),
                       dim3(dl_threads<kDlpCfg>()), 0, s, p);
    return hipGetLastError();
}

}  // namespace

GemmLaunchFn dlp_launcher(int la, int lb) {
    static const GemmLaunchFn table[2][2] = {
        {launch_dlp<L_KV, L_KV>, launch_dlp<L_KV, L_MV>},
        {launch_dlp<L_MV, L_KV>, launch_dlp<L_MV, L_MV>}};
    return table[la][lb];
}

}  // namespace mtk

// gemm_skinny_instances.hip -- instantiates the vector-ALU kernels of the
// HBM-bound shapes (gemm_skinny_kernel.hpp): the GEMV kernels for 1, 2, 4 and
// 8 rows with B mn- or k-contiguous, the rank-k kernel for K <= 4 and
// K <= 16, and the reduction of the GEMV kernels' split-K partials.
#include "gemm_configs.hpp"
#include "gemm_skinny_kernel.hpp"

namespace mtk {
namespace {

template <int MR>
hipError_t launch_gemv_mv(const GemmParams& p, unsigned nblocks, hipStream_t s) {
    hipLaunchKernelGGL(gemv_mv_f32<MR>, dim3(nblocks), dim3(64 * gemv_mv_waves<MR>()), 0, s, p);
    return hipGetLastError();
}

template <int MR>
hipError_t launch_gemv_kv(const GemmParams& p, unsigned nblocks, hipStream_t s) {
    hipLaunchKernelGGL(gemv_kv_f32<MR>, dim3(nblocks), dim3(256), 0, s, p);
    return hipGetLastError();
}

template <int KMAX>
hipError_t launch_rankk(const GemmParams& p, unsigned nblocks, hipStream_t s) {
    hipLaunchKernelGGL(rankk_f32<KMAX>, dim3(nblocks), dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace

GemmLaunchFn gemv_launcher(bool kv, int rows) {
    static const GemmLaunchFn mv[4] = {launch_gemv_mv<1>, launch_gemv_mv<2>, launch_gemv_mv<4>,
                                       launch_gemv_mv<8>};
    static const GemmLaunchFn kvt[4] = {launch_gemv_kv<1>, launch_gemv_kv<2>, launch_gemv_kv<4>,
                                        launch_gemv_kv<8>};
    const int i = rows <= 1 ? 0 : rows <= 2 ? 1 : rows <= 4 ? 2 : rows <= 8 ? 3 : -1;
    if (i < 0) return nullptr;
    return kv ? kvt[i] : mv[i];
}

GemmLaunchFn rankk_launcher(int K) {
    if (K < 1 || K > kRankKMax) return nullptr;
    return K <= 4 ? launch_rankk<4> : launch_rankk<16>;
}

hipError_t launch_skinny_reduce(const GemmParams& p, hipStream_t s) {
    const dim3 grid((unsigned)((p.N / 4 + kSkRedCols - 1) / kSkRedCols), (unsigned)(p.M * p.batch));
    hipLaunchKernelGGL(skinny_reduce_f32, grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace mtk

// gemm_dl16_instances.hip -- instantiates the convolution kernel on 16x16
// MFMA blocks (gemm_f32_dl16: A = k-contiguous weights, B = L_IM from a
// channels-last input) for every Dl16Cfg.
#include "gemm_configs.hpp"
#include "gemm_dl16_kernel.hpp"

namespace mtk {
namespace {

template <int CFG>
hipError_t launch_dl16(const GemmParams& p, unsigned nblocks, hipStream_t s) {
    using C = Dl16Cfg<CFG>;
    constexpr int threads = C::KG * (C::BM / C::WM) * (C::BN / C::WN) * 64;
    hipLaunchKernelGGL((gemm_f32_dl16<C::BM, C::BN, C::WM, C::WN, C::KG, C::STAGES, C::PRE>),
                       dim3(nblocks), dim3(threads), 0, s, p);
    return hipGetLastError();
}

}  // namespace

GemmLaunchFn dl16_conv_launcher(int cfg16) {
    static const GemmLaunchFn table[kNumDl16Cfg] = {launch_dl16<0>};
    return cfg16 >= 0 && cfg16 < kNumDl16Cfg ? table[cfg16] : nullptr;
}

void dl16_tile(int cfg16, int* bm, int* bn) {
    static constexpr int kBm[kNumDl16Cfg] = {Dl16Cfg<0>::BM};
    static constexpr int kBn[kNumDl16Cfg] = {Dl16Cfg<0>::BN};
    *bm = kBm[cfg16];
    *bn = kBn[cfg16];
}

}  // namespace mtk

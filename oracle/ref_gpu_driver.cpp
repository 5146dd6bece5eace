// ref_gpu_driver.cpp -- TEST INFRASTRUCTURE ONLY.  A C-ABI shim, written for
// this repository, around the reference's own GPU matmul, so the tests can run
// the reference's kernel on the same MI355X as this build and compare time and
// results.  It is compiled with hipcc for gfx950 against the reference headers
// where they lie, and linked with the reference's src/gpu_ops.cpp compiled
// unchanged (oracle/Makefile, target ref_gpu) into oracle/_ref/libref_gpu.so.
// No reference source is copied here; only its public API is called:
//   matmul_gpu<float>          src/gpu_ops.cpp:1103-1144 -> sgemm_kernel_v2 (932-1101)
//   matmul_gpu_strided<float>  src/gpu_ops.cpp:1199-1223 -> matmul_kernel_strided (909-930)
// on the reference's GPU tensors (Tensor::to(Device{DeviceType::CUDA})), timed
// the way its benchmark times them (test/benchmark.cpp:162-190: preallocated
// A, B, C, warm-up, then back-to-back calls), here with HIP events.
#include <hip/hip_runtime.h>

#include <cstring>
#include <vector>

#include "Tensor.hpp"
#include "TensorOps.hpp"

namespace {

Tensor<float> gpu_tensor(const float* src, std::vector<size_t> shape) {
    Tensor<float> t(shape, Device{DeviceType::CPU});
    std::memcpy(t.data(), src, t.total_elements() * sizeof(float));
    return t.to(Device{DeviceType::CUDA});
}

}  // namespace

extern "C" {

// which = 0: matmul_gpu (the contiguous launcher, v2 kernel for M, N >= 64);
// which = 1: matmul_gpu_strided with B read through its transpose view
//            (b holds Bᵀ [N][K]: the benchmark's config 3 access pattern).
// Writes C [M][N] to c and the mean ms per call to *ms.  Returns 0, or -1 on
// a HIP error.
int ref_gpu_matmul_f32(const float* a, const float* b, float* c, int M, int K, int N, int which,
                       int warmup, int reps, double* ms) {
    Tensor<float> A = gpu_tensor(a, {(size_t)M, (size_t)K});
    Tensor<float> B = which == 1 ? gpu_tensor(b, {(size_t)N, (size_t)K}).transpose(0, 1)
                                 : gpu_tensor(b, {(size_t)K, (size_t)N});
    Tensor<float> C({(size_t)M, (size_t)N}, Device{DeviceType::CUDA});
    auto call = [&] {
        if (which == 1) matmul_gpu_strided<float>(A, B, C);
        else matmul_gpu<float>(A, B, C);
    };
    for (int i = 0; i < warmup; ++i) call();
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1;
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    hipEventRecord(e0, active_stream());
    for (int i = 0; i < reps; ++i) call();
    hipEventRecord(e1, active_stream());
    if (hipEventSynchronize(e1) != hipSuccess) return -1;
    float total = 0.f;
    hipEventElapsedTime(&total, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    *ms = reps > 0 ? total / reps : 0.0;
    Tensor<float> h = C.to(Device{DeviceType::CPU});
    std::memcpy(c, h.data() + h.offset(), (size_t)M * N * sizeof(float));
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"

// Verification hook for the sampler's libm (no reference counterpart): evaluates the device
// expf / exp / logf of glibc_math.h, exactly as the sampler and beam kernels call them, on
// the float inputs with bit patterns first + i * stride (i < count).  exp takes the float
// widened to double, as the sampler does (gpt_sampling.cpp:96, :144).
#include <hip/hip_runtime.h>

#include "chain_sum.h"
#include "glibc_math.h"
#include "itts_gpt.h"

namespace itts {
namespace {

__global__ void libm_eval_kernel(int fn, uint64_t first, uint64_t stride, uint64_t count, void* out) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const float x = __uint_as_float(static_cast<uint32_t>(first + i * stride));
        if (fn == ITTS_LIBM_EXPF)
            static_cast<float*>(out)[i] = libm::expf_glibc(x);
        else if (fn == ITTS_LIBM_EXP)
            static_cast<double*>(out)[i] = libm::exp_glibc(static_cast<double>(x));
        else
            static_cast<float*>(out)[i] = libm::logf_glibc(x);
    }
}

// One workgroup per row of 8194 values: the row is staged in LDS (zero-padded as
// chain::sum_wave expects), then wave 0 forms the beam scores' index-order float sum.
constexpr int kChainThreads = 1024;
__global__ __launch_bounds__(kChainThreads) void chain_sum_kernel(const float* in, float* out) {
    __shared__ __align__(16) float e[chain::kPad];
    const float* row = in + static_cast<size_t>(blockIdx.x) * kMelVocab;
    constexpr int kPer = (chain::kPad + kChainThreads - 1) / kChainThreads;
    float v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = threadIdx.x + u * kChainThreads;
        v[u] = i < kMelVocab ? row[i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = threadIdx.x + u * kChainThreads;
        if (i < chain::kPad) e[i] = v[u];
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const float s = chain::sum_wave(e, threadIdx.x);
        if (threadIdx.x == 0) out[blockIdx.x] = s;
    }
}

}  // namespace
}  // namespace itts

extern "C" int itts_chain_sum_eval(const float* values, uint32_t rows, float* out) {
    if (!values || !out || rows == 0 || rows > 65536) return ITTS_EINVAL;
    const size_t in_bytes = static_cast<size_t>(rows) * itts::kMelVocab * 4;
    float* d = nullptr;
    if (hipMalloc(&d, in_bytes + rows * 4) != hipSuccess) return ITTS_ERUNTIME;
    hipError_t e = hipMemcpy(d, values, in_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(itts::chain_sum_kernel, dim3(rows), dim3(itts::kChainThreads), 0, nullptr, d, d + static_cast<size_t>(rows) * itts::kMelVocab);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(out, d + static_cast<size_t>(rows) * itts::kMelVocab, rows * 4, hipMemcpyDeviceToHost);
    (void)hipFree(d);
    return e == hipSuccess ? ITTS_OK : ITTS_ERUNTIME;
}

extern "C" int itts_libm_eval(int32_t fn, uint64_t first_bits, uint64_t stride, uint64_t count, void* out) {
    if (fn < ITTS_LIBM_EXPF || fn > ITTS_LIBM_LOGF || !out || count == 0 || count > (1ull << 28) || stride == 0 ||
        first_bits + (count - 1) * stride > 0xffffffffull)
        return ITTS_EINVAL;
    const size_t bytes = count * (fn == ITTS_LIBM_EXP ? 8 : 4);
    void* d = nullptr;
    if (hipMalloc(&d, bytes) != hipSuccess) return ITTS_ERUNTIME;
    hipLaunchKernelGGL(itts::libm_eval_kernel, dim3(4096), dim3(256), 0, nullptr, fn, first_bits, stride, count, d);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipMemcpy(out, d, bytes, hipMemcpyDeviceToHost);
    (void)hipFree(d);
    return e == hipSuccess ? ITTS_OK : ITTS_ERUNTIME;
}

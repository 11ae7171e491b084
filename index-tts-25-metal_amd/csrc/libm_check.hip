// Verification hook for the sampler's libm (no reference counterpart): evaluates the device
// expf / exp / logf of glibc_math.h, exactly as the sampler and beam kernels call them, on
// the float inputs with bit patterns first + i * stride (i < count).  exp takes the float
// widened to double, as the sampler does (gpt_sampling.cpp:96, :144).
#include <hip/hip_runtime.h>

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

}  // namespace
}  // namespace itts

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

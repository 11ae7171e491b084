// On-device logits processors and sampler for decode and for the processor/sampler API:
// one 1024-thread workgroup per sequence (see sampler_dev.h for what is restated from
// src/gpt_sampling.cpp and how the reference's summation order is kept).
#include "sampler_dev.h"

namespace itts {
namespace {
using namespace sampling;

__global__ __launch_bounds__(NT) void sampler_kernel(SampleArgs a) {
    __shared__ Smem sm;
    sample_sequence<NT, true>(sm, a, blockIdx.x);
}

}  // namespace

hipError_t launch_sampler(const SampleArgs& a, int batch, hipStream_t s) {
    hipLaunchKernelGGL(sampler_kernel, dim3(batch), dim3(NT), 0, s, a);
    return hipGetLastError();
}

}  // namespace itts

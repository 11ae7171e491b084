// On-device logits processors and sampler for decode and for the processor/sampler API:
// one 1024-thread workgroup per sequence (see sampler_dev.h for what is restated from
// src/gpt_sampling.cpp and how the reference's summation order is kept).
#include "sampler_dev.h"

namespace itts {
namespace {
using namespace sampling;

__global__ __launch_bounds__(NT) void sampler_kernel(SampleArgs a) {
    __shared__ Smem sm;
    const int b = blockIdx.x, t = threadIdx.x;
    SeqState& st = a.state[b];
    if (a.mode == kModeDecode && !st.active) return;
    const bool processors = a.mode != kModeDraw;
    const bool need_sample = a.mode == kModeDraw || (a.mode == kModeDecode && st.do_sample);
    const float* lg = a.logits + static_cast<size_t>(b) * a.logit_stride;
    {
        float v[IPT];  // all loads in flight before the first store
#pragma unroll
        for (int q = 0; q < IPT; ++q) {
            const int i = t + q * NT;
            v[q] = i < V ? lg[i] : 0.0f;
        }
        const bool drop_stop = processors && st.suppress_stop;
#pragma unroll
        for (int q = 0; q < IPT; ++q) {
            const int i = t + q * NT;
            if (i < V) sm.s[i] = drop_stop && (i == kMelStart || i == kMelStop) ? -INFINITY : v[q];
        }
    }
    __syncthreads();
    double* Pg = a.probs + static_cast<size_t>(b) * V;
    uint32_t status = kOk;
    bool topp = false;
    if (processors)
        status = run_processors(sm, a.seen + static_cast<size_t>(b) * V, st.penalty, st.temperature, st.top_k, st.top_p,
                                st.num_beams, Pg, a.mode == kModeProcessors, &topp);
    uint32_t token = 0;
    if (status == kOk) {
        if (a.mode == kModeProcessors) {
            float* out = a.out_scores + static_cast<size_t>(b) * V;
            for (int i = t; i < V; i += NT) out[i] = sm.s[i];
        } else if (!need_sample) {
            token = block_argmax(sm);  // greedy: std::max_element
        } else {
            uint32_t m = sm.m;
            if (!topp) {
                m = compact_finite(sm);
                if (m == 0) status = kNoFinite;
                else {
                    double* P = m <= static_cast<uint32_t>(kSmallProbs) ? sm.probs : Pg;
                    const float mx = sm.mx;
                    for (uint32_t j = t; j < m; j += NT) P[j] = libm::exp_glibc(static_cast<double>(sm.s[sm.list[j]] - mx));
                    __syncthreads();
                }
            }
            if (status == kOk && t < 64) {
                // wave 0 draws; every lane holds the same rng, token and status
                const double* P = m <= static_cast<uint32_t>(kSmallProbs) ? sm.probs : Pg;
                uint64_t rng = st.rng;
                const int draws = a.mode == kModeDraw ? a.draws : 1;
                for (int d = 0; d < draws && status == kOk; ++d) {
                    token = draw_token_wave(sm, m, P, rng, &status);
                    if (a.mode == kModeDraw && t == 0) a.out_tokens[d] = token;
                }
                if (t == 0) st.rng = rng;
            }
        }
    }
    if (t != 0) return;
    a.status[b] = status;
    if (a.mode != kModeDecode) return;
    if (status != kOk) {
        st.error = 1;
        st.active = 0;
        return;
    }
    // Accept the token and advance the state (gpt_sampling.cpp:181-186).
    if (token == static_cast<uint32_t>(kMelStop)) {
        st.stopped = 1;
        st.active = 0;
    } else if (token >= static_cast<uint32_t>(kMelStart)) {
        a.status[b] = kInvalidCode;
        st.error = 1;
        st.active = 0;
    } else {
        a.codes[static_cast<size_t>(b) * a.code_stride + st.count] = token;
        st.count += 1;
        a.seen[static_cast<size_t>(b) * V + token] = 1;
        if (st.count >= st.max_tokens) {
            st.active = 0;
        } else {
            st.token = token;
            st.position = st.count + 1;  // the first generated code sits at mel position 2
            st.n = st.prefix_rows + st.count - 1;
        }
    }
}

}  // namespace

hipError_t launch_sampler(const SampleArgs& a, int batch, hipStream_t s) {
    hipLaunchKernelGGL(sampler_kernel, dim3(batch), dim3(NT), 0, s, a);
    return hipGetLastError();
}

}  // namespace itts

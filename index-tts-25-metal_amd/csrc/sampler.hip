// On-device logits processors and sampler: one 1024-thread workgroup per sequence.
//
// Restates, in the reference's order and arithmetic:
//   apply_gpt_sampling_processors   src/gpt_sampling.cpp:28-128
//     repetition penalty once per distinct history id (x<0 ? x*p : x/p), then /= T,
//     then top-k (pivot = k-th largest, values below it -> -inf, ties survive), then
//     top-p (ascending (score, index) order, double softmax, drop while cumulative <= 1-p,
//     always keep the top 1, or top 2 for beams);
//   sample_gpt_token_from_logits    src/gpt_sampling.cpp:130-165
//     p_i = exp(double(s_i - max)), total in index order, target = u * total, first i
//     (index order) with target < cumulative, else the last finite one;
//   SplitMix64                       src/gpt_sampling.cpp:11-26 (state kept in SeqState).
// Only the ordering-free parts run in parallel (elementwise penalty/temperature, a
// 4-pass radix select for the top-k pivot, compaction, a bitonic sort of the
// survivors).  Every floating-point sum the reference forms sequentially (probability
// totals, cumulative sums) is formed by one thread in the same order, so the mask and
// the drawn token follow the reference exactly given the same logits and RNG state.
#include "kernels.h"

namespace itts {
namespace {

constexpr int V = kMelVocab;
constexpr int NT = 1024;
constexpr int NWAVE = NT / 64;
constexpr int IPT = (V + NT - 1) / NT;  // contiguous indices per thread for compaction (9)
constexpr int kSortMax = 16384;          // next power of two >= V
constexpr int kSmallProbs = 1024;
constexpr uint16_t kRemoved = 0x8000;

enum Status : uint32_t {
    kOk = 0,
    kTopPEmpty = 1,    // "GPT top_p filtering removed all logits"
    kZeroMass = 2,     // "GPT sampling probability mass is zero"
    kNoFinite = 3,     // "GPT sampling received no finite logits"
    kInvalidCode = 4,  // "GPT generated invalid semantic code"
};

struct Smem {
    union {
        float s[V];
        uint64_t sortbuf[kSortMax];
    };
    uint16_t list[V];  // finite survivors in index order; bit 15 = removed by top-p
    double probs[kSmallProbs];
    uint32_t hist[256];
    uint32_t wtot[NWAVE];
    float wmax[NWAVE];
    uint32_t widx[NWAVE];
    uint32_t sel[2];
    uint32_t m;
    uint32_t token;
    uint32_t status;
    float mx;
};

__device__ __forceinline__ uint64_t splitmix_next(uint64_t& state) {
    uint64_t z = (state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ double splitmix_unit(uint64_t& state) {
    return static_cast<double>(splitmix_next(state) >> 11) * (1.0 / 9007199254740992.0);
}

__device__ __forceinline__ bool finite_f(float v) { return fabsf(v) <= 3.402823466e38f; }

// kk-th largest value (1-based) of s[0..V): MSB-first radix select on order-preserving keys.
__device__ float radix_kth_largest(Smem& sm, uint32_t kk) {
    const int t = threadIdx.x, lane = t & 63;
    uint32_t prefix = 0, mask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (t < 256) sm.hist[t] = 0;
        __syncthreads();
        for (int i = t; i < V; i += NT) {
            const uint32_t k = float_key(sm.s[i]);
            if ((k & mask) == prefix) atomicAdd(&sm.hist[(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (t < 64) {
            uint32_t c[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) c[q] = sm.hist[255 - 4 * lane - q];
            const uint32_t loc = c[0] + c[1] + c[2] + c[3];
            uint32_t inc = loc;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t v = __shfl_up(inc, o, 64);
                if (lane >= o) inc += v;
            }
            const uint32_t exc = inc - loc;
            if (exc < kk && kk <= inc) {
                uint32_t run = exc;
                int d = -1;
                uint32_t above = 0;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (d < 0) {
                        if (run + c[q] >= kk) {
                            d = 255 - 4 * lane - q;
                            above = run;
                        } else {
                            run += c[q];
                        }
                    }
                }
                sm.sel[0] = static_cast<uint32_t>(d);
                sm.sel[1] = above;
            }
        }
        __syncthreads();
        prefix |= sm.sel[0] << shift;
        mask |= 0xffu << shift;
        kk -= sm.sel[1];
        __syncthreads();
    }
    return key_float(prefix);
}

// Compact finite entries of s into sm.list (index order); returns the count, sets sm.mx.
__device__ uint32_t compact_finite(Smem& sm) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int i0 = t * IPT, i1 = min(V, i0 + IPT);
    uint32_t c = 0;
    float mloc = -INFINITY;
    for (int i = i0; i < i1; ++i) {
        const float v = sm.s[i];
        if (finite_f(v)) {
            ++c;
            mloc = fmaxf(mloc, v);
        }
    }
    uint32_t inc = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(inc, o, 64);
        if (lane >= o) inc += v;
    }
    const float wm = wave_max(mloc);
    if (lane == 63) sm.wtot[wave] = inc;
    if (lane == 0) sm.wmax[wave] = wm;
    __syncthreads();
    uint32_t off = 0, total = 0;
    float mx = -INFINITY;
    for (int w = 0; w < NWAVE; ++w) {
        if (w < wave) off += sm.wtot[w];
        total += sm.wtot[w];
        mx = fmaxf(mx, sm.wmax[w]);
    }
    off += inc - c;
    for (int i = i0; i < i1; ++i)
        if (finite_f(sm.s[i])) sm.list[off++] = static_cast<uint16_t>(i);
    if (t == 0) {
        sm.m = total;
        sm.mx = mx;
    }
    __syncthreads();
    return total;
}

// First index of the maximum (std::max_element semantics).
__device__ uint32_t block_argmax(Smem& sm) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    float best = -INFINITY;
    uint32_t bi = V;
    for (int i = t; i < V; i += NT) {
        const float v = sm.s[i];
        if (v > best || (v == best && static_cast<uint32_t>(i) < bi)) {
            best = v;
            bi = static_cast<uint32_t>(i);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const uint32_t oi = __shfl_xor(bi, o, 64);
        if (ov > best || (ov == best && oi < bi)) {
            best = ov;
            bi = oi;
        }
    }
    if (lane == 0) {
        sm.wmax[wave] = best;
        sm.widx[wave] = bi;
    }
    __syncthreads();
    float b2 = sm.wmax[0];
    uint32_t i2 = sm.widx[0];
    for (int w = 1; w < NWAVE; ++w)
        if (sm.wmax[w] > b2 || (sm.wmax[w] == b2 && sm.widx[w] < i2)) {
            b2 = sm.wmax[w];
            i2 = sm.widx[w];
        }
    __syncthreads();
    return i2;
}

// Ascending bitonic sort of sm.sortbuf[0..n), n a power of two.
__device__ void bitonic_sort(Smem& sm, int n) {
    const int t = threadIdx.x;
    if (n <= 64) {
        if (t < 64) {
            uint64_t v = t < n ? sm.sortbuf[t] : ~0ull;
            for (int k = 2; k <= 64; k <<= 1)
                for (int j = k >> 1; j > 0; j >>= 1) {
                    const uint64_t o = __shfl_xor(v, j, 64);
                    const bool lower = (t & j) == 0;
                    const bool asc = (t & k) == 0;
                    const uint64_t lo = v < o ? v : o, hi = v < o ? o : v;
                    v = (lower == asc) ? lo : hi;
                }
            if (t < n) sm.sortbuf[t] = v;
        }
        __syncthreads();
        return;
    }
    for (int k = 2; k <= n; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int p = t; p < n / 2; p += NT) {
                const int i = (p / j) * 2 * j + (p % j);
                const int l = i + j;
                const bool asc = (i & k) == 0;
                const uint64_t a = sm.sortbuf[i], c = sm.sortbuf[l];
                if ((a > c) == asc) {
                    sm.sortbuf[i] = c;
                    sm.sortbuf[l] = a;
                }
            }
            __syncthreads();
        }
}

__global__ __launch_bounds__(NT) void sampler_kernel(SampleArgs a) {
    __shared__ Smem sm;
    const int b = blockIdx.x, t = threadIdx.x;
    SeqState& st = a.state[b];
    if (a.mode == kModeDecode && !st.active) return;
    const float T = st.temperature, top_p = st.top_p, pen = st.penalty;
    const uint32_t top_k = st.top_k, beams = st.num_beams;
    const bool processors = a.mode != kModeDraw;
    const bool need_sample = a.mode == kModeDraw || (a.mode == kModeDecode && st.do_sample);
    const float* lg = a.logits + static_cast<size_t>(b) * a.logit_stride;
    const uint8_t* seen = a.seen + static_cast<size_t>(b) * V;

    for (int i = t; i < V; i += NT) {
        float v = lg[i];
        if (processors) {
            if (st.suppress_stop && (i == kMelStart || i == kMelStop)) v = -INFINITY;
            if (pen != 1.0f && seen[i]) v = v < 0.0f ? v * pen : v / pen;
            if (T != 1.0f) v = v / T;
        }
        sm.s[i] = v;
    }
    if (t == 0) sm.status = kOk;
    __syncthreads();

    if (processors && top_k > 0 && top_k < static_cast<uint32_t>(V)) {
        const uint32_t k = max(top_k, beams > 1 ? 2u : 1u);
        const float pivot = radix_kth_largest(sm, k);
        for (int i = t; i < V; i += NT)
            if (sm.s[i] < pivot) sm.s[i] = -INFINITY;
        __syncthreads();
    }
    const bool do_topp = processors && top_p < 1.0f;
    float* out_scores = a.mode == kModeProcessors ? a.out_scores + static_cast<size_t>(b) * V : nullptr;

    if (!do_topp && !need_sample) {
        if (out_scores) {
            for (int i = t; i < V; i += NT) out_scores[i] = sm.s[i];
            if (t == 0) a.status[b] = kOk;
            return;
        }
        const uint32_t tok = block_argmax(sm);  // greedy: std::max_element
        if (t == 0) sm.token = tok;
    } else {
        if (out_scores)
            for (int i = t; i < V; i += NT) out_scores[i] = sm.s[i];
        const uint32_t m = compact_finite(sm);
        if (m == 0) {
            if (t == 0) a.status[b] = do_topp ? kTopPEmpty : kNoFinite;
            if (t == 0 && a.mode == kModeDecode) {
                st.error = 1;
                st.active = 0;
            }
            return;
        }
        const float mx = sm.mx;
        double* P = m <= static_cast<uint32_t>(kSmallProbs) ? sm.probs : a.probs + static_cast<size_t>(b) * V;
        for (uint32_t j = t; j < m; j += NT) P[j] = exp(static_cast<double>(sm.s[sm.list[j]] - mx));
        __syncthreads();
        if (do_topp) {
            // Keys: (score key << 32) | j; j increases with the index, so ties break by index.
            int n = 64;
            while (n < static_cast<int>(m)) n <<= 1;
            uint64_t keys[kSortMax / NT];
#pragma unroll
            for (int q = 0; q < kSortMax / NT; ++q) {
                const int j = t + q * NT;
                keys[q] = j < static_cast<int>(m) ? (static_cast<uint64_t>(float_key(sm.s[sm.list[j]])) << 32) | static_cast<uint32_t>(j)
                                                  : ~0ull;
            }
            __syncthreads();  // s[] is overwritten by the sort buffer below
#pragma unroll
            for (int q = 0; q < kSortMax / NT; ++q) {
                const int j = t + q * NT;
                if (j < n) sm.sortbuf[j] = keys[q];
            }
            __syncthreads();
            bitonic_sort(sm, n);
            if (t == 0) {
                double total = 0.0;
                for (uint32_t j = 0; j < m; ++j) total += P[j];
                if (total <= 0.0) {
                    sm.status = kZeroMass;
                } else {
                    const double threshold = 1.0 - static_cast<double>(top_p);
                    double cumulative = 0.0;
                    for (uint32_t q = 0; q < m; ++q) {
                        const uint32_t j = static_cast<uint32_t>(sm.sortbuf[q]);
                        cumulative += P[j] / total;
                        if (cumulative <= threshold) sm.list[j] |= kRemoved;
                    }
                    const uint32_t keep = min(m, beams > 1 ? 2u : 1u);
                    for (uint32_t q = m - keep; q < m; ++q) sm.list[static_cast<uint32_t>(sm.sortbuf[q])] &= ~kRemoved;
                }
            }
            __syncthreads();
            if (sm.status != kOk) {
                if (t == 0) {
                    a.status[b] = sm.status;
                    if (a.mode == kModeDecode) {
                        st.error = 1;
                        st.active = 0;
                    }
                }
                return;
            }
            if (out_scores) {
                for (uint32_t j = t; j < m; j += NT)
                    if (sm.list[j] & kRemoved) out_scores[sm.list[j] & 0x7fff] = -INFINITY;
                if (t == 0) a.status[b] = kOk;
                return;
            }
        }
        // sample_gpt_token_from_logits (the max of the survivors is still mx: the top entry is kept).
        if (t == 0) {
            double total = 0.0;
            for (uint32_t j = 0; j < m; ++j)
                if (!(sm.list[j] & kRemoved)) total += P[j];
            if (total <= 0.0) {
                sm.status = kZeroMass;
            } else {
                uint64_t rng = st.rng;
                const int draws = a.mode == kModeDraw ? a.draws : 1;
                for (int d = 0; d < draws; ++d) {
                    const double target = splitmix_unit(rng) * total;
                    double cumulative = 0.0;
                    uint32_t last_finite = 0, tok = 0xffffffffu;
                    for (uint32_t j = 0; j < m; ++j) {
                        const uint16_t e = sm.list[j];
                        if (e & kRemoved) continue;
                        const double p = P[j];
                        if (p <= 0.0) continue;
                        last_finite = e;
                        cumulative += p;
                        if (target < cumulative) {
                            tok = e;
                            break;
                        }
                    }
                    if (tok == 0xffffffffu) tok = last_finite;
                    if (a.mode == kModeDraw) a.out_tokens[d] = tok;
                    sm.token = tok;
                }
                st.rng = rng;
            }
        }
        __syncthreads();
        if (sm.status != kOk) {
            if (t == 0) {
                a.status[b] = sm.status;
                if (a.mode == kModeDecode) {
                    st.error = 1;
                    st.active = 0;
                }
            }
            return;
        }
        if (a.mode == kModeDraw) {
            if (t == 0) a.status[b] = kOk;
            return;
        }
    }
    // Decode: accept the token and advance the state (gpt_sampling.cpp:181-186).
    if (t == 0) {
        const uint32_t tok = sm.token;
        a.status[b] = kOk;
        if (tok == static_cast<uint32_t>(kMelStop)) {
            st.stopped = 1;
            st.active = 0;
        } else if (tok >= static_cast<uint32_t>(kMelStart)) {
            a.status[b] = kInvalidCode;
            st.error = 1;
            st.active = 0;
        } else {
            a.codes[static_cast<size_t>(b) * a.code_stride + st.count] = tok;
            st.count += 1;
            a.seen[static_cast<size_t>(b) * V + tok] = 1;
            if (st.count >= st.max_tokens) {
                st.active = 0;
            } else {
                st.token = tok;
                st.position = st.count + 1;  // first generated code sits at mel position 2
                st.n = st.prefix_rows + st.count - 1;
            }
        }
    }
}

}  // namespace

hipError_t launch_sampler(const SampleArgs& a, int batch, hipStream_t s) {
    hipLaunchKernelGGL(sampler_kernel, dim3(batch), dim3(NT), 0, s, a);
    return hipGetLastError();
}

}  // namespace itts

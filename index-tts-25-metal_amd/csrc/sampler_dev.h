// Device-side pieces of the logits processors and sampler, shared by the decode
// sampler (sampler.hip) and the beam-search kernels (beam.hip).  One 1024-thread
// workgroup works on one 8194-entry score row held in LDS.
//
// Restated from the reference (src/gpt_sampling.cpp):
//   run_processors  :28-128  repetition penalty once per distinct history id
//                            (x<0 ? x*p : x/p), /= T, top-k (k-th largest is the pivot,
//                            values below it -> -inf, ties survive), top-p (ascending
//                            (score, index) order, double softmax, drop while the
//                            cumulative <= 1 - p, keep the top 1, or 2 for beams);
//   draw_token      :130-165 p_i = exp(double(s_i - max)), total in index order,
//                            target = u * total, first i with target < cumulative,
//                            else the last positive one;
//   splitmix_*      :11-26   SplitMix64.
// Only ordering-free work runs in parallel (elementwise ops, a radix select for the top-k
// pivot, index-order compaction, a bitonic sort of survivors, the divisions of top-p).  Every floating-point
// sum the reference forms sequentially is formed by one lane in the same order: wave 0
// loads 64 terms at a time into its lanes and lane-serial code reads them back with
// v_readlane, so the chain of adds waits on no LDS round trip.
#pragma once
#include "glibc_math.h"
#include "kernels.h"

namespace itts {
namespace sampling {

constexpr int V = kMelVocab;
constexpr int NT = 1024;
constexpr int NWAVE = NT / 64;
constexpr int IPT = (V + NT - 1) / NT;  // score entries per thread (9): i = t + q * NT, q < IPT
constexpr int kSortMax = 16384;          // next power of two >= V
constexpr int kSmallProbs = 1024;
static_assert(kSortMax / 2 >= kSmallProbs + 8, "running sums past the keys in the sort buffer");
constexpr uint16_t kRemoved = 0x8000;

enum Status : uint32_t {
    kOk = 0,
    kTopPEmpty = 1,    // "GPT top_p filtering removed all logits"
    kZeroMass = 2,     // "GPT sampling probability mass is zero"
    kNoFinite = 3,     // "GPT sampling received no finite logits"
    kInvalidCode = 4,  // "GPT generated invalid semantic code"
};

// LDS of one workgroup of NTT threads working on one score row.  The decode sampler and the
// beam kernels run 1024 threads (Smem); the persistent step kernel's fused sampling tail runs
// its 512.  Every function below taking an SmemT works for either: only order-free parallel
// work depends on the thread count.
template <int NTT>
struct SmemT {
    static constexpr int kWaves = NTT / 64, kIpt = (V + NTT - 1) / NTT;
    // s[] / the sort keys; with at most kSmallProbs survivors the keys leave the upper half
    // free for the draw's and the top-p cut's running sums (16-byte aligned double pairs)
    union alignas(16) {
        float s[V];
        uint64_t sortbuf[kSortMax];
    };
    uint16_t list[V];  // finite survivors in index order; bit 15 = removed by top-p
    uint32_t qoff[kIpt][kWaves];  // compaction: survivors before (q, wave) in index order
    double probs[kSmallProbs];
    uint32_t hist[2][256];  // radix counters, one set per pass parity
    uint32_t wtot[kWaves];
    float wmax[kWaves];
    uint32_t widx[kWaves];
    uint32_t sel[2][2];     // radix choice (digit, count above it), one per pass parity
    uint32_t m;
    uint32_t token;
    uint32_t status;
    float mx;
};
using Smem = SmemT<NT>;

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

// Lane l's value of a wave-uniform lane index l (v_readlane; the halves are widened as
// unsigned so no sign bit leaks into the other half).
__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int l) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), l));
}
__device__ __forceinline__ double readlane_f64(double v, int l) {
    const uint64_t u = static_cast<uint64_t>(__double_as_longlong(v));
    const uint64_t lo = readlane_u32(static_cast<uint32_t>(u), l);
    const uint64_t hi = readlane_u32(static_cast<uint32_t>(u >> 32), l);
    return __longlong_as_double(static_cast<long long>((hi << 32) | lo));
}
// X[0] + X[1] + ... + X[n8 - 1] in index order (double), by the calling lane, with X in
// LDS (16-byte aligned, n8 a multiple of 8); with kWrite, X[j] becomes the running sum
// X[0] + ... + X[j].  Each group of 8 is read while the previous one is added.
template <bool kWrite>
__device__ __forceinline__ double running_sum(double* X, uint32_t n8) {
    double2* x2 = reinterpret_cast<double2*>(X);
    double t = 0.0;
    double2 c[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) c[k] = x2[k];
    for (uint32_t j = 0; j < n8; j += 8) {
        const uint32_t nx = min(j + 8, n8 - 8) >> 1;  // in bounds; unused past the end
        double2 nn[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) nn[k] = x2[nx + k];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            t += c[k].x;
            c[k].x = t;
            t += c[k].y;
            c[k].y = t;
            if (kWrite) x2[(j >> 1) + k] = c[k];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) c[k] = nn[k];
    }
    return t;
}

// Maximum of v over the wave (the xor butterfly of common.h's wave reductions, on integers).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    {
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        v = max(p[0], p[1]);
    }
    {
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        v = max(p[0], p[1]);
    }
    int x = static_cast<int>(v);
    x = static_cast<int>(max(static_cast<uint32_t>(x), static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false))));
    {
        int t = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xF, 0x5, false);  // banks 0, 2: lane + 4
        t = __builtin_amdgcn_update_dpp(t, x, 0x114, 0xF, 0xA, false);      // banks 1, 3: lane - 4
        x = static_cast<int>(max(static_cast<uint32_t>(x), static_cast<uint32_t>(t)));
    }
    x = static_cast<int>(max(static_cast<uint32_t>(x), static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false))));
    x = static_cast<int>(max(static_cast<uint32_t>(x), static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false))));
    return static_cast<uint32_t>(x);
}

// kk-th largest value (1-based) of s[0..V): MSB-first radix select on order-preserving keys,
// 8 bits per pass.  Each thread keeps its keys in registers; the counters and the choice are
// double-buffered by pass parity, so a pass needs two barriers (counts done, choice made):
// the next pass's counters are cleared while this pass counts (the previous pass's scan,
// their last reader, finished before this pass began).
// The first digit (sign and exponent bits) falls in a few bins, where the per-lane counter
// atomics collide.  So the keys' maximum comes first: when at least kk keys share its first
// digit, that digit is the answer's (no key lies in a higher bin) and the first pass is
// skipped; otherwise it runs as the others.
template <int NTT>
__device__ inline float radix_kth_largest(SmemT<NTT>& sm, uint32_t kk) {
    [[maybe_unused]] constexpr int NT = NTT, NWAVE = NTT / 64, IPT = (V + NTT - 1) / NTT;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    uint32_t key[IPT];
    uint32_t kmax = 0;
#pragma unroll
    for (int q = 0; q < IPT; ++q) {
        const int i = t + q * NT;
        key[q] = i < V ? float_key(sm.s[i]) : 0u;
        kmax = max(kmax, key[q]);  // padding keys are 0, below every real key but -NaN's
    }
    kmax = wave_max_u32(kmax);
    if (lane == 0) sm.qoff[0][wave] = kmax;
    if (t < 256) {
        sm.hist[0][t] = 0;
        sm.hist[1][t] = 0;
    }
    __syncthreads();
    kmax = sm.qoff[0][0];
#pragma unroll
    for (int w = 1; w < NWAVE; ++w) kmax = max(kmax, sm.qoff[0][w]);
    const uint32_t top = kmax >> 24;
    uint32_t c = 0;
#pragma unroll
    for (int q = 0; q < IPT; ++q) {
        const int i = t + q * NT;
        c += static_cast<uint32_t>(__popcll(__ballot(i < V && (key[q] >> 24) == top)));
    }
    if (lane == 0) sm.wtot[wave] = c;
    __syncthreads();
    uint32_t same = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) same += sm.wtot[w];
    uint32_t prefix = 0, mask = 0;
    const int first = same >= kk ? 1 : 0;
    if (first) {
        prefix = top << 24;
        mask = 0xffu << 24;
    }
    for (int pass = first; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        uint32_t* h = sm.hist[pass & 1];
#pragma unroll
        for (int q = 0; q < IPT; ++q) {
            const int i = t + q * NT;
            if (i < V && (key[q] & mask) == prefix) atomicAdd(&h[(key[q] >> shift) & 255u], 1u);
        }
        if (pass < 3 && t < 256) sm.hist[(pass + 1) & 1][t] = 0;
        __syncthreads();
        if (t < 64) {
            uint32_t cc[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) cc[q] = h[255 - 4 * lane - q];
            const uint32_t loc = cc[0] + cc[1] + cc[2] + cc[3];
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
                        if (run + cc[q] >= kk) {
                            d = 255 - 4 * lane - q;
                            above = run;
                        } else {
                            run += cc[q];
                        }
                    }
                }
                sm.sel[pass & 1][0] = static_cast<uint32_t>(d);
                sm.sel[pass & 1][1] = above;
            }
        }
        __syncthreads();
        prefix |= sm.sel[pass & 1][0] << shift;
        mask |= 0xffu << shift;
        kk -= sm.sel[pass & 1][1];
    }
    return key_float(prefix);
}

// Compact finite entries of s into sm.list (index order); returns the count, sets sm.m and
// sm.mx.  Entry i = t + q * NT sits at position (q, t) in index order, so a ballot per
// (q, wave) plus one exclusive scan over the IPT x NWAVE counts places every survivor.
template <int NTT>
__device__ inline uint32_t compact_finite(SmemT<NTT>& sm) {
    [[maybe_unused]] constexpr int NT = NTT, NWAVE = NTT / 64, IPT = (V + NTT - 1) / NTT;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    uint64_t bal[IPT];
    float mloc = -INFINITY;
#pragma unroll
    for (int q = 0; q < IPT; ++q) {
        const int i = t + q * NT;
        const float v = i < V ? sm.s[i] : -INFINITY;
        const bool f = i < V && finite_f(v);
        if (f) mloc = fmaxf(mloc, v);
        bal[q] = __ballot(f);
    }
    const float wm = wave_max(mloc);
    if (lane == 0) {
#pragma unroll
        for (int q = 0; q < IPT; ++q) sm.qoff[q][wave] = static_cast<uint32_t>(__popcll(bal[q]));
        sm.wmax[wave] = wm;
    }
    __syncthreads();
    if (wave == 0) {
        // exclusive scan of the counts in (q, wave) order, 64 at a time
        constexpr int kCells = IPT * NWAVE;
        uint32_t* cell = &sm.qoff[0][0];
        uint32_t carry = 0;
        for (int c0 = 0; c0 < kCells; c0 += 64) {
            const int f = c0 + lane;
            const uint32_t cnt = f < kCells ? cell[f] : 0u;
            uint32_t inc = cnt;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t v = __shfl_up(inc, o, 64);
                if (lane >= o) inc += v;
            }
            if (f < kCells) cell[f] = carry + inc - cnt;
            carry += readlane_u32(inc, 63);
        }
        const float mx = wave_max(lane < NWAVE ? sm.wmax[lane] : -INFINITY);
        if (lane == 0) {
            sm.m = carry;
            sm.mx = mx;
        }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < IPT; ++q) {
        if ((bal[q] >> lane) & 1ull) {
            const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal[q] >> 32),
                                                             __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal[q]), 0u));
            sm.list[sm.qoff[q][wave] + below] = static_cast<uint16_t>(t + q * NT);
        }
    }
    __syncthreads();
    return sm.m;
}

// First index of the maximum (std::max_element semantics).
template <int NTT>
__device__ inline uint32_t block_argmax(SmemT<NTT>& sm) {
    [[maybe_unused]] constexpr int NT = NTT, NWAVE = NTT / 64, IPT = (V + NTT - 1) / NTT;
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
template <int NTT>
__device__ inline void bitonic_sort(SmemT<NTT>& sm, int n) {
    [[maybe_unused]] constexpr int NT = NTT, NWAVE = NTT / 64, IPT = (V + NTT - 1) / NTT;
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


// gpt_sampling.cpp:28-128 on sm.s (already holding the input scores).  On return:
//   sm.s holds the processed scores, unless top-p ran with rebuild == false, in which
//   case sm.s is clobbered and the survivors are described by sm.list (index order,
//   kRemoved flags), sm.m, sm.mx and P[0..m) (exp(double(s - mx)) of each survivor).
// *topp_ran tells which.  Returns a Status.
// SEEN_AT_ONCE: the repetition-set bytes are requested together, with no branch around a load
// (under a per-element branch each byte was waited for before the next was requested: one memory
// round trip each).  The separate sampler kernel uses it; the step kernel's fused tail keeps the
// per-element form, because any change to that inlined code changes the step kernel's schedule
// as a whole (a 12% slower step was measured).
template <int NTT, bool SEEN_AT_ONCE = false>
__device__ inline uint32_t run_processors(SmemT<NTT>& sm, const uint8_t* __restrict__ seen, float pen, float T, uint32_t top_k,
                                          float top_p, uint32_t beams, double* P_global, bool rebuild, bool* topp_ran) {
    [[maybe_unused]] constexpr int NT = NTT, NWAVE = NTT / 64, IPT = (V + NTT - 1) / NTT;
    const int t = threadIdx.x;
    *topp_ran = false;
    if (pen != 1.0f || T != 1.0f) {
        if constexpr (SEEN_AT_ONCE) {
            uint32_t hit[IPT];
#pragma unroll
            for (int q = 0; q < IPT; ++q) hit[q] = 0;
            if (pen != 1.0f) {
#pragma unroll
                for (int q = 0; q < IPT; ++q) {
                    const int i = t + q * NT;
                    hit[q] = seen[i < V ? i : 0];  // past the end: entry 0's byte, unused
                }
            }
#pragma unroll
            for (int q = 0; q < IPT; ++q) {
                const int i = t + q * NT;
                if (i < V) {
                    float v = sm.s[i];
                    if (hit[q]) v = v < 0.0f ? v * pen : v / pen;
                    if (T != 1.0f) v = v / T;
                    sm.s[i] = v;
                }
            }
        } else {
            uint8_t hit[IPT];
#pragma unroll
            for (int q = 0; q < IPT; ++q) {
                const int i = t + q * NT;
                hit[q] = pen != 1.0f && i < V ? seen[i] : 0;
            }
#pragma unroll
            for (int q = 0; q < IPT; ++q) {
                const int i = t + q * NT;
                if (i < V) {
                    float v = sm.s[i];
                    if (hit[q]) v = v < 0.0f ? v * pen : v / pen;
                    if (T != 1.0f) v = v / T;
                    sm.s[i] = v;
                }
            }
        }
        __syncthreads();
    }
    if (top_k > 0 && top_k < static_cast<uint32_t>(V)) {
        const uint32_t k = max(top_k, beams > 1 ? 2u : 1u);
        const float pivot = radix_kth_largest(sm, k);
        for (int i = t; i < V; i += NT)
            if (sm.s[i] < pivot) sm.s[i] = -INFINITY;
        __syncthreads();
    }
    if (!(top_p < 1.0f)) return kOk;
    *topp_ran = true;
    const uint32_t m = compact_finite(sm);
    if (m == 0) return kTopPEmpty;
    const float mx = sm.mx;
    double* P = m <= static_cast<uint32_t>(kSmallProbs) ? sm.probs : P_global;
    for (uint32_t j = t; j < m; j += NT) P[j] = libm::exp_glibc(static_cast<double>(sm.s[sm.list[j]] - mx));
    // Keys: (score key << 32) | (j << 1) | negative-zero flag.  j increases with the index, so
    // ties break by index; -0 and +0 share the key of +0, since the reference's comparator
    // (gpt_sampling.cpp:78-83) finds them equal, and the flag (below j, so it never decides
    // the order) brings back the sign when the scores are rebuilt.
    int n = 64;
    while (n < static_cast<int>(m)) n <<= 1;
    uint64_t keys[kSortMax / NT];
#pragma unroll
    for (int q = 0; q < kSortMax / NT; ++q) {
        const int j = t + q * NT;
        if (j < static_cast<int>(m)) {
            const float v = sm.s[sm.list[j]];
            const uint32_t nz = __float_as_uint(v) == 0x80000000u ? 1u : 0u;
            keys[q] = (static_cast<uint64_t>(float_key(nz ? 0.0f : v)) << 32) | (static_cast<uint32_t>(j) << 1) | nz;
        } else {
            keys[q] = ~0ull;
        }
    }
    __syncthreads();  // s[] is overwritten by the sort buffer below
#pragma unroll
    for (int q = 0; q < kSortMax / NT; ++q) {
        const int j = t + q * NT;
        if (j < n) sm.sortbuf[j] = keys[q];
    }
    __syncthreads();
    bitonic_sort(sm, n);
    if (t < 64 && m <= static_cast<uint32_t>(kSmallProbs)) {
        // total in index order, then the cumulative mass in ascending (score, index) order.
        // Both sums run on lane 0 over values staged in LDS (the sort buffer's upper half:
        // the keys take at most kSmallProbs entries here); the divisions P[j] / total and the
        // threshold tests run on all lanes.
        const int lane = t;
        double* R = reinterpret_cast<double*>(sm.sortbuf) + kSortMax / 2;
        const uint32_t m8 = (m + 7u) & ~7u;
        for (uint32_t j = lane; j < m8; j += 64) R[j] = j < m ? P[j] : 0.0;
        double total = lane == 0 ? running_sum<false>(R, m8) : 0.0;
        total = __shfl(total, 0, 64);
        if (total <= 0.0) {
            if (lane == 0) sm.status = kZeroMass;
        } else {
            if (lane == 0) sm.status = kOk;
            const double threshold = 1.0 - static_cast<double>(top_p);
            for (uint32_t q = lane; q < m8; q += 64) R[q] = q < m ? P[static_cast<uint32_t>(sm.sortbuf[q]) >> 1] / total : 0.0;
            if (lane == 0) (void)running_sum<true>(R, m8);
            for (uint32_t q = lane; q < m; q += 64)
                if (R[q] <= threshold) sm.list[static_cast<uint32_t>(sm.sortbuf[q]) >> 1] |= kRemoved;
            const uint32_t keep = min(m, beams > 1 ? 2u : 1u);
            if (static_cast<uint32_t>(lane) < keep) {
                const uint32_t q = m - keep + lane;
                sm.list[static_cast<uint32_t>(sm.sortbuf[q]) >> 1] &= ~kRemoved;
            }
        }
    } else if (t < 64) {
        // more survivors (weights in global memory): the same sums, lane-serially
        const int lane = t;
        double total = 0.0;
        for (uint32_t c0 = 0; c0 < m; c0 += 64) {
            const double p = c0 + lane < m ? P[c0 + lane] : 0.0;
            const int cn = static_cast<int>(min(64u, m - c0));
            for (int q = 0; q < cn; ++q) total += readlane_f64(p, q);
        }
        if (total <= 0.0) {
            if (lane == 0) sm.status = kZeroMass;
        } else {
            if (lane == 0) sm.status = kOk;
            const double threshold = 1.0 - static_cast<double>(top_p);
            double cumulative = 0.0;
            for (uint32_t c0 = 0; c0 < m; c0 += 64) {
                const uint32_t q = c0 + lane;
                const uint32_t j = q < m ? static_cast<uint32_t>(sm.sortbuf[q]) >> 1 : 0u;
                const double r = q < m ? P[j] / total : 0.0;
                const int cn = static_cast<int>(min(64u, m - c0));
                uint64_t removed = 0;
                for (int qq = 0; qq < cn; ++qq) {
                    cumulative += readlane_f64(r, qq);
                    if (cumulative <= threshold) removed |= 1ull << qq;
                }
                if (q < m && ((removed >> lane) & 1ull)) sm.list[j] |= kRemoved;
            }
            const uint32_t keep = min(m, beams > 1 ? 2u : 1u);
            if (static_cast<uint32_t>(lane) < keep) {
                const uint32_t q = m - keep + lane;
                sm.list[static_cast<uint32_t>(sm.sortbuf[q]) >> 1] &= ~kRemoved;
            }
        }
    }
    __syncthreads();
    const uint32_t st = sm.status;
    if (st != kOk || !rebuild) return st;
    // Rebuild s[] from the sorted keys (the key carries the score).
#pragma unroll
    for (int q = 0; q < kSortMax / NT; ++q) {
        const int j = t + q * NT;
        keys[q] = j < n ? sm.sortbuf[j] : ~0ull;
    }
    __syncthreads();
    for (int i = t; i < V; i += NT) sm.s[i] = -INFINITY;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kSortMax / NT; ++q) {
        const uint64_t k = keys[q];
        if (k == ~0ull) continue;
        const uint32_t j = static_cast<uint32_t>(k) >> 1;
        const uint16_t e = sm.list[j];
        if (!(e & kRemoved)) sm.s[e & 0x7fff] = (k & 1u) ? -0.0f : key_float(static_cast<uint32_t>(k >> 32));
    }
    __syncthreads();
    return kOk;
}

// gpt_sampling.cpp:130-165 over the survivors sm.list[0..m) with weights P, run by the 64
// lanes of one wave (every lane returns the same token): the total over the survivors in
// index order, target = u * total, then the first survivor whose cumulative mass exceeds
// the target, else the last one with positive mass.  Both sums run lane-serially in index
// order.  Returns the token, or 0xffffffff with *status set when the mass is zero.
template <int NTT>
__device__ inline uint32_t draw_token_wave(const SmemT<NTT>& sm, uint32_t m, const double* P, uint64_t& rng, uint32_t* status) {
    const int lane = threadIdx.x & 63;
    double total = 0.0;
    for (uint32_t c0 = 0; c0 < m; c0 += 64) {
        const bool in = c0 + lane < m;
        const double p = in && !(sm.list[c0 + lane] & kRemoved) ? P[c0 + lane] : 0.0;
        const uint32_t live = static_cast<uint32_t>(in && !(sm.list[c0 + lane] & kRemoved));
        const int cn = static_cast<int>(min(64u, m - c0));
        for (int q = 0; q < cn; ++q)
            if (readlane_u32(live, q)) total += readlane_f64(p, q);
    }
    if (total <= 0.0) {
        *status = kZeroMass;
        return 0xffffffffu;
    }
    const double target = splitmix_unit(rng) * total;
    double cumulative = 0.0;
    uint32_t last_finite = 0;
    for (uint32_t c0 = 0; c0 < m; c0 += 64) {
        const bool in = c0 + lane < m;
        const uint32_t e = in ? sm.list[c0 + lane] : static_cast<uint32_t>(kRemoved);
        const double p = in ? P[c0 + lane] : 0.0;
        const int cn = static_cast<int>(min(64u, m - c0));
        for (int q = 0; q < cn; ++q) {
            const uint32_t eq = readlane_u32(e, q);
            if (eq & kRemoved) continue;
            const double pq = readlane_f64(p, q);
            if (pq <= 0.0) continue;
            last_finite = eq;
            cumulative += pq;
            if (target < cumulative) return eq;
        }
    }
    return last_finite;
}

// draw_token_wave for up to kSmallProbs survivors (weights P in LDS), `draws` times from the
// same weights: lane 0 forms the running sums of the live weights in index order once, in
// LDS (the sort buffer's upper half, free once the processors are done); the walk's running
// value at survivor j is that sum (it adds the same values in the same order, zeros aside),
// so each draw's pick, the first live survivor with target < its running sum (else the last
// live one), takes one ballot per 64 survivors.  Writes the tokens through emit(d, token);
// returns kOk or kZeroMass.
template <int NTT, class Emit>
__device__ inline uint32_t draw_tokens_lds(SmemT<NTT>& sm, uint32_t m, const double* P, uint64_t& rng, int draws, Emit emit) {
    const int lane = threadIdx.x & 63;
    double* W = reinterpret_cast<double*>(sm.sortbuf) + kSortMax / 2;
    const uint32_t m8 = (m + 7u) & ~7u;
    for (uint32_t j = lane; j < m8; j += 64) W[j] = j < m && !(sm.list[j] & kRemoved) ? P[j] : 0.0;
    double total = lane == 0 ? running_sum<true>(W, m8) : 0.0;
    total = __shfl(total, 0, 64);
    if (total <= 0.0) return kZeroMass;
    for (int d = 0; d < draws; ++d) {
        const double target = splitmix_unit(rng) * total;
        uint32_t pick = 0xffffffffu, last = 0xffffffffu;
        for (uint32_t c0 = 0; c0 < m; c0 += 64) {
            const uint32_t j = c0 + lane;
            const bool live = j < m && !(sm.list[j] & kRemoved) && P[j] > 0.0;
            const uint64_t hit = __ballot(live && target < W[j]);
            const uint64_t any = __ballot(live);
            if (hit) {
                pick = c0 + static_cast<uint32_t>(__builtin_ctzll(hit));
                break;
            }
            if (any) last = c0 + 63u - static_cast<uint32_t>(__builtin_clzll(any));
        }
        if (pick == 0xffffffffu) pick = last;
        emit(d, static_cast<uint32_t>(sm.list[pick] & 0x7fff));
    }
    return kOk;
}

// One sequence's sampler pass (the body of sampler_kernel, and the fused tail of the persistent
// step kernel): the processors and the draw on row b of the logits, then, in decode mode, the
// token accepted and the state advanced (gpt_sampling.cpp:168-189 per step).  Every thread of
// the workgroup calls it.
// STANDALONE: the sampler kernel's own launch.  Its loads are ordered for a kernel that runs by
// itself: the repetition set's bytes are requested at once (run_processors' SEEN_AT_ONCE), the
// logits before the state's active flag is tested, and the state entry is read once into
// registers (st below).  The step kernel's fused tail keeps the plain form, which its own
// schedule was measured with: there, the same source changes made the whole step 12% slower.
template <int NTT, bool STANDALONE = false>
__device__ inline void sample_loaded(SmemT<NTT>& sm, const SampleArgs& a, int b, const SeqState& st);
template <int NTT, bool STANDALONE = false>
__device__ inline void sample_loaded(SmemT<NTT>& sm, const SampleArgs& a, int b) {
    sample_loaded<NTT, STANDALONE>(sm, a, b, a.state[b]);
}

template <int NTT, bool STANDALONE = false>
__device__ inline void sample_sequence(SmemT<NTT>& sm, const SampleArgs& a, int b) {
    [[maybe_unused]] constexpr int NT = NTT, IPT = (V + NTT - 1) / NTT;
    const int t = threadIdx.x;
    const float* lg = a.logits + static_cast<size_t>(b) * a.logit_stride;
    if constexpr (STANDALONE) {
        // The logits requested first, then the whole state entry (one request, so no later field
        // read waits behind a store that might alias it); the flag tested only then.  Testing it
        // first made the logits wait for its round trip.
        float v[IPT];
#pragma unroll
        for (int q = 0; q < IPT; ++q) {
            const int i = t + q * NT;
            v[q] = i < V ? lg[i] : 0.0f;
        }
        const SeqState st = a.state[b];
        if (a.mode == kModeDecode && !st.active) return;
#pragma unroll
        for (int q = 0; q < IPT; ++q) {
            const int i = t + q * NT;
            if (i < V) sm.s[i] = v[q];
        }
        __syncthreads();
        sample_loaded<NTT, true>(sm, a, b, st);
    } else {
        const SeqState& st = a.state[b];
        if (a.mode == kModeDecode && !st.active) return;
        float v[IPT];  // all loads in flight before the first store
#pragma unroll
        for (int q = 0; q < IPT; ++q) {
            const int i = t + q * NT;
            v[q] = i < V ? lg[i] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < IPT; ++q) {
            const int i = t + q * NT;
            if (i < V) sm.s[i] = v[q];
        }
        __syncthreads();
        sample_loaded<NTT, false>(sm, a, b);
    }
}

// sample_sequence after the scores are in sm.s (every thread calls it; decode mode expects an
// active state).  st: the state entry as read (the entry itself, or the standalone sampler's
// copy in registers); every write goes to the entry, sw.
template <int NTT, bool STANDALONE>
__device__ inline void sample_loaded(SmemT<NTT>& sm, const SampleArgs& a, int b, const SeqState& st) {
    [[maybe_unused]] constexpr int NT = NTT, IPT = (V + NTT - 1) / NTT;
    const int t = threadIdx.x;
    SeqState& sw = a.state[b];
    const bool processors = a.mode != kModeDraw;
    const bool need_sample = a.mode == kModeDraw || (a.mode == kModeDecode && st.do_sample);
    if (processors && st.suppress_stop) {  // raw logits 8192 and 8193 dropped before any processor
        if (t == 0) {
            sm.s[kMelStart] = -INFINITY;
            sm.s[kMelStop] = -INFINITY;
        }
        __syncthreads();
    }
    double* Pg = a.probs + static_cast<size_t>(b) * V;
    uint32_t status = kOk;
    bool topp = false;
    if (processors)
        status = run_processors<NTT, STANDALONE>(sm, a.seen + static_cast<size_t>(b) * V, st.penalty, st.temperature, st.top_k, st.top_p,
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
                if (m <= static_cast<uint32_t>(kSmallProbs)) {
                    status = draw_tokens_lds(sm, m, P, rng, draws, [&](int d, uint32_t tk) {
                        token = tk;
                        if (a.mode == kModeDraw && t == 0) a.out_tokens[d] = tk;
                    });
                } else {
                    for (int d = 0; d < draws && status == kOk; ++d) {
                        token = draw_token_wave(sm, m, P, rng, &status);
                        if (a.mode == kModeDraw && t == 0) a.out_tokens[d] = token;
                    }
                }
                if (t == 0) sw.rng = rng;
            }
        }
    }
    if (t != 0) return;
    if constexpr (STANDALONE) {
        // Accept the token and advance the state (gpt_sampling.cpp:181-186), from the fields
        // read at the start: read after the stores below, each waited for the store before it.
        a.status[b] = status;
        if (a.mode != kModeDecode) return;
        if (status != kOk) {
            sw.error = 1;
            sw.active = 0;
            return;
        }
        if (token == static_cast<uint32_t>(kMelStop)) {
            sw.stopped = 1;
            sw.active = 0;
        } else if (token >= static_cast<uint32_t>(kMelStart)) {
            a.status[b] = kInvalidCode;
            sw.error = 1;
            sw.active = 0;
        } else {
            const uint32_t count = st.count + 1;
            a.codes[static_cast<size_t>(b) * a.code_stride + st.count] = token;
            sw.count = count;
            a.seen[static_cast<size_t>(b) * V + token] = 1;
            if (count >= st.max_tokens) {
                sw.active = 0;
            } else {
                sw.token = token;
                sw.position = count + 1;  // the first generated code sits at mel position 2
                sw.n = st.prefix_rows + count - 1;
            }
        }
        return;
    }
    a.status[b] = status;
    if (a.mode != kModeDecode) return;
    if (status != kOk) {
        sw.error = 1;
        sw.active = 0;
        return;
    }
    // Accept the token and advance the state (gpt_sampling.cpp:181-186).
    if (token == static_cast<uint32_t>(kMelStop)) {
        sw.stopped = 1;
        sw.active = 0;
    } else if (token >= static_cast<uint32_t>(kMelStart)) {
        a.status[b] = kInvalidCode;
        sw.error = 1;
        sw.active = 0;
    } else {
        a.codes[static_cast<size_t>(b) * a.code_stride + sw.count] = token;
        sw.count += 1;
        a.seen[static_cast<size_t>(b) * V + token] = 1;
        if (sw.count >= sw.max_tokens) {
            sw.active = 0;
        } else {
            sw.token = token;
            sw.position = sw.count + 1;  // the first generated code sits at mel position 2
            sw.n = sw.prefix_rows + sw.count - 1;
        }
    }
}

}  // namespace sampling
}  // namespace itts

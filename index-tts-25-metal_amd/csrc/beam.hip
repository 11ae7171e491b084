// Beam-search scoring and candidate selection (src/gpt_sampling.cpp:190-245) on the device.
//
// beam_scores_kernel, one 1024-thread workgroup per parent beam:
//   log_probs = logits - (peak + log(sum_i exp(logit_i - peak)))   (:207-210, float; the
//   sum is the reference's index-order float chain bit for bit, formed by one wave
//   (chain_sum.h); expf/logf bit for bit those of glibc (glibc_math.h)), then the processors with the
//   parent's repetition set (:211-212), then + the parent's beam score (:213).
// beam_select_kernel, one workgroup:
//   greedy: the take = 2*beams best of all parents' scores by (score desc, index asc)
//   (std::partial_sort with index ties, :223-227); sampled: take draws without
//   replacement with sample_gpt_token_from_logits (:217-222), by wave 0 alone with the
//   finite candidates in LDS when there are at most kLdsCands of them (each draw's sums
//   lane-serial in index order); then a stable sort of the candidates by score (:228).
// beam_advance_kernel picks the children on the device (the next forward is queued without
// waiting for the host) and reorders their row owners and repetition sets; the host reads
// the candidates (written into pinned memory by beam_select_kernel) a step or two later and
// runs the reference's child/finish bookkeeping.
#include "chain_sum.h"
#include "sampler_dev.h"

namespace itts {
namespace {
using namespace sampling;


__global__ __launch_bounds__(NT) void beam_scores_kernel(BeamArgs a) {
    __shared__ Smem sm;
    __shared__ float wred[NWAVE];
    __shared__ float log_sum_s;
    const int p = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const float* lg = a.logits + static_cast<size_t>(p) * V;  // rows < parents: in bounds
    uint32_t hits;
    float* e = reinterpret_cast<float*>(sm.sortbuf) + V + 2;  // after s[] inside the union, 16-byte aligned
    static_assert(V + 2 + chain::kPad <= kSortMax * 2, "the padded exponentials fit in the sort buffer");
    float mloc = -INFINITY;
    {
        float v[IPT];  // all loads in flight before the first store
#pragma unroll
        for (int q = 0; q < IPT; ++q) {
            const int i = t + q * NT;
            v[q] = i < V ? lg[i] : -INFINITY;
        }
        // the parent's repetition set, behind the logits: the log-softmax hides its round trip
        hits = 0;
        if (a.penalty != 1.0f) {
            uint8_t hit[IPT];
#pragma unroll
            for (int q = 0; q < IPT; ++q) {
                const int i = t + q * NT;
                hit[q] = i < V ? a.seen[static_cast<size_t>(p) * V + i] : 0;
            }
#pragma unroll
            for (int q = 0; q < IPT; ++q) hits |= hit[q] ? 1u << q : 0u;
        }
        // this step's parent count, read behind the loads above
        if (a.parents_dev && p >= static_cast<int>(*a.parents_dev)) {  // the whole workgroup leaves together
            if (t == 0) a.status[1 + p] = kOk;
            return;
        }
#pragma unroll
        for (int q = 0; q < IPT; ++q) {
            const int i = t + q * NT;
            if (i < V) {
                const float x = a.suppress_stop && (i == kMelStart || i == kMelStop) ? -INFINITY : v[q];
                sm.s[i] = x;
                mloc = fmaxf(mloc, x);
            }
        }
    }
    mloc = wave_max(mloc);
    if (lane == 0) wred[wave] = mloc;
    __syncthreads();
    float peak = wred[0];
    for (int w = 1; w < NWAVE; ++w) peak = fmaxf(peak, wred[w]);
    for (int i = t; i < V; i += NT) e[i] = libm::expf_glibc(sm.s[i] - peak);
    for (int i = V + t; i < chain::kPad; i += NT) e[i] = 0.0f;  // adding +0 leaves the sum unchanged
    __syncthreads();
    if (wave == 0) {
        const float sum = chain::sum_wave(e, lane);
        if (lane == 0) log_sum_s = peak + libm::logf_glibc(sum);
    }
    __syncthreads();
    const float log_sum = log_sum_s;
    for (int i = t; i < V; i += NT) sm.s[i] = sm.s[i] - log_sum;
    __syncthreads();
    // The repetition penalty (gpt_sampling.cpp:33-49) here, from the bits read at the start;
    // run_processors then goes on with the temperature (the same operations in the same order).
    if (a.penalty != 1.0f) {
#pragma unroll
        for (int q = 0; q < IPT; ++q) {
            const int i = t + q * NT;
            if (i < V && ((hits >> q) & 1u)) {
                const float v = sm.s[i];
                sm.s[i] = v < 0.0f ? v * a.penalty : v / a.penalty;
            }
        }  // each thread's own entries, which run_processors reads in the same thread
    }
    bool topp = false;
    const uint32_t st = run_processors(sm, a.seen + static_cast<size_t>(p) * V, 1.0f, a.temperature, a.top_k, a.top_p,
                                       a.num_beams, a.probs + static_cast<size_t>(p) * V, true, &topp);
    if (t == 0) a.status[1 + p] = st;
    if (st != kOk) return;
    const float score = a.beam_score[p];
    float* out = a.all_scores + static_cast<size_t>(p) * V;
    for (int i = t; i < V; i += NT) out[i] = sm.s[i] + score;
}

// Calls f(i, src[i]) for i = first, first + step, ... < end, in that order, with the loads of
// eight consecutive visits in flight together: a loop that waits for each global load before
// the next pays one memory round trip per element.
template <class F>
__device__ __forceinline__ void for_each_batched(const float* src, int first, int end, int step, F f) {
    for (int base = first; base < end; base += 8 * step) {
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = base + u * step;
            x[u] = i < end ? src[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = base + u * step;
            if (i < end) f(i, x[u]);
        }
    }
}

// kk-th largest (1-based) of src[0..n) in global memory.
__device__ float radix_kth_largest_global(const float* src, int n, uint32_t kk, uint32_t* hist, uint32_t* sel) {
    const int t = threadIdx.x, lane = t & 63;
    uint32_t prefix = 0, mask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (t < 256) hist[t] = 0;
        __syncthreads();
        for_each_batched(src, t, n, NT, [&](int, float v) {
            const uint32_t k = float_key(v);
            if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
        });
        __syncthreads();
        if (t < 64) {
            uint32_t c[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) c[q] = hist[255 - 4 * lane - q];
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
                for (int q = 0; q < 4; ++q)
                    if (d < 0) {
                        if (run + c[q] >= kk) {
                            d = 255 - 4 * lane - q;
                            above = run;
                        } else {
                            run += c[q];
                        }
                    }
                sel[0] = static_cast<uint32_t>(d);
                sel[1] = above;
            }
        }
        __syncthreads();
        prefix |= sel[0] << shift;
        mask |= 0xffu << shift;
        kk -= sel[1];
        __syncthreads();
    }
    return key_float(prefix);
}

// Block-wide exclusive scan of one count per thread; returns the thread's offset, *total the sum.
__device__ uint32_t block_scan(uint32_t c, uint32_t* wtot, uint32_t* total) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    uint32_t inc = c;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(inc, o, 64);
        if (lane >= o) inc += v;
    }
    if (lane == 63) wtot[wave] = inc;
    __syncthreads();
    uint32_t off = 0, tot = 0;
    for (int w = 0; w < NWAVE; ++w) {
        if (w < wave) off += wtot[w];
        tot += wtot[w];
    }
    __syncthreads();
    *total = tot;
    return off + inc - c;
}

// Sampled candidate selection for sampled beams when at most kLdsCands scores are
// finite, by wave 0 with the candidates in LDS: take draws without replacement, each
// (gpt_sampling.cpp:130-165 on the remaining candidates) with its maximum, its total and
// its cumulative scan in index order.
// - Weights: w[j] = exp(double(score_j - max)), 0 for drawn candidates, in pw.  They are
//   recomputed only when the maximum changes (the same values otherwise); pw is padded
//   with zeros to a multiple of 8.
// - Total: lane 0 adds w[0], w[1], ... in index order (the reference's total) and keeps
//   each partial sum in pre[j].  The reference's cumulative walk skips zero weights and
//   adds the others in the same order, so its running value at candidate j is pre[j] too:
//   the pick, the first j with w[j] > 0 and target < pre[j] (else the last j with
//   w[j] > 0), is found with one ballot per 64 candidates instead of a second serial pass.
// Returns kOk or the failing status; ids[0..take) on success.
constexpr int kLdsCands = 2048;
__device__ uint32_t draw_candidates_wave(uint32_t* lid, const float* lsc, double* pw, double* pre, uint32_t F, int take, uint64_t& rng,
                                         uint32_t* ids, float* idsc) {
    const int lane = threadIdx.x & 63;
    constexpr uint32_t kTaken = 0x80000000u;
    constexpr uint32_t kNone = 0xffffffffu;
    const uint32_t F8 = (F + 7u) & ~7u;
    float mprev = NAN;
    for (int d = 0; d < take; ++d) {
        float m = -INFINITY;  // max over the still-available entries
        for (uint32_t j = lane; j < F; j += 64)
            if (!(lid[j] & kTaken)) m = fmaxf(m, lsc[j]);
        m = wave_max(m);
        if (m == -INFINITY) return kNoFinite;
        if (!(m == mprev)) {
            for (uint32_t j = lane; j < F8; j += 64)
                pw[j] = j < F && !(lid[j] & kTaken) ? libm::exp_glibc(static_cast<double>(lsc[j] - m)) : 0.0;
            mprev = m;
        }
        double total = 0.0;
        if (lane == 0) {
            // w[j] in index order; each chunk of 8 is read while the previous one is added
            const double2* w2 = reinterpret_cast<const double2*>(pw);
            double2* p2 = reinterpret_cast<double2*>(pre);
            double2 c[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) c[k] = w2[k];
            for (uint32_t j = 0; j < F8; j += 8) {
                const uint32_t nx = min(j + 8, F8 - 8) >> 1;  // in bounds; unused past the end
                double2 n[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) n[k] = w2[nx + k];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    double2 r;
                    total += c[k].x;
                    r.x = total;
                    total += c[k].y;
                    r.y = total;
                    p2[(j >> 1) + k] = r;
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) c[k] = n[k];
            }
        }
        total = __shfl(total, 0, 64);
        if (total <= 0.0) return kZeroMass;
        const double target = splitmix_unit(rng) * total;
        uint32_t pick = kNone, last = kNone;
        for (uint32_t c0 = 0; c0 < F; c0 += 64) {
            const uint32_t j = c0 + lane;
            const bool live = j < F && pw[j] > 0.0;
            const uint64_t hit = __ballot(live && target < pre[j]);
            const uint64_t any = __ballot(live);
            if (hit) {
                pick = c0 + static_cast<uint32_t>(__builtin_ctzll(hit));
                break;
            }
            if (any) last = c0 + 63u - static_cast<uint32_t>(__builtin_clzll(any));
        }
        if (pick == kNone) pick = last;
        if (lane == 0) {
            ids[d] = lid[pick];
            idsc[d] = lsc[pick];
            lid[pick] |= kTaken;
            pw[pick] = 0.0;
        }
    }
    return kOk;
}

// The finite scores of S[0..parents * V) in index order: ids into lid and scores into lsc
// when there are at most kLdsCands of them, else ids into list; returns their count.
// Wave w reads rows [w * RW, w * RW + RW) of 64 scores, lane l column l, so every load is one
// coalesced 256-byte row, and all RW loads are in flight together.  A ballot per row and an
// exclusive sum of the 16 waves' counts place every entry.
template <int P>
__device__ uint32_t finite_in_order(const float* S, uint32_t* wtot, uint32_t* lid, float* lsc, uint32_t* list) {
    constexpr int n = P * V;
    constexpr int RW = ((n + 63) / 64 + NWAVE - 1) / NWAVE;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    float v[RW];
#pragma unroll
    for (int k = 0; k < RW; ++k) v[k] = S[min((wave * RW + k) * 64 + lane, n - 1)];
    uint64_t bal[RW];
    uint32_t c = 0;
#pragma unroll
    for (int k = 0; k < RW; ++k) {
        bal[k] = __ballot((wave * RW + k) * 64 + lane < n && finite_f(v[k]));
        c += static_cast<uint32_t>(__builtin_popcountll(bal[k]));
    }
    if (lane == 0) wtot[wave] = c;
    __syncthreads();
    uint32_t off = 0, F = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
        const uint32_t x = wtot[w];
        off += w < wave ? x : 0u;
        F += x;
    }
    const bool to_lds = F <= static_cast<uint32_t>(kLdsCands);
#pragma unroll
    for (int k = 0; k < RW; ++k) {
        const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal[k] >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal[k]), 0u));
        if ((bal[k] >> lane) & 1u) {
            const uint32_t pos = off + below;
            const uint32_t i = static_cast<uint32_t>((wave * RW + k) * 64 + lane);
            if (to_lds) {
                lid[pos] = i;
                lsc[pos] = v[k];
            } else {
                list[pos] = i;
            }
        }
        off += static_cast<uint32_t>(__builtin_popcountll(bal[k]));
    }
    __syncthreads();
    return F;
}

// Stable sort of (ids, scores)[0..n) by score, descending (insertion sort, one thread): the
// reference is built with libc++, whose std::sort keeps equal candidates in order below 24
// elements (n <= 20).  The scores are the chosen ids' own, held in LDS beside them.
__device__ __forceinline__ void stable_sort_desc(uint32_t* ids, float* sc, int n) {
    for (int x = 1; x < n; ++x) {
        const uint32_t v = ids[x];
        const float sv = sc[x];
        int y = x - 1;
        while (y >= 0 && sc[y] < sv) {
            ids[y + 1] = ids[y];
            sc[y + 1] = sc[y];
            --y;
        }
        ids[y + 1] = v;
        sc[y + 1] = sv;
    }
}

__device__ __forceinline__ void select_candidates(const BeamArgs& a) {
    __shared__ uint32_t hist[256], sel[2], wtot[NWAVE];
    __shared__ uint32_t lid[kLdsCands];
    __shared__ float lsc[kLdsCands];
    __shared__ __align__(16) double pw[kLdsCands], pre[kLdsCands];
    __shared__ uint32_t ids[2 * kMaxBeamTake];
    __shared__ float idsc[2 * kMaxBeamTake];  // the score of each chosen id (sorted with it)
    __shared__ float wmax[NWAVE];
    __shared__ float mx_s;
    __shared__ uint32_t stop_s;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int n = (a.parents_dev ? static_cast<int>(*a.parents_dev) : a.parents) * V;
    const float* S = a.all_scores;
    const int take = a.take;
    const int chunk = (n + NT - 1) / NT;
    const int i0 = min(n, t * chunk), i1 = min(n, i0 + chunk);
    if (!a.do_sample) {
        const float pivot = radix_kth_largest_global(S, n, static_cast<uint32_t>(take), hist, sel);
        uint32_t cg = 0, ce = 0;
        for_each_batched(S, i0, i1, 1, [&](int, float v) {
            cg += v > pivot;
            ce += v == pivot;
        });
        uint32_t ng = 0, ne = 0;
        uint32_t og = block_scan(cg, wtot, &ng);
        uint32_t oe = block_scan(ce, wtot, &ne);
        const uint32_t need = static_cast<uint32_t>(take) - ng;  // ties at the pivot, smallest indices first
        for_each_batched(S, i0, i1, 1, [&](int i, float v) {
            if (v > pivot) ids[og++] = static_cast<uint32_t>(i);
            else if (v == pivot) {
                if (oe < need) ids[ng + oe] = static_cast<uint32_t>(i);
                ++oe;
            }
        });
        __syncthreads();
        if (t < take) idsc[t] = S[ids[t]];  // one parallel read; the sort compares in LDS
        __syncthreads();
        if (t == 0) {
            // (score desc, index asc): the order std::partial_sort produces with index ties.
            for (int x = 1; x < take; ++x) {
                const uint32_t v = ids[x];
                const float sv = idsc[x];
                int y = x - 1;
                while (y >= 0 && (idsc[y] < sv || (idsc[y] == sv && ids[y] > v))) {
                    ids[y + 1] = ids[y];
                    idsc[y + 1] = idsc[y];
                    --y;
                }
                ids[y + 1] = v;
                idsc[y + 1] = sv;
            }
            a.status[0] = kOk;
        }
    } else {
        // Finite entries in index order: in LDS (lid, lsc) when there are at most kLdsCands,
        // else in global scratch (a.list) with the weights in a.probs.
        uint32_t F = 0;
        switch (n / V) {
            case 1: F = finite_in_order<1>(S, wtot, lid, lsc, a.list); break;
            case 2: F = finite_in_order<2>(S, wtot, lid, lsc, a.list); break;
            case 3: F = finite_in_order<3>(S, wtot, lid, lsc, a.list); break;
            case 4: F = finite_in_order<4>(S, wtot, lid, lsc, a.list); break;
            default: {
                uint32_t c = 0;
                for_each_batched(S, i0, i1, 1, [&](int, float v) { c += finite_f(v); });
                uint32_t off = block_scan(c, wtot, &F);
                const bool to_lds = F <= static_cast<uint32_t>(kLdsCands);
                for_each_batched(S, i0, i1, 1, [&](int i, float v) {
                    if (finite_f(v)) {
                        if (to_lds) {
                            lid[off] = static_cast<uint32_t>(i);
                            lsc[off] = v;
                        } else {
                            a.list[off] = static_cast<uint32_t>(i);
                        }
                        ++off;
                    }
                });
                __syncthreads();
            }
        }
        if (F <= static_cast<uint32_t>(kLdsCands)) {
            if (wave != 0) return;
            uint64_t rng = *a.rng;
            const uint32_t st = draw_candidates_wave(lid, lsc, pw, pre, F, take, rng, ids, idsc);
            if (st != kOk) {
                if (t == 0) a.status[0] = st;
                return;
            }
            if (t == 0) {
                *a.rng = rng;
                stable_sort_desc(ids, idsc, take);
                a.status[0] = kOk;
            }
            if (t < take) {
                const uint32_t id = ids[t];
                a.cand[t] = BeamCand{id / static_cast<uint32_t>(V), id % static_cast<uint32_t>(V), idsc[t], 0u};
            }
            return;
        }
        if (t == 0) stop_s = 0;
        uint64_t rng = *a.rng;
        for (int d = 0; d < take; ++d) {
            float m = -INFINITY;  // max over the still-available finite entries
            for (uint32_t j = t; j < F; j += NT) {
                const uint32_t id = a.list[j];
                if (!(id & 0x80000000u)) m = fmaxf(m, S[id]);
            }
            m = wave_max(m);
            if (lane == 0) wmax[wave] = m;
            __syncthreads();
            if (t == 0) {
                float g = wmax[0];
                for (int w = 1; w < NWAVE; ++w) g = fmaxf(g, wmax[w]);
                mx_s = g;
            }
            __syncthreads();
            const float mx = mx_s;
            if (mx == -INFINITY) {
                if (t == 0) a.status[0] = kNoFinite;
                return;
            }
            for (uint32_t j = t; j < F; j += NT) {
                const uint32_t id = a.list[j];
                a.probs[j] = (id & 0x80000000u) ? 0.0 : libm::exp_glibc(static_cast<double>(S[id] - mx));
            }
            __syncthreads();
            if (t == 0) {
                double total = 0.0;
                for (uint32_t j = 0; j < F; ++j) total += a.probs[j];
                if (total <= 0.0) {
                    stop_s = kZeroMass;
                } else {
                    const double target = splitmix_unit(rng) * total;
                    double cumulative = 0.0;
                    uint32_t pick = 0xffffffffu, last = 0xffffffffu;
                    for (uint32_t j = 0; j < F; ++j) {
                        const double p = a.probs[j];
                        if (p <= 0.0) continue;
                        last = j;
                        cumulative += p;
                        if (target < cumulative) {
                            pick = j;
                            break;
                        }
                    }
                    if (pick == 0xffffffffu) pick = last;
                    ids[d] = a.list[pick];
                    a.list[pick] |= 0x80000000u;
                }
            }
            __syncthreads();
            if (stop_s) {
                if (t == 0) a.status[0] = stop_s;
                return;
            }
        }
        if (t < take) idsc[t] = S[ids[t]];
        __syncthreads();
        if (t == 0) {
            *a.rng = rng;
            stable_sort_desc(ids, idsc, take);
            a.status[0] = kOk;
        }
    }
    if (t < take) {
        const uint32_t id = ids[t];
        a.cand[t] = BeamCand{id / static_cast<uint32_t>(V), id % static_cast<uint32_t>(V), idsc[t], 0u};
    }
}

// The selection, then (when a.host_cand is set) its candidates and every status of the step
// copied into pinned host memory, so the host needs no copy launches to read them.  Every
// thread returns from select_candidates before the barrier.
__global__ __launch_bounds__(NT) void beam_select_kernel(BeamArgs a) {
    select_candidates(a);
    if (!a.host_cand) return;
    __syncthreads();
    const int t = threadIdx.x;
    if (t < a.take) a.host_cand[t] = a.cand[t];
    if (t <= a.parents) a.host_status[t] = a.status[t];
}

// dst[0..bytes) = src[0..bytes) by the workgroup, 16 bytes per thread and step (both
// buffers 16-byte aligned, not overlapping).
__device__ __forceinline__ void copy_block(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, uint32_t bytes) {
    const uint32_t n16 = bytes / 16;
    const uint4* s16 = reinterpret_cast<const uint4*>(src);
    uint4* d16 = reinterpret_cast<uint4*>(dst);
    for (uint32_t i = threadIdx.x; i < n16; i += NT) d16[i] = s16[i];
    for (uint32_t i = n16 * 16 + threadIdx.x; i < bytes; i += NT) dst[i] = src[i];
}

// Children (thread 0; at most 2 * 10 candidates and 10 children), then the reorder by the
// whole workgroup: the first `beams` repetition sets and table rows (each a contiguous block)
// are staged, then each child's written from its parent's.  A repetition set (8194 bytes,
// rows 2-byte aligned) is copied in 2-byte pieces, the child's token set in its piece.
__global__ __launch_bounds__(NT) void beam_advance_kernel(BeamAdvanceArgs a) {
    __shared__ uint32_t par_s[kMaxBatch], tok_s[kMaxBatch];
    const int t = threadIdx.x;
    const int beams = a.beams;
    if (t == 0) {
        const uint32_t P = *a.parents_dev;
        int C = 0;
        for (int r = 0; r < a.take && C < beams; ++r) {
            const BeamCand c = a.cand[r];
            if (c.token == static_cast<uint32_t>(kMelStop)) continue;
            if (c.token >= static_cast<uint32_t>(kMelStart) || c.parent >= P) {
                C = 0;
                break;
            }
            par_s[C] = c.parent;
            tok_s[C] = c.token;
            a.score[C] = c.score;
            ++C;
        }
        for (int c = 0; c < beams; ++c) {
            SeqState st = *a.tmpl;
            st.n = a.n;
            st.position = a.position;
            if (c < C) {
                st.token = tok_s[c];
            } else {
                par_s[c] = 0;
                tok_s[c] = 0;
                a.score[c] = -INFINITY;
                st.token = 0;
                st.active = 0;
            }
            a.parent[c] = par_s[c];
            a.token[c] = tok_s[c];
            a.state[c] = st;
        }
        *a.parents_dev = C > 0 ? static_cast<uint32_t>(C) : 1u;
    }
    const uint32_t n = a.n, cap = a.cap;
    copy_block(a.seen_tmp, a.seen, static_cast<uint32_t>(beams) * V);
    copy_block(a.table_tmp, a.table, static_cast<uint32_t>(beams) * cap);
    __syncthreads();  // the staged rows, par_s and tok_s are seen by the whole workgroup
    static_assert(V % 2 == 0, "repetition sets in 2-byte pieces");
    constexpr uint32_t kHalf = V / 2;
    for (int c = 0; c < beams; ++c) {
        const uint32_t p = par_s[c], tk = tok_s[c];
        const uint16_t* __restrict__ src = reinterpret_cast<const uint16_t*>(a.seen_tmp + static_cast<size_t>(p) * V);
        uint16_t* __restrict__ dst = reinterpret_cast<uint16_t*>(a.seen + static_cast<size_t>(c) * V);
        uint16_t v[(kHalf + NT - 1) / NT];
#pragma unroll
        for (int u = 0; u < (kHalf + NT - 1) / NT; ++u) {
            const uint32_t j = t + u * NT;
            v[u] = j < kHalf ? src[j] : 0;
        }
#pragma unroll
        for (int u = 0; u < (kHalf + NT - 1) / NT; ++u) {
            const uint32_t j = t + u * NT;
            if (j < kHalf) {
                uint16_t x = v[u];
                if (j == tk >> 1) x = (tk & 1u) ? static_cast<uint16_t>((x & 0x00ffu) | 0x0100u) : static_cast<uint16_t>((x & 0xff00u) | 0x0001u);
                dst[j] = x;
            }
        }
        const uint8_t* __restrict__ ts = a.table_tmp + static_cast<size_t>(p) * cap;
        uint8_t* __restrict__ td = a.table + static_cast<size_t>(c) * cap;
        for (uint32_t r = t; r <= n; r += NT) td[r] = r == n ? static_cast<uint8_t>(c) : ts[r];
    }
}

}  // namespace

hipError_t launch_beam_advance(const BeamAdvanceArgs& a, hipStream_t s) {
    if (a.take < 1 || a.take > kMaxBeamTake || a.beams < 1 || a.beams > kMaxBatch || a.n + 1 > a.cap) return hipErrorInvalidValue;
    hipLaunchKernelGGL(beam_advance_kernel, dim3(1), dim3(NT), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_beam_scores(const BeamArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(beam_scores_kernel, dim3(a.parents), dim3(NT), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_beam_select(const BeamArgs& a, hipStream_t s) {
    if (a.take < 1 || a.take > kMaxBeamTake) return hipErrorInvalidValue;
    hipLaunchKernelGGL(beam_select_kernel, dim3(1), dim3(NT), 0, s, a);
    return hipGetLastError();
}

}  // namespace itts

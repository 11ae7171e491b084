// The float sum of 8194 values in index order, bit for bit, by one wave: the log-softmax
// denominator of the beam scores (gpt_sampling.cpp:208).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace itts {
namespace chain {

// ((e[0] + e[1]) + e[2]) + ... + e[8193] in float, bit for bit the reference's index-order
// chain (gpt_sampling.cpp:208), for e[j] >= 0 (+inf and NaN included), formed by one wave
// without 8194 dependent float adds.
// Once the running sum is NaN the chain stays NaN; once it is +inf it stays +inf unless a
// later value is NaN.  Both are decided at the top of the loop, before the binade
// arithmetic (which needs a finite sum).
// While the running sum s stays in one binade [2^k, 2^(k+1)) (k >= -126; below 2^-125 the
// spacing is the subnormal one, so s = 0 counts as k = -126), every representable value
// there is a multiple of u = 2^(k-23), s = M u with M < 2^24 an integer, and float addition
// is s + e -> u * round(M + e/u) (round to nearest, ties to even) as long as the exact
// sum stays below 2^(k+1).  So for 64 consecutive e (one per lane), with q = e/u rounded to
// nearest, not a tie (fraction exactly 1/2) and M + sum(q) <= 2^24 - 1, every one of the 64
// additions is exact in that form: their result is (M + sum(q)) u, with sum(q) an exact
// integer sum.  Chunks that fail the test (a tie, or the sum reaching the next binade) are
// added one value at a time in float, as the reference does.  The q of eight chunks are
// formed and summed together; after a chunk added one at a time ends in another binade, the
// following chunks' q are formed again for the new u.
// e (LDS) must hold zeros from index 8194 up to kPad = 64 * (kChunks + kGroup).
constexpr int kChunks = (kMelVocab + 63) / 64;
constexpr int kGroup = 8;
constexpr int kPad = 64 * (kChunks + kGroup);
__device__ __forceinline__ int binade(float s) {
    const uint32_t ex = (__float_as_uint(s) >> 23) & 0xffu;
    return ex == 0 ? -126 : static_cast<int>(ex) - 127;
}
// Integer wave sums of a, b, c, d with VALU lane exchanges (the butterfly of common.h's
// wave_sum4): lanes 0-15 end with sum(a), 16-31 sum(c), 32-47 sum(b), 48-63 sum(d).
__device__ __forceinline__ uint32_t xsum32_u(uint32_t a, uint32_t b) {
    const auto p = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    return p[0] + p[1];
}
__device__ __forceinline__ uint32_t xsum16_u(uint32_t a, uint32_t b) {
    const auto p = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    return p[0] + p[1];
}
__device__ __forceinline__ uint32_t row16_sum_u(uint32_t v) {
    int x = static_cast<int>(v);
    x += __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false);  // lane ^ 8 (row_ror:8)
    {
        int t = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xF, 0x5, false);  // banks 0, 2: lane + 4
        t = __builtin_amdgcn_update_dpp(t, x, 0x114, 0xF, 0xA, false);      // banks 1, 3: lane - 4
        x += t;
    }
    x += __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);  // lane ^ 2
    x += __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);  // lane ^ 1
    return static_cast<uint32_t>(x);
}
__device__ __forceinline__ void wave_sum4_u(uint32_t& a, uint32_t& b, uint32_t& c, uint32_t& d) {
    const uint32_t v = row16_sum_u(xsum16_u(xsum32_u(a, b), xsum32_u(c, d)));
    a = __builtin_amdgcn_readlane(v, 0);
    c = __builtin_amdgcn_readlane(v, 16);
    b = __builtin_amdgcn_readlane(v, 32);
    d = __builtin_amdgcn_readlane(v, 48);
}
__device__ inline float sum_wave(const float* __restrict__ e, int lane) {
    float s = 0.0f;
    int c = 0;
    while (c < kChunks) {
        if (!(s <= 3.40282347e38f)) {  // NaN or +inf (the sum is never negative)
            if (s != s) return s;
            bool nan = false;
            for (int j = 64 * c + lane; j < kMelVocab; j += 64) nan |= e[j] != e[j];
            return __ballot(nan) ? __builtin_nanf("") : s;
        }
        const int k = binade(s);
        const int sh = 23 - k;                                    // e / u = e * 2^sh
        uint32_t M = static_cast<uint32_t>(ldexpf(s, sh));        // s / u, an integer < 2^24
        uint32_t Q[kGroup];
        uint64_t bad = 0;
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
            const float t = ldexpf(e[64 * (c + g) + lane], sh);  // exact, or inf (then big)
            const bool big = !(t < 16777216.0f);                 // also NaN
            const float fl = floorf(t), fr = t - fl;             // exact below 2^24
            const bool tie = fr == 0.5f;
            Q[g] = big ? (1u << 25) : static_cast<uint32_t>(fl) + (fr > 0.5f ? 1u : 0u);
            if (__ballot(big || tie)) bad |= 1ull << g;
        }
        wave_sum4_u(Q[0], Q[1], Q[2], Q[3]);
        wave_sum4_u(Q[4], Q[5], Q[6], Q[7]);
        bool rescaled = false;
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
            if (rescaled || c + g >= kChunks) continue;
            if (!((bad >> g) & 1u) && M + Q[g] <= 16777215u) {
                M += Q[g];
                continue;
            }
            // one value at a time from s = M u (exact), as the reference adds them
            float ss = ldexpf(static_cast<float>(M), -sh);
            const float4* e4 = reinterpret_cast<const float4*>(e + 64 * (c + g));
            float4 x[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] = e4[i];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                ss += x[i].x;
                ss += x[i].y;
                ss += x[i].z;
                ss += x[i].w;
            }
            if (binade(ss) != k) {
                s = ss;
                c += g + 1;
                rescaled = true;
            } else {
                M = static_cast<uint32_t>(ldexpf(ss, sh));
            }
        }
        if (!rescaled) {
            s = ldexpf(static_cast<float>(M), -sh);
            c += kGroup;
        }
    }
    return s;
}

}  // namespace chain
}  // namespace itts

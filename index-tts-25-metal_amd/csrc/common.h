// Shared constants, device helpers and launch-argument structs for the CDNA4
// (gfx950) kernels of the GPT semantic-token loop.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

namespace itts {

// GPT shape (src/gpt.cpp:7): width 1280, 20 heads x 64, FFN 5120.
constexpr int kWidth = 1280;
constexpr int kHeads = 20;
constexpr int kHeadDim = 64;
constexpr int kFfn = 5120;
constexpr int kQkv = 3 * kWidth;
constexpr int kMelVocab = 8194;
constexpr int kMelStart = 8192;
constexpr int kMelStop = 8193;
constexpr int kMaxBatch = 10;
constexpr float kLnEps = 1e-5f;
// Per-layer small parameters, packed: ln1 w/b, qkv bias, proj bias, ln2 w/b, fc bias, fc2 bias.
constexpr int kParLn1W = 0;
constexpr int kParLn1B = kParLn1W + kWidth;
constexpr int kParQkvB = kParLn1B + kWidth;
constexpr int kParProjB = kParQkvB + kQkv;
constexpr int kParLn2W = kParProjB + kWidth;
constexpr int kParLn2B = kParLn2W + kWidth;
constexpr int kParFcB = kParLn2B + kWidth;
constexpr int kParFc2B = kParFcB + kFfn;
constexpr int kParLayer = kParFc2B + kWidth;  // 16640 floats
// Head parameters: ln_f w/b, final_norm w/b, mel_head bias.
constexpr int kHeadLnfW = 0;
constexpr int kHeadLnfB = kWidth;
constexpr int kHeadFnW = 2 * kWidth;
constexpr int kHeadFnB = 3 * kWidth;
constexpr int kHeadBias = 4 * kWidth;
constexpr int kHeadPar = kHeadBias + kMelVocab;

// Per-sequence decode state, device resident.  The forward reads token/position/n;
// the sampler advances them, so a captured step graph replays with no host input.
struct SeqState {
    uint32_t n;           // KV rows valid before this forward; the new row goes to row n
    uint32_t position;    // mel position of the input code
    uint32_t token;       // input code of this forward
    uint32_t active;      // 1 while the sequence decodes
    uint32_t count;       // codes accepted so far
    uint32_t max_tokens;  // generation length limit
    uint32_t prefix_rows; // P
    uint32_t stopped;     // sampled 8193
    uint32_t error;       // sampled a code >= 8192 other than 8193
    uint32_t do_sample;
    uint32_t top_k;
    uint32_t num_beams;
    float temperature;
    float top_p;
    float penalty;
    uint32_t suppress_stop;
    uint64_t rng;         // SplitMix64 state (gpt_sampling.cpp:11-26)
    uint32_t _pad[2];
};
static_assert(sizeof(SeqState) == 80, "SeqState layout");

__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float(static_cast<uint32_t>(v) << 16); }

// Weight element loads: fp32 rows stream as float4; bf16 rows as 4 x bf16 (8 bytes).
template <typename WT>
struct WLoad;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <>
struct WLoad<float> {
    using vec = f32x4;
    __device__ __forceinline__ static f32x4 load(const float* p, size_t idx4) {
        return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p) + idx4);
    }
    __device__ __forceinline__ static float4 to_f4(f32x4 v) { return make_float4(v.x, v.y, v.z, v.w); }
};
template <>
struct WLoad<uint16_t> {
    using vec = u32x2;
    __device__ __forceinline__ static u32x2 load(const uint16_t* p, size_t idx4) {
        return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p) + idx4);
    }
    __device__ __forceinline__ static float4 to_f4(u32x2 v) {
        return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                           __uint_as_float(v.y & 0xffff0000u));
    }
};

// Wave reductions: the xor butterfly over distances 32, 16, 8, 4, 2, 1 (each lane combines
// its value with lane ^ d's), so every lane ends with the same result.  The exchanges run
// on the VALU instead of the LDS crossbar (ds_bpermute): distance 32 and 16 with gfx950's
// v_permlane32_swap / v_permlane16_swap, 8 with DPP row_ror:8, 4 with two bank-masked DPP
// row shifts, 2 and 1 with DPP quad permutes.
//
// permlane*_swap(a, b) returns {a with its upper half (32) / odd rows (16) replaced by b's
// lower half / even rows, b with its lower half / even rows replaced by a's upper half /
// odd rows}; the element-wise sum of the two is the distance-32 (16) pair sum of a in the
// lower half (even rows) and of b in the upper half (odd rows).  Passing a == b gives one
// butterfly step; passing two different values reduces two rows at once.
__device__ __forceinline__ float xsum32(float a, float b) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float xsum16(float a, float b) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float xmax32(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xmax16(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
// value of lane ^ 8, ^ 4, ^ 2, ^ 1
__device__ __forceinline__ float lane_x8(float v) { return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false)); }
__device__ __forceinline__ float lane_x4(float v) {
    int t = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x104, 0xF, 0x5, false);  // banks 0, 2: lane + 4
    t = __builtin_amdgcn_update_dpp(t, __float_as_int(v), 0x114, 0xF, 0xA, false);                    // banks 1, 3: lane - 4
    return __int_as_float(t);
}
__device__ __forceinline__ float lane_x2(float v) { return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)); }
__device__ __forceinline__ float lane_x1(float v) { return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)); }
// distances 8, 4, 2, 1 (within 16-lane rows)
__device__ __forceinline__ float row16_sum(float v) {
    v += lane_x8(v);
    v += lane_x4(v);
    v += lane_x2(v);
    v += lane_x1(v);
    return v;
}
// distances 1, 2, 4, 8: the sum over each aligned group of 16 lanes (attention's q.k)
__device__ __forceinline__ float sum16_up(float v) {
    v += lane_x1(v);
    v += lane_x2(v);
    v += lane_x4(v);
    v += lane_x8(v);
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    const float u = xsum32(v, v);
    return row16_sum(xsum16(u, u));
}
// Two rows at once, each with wave_sum's pairings: lanes 0-31 end with sum(a), 32-63 with sum(b).
__device__ __forceinline__ float wave_sum2(float a, float b) {
    const float v = xsum32(a, b);
    return row16_sum(xsum16(v, v));
}
// Four rows at once: lanes 0-15 end with sum(a), 16-31 sum(c), 32-47 sum(b), 48-63 sum(d).
__device__ __forceinline__ float wave_sum4(float a, float b, float c, float d) { return row16_sum(xsum16(xsum32(a, b), xsum32(c, d))); }
__device__ __forceinline__ float wave_max(float v) {
    v = xmax16(xmax32(v));
    v = fmaxf(v, lane_x8(v));
    v = fmaxf(v, lane_x4(v));
    v = fmaxf(v, lane_x2(v));
    return fmaxf(v, lane_x1(v));
}

// Order-preserving map float -> uint32 (larger float -> larger key).
__device__ __forceinline__ uint32_t float_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// tanh-GELU with the +-10 clamp of kernels.metal:486-503.
__device__ __forceinline__ float gelu_f(float v) {
    const float c = 0.7978845608028654f;
    if (v > 10.0f) return v;
    if (v < -10.0f) return 0.0f;
    return 0.5f * v * (1.0f + tanhf(c * (v + 0.044715f * v * v * v)));
}

// LayerNorm over one 1280-wide row per sequence, values distributed 5 per thread
// (index tid + 256 i).  Fixed-order reduction: wave butterfly, then 4 wave partials.
template <int B, int PER>
__device__ __forceinline__ void ln_block(float (&v)[B][PER], const float* __restrict__ g, const float* __restrict__ be,
                                         float* red) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float mean[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < PER; ++i) s += v[b][i];
        s = wave_sum(s);
        if (lane == 0) red[b * 4 + wave] = s;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < B; ++b)
        mean[b] = (((red[b * 4 + 0] + red[b * 4 + 1]) + red[b * 4 + 2]) + red[b * 4 + 3]) / float(kWidth);
    __syncthreads();
#pragma unroll
    for (int b = 0; b < B; ++b) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const float d = v[b][i] - mean[b];
            s += d * d;
        }
        s = wave_sum(s);
        if (lane == 0) red[b * 4 + wave] = s;
    }
    __syncthreads();
#pragma unroll
    for (int b = 0; b < B; ++b) {
        const float var = (((red[b * 4 + 0] + red[b * 4 + 1]) + red[b * 4 + 2]) + red[b * 4 + 3]) / float(kWidth);
        const float inv = 1.0f / sqrtf(var + kLnEps);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int c = tid + 256 * i;
            v[b][i] = (v[b][i] - mean[b]) * inv * g[c] + be[c];
        }
    }
    __syncthreads();
}

__device__ __forceinline__ float lane_value(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

// A 1280-wide row in LDS, as the 256 threads of ln_block<1, 5> (common.h) hold it:
// v[w][i] = row[64 w + lane + 256 i], i.e. thread 64 w + lane's five values.
__device__ __forceinline__ void ln_layout_load(const float* row, int lane, float (&v)[4][5]) {
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int i = 0; i < 5; ++i) v[w][i] = row[64 * w + lane + 256 * i];
}

// Mean and 1 / sqrt(var + eps) of that row in ln_block<1, 5>'s order (each thread sums its
// five values, each wave reduces its threads by butterfly, the four wave sums are added in
// order), computed by one wave for all four: wave_sum4 reduces the four waves' values with
// wave_sum's pairings, so every compute wave gets the statistics without a barrier.
__device__ __forceinline__ void ln_stats(const float (&v)[4][5], float& mean, float& inv) {
    float s[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        s[w] = 0.0f;
#pragma unroll
        for (int i = 0; i < 5; ++i) s[w] += v[w][i];
    }
    float r = wave_sum4(s[0], s[1], s[2], s[3]);  // waves 0, 1, 2, 3 in lanes 0, 32, 16, 48
    mean = (((lane_value(r, 0) + lane_value(r, 32)) + lane_value(r, 16)) + lane_value(r, 48)) / float(kWidth);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        s[w] = 0.0f;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const float d = v[w][i] - mean;
            s[w] += d * d;
        }
    }
    r = wave_sum4(s[0], s[1], s[2], s[3]);
    const float var = (((lane_value(r, 0) + lane_value(r, 32)) + lane_value(r, 16)) + lane_value(r, 48)) / float(kWidth);
    inv = 1.0f / sqrtf(var + kLnEps);
}
// ln_block's per-element step
__device__ __forceinline__ float ln_apply(float v, float mean, float inv, float g, float b) { return (v - mean) * inv * g + b; }


}  // namespace itts

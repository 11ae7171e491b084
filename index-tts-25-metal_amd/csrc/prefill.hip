// Prefill kernels (the P-row prefix forward of gpt.cpp:88-125 with initial=true).
//
// * ln_rows: LayerNorm of each 1280-wide row (kernels.metal:618-669), one workgroup per row.
// * gemm: C[M][N] = A[M][K] * W[N][K]^T + bias on the FP32 matrix cores
//   (v_mfma_f32_32x32x2f32), replacing the broadcast-bias + MPS GEMM pair of
//   metal_context.mm:368-410.  64x64 tile per 256-thread workgroup, 2x2 waves of
//   32x32, K staged through LDS 16 at a time with the next slab prefetched into
//   registers.  Epilogues: q rows + K/V cache store (kernels.metal:1250-1266),
//   residual add in place, GELU.  When the tiles alone would leave most CUs idle (a
//   155-row prefix has 60 tiles of a 1280-wide output), K is split over gridDim.z:
//   each split writes its partial tile to a workspace and gemm_reduce adds the splits
//   in order, then the bias and the epilogue.
// * causal_attention: one wave per (query row, head); 64 keys per pass, lane = key for
//   the scores, lane = dimension for the weighted V sum, online max/sum rescaling
//   (same recurrence as mit2_gpt_causal_attention_sgq_f32, kernels.metal:2249-2292).
// Rows of several sequences may be stacked (ragged batch prefill): row m belongs to
// cache slot row_slot[m] at position row_pos[m] and attends to that slot's rows
// 0..row_pos[m].
#include "kernels.h"

namespace itts {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void ln_rows_kernel(LnRowsArgs a) {
    __shared__ float red[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    float v[1][5];
#pragma unroll
    for (int i = 0; i < 5; ++i) v[0][i] = a.x[static_cast<size_t>(row) * kWidth + tid + 256 * i];
    ln_block<1, 5>(v, a.w, a.b, red);
#pragma unroll
    for (int i = 0; i < 5; ++i) a.y[static_cast<size_t>(row) * kWidth + tid + 256 * i] = v[0][i];
}

constexpr int BM = 64, BN = 64, BK = 16, LDP = 4;

// Output element (row, col) of the GEMM, v = dot + bias: the epilogue.
template <int EPI>
__device__ __forceinline__ void gemm_store(const GemmArgs& a, int row, int col, float v) {
    if constexpr (EPI == kGemmQkv) {
        if (col < kWidth) {
            a.c[static_cast<size_t>(row) * kWidth + col] = v;
        } else {
            const int rr = col - kWidth;
            const bool is_v = rr >= kWidth;
            const int c = is_v ? rr - kWidth : rr;
            const size_t off = static_cast<size_t>(a.row_slot[row]) * a.kv_slot_stride + a.kv_layer_off + (is_v ? a.kv_v_off : 0) +
                               (static_cast<size_t>(c >> 6) * a.kv_cap + a.row_pos[row]) * kHeadDim + (c & 63);
            a.kv[off] = v;
        }
    } else if constexpr (EPI == kGemmResid) {
        float* p = a.c + static_cast<size_t>(row) * a.N + col;
        *p = *p + v;
    } else if constexpr (EPI == kGemmStore) {
        a.c[static_cast<size_t>(row) * a.N + col] = v;
    } else {
        a.c[static_cast<size_t>(row) * a.N + col] = gelu_f(v);
    }
}

// SiLU-gated product of one (gate, up) column pair (kernels.metal:363-374).
__device__ __forceinline__ float swiglu_f(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// SPLIT: this workgroup covers K range [z Kz, (z + 1) Kz) of split z = blockIdx.z and
// writes its raw partial tile to a.ws[z][M][N]; gemm_reduce_kernel finishes it.
template <typename WT, int EPI, bool SPLIT>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs a) {
    __shared__ float As[BK][BM + LDP];
    __shared__ float Bs[BK][BN + LDP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int lrow = tid >> 2, lk = (tid & 3) * 4;  // loader: one 4-wide K chunk of one row
    const int am = m0 + lrow;
    const bool arow_ok = am < a.M;
    const int kz = SPLIT ? a.K / a.splits : a.K;  // this split's K extent, a multiple of BK
    const int kbase = SPLIT ? static_cast<int>(blockIdx.z) * kz : 0;
    const float* arow = a.a + static_cast<size_t>(arow_ok ? am : 0) * a.K + kbase + lk;
    const WT* wrow = static_cast<const WT*>(a.w) + static_cast<size_t>(n0 + lrow) * a.K + kbase + lk;

    auto load_a = [&](int k0) -> float4 {
        return arow_ok ? *reinterpret_cast<const float4*>(arow + k0) : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    auto load_b = [&](int k0) -> float4 {
        if constexpr (sizeof(WT) == 4) {
            return *reinterpret_cast<const float4*>(wrow + k0);
        } else {
            const uint2 v = *reinterpret_cast<const uint2*>(wrow + k0);
            return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                               __uint_as_float(v.y & 0xffff0000u));
        }
    };

    floatx16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    float4 ra = load_a(0), rb = load_b(0);
    for (int k0 = 0; k0 < kz; k0 += BK) {
        As[lk + 0][lrow] = ra.x;
        As[lk + 1][lrow] = ra.y;
        As[lk + 2][lrow] = ra.z;
        As[lk + 3][lrow] = ra.w;
        Bs[lk + 0][lrow] = rb.x;
        Bs[lk + 1][lrow] = rb.y;
        Bs[lk + 2][lrow] = rb.z;
        Bs[lk + 3][lrow] = rb.w;
        __syncthreads();
        if (k0 + BK < kz) {
            ra = load_a(k0 + BK);
            rb = load_b(k0 + BK);
        }
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            const float av = As[kk + (lane >> 5)][wm * 32 + (lane & 31)];
            const float bv = Bs[kk + (lane >> 5)][wn * 32 + (lane & 31)];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
        }
        __syncthreads();
    }

    // D layout of v_mfma_f32_32x32x2f32: lane l, element i -> row 8(i/4) + 4(l/32) + i%4, col l%32.
    const int col = n0 + wn * 32 + (lane & 31);
    if constexpr (SPLIT) {
        float* ws = a.ws + static_cast<size_t>(blockIdx.z) * a.M * a.N;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = m0 + wm * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
            if (row < a.M) ws[static_cast<size_t>(row) * a.N + col] = acc[i];
        }
    } else if constexpr (EPI == kGemmSwiglu) {
        // columns col and col ^ 1 sit in lanes l and l ^ 1, on the same rows
        const float bias = a.bias[col];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = m0 + wm * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
            const float v = acc[i] + bias;
            const float u = __shfl_xor(v, 1, 64);
            if (row < a.M && !(col & 1)) a.c[static_cast<size_t>(row) * (a.N / 2) + col / 2] = swiglu_f(v, u);
        }
    } else {
        const float bias = a.bias[col];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = m0 + wm * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
            if (row < a.M) gemm_store<EPI>(a, row, col, acc[i] + bias);
        }
    }
}

// Finishes a split-K GEMM: dot = partial 0 + partial 1 + ... in split order, then + bias and
// the epilogue; one thread per output element.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmArgs a) {
    const size_t total = static_cast<size_t>(a.M) * a.N, plane = total;
    if constexpr (EPI == kGemmSwiglu) {  // one thread per (gate, up) column pair
        for (size_t e2 = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; e2 < total / 2;
             e2 += static_cast<size_t>(gridDim.x) * blockDim.x) {
            const size_t e = 2 * e2;
            float g = a.ws[e], u = a.ws[e + 1];
            for (int z = 1; z < a.splits; ++z) {
                g += a.ws[z * plane + e];
                u += a.ws[z * plane + e + 1];
            }
            const int col = static_cast<int>(e % a.N);
            a.c[e2] = swiglu_f(g + a.bias[col], u + a.bias[col + 1]);
        }
        return;
    }
    for (size_t e = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total; e += static_cast<size_t>(gridDim.x) * blockDim.x) {
        float d = a.ws[e];
        for (int z = 1; z < a.splits; ++z) d += a.ws[z * plane + e];
        const int row = static_cast<int>(e / a.N), col = static_cast<int>(e % a.N);
        gemm_store<EPI>(a, row, col, d + a.bias[col]);
    }
}

__device__ __forceinline__ float lane_value_f(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

__global__ __launch_bounds__(64) void causal_attention_kernel(CausalArgs a) {
    const int m = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    __shared__ float qs[kHeadDim];
    qs[lane] = a.q[static_cast<size_t>(m) * kWidth + h * kHeadDim + lane];
    __syncthreads();
    const uint32_t slot = a.row_slot[m];
    const int pos = static_cast<int>(a.row_pos[m]);
    const float* kb = a.kv + static_cast<size_t>(slot) * a.kv_slot_stride + a.kv_layer_off + static_cast<size_t>(h) * a.kv_cap * kHeadDim;
    const float* vb = kb + a.kv_v_off;
    float mrun = -INFINITY, lrun = 0.0f, acc = 0.0f;
    for (int c0 = 0; c0 <= pos; c0 += 64) {
        const int key = c0 + lane;
        const bool valid = key <= pos;
        float s = -INFINITY;
        if (valid) {
            const float4* kr = reinterpret_cast<const float4*>(kb + static_cast<size_t>(key) * kHeadDim);
            float d = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float4 k4 = kr[j];
                d = __builtin_fmaf(qs[4 * j + 0], k4.x, d);
                d = __builtin_fmaf(qs[4 * j + 1], k4.y, d);
                d = __builtin_fmaf(qs[4 * j + 2], k4.z, d);
                d = __builtin_fmaf(qs[4 * j + 3], k4.w, d);
            }
            s = d * 0.125f;
        }
        const float cm = wave_max(s);
        const float mnew = fmaxf(mrun, cm);
        const float corr = mrun == -INFINITY ? 0.0f : expf(mrun - mnew);
        const float p = valid ? expf(s - mnew) : 0.0f;
        lrun = lrun * corr + wave_sum(p);
        acc *= corr;
        // acc += p_k V[k] for the chunk's keys in order; 16 V rows in flight at a time, p_k read
        // from lane k (a wave-uniform lane index)
        const int nk = min(64, pos + 1 - c0);
        for (int k0 = 0; k0 < nk; k0 += 16) {
            float vv[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) vv[j] = k0 + j < nk ? vb[static_cast<size_t>(c0 + k0 + j) * kHeadDim + lane] : 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (k0 + j < nk) acc = __builtin_fmaf(lane_value_f(p, k0 + j), vv[j], acc);
        }
        mrun = mnew;
    }
    a.out[static_cast<size_t>(m) * kWidth + h * kHeadDim + lane] = acc / lrun;
}

}  // namespace

hipError_t launch_ln_rows(const LnRowsArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(ln_rows_kernel, dim3(a.rows), dim3(256), 0, s, a);
    return hipGetLastError();
}

int gemm_splits(int M, int N, int K) {
    const int tiles = (N / BN) * ((M + BM - 1) / BM);
    int s = std::min(kGemmMaxSplits, std::max(1, kGemmTargetTiles / std::max(1, tiles)));
    while (s > 1 && (K % (s * BK) != 0)) --s;
    return s;
}

hipError_t launch_gemm(const GemmArgs& a, int epi, bool bf16, hipStream_t s) {
    if (a.N % BN || a.K % BK || a.splits < 1 || a.K % (a.splits * BK) || (a.splits > 1 && !a.ws)) return hipErrorInvalidValue;
    const bool split = a.splits > 1;
    const dim3 grid(a.N / BN, (a.M + BM - 1) / BM, a.splits);
    const int rblocks = static_cast<int>(std::min<size_t>((static_cast<size_t>(a.M) * a.N + 255) / 256, 2048));
#define ITTS_GEMM(WT, E)                                                                       \
    do {                                                                                       \
        if (split) {                                                                           \
            hipLaunchKernelGGL((gemm_kernel<WT, E, true>), grid, dim3(256), 0, s, a);          \
            hipLaunchKernelGGL((gemm_reduce_kernel<E>), dim3(rblocks), dim3(256), 0, s, a);    \
        } else {                                                                               \
            hipLaunchKernelGGL((gemm_kernel<WT, E, false>), grid, dim3(256), 0, s, a);         \
        }                                                                                      \
    } while (0)
    if (epi == kGemmStore || epi == kGemmSwiglu) {  // FP32 weights only (the Qwen decoder)
        if (bf16) return hipErrorInvalidValue;
        if (epi == kGemmStore) ITTS_GEMM(float, kGemmStore);
        else ITTS_GEMM(float, kGemmSwiglu);
    } else if (bf16) {
        if (epi == kGemmQkv) ITTS_GEMM(uint16_t, kGemmQkv);
        else if (epi == kGemmResid) ITTS_GEMM(uint16_t, kGemmResid);
        else ITTS_GEMM(uint16_t, kGemmGelu);
    } else {
        if (epi == kGemmQkv) ITTS_GEMM(float, kGemmQkv);
        else if (epi == kGemmResid) ITTS_GEMM(float, kGemmResid);
        else ITTS_GEMM(float, kGemmGelu);
    }
#undef ITTS_GEMM
    return hipGetLastError();
}

hipError_t launch_causal_attention(const CausalArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(causal_attention_kernel, dim3(a.M, kHeads), dim3(64), 0, s, a);
    return hipGetLastError();
}

}  // namespace itts

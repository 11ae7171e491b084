// Prefill kernels (the P-row prefix forward of gpt.cpp:88-125 with initial=true).
//
// * ln_rows: LayerNorm of each 1280-wide row (kernels.metal:618-669), one workgroup per row.
// * gemm: C[M][N] = A[M][K] * W[N][K]^T + bias on the FP32 matrix cores
//   (v_mfma_f32_16x16x4f32), replacing the broadcast-bias + MPS GEMM pair of
//   metal_context.mm:368-410.  A workgroup covers up to 192 rows x 64 columns: the A rows
//   go through LDS (double-buffered, 32 k per stage), each wave's 16 weight rows straight
//   into registers one stage pair ahead.  Epilogues: q rows + K/V cache store
//   (kernels.metal:1250-1266), residual add in place, GELU, plain store, SiLU-gated pairs.
//   When the tiles alone would leave CUs idle (a 155-row prefix has 20 tiles of a
//   1280-wide output), K is split over gridDim.z: each split writes its partial tile to a
//   workspace and gemm_reduce adds the splits in order, then the bias and the epilogue.
// * causal_attention: one 8-wave workgroup per (16 query rows, head); the keys move through LDS
//   64 at a time (K transposed), lane = key for the scores, lane = dimension for the
//   weighted V sum, online max/sum rescaling (same recurrence as
//   mit2_gpt_causal_attention_sgq_f32, kernels.metal:2249-2292).
// Rows of several sequences may be stacked (ragged batch prefill): row m belongs to
// cache slot row_slot[m] at position row_pos[m] and attends to that slot's rows
// 0..row_pos[m].
#include <type_traits>

#include "kernels.h"

namespace itts {
namespace {

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

// GEMM tiling.  A workgroup owns up to 192 rows (row tiles of 16) x 64 columns; wave w owns
// columns 16w .. 16w + 15 of that for every row tile, so the A rows are shared through LDS
// and each wave streams its own 16 weight rows straight into registers.
// v_mfma_f32_16x16x4f32 operands: A lane l -> row l & 15, k l >> 4; B lane l -> k l >> 4,
// column l & 15; D lane l, element r -> row 4 (l >> 4) + r, column l & 15.  Which k the four
// lane groups carry is free as long as A and B agree: in the c-th of four back-to-back
// instructions lane group g carries k = k0 + 4g + c, so every lane reads four consecutive k
// of its row with one 16-byte load (a weight row in global memory, an A row in LDS).
constexpr int kBN = 64;                // output columns per workgroup
constexpr int kBK = 64;                // K per LDS stage (four 16-wide MFMA steps)
constexpr int kMaxRT = 12;             // row tiles of 16 per workgroup (RT: 2, 4, ..., 12)
constexpr int kAS = kBK + 4;           // A row stride in LDS, 4 x odd: conflict-free 16-byte reads
constexpr int kGemmThreads = 512;      // eight waves

typedef float floatx4 __attribute__((ext_vector_type(4)));

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

// A value held in a register at this point of the program: an empty asm takes it.  The GEMM
// epilogues form every output (and read every loaded operand) before the first row's store
// this way; left to the compiler, each row's arithmetic sank into that row's branch, where the
// use of a load still in flight made it wait for every memory access outstanding, the
// earlier rows' stores included (one store completion per row).
template <typename T>
__device__ __forceinline__ void pin_value(T v) {
    asm volatile("" ::"v"(v));
}

// SiLU-gated product of one (gate, up) column pair (kernels.metal:363-374).
__device__ __forceinline__ float swiglu_f(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// Four consecutive k of one weight row as floats.
__device__ __forceinline__ floatx4 gemm_load_b(const float* p) { return *reinterpret_cast<const floatx4*>(p); }
__device__ __forceinline__ floatx4 gemm_load_b(const uint16_t* p) {
    typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
    const u32x2v v = *reinterpret_cast<const u32x2v*>(p);
    return floatx4{__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                   __uint_as_float(v.y & 0xffff0000u)};
}

// One LDS stage (kBK = 64 k): four 16-wide steps over this wave's NT row tiles (tile
// t0 + 2 t).  The A fragments of step h + 1 are read while step h's instructions run;
// per step the instructions go c-major (instruction c of every tile, then c + 1), so
// consecutive instructions use different accumulators.
template <int NT>
__device__ __forceinline__ void gemm_stage(const float (*As)[kAS], int t0, int lane, const floatx4 (&b)[4], floatx4 (&acc)[NT]) {
    floatx4 av[2][NT];
    const float* base = &As[t0 * 16 + (lane & 15)][4 * (lane >> 4)];
#pragma unroll
    for (int t = 0; t < NT; ++t) av[0][t] = *reinterpret_cast<const floatx4*>(base + 32 * t * kAS);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        if (h < 3) {
#pragma unroll
            for (int t = 0; t < NT; ++t) av[(h + 1) & 1][t] = *reinterpret_cast<const floatx4*>(base + 32 * t * kAS + 16 * (h + 1));
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[h & 1][t][c], b[h][c], acc[t], 0, 0, 0);
    }
}

// Row block y covers rows [y RT 16, (y + 1) RT 16) of A; split z covers K range
// [z kchunk, min(K, (z + 1) kchunk)) and, with SPLIT, writes its raw partial tile to
// a.ws[z][M][N] for gemm_reduce_kernel.  K ranges are multiples of 2 kBK.  Eight waves:
// wave w owns columns 16 (w % 4) .. + 15 and the row tiles w / 4, w / 4 + 2, ..., so each
// SIMD runs two waves.  The main loop has no branches (rows past M and loads past the K
// range are clamped to valid addresses, their results unused), so the compiler's wait
// counts stay exact and the prefetched loads stay in flight across the matrix instructions.
template <typename WT, int EPI, bool SPLIT, int RT>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(GemmArgs a, int kchunk) {
    constexpr int BM = RT * 16, NT = RT / 2;
    constexpr int NP = BM * (kBK / 4), APER = (NP + kGemmThreads - 1) / kGemmThreads;  // A pieces per stage, per thread
    __shared__ __align__(16) float As[2][BM][kAS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int strip = wave & 3, t0 = wave >> 2;
    // Workgroup L runs on XCD L % 8 (round-robin dispatch).  The logical index j gives each
    // XCD one contiguous range, row blocks fastest, then splits, then column tiles, so the
    // workgroups sharing a column tile's weights mostly share one L2.
    const int nwg = gridDim.x * gridDim.y * gridDim.z;
    const int L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    const int per = nwg / 8, rem = nwg % 8, xcd = L % 8;
    const int j = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + L / 8;
    const int by = j % gridDim.y, bz = (j / gridDim.y) % gridDim.z, bx = j / (gridDim.y * gridDim.z);
    const int m0 = by * BM;
    const int mrows = min(BM, a.M - m0);
    const int kb = SPLIT ? bz * kchunk : 0;
    const int ke = SPLIT ? min(a.K, kb + kchunk) : a.K;
    const int nst = (ke - kb) / kBK;  // even

    // A stage loader: piece f = tid + kGemmThreads i (mod NP) is 4 consecutive k at column
    // 4 (f % 16) of row f / 16 (pieces past NP repeat earlier ones: the same value is stored
    // twice); rows past M read row M - 1 (their output rows are not stored).  Native
    // vector types: arrays of the float4 struct are copied with memcpy, which the compiler
    // left in scratch memory.
    int aoff[APER], aoffs[APER];
#pragma unroll
    for (int i = 0; i < APER; ++i) {
        const int f = (tid + kGemmThreads * i) % NP, r = f / (kBK / 4), c = (f % (kBK / 4)) * 4;
        aoff[i] = min(m0 + r, a.M - 1) * a.K + c;
        aoffs[i] = r * kAS + c;
    }
    // B: this lane's weight row (column n of the output) at k offset 4 (lane >> 4).
    const WT* wrow = static_cast<const WT*>(a.w) + static_cast<size_t>(bx * kBN + strip * 16 + (lane & 15)) * a.K + 4 * (lane >> 4);

    floatx4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Software pipeline over stages s = 0 .. nst - 1 (nst even), unrolled by two so every
    // ring index is a constant: stage s computes on LDS buffer s % 2 with weights rb[s % 2];
    // it requests the A rows of stage s + 2 (into ra[s % 2], stored a stage ago) and then
    // the weights of stage s + 2 (into rb[s % 2], once read), and ends by storing the A
    // rows of stage s + 1 (requested a stage earlier) into buffer (s + 1) % 2.  Loads
    // complete in order, so that store never waits for a load requested after it.  Loads
    // past the last stage reread it (results unused).
    floatx4 ra[2][APER], rb[2][4];
    const int klast = ke - kBK;
    auto kst = [&](int st) { return min(kb + kBK * st, klast); };
#define ITTS_LOAD_A(set, st)                                                                  \
    _Pragma("unroll") for (int i = 0; i < APER; ++i) ra[set][i] = *reinterpret_cast<const floatx4*>(a.a + aoff[i] + kst(st))
#define ITTS_LOAD_B(set, st)                                                                  \
    _Pragma("unroll") for (int q = 0; q < 4; ++q) rb[set][q] = gemm_load_b(wrow + kst(st) + 16 * q)
#define ITTS_STORE_A(set, buf)                                                                \
    _Pragma("unroll") for (int i = 0; i < APER; ++i) *reinterpret_cast<floatx4*>(&As[buf][0][0] + aoffs[i]) = ra[set][i]
#define ITTS_STAGE(Q)                                                                         \
    do {                                                                                      \
        floatx4 bcur[4];                                                                      \
        _Pragma("unroll") for (int q = 0; q < 4; ++q) bcur[q] = rb[Q][q];                     \
        ITTS_LOAD_A(Q, s + Q + 2);                                                            \
        ITTS_LOAD_B(Q, s + Q + 2);                                                            \
        __builtin_amdgcn_sched_barrier(0);                                                    \
        gemm_stage<NT>(As[Q], t0, lane, bcur, acc);                                           \
        __builtin_amdgcn_sched_barrier(0);                                                    \
        ITTS_STORE_A(1 - Q, 1 - Q);                                                           \
        __syncthreads();                                                                      \
    } while (0)
    ITTS_LOAD_A(0, 0);
    ITTS_LOAD_B(0, 0);
    ITTS_LOAD_A(1, 1);
    ITTS_LOAD_B(1, 1);
    ITTS_STORE_A(0, 0);
    __syncthreads();
    for (int s = 0; s < nst; s += 2) {
        ITTS_STAGE(0);
        ITTS_STAGE(1);
    }
#undef ITTS_STAGE
#undef ITTS_STORE_A
#undef ITTS_LOAD_B
#undef ITTS_LOAD_A

    const int col = bx * kBN + strip * 16 + (lane & 15);
    const int rq = 4 * (lane >> 4);
    if constexpr (SPLIT) {
        // Every destination's 32-bit element offset formed before the first store (a split's
        // plane is M x N < 2^31 elements): with one register pair reused for each row's
        // address, the compiler let only about two stores be in flight at a time.
        float* ws = a.ws + static_cast<size_t>(bz) * a.M * a.N;
        uint32_t off[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                off[t][r] = static_cast<uint32_t>((m0 + (t0 + 2 * t) * 16 + rq + r) * a.N + col);
                pin_value(off[t][r]);
            }
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = (t0 + 2 * t) * 16 + rq + r;
                if (row < mrows) ws[off[t][r]] = acc[t][r];
            }
    } else if constexpr (EPI == kGemmSwiglu) {
        // columns col and col ^ 1 sit in lanes l and l ^ 1, on the same rows
        const float bias = a.bias[col];
        float out[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = (t0 + 2 * t) * 16 + rq + r;
                const float v = acc[t][r] + bias;
                const float u = __shfl_xor(v, 1, 64);
                out[t][r] = swiglu_f(v, u);
                pin_value(out[t][r]);
            }
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = (t0 + 2 * t) * 16 + rq + r;
                if (row < mrows && !(col & 1)) a.c[static_cast<size_t>(m0 + row) * (a.N / 2) + col / 2] = out[t][r];
            }
    } else if constexpr (EPI == kGemmResid) {
        // Every row's residual requested before the first store (rows past the block read the
        // block's first row): a load under the per-row branch was waited for before the next.
        const float bias = a.bias[col];
        float res[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = (t0 + 2 * t) * 16 + rq + r;
                res[t][r] = a.c[static_cast<size_t>(m0 + (row < mrows ? row : 0)) * a.N + col];
            }
        float out[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                out[t][r] = res[t][r] + (acc[t][r] + bias);
                pin_value(out[t][r]);
            }
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = (t0 + 2 * t) * 16 + rq + r;
                if (row < mrows) a.c[static_cast<size_t>(m0 + row) * a.N + col] = out[t][r];
            }
    } else if constexpr (EPI == kGemmQkv) {
        // K/V columns: every row's cache slot and position requested before the first store, as
        // above (a workgroup's 64 columns are all q or all K/V: 1280 is a multiple of 64).
        const float bias = a.bias[col];
        float out[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                out[t][r] = acc[t][r] + bias;
                pin_value(out[t][r]);
            }
        if (bx * kBN < kWidth) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = (t0 + 2 * t) * 16 + rq + r;
                    if (row < mrows) a.c[static_cast<size_t>(m0 + row) * kWidth + col] = out[t][r];
                }
        } else {
            uint32_t rs[NT][4], rp[NT][4];
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = (t0 + 2 * t) * 16 + rq + r, rc = m0 + (row < mrows ? row : 0);
                    rs[t][r] = a.row_slot[rc];
                    rp[t][r] = a.row_pos[rc];
                }
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    pin_value(rs[t][r]);
                    pin_value(rp[t][r]);
                }
            const int rr = col - kWidth;
            const bool is_v = rr >= kWidth;
            const int c = is_v ? rr - kWidth : rr;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = (t0 + 2 * t) * 16 + rq + r;
                    if (row < mrows) {
                        const size_t off = static_cast<size_t>(rs[t][r]) * a.kv_slot_stride + a.kv_layer_off + (is_v ? a.kv_v_off : 0) +
                                           (static_cast<size_t>(c >> 6) * a.kv_cap + rp[t][r]) * kHeadDim + (c & 63);
                        a.kv[off] = out[t][r];
                    }
                }
        }
    } else {
        // Every value (GELU included) formed before the first store, as above.
        const float bias = a.bias[col];
        float out[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                out[t][r] = EPI == kGemmGelu ? gelu_f(acc[t][r] + bias) : acc[t][r] + bias;
                pin_value(out[t][r]);
            }
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = (t0 + 2 * t) * 16 + rq + r;
                if (row < mrows) a.c[static_cast<size_t>(m0 + row) * a.N + col] = out[t][r];
            }
    }
}

// Partial 0 + partial 1 + ... of element e in split order.  Every split's load is issued
// before the first add (SM, a power of two >= the split count, loads per element; indices
// past the split count reread the last split and their adds are skipped), so the loads
// overlap instead of forming a chain of round trips.
template <int SM>
__device__ __forceinline__ float split_sum_n(const GemmArgs& a, size_t e, size_t plane) {
    float w[SM];
#pragma unroll
    for (int z = 0; z < SM; ++z) w[z] = a.ws[static_cast<size_t>(min(z, a.splits - 1)) * plane + e];
    float d = w[0];
#pragma unroll
    for (int z = 1; z < SM; ++z)
        if (z < a.splits) d += w[z];
    return d;
}
__device__ __forceinline__ float split_sum(const GemmArgs& a, size_t e, size_t plane) {
    if (a.splits <= 2) return split_sum_n<2>(a, e, plane);
    if (a.splits <= 4) return split_sum_n<4>(a, e, plane);
    if (a.splits <= 8) return split_sum_n<8>(a, e, plane);
    return split_sum_n<kGemmMaxSplits>(a, e, plane);
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
            const float g = split_sum(a, e, plane), u = split_sum(a, e + 1, plane);
            const int col = static_cast<int>(e % a.N);
            a.c[e2] = swiglu_f(g + a.bias[col], u + a.bias[col + 1]);
        }
        return;
    }
    for (size_t e = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total; e += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const int row = static_cast<int>(e / a.N), col = static_cast<int>(e % a.N);
        const float bias = a.bias[col];
        if constexpr (EPI == kGemmQkv) {
            // the row's cache slot and position requested with the partials, not after them
            const uint32_t rs = a.row_slot[row], rp = a.row_pos[row];
            const float v = split_sum(a, e, plane) + bias;
            if (col < kWidth) {
                a.c[static_cast<size_t>(row) * kWidth + col] = v;
            } else {
                const int rr = col - kWidth;
                const bool is_v = rr >= kWidth;
                const int c = is_v ? rr - kWidth : rr;
                a.kv[static_cast<size_t>(rs) * a.kv_slot_stride + a.kv_layer_off + (is_v ? a.kv_v_off : 0) +
                     (static_cast<size_t>(c >> 6) * a.kv_cap + rp) * kHeadDim + (c & 63)] = v;
            }
        } else {
            gemm_store<EPI>(a, row, col, split_sum(a, e, plane) + bias);
        }
    }
}

// Finishes a split-K kGemmResid GEMM of 1280-wide rows and the LayerNorm after it, one
// workgroup per row: c[m] += (partials in split order + bias), then ln_out[m] =
// LayerNorm(c[m]).  Thread t holds columns t + 256 i as ln_rows_kernel does, so both
// results are bitwise those of gemm_reduce_kernel<kGemmResid> followed by ln_rows_kernel.
__global__ __launch_bounds__(256) void gemm_reduce_ln_kernel(GemmArgs a) {
    __shared__ float red[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const size_t plane = static_cast<size_t>(a.M) * a.N;
    // Every load of the five columns before the first add and store, within one split-count
    // case: per column, the split sums behind a branch and the store to c before the next
    // column's loads made each column a memory round trip of its own.
    float v[1][5];
    auto body = [&](auto sm) {
        constexpr int SM = decltype(sm)::value;
        float cv[5], bv[5], w[5][SM];
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int col = tid + 256 * i;
            const size_t e = static_cast<size_t>(row) * a.N + col;
            cv[i] = a.c[e];
            bv[i] = a.bias[col];
#pragma unroll
            for (int z = 0; z < SM; ++z) w[i][z] = a.ws[static_cast<size_t>(min(z, a.splits - 1)) * plane + e];
        }
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            float s = w[i][0];  // split_sum_n's order
#pragma unroll
            for (int z = 1; z < SM; ++z)
                if (z < a.splits) s += w[i][z];
            v[0][i] = cv[i] + (s + bv[i]);
            a.c[static_cast<size_t>(row) * a.N + tid + 256 * i] = v[0][i];
        }
    };
    if (a.splits <= 2)
        body(std::integral_constant<int, 2>{});
    else if (a.splits <= 4)
        body(std::integral_constant<int, 4>{});
    else if (a.splits <= 8)
        body(std::integral_constant<int, 8>{});
    else
        body(std::integral_constant<int, kGemmMaxSplits>{});
    ln_block<1, 5>(v, a.ln_w, a.ln_b, red);
#pragma unroll
    for (int i = 0; i < 5; ++i) a.ln_out[static_cast<size_t>(row) * kWidth + tid + 256 * i] = v[0][i];
}

// Causal attention over one head for a block of kQB consecutive rows.  The block's rows are
// taken in runs that share a cache slot (stacked sequences: positions restart at 0 in each
// slot); for each run the slot's keys 0 .. max position move through LDS kKC at a time.
// Wave w of 8 owns rows w and w + 8 and keeps their running max, sum and weighted V sum
// (lane = dimension).  Per row the arithmetic is that of one query at a time: the dot
// product over dimensions in order from 0, scores scaled by 1/8, max-subtracted exp with
// the running rescale, the V rows added in key order (kernels.metal:2249-2292).  The loop
// has no per-row branches: a key past a row's position gets score -inf and weight 0, and a
// row past its last key sees a rescale of exactly 1, so its state does not change.
constexpr int kQB = 16, kKC = 64, kAttnThreads = 512, kAttnRows = kQB / (kAttnThreads / 64);

__global__ __launch_bounds__(kAttnThreads) void causal_attention_kernel(CausalArgs a) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int NW = kAttnThreads / 64, R = kAttnRows;
    __shared__ f4 Kt[kHeadDim / 4][kKC];                 // [dimension group][key]
    __shared__ float Vs[kKC][kHeadDim + 4];
    __shared__ f4 qs[kQB][kHeadDim / 4];
    __shared__ f4 ps[NW][R][kKC / 4];                    // [wave][row of the wave][key group]
    __shared__ uint32_t rslot[kQB], rpos[kQB];
    const int m0 = blockIdx.x * kQB, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nq = min(kQB, a.M - m0);
    if (tid < kQB * kHeadDim / 4) {
        const int r = tid >> 4, c = tid & 15;
        qs[r][c] = *reinterpret_cast<const f4*>(a.q + static_cast<size_t>(m0 + min(r, nq - 1)) * kWidth + h * kHeadDim + 4 * c);
    }
    if (tid < kQB) {
        rslot[tid] = tid < nq ? a.row_slot[m0 + tid] : 0u;
        rpos[tid] = tid < nq ? a.row_pos[m0 + tid] : 0u;
    }
    __syncthreads();

    for (int r0 = 0; r0 < nq;) {
        const uint32_t slot = rslot[r0];
        int r1 = r0 + 1;
        while (r1 < nq && rslot[r1] == slot) ++r1;
        int kn = 0;
        for (int r = r0; r < r1; ++r) kn = max(kn, static_cast<int>(rpos[r]) + 1);
        const float* kb = a.kv + static_cast<size_t>(slot) * a.kv_slot_stride + a.kv_layer_off + static_cast<size_t>(h) * a.kv_cap * kHeadDim;
        const float* vb = kb + a.kv_v_off;
        // chunk loads, keys past kn clamped to kn - 1 (masked below):
        //   K piece j: key tid % 64, dimension group tid / 64 + 8 j (LDS writes conflict-free)
        //   V piece j: key tid / 16 + 32 j, dimension group tid % 16 (256-byte rows)
        f4 kr[2], vr[2];
        auto load_chunk = [&](int c0) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int kk = min(c0 + lane, kn - 1), kv = min(c0 + (tid >> 4) + 32 * j, kn - 1);
                kr[j] = *reinterpret_cast<const f4*>(kb + static_cast<size_t>(kk) * kHeadDim + 4 * (wave + NW * j));
                vr[j] = *reinterpret_cast<const f4*>(vb + static_cast<size_t>(kv) * kHeadDim + 4 * (tid & 15));
            }
        };
        int pos[R];
        float mrun[R], lrun[R], acc[R];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int r = wave + NW * i;
            pos[i] = r >= r0 && r < r1 ? static_cast<int>(rpos[r]) : -1;  // -1: not in this run
            mrun[i] = -INFINITY;
            lrun[i] = 0.0f;
            acc[i] = 0.0f;
        }
        load_chunk(0);
        for (int c0 = 0; c0 < kn; c0 += kKC) {
            __syncthreads();  // the previous chunk's readers are done
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                Kt[wave + NW * j][lane] = kr[j];
                *reinterpret_cast<f4*>(&Vs[(tid >> 4) + 32 * j][4 * (tid & 15)]) = vr[j];
            }
            __syncthreads();
            if (c0 + kKC < kn) load_chunk(c0 + kKC);
            __builtin_amdgcn_sched_barrier(0);
            // scores: lane = key
            float d[R];
#pragma unroll
            for (int i = 0; i < R; ++i) d[i] = 0.0f;
#pragma unroll
            for (int g = 0; g < kHeadDim / 4; ++g) {
                const f4 k4 = Kt[g][lane];
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    const f4 q4 = qs[wave + NW * i][g];
                    d[i] = __builtin_fmaf(q4.x, k4.x, d[i]);
                    d[i] = __builtin_fmaf(q4.y, k4.y, d[i]);
                    d[i] = __builtin_fmaf(q4.z, k4.z, d[i]);
                    d[i] = __builtin_fmaf(q4.w, k4.w, d[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const bool valid = c0 + lane <= pos[i];
                const float s = valid ? d[i] * 0.125f : -INFINITY;
                const float cm = wave_max(s);
                const float mnew = fmaxf(mrun[i], cm);
                const float corr = mrun[i] == -INFINITY ? 0.0f : expf(mrun[i] - mnew);
                const float p = valid ? expf(s - mnew) : 0.0f;
                lrun[i] = lrun[i] * corr + wave_sum(p);
                acc[i] *= corr;
                mrun[i] = mnew;
                reinterpret_cast<float*>(ps[wave][i])[lane] = p;
            }
            // acc += p_k V[k], keys in order; lane = dimension
            const int nkc = min(kKC, kn - c0);
            for (int k4 = 0; k4 < (nkc + 3) / 4; ++k4) {
                f4 pv[R];
#pragma unroll
                for (int i = 0; i < R; ++i) pv[i] = ps[wave][i][k4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v = Vs[4 * k4 + e][lane];
#pragma unroll
                    for (int i = 0; i < R; ++i) acc[i] = __builtin_fmaf(pv[i][e], v, acc[i]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < R; ++i)
            if (pos[i] >= 0) a.out[static_cast<size_t>(m0 + wave + NW * i) * kWidth + h * kHeadDim + lane] = acc[i] / lrun[i];
        r0 = r1;
    }
}

}  // namespace

hipError_t launch_ln_rows(const LnRowsArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(ln_rows_kernel, dim3(a.rows), dim3(256), 0, s, a);
    return hipGetLastError();
}

namespace {

int ceil_div(int a, int b) { return (a + b - 1) / b; }

int device_cus() {
    static int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 256;
        return n > 0 ? n : 256;
    }();
    return cus;
}

// How one GEMM is cut: row blocks of RT tiles of 16 (RT even, at most kMaxRT), K cut into
// `splits` ranges of kchunk (a multiple of 2 kBK).
struct GemmPlan {
    int rt, mblocks, splits, kchunk;
};

// The plan with the least estimated time, over every RT and split count.  The estimate is
// a least-squares fit to timings of this kernel on MI355X over RT 2..12 and 1..16 splits
// for the 1280/5120-wide and the 1024/3072/4096/6144-wide shapes at 64, 155 and 900 rows
// (median error 2.3%), in microseconds:
//   4.3 + 0.0039 rounds RT kchunk + 0.86 rounds kchunk / 128
//       + 0.11 mblocks N K / 1e6 + (split: 2.35 + 2.98 splits M N / 1e6)
// where rounds = ceil(workgroups / CUs).  The RT kchunk term is the matrix-core work of a
// workgroup (about 85% of peak); the kchunk / 128 term is a fixed cost per pair of LDS
// stages (barriers and the LDS reads after them), which is what makes short stages and
// small RT expensive; the split term is the partial tiles' round trip plus the reduce
// kernel.  max_splits caps the split count (the workspace holds kGemmWsFloats floats).
GemmPlan gemm_plan(int M, int N, int K, int max_splits, bool /*bf16*/) {
    const int rtot = ceil_div(M, 16), ntiles = N / kBN, cus = device_cus();
    const size_t mn = static_cast<size_t>(M) * N;
    const int smax = std::max(1, std::min<int>(max_splits, static_cast<int>(std::min<size_t>(kGemmMaxSplits, kGemmWsFloats / std::max<size_t>(1, mn)))));
    GemmPlan best{kMaxRT, ceil_div(rtot, kMaxRT), 1, K};
    double best_t = 1e30;
    for (int rt = 2; rt <= kMaxRT; rt += 2) {
        const int mb = ceil_div(rtot, rt);
        if (rt > 2 && ceil_div(rtot, rt - 2) == mb) continue;  // a smaller RT covers the rows in as many blocks
        for (int s = 1; s <= smax; ++s) {
            const int kc = ceil_div(ceil_div(K, s), 2 * kBK) * 2 * kBK;
            const int sp = ceil_div(K, kc);
            if (sp != s) continue;
            const long wgs = static_cast<long>(ntiles) * mb * sp;
            const double rounds = std::ceil(static_cast<double>(wgs) / cus);
            double t = 4.3 + 0.0039 * rounds * rt * kc + 0.86 * rounds * kc / (2.0 * kBK) + 0.11 * mb * static_cast<double>(N) * K / 1e6;
            if (sp > 1) t += 2.35 + 2.98 * sp * static_cast<double>(mn) / 1e6;
            if (t < best_t) {
                best_t = t;
                best = GemmPlan{rt, mb, sp, kc};
            }
        }
    }
    return best;
}

template <typename WT, int EPI, bool SPLIT>
void launch_gemm_rt(const GemmArgs& a, const GemmPlan& p, dim3 grid, hipStream_t s) {
    switch (p.rt) {
        case 2: hipLaunchKernelGGL((gemm_kernel<WT, EPI, SPLIT, 2>), grid, dim3(kGemmThreads), 0, s, a, p.kchunk); break;
        case 4: hipLaunchKernelGGL((gemm_kernel<WT, EPI, SPLIT, 4>), grid, dim3(kGemmThreads), 0, s, a, p.kchunk); break;
        case 6: hipLaunchKernelGGL((gemm_kernel<WT, EPI, SPLIT, 6>), grid, dim3(kGemmThreads), 0, s, a, p.kchunk); break;
        case 8: hipLaunchKernelGGL((gemm_kernel<WT, EPI, SPLIT, 8>), grid, dim3(kGemmThreads), 0, s, a, p.kchunk); break;
        case 10: hipLaunchKernelGGL((gemm_kernel<WT, EPI, SPLIT, 10>), grid, dim3(kGemmThreads), 0, s, a, p.kchunk); break;
        default: hipLaunchKernelGGL((gemm_kernel<WT, EPI, SPLIT, 12>), grid, dim3(kGemmThreads), 0, s, a, p.kchunk); break;
    }
}

}  // namespace

int gemm_splits(int M, int N, int K) { return gemm_plan(M, N, K, kGemmMaxSplits, false).splits; }

hipError_t launch_gemm(const GemmArgs& args, int epi, bool bf16, hipStream_t s) {
    if (args.N % kBN || args.K % (2 * kBK) || args.M < 1 || args.splits < 1 || (args.splits > 1 && !args.ws)) return hipErrorInvalidValue;
    if ((epi == kGemmStore || epi == kGemmSwiglu) && bf16) return hipErrorInvalidValue;  // FP32 weights only (the Qwen decoder)
    const GemmPlan p = gemm_plan(args.M, args.N, args.K, args.splits, bf16);
    GemmArgs a = args;
    a.splits = p.splits;
    const dim3 grid(a.N / kBN, p.mblocks, p.splits);
    const bool ln = args.ln_out != nullptr;
    if (ln && (epi != kGemmResid || args.N != kWidth)) return hipErrorInvalidValue;
    if (p.splits > 1) {
        // the partial tiles do not depend on the epilogue
        if (bf16) launch_gemm_rt<uint16_t, kGemmStore, true>(a, p, grid, s);
        else launch_gemm_rt<float, kGemmStore, true>(a, p, grid, s);
        if (ln) {
            hipLaunchKernelGGL(gemm_reduce_ln_kernel, dim3(a.M), dim3(256), 0, s, a);
            return hipGetLastError();
        }
        const int rblocks = static_cast<int>(std::min<size_t>((static_cast<size_t>(a.M) * a.N + 255) / 256, 2048));
        switch (epi) {
            case kGemmQkv: hipLaunchKernelGGL((gemm_reduce_kernel<kGemmQkv>), dim3(rblocks), dim3(256), 0, s, a); break;
            case kGemmResid: hipLaunchKernelGGL((gemm_reduce_kernel<kGemmResid>), dim3(rblocks), dim3(256), 0, s, a); break;
            case kGemmGelu: hipLaunchKernelGGL((gemm_reduce_kernel<kGemmGelu>), dim3(rblocks), dim3(256), 0, s, a); break;
            case kGemmStore: hipLaunchKernelGGL((gemm_reduce_kernel<kGemmStore>), dim3(rblocks), dim3(256), 0, s, a); break;
            default: hipLaunchKernelGGL((gemm_reduce_kernel<kGemmSwiglu>), dim3(rblocks), dim3(256), 0, s, a); break;
        }
        return hipGetLastError();
    }
    switch (epi) {
        case kGemmQkv: bf16 ? launch_gemm_rt<uint16_t, kGemmQkv, false>(a, p, grid, s) : launch_gemm_rt<float, kGemmQkv, false>(a, p, grid, s); break;
        case kGemmResid: bf16 ? launch_gemm_rt<uint16_t, kGemmResid, false>(a, p, grid, s) : launch_gemm_rt<float, kGemmResid, false>(a, p, grid, s); break;
        case kGemmGelu: bf16 ? launch_gemm_rt<uint16_t, kGemmGelu, false>(a, p, grid, s) : launch_gemm_rt<float, kGemmGelu, false>(a, p, grid, s); break;
        case kGemmStore: launch_gemm_rt<float, kGemmStore, false>(a, p, grid, s); break;
        default: launch_gemm_rt<float, kGemmSwiglu, false>(a, p, grid, s); break;
    }
    if (ln) hipLaunchKernelGGL(ln_rows_kernel, dim3(a.M), dim3(256), 0, s, LnRowsArgs{a.c, a.ln_out, a.ln_w, a.ln_b, a.M});
    return hipGetLastError();
}

hipError_t launch_causal_attention(const CausalArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(causal_attention_kernel, dim3((a.M + kQB - 1) / kQB, kHeads), dim3(kAttnThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace itts

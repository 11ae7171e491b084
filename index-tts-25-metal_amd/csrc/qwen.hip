// Qwen3-0.6B emotion-text decoder (itts25::QwenDecoder, src/qwen.cpp:5-49) on the MI355X:
// kernels, the host engine and the C ABI of include/itts_qwen.h.
//
// Model: 28 layers, width 1024, 16 query heads over 8 KV heads of 128, RMSNorm (eps 1e-6)
// before attention and MLP and per head on q and k, rotate-half RoPE (theta 1e6), SiLU-gated
// MLP of 3072, final RMSNorm, logits through the tied 151936 x 1024 embedding, greedy argmax.
//
// Layout in HBM (one handle):
//   * weight slab, per layer in consumption order, row-major [out][in]: q|k|v projections as
//     one [4096][1024] matrix, o_proj [1024][2048], gate/up interleaved as [6144][1024]
//     (row 2i = gate_i, row 2i + 1 = up_i, so one wave's row pair yields silu(gate) * up),
//     down_proj [1024][3072]; the embedding [151936][1024] separately (input rows and head);
//   * KV cache [layer][K|V][kv head][row][128], 4096 rows (gptKvCacheCreate(28, 4096, 1024),
//     metal_context.mm:5675-5700, keeps [layer][K|V][row][1024]): a head's rows are
//     contiguous, so a decode-attention tile is one contiguous range per K and per V.
// Decode (one token): per layer
//   q_gemv<RMSNorm, store>  (the layer-0 one gathers the embedding row of the state's token)
//   q_attn_kernel           per-head RMSNorm of q and k and RoPE, the step's K/V row into the
//                           cache, then split-KV attention, 64 rows x one KV head per tile,
//                           both query heads of the KV head, partial (max, sum, weighted V)
//   q_attn_merge_kernel     the splits merged with exp(m_s - M) rescaling
//   q_gemv<-, residual>     o_proj, added to the residual stream in place
//   q_gemv<RMSNorm, swiglu> gate/up pairs -> silu(gate) * up
//   q_gemv<-, residual>     down_proj
// then q_gemv<RMSNorm, argmax> over the embedding rows (logits and a per-workgroup best) and
// q_argmax_kernel, which picks the token and advances the device state.  The step is
// captured once as a hipGraph; token, cache length and count live in device QState, so
// generate() replays it with no per-token host work and polls a flag every 16 tokens.
// Prefill (P ids): embedding rows, RMSNorm rows, FP32 MFMA GEMMs of prefill.hip (store, residual
// and SwiGLU epilogues, split K when tiles are few), q_prep_kernel over P rows, causal
// attention, then the head on the last row.
#include <type_traits>
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "itts_qwen.h"
#include "kernels.h"

namespace itts {
namespace qwen {

constexpr int kV = 151936, kD = 1024, kQ = 2048, kKV = 1024, kQkvN = kQ + 2 * kKV, kF = 3072, kHd = 128;
constexpr int kQH = 16, kKVH = 8;
constexpr int kCap = 4096, kPrompt = 3072, kMaxGen = 1024;
constexpr uint32_t kEos = 151643;
constexpr float kEps = 1e-6f;
constexpr float kScale = 0.08838834764831844f;  // 1 / sqrt(128), qwen_attention (kernels.metal:3122)
constexpr int kSplitRows = 64, kMaxSplits = kCap / kSplitRows;
constexpr int kAttnGrid = 256;
constexpr int kHeadRpw = 4, kHeadBlocks = kV / (4 * kHeadRpw);  // 9496 workgroups of 16 rows
static_assert(kV % (4 * kHeadRpw) == 0, "head rows per workgroup");
// per-layer slab offsets (floats)
constexpr size_t kOffO = size_t(kQkvN) * kD, kOffGu = kOffO + size_t(kD) * kQ, kOffD = kOffGu + size_t(2 * kF) * kD;
constexpr size_t kLayerFloats = kOffD + size_t(kD) * kF;
// per-layer small parameters: input_layernorm, post_attention_layernorm, q_norm, k_norm
constexpr int kNormIn = 0, kNormPost = kD, kNormQ = 2 * kD, kNormK = 2 * kD + kHd, kNormLayer = 2 * kD + 2 * kHd;

// Device-side decode state.  `cached` is the number of cache rows before the running pass;
// the argmax kernel appends the token and advances it.
struct QState {
    uint32_t token, cached, count, active, maximum, eos, no_stop, pad;
};
// Pinned host staging: `up` is copied to the device state, `down` and `flag` receive copies
// of it (the stop flag of two polls in flight).
struct HostStage {
    QState up, down;
    uint32_t flag[2];
};

enum : int { kProNone = 0, kProRms = 1, kProEmbedRms = 2 };
enum : int { kEpiStore = 0, kEpiResid = 1, kEpiSwiglu = 2, kEpiArgmax = 3 };

struct QGemvArgs {
    const float* w;        // [rows][COLS]
    int rows;
    const float* x;        // input row (COLS floats); unused for kProEmbedRms
    const float* norm_w;   // RMSNorm weight (COLS)
    const float* embed;    // kProEmbedRms: the embedding table
    float* h_out;          // kProEmbedRms: the gathered row is the residual stream
    float* out;            // store: [rows]; swiglu: [rows / 2]; argmax: logits [rows]
    float* resid;          // kEpiResid: out[row] = resid[row] + dot (may alias out)
    float2* best;          // kEpiArgmax: per-workgroup (value, index bits)
    const QState* st;
};

struct QPrepArgs {
    const float* qkv;      // [rows][4096]: q | k | v
    int rows;
    float* q;              // [rows][2048]
    float* kc;             // this layer's K cache [8][kCap][128]
    float* vc;
    const float* q_norm;
    const float* k_norm;
    const float* inv_freq; // [64]
    const QState* st;      // decode: rows start at st->cached; null (prefill): at 0
};

struct QAttnArgs {
    const float* qkv;      // the step row's raw q | k | v [4096]
    float* kc;             // this layer's K cache [8][kCap][128]
    float* vc;
    const float* q_norm;
    const float* k_norm;
    const float* inv_freq;
    float* part_acc;       // [kMaxSplits][16][128]
    float* part_ml;        // [kMaxSplits][16][2]: max, sum
    float* att;            // [2048] the merged attention output
    const QState* st;
};

struct QCausalArgs {
    const float* q;        // [rows][2048]
    const float* kc;
    const float* vc;
    float* out;            // [rows][2048]
    int rows;
};

struct QArgmaxArgs {
    const float2* best;
    int nbest;
    QState* st;
    uint32_t* tokens;      // [kMaxGen]
    uint32_t advance;      // cache rows the pass added (prompt length or 1)
};

__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float t = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return t;
}

// The sum over each 32-lane half of the wave (both halves at once).
__device__ __forceinline__ float half_sum(float v) {
    const float u = row16_sum(v);
    return xsum16(u, u);
}

__device__ __forceinline__ float dot4(float4 a, float4 b, float acc) {
    acc = __builtin_fmaf(a.x, b.x, acc);
    acc = __builtin_fmaf(a.y, b.y, acc);
    acc = __builtin_fmaf(a.z, b.z, acc);
    return __builtin_fmaf(a.w, b.w, acc);
}

__device__ __forceinline__ float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// One head's per-head RMSNorm then RoPE at position pos (qwen.cpp:29-32; qwen_rope,
// kernels.metal:3111-3115), by one wave: lane l holds dimensions l and l + 64, the pair the
// rotation mixes, with its weights g1 = g[l], g2 = g[l + 64] and frequency f = inv_freq[l].
// Returns the two outputs.
__device__ __forceinline__ float2 head_norm_rope(float x1, float x2, float g1, float g2, float f, uint32_t pos) {
    const float ss = wave_sum(__builtin_fmaf(x1, x1, x2 * x2));
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(kHd) + kEps);
    const float n1 = x1 * inv * g1, n2 = x2 * inv * g2;
    float sn, cs;
    sincosf(static_cast<float>(pos) * f, &sn, &cs);
    return make_float2(n1 * cs + (-n2) * sn, n2 * cs + n1 * sn);
}
// The same, reading the lane's weights from g and its frequency from inv_freq.
__device__ __forceinline__ float2 head_norm_rope(float x1, float x2, const float* g, const float* inv_freq, uint32_t pos) {
    const int l = threadIdx.x & 63;
    return head_norm_rope(x1, x2, g[l], g[l + 64], inv_freq[l], pos);
}

// (v, i) replaces (bv, bi) under mit2_gpt_argmax_f32's rule (kernels.metal:1283-1297).
__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) { return v > bv || (v == bv && i < bi); }

// ---------------------------------------------------------------------------- decode GEMV
// Each of the 4 waves owns RPW whole rows: lane l multiplies the 16-byte chunks l, l + 64, ...
// of each row with the matching input chunks (one FMA chain per row), then an xor-butterfly
// wave sum; no atomics.  All weight loads are issued before the prologue (input row, RMSNorm
// into LDS), so the normalisation overlaps the weight fetch.
template <int COLS, int RPW, int PRO, int EPI>
__global__ __launch_bounds__(256) void q_gemv_kernel(QGemvArgs a) {
    constexpr int J = COLS / 256;  // 16-byte chunks per lane per row, and input floats per thread
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (!a.st->active) return;
    const int row0 = (blockIdx.x * 4 + wave) * RPW;

    float xv[J], nw[J];
    if constexpr (PRO == kProEmbedRms) {
        const size_t base = static_cast<size_t>(a.st->token) * COLS;
#pragma unroll
        for (int i = 0; i < J; ++i) xv[i] = a.embed[base + tid + 256 * i];
    } else {
#pragma unroll
        for (int i = 0; i < J; ++i) xv[i] = a.x[tid + 256 * i];
    }
    if constexpr (PRO != kProNone) {
#pragma unroll
        for (int i = 0; i < J; ++i) nw[i] = a.norm_w[tid + 256 * i];
    }

    using LD = WLoad<float>;
    f32x4 wv[RPW][J];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int rr = min(row0 + r, a.rows - 1);  // loads stay in bounds; result discarded
#pragma unroll
        for (int j = 0; j < J; ++j) wv[r][j] = LD::load(a.w, static_cast<size_t>(rr) * (COLS / 4) + j * 64 + lane);
    }

    __shared__ __align__(16) float xs[COLS];
    __shared__ float red[4];
    if constexpr (PRO != kProNone) {
        if (PRO == kProEmbedRms && blockIdx.x == 0) {
#pragma unroll
            for (int i = 0; i < J; ++i) a.h_out[tid + 256 * i] = xv[i];
        }
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < J; ++i) ss = __builtin_fmaf(xv[i], xv[i], ss);
        ss = block_sum256(ss, red);
        const float inv = 1.0f / sqrtf(ss / static_cast<float>(COLS) + kEps);
#pragma unroll
        for (int i = 0; i < J; ++i) xs[tid + 256 * i] = xv[i] * inv * nw[i];
    } else {
#pragma unroll
        for (int i = 0; i < J; ++i) xs[tid + 256 * i] = xv[i];
    }
    __syncthreads();

    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const float4 x4 = *reinterpret_cast<const float4*>(&xs[(j * 64 + lane) * 4]);
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[r] = dot4(LD::to_f4(wv[r][j]), x4, acc[r]);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = wave_sum(acc[r]) + 0.0f;  // + the zero bias (qwen.cpp:17-19)

    if constexpr (EPI == kEpiStore || EPI == kEpiArgmax) {
#pragma unroll
        for (int r = 0; r < RPW; ++r)
            if (lane == r && row0 + r < a.rows) a.out[row0 + r] = acc[r];
    } else if constexpr (EPI == kEpiResid) {
#pragma unroll
        for (int r = 0; r < RPW; ++r)
            if (lane == r && row0 + r < a.rows) a.out[row0 + r] = a.resid[row0 + r] + acc[r];
    } else {
        static_assert(EPI != kEpiSwiglu || RPW % 2 == 0, "gate/up rows come in pairs");
#pragma unroll
        for (int r = 0; r < RPW; r += 2)
            if (lane == r && row0 + r + 1 < a.rows) a.out[(row0 + r) / 2] = silu_mul(acc[r], acc[r + 1]);
    }
    if constexpr (EPI == kEpiArgmax) {
        __shared__ float bvs[4];
        __shared__ uint32_t bis[4];
        float bv = -INFINITY;
        uint32_t bi = 0;
#pragma unroll
        for (int r = 0; r < RPW; ++r)
            if (row0 + r < a.rows && better(acc[r], static_cast<uint32_t>(row0 + r), bv, bi)) {
                bv = acc[r];
                bi = static_cast<uint32_t>(row0 + r);
            }
        if (lane == 0) {
            bvs[wave] = bv;
            bis[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            float v = bvs[0];
            uint32_t i = bis[0];
            for (int w = 1; w < 4; ++w)
                if (better(bvs[w], bis[w], v, i)) {
                    v = bvs[w];
                    i = bis[w];
                }
            a.best[blockIdx.x] = make_float2(v, __uint_as_float(i));
        }
    }
}

// The token: the best of the workgroups' bests, then the state advance (qwen.cpp:48).
__global__ __launch_bounds__(1024) void q_argmax_kernel(QArgmaxArgs a) {
    QState* st = a.st;
    if (!st->active) return;
    __shared__ float sv[1024];
    __shared__ uint32_t si[1024];
    const int t = threadIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0;
    // every best this thread folds requested at once (kHeadBlocks bounds nbest), in the same order
    constexpr int KB = (kHeadBlocks + 1023) / 1024;
    float2 bs[KB];
#pragma unroll
    for (int r = 0; r < KB; ++r) bs[r] = a.best[min(t + 1024 * r, a.nbest - 1)];
#pragma unroll
    for (int r = 0; r < KB; ++r) {
        const uint32_t i = __float_as_uint(bs[r].y);
        if (t + 1024 * r < a.nbest && better(bs[r].x, i, bv, bi)) {
            bv = bs[r].x;
            bi = i;
        }
    }
    sv[t] = bv;
    si[t] = bi;
    __syncthreads();
    for (int s = 512; s > 0; s >>= 1) {
        if (t < s && better(sv[t + s], si[t + s], sv[t], si[t])) {
            sv[t] = sv[t + s];
            si[t] = si[t + s];
        }
        __syncthreads();
    }
    if (t == 0) {
        const uint32_t tok = si[0];
        st->token = tok;
        a.tokens[st->count % kMaxGen] = tok;
        st->count += 1;
        st->cached += a.advance;
        if (!st->no_stop) {
            if (tok == kEos) {
                st->eos = 1;
                st->active = 0;
            } else if (st->count >= st->maximum) {
                st->active = 0;
            }
        }
    }
}

// ------------------------------------------------------------- q/k norm, RoPE, cache rows
// One wave per (row, head of q|k|v): lane l holds dimensions l and l + 64, the pair RoPE
// rotates together (qwen_rope, kernels.metal:3111-3115; the per-head RMSNorm of
// qwen.cpp:29-30 first).  V rows are copied into the cache unchanged.
__global__ __launch_bounds__(64) void q_prep_kernel(QPrepArgs a) {
    const int r = blockIdx.x, hh = blockIdx.y, l = threadIdx.x;
    uint32_t base = 0;
    if (a.st) {
        if (!a.st->active) return;
        base = a.st->cached;
    }
    const uint32_t pos = base + static_cast<uint32_t>(r);
    const float* src = a.qkv + static_cast<size_t>(r) * kQkvN;
    if (hh >= kQH + kKVH) {
        const int vh = hh - kQH - kKVH;
        float* dst = a.vc + (static_cast<size_t>(vh) * kCap + pos) * kHd;
        dst[l] = src[kQ + kKV + vh * kHd + l];
        dst[l + 64] = src[kQ + kKV + vh * kHd + l + 64];
        return;
    }
    const bool isq = hh < kQH;
    const int col = isq ? hh * kHd : kQ + (hh - kQH) * kHd;
    const float2 o = head_norm_rope(src[col + l], src[col + l + 64], isq ? a.q_norm : a.k_norm, a.inv_freq, pos);
    float* dst = isq ? a.q + static_cast<size_t>(r) * kQ + hh * kHd : a.kc + (static_cast<size_t>(hh - kQH) * kCap + pos) * kHd;
    dst[l] = o.x;
    dst[l + 64] = o.y;
}

// ------------------------------------------------------------------- decode attention
// Tiles (split, KV head) over a fixed grid (the graph is captured before the length is known):
// a tile is cache rows [64 s, 64 s + 64) of one KV head against both of its query heads
// (head / 2 = KV head, kernels.metal:3120).  Each tile first forms its two query heads from the
// raw projection (per-head RMSNorm, RoPE at the step's position: waves 0 and 1); the tile that
// holds the step's own row also forms that row's K (wave 2) and V (wave 3), uses them from LDS
// and writes them to the cache (kernels.metal:3116-3118).  Eight 32-lane groups take 8 rows
// each, one float4 of the 128 dimensions per lane, K and V loaded up front.  Partial results:
// the split's max score, its sum of exp(score - max) and its weighted V sum.
__global__ __launch_bounds__(256) void q_attn_kernel(QAttnArgs a) {
    if (!a.st->active) return;
    const uint32_t cached = a.st->cached;
    const int L = static_cast<int>(cached) + 1;
    const int own = static_cast<int>(cached) / kSplitRows;  // the split holding the step's row
    const int tiles = ((L + kSplitRows - 1) / kSplitRows) * kKVH;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = tid >> 5, j = tid & 31;
    __shared__ __align__(16) float qs[2][kHd];
    __shared__ __align__(16) float knew[kHd], vnew[kHd];
    __shared__ float gm[2][8], gl[2][8];
    __shared__ float4 gacc[8][2][32];
    for (int t = blockIdx.x; t < tiles; t += gridDim.x) {
        const int split = t / kKVH, kvh = t % kKVH;
        float* kb = a.kc + static_cast<size_t>(kvh) * kCap * kHd;
        float* vb = a.vc + static_cast<size_t>(kvh) * kCap * kHd;
        const int r0 = split * kSplitRows + g * 8;
        // This wave's pair of projection values with its RMSNorm weights and RoPE frequency
        // (waves 0, 1: the two query heads; 2: the step's K row; 3: its V row, used by the
        // tile that holds the step's row), requested before the cache rows below so that the
        // waits for them do not also wait for the rows (loads complete in order).
        const int col = wave < 2 ? (2 * kvh + wave) * kHd : wave == 2 ? kQ + kvh * kHd : kQ + kKV + kvh * kHd;
        const float* gw = wave < 2 ? a.q_norm : a.k_norm;
        const float x1 = a.qkv[col + lane], x2 = a.qkv[col + lane + 64];
        const float g1 = gw[lane], g2 = gw[lane + 64], fr = a.inv_freq[lane];
        // The cached rows' K and V do not depend on this step's projection, so they are
        // requested next and arrive while the query heads are formed.  Rows from `cached` on
        // read row 0 (in bounds) and take the step's own row from LDS after the barrier.
        float4 kr[8], vr[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int row = r0 + i;
            const size_t off = static_cast<size_t>(row < static_cast<int>(cached) ? row : 0) * kHd + 4 * j;
            kr[i] = *reinterpret_cast<const float4*>(kb + off);
            vr[i] = *reinterpret_cast<const float4*>(vb + off);
        }
        if (wave < 2) {
            const float2 o = head_norm_rope(x1, x2, g1, g2, fr, cached);
            qs[wave][lane] = o.x;
            qs[wave][lane + 64] = o.y;
        } else if (split == own) {
            if (wave == 2) {
                const float2 o = head_norm_rope(x1, x2, g1, g2, fr, cached);
                knew[lane] = o.x;
                knew[lane + 64] = o.y;
                kb[static_cast<size_t>(cached) * kHd + lane] = o.x;
                kb[static_cast<size_t>(cached) * kHd + lane + 64] = o.y;
            } else {
                vnew[lane] = x1;
                vnew[lane + 64] = x2;
                vb[static_cast<size_t>(cached) * kHd + lane] = x1;
                vb[static_cast<size_t>(cached) * kHd + lane + 64] = x2;
            }
        }
        __syncthreads();
        const float4 q0 = *reinterpret_cast<const float4*>(&qs[0][4 * j]);
        const float4 q1 = *reinterpret_cast<const float4*>(&qs[1][4 * j]);
        const float4 kn = *reinterpret_cast<const float4*>(&knew[4 * j]);
        const float4 vn = *reinterpret_cast<const float4*>(&vnew[4 * j]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (!(r0 + i < static_cast<int>(cached))) {
                kr[i] = kn;
                vr[i] = vn;
            }
        }
        float s0[8], s1[8], m0 = -INFINITY, m1 = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            s0[i] = half_sum(dot4(q0, kr[i], 0.0f)) * kScale;
            s1[i] = half_sum(dot4(q1, kr[i], 0.0f)) * kScale;
            if (r0 + i >= L) s0[i] = s1[i] = -INFINITY;
            m0 = fmaxf(m0, s0[i]);
            m1 = fmaxf(m1, s1[i]);
        }
        if (j == 0) {
            gm[0][g] = m0;
            gm[1][g] = m1;
        }
        __syncthreads();
        float M0 = gm[0][0], M1 = gm[1][0];
#pragma unroll
        for (int k = 1; k < 8; ++k) {
            M0 = fmaxf(M0, gm[0][k]);
            M1 = fmaxf(M1, gm[1][k]);
        }
        float l0 = 0.0f, l1 = 0.0f;
        float4 a0 = make_float4(0.f, 0.f, 0.f, 0.f), a1 = a0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const bool ok = r0 + i < L;
            const float p0 = ok ? expf(s0[i] - M0) : 0.0f, p1 = ok ? expf(s1[i] - M1) : 0.0f;
            l0 += p0;
            l1 += p1;
            a0.x = __builtin_fmaf(p0, vr[i].x, a0.x);
            a0.y = __builtin_fmaf(p0, vr[i].y, a0.y);
            a0.z = __builtin_fmaf(p0, vr[i].z, a0.z);
            a0.w = __builtin_fmaf(p0, vr[i].w, a0.w);
            a1.x = __builtin_fmaf(p1, vr[i].x, a1.x);
            a1.y = __builtin_fmaf(p1, vr[i].y, a1.y);
            a1.z = __builtin_fmaf(p1, vr[i].z, a1.z);
            a1.w = __builtin_fmaf(p1, vr[i].w, a1.w);
        }
        if (j == 0) {
            gl[0][g] = l0;
            gl[1][g] = l1;
        }
        gacc[g][0][j] = a0;
        gacc[g][1][j] = a1;
        __syncthreads();
        const int h = tid >> 7, d = tid & 127;
        // Dimension d of group k's sum is float d of gacc[k][h] (component d & 3 of float4
        // d >> 2), read as one float: a select over the four components compiled to a chain
        // of branches, each waiting for its own LDS read.
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) s += reinterpret_cast<const float*>(gacc[k][h])[d];
        const int qh = 2 * kvh + h;
        a.part_acc[(static_cast<size_t>(split) * kQH + qh) * kHd + d] = s;
        if (d == 0) {
            float l = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) l += gl[h][k];
            a.part_ml[(split * kQH + qh) * 2] = h ? M1 : M0;
            a.part_ml[(split * kQH + qh) * 2 + 1] = l;
        }
        __syncthreads();  // qs / knew / vnew / gm / gl / gacc are reused by the next tile
    }
}

// The splits of each query head merged with exp(m_s - M) rescaling, in split order.
__global__ __launch_bounds__(128) void q_attn_merge_kernel(QAttnArgs a) {
    const int qh = blockIdx.x, d = threadIdx.x;
    // The flag and the row count, requested first and together (scalar loads: no asm statement
    // precedes them, which the compiler would count as a possible store).  The empty asm below
    // keeps both loads above it, so the count is not read behind a branch on the flag.
    const uint32_t act = a.st->active, cached = a.st->cached;
    // The first PE splits' partials are requested before the split count is known (a cache of
    // up to 512 rows then waits for one memory round trip, not two); splits past the count are
    // skipped below, whatever was read for them.  The (max, sum) pairs are read at a per-lane
    // offset of zero that the compiler cannot see through: as uniform scalar loads they were
    // spilled to vector lanes and waited for one at a time.
    constexpr int PE = 8;
    static_assert(PE <= kMaxSplits, "the partial buffers hold kMaxSplits splits");
    int vz = 0;
    asm volatile("" : "+v"(vz));
    const float* ml = a.part_ml + vz;
    float m0[PE], l0[PE], v0[PE];
#pragma unroll
    for (int s = 0; s < PE; ++s) {
        m0[s] = ml[(s * kQH + qh) * 2];
        l0[s] = ml[(s * kQH + qh) * 2 + 1];
        v0[s] = a.part_acc[(static_cast<size_t>(s) * kQH + qh) * kHd + d];
    }
    const bool active = act != 0;
    const int splits = active ? (static_cast<int>(cached) + 1 + kSplitRows - 1) / kSplitRows : 0;
    // Every further split's partials requested before the first use (SM >= splits; indices past
    // the count reread the last split and are skipped): the loops over the splits issued one
    // load at a time, each a memory round trip.  Same operations in the same order as before.
    auto merge = [&](auto sm) {
        constexpr int SM = decltype(sm)::value;
        float m[SM], l[SM], v[SM];
#pragma unroll
        for (int s = 0; s < SM; ++s) {
            if (s < PE) {
                m[s] = m0[s];
                l[s] = l0[s];
                v[s] = v0[s];
            } else {
                const int sc = min(s, splits - 1);
                m[s] = ml[(sc * kQH + qh) * 2];
                l[s] = ml[(sc * kQH + qh) * 2 + 1];
                v[s] = a.part_acc[(static_cast<size_t>(sc) * kQH + qh) * kHd + d];
            }
        }
        float M = -INFINITY;
#pragma unroll
        for (int s = 0; s < SM; ++s)
            if (s < splits) M = fmaxf(M, m[s]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int s = 0; s < SM; ++s)
            if (s < splits) {
                const float w = expf(m[s] - M);
                num = __builtin_fmaf(w, v[s], num);
                den = __builtin_fmaf(w, l[s], den);
            }
        if (active) a.att[qh * kHd + d] = num / den;
    };
    if (splits <= PE)
        merge(std::integral_constant<int, PE>{});
    else if (splits <= 32)
        merge(std::integral_constant<int, 32>{});
    else
        merge(std::integral_constant<int, kMaxSplits>{});
}

// ------------------------------------------------------------------------ prefill pieces
__global__ __launch_bounds__(256) void q_embed_rows_kernel(const float* embed, const uint32_t* ids, float* x) {
    const int r = blockIdx.x, t = threadIdx.x;
    const float4 v = *reinterpret_cast<const float4*>(embed + static_cast<size_t>(ids[r]) * kD + 4 * t);
    *reinterpret_cast<float4*>(x + static_cast<size_t>(r) * kD + 4 * t) = v;
}

// RMSNorm of each 1024-wide row (mit2_rmsnorm_f32_rows_eps, kernels.metal:995-1030).
__global__ __launch_bounds__(256) void q_rms_rows_kernel(const float* x, const float* w, float* y) {
    __shared__ float red[4];
    const int r = blockIdx.x, t = threadIdx.x;
    const float4 v = *reinterpret_cast<const float4*>(x + static_cast<size_t>(r) * kD + 4 * t);
    const float4 g = *reinterpret_cast<const float4*>(w + 4 * t);
    float ss = __builtin_fmaf(v.x, v.x, v.y * v.y);
    ss = __builtin_fmaf(v.z, v.z, ss);
    ss = __builtin_fmaf(v.w, v.w, ss);
    ss = block_sum256(ss, red);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(kD) + kEps);
    *reinterpret_cast<float4*>(y + static_cast<size_t>(r) * kD + 4 * t) =
        make_float4(v.x * inv * g.x, v.y * inv * g.y, v.z * inv * g.z, v.w * inv * g.w);
}

// Causal attention of the prompt rows (qwen_attention, kernels.metal:3119-3129, offset 0): one
// wave per (row, query head); 64 keys per pass with lane = key for the scores, lanes = the
// dimension pairs (l, l + 64) for the weighted V sum; online max / sum rescaling.
__global__ __launch_bounds__(64) void q_causal_attn_kernel(QCausalArgs a) {
    const int m = blockIdx.x, h = blockIdx.y, lane = threadIdx.x, kvh = h >> 1;
    __shared__ __align__(16) float qs[kHd];
    qs[lane] = a.q[static_cast<size_t>(m) * kQ + h * kHd + lane];
    qs[lane + 64] = a.q[static_cast<size_t>(m) * kQ + h * kHd + lane + 64];
    __syncthreads();
    const float* kb = a.kc + static_cast<size_t>(kvh) * kCap * kHd;
    const float* vb = a.vc + static_cast<size_t>(kvh) * kCap * kHd;
    float mrun = -INFINITY, lrun = 0.0f, acc1 = 0.0f, acc2 = 0.0f;
    for (int c0 = 0; c0 <= m; c0 += 64) {
        const int key = c0 + lane;
        const bool valid = key <= m;
        float s = -INFINITY;
        if (valid) {
            const float4* kr = reinterpret_cast<const float4*>(kb + static_cast<size_t>(key) * kHd);
            const float4* q4 = reinterpret_cast<const float4*>(qs);
            float d = 0.0f;
#pragma unroll 8
            for (int i = 0; i < kHd / 4; ++i) d = dot4(q4[i], kr[i], d);
            s = d * kScale;
        }
        const float cm = wave_max(s);
        const float mnew = fmaxf(mrun, cm);
        const float corr = mrun == -INFINITY ? 0.0f : expf(mrun - mnew);
        const float p = valid ? expf(s - mnew) : 0.0f;
        lrun = lrun * corr + wave_sum(p);
        acc1 *= corr;
        acc2 *= corr;
        const int nk = min(64, m + 1 - c0);
        for (int k0 = 0; k0 < nk; k0 += 16) {
            float v1[16], v2[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const bool ok = k0 + i < nk;
                const size_t off = static_cast<size_t>(c0 + (ok ? k0 + i : 0)) * kHd + lane;
                v1[i] = ok ? vb[off] : 0.0f;
                v2[i] = ok ? vb[off + 64] : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (k0 + i < nk) {
                    const float pk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), k0 + i));
                    acc1 = __builtin_fmaf(pk, v1[i], acc1);
                    acc2 = __builtin_fmaf(pk, v2[i], acc2);
                }
        }
        mrun = mnew;
    }
    a.out[static_cast<size_t>(m) * kQ + h * kHd + lane] = acc1 / lrun;
    a.out[static_cast<size_t>(m) * kQ + h * kHd + lane + 64] = acc2 / lrun;
}

#define QWEN_CHECK(x)                                                                                        \
    do {                                                                                                     \
        const hipError_t e_ = (x);                                                                           \
        if (e_ != hipSuccess) throw std::runtime_error(std::string("HIP error ") + hipGetErrorString(e_) + " in " #x); \
    } while (0)

template <class T>
struct Buf {
    T* p = nullptr;
    size_t n = 0;
    Buf() = default;
    Buf(const Buf&) = delete;
    Buf& operator=(const Buf&) = delete;
    ~Buf() { reset(); }
    void reset() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
    void alloc(size_t count) {
        reset();
        if (count) QWEN_CHECK(hipMalloc(&p, count * sizeof(T)));
        n = count;
    }
};

struct Tensor {
    const float* data;
    std::vector<int64_t> shape;
};

template <int COLS, int RPW, int PRO, int EPI>
void gemv(const QGemvArgs& a, hipStream_t s) {
    if (a.rows % (4 * RPW)) throw std::logic_error("GEMV rows per workgroup");
    hipLaunchKernelGGL((q_gemv_kernel<COLS, RPW, PRO, EPI>), dim3(a.rows / (4 * RPW)), dim3(256), 0, s, a);
    QWEN_CHECK(hipGetLastError());
}

struct Engine {
    std::string last_error;
    int layers = 28;
    hipStream_t stream = nullptr;
    hipEvent_t ev[2] = {nullptr, nullptr};
    Buf<float> slab, embed, norms, inv_freq, zeros, kv;
    Buf<float> h, qkv, att, ff, logits, part_acc, part_ml;
    Buf<float2> best;
    Buf<QState> st;
    Buf<uint32_t> toks, ids;
    Buf<float> X, Xn, QKV, Qp, ATT, FF, ws;
    int pcap = 0;
    HostStage* pinned = nullptr;
    hipEvent_t up_done = nullptr;  // the last copy out of pinned->up
    bool up_pending = false;
    hipGraphExec_t step_graph = nullptr;
    bool use_graphs = true;
    uint32_t cached = 0;
    uint64_t submissions = 0;

    ~Engine() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (step_graph) (void)hipGraphExecDestroy(step_graph);
        for (auto& e : ev)
            if (e) (void)hipEventDestroy(e);
        if (up_done) (void)hipEventDestroy(up_done);
        if (pinned) (void)hipHostFree(pinned);
        if (stream) (void)hipStreamDestroy(stream);
    }

    const float* W(int l) const { return slab.p + static_cast<size_t>(l) * kLayerFloats; }
    const float* N(int l) const { return norms.p + static_cast<size_t>(l) * kNormLayer; }
    float* K(int l) const { return kv.p + static_cast<size_t>(2 * l) * kKVH * kCap * kHd; }
    float* Vc(int l) const { return kv.p + static_cast<size_t>(2 * l + 1) * kKVH * kCap * kHd; }

    void create(const std::unordered_map<std::string, Tensor>& t, uint32_t nlayers) {
        layers = nlayers ? static_cast<int>(nlayers) : 28;
        if (layers < 1 || layers > 28) throw std::invalid_argument("Unsupported Qwen layer count");
        auto get = [&](const std::string& name, std::vector<int64_t> shape) -> const float* {
            auto it = t.find(name);
            if (it == t.end()) throw std::runtime_error("Missing tensor: " + name);
            if (it->second.shape != shape) throw std::invalid_argument("Unsupported Qwen shape: " + name);
            return it->second.data;
        };
        // qwen.cpp:7-13, in its order; then the norm weights run() reads
        const float* E = get("qwen.model.embed_tokens.weight", {kV, kD});
        struct LW {
            const float *q, *k, *v, *o, *qn, *kn, *g, *u, *d, *in, *post;
        };
        std::vector<LW> lw(layers);
        for (int i = 0; i < layers; ++i) {
            const std::string p = "qwen.model.layers." + std::to_string(i);
            LW& w = lw[i];
            w.q = get(p + ".self_attn.q_proj.weight", {kQ, kD});
            w.k = get(p + ".self_attn.k_proj.weight", {kKV, kD});
            w.v = get(p + ".self_attn.v_proj.weight", {kKV, kD});
            w.o = get(p + ".self_attn.o_proj.weight", {kD, kQ});
            w.qn = get(p + ".self_attn.q_norm.weight", {kHd});
            w.kn = get(p + ".self_attn.k_norm.weight", {kHd});
            w.g = get(p + ".mlp.gate_proj.weight", {kF, kD});
            w.u = get(p + ".mlp.up_proj.weight", {kF, kD});
            w.d = get(p + ".mlp.down_proj.weight", {kD, kF});
        }
        for (int i = 0; i < layers; ++i) {
            const std::string p = "qwen.model.layers." + std::to_string(i);
            lw[i].in = get(p + ".input_layernorm.weight", {kD});
            lw[i].post = get(p + ".post_attention_layernorm.weight", {kD});
        }
        const float* fin = get("qwen.model.norm.weight", {kD});

        QWEN_CHECK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
        for (auto& e : ev) QWEN_CHECK(hipEventCreate(&e));
        QWEN_CHECK(hipEventCreateWithFlags(&up_done, hipEventDisableTiming));
        QWEN_CHECK(hipHostMalloc(&pinned, sizeof(HostStage), hipHostMallocDefault));
        const char* env = std::getenv("ITTS_QWEN_GRAPHS");
        use_graphs = !(env && std::strcmp(env, "0") == 0);

        slab.alloc(static_cast<size_t>(layers) * kLayerFloats);
        std::vector<float> host(kLayerFloats);
        for (int i = 0; i < layers; ++i) {
            const LW& w = lw[i];
            float* hp = host.data();
            std::memcpy(hp, w.q, sizeof(float) * kQ * kD);
            std::memcpy(hp + size_t(kQ) * kD, w.k, sizeof(float) * kKV * kD);
            std::memcpy(hp + size_t(kQ + kKV) * kD, w.v, sizeof(float) * kKV * kD);
            std::memcpy(hp + kOffO, w.o, sizeof(float) * kD * kQ);
            for (int r = 0; r < kF; ++r) {
                std::memcpy(hp + kOffGu + size_t(2 * r) * kD, w.g + size_t(r) * kD, sizeof(float) * kD);
                std::memcpy(hp + kOffGu + size_t(2 * r + 1) * kD, w.u + size_t(r) * kD, sizeof(float) * kD);
            }
            std::memcpy(hp + kOffD, w.d, sizeof(float) * kD * kF);
            QWEN_CHECK(hipMemcpy(slab.p + static_cast<size_t>(i) * kLayerFloats, hp, sizeof(float) * kLayerFloats, hipMemcpyHostToDevice));
        }
        embed.alloc(static_cast<size_t>(kV) * kD);
        QWEN_CHECK(hipMemcpy(embed.p, E, sizeof(float) * kV * kD, hipMemcpyHostToDevice));
        std::vector<float> nh(static_cast<size_t>(layers) * kNormLayer + kD);
        for (int i = 0; i < layers; ++i) {
            float* np = nh.data() + static_cast<size_t>(i) * kNormLayer;
            std::memcpy(np + kNormIn, lw[i].in, sizeof(float) * kD);
            std::memcpy(np + kNormPost, lw[i].post, sizeof(float) * kD);
            std::memcpy(np + kNormQ, lw[i].qn, sizeof(float) * kHd);
            std::memcpy(np + kNormK, lw[i].kn, sizeof(float) * kHd);
        }
        std::memcpy(nh.data() + static_cast<size_t>(layers) * kNormLayer, fin, sizeof(float) * kD);
        norms.alloc(nh.size());
        QWEN_CHECK(hipMemcpy(norms.p, nh.data(), sizeof(float) * nh.size(), hipMemcpyHostToDevice));
        // qwen_rope's frequencies, pow(1e6, -j / 64) for j < 64 (kernels.metal:3113), formed
        // once on the host in float
        std::vector<float> f(64);
        for (int j = 0; j < 64; ++j) f[j] = std::pow(1000000.0f, -static_cast<float>(j) / 64.0f);
        inv_freq.alloc(64);
        QWEN_CHECK(hipMemcpy(inv_freq.p, f.data(), sizeof(float) * 64, hipMemcpyHostToDevice));
        std::vector<float> z(2 * kF, 0.0f);
        zeros.alloc(z.size());
        QWEN_CHECK(hipMemcpy(zeros.p, z.data(), sizeof(float) * z.size(), hipMemcpyHostToDevice));

        kv.alloc(static_cast<size_t>(layers) * 2 * kKVH * kCap * kHd);
        h.alloc(kD);
        qkv.alloc(kQkvN);
        ff.alloc(kF);
        logits.alloc(kV);
        part_acc.alloc(static_cast<size_t>(kMaxSplits) * kQH * kHd);
        part_ml.alloc(static_cast<size_t>(kMaxSplits) * kQH * 2);
        att.alloc(kQ);
        best.alloc(kHeadBlocks);
        st.alloc(1);
        toks.alloc(kMaxGen);
        ids.alloc(kPrompt);
        QWEN_CHECK(hipDeviceSynchronize());
    }

    void ensure_prefill(int P) {
        if (P <= pcap) return;
        const int cap = std::max(P, 256);
        X.alloc(static_cast<size_t>(cap) * kD);
        Xn.alloc(static_cast<size_t>(cap) * kD);
        QKV.alloc(static_cast<size_t>(cap) * kQkvN);
        Qp.alloc(static_cast<size_t>(cap) * kQ);
        ATT.alloc(static_cast<size_t>(cap) * kQ);
        FF.alloc(static_cast<size_t>(cap) * kF);
        if (!ws.p) ws.alloc(kGemmWsFloats);
        pcap = cap;
    }

    // The device state from the host: the pinned source is rewritten only after the previous
    // copy out of it has run.
    void set_state(const QState& s) {
        if (up_pending) QWEN_CHECK(hipEventSynchronize(up_done));
        pinned->up = s;
        QWEN_CHECK(hipMemcpyAsync(st.p, &pinned->up, sizeof(QState), hipMemcpyHostToDevice, stream));
        QWEN_CHECK(hipEventRecord(up_done, stream));
        up_pending = true;
    }

    void gemm(const float* A, const float* Wt, int M, int Nn, int Kk, float* C, int epi) {
        GemmArgs g{};
        g.a = A;
        g.w = Wt;
        g.bias = zeros.p;
        g.M = M;
        g.N = Nn;
        g.K = Kk;
        g.c = C;
        g.splits = gemm_splits(M, Nn, Kk);
        g.ws = ws.p;
        QWEN_CHECK(launch_gemm(g, epi, false, stream));
    }

    // The head on one row x (RMSNorm with the final weight, logits, workgroup bests) and the
    // token pick advancing the state by `advance` cache rows.
    void enqueue_head(const float* x, uint32_t advance) {
        QGemvArgs a{};
        a.w = embed.p;
        a.rows = kV;
        a.x = x;
        a.norm_w = norms.p + static_cast<size_t>(layers) * kNormLayer;
        a.out = logits.p;
        a.best = best.p;
        a.st = st.p;
        gemv<kD, kHeadRpw, kProRms, kEpiArgmax>(a, stream);
        QArgmaxArgs m{best.p, kHeadBlocks, st.p, toks.p, advance};
        hipLaunchKernelGGL(q_argmax_kernel, dim3(1), dim3(1024), 0, stream, m);
        QWEN_CHECK(hipGetLastError());
    }

    // qwen.cpp:23-45 for P prompt ids already in `ids`, at cache rows 0..P-1.
    void enqueue_prefill(int P) {
        ensure_prefill(P);
        hipStream_t s = stream;
        hipLaunchKernelGGL(q_embed_rows_kernel, dim3(P), dim3(256), 0, s, embed.p, ids.p, X.p);
        QWEN_CHECK(hipGetLastError());
        for (int l = 0; l < layers; ++l) {
            const float* w = W(l);
            hipLaunchKernelGGL(q_rms_rows_kernel, dim3(P), dim3(256), 0, s, X.p, N(l) + kNormIn, Xn.p);
            QWEN_CHECK(hipGetLastError());
            gemm(Xn.p, w, P, kQkvN, kD, QKV.p, kGemmStore);
            QPrepArgs pa{QKV.p, P, Qp.p, K(l), Vc(l), N(l) + kNormQ, N(l) + kNormK, inv_freq.p, nullptr};
            hipLaunchKernelGGL(q_prep_kernel, dim3(P, kQH + 2 * kKVH), dim3(64), 0, s, pa);
            QWEN_CHECK(hipGetLastError());
            QCausalArgs ca{Qp.p, K(l), Vc(l), ATT.p, P};
            hipLaunchKernelGGL(q_causal_attn_kernel, dim3(P, kQH), dim3(64), 0, s, ca);
            QWEN_CHECK(hipGetLastError());
            gemm(ATT.p, w + kOffO, P, kD, kQ, X.p, kGemmResid);
            hipLaunchKernelGGL(q_rms_rows_kernel, dim3(P), dim3(256), 0, s, X.p, N(l) + kNormPost, Xn.p);
            QWEN_CHECK(hipGetLastError());
            gemm(Xn.p, w + kOffGu, P, 2 * kF, kD, FF.p, kGemmSwiglu);
            gemm(FF.p, w + kOffD, P, kD, kF, X.p, kGemmResid);
        }
        enqueue_head(X.p + static_cast<size_t>(P - 1) * kD, static_cast<uint32_t>(P));
    }

    // One decode step for the state's token at row st.cached.
    void enqueue_step() {
        hipStream_t s = stream;
        for (int l = 0; l < layers; ++l) {
            const float* w = W(l);
            QGemvArgs a{};
            a.st = st.p;
            a.w = w;
            a.rows = kQkvN;
            a.x = h.p;
            a.norm_w = N(l) + kNormIn;
            a.embed = embed.p;
            a.h_out = h.p;
            a.out = qkv.p;
            if (l == 0) gemv<kD, 2, kProEmbedRms, kEpiStore>(a, s);
            else gemv<kD, 2, kProRms, kEpiStore>(a, s);
            QAttnArgs aa{qkv.p, K(l), Vc(l), N(l) + kNormQ, N(l) + kNormK, inv_freq.p, part_acc.p, part_ml.p, att.p, st.p};
            hipLaunchKernelGGL(q_attn_kernel, dim3(kAttnGrid), dim3(256), 0, s, aa);
            QWEN_CHECK(hipGetLastError());
            hipLaunchKernelGGL(q_attn_merge_kernel, dim3(kQH), dim3(kHd), 0, s, aa);
            QWEN_CHECK(hipGetLastError());
            QGemvArgs o{};
            o.st = st.p;
            o.w = w + kOffO;
            o.rows = kD;
            o.x = att.p;
            o.out = h.p;
            o.resid = h.p;
            gemv<kQ, 1, kProNone, kEpiResid>(o, s);
            QGemvArgs gu{};
            gu.st = st.p;
            gu.w = w + kOffGu;
            gu.rows = 2 * kF;
            gu.x = h.p;
            gu.norm_w = N(l) + kNormPost;
            gu.out = ff.p;
            gemv<kD, 2, kProRms, kEpiSwiglu>(gu, s);
            QGemvArgs d{};
            d.st = st.p;
            d.w = w + kOffD;
            d.rows = kD;
            d.x = ff.p;
            d.out = h.p;
            d.resid = h.p;
            gemv<kF, 1, kProNone, kEpiResid>(d, s);
        }
        enqueue_head(h.p, 1);
    }

    void run_step() {
        if (!use_graphs) {
            enqueue_step();
            return;
        }
        if (!step_graph) {
            hipGraph_t g = nullptr;
            QWEN_CHECK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
            try {
                enqueue_step();
            } catch (...) {
                (void)hipStreamEndCapture(stream, &g);
                if (g) (void)hipGraphDestroy(g);
                throw;
            }
            QWEN_CHECK(hipStreamEndCapture(stream, &g));
            const hipError_t e = hipGraphInstantiate(&step_graph, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            QWEN_CHECK(e);
        }
        QWEN_CHECK(hipGraphLaunch(step_graph, stream));
    }

    static void check_prompt(const uint32_t* p, uint32_t n) {
        if (n == 0 || n > static_cast<uint32_t>(kPrompt) || !p) throw std::invalid_argument("Qwen prompt capacity is 3072 tokens");
    }
    static void check_ids(const uint32_t* p, uint32_t n) {
        for (uint32_t i = 0; i < n; ++i)
            if (p[i] >= static_cast<uint32_t>(kV)) throw std::invalid_argument("Invalid Qwen token");
    }

    void upload_ids(const uint32_t* p, uint32_t n) {
        QWEN_CHECK(hipMemcpyAsync(ids.p, p, n * sizeof(uint32_t), hipMemcpyHostToDevice, stream));
    }

    void prefill(const uint32_t* p, uint32_t n, float* out) {
        check_prompt(p, n);
        check_ids(p, n);
        upload_ids(p, n);
        set_state(QState{0, 0, 0, 1, 1, 0, 0, 0});
        enqueue_prefill(static_cast<int>(n));
        QWEN_CHECK(hipMemcpyAsync(out, logits.p, sizeof(float) * kV, hipMemcpyDeviceToHost, stream));
        QWEN_CHECK(hipStreamSynchronize(stream));
        cached = n;
        ++submissions;
    }

    void step(uint32_t id, float* out) {
        if (!cached || cached >= static_cast<uint32_t>(kCap)) throw std::invalid_argument("Qwen cache capacity exceeded");
        if (id >= static_cast<uint32_t>(kV)) throw std::invalid_argument("Invalid Qwen token");
        set_state(QState{id, cached, 0, 1, 1, 0, 0, 0});
        run_step();
        QWEN_CHECK(hipMemcpyAsync(out, logits.p, sizeof(float) * kV, hipMemcpyDeviceToHost, stream));
        QWEN_CHECK(hipStreamSynchronize(stream));
        ++cached;
        ++submissions;
    }

    void generate(const uint32_t* p, uint32_t n, uint32_t maximum, uint32_t* out, uint32_t* count) {
        if (!maximum || maximum > static_cast<uint32_t>(kMaxGen) || static_cast<uint64_t>(n) + maximum > static_cast<uint64_t>(kCap))
            throw std::invalid_argument("Qwen generation capacity exceeded");
        check_prompt(p, n);
        check_ids(p, n);
        if (!out) throw std::invalid_argument("Qwen generation capacity exceeded");
        if (use_graphs && !step_graph) {  // captured before any work of this call is queued
            set_state(QState{0, 0, 0, 0, 1, 0, 0, 0});
            run_step();
        }
        upload_ids(p, n);
        set_state(QState{0, 0, 0, 1, maximum, 0, 0, 0});
        enqueue_prefill(static_cast<int>(n));
        // greedy steps, 16 replays at a time; a replay after the stop does nothing
        constexpr uint32_t kChunk = 16;
        uint32_t launched = 0;
        int k = 0;
        while (launched + 1 < maximum) {
            const uint32_t c = std::min(kChunk, maximum - 1 - launched);
            for (uint32_t i = 0; i < c; ++i) run_step();
            launched += c;
            QWEN_CHECK(hipMemcpyAsync(&pinned->flag[k & 1], &st.p->active, 4, hipMemcpyDeviceToHost, stream));
            QWEN_CHECK(hipEventRecord(ev[k & 1], stream));
            if (k >= 1) {
                QWEN_CHECK(hipEventSynchronize(ev[(k - 1) & 1]));
                if (!pinned->flag[(k - 1) & 1]) break;
            }
            ++k;
        }
        QWEN_CHECK(hipMemcpyAsync(&pinned->down, st.p, sizeof(QState), hipMemcpyDeviceToHost, stream));
        QWEN_CHECK(hipStreamSynchronize(stream));
        const QState s = pinned->down;
        *count = std::min(s.count, maximum);
        QWEN_CHECK(hipMemcpy(out, toks.p, sizeof(uint32_t) * *count, hipMemcpyDeviceToHost));
        cached = n + *count - 1;
        submissions += *count;
        if (!s.eos) throw std::runtime_error("Qwen did not reach EOS within 1024 generated tokens");
    }

    void bench(uint32_t prompt, uint32_t rows, uint32_t iters, float* prefill_ms, float* step_us) {
        if (prompt < 1 || prompt > static_cast<uint32_t>(kPrompt) || rows < 1 || !iters ||
            static_cast<uint64_t>(rows) + iters + 2 > static_cast<uint64_t>(kCap))
            throw std::invalid_argument("Invalid Qwen benchmark request");
        std::vector<uint32_t> p(prompt);
        for (uint32_t i = 0; i < prompt; ++i) p[i] = (i * 2654435761u) % static_cast<uint32_t>(kV);
        upload_ids(p.data(), prompt);
        set_state(QState{0, 0, 0, 1, 1, 0, 0, 0});
        enqueue_prefill(static_cast<int>(prompt));  // warm-up
        set_state(QState{0, 0, 0, 1, 1, 0, 0, 0});
        QWEN_CHECK(hipEventRecord(ev[0], stream));
        enqueue_prefill(static_cast<int>(prompt));
        QWEN_CHECK(hipEventRecord(ev[1], stream));
        QWEN_CHECK(hipEventSynchronize(ev[1]));
        QWEN_CHECK(hipEventElapsedTime(prefill_ms, ev[0], ev[1]));
        set_state(QState{1, rows, 0, 1, 0xffffffffu, 0, 1, 0});
        run_step();
        run_step();
        QWEN_CHECK(hipEventRecord(ev[0], stream));
        for (uint32_t i = 0; i < iters; ++i) run_step();
        QWEN_CHECK(hipEventRecord(ev[1], stream));
        QWEN_CHECK(hipEventSynchronize(ev[1]));
        float ms = 0;
        QWEN_CHECK(hipEventElapsedTime(&ms, ev[0], ev[1]));
        *step_us = 1000.0f * ms / static_cast<float>(iters);
        cached = 0;  // the cache holds benchmark rows
    }
};

}  // namespace qwen
}  // namespace itts

struct itts_qwen {
    itts::qwen::Engine e;
};

namespace {
thread_local std::string g_qwen_create_error;

template <class F>
int qwen_guarded(itts_qwen* q, F&& f) {
    try {
        f();
        return ITTS_OK;
    } catch (const std::invalid_argument& e) {
        (q ? q->e.last_error : g_qwen_create_error) = e.what();
        return ITTS_EINVAL;
    } catch (const std::runtime_error& e) {
        (q ? q->e.last_error : g_qwen_create_error) = e.what();
        return ITTS_ERUNTIME;
    } catch (const std::exception& e) {
        (q ? q->e.last_error : g_qwen_create_error) = e.what();
        return ITTS_ELOGIC;
    }
}

int qwen_create(const std::unordered_map<std::string, itts::qwen::Tensor>& t, const itts_qwen_config* cfg, itts_qwen** out) {
    if (!out) return ITTS_EINVAL;
    *out = nullptr;
    auto q = std::make_unique<itts_qwen>();
    const int st = qwen_guarded(nullptr, [&] { q->e.create(t, cfg ? cfg->layers : 0); });
    if (st == ITTS_OK) *out = q.release();
    return st;
}
}  // namespace

extern "C" {

int itts_qwen_create(const itts_tensor* tensors, int32_t count, const itts_qwen_config* cfg, itts_qwen** out) {
    std::unordered_map<std::string, itts::qwen::Tensor> t;
    for (int32_t i = 0; tensors && i < count; ++i) {
        const itts_tensor& x = tensors[i];
        if (!x.name || !x.data || x.ndim < 0 || x.ndim > 4) {
            g_qwen_create_error = "Invalid tensor table";
            return ITTS_EINVAL;
        }
        t[x.name] = {x.data, std::vector<int64_t>(x.shape, x.shape + x.ndim)};
    }
    return qwen_create(t, cfg, out);
}

int itts_qwen_create_from_bundle(const itts_bundle* b, const itts_qwen_config* cfg, itts_qwen** out) {
    if (!b) {
        g_qwen_create_error = "Invalid bundle";
        return ITTS_EINVAL;
    }
    std::unordered_map<std::string, itts::qwen::Tensor> t;
    const int32_t n = itts_bundle_count(b);
    for (int32_t i = 0; i < n; ++i) {
        itts_bundle_tensor bt{};
        if (itts_bundle_tensor_at(b, i, &bt) != ITTS_OK) continue;
        const std::string name = bt.name;
        if (name.rfind("qwen.", 0) != 0 || bt.dtype != ITTS_DTYPE_F32) continue;
        t[name] = {static_cast<const float*>(bt.data), std::vector<int64_t>(bt.shape, bt.shape + bt.ndim)};
    }
    return qwen_create(t, cfg, out);
}

void itts_qwen_destroy(itts_qwen* q) { delete q; }

const char* itts_qwen_last_error(const itts_qwen* q) { return q ? q->e.last_error.c_str() : g_qwen_create_error.c_str(); }

int itts_qwen_prefill(itts_qwen* q, const uint32_t* ids, uint32_t n, float* logits) {
    if (!q) return ITTS_EINVAL;
    return qwen_guarded(q, [&] {
        if (!logits) throw std::invalid_argument("Qwen prompt capacity is 3072 tokens");
        q->e.prefill(ids, n, logits);
    });
}

int itts_qwen_step(itts_qwen* q, uint32_t id, float* logits) {
    if (!q) return ITTS_EINVAL;
    return qwen_guarded(q, [&] {
        if (!logits) throw std::invalid_argument("Qwen cache capacity exceeded");
        q->e.step(id, logits);
    });
}

int itts_qwen_generate(itts_qwen* q, const uint32_t* ids, uint32_t n, uint32_t maximum, uint32_t* out, uint32_t* count) {
    if (!q || !count) return ITTS_EINVAL;
    *count = 0;
    return qwen_guarded(q, [&] { q->e.generate(ids, n, maximum, out, count); });
}

uint64_t itts_qwen_submissions(const itts_qwen* q) { return q ? q->e.submissions : 0; }

int itts_qwen_bench(itts_qwen* q, uint32_t prompt, uint32_t cached_rows, uint32_t iters, float* prefill_ms, float* step_us) {
    if (!q || !prefill_ms || !step_us) return ITTS_EINVAL;
    return qwen_guarded(q, [&] { q->e.bench(prompt, cached_rows, iters, prefill_ms, step_us); });
}

}  // extern "C"

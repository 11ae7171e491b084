// Persistent decode step: the whole 24-layer forward of one sequence (plus ln_f,
// final_norm and the mel_head GEMV) as ONE launch of one 512-thread workgroup per CU,
// instead of 6 launches per layer.
//
// Residency: the kernel needs > 128 VGPRs per thread, so a CU holds one of its
// workgroups at most, and the grid is the CU count: on a GPU with free CUs every
// workgroup is resident at once.  A plain launch is used rather than a cooperative one:
// ROCm grants cooperative launches to one process per GPU at a time, which would make
// a second process on the GPU fail.  Workgroups that start late (CUs held by other
// work) only delay the hand-offs; every wait is bounded and reports an error instead
// of hanging.
//
// Why: at batch 1 each GEMV launch carries 2.5-3 us of fixed cost (dispatch, first HBM
// round trip, end-of-kernel cache flush) and the step has ~146 of them, so the launch
// chain, not HBM, bounds the token rate.  Here a phase boundary is a data hand-off
// between workgroups instead of a kernel boundary:
//   * every value that crosses workgroups (h, q|k|v, attention partials, attention
//     output, hmid, ffn activations) is written as ONE 64-bit agent-scope atomic store
//     {float bits, epoch} and read with agent-scope atomic loads that are retried until
//     the epoch matches.  The tag makes each element self-validating: no counters, no
//     fences, no cache writeback/invalidate (a fence-based grid barrier costs ~14 us on
//     gfx950, a tagged hand-off ~2 us);
//   * each phase first issues the loads of its weight slice (registers), then waits for
//     its input vector, so the HBM stream overlaps the hand-off latency;
//   * a workgroup never waits for its own stores, so nothing drains the weight loads.
// Epochs: base + 8*layer + kind, with a fresh base per launch (host-side counter), so
// stale values from earlier launches or layers never match.  Each exchange vector has a
// single buffer: a producer of layer l+1's value can only run after every workgroup has
// consumed layer l's value (every phase consumes every producer of the phase before).
//
// Arithmetic is that of the multi-kernel path (decode.hip) operation for operation: the
// same per-row FMA order (lane l takes 16-byte chunks l, l+64, ... then a xor-butterfly),
// the same 4-wave LayerNorm reduction, the same split-KV attention tiles and merge, so
// logits are bitwise equal to it (the GPU tests check this).
//
// Reference ops replaced: gpt.cpp:88-125 (run on one step row), i.e. kernels.metal
// mit2_linear_gemv_f32 (1054-1080), mit2_layernorm_f32_rows (618-669),
// mit2_gpt_cached_attention_resident_f32 (2064-2145), mit2_gelu_f32 (486-503),
// mit2_add_f32 (161-171), mit2_gpt_build_current_f32 (1310-1324).
#include "kernels.h"

namespace itts {
namespace {

constexpr int kST = kStepThreads;  // 512
constexpr int kSW = kST / 64;       // waves per workgroup
constexpr int kSH = kST / 256;      // 256-thread attention groups per workgroup
constexpr unsigned kSpinLimit = 1u << 20;
// Rows per wave held in registers, per phase, for one workgroup per CU on 256 CUs
// (step_fits checks the grid against these).
constexpr int kRQkv = 2, kRProj = 1, kRFc = 3, kRFc2 = 1, kRHead = 5;

// Exchange layout (uint64 slots).
constexpr int kXh = 0;
constexpr int kXqkv = kXh + kWidth;
constexpr int kXattn = kXqkv + kQkv;
constexpr int kXhmid = kXattn + kWidth;
constexpr int kXff = kXhmid + kWidth;
constexpr int kXpart = kXff + kFfn;
static_assert(kXpart + kHeads * kAttnMaxSplits * 68 == kStepExchange, "exchange layout");
static_assert(kFfn % kST == 0 && kST >= 256 && kST % 256 == 0, "thread layout");

enum Kind : uint32_t { kEpXh = 0, kEpQkv = 1, kEpPart = 2, kEpAttn = 3, kEpHmid = 4, kEpFf = 5 };

__device__ __forceinline__ uint64_t xld(const uint64_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// base + 32-bit unsigned element offset (lets the compiler use a scalar base + one VGPR)
__device__ __forceinline__ uint64_t xld(const uint64_t* base, int off) { return xld(base + static_cast<uint32_t>(off)); }
__device__ __forceinline__ void xst(uint64_t* p, uint32_t epoch, float v) {
    __hip_atomic_store(p, (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Reads N tagged values (all loads issued first), retrying each until its epoch is `e`.
// A bounded wait: past kSpinLimit retries the error flag is raised and the thread stops
// waiting for the rest of the launch (the host reports the failure).
template <int N>
__device__ __forceinline__ void xread(const uint64_t* base, const int (&idx)[N], const bool (&use)[N], uint32_t e, float (&out)[N],
                                      uint32_t* err, bool& failed) {
    uint64_t v[N];
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = use[i] ? xld(base, idx[i]) : (static_cast<uint64_t>(e) << 32);
    // One retry loop for all N (per-element loops would each keep the caller's state live).
    unsigned spins = 0;
#pragma clang loop unroll(disable)
    while (true) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < N; ++i) ok &= static_cast<uint32_t>(v[i] >> 32) == e;
        if (ok) break;
        if (failed || ++spins > kSpinLimit) {
            if (!failed) atomicOr(err, 1u);
            failed = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int i = 0; i < N; ++i)
            if (static_cast<uint32_t>(v[i] >> 32) != e) v[i] = xld(base, idx[i]);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __uint_as_float(static_cast<uint32_t>(v[i]));
}

// threadIdx.x through an empty asm: per-thread offsets derived from it are recomputed in
// each phase instead of being hoisted out of the layer loop and held live across all phases.
__device__ __forceinline__ int opaque_tid() {
    int t = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(t)::"memory");
    return t;
}

// LayerNorm of one 1280-wide row held by threads 0..255 (value tid + 256 i), in the order
// of ln_block<1, 5> (common.h): wave butterfly, then the 4 wave partials in order.  Every
// thread of the workgroup calls it (it contains workgroup barriers).
__device__ __forceinline__ void ln256(float (&v)[5], const float* __restrict__ g, const float* __restrict__ be, float* red, int tid) {
    const int lane = tid & 63, wave = tid >> 6;
    const bool act = tid < 256;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 5; ++i) s += v[i];
    s = wave_sum(s);
    if (act && lane == 0) red[wave] = s;
    __syncthreads();
    const float mean = (((red[0] + red[1]) + red[2]) + red[3]) / float(kWidth);
    __syncthreads();
    s = 0.0f;
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const float d = v[i] - mean;
        s += d * d;
    }
    s = wave_sum(s);
    if (act && lane == 0) red[wave] = s;
    __syncthreads();
    const float var = (((red[0] + red[1]) + red[2]) + red[3]) / float(kWidth);
    const float inv = 1.0f / sqrtf(var + kLnEps);
    if (act) {
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int c = tid + 256 * i;
            v[i] = (v[i] - mean) * inv * g[c] + be[c];
        }
    }
    __syncthreads();
}

// Weight rows of this workgroup's slice, wave w holding local rows w, w+8, ... (MAXR of
// them), each as J 16-byte chunks per lane (chunk j*64 + lane of the row).
template <typename WT, int J, int MAXR>
struct Rows {
    using LD = WLoad<WT>;
    typename LD::vec w[MAXR][J];
    int r0, cnt;  // first global row of the slice, rows in the slice (may be <= 0)

    __device__ __forceinline__ void load(const WT* __restrict__ W, int rows, int wave, int lane) {
        const int per = (rows + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
        r0 = static_cast<int>(blockIdx.x) * per;
        cnt = min(per, rows - r0);
#pragma unroll
        for (int r = 0; r < MAXR; ++r) {
            const int lr = wave + kSW * r;
            if (lr < cnt) {
                const uint32_t row = static_cast<uint32_t>(r0 + lr);
#pragma unroll
                for (int j = 0; j < J; ++j) w[r][j] = LD::load(W, row * (J * 64) + static_cast<uint32_t>(j * 64 + lane));
            }
        }
    }
    // acc[r] = sum over the row of w * xs, in the multi-kernel GEMV's order.
    __device__ __forceinline__ void dot(const float* xs, float (&acc)[MAXR], int wave, int lane) const {
#pragma unroll
        for (int r = 0; r < MAXR; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const float4 x4 = *reinterpret_cast<const float4*>(xs + (j * 64 + lane) * 4);
#pragma unroll
            for (int r = 0; r < MAXR; ++r) {
                if (wave + kSW * r >= cnt) continue;
                const float4 w4 = LD::to_f4(w[r][j]);
                acc[r] = __builtin_fmaf(w4.x, x4.x, acc[r]);
                acc[r] = __builtin_fmaf(w4.y, x4.y, acc[r]);
                acc[r] = __builtin_fmaf(w4.z, x4.z, acc[r]);
                acc[r] = __builtin_fmaf(w4.w, x4.w, acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < MAXR; ++r) acc[r] = wave_sum(acc[r]);
    }
};

__device__ __forceinline__ int live_splits_dev(int L, int max_splits) {
    return min(max_splits, max(1, (L + kAttnSplitRows - 1) / kAttnSplitRows));
}

struct Smem {
    float xs[kFfn];      // phase input (normalised where a LayerNorm precedes the GEMV)
    float hraw[kWidth];  // layer input h (residual of attn.c_proj)
    float mraw[kWidth];  // hmid (residual of mlp.c_proj)
    float red[4];
    float redm[kSH][4], reds[kSH][4];
    float accs[kSH][16][kHeadDim + 4];
    float mwm[4], mwden[4];
    float mwnum[4][kHeadDim];
    float mpart[kAttnMaxSplits][2 + kHeadDim];  // gathered attention partials of one head
};

template <typename WT>
__global__ __launch_bounds__(kST) void step_kernel(StepArgs a) {
    __shared__ Smem sm;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const SeqState st = *a.state;
    if (!st.active) return;
    bool failed = false;
    const uint32_t n = st.n;
    const int L = static_cast<int>(n) + 1;
    const int S = live_splits_dev(L, a.splits);
    const int G = static_cast<int>(gridDim.x);
    const WT* __restrict__ W = static_cast<const WT*>(a.w);
    uint64_t* __restrict__ X = a.xch;
    const uint32_t e0 = a.epoch;
    auto ep = [&](int l, uint32_t kind) { return e0 + 8u * static_cast<uint32_t>(l) + kind; };

#pragma clang loop unroll(disable)
    for (int l = 0; l < a.layers; ++l) {
        const float* __restrict__ par = a.params + static_cast<size_t>(l) * kParLayer;
        const WT* __restrict__ wl = W + static_cast<size_t>(l) * a.layer_stride;
        const size_t kvl = static_cast<size_t>(l) * a.kv_layer_stride;

        // ------------------------------------------------ LN1 + c_attn (+ K/V append)
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            Rows<WT, kWidth / 256, kRQkv> R;
            R.load(wl, kQkv, wave, lane);
            float hv[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
            if (tid < 256) {
                if (l == 0) {
                    // h = mel_emb[token] + mel_pos[position] (gpt.cpp:79-85, kernels.metal:1310-1324)
#pragma unroll
                    for (int i = 0; i < 5; ++i) {
                        const int c = tid + 256 * i;
                        hv[i] = a.mel_emb[static_cast<size_t>(st.token) * kWidth + c] + a.mel_pos[static_cast<size_t>(st.position) * kWidth + c];
                    }
                } else {
                    int idx[5];
                    bool use[5];
#pragma unroll
                    for (int i = 0; i < 5; ++i) {
                        idx[i] = kXh + tid + 256 * i;
                        use[i] = true;
                    }
                    xread<5>(X, idx, use, ep(l, kEpXh), hv, a.err, failed);
                }
#pragma unroll
                for (int i = 0; i < 5; ++i) sm.hraw[tid + 256 * i] = hv[i];
            }
            ln256(hv, par + kParLn1W, par + kParLn1B, sm.red, tid);
            if (tid < 256) {
#pragma unroll
                for (int i = 0; i < 5; ++i) sm.xs[tid + 256 * i] = hv[i];
            }
            __syncthreads();
            float acc[kRQkv];
            R.dot(sm.xs, acc, wave, lane);
            const uint32_t e = ep(l, kEpQkv);
#pragma unroll
            for (int r = 0; r < kRQkv; ++r) {
                const int lr = wave + kSW * r;
                if (lr >= R.cnt || lane != 0) continue;
                const int row = R.r0 + lr;
                const float v = acc[r] + par[kParQkvB + row];
                xst(X + kXqkv + row, e, v);
                if (row >= kWidth) {
                    const int rr = row - kWidth;
                    const bool is_v = rr >= kWidth;
                    const int c = is_v ? rr - kWidth : rr;
                    a.kv[kvl + (is_v ? a.kv_v_off : 0) + (static_cast<size_t>(c >> 6) * a.kv_cap + n) * kHeadDim + (c & 63)] = v;
                }
            }
        }

        // ------------------------------------------------ split-KV attention tiles
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            const int ntiles = kHeads * S;
            const int quarter = tid >> 8, t = tid & 255, g = t >> 4, sub = t & 15, qw = (t >> 6);
            const int chunk = (L + S - 1) / S;
            const int rounds = (ntiles + kSH * G - 1) / (kSH * G);
            const uint32_t eq = ep(l, kEpQkv), epart = ep(l, kEpPart);
#pragma clang loop unroll(disable)
            for (int rd = 0; rd < rounds; ++rd) {
                const int tile = static_cast<int>(blockIdx.x) + G * (kSH * rd + quarter);
                const bool act = tile < ntiles;
                const int h = act ? tile % kHeads : 0, s = act ? tile / kHeads : 0;
                const int p0 = s * chunk, p1 = min(L, p0 + chunk);
                // 8 arithmetic slots as attention_kernel; a tile has <= 64 rows here (KV capacity
                // <= 4096, checked on the host), so only slots 0..3 can hold a row and slots
                // 4..7 stay constant zeros (-inf scores) exactly as in the multi-kernel path.
                constexpr int PER = kAttnMaxChunk / 16;
                constexpr int PERL = 4;
                float4 k4[PER], v4[PER];
                // cached rows first (no dependency on this step), the new row and q after
#pragma unroll
                for (int i = 0; i < PER; ++i) {
                    const int p = p0 + g + 16 * i;
                    if (i < PERL && act && p < p1 && p != static_cast<int>(n)) {
                        const size_t base = kvl + (static_cast<size_t>(h) * a.kv_cap + p) * kHeadDim + sub * 4;
                        k4[i] = *reinterpret_cast<const float4*>(a.kv + base);
                        v4[i] = *reinterpret_cast<const float4*>(a.kv + base + a.kv_v_off);
                    } else {
                        k4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                        v4[i] = k4[i];
                    }
                }
                // q and, in the tile holding it, the row appended by this step (row n): one
                // gather of tagged values each; row n sits at slot i_new of thread group g.
                const int dn = static_cast<int>(n) - p0 - g;
                const int i_new = (act && static_cast<int>(n) < p1 && dn >= 0 && (dn & 15) == 0 && (dn >> 4) < PERL) ? (dn >> 4) : -1;
                float4 q4 = make_float4(0.f, 0.f, 0.f, 0.f);
                {
                    int idx[12];
                    bool use[12];
                    float qv[12];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        idx[k] = kXqkv + h * kHeadDim + sub * 4 + k;
                        idx[4 + k] = kXqkv + kWidth + h * kHeadDim + sub * 4 + k;
                        idx[8 + k] = kXqkv + 2 * kWidth + h * kHeadDim + sub * 4 + k;
                        use[k] = act;
                        use[4 + k] = use[8 + k] = i_new >= 0;
                    }
                    xread<12>(X, idx, use, eq, qv, a.err, failed);
                    q4 = make_float4(qv[0], qv[1], qv[2], qv[3]);
                    const float4 kn = make_float4(qv[4], qv[5], qv[6], qv[7]);
                    const float4 vn = make_float4(qv[8], qv[9], qv[10], qv[11]);
#pragma unroll
                    for (int i = 0; i < PER; ++i) {
                        if (i == i_new) {
                            k4[i] = kn;
                            v4[i] = vn;
                        }
                    }
                }
                // scores, max-subtracted exp, partial sums: attention_kernel (decode.hip) op for op
                float sc[PER];
                float mloc = -INFINITY;
#pragma unroll
                for (int i = 0; i < PER; ++i) {
                    float d = q4.x * k4[i].x;
                    d = __builtin_fmaf(q4.y, k4[i].y, d);
                    d = __builtin_fmaf(q4.z, k4[i].z, d);
                    d = __builtin_fmaf(q4.w, k4[i].w, d);
                    d += __shfl_xor(d, 1, 64);
                    d += __shfl_xor(d, 2, 64);
                    d += __shfl_xor(d, 4, 64);
                    d += __shfl_xor(d, 8, 64);
                    const bool valid = i < PERL && act && p0 + g + 16 * i < p1;
                    sc[i] = valid ? d * 0.125f : -INFINITY;
                    mloc = fmaxf(mloc, sc[i]);
                }
                const float wm = wave_max(mloc);
                if (lane == 0) sm.redm[quarter][qw] = wm;
                __syncthreads();
                const float M = fmaxf(fmaxf(sm.redm[quarter][0], sm.redm[quarter][1]), fmaxf(sm.redm[quarter][2], sm.redm[quarter][3]));
                float lsum = 0.0f;
                float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int i = 0; i < PER; ++i) {
                    const bool valid = i < PERL && act && p0 + g + 16 * i < p1;
                    const float e = valid ? expf(sc[i] - M) : 0.0f;
                    lsum += e;
                    acc.x = __builtin_fmaf(e, v4[i].x, acc.x);
                    acc.y = __builtin_fmaf(e, v4[i].y, acc.y);
                    acc.z = __builtin_fmaf(e, v4[i].z, acc.z);
                    acc.w = __builtin_fmaf(e, v4[i].w, acc.w);
                }
                const float ws = wave_sum(sub == 0 ? lsum : 0.0f);
                if (lane == 0) sm.reds[quarter][qw] = ws;
                sm.accs[quarter][g][sub * 4 + 0] = acc.x;
                sm.accs[quarter][g][sub * 4 + 1] = acc.y;
                sm.accs[quarter][g][sub * 4 + 2] = acc.z;
                sm.accs[quarter][g][sub * 4 + 3] = acc.w;
                __syncthreads();
                if (act && t < kHeadDim) {
                    float tot = 0.0f;
#pragma unroll
                    for (int gg = 0; gg < 16; ++gg) tot += sm.accs[quarter][gg][t];
                    uint64_t* part = X + kXpart + (static_cast<size_t>(h) * kAttnMaxSplits + s) * 68;
                    xst(part + 4 + t, epart, tot);
                    if (t == 0) {
                        xst(part + 0, epart, M);
                        xst(part + 1, epart,
                            ((sm.reds[quarter][0] + sm.reds[quarter][1]) + sm.reds[quarter][2]) + sm.reds[quarter][3]);
                    }
                }
                __syncthreads();  // accs/redm are reused by the next round
            }
        }

        // ------------------------------------------------ merge of the splits of head h (workgroup h)
        if (static_cast<int>(blockIdx.x) < kHeads) {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            // All threads gather the S partial records (m, l, acc[64]) of head h into LDS,
            // then waves 0-3 merge them in the order of attention_merge_kernel (decode.hip).
            const int h = blockIdx.x;
            const uint64_t* pb = X + kXpart + static_cast<size_t>(h) * kAttnMaxSplits * 68;
            constexpr int kRec = 2 + kHeadDim;  // values used per record
            constexpr int NPT = (kAttnMaxSplits * kRec + kST - 1) / kST;
            {
                int idx[NPT];
                bool use[NPT];
                float v[NPT];
#pragma unroll
                for (int i = 0; i < NPT; ++i) {
                    const int q = tid + kST * i;  // record q / kRec, field q % kRec
                    const int k = q / kRec, f = q % kRec;
                    idx[i] = k * 68 + (f < 2 ? f : f + 2);
                    use[i] = k < S;
                }
                xread<NPT>(pb, idx, use, ep(l, kEpPart), v, a.err, failed);
#pragma unroll
                for (int i = 0; i < NPT; ++i) {
                    const int q = tid + kST * i;
                    if (use[i]) sm.mpart[q / kRec][q % kRec] = v[i];
                }
            }
            __syncthreads();
            const bool act = tid < 256;
            constexpr int PW = kAttnMaxSplits / 4;
            float mk[PW], lk[PW], ak[PW];
#pragma unroll
            for (int i = 0; i < PW; ++i) {
                const int k = wave + 4 * i;
                const bool ok = act && k < S;
                mk[i] = ok ? sm.mpart[k][0] : -INFINITY;
                lk[i] = ok ? sm.mpart[k][1] : 0.0f;
                ak[i] = ok ? sm.mpart[k][2 + lane] : 0.0f;
            }
            float m = -INFINITY;
#pragma unroll
            for (int i = 0; i < PW; ++i) m = fmaxf(m, mk[i]);
            if (act && lane == 0) sm.mwm[wave] = m;
            __syncthreads();
            const float mg = fmaxf(fmaxf(sm.mwm[0], sm.mwm[1]), fmaxf(sm.mwm[2], sm.mwm[3]));
            float den = 0.0f, num = 0.0f;
#pragma unroll
            for (int i = 0; i < PW; ++i) {
                const float wgt = mk[i] == -INFINITY ? 0.0f : expf(mk[i] - mg);
                den = __builtin_fmaf(lk[i], wgt, den);
                num = __builtin_fmaf(ak[i], wgt, num);
            }
            if (act) {
                sm.mwnum[wave][lane] = num;
                if (lane == 0) sm.mwden[wave] = den;
            }
            __syncthreads();
            if (wave == 0) {
                const float d = ((sm.mwden[0] + sm.mwden[1]) + sm.mwden[2]) + sm.mwden[3];
                const float nn = ((sm.mwnum[0][lane] + sm.mwnum[1][lane]) + sm.mwnum[2][lane]) + sm.mwnum[3][lane];
                xst(X + kXattn + h * kHeadDim + lane, ep(l, kEpAttn), nn / d);
            }
        }

        // ------------------------------------------------ attn.c_proj + residual
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            Rows<WT, kWidth / 256, kRProj> R;
            R.load(wl + static_cast<size_t>(kQkv) * kWidth, kWidth, wave, lane);
            {
                constexpr int NA = (kWidth + kST - 1) / kST;
                int idx[NA];
                bool use[NA];
                float v[NA];
#pragma unroll
                for (int i = 0; i < NA; ++i) {
                    idx[i] = kXattn + tid + kST * i;
                    use[i] = tid + kST * i < kWidth;
                }
                xread<NA>(X, idx, use, ep(l, kEpAttn), v, a.err, failed);
#pragma unroll
                for (int i = 0; i < NA; ++i)
                    if (use[i]) sm.xs[tid + kST * i] = v[i];
            }
            __syncthreads();
            float acc[kRProj];
            R.dot(sm.xs, acc, wave, lane);
            const uint32_t e = ep(l, kEpHmid);
#pragma unroll
            for (int r = 0; r < kRProj; ++r) {
                const int lr = wave + kSW * r;
                if (lr >= R.cnt || lane != 0) continue;
                const int row = R.r0 + lr;
                xst(X + kXhmid + row, e, sm.hraw[row] + (acc[r] + par[kParProjB + row]));
            }
        }

        // ------------------------------------------------ LN2 + c_fc + GELU
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            Rows<WT, kWidth / 256, kRFc> R;
            R.load(wl + static_cast<size_t>(kQkv + kWidth) * kWidth, kFfn, wave, lane);
            float hv[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
            if (tid < 256) {
                int idx[5];
                bool use[5];
#pragma unroll
                for (int i = 0; i < 5; ++i) {
                    idx[i] = kXhmid + tid + 256 * i;
                    use[i] = true;
                }
                xread<5>(X, idx, use, ep(l, kEpHmid), hv, a.err, failed);
#pragma unroll
                for (int i = 0; i < 5; ++i) sm.mraw[tid + 256 * i] = hv[i];
            }
            ln256(hv, par + kParLn2W, par + kParLn2B, sm.red, tid);
            if (tid < 256) {
#pragma unroll
                for (int i = 0; i < 5; ++i) sm.xs[tid + 256 * i] = hv[i];
            }
            __syncthreads();
            float acc[kRFc];
            R.dot(sm.xs, acc, wave, lane);
            const uint32_t e = ep(l, kEpFf);
#pragma unroll
            for (int r = 0; r < kRFc; ++r) {
                const int lr = wave + kSW * r;
                if (lr >= R.cnt || lane != 0) continue;
                const int row = R.r0 + lr;
                xst(X + kXff + row, e, gelu_f(acc[r] + par[kParFcB + row]));
            }
        }

        // ------------------------------------------------ mlp.c_proj + residual -> next h
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            Rows<WT, kFfn / 256, kRFc2> R;
            R.load(wl + static_cast<size_t>(kQkv + kWidth + kFfn) * kWidth, kWidth, wave, lane);
            {
                constexpr int NF = kFfn / kST;
                int idx[NF];
                bool use[NF];
                float v[NF];
#pragma unroll
                for (int i = 0; i < NF; ++i) {
                    idx[i] = kXff + tid + kST * i;
                    use[i] = true;
                }
                xread<NF>(X, idx, use, ep(l, kEpFf), v, a.err, failed);
#pragma unroll
                for (int i = 0; i < NF; ++i) sm.xs[tid + kST * i] = v[i];
            }
            __syncthreads();
            float acc[1];
            R.dot(sm.xs, acc, wave, lane);
            if (wave < R.cnt && lane == 0) {
                const int row = R.r0 + wave;
                xst(X + kXh + row, ep(l + 1, kEpXh), sm.mraw[row] + (acc[0] + par[kParFc2B + row]));
            }
        }
    }

    // ---------------------------------------------------- ln_f, final_norm, mel_head
    {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
        Rows<WT, kWidth / 256, kRHead> R;
        R.load(W + a.off_head, kMelVocab, wave, lane);
        float hv[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
        if (tid < 256) {
            int idx[5];
            bool use[5];
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                idx[i] = kXh + tid + 256 * i;
                use[i] = true;
            }
            xread<5>(X, idx, use, ep(a.layers, kEpXh), hv, a.err, failed);
        }
        ln256(hv, a.head + kHeadLnfW, a.head + kHeadLnfB, sm.red, tid);
        ln256(hv, a.head + kHeadFnW, a.head + kHeadFnB, sm.red, tid);
        if (tid < 256) {
#pragma unroll
            for (int i = 0; i < 5; ++i) sm.xs[tid + 256 * i] = hv[i];
        }
        __syncthreads();
        float acc[kRHead];
        R.dot(sm.xs, acc, wave, lane);
#pragma unroll
        for (int r = 0; r < kRHead; ++r) {
            const int lr = wave + kSW * r;
            if (lr >= R.cnt || lane != 0) continue;
            const int row = R.r0 + lr;
            a.logits[row] = acc[r] + a.head[kHeadBias + row];
        }
    }
}

}  // namespace

bool step_fits(int grid) {
    auto per = [&](int rows) { return (rows + grid - 1) / grid; };
    return grid > 0 && per(kQkv) <= kSW * kRQkv && per(kWidth) <= kSW * kRProj && per(kFfn) <= kSW * kRFc &&
           per(kWidth) <= kSW * kRFc2 && per(kMelVocab) <= kSW * kRHead && grid >= kHeads;
}

// FP32 weights only: the BF16 instantiation does not fit the register file without
// spilling, so BF16 decoders keep the multi-kernel path.
hipError_t step_occupancy(bool bf16, int* blocks_per_cu) {
    if (bf16) return hipErrorInvalidValue;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, step_kernel<float>, kST, 0);
}

hipError_t launch_step(const StepArgs& a, int grid, bool bf16, hipStream_t s) {
    if (bf16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(step_kernel<float>, dim3(grid), dim3(kST), 0, s, a);
    return hipGetLastError();
}

}  // namespace itts

// Persistent decode step: the whole 24-layer forward of one sequence (plus ln_f,
// final_norm and the mel_head GEMV) as ONE launch of one 512-thread workgroup per CU,
// instead of 6 launches per layer.
//
// Why: at batch 1 each GEMV launch carries 2.5-3 us of fixed cost (dispatch, first HBM
// round trip, end-of-kernel cache flush) and the multi-kernel step has 146 of them, so
// the launch chain, not HBM, bounds the token rate.
//
// Structure of a workgroup (one per CU):
//   * waves 4..7 are LOADERS: they walk this workgroup's whole weight stream for the step
//     (per layer: its rows of c_attn, the K/V rows of its attention tiles, its rows of
//     attn.c_proj, mlp.c_fc, mlp.c_proj; then its mel_head rows) in 5 KB chunks, load each
//     chunk into registers (2 chunks per loader wave in flight or waiting) and copy it into
//     a 24-chunk LDS ring as soon as its slot is free.  Loaders never wait on other
//     workgroups, and the register stage lets HBM keep streaming the next phase's rows
//     while the ring is full and the compute waves wait for a hand-off;
//   * waves 0..3 COMPUTE: they wait for each phase's input vector from the other
//     workgroups, form LayerNorms, take their rows' weights from the ring, and publish
//     outputs.  Row k of a phase slice belongs to compute wave k % 4; attention tiles use
//     all four waves;
//   * ring hand-shake, all in LDS: loader w publishes done[w] = (last chunk it landed)+1
//     (chunks w, w+4, w+8, ... are its own), compute wave c publishes need[c] = the first
//     chunk it may still read; a loader writes chunk x only when x < min(need) + 24.
//     A compute wave never waits for a chunk 24 or more past its own need, so a loader
//     blocked on ring space always has a compute wave able to move need forward.
// Hand-offs between workgroups: every value that crosses workgroups (h, q|k|v, attention
// partials, attention output, hmid, FFN activations) is ONE 64-bit agent-scope store
// {float bits, epoch}, read with agent-scope loads that are retried until the epoch
// matches.  The tag makes each element self-validating: no counters, fences or cache
// maintenance (a fence-based grid barrier measured ~14 us on gfx950, a tagged hand-off
// ~2 us).  Epochs: base + 8*layer + kind with a fresh base per launch, so stale values
// of earlier launches or layers never match.  One buffer per exchange vector suffices:
// a producer of layer l+1's value only runs after every workgroup consumed layer l's.
//
// Residency: 155 KB of LDS per workgroup allows one workgroup per CU and the grid is the
// CU count, so on a GPU with free CUs every workgroup is resident at once.  A plain
// launch is used rather than a cooperative one: ROCm grants cooperative launches to one
// process per GPU at a time, which would make a second process on the GPU fail.
// Workgroups that start late only delay the hand-offs; every wait is bounded and reports
// an error instead of hanging.
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
#include "sampler_dev.h"
#include "step_common.h"

namespace itts {
namespace {
using namespace stepc;

constexpr int kRing = 24;          // chunks in the LDS ring

// This workgroup's share of the step, identical in every wave.
struct Plan {
    int G, b;
    uint32_t n;  // cached rows before this step (the new row goes to row n)
    int L, S, ntiles, chunk_rows, rounds;
    int q0, qn, p0, pn, f0, fn, g0, gn, h0, hn;  // row slices: c_attn, c_proj, c_fc, mlp.c_proj, mel_head
    int att_chunks, layer_chunks;
    int o_att, o_proj, o_fc, o_fc2;  // chunk offsets inside a layer

    __device__ static void slice(int rows, int G, int b, int& r0, int& cnt) {
        const int per = (rows + G - 1) / G;
        r0 = b * per;
        cnt = max(0, min(per, rows - r0));
    }
    // Attention tile of round rd: head h, split s, first row t0, cached rows R (< n) in it.
    __device__ __forceinline__ bool tile(int rd, int& h, int& s, int& t0, int& R) const {
        const int t = b + G * rd;
        if (t >= ntiles) return false;
        h = t % kHeads;
        s = t / kHeads;
        t0 = s * chunk_rows;
        const int t1 = min(L, t0 + chunk_rows);
        R = max(0, min(t1, static_cast<int>(n)) - t0);
        return true;
    }
    __device__ __forceinline__ static int kv_chunks(int R) { return (R + kKvRowsPerChunk - 1) / kKvRowsPerChunk; }

    __device__ __forceinline__ void init(uint32_t n_, int splits) {
        G = static_cast<int>(gridDim.x);
        b = static_cast<int>(blockIdx.x);
        n = n_;
        L = static_cast<int>(n) + 1;
        S = live_splits_dev(L, splits);
        ntiles = kHeads * S;
        chunk_rows = (L + S - 1) / S;
        rounds = (ntiles + G - 1) / G;
        slice(kQkv, G, b, q0, qn);
        slice(kWidth, G, b, p0, pn);
        slice(kFfn, G, b, f0, fn);
        slice(kWidth, G, b, g0, gn);
        slice(kMelVocab, G, b, h0, hn);
        att_chunks = 0;
        for (int rd = 0; rd < rounds; ++rd) {
            int h, s, t0, R;
            if (tile(rd, h, s, t0, R)) att_chunks += 2 * kv_chunks(R);
        }
        o_att = qn;
        o_proj = o_att + att_chunks;
        o_fc = o_proj + pn;
        o_fc2 = o_fc + fn;
        layer_chunks = o_fc2 + 4 * gn;
    }
};

struct Smem {
    union {
        float xs[kFfn];                             // GEMV input of attn.c_proj and mlp.c_proj; ln_f output
        float mpart[kAttnMaxSplits][2 + kHeadDim];  // gathered attention partials of one head (merge)
    };
    float hraw[kWidth];  // layer input h (residual of attn.c_proj)
    float mraw[kWidth];  // hmid (residual of mlp.c_proj)
    float redm[4], reds[4];
    float accs[16][kHeadDim + 4];
};

// ------------------------------------------------------------------ loader waves

// Source of the 5 lines of chunk r of layer l of this workgroup's stream (l == layers:
// chunk r of its mel_head rows): a wave-uniform base, the chunk's extent in bytes from it,
// and the lane's byte offset of each line.  Line k of a chunk lands at ring line k, lane i's
// 16 bytes at +16 i.
__device__ __forceinline__ void chunk_src(const StepArgs& a, const Plan& P, const float* W, int l, int r, int lane,
                                          const float*& base, uint32_t& extent, uint32_t (&off)[kLines]) {
    if (l >= a.layers) {
        base = W + a.off_head + static_cast<size_t>(P.h0 + r) * kWidth;
    } else {
        const float* wl = W + static_cast<size_t>(l) * a.layer_stride;
        if (r < P.o_att) {
            base = wl + static_cast<size_t>(P.q0 + r) * kWidth;
        } else if (r < P.o_proj) {
            // attention tile chunks: K chunks 0..kc-1 then V chunks, 20 cached rows each,
            // lane l covers row 4 k + l / 16 of line k, 16 bytes (l % 16) of it
            int q = r - P.o_att, h = 0, s = 0, t0 = 0, R = 0, kc = 0;
            for (int rd = 0; rd < P.rounds; ++rd) {
                if (!P.tile(rd, h, s, t0, R)) continue;
                kc = Plan::kv_chunks(R);
                if (q < 2 * kc) break;
                q -= 2 * kc;
            }
            const bool is_v = q >= kc;
            const int j = is_v ? q - kc : q;
            const float* kvb = a.kv + static_cast<size_t>(l) * a.kv_layer_stride + (is_v ? a.kv_v_off : 0) +
                               static_cast<size_t>(h) * a.kv_cap * kHeadDim;
            base = kvb + static_cast<size_t>(t0) * kHeadDim;
            extent = static_cast<uint32_t>(R) * kHeadDim * 4;
#pragma unroll
            for (int k = 0; k < kLines; ++k) {
                int row = kKvRowsPerChunk * j + 4 * k + (lane >> 4);  // tile-local row
                if (row >= R) row = 0;                                 // clamped: loaded, never read
                off[k] = static_cast<uint32_t>((row * kHeadDim + (lane & 15) * 4) * 4);
            }
            return;
        } else if (r < P.o_fc) {
            base = wl + static_cast<size_t>(kQkv) * kWidth + static_cast<size_t>(P.p0 + r - P.o_proj) * kWidth;
        } else if (r < P.o_fc2) {
            base = wl + static_cast<size_t>(kQkv + kWidth) * kWidth + static_cast<size_t>(P.f0 + r - P.o_fc) * kWidth;
        } else {
            const int q = r - P.o_fc2;  // mlp.c_proj rows are 5120 wide: 4 chunks each
            base = wl + static_cast<size_t>(kQkv + kWidth + kFfn) * kWidth + static_cast<size_t>(P.g0 + (q >> 2)) * kFfn +
                   (q & 3) * kChunkF;
        }
    }
    extent = kChunkF * 4;
#pragma unroll
    for (int k = 0; k < kLines; ++k) off[k] = static_cast<uint32_t>((k * 256 + lane * 4) * 4);
}

// The batch-1 stream: chunk_src over this workgroup's Plan.
__device__ __forceinline__ void run_loader(const StepArgs& a, const Plan& P, float* ring, Ctl& ctl, int lw, int lane) {
    const float* __restrict__ W = static_cast<const float*>(a.w);
    stepc::run_loader<kRing>(a, P.layer_chunks, P.hn, ring, ctl, lw, lane,
                             [&](int l, int r, const float*& base, uint32_t& extent, uint32_t(&off)[kLines]) {
                                 chunk_src(a, P, W, l, r, lane, base, extent, off);
                             });
}

// ------------------------------------------------------------------ compute waves

// One group of a wave's rows of a 1280-wide GEMV slice: rows k0 + 4 t (t = 0..3, those
// below cnt), row k in ring chunk c0 + k.  The four dot products run interleaved and are
// reduced together (wave_sum4): row k0 + 4 t ends in lanes 0-15, 32-47, 16-31, 48-63 for
// t = 0, 1, 2, 3.  The group's chunks all come from one loader, which lands its chunks in
// order, so one poll (for the last) covers them; they span 13 < kRing chunks, so holding
// need at the first one cannot stall the loaders.
// N = 5: the same with a fifth row k0 + 16 (its chunks span 17 < kRing), reduced alone
// (wave_sum, every lane) into *fifth: a wave's last five rows in one pass instead of a
// group of four followed by a group of one.
template <int N>
__device__ __forceinline__ float rowsN(Ctl& ctl, const float* ring, int c0, int k0, int cnt, const XRow& xr, int wave, int lane,
                                       uint32_t* err, bool& failed, float* fifth) {
    static_assert(N == 4 || N == 5, "row group size");
    release_to(ctl, c0 + k0, wave);
    const int nt = N == 5 ? 5 : min(4, (cnt - k0 + 3) >> 2);  // rows present, >= 1
    (void)wait_chunk<kRing>(ctl, ring, c0 + k0 + 4 * (nt - 1), err, failed);
    const float* ch[N];
#pragma unroll
    for (int t = 0; t < N; ++t) ch[t] = ring + ((c0 + k0 + 4 * (t < nt ? t : 0)) % kRing) * kChunkF;  // absent rows re-read row k0
    // all reads first (the scheduler would otherwise issue each read right before its
    // FMAs and wait for it, one LDS round trip per read)
    float4 w[N][5];
#pragma unroll
    for (int j = 0; j < 5; ++j)
#pragma unroll
        for (int t = 0; t < N; ++t) w[t][j] = *reinterpret_cast<const float4*>(ch[t] + (j * 64 + lane) * 4);
    __builtin_amdgcn_sched_barrier(0);
    float acc[N];
#pragma unroll
    for (int t = 0; t < N; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int j = 0; j < 5; ++j) {
#pragma unroll
        for (int t = 0; t < N; ++t) {
            acc[t] = __builtin_fmaf(w[t][j].x, xr.x[j].x, acc[t]);
            acc[t] = __builtin_fmaf(w[t][j].y, xr.x[j].y, acc[t]);
            acc[t] = __builtin_fmaf(w[t][j].z, xr.x[j].z, acc[t]);
            acc[t] = __builtin_fmaf(w[t][j].w, xr.x[j].w, acc[t]);
        }
    }
    if constexpr (N == 5) *fifth = wave_sum(acc[4]);
    return wave_sum4(acc[0], acc[1], acc[2], acc[3]);
}

// Runs a wave's rows k = wave + 4 i (< cnt) of a 1280-wide GEMV slice whose row k sits in
// ring chunk c0 + k, against the input x in registers, four rows per reduction, and calls
// out(k, bias, sum) in the lane that holds row k's sum.  Groups g < NG take their bias from
// `bias`, later ones from bias_mem.
template <int NG, class Out>
__device__ __forceinline__ void gemv_rows(Ctl& ctl, const float* ring, int c0, int cnt, const XRow& xr, const LaneBias<NG, false>& bias,
                                          const float* __restrict__ bias_mem, int wave, int lane, uint32_t* err, bool& failed, Out out) {
    const int t = row_of_lane4(lane);
    const bool holder = (lane & 15) == 0;
    bool done = false;  // the previous group took this one's row as its fifth
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int k0 = wave + 16 * g;
        if (k0 < cnt && !done) {
            const int k = k0 + 4 * t;
            if (k0 + 16 < cnt && k0 + 20 >= cnt) {  // exactly five rows left
                float v5;
                const float v = rowsN<5>(ctl, ring, c0, k0, cnt, xr, wave, lane, err, failed, &v5);
                if (holder && k < cnt) out(k, bias.v[g], v);
                if (lane == 0) out(k0 + 16, g + 1 < NG ? bias.v[g + 1 < NG ? g + 1 : 0] : bias_mem[k0 + 16], v5);
                done = true;
            } else {
                const float v = rowsN<4>(ctl, ring, c0, k0, cnt, xr, wave, lane, err, failed, nullptr);
                if (holder && k < cnt) out(k, bias.v[g], v);
            }
        }
    }
    if (done) return;
    for (int k0 = wave + 16 * NG; k0 < cnt; k0 += 16) {
        const int k = k0 + 4 * t;
        if (k0 + 16 < cnt && k0 + 20 >= cnt) {
            float v5;
            const float v = rowsN<5>(ctl, ring, c0, k0, cnt, xr, wave, lane, err, failed, &v5);
            if (holder && k < cnt) out(k, bias_mem[k], v);
            if (lane == 0) out(k0 + 16, bias_mem[k0 + 16], v5);
            return;
        }
        const float v = rowsN<4>(ctl, ring, c0, k0, cnt, xr, wave, lane, err, failed, nullptr);
        if (holder && k < cnt) out(k, bias_mem[k], v);
    }
}

// Chunk m (1280 columns) of two 5120-wide rows: the input's 5 float4 and the rows' 10.
__device__ __forceinline__ void wide_load(const float* xs, const float* c0, const float* c1, int m, int lane, float4 (&x)[5],
                                          float4 (&w0)[5], float4 (&w1)[5]) {
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        x[j] = *reinterpret_cast<const float4*>(xs + ((5 * m + j) * 64 + lane) * 4);
        w0[j] = *reinterpret_cast<const float4*>(c0 + (j * 64 + lane) * 4);
        w1[j] = *reinterpret_cast<const float4*>(c1 + (j * 64 + lane) * 4);
    }
}
__device__ __forceinline__ void wide_fma(const float4 (&x)[5], const float4 (&w0)[5], const float4 (&w1)[5], float& a0, float& a1) {
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        a0 = __builtin_fmaf(w0[j].x, x[j].x, a0);
        a0 = __builtin_fmaf(w0[j].y, x[j].y, a0);
        a0 = __builtin_fmaf(w0[j].z, x[j].z, a0);
        a0 = __builtin_fmaf(w0[j].w, x[j].w, a0);
        a1 = __builtin_fmaf(w1[j].x, x[j].x, a1);
        a1 = __builtin_fmaf(w1[j].y, x[j].y, a1);
        a1 = __builtin_fmaf(w1[j].z, x[j].z, a1);
        a1 = __builtin_fmaf(w1[j].w, x[j].w, a1);
    }
}

// Two 5120-wide rows (mlp.c_proj) k0, k0 + 4 (the second if below cnt), row k in ring chunks
// c0 + 4 k + m, m = 0..3, reduced together (wave_sum2: lanes 0 and 32).  A pair's chunks
// span 20 < kRing.
__device__ __forceinline__ float rows2_wide(Ctl& ctl, const float* ring, int c0, int k0, int cnt, const float* xs, int wave, int lane,
                                            uint32_t* err, bool& failed) {
    const bool two = k0 + kCW < cnt;
    release_to(ctl, c0 + 4 * k0, wave);
    // chunks c .. c + 3 of the later row come from the four loaders: one poll of all four
    wait_run4(ctl, c0 + 4 * (two ? k0 + kCW : k0), err, failed);
    // the four 1280-column chunks in a two-stage pipeline: chunk m + 1's 15 LDS reads are in
    // flight while chunk m's FMAs run
    const float* c_0[4];
    const float* c_1[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        c_0[m] = ring + ((c0 + 4 * k0 + m) % kRing) * kChunkF;
        c_1[m] = two ? ring + ((c0 + 4 * (k0 + kCW) + m) % kRing) * kChunkF : c_0[m];
    }
    float4 xa[5], wa0[5], wa1[5], xb[5], wb0[5], wb1[5];
    float a0 = 0.0f, a1 = 0.0f;
    wide_load(xs, c_0[0], c_1[0], 0, lane, xa, wa0, wa1);
    wide_load(xs, c_0[1], c_1[1], 1, lane, xb, wb0, wb1);
    __builtin_amdgcn_sched_barrier(0);
    wide_fma(xa, wa0, wa1, a0, a1);
    __builtin_amdgcn_sched_barrier(0);
    wide_load(xs, c_0[2], c_1[2], 2, lane, xa, wa0, wa1);
    __builtin_amdgcn_sched_barrier(0);
    wide_fma(xb, wb0, wb1, a0, a1);
    __builtin_amdgcn_sched_barrier(0);
    wide_load(xs, c_0[3], c_1[3], 3, lane, xb, wb0, wb1);
    __builtin_amdgcn_sched_barrier(0);
    wide_fma(xa, wa0, wa1, a0, a1);
    __builtin_amdgcn_sched_barrier(0);
    wide_fma(xb, wb0, wb1, a0, a1);
    return wave_sum2(a0, a1);
}
template <int NG, class Out>
__device__ __forceinline__ void gemv_rows_wide(Ctl& ctl, const float* ring, int c0, int cnt, const float* xs, const LaneBias<NG, true>& bias,
                                               const float* __restrict__ bias_mem, int wave, int lane, uint32_t* err, bool& failed,
                                               Out out) {
    const int t = lane >> 5;
    const bool holder = (lane & 31) == 0;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int k0 = wave + 8 * g;
        if (k0 < cnt) {
            const float v = rows2_wide(ctl, ring, c0, k0, cnt, xs, wave, lane, err, failed);
            const int k = k0 + 4 * t;
            if (holder && k < cnt) out(k, bias.v[g], v);
        }
    }
    for (int k0 = wave + 8 * NG; k0 < cnt; k0 += 8) {
        const float v = rows2_wide(ctl, ring, c0, k0, cnt, xs, wave, lane, err, failed);
        const int k = k0 + 4 * t;
        if (holder && k < cnt) out(k, bias_mem[k], v);
    }
}

// Row groups per compute wave whose biases are prefetched, per phase: all of them for the
// slices of a 256-CU grid (15, 5, 20, 5 and 33 rows per workgroup).
constexpr int kGQkv = 1, kGProj = 1, kGFc = 2, kGFc2 = 1, kGHead = 3;
// Attention merges of at most this many splits run from registers (KV up to 1024 rows).
constexpr int kMergeRegSplits = 16;

// The workgroup's LDS: the weight ring and the phase buffers while the step runs; the
// sampler's buffers in the fused sampling tail, after every wave is done with the former.
struct StepLds {
    float ring[kRing * kChunkF];
    Smem sm;
};
union StepTailLds {
    StepLds step;
    sampling::SmemT<kST> samp;
};

// The fused sampling tail (gpt_sampling.cpp:168-189 for the step's token), run by all eight
// waves of every workgroup after their last step work.  Each workgroup has stored its
// mel_head rows also as tagged exchange slots {logit, epoch}; it counts itself in, and the
// last to arrive (nobody waits for a count) reads the whole row from those slots (re-reading
// any slot whose tag is not yet this launch's, with the bounded wait of every hand-off) and
// samples from it exactly as sampler_kernel does, with its 512 threads, then resets the
// counter for the next launch.  The tags make the data's arrival explicit, so no device-wide
// fence (an L2 write-back) is needed.  This replaces a separate sampler launch per token.
__device__ inline void sampling_tail(const StepArgs& a, Ctl& ctl, StepTailLds& lds, uint32_t e) {
    if (!a.tail) return;
    __syncthreads();  // the second full barrier of the kernel: loaders and compute waves all here
    const int tid = threadIdx.x;
    if (tid == 0)
        ctl.last = __hip_atomic_fetch_add(a.tail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1 ? 1u : 0u;
    __syncthreads();
    if (!ctl.last) return;
    if (tid == 0) __hip_atomic_store(a.tail, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!a.state->active) return;
    auto& sm = lds.samp;
    constexpr int kPer = (kMelVocab + kST - 1) / kST;
    uint64_t v[kPer];
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const int i = tid + q * kST;
        v[q] = i < kMelVocab ? xld(a.xch + kXlogit + i) : (static_cast<uint64_t>(e) << 32);
    }
    bool failed = false;
    for (unsigned spins = 0;;) {
        bool ok = true;
#pragma unroll
        for (int q = 0; q < kPer; ++q) ok &= static_cast<uint32_t>(v[q] >> 32) == e;
        if (ok) break;
        if (++spins > kSpinLimit) {
            atomicOr(a.err, 1u);
            failed = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int i = tid + q * kST;
            if (static_cast<uint32_t>(v[q] >> 32) != e) v[q] = xld(a.xch + kXlogit + i);
        }
    }
    (void)failed;
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
        const int i = tid + q * kST;
        if (i < kMelVocab) sm.s[i] = __uint_as_float(static_cast<uint32_t>(v[q]));
    }
    __syncthreads();
    sampling::sample_loaded(sm, a.sample, 0);
}

__global__ __launch_bounds__(kST) void step_kernel(StepArgs a) {
    __shared__ StepTailLds lds;
    __shared__ Ctl ctl;
    float* ring = lds.step.ring;
    Smem& sm = lds.step.sm;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const SeqState st = *a.state;
    if (!st.active) return;
    if (tid < kLW) ctl.done[tid] = 0;
    if (tid < kCW) ctl.need[tid] = 0;
    if (tid == 0) {
        ctl.bar = 0;
        ctl.go = 0;
    }
    __syncthreads();  // the only barrier of the whole workgroup; roles split below

    Plan P;
    P.init(st.n, a.splits);
    const int total_chunks = a.layers * P.layer_chunks + P.hn;

    // ================================================================ loaders
    // They start once the compute waves hold layer 0's input row: requested first, those
    // loads do not queue behind the whole grid's first weight chunks (which held layer 0's
    // start back by 6-10 us).
    if (wave >= kCW) {
        wait_go(ctl, a.err);
        run_loader(a, P, ring, ctl, __builtin_amdgcn_readfirstlane(wave - kCW), lane);
        sampling_tail(a, ctl, lds, a.epoch + 8u * static_cast<uint32_t>(a.layers) + kEpLogit);
        return;
    }

    // h = mel_emb[token] + mel_pos[position] (gpt.cpp:79-85, kernels.metal:1310-1324)
    float h0[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const int c = tid + 256 * i;
        h0[i] = a.mel_emb[static_cast<size_t>(st.token) * kWidth + c] + a.mel_pos[static_cast<size_t>(st.position) * kWidth + c];
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    if (tid == 0) lds_st(&ctl.go, 1u);

    // ================================================================ compute waves
    bool failed = false;
    uint32_t gen = 0;
    uint64_t* __restrict__ X = a.xch;                             // copy 0: written by producers, partials
    const uint64_t* __restrict__ XB = a.xch + xcopy(P.b % kStepCopies, 0);  // this workgroup's copy for reading
    const uint32_t e0 = a.epoch;
    auto ep = [&](int l, uint32_t kind) { return e0 + 8u * static_cast<uint32_t>(l) + kind; };
    const uint32_t n = P.n;
    // phase-end clocks for measurement (one lane, only when the host asks for them)
    auto stamp = [&](int l, int k) {
        if (a.stamps && opaque_tid() == 0)
            a.stamps[(static_cast<size_t>(P.b) * (a.layers + 1) + l) * kStepStampsPerLayer + k] = __builtin_amdgcn_s_memrealtime();
    };

    for (int l = 0; l < a.layers; ++l) {
        const float* __restrict__ par = a.params + static_cast<size_t>(l) * kParLayer;
        const size_t kvl = static_cast<size_t>(l) * a.kv_layer_stride;
        const int cb = l * P.layer_chunks;  // first chunk of this layer
        stamp(l, 0);

        // ------------------------------------------------ LN1 + c_attn (+ K/V append)
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            release_to(ctl, cb, wave);
            // input loads in flight while this wave's c_attn rows move from the ring to registers
            int idx[5];
            bool use[5];
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                idx[i] = kXh + tid + 256 * i;
                use[i] = l > 0;
            }
            XRead<5> xr;
            if (l > 0) poll_delay();
            xr.issue(XB, idx, use, ep(l, kEpXh));
            LnParDot ln;
            ln.load(par + kParLn1W, par + kParLn1B, lane);
            LaneBias<kGQkv, false> bias;
            bias.load(par + kParQkvB + P.q0, P.qn, wave, lane);
            float hv[5];
            if (l == 0) {
#pragma unroll
                for (int i = 0; i < 5; ++i) hv[i] = h0[i];
            } else {
                xr.wait(XB, idx, ep(l, kEpXh), hv, a.err, failed);
            }
#pragma unroll
            for (int i = 0; i < 5; ++i) sm.hraw[tid + 256 * i] = hv[i];
            cbar(ctl, gen, a.err, failed);
            XRow x;
            {
                float v[4][5], mean, inv;
                ln_layout_load(sm.hraw, lane, v);
                ln_stats(v, mean, inv);
                ln_to_xrow(sm.hraw, lane, mean, inv, ln, x);
            }
            const uint32_t e = ep(l, kEpQkv);
            auto out = [&](int k, float b, float acc) {  // called by the lane holding row k's sum
                const int row = P.q0 + k;
                const float v = acc + b;
                xst_bcast(X, kXqkv + row, e, v);
                if (row >= kWidth) {
                    const int rr = row - kWidth;
                    const bool is_v = rr >= kWidth;
                    const int c = is_v ? rr - kWidth : rr;
                    a.kv[kvl + (is_v ? a.kv_v_off : 0) + (static_cast<size_t>(c >> 6) * a.kv_cap + n) * kHeadDim + (c & 63)] = v;
                }
            };
            gemv_rows(ctl, ring, cb, P.qn, x, bias, par + kParQkvB + P.q0, wave, lane, a.err, failed, out);
            stores_done();
        }
        stamp(l, 1);

        // ------------------------------------------------ split-KV attention tiles
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            const int g = tid >> 4, sub = tid & 15;
            const uint32_t eq = ep(l, kEpQkv), epart = ep(l, kEpPart);
            int ca = cb + P.o_att;  // first chunk of the current tile
            release_to(ctl, ca, wave);
            for (int rd = 0; rd < P.rounds; ++rd) {
                int h = 0, s = 0, t0 = 0, R = 0;
                const bool act = P.tile(rd, h, s, t0, R);
                const int p1 = act ? min(P.L, t0 + P.chunk_rows) : 0;
                const int kc = act ? Plan::kv_chunks(R) : 0;
                // 8 arithmetic slots as attention_kernel (rows g + 16 i of a tile of up to
                // kAttnMaxChunk rows); slots past the tile's rows are zeros with -inf scores,
                // exactly as in the multi-kernel path.  Slots 4-7 hold rows only in tiles of
                // more than 64 rows (caches past 768 rows; wide, uniform): other tiles run the
                // code with four slots, where those slots' -inf scores and zero weights, which
                // leave every sum unchanged, are dropped at compile time.
                constexpr int PER = kAttnMaxChunk / 16;
                const bool wide = act && p1 - t0 > 64;
                const int dn = static_cast<int>(n) - t0 - g;
                const int i_new = (act && static_cast<int>(n) < p1 && dn >= 0 && (dn & 15) == 0 && (dn >> 4) < PER) ? (dn >> 4) : -1;
                // q and, in the tile holding it, the row appended by this step (row n): loads in
                // flight while the cached rows move from the ring to registers
                int idx[12];
                bool use[12];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    idx[k] = kXqkv + h * kHeadDim + sub * 4 + k;
                    idx[4 + k] = kXqkv + kWidth + h * kHeadDim + sub * 4 + k;
                    idx[8 + k] = kXqkv + 2 * kWidth + h * kHeadDim + sub * 4 + k;
                    use[k] = act;
                    use[4 + k] = use[8 + k] = i_new >= 0;
                }
                XRead<12> xr;
                xr.issue(XB, idx, use, eq);
                float M = 0.0f, lsum = 0.0f;
                float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
                auto tile_math = [&](auto slots) {
                    constexpr int PERL = decltype(slots)::value;
                    float4 k4[PERL], v4[PERL];
#pragma unroll
                    for (int i = 0; i < PERL; ++i) {
                        k4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                        v4[i] = k4[i];
                    }
                    // cached rows from the ring; need stays at the tile's first chunk until its
                    // rows are in registers
                    for (int j = 0; j < 2 * kc; ++j) (void)wait_chunk<kRing>(ctl, ring, ca + j, a.err, failed);
#pragma unroll
                    for (int i = 0; i < PERL; ++i) {
                        const int r = g + 16 * i;  // tile-local row
                        if (act && r < R) {
                            const float* kch = ring + ((ca + r / kKvRowsPerChunk) % kRing) * kChunkF;
                            const float* vch = ring + ((ca + kc + r / kKvRowsPerChunk) % kRing) * kChunkF;
                            const int off = (r % kKvRowsPerChunk) * kHeadDim + sub * 4;
                            k4[i] = *reinterpret_cast<const float4*>(kch + off);
                            v4[i] = *reinterpret_cast<const float4*>(vch + off);
                        }
                    }
                    ca += 2 * kc;
                    release_to(ctl, ca, wave);  // this tile's chunks are in registers now
                    float4 q4;
                    {
                        float qv[12];
                        xr.wait(XB, idx, eq, qv, a.err, failed);
                        q4 = make_float4(qv[0], qv[1], qv[2], qv[3]);
                        const float4 kn = make_float4(qv[4], qv[5], qv[6], qv[7]);
                        const float4 vn = make_float4(qv[8], qv[9], qv[10], qv[11]);
#pragma unroll
                        for (int i = 0; i < PERL; ++i) {
                            if (i == i_new) {
                                k4[i] = kn;
                                v4[i] = vn;
                            }
                        }
                    }
                    // scores, max-subtracted exp, partial sums: attention_kernel (decode.hip) op for op
                    float sc[PERL];
                    float mloc = -INFINITY;
#pragma unroll
                    for (int i = 0; i < PERL; ++i) {
                        float d = q4.x * k4[i].x;
                        d = __builtin_fmaf(q4.y, k4[i].y, d);
                        d = __builtin_fmaf(q4.z, k4[i].z, d);
                        d = __builtin_fmaf(q4.w, k4[i].w, d);
                        d = sum16_up(d);
                        const bool valid = act && t0 + g + 16 * i < p1;
                        sc[i] = valid ? d * 0.125f : -INFINITY;
                        mloc = fmaxf(mloc, sc[i]);
                    }
                    const float wm = wave_max(mloc);
                    if (lane == 0) sm.redm[wave] = wm;
                    cbar(ctl, gen, a.err, failed);
                    M = fmaxf(fmaxf(sm.redm[0], sm.redm[1]), fmaxf(sm.redm[2], sm.redm[3]));
#pragma unroll
                    for (int i = 0; i < PERL; ++i) {
                        const bool valid = act && t0 + g + 16 * i < p1;
                        const float e = valid ? expf(sc[i] - M) : 0.0f;
                        lsum += e;
                        acc.x = __builtin_fmaf(e, v4[i].x, acc.x);
                        acc.y = __builtin_fmaf(e, v4[i].y, acc.y);
                        acc.z = __builtin_fmaf(e, v4[i].z, acc.z);
                        acc.w = __builtin_fmaf(e, v4[i].w, acc.w);
                    }
                };
                if (wide)
                    tile_math(std::integral_constant<int, PER>{});
                else
                    tile_math(std::integral_constant<int, PER / 2>{});
                const float ws = wave_sum(sub == 0 ? lsum : 0.0f);
                if (lane == 0) sm.reds[wave] = ws;
                sm.accs[g][sub * 4 + 0] = acc.x;
                sm.accs[g][sub * 4 + 1] = acc.y;
                sm.accs[g][sub * 4 + 2] = acc.z;
                sm.accs[g][sub * 4 + 3] = acc.w;
                cbar(ctl, gen, a.err, failed);
                if (act && tid < kHeadDim) {
                    float tot = 0.0f;
#pragma unroll
                    for (int gg = 0; gg < 16; ++gg) tot += sm.accs[gg][tid];
                    uint64_t* part = X + kXpart + (static_cast<size_t>(h) * kAttnMaxSplits + s) * 68;
                    xst(part + 4 + tid, epart, tot);
                    if (tid == 0) {
                        xst(part + 0, epart, M);
                        xst(part + 1, epart, ((sm.reds[0] + sm.reds[1]) + sm.reds[2]) + sm.reds[3]);
                    }
                }
                if (rd + 1 < P.rounds) cbar(ctl, gen, a.err, failed);  // redm/reds/accs are reused by the next round
            }
            release_to(ctl, cb + P.o_proj, wave);
            stores_done();
        }
        stamp(l, 2);

        // ------------------------------------------------ merge of the splits of head h (workgroup h)
        // In attention_merge_kernel's order (decode.hip): its wave w takes splits w, w+4, ...
        // and the four partial denominators and numerators are added in order.  Lane k
        // computes split k's weight exp(m_k - max m); the sums then run over k with the
        // weights broadcast from their lanes.  The maximum is exact in any order.
        if (P.b < kHeads && P.S <= kMergeRegSplits) {
            // up to 16 splits: wave 0 reads the records straight into registers (lane d holds
            // acc[k][d] for every k, lane k holds m_k and l_k) and merges them alone
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            if (wave == 0) {
                const int h = P.b, S = opaque_s(P.S);
                const uint64_t* pb = X + kXpart + static_cast<size_t>(h) * kAttnMaxSplits * 68;
                constexpr int NR = kMergeRegSplits + 2;
                int idx[NR];
                bool use[NR];
#pragma unroll
                for (int k = 0; k < kMergeRegSplits; ++k) {
                    idx[k] = k * 68 + 4 + lane;
                    use[k] = k < S;
                }
                idx[kMergeRegSplits] = lane * 68;
                idx[kMergeRegSplits + 1] = lane * 68 + 1;
                use[kMergeRegSplits] = use[kMergeRegSplits + 1] = lane < S;
                float v[NR];
                xread<NR>(pb, idx, use, ep(l, kEpPart), v, a.err, failed);
                const float mk = lane < S ? v[kMergeRegSplits] : -INFINITY;
                const float lk = lane < S ? v[kMergeRegSplits + 1] : 0.0f;
                const float mg = wave_max(mk);
                const float wk = mk == -INFINITY ? 0.0f : expf(mk - mg);
                float den[4] = {0.0f, 0.0f, 0.0f, 0.0f}, num[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int k = 0; k < kMergeRegSplits; ++k) {
                    if (k < S) {
                        const float wgt = lane_value(wk, k);
                        den[k & 3] = __builtin_fmaf(lane_value(lk, k), wgt, den[k & 3]);
                        num[k & 3] = __builtin_fmaf(v[k], wgt, num[k & 3]);
                    }
                }
                const float d = ((den[0] + den[1]) + den[2]) + den[3];
                const float nn = ((num[0] + num[1]) + num[2]) + num[3];
                xst_bcast(X, kXattn + h * kHeadDim + lane, ep(l, kEpAttn), nn / d);
                stores_done();
            }
        } else if (P.b < kHeads) {
            // more splits: the compute threads gather the records into LDS, wave 0 merges
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            const int h = P.b;
            const uint64_t* pb = X + kXpart + static_cast<size_t>(h) * kAttnMaxSplits * 68;
            constexpr int kRec = 2 + kHeadDim;  // values used per record
            constexpr int NPT = (kAttnMaxSplits * kRec + kCT - 1) / kCT;
            {
                int idx[NPT];
                bool use[NPT];
                float v[NPT];
#pragma unroll
                for (int i = 0; i < NPT; ++i) {
                    const int q = tid + kCT * i;  // record q / kRec, field q % kRec
                    const int k = q / kRec, f = q % kRec;
                    idx[i] = k * 68 + (f < 2 ? f : f + 2);
                    use[i] = k < P.S;
                }
                xread<NPT>(pb, idx, use, ep(l, kEpPart), v, a.err, failed);
#pragma unroll
                for (int i = 0; i < NPT; ++i) {
                    const int q = tid + kCT * i;
                    if (use[i]) sm.mpart[q / kRec][q % kRec] = v[i];
                }
            }
            cbar(ctl, gen, a.err, failed);
            if (wave == 0) {
                const int S = P.S;
                const float mk = lane < S ? sm.mpart[lane][0] : -INFINITY;
                const float lk = lane < S ? sm.mpart[lane][1] : 0.0f;
                const float mg = wave_max(mk);
                const float wk = mk == -INFINITY ? 0.0f : expf(mk - mg);
                float den[4] = {0.0f, 0.0f, 0.0f, 0.0f}, num[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int k0 = 0; k0 < S; k0 += 4) {
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        const int k = k0 + w;
                        if (k < S) {
                            const float wgt = lane_value(wk, k);
                            den[w] = __builtin_fmaf(lane_value(lk, k), wgt, den[w]);
                            num[w] = __builtin_fmaf(sm.mpart[k][2 + lane], wgt, num[w]);
                        }
                    }
                }
                const float d = ((den[0] + den[1]) + den[2]) + den[3];
                const float nn = ((num[0] + num[1]) + num[2]) + num[3];
                xst_bcast(X, kXattn + h * kHeadDim + lane, ep(l, kEpAttn), nn / d);
                stores_done();
            }
            cbar(ctl, gen, a.err, failed);  // mpart aliases xs, written below
        }
        stamp(l, 3);

        // ------------------------------------------------ attn.c_proj + residual
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            const int cp = cb + P.o_proj;
            int idx[5];
            bool use[5];
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                idx[i] = kXattn + tid + 256 * i;
                use[i] = true;
            }
            XRead<5> xr;
            poll_delay();
            xr.issue(XB, idx, use, ep(l, kEpAttn));
            LaneBias<kGProj, false> bias;
            bias.load(par + kParProjB + P.p0, P.pn, wave, lane);
            {
                float v[5];
                xr.wait(XB, idx, ep(l, kEpAttn), v, a.err, failed);
#pragma unroll
                for (int i = 0; i < 5; ++i) sm.xs[tid + 256 * i] = v[i];
            }
            cbar(ctl, gen, a.err, failed);
            XRow x;
            x.load(sm.xs, lane);
            const uint32_t e = ep(l, kEpHmid);
            auto out = [&](int k, float b, float acc) {
                const int row = P.p0 + k;
                xst_bcast(X, kXhmid + row, e, sm.hraw[row] + (acc + b));
            };
            gemv_rows(ctl, ring, cp, P.pn, x, bias, par + kParProjB + P.p0, wave, lane, a.err, failed, out);
            release_to(ctl, cb + P.o_fc, wave);
            stores_done();
        }
        stamp(l, 4);

        // ------------------------------------------------ LN2 + c_fc + GELU
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            const int cf = cb + P.o_fc;
            int idx[5];
            bool use[5];
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                idx[i] = kXhmid + tid + 256 * i;
                use[i] = true;
            }
            XRead<5> xr;
            poll_delay();
            xr.issue(XB, idx, use, ep(l, kEpHmid));
            LnParDot ln;
            ln.load(par + kParLn2W, par + kParLn2B, lane);
            LaneBias<kGFc, false> bias;
            bias.load(par + kParFcB + P.f0, P.fn, wave, lane);
            float hv[5];
            xr.wait(XB, idx, ep(l, kEpHmid), hv, a.err, failed);
#pragma unroll
            for (int i = 0; i < 5; ++i) sm.mraw[tid + 256 * i] = hv[i];
            cbar(ctl, gen, a.err, failed);  // also: every wave is past its c_proj reads of xs
            XRow x;
            {
                float v[4][5], mean, inv;
                ln_layout_load(sm.mraw, lane, v);
                ln_stats(v, mean, inv);
                ln_to_xrow(sm.mraw, lane, mean, inv, ln, x);
            }
            const uint32_t e = ep(l, kEpFf);
            auto out = [&](int k, float b, float acc) {
                const int row = P.f0 + k;
                xst_bcast(X, kXff + row, e, gelu_f(acc + b));
            };
            gemv_rows(ctl, ring, cf, P.fn, x, bias, par + kParFcB + P.f0, wave, lane, a.err, failed, out);
            release_to(ctl, cb + P.o_fc2, wave);
            stores_done();
        }
        stamp(l, 5);

        // ------------------------------------------------ mlp.c_proj + residual -> next h
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            const int cg = cb + P.o_fc2;
            constexpr int NF = kFfn / kCT;
            int idx[NF];
            bool use[NF];
#pragma unroll
            for (int i = 0; i < NF; ++i) {
                idx[i] = kXff + tid + kCT * i;
                use[i] = true;
            }
            XRead<NF> xr;
            poll_delay();
            xr.issue(XB, idx, use, ep(l, kEpFf));
            LaneBias<kGFc2, true> bias;
            bias.load(par + kParFc2B + P.g0, P.gn, wave, lane);
            // xs was last read by the c_proj phase, which every wave left before the c_fc
            // phase's barrier
            {
                float v[NF];
                xr.wait(XB, idx, ep(l, kEpFf), v, a.err, failed);
#pragma unroll
                for (int i = 0; i < NF; ++i) sm.xs[tid + kCT * i] = v[i];
            }
            cbar(ctl, gen, a.err, failed);
            auto out = [&](int k, float b, float acc) {
                const int row = P.g0 + k;
                xst_bcast(X, kXh + row, ep(l + 1, kEpXh), sm.mraw[row] + (acc + b));
            };
            gemv_rows_wide(ctl, ring, cg, P.gn, sm.xs, bias, par + kParFc2B + P.g0, wave, lane, a.err, failed, out);
            release_to(ctl, (l + 1) * P.layer_chunks, wave);
            stores_done();
            // xs and mraw are next written after the next layer's first barrier
        }
        stamp(l, 6);
    }
    stamp(a.layers, 0);

    // ---------------------------------------------------- ln_f, final_norm, mel_head
    {
        const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
        const int chd = a.layers * P.layer_chunks;
        int idx[5];
        bool use[5];
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            idx[i] = kXh + tid + 256 * i;
            use[i] = true;
        }
        XRead<5> xr;
        poll_delay();
        xr.issue(XB, idx, use, ep(a.layers, kEpXh));
        LnPar lf;
        lf.load(a.head + kHeadLnfW, a.head + kHeadLnfB, tid);
        LnParDot fn;
        fn.load(a.head + kHeadFnW, a.head + kHeadFnB, lane);
        LaneBias<kGHead, false> bias;
        bias.load(a.head + kHeadBias + P.h0, P.hn, wave, lane);
        float hv[5];
        xr.wait(XB, idx, ep(a.layers, kEpXh), hv, a.err, failed);
        // ln_f: statistics from the whole row, then this thread's five values to xs
#pragma unroll
        for (int i = 0; i < 5; ++i) sm.hraw[tid + 256 * i] = hv[i];
        cbar(ctl, gen, a.err, failed);
        {
            float v[4][5], mean, inv;
            ln_layout_load(sm.hraw, lane, v);
            ln_stats(v, mean, inv);
#pragma unroll
            for (int i = 0; i < 5; ++i) sm.xs[tid + 256 * i] = ln_apply(hv[i], mean, inv, lf.g[i], lf.b[i]);
        }
        cbar(ctl, gen, a.err, failed);
        // final_norm of ln_f's output, straight into the GEMV's registers
        XRow x;
        {
            float v[4][5], mean, inv;
            ln_layout_load(sm.xs, lane, v);
            ln_stats(v, mean, inv);
            ln_to_xrow(sm.xs, lane, mean, inv, fn, x);
        }
        auto out = [&](int k, float b, float acc) {
            a.logits[P.h0 + k] = acc + b;
            if (a.tail) xst(X + kXlogit + P.h0 + k, ep(a.layers, kEpLogit), acc + b);
        };
        gemv_rows(ctl, ring, chd, P.hn, x, bias, a.head + kHeadBias + P.h0, wave, lane, a.err, failed, out);
        release_to(ctl, total_chunks, wave);
    }
    stamp(a.layers, 6);
    sampling_tail(a, ctl, lds, ep(a.layers, kEpLogit));
}

}  // namespace

bool step_fits(int grid) { return grid >= kHeads; }

// FP32 weights only (the loaders copy 16-byte FP32 lines); BF16 decoders keep the
// multi-kernel path.
hipError_t step_occupancy(bool bf16, int* blocks_per_cu) {
    if (bf16) return hipErrorInvalidValue;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, step_kernel, kST, 0);
}

hipError_t launch_step(const StepArgs& a, int grid, bool bf16, hipStream_t s) {
    if (bf16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(step_kernel, dim3(grid), dim3(kST), 0, s, a);
    return hipGetLastError();
}

}  // namespace itts

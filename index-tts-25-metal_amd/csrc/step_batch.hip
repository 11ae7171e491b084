// Persistent decode step for B = 2..4 sequences at once (batched requests): the batch-1
// step kernel's structure (step.hip) with every activation vector, attention tile, merge,
// residual and logits row per sequence, and the weights streamed once for all of them.
//
// What is per sequence q:
//   * the exchange: sequence q owns a whole batch-1 exchange layout at q * kStepExchangeTotal
//     (broadcast copies included), tagged with the launch's epochs;
//   * the KV cache of slot q (kv + q * kv_slot_stride; with a beam row-owner table, row r of
//     sequence q is in slot table[q][r]), its cached length n_q and its attention tiles: the
//     tile list is sequence 0's 20 x S_0 tiles, then sequence 1's, ..., dealt to workgroups
//     round by round as in step.hip; the merge of (q, head h) runs on workgroup 20 q + h;
//   * the logits row (logits + q * logit_stride) and the decode state (state[q]).
// A workgroup's GEMV rows are the same as in step.hip; each row group's weights are read
// from the LDS ring once and multiplied with the B input vectors (B FMA chains, each in the
// batch-1 order and reduced with the batch-1 pairings), so every sequence's logits are
// bitwise those of a batch-1 step.
//
// LDS: the phase inputs of all B sequences share one staging area of 2560 floats per
// sequence, and the ring takes the rest (26, 24, 22 chunks for B = 2, 3, 4), enough to hold
// a workgroup's 20 mlp.c_fc chunks, or its 20 mlp.c_proj chunks, at once.  mlp.c_proj's
// 5120-wide rows run in two halves (first two chunks of every row against activations
// 0-2559, then the last two), the accumulators carried across.  Rows go in groups of four,
// a wave's last five in one group; 5120-wide rows one at a time (step.hip's row pairs need
// more registers than B inputs leave).  A GEMV's input rows stay in LDS (a LayerNorm phase
// writes the normalised row next to the raw one) and are read 16 bytes per lane per piece,
// so the registers hold only the row group's weights and B accumulators.  Since
// consecutive phases reuse the staging area, each phase ends its reads of it at a
// compute-wave barrier before the next phase writes.
//
// Attention differs from step.hip in where the cached K/V rows come from: the compute threads
// load their tile rows straight into registers, two rounds ahead, instead of the loaders
// staging them in the ring.  Those rows are in the cache before the step starts, so their
// loads overlap the q hand-off, and with several rounds per layer no round waits behind
// the loaders' weight stream.  q and the new K/V row of a window of four rounds are polled
// once into LDS.  The loaders stream weights only.
//
// Reference ops replaced: gpt.cpp:88-125 for several step rows (as step.hip), the batched
// form of the reference's per-row GEMV (kernels.metal mit2_linear_gemv_f32 :1054-1080).
#include "step_common.h"

namespace itts {
namespace {
using namespace stepc;

template <int B>
struct BCfg {
    static_assert(B >= 2 && B <= kStepBatchMax, "batch of the persistent batch step");
    // The staging area holds 2560 floats per sequence, so the ring keeps every mlp.c_fc and
    // mlp.c_proj chunk of a workgroup (20 each) resident with room to prefetch.
    static constexpr int kRing = B == 2 ? 26 : B == 3 ? 24 : 22;
    static constexpr bool kFive = true;         // a wave's last five rows in one pass
};
constexpr int kResidMax = 16;  // own rows of attn.c_proj / mlp.c_proj per workgroup (grid >= 80)

// Exchange region of sequence q (a batch-1 layout).
__device__ __forceinline__ uint64_t* xregion(uint64_t* x, int q) { return x + static_cast<size_t>(q) * kStepExchangeTotal; }

// Value a[q] of a small register array, as a chain of selects.  Each element passes through
// an empty asm: otherwise the compiler turns the chain back into an indexed load, which puts
// the whole array in scratch memory.
template <int B>
__device__ __forceinline__ int pick(const int (&a)[B], int q) {
    int v = a[0];
#pragma unroll
    for (int i = 1; i < B; ++i) {
        int ai = a[i];
        asm volatile("" : "+v"(ai));
        v = q == i ? ai : v;
    }
    return v;
}

// This workgroup's share of the step, identical in every wave.
template <int B>
struct PlanB {
    int G, b;
    int n[B], L[B], S[B], chunk_rows[B], tiles[B];  // per sequence: cached rows, keys, splits, rows per split, tiles
    int active[B];                                   // per sequence: still decoding (its K/V row is appended)
    int ntiles, rounds;
    int q0, qn, p0, pn, f0, fn, g0, gn, h0, hn;  // row slices: c_attn, c_proj, c_fc, mlp.c_proj, mel_head
    int layer_chunks;
    int o_att, o_proj, o_fc, o_fc2;

    __device__ static void slice(int rows, int G, int b, int& r0, int& cnt) {
        const int per = (rows + G - 1) / G;
        r0 = b * per;
        cnt = max(0, min(per, rows - r0));
    }
    // Attention tile of round rd: sequence sq, head h, split s, first row t0, cached rows R.
    __device__ __forceinline__ bool tile(int rd, int& sq, int& h, int& s, int& t0, int& R) const {
        int t = b + G * rd;
        if (t >= ntiles) return false;
        sq = 0;
#pragma unroll
        for (int q = 0; q + 1 < B; ++q)
            if (sq == q && t >= tiles[q]) {
                t -= tiles[q];
                sq = q + 1;
            }
        h = t % kHeads;
        s = t / kHeads;
        const int cr = pick(chunk_rows, sq);
        t0 = s * cr;
        const int t1 = min(pick(L, sq), t0 + cr);
        R = max(0, min(t1, pick(n, sq)) - t0);
        return true;
    }

    __device__ __forceinline__ void init(const SeqState* st, int splits) {
        G = static_cast<int>(gridDim.x);
        b = static_cast<int>(blockIdx.x);
        ntiles = 0;
#pragma unroll
        for (int q = 0; q < B; ++q) {
            n[q] = static_cast<int>(st[q].n);
            active[q] = st[q].active != 0;
            L[q] = n[q] + 1;
            S[q] = live_splits_dev(L[q], splits);
            chunk_rows[q] = (L[q] + S[q] - 1) / S[q];
            tiles[q] = kHeads * S[q];
            ntiles += tiles[q];
        }
        rounds = (ntiles + G - 1) / G;
        slice(kQkv, G, b, q0, qn);
        slice(kWidth, G, b, p0, pn);
        slice(kFfn, G, b, f0, fn);
        slice(kWidth, G, b, g0, gn);
        slice(kMelVocab, G, b, h0, hn);
        o_att = qn;
        o_proj = o_att;  // cached K/V rows are loaded by the compute threads, not streamed
        o_fc = o_proj + pn;
        o_fc2 = o_fc + fn;
        layer_chunks = o_fc2 + 4 * gn;
    }
};

constexpr int kQWin = 4;    // rounds whose q / new K / new V are polled together
constexpr int kQRec = 192;  // floats per round in the window: q, new K, new V (64 each)
constexpr int kStageF = 2 * kWidth;  // staging floats per sequence
template <int B>
struct SmemB {
    union {
        float stage[B][kStageF];                    // the phase's inputs, per sequence
        float mpart[kAttnMaxSplits][2 + kHeadDim];  // gathered attention partials of one head (merge)
    };
    float qwin[kQWin * kQRec];  // q / new K / new V of kQWin attention rounds
    float resid_h[B][kResidMax];  // h at this workgroup's attn.c_proj rows (their residual)
    float resid_m[B][kResidMax];  // hmid at this workgroup's mlp.c_proj rows
    float redm[4], reds[4];
    float lnst[B][2];  // LayerNorm mean and 1 / sqrt(var + eps) of each sequence's row
    float accs[16][kHeadDim + 4];
};

// ------------------------------------------------------------------ loader waves

// chunk_src of step.hip without the K/V chunks (the compute threads load those).
template <int B>
__device__ __forceinline__ void chunk_src_b(const StepArgs& a, const PlanB<B>& P, const float* W, int l, int r, int lane,
                                            const float*& base, uint32_t& extent, uint32_t (&off)[kLines]) {
    if (l >= a.layers) {
        base = W + a.off_head + static_cast<size_t>(P.h0 + r) * kWidth;
    } else {
        const float* wl = W + static_cast<size_t>(l) * a.layer_stride;
        if (r < P.o_att) {
            base = wl + static_cast<size_t>(P.q0 + r) * kWidth;
        } else if (r < P.o_fc) {
            base = wl + static_cast<size_t>(kQkv) * kWidth + static_cast<size_t>(P.p0 + r - P.o_proj) * kWidth;
        } else if (r < P.o_fc2) {
            base = wl + static_cast<size_t>(kQkv + kWidth) * kWidth + static_cast<size_t>(P.f0 + r - P.o_fc) * kWidth;
        } else {
            // mlp.c_proj: the first two chunks of every row (activations 0-2559), then the last two
            const int q = r - P.o_fc2;
            const int h = q < 2 * P.gn ? 0 : 1;
            const int p = q - 2 * P.gn * h;
            base = wl + static_cast<size_t>(kQkv + kWidth + kFfn) * kWidth + static_cast<size_t>(P.g0 + (p >> 1)) * kFfn +
                   (2 * h + (p & 1)) * kChunkF;
        }
    }
    extent = kChunkF * 4;
#pragma unroll
    for (int k = 0; k < kLines; ++k) off[k] = static_cast<uint32_t>((k * 256 + lane * 4) * 4);
}

// ------------------------------------------------------------------ compute waves

// Element offsets (from a.kv) of the cached K rows of round rd's tile that thread (g, sub)
// holds in slots i0 .. i0 + 3: rows g + 16 i, columns 4 sub .. 4 sub + 3; ~0u for rows at or
// past the tile's cached rows.  The V rows sit a.kv_v_off further.  (The offsets fit 32
// bits: launch_step_batch checks kStepBatchMax * kv_slot_stride.)
template <int B>
__device__ __forceinline__ void tile_rows(const StepArgs& a, const PlanB<B>& P, int rd, int i0, size_t kvl, int g, int sub,
                                          uint32_t (&off)[4]) {
    int sq = 0, h = 0, s = 0, t0 = 0, R = 0;
    const bool act = P.tile(rd, sq, h, s, t0, R);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = g + 16 * (i0 + i);
        off[i] = ~0u;
        if (act && r < R) {
            const int row = t0 + r;
            const int slot = a.table ? static_cast<int>(a.table[static_cast<size_t>(sq) * a.kv_cap + row]) : sq;
            off[i] = static_cast<uint32_t>(static_cast<size_t>(slot) * a.kv_slot_stride + kvl +
                                           (static_cast<size_t>(h) * a.kv_cap + row) * kHeadDim + sub * 4);
        }
    }
}
// Issues the loads of four rows (zero where off is ~0u); the compiler waits for them where
// they are used.
__device__ __forceinline__ void load_rows(const float* base, const uint32_t (&off)[4], float4 (&d)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) d[i] = off[i] != ~0u ? *reinterpret_cast<const float4*>(base + off[i]) : make_float4(0.f, 0.f, 0.f, 0.f);
}

// stage[q][dst + c] = LayerNorm(stage[q][src + c]) for this thread's 5 columns c = tid + 256 i
// of each of the B staging rows.  Compute wave q (< B) forms row q's statistics with ln_stats
// (so the values equal ln_to_xrow's) and passes them through lnst across one compute-wave
// barrier; every thread then normalises its own columns.  (Each wave forming every row's
// statistics itself, as the batch-1 kernel does to save the barrier, costs B times the LDS
// reads and reductions.)
template <int B>
__device__ __forceinline__ void ln_stage_rows(float (*stage)[kStageF], int src, int dst, const LnPar& p, int tid, int lane,
                                              float (*lnst)[2], Ctl& ctl, uint32_t& gen, uint32_t* err, bool& failed) {
    static_assert(B <= kCW, "one compute wave per row's statistics");
    const int wave = tid >> 6;
    if (wave < B) {
        float v[4][5], mean, inv;
        ln_layout_load(stage[wave] + src, lane, v);
        ln_stats(v, mean, inv);
        if (lane == 0) {
            lnst[wave][0] = mean;
            lnst[wave][1] = inv;
        }
    }
    cbar(ctl, gen, err, failed);
#pragma unroll
    for (int q = 0; q < B; ++q) {
        const float mean = lnst[q][0], inv = lnst[q][1];
#pragma unroll
        for (int i = 0; i < 5; ++i)
            stage[q][dst + tid + 256 * i] = ln_apply(stage[q][src + tid + 256 * i], mean, inv, p.g[i], p.b[i]);
    }
}

// rowsN of step.hip for B inputs: rows k0 + 4 t (t < N, those below cnt) of a 1280-wide slice,
// each multiplied with every sequence's input row xs[q] (in LDS, read 16 bytes per lane per
// piece j as the batch-1 XRow holds it); res[q] as wave_sum4 leaves it (row k0 + 4 t in lanes
// 0-15, 32-47, 16-31, 48-63 for t = 0..3), fifth[q] the fifth row's sum (N == 5).
template <int N, int B, int RING>
__device__ __forceinline__ void rowsNB(Ctl& ctl, const float* ring, int c0, int k0, int cnt, const float* const (&xs)[B], int wave,
                                       int lane, uint32_t* err, bool& failed, float (&res)[B], float (&fifth)[B]) {
    static_assert(N == 4 || N == 5, "row group size");
    release_to(ctl, c0 + k0, wave);
    const int nt = N == 5 ? 5 : min(4, (cnt - k0 + 3) >> 2);
    (void)wait_chunk<RING>(ctl, ring, c0 + k0 + 4 * (nt - 1), err, failed);
    const float* ch[N];
#pragma unroll
    for (int t = 0; t < N; ++t) ch[t] = ring + ((c0 + k0 + 4 * (t < nt ? t : 0)) % RING) * kChunkF;  // absent rows re-read row k0
    float4 w[N][5];
#pragma unroll
    for (int j = 0; j < 5; ++j)
#pragma unroll
        for (int t = 0; t < N; ++t) w[t][j] = *reinterpret_cast<const float4*>(ch[t] + (j * 64 + lane) * 4);
    __builtin_amdgcn_sched_barrier(0);
    float acc[N][B];
#pragma unroll
    for (int t = 0; t < N; ++t)
#pragma unroll
        for (int q = 0; q < B; ++q) acc[t][q] = 0.0f;
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        float4 x[B];
#pragma unroll
        for (int q = 0; q < B; ++q) x[q] = *reinterpret_cast<const float4*>(xs[q] + (j * 64 + lane) * 4);
#pragma unroll
        for (int t = 0; t < N; ++t)
#pragma unroll
            for (int q = 0; q < B; ++q) {
                acc[t][q] = __builtin_fmaf(w[t][j].x, x[q].x, acc[t][q]);
                acc[t][q] = __builtin_fmaf(w[t][j].y, x[q].y, acc[t][q]);
                acc[t][q] = __builtin_fmaf(w[t][j].z, x[q].z, acc[t][q]);
                acc[t][q] = __builtin_fmaf(w[t][j].w, x[q].w, acc[t][q]);
            }
    }
#pragma unroll
    for (int q = 0; q < B; ++q) {
        if constexpr (N == 5) fifth[q] = wave_sum(acc[4][q]);
        res[q] = wave_sum4(acc[0][q], acc[1][q], acc[2][q], acc[3][q]);
    }
}

// gemv_rows of step.hip for B inputs: out(k, bias, q, sum) in the lane holding row k's sum of
// sequence q.  Biases come from `bias` for the first NG groups, later from bias_mem.
template <int B, int RING, bool kFive, int NG, class Out>
__device__ __forceinline__ void gemv_rows_b(Ctl& ctl, const float* ring, int c0, int cnt, const float* const (&xr)[B], const LaneBias<NG, false>& bias,
                                            const float* __restrict__ bias_mem, int wave, int lane, uint32_t* err, bool& failed, Out out) {
    const int t = row_of_lane4(lane);
    const bool holder = (lane & 15) == 0;
    int g = 0;
    for (int k0 = wave; k0 < cnt; k0 += 16, ++g) {
        const int k = k0 + 4 * t;
        float b4 = 0.0f;
#pragma unroll
        for (int i = 0; i < NG; ++i)
            if (g == i) b4 = bias.v[i];
        if (g >= NG && holder && k < cnt) b4 = bias_mem[k];
        float res[B], fifth[B];
        if (kFive && k0 + 16 < cnt && k0 + 20 >= cnt) {  // exactly five rows left
            rowsNB<kFive ? 5 : 4, B, RING>(ctl, ring, c0, k0, cnt, xr, wave, lane, err, failed, res, fifth);
            const float b5 = bias_mem[k0 + 16];
#pragma unroll
            for (int q = 0; q < B; ++q) {
                if (holder && k < cnt) out(k, b4, q, res[q]);
                if (lane == 0) out(k0 + 16, b5, q, fifth[q]);
            }
            return;
        }
        rowsNB<4, B, RING>(ctl, ring, c0, k0, cnt, xr, wave, lane, err, failed, res, fifth);
#pragma unroll
        for (int q = 0; q < B; ++q)
            if (holder && k < cnt) out(k, b4, q, res[q]);
    }
}

// Half h of mlp.c_proj row k (5120 wide): its chunks m = 2h and 2h + 1, ring chunks
// c0 + 2 gn h + 2k and the next, times the staged half of each sequence's activations xs[q]
// (activations 2560 h + 1280 (m - 2h) + 4 (j*64 + lane) .. + 3), added to a[q].  The two
// calls of a row continue one FMA chain per lane in chunk order (rows_wide of step.hip).
template <int B, int RING>
__device__ __forceinline__ void wide_half(Ctl& ctl, const float* ring, int c, const float (*xs)[kStageF], int lane, uint32_t* err,
                                          bool& failed, float (&a)[B]) {
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
        const float* r0 = wait_chunk<RING>(ctl, ring, c + mm, err, failed);
        float4 w0[5];
#pragma unroll
        for (int j = 0; j < 5; ++j) w0[j] = *reinterpret_cast<const float4*>(r0 + (j * 64 + lane) * 4);
#pragma unroll
        for (int q = 0; q < B; ++q) {
            float4 x[5];
#pragma unroll
            for (int j = 0; j < 5; ++j) x[j] = *reinterpret_cast<const float4*>(xs[q] + ((5 * mm + j) * 64 + lane) * 4);
#pragma unroll
            for (int j = 0; j < 5; ++j) {
                a[q] = __builtin_fmaf(w0[j].x, x[j].x, a[q]);
                a[q] = __builtin_fmaf(w0[j].y, x[j].y, a[q]);
                a[q] = __builtin_fmaf(w0[j].z, x[j].z, a[q]);
                a[q] = __builtin_fmaf(w0[j].w, x[j].w, a[q]);
            }
        }
    }
}

constexpr int kGQkv = 1, kGProj = 1, kGFc = 2, kGHead = 3;
constexpr int kMergeRegSplits = 16;

template <int B>
__global__ __launch_bounds__(kST) void step_batch_kernel(StepArgs a) {
    using C = BCfg<B>;
    constexpr int RING = C::kRing;
    __shared__ float ring[RING * kChunkF];
    __shared__ Ctl ctl;
    __shared__ SmemB<B> sm;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    {
        bool any = false;
#pragma unroll
        for (int q = 0; q < B; ++q) any |= a.state[q].active != 0;
        if (!any) return;
    }
    if (tid < kLW) ctl.done[tid] = 0;
    if (tid < kCW) ctl.need[tid] = 0;
    if (tid == 0) ctl.bar = 0;
    __syncthreads();  // the only barrier of the whole workgroup; roles split below

    PlanB<B> P;
    P.init(a.state, a.splits);
    const int total_chunks = a.layers * P.layer_chunks + P.hn;

    // ================================================================ loaders
    if (wave >= kCW) {
        const float* __restrict__ W = static_cast<const float*>(a.w);
        const int lw = __builtin_amdgcn_readfirstlane(wave - kCW);
        run_loader<RING>(a, P.layer_chunks, P.hn, ring, ctl, lw, lane,
                         [&](int l, int r, const float*& base, uint32_t& extent, uint32_t(&off)[kLines]) {
                             chunk_src_b<B>(a, P, W, l, r, lane, base, extent, off);
                         });
        return;
    }

    // ================================================================ compute waves
    bool failed = false;
    uint32_t gen = 0;
    const int cpy = P.b % kStepCopies;
    const uint32_t e0 = a.epoch;
    auto ep = [&](int l, uint32_t kind) { return e0 + 8u * static_cast<uint32_t>(l) + kind; };
    auto XW = [&](int q) { return xregion(a.xch, q); };                                  // written by producers
    auto XR = [&](int q) -> const uint64_t* { return xregion(a.xch, q) + xcopy(cpy, 0); };  // this workgroup's copy
    // phase-end clocks for measurement (one lane, only when the host asks for them)
    auto stamp = [&](int l, int k) {
        if (a.stamps && opaque_tid() == 0)
            a.stamps[(static_cast<size_t>(P.b) * (a.layers + 1) + l) * kStepStampsPerLayer + k] = __builtin_amdgcn_s_memrealtime();
    };

    for (int l = 0; l < a.layers; ++l) {
        const float* __restrict__ par = a.params + static_cast<size_t>(l) * kParLayer;
        const size_t kvl = static_cast<size_t>(l) * a.kv_layer_stride;
        const int cb = l * P.layer_chunks;
        stamp(l, 0);

        // ------------------------------------------------ LN1 + c_attn (+ K/V append)
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            release_to(ctl, cb, wave);
            int idx[5];
            bool use[5];
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                idx[i] = kXh + tid + 256 * i;
                use[i] = l > 0;
            }
            XRead<5> xr[B];
#pragma unroll
            for (int q = 0; q < B; ++q) xr[q].issue(XR(q), idx, use, ep(l, kEpXh));
            LnPar ln;
            ln.load(par + kParLn1W, par + kParLn1B, tid);
            LaneBias<kGQkv, false> bias;
            bias.load(par + kParQkvB + P.q0, P.qn, wave, lane);
#pragma unroll
            for (int q = 0; q < B; ++q) {
                float hv[5];
                if (l == 0) {
                    const SeqState& sq = a.state[q];
#pragma unroll
                    for (int i = 0; i < 5; ++i) {
                        const int c = tid + 256 * i;
                        hv[i] = a.mel_emb[static_cast<size_t>(sq.token) * kWidth + c] + a.mel_pos[static_cast<size_t>(sq.position) * kWidth + c];
                    }
                } else {
                    xr[q].wait(XR(q), idx, ep(l, kEpXh), hv, a.err, failed);
                }
#pragma unroll
                for (int i = 0; i < 5; ++i) sm.stage[q][tid + 256 * i] = hv[i];
            }
            cbar(ctl, gen, a.err, failed);
            if (wave == 0 && lane < P.pn) {
#pragma unroll
                for (int q = 0; q < B; ++q) sm.resid_h[q][lane] = sm.stage[q][P.p0 + lane];
            }
            ln_stage_rows<B>(sm.stage, 0, kWidth, ln, tid, lane, sm.lnst, ctl, gen, a.err, failed);
            cbar(ctl, gen, a.err, failed);
            const float* x[B];
#pragma unroll
            for (int q = 0; q < B; ++q) x[q] = sm.stage[q] + kWidth;
            const uint32_t e = ep(l, kEpQkv);
            auto out = [&](int k, float b, int q, float acc) {
                const int row = P.q0 + k;
                const float v = acc + b;
                xst_bcast(XW(q), kXqkv + row, e, v);
                if (row >= kWidth && pick(P.active, q)) {
                    const int rr = row - kWidth;
                    const bool is_v = rr >= kWidth;
                    const int c = is_v ? rr - kWidth : rr;
                    const size_t nrow = static_cast<size_t>(pick(P.n, q));
                    a.kv[static_cast<size_t>(q) * a.kv_slot_stride + kvl + (is_v ? a.kv_v_off : 0) +
                         (static_cast<size_t>(c >> 6) * a.kv_cap + nrow) * kHeadDim + (c & 63)] = v;
                }
            };
            gemv_rows_b<B, RING, C::kFive>(ctl, ring, cb, P.qn, x, bias, par + kParQkvB + P.q0, wave, lane, a.err, failed, out);
            stores_done();
        }

        stamp(l, 1);

        // ------------------------------------------------ split-KV attention tiles
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            const int g = tid >> 4, sub = tid & 15;
            const uint32_t eq = ep(l, kEpQkv), epart = ep(l, kEpPart);
            release_to(ctl, cb + P.o_att, wave);  // c_attn's rows are done: the loaders go on to c_proj
            // The window of q / new K / new V records is apart from the staging area that
            // c_attn reads, so it may be written while other waves still run c_attn.
            float* qwin = sm.qwin;
            // One tile's rows in registers: the next tile round's K is issued once this tile
            // round's scores are formed, its V once its weighted sum is.  A tile of more than
            // 64 rows (caches past 768 rows) has the 8 arithmetic slots of attention_kernel:
            // slots 4-7 are loaded into the same registers once slots 0-3 are used, K for the
            // scores, then V for the weighted sum, which keeps attention_kernel's order.
            uint32_t off[4];
            float4 kk[4], vv[4];
            tile_rows<B>(a, P, 0, 0, kvl, g, sub, off);
            load_rows(a.kv, off, kk);
            load_rows(a.kv + a.kv_v_off, off, vv);
            for (int rd = 0; rd < P.rounds; ++rd) {
                // A later window overwrites the last one after the previous round's closing
                // barrier; every wave read its record before that round's first barrier.
                if (rd % kQWin == 0) {
                    if (tid < kQRec) {
                        const int part = tid >> 6, c = tid & 63;  // part 0: q, 1: new K, 2: new V
                        int idx[kQWin];
                        bool use[kQWin];
#pragma unroll
                        for (int w = 0; w < kQWin; ++w) {
                            int sq = 0, h = 0, s = 0, t0 = 0, R = 0;
                            const bool act = P.tile(rd + w, sq, h, s, t0, R);
                            const int nq = act ? pick(P.n, sq) : 0;
                            const int p1 = act ? min(pick(P.L, sq), t0 + pick(P.chunk_rows, sq)) : 0;
                            idx[w] = sq * static_cast<int>(kStepExchangeTotal) + kXqkv + part * kWidth + h * kHeadDim + c;
                            use[w] = act && (part == 0 || (nq >= t0 && nq < p1));
                        }
                        float v[kQWin];
                        xread<kQWin>(XR(0), idx, use, eq, v, a.err, failed);
#pragma unroll
                        for (int w = 0; w < kQWin; ++w)
                            if (use[w]) qwin[w * kQRec + tid] = v[w];
                    }
                    cbar(ctl, gen, a.err, failed);
                }
                int sq = 0, h = 0, s = 0, t0 = 0, R = 0;
                const bool act = P.tile(rd, sq, h, s, t0, R);
                const int nq = act ? pick(P.n, sq) : 0;
                const int p1 = act ? min(pick(P.L, sq), t0 + pick(P.chunk_rows, sq)) : 0;
                const int dn = nq - t0 - g;
                const int i_new = (act && nq < p1 && dn >= 0 && (dn & 15) == 0 && (dn >> 4) < 8) ? (dn >> 4) : -1;
                const bool wide = act && p1 - t0 > 64;  // the tile has rows in slots 4-7 (uniform)
                const float* qr = qwin + (rd % kQWin) * kQRec;
                const float4 q4 = *reinterpret_cast<const float4*>(qr + sub * 4);
                if (i_new >= 0 && i_new < 4) {
                    const float4 kn = *reinterpret_cast<const float4*>(qr + kHeadDim + sub * 4);
                    const float4 vn = *reinterpret_cast<const float4*>(qr + 2 * kHeadDim + sub * 4);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (i == i_new) {
                            kk[i] = kn;
                            vv[i] = vn;
                        }
                    }
                }
                float sc[8];
                float mloc = -INFINITY;
                auto scores = [&](int i0) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        float d = q4.x * kk[i].x;
                        d = __builtin_fmaf(q4.y, kk[i].y, d);
                        d = __builtin_fmaf(q4.z, kk[i].z, d);
                        d = __builtin_fmaf(q4.w, kk[i].w, d);
                        d = sum16_up(d);
                        const bool valid = act && t0 + g + 16 * (i0 + i) < p1;
                        sc[i0 + i] = valid ? d * 0.125f : -INFINITY;
                        mloc = fmaxf(mloc, sc[i0 + i]);
                    }
                };
                scores(0);
                uint32_t offw[4];
                if (wide) {
                    tile_rows<B>(a, P, rd, 4, kvl, g, sub, offw);
                    load_rows(a.kv, offw, kk);
                    if (i_new >= 4) {
                        const float4 kn = *reinterpret_cast<const float4*>(qr + kHeadDim + sub * 4);
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (4 + i == i_new) kk[i] = kn;
                    }
                    scores(4);
                } else {
#pragma unroll
                    for (int i = 4; i < 8; ++i) sc[i] = -INFINITY;
                }
                const bool more = rd + 1 < P.rounds;
                if (more) {
                    tile_rows<B>(a, P, rd + 1, 0, kvl, g, sub, off);
                    load_rows(a.kv, off, kk);
                }
                const float wm = wave_max(mloc);
                if (lane == 0) sm.redm[wave] = wm;
                cbar(ctl, gen, a.err, failed);
                const float M = fmaxf(fmaxf(sm.redm[0], sm.redm[1]), fmaxf(sm.redm[2], sm.redm[3]));
                float lsum = 0.0f;
                float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
                auto weigh = [&](int i0) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const bool valid = act && t0 + g + 16 * (i0 + i) < p1;
                        const float e = valid ? expf(sc[i0 + i] - M) : 0.0f;
                        lsum += e;
                        acc.x = __builtin_fmaf(e, vv[i].x, acc.x);
                        acc.y = __builtin_fmaf(e, vv[i].y, acc.y);
                        acc.z = __builtin_fmaf(e, vv[i].z, acc.z);
                        acc.w = __builtin_fmaf(e, vv[i].w, acc.w);
                    }
                };
                weigh(0);
                if (wide) {
                    load_rows(a.kv + a.kv_v_off, offw, vv);
                    if (i_new >= 4) {
                        const float4 vn = *reinterpret_cast<const float4*>(qr + 2 * kHeadDim + sub * 4);
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (4 + i == i_new) vv[i] = vn;
                    }
                    weigh(4);
                }
                if (more) load_rows(a.kv + a.kv_v_off, off, vv);
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
                    uint64_t* part = XW(sq) + kXpart + (static_cast<size_t>(h) * kAttnMaxSplits + s) * 68;
                    xst(part + 4 + tid, epart, tot);
                    if (tid == 0) {
                        xst(part + 0, epart, M);
                        xst(part + 1, epart, ((sm.reds[0] + sm.reds[1]) + sm.reds[2]) + sm.reds[3]);
                    }
                }
                if (more) cbar(ctl, gen, a.err, failed);
            }
            release_to(ctl, cb + P.o_proj, wave);
            stores_done();
        }

        stamp(l, 2);

        // ------------------------------------------------ merge of (sequence, head) = (b / 20, b % 20)
        if (P.b < kHeads * B) {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            const int sq = P.b / kHeads, h = P.b % kHeads;
            const int S = pick(P.S, sq);
            const uint64_t* pb = XW(sq) + kXpart + static_cast<size_t>(h) * kAttnMaxSplits * 68;
            if (S <= kMergeRegSplits) {
                if (wave == 0) {
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
                    xst_bcast(XW(sq), kXattn + h * kHeadDim + lane, ep(l, kEpAttn), nn / d);
                    stores_done();
                }
            } else {
                constexpr int kRec = 2 + kHeadDim;
                constexpr int NPT = (kAttnMaxSplits * kRec + kCT - 1) / kCT;
                {
                    int idx[NPT];
                    bool use[NPT];
                    float v[NPT];
#pragma unroll
                    for (int i = 0; i < NPT; ++i) {
                        const int qq = tid + kCT * i;
                        const int k = qq / kRec, f = qq % kRec;
                        idx[i] = k * 68 + (f < 2 ? f : f + 2);
                        use[i] = k < S;
                    }
                    xread<NPT>(pb, idx, use, ep(l, kEpPart), v, a.err, failed);
#pragma unroll
                    for (int i = 0; i < NPT; ++i) {
                        const int qq = tid + kCT * i;
                        if (use[i]) sm.mpart[qq / kRec][qq % kRec] = v[i];
                    }
                }
                cbar(ctl, gen, a.err, failed);
                if (wave == 0) {
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
                    xst_bcast(XW(sq), kXattn + h * kHeadDim + lane, ep(l, kEpAttn), nn / d);
                    stores_done();
                }
                cbar(ctl, gen, a.err, failed);  // mpart aliases the staging area, written below
            }
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
            XRead<5> xr[B];
#pragma unroll
            for (int q = 0; q < B; ++q) xr[q].issue(XR(q), idx, use, ep(l, kEpAttn));
            LaneBias<kGProj, false> bias;
            bias.load(par + kParProjB + P.p0, P.pn, wave, lane);
#pragma unroll
            for (int q = 0; q < B; ++q) {
                float v[5];
                xr[q].wait(XR(q), idx, ep(l, kEpAttn), v, a.err, failed);
#pragma unroll
                for (int i = 0; i < 5; ++i) sm.stage[q][tid + 256 * i] = v[i];
            }
            cbar(ctl, gen, a.err, failed);
            const float* x[B];
#pragma unroll
            for (int q = 0; q < B; ++q) x[q] = sm.stage[q];
            const uint32_t e = ep(l, kEpHmid);
            auto out = [&](int k, float b, int q, float acc) { xst_bcast(XW(q), kXhmid + P.p0 + k, e, sm.resid_h[q][k] + (acc + b)); };
            gemv_rows_b<B, RING, C::kFive>(ctl, ring, cp, P.pn, x, bias, par + kParProjB + P.p0, wave, lane, a.err, failed, out);
            release_to(ctl, cb + P.o_fc, wave);
            stores_done();
            cbar(ctl, gen, a.err, failed);  // the staging area is written by the next phase
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
            XRead<5> xr[B];
#pragma unroll
            for (int q = 0; q < B; ++q) xr[q].issue(XR(q), idx, use, ep(l, kEpHmid));
            LnPar ln;
            ln.load(par + kParLn2W, par + kParLn2B, tid);
            LaneBias<kGFc, false> bias;
            bias.load(par + kParFcB + P.f0, P.fn, wave, lane);
#pragma unroll
            for (int q = 0; q < B; ++q) {
                float hv[5];
                xr[q].wait(XR(q), idx, ep(l, kEpHmid), hv, a.err, failed);
#pragma unroll
                for (int i = 0; i < 5; ++i) sm.stage[q][tid + 256 * i] = hv[i];
            }
            cbar(ctl, gen, a.err, failed);
            if (wave == 0 && lane < P.gn) {
#pragma unroll
                for (int q = 0; q < B; ++q) sm.resid_m[q][lane] = sm.stage[q][P.g0 + lane];
            }
            ln_stage_rows<B>(sm.stage, 0, kWidth, ln, tid, lane, sm.lnst, ctl, gen, a.err, failed);
            cbar(ctl, gen, a.err, failed);
            const float* x[B];
#pragma unroll
            for (int q = 0; q < B; ++q) x[q] = sm.stage[q] + kWidth;
            const uint32_t e = ep(l, kEpFf);
            auto out = [&](int k, float b, int q, float acc) { xst_bcast(XW(q), kXff + P.f0 + k, e, gelu_f(acc + b)); };
            gemv_rows_b<B, RING, C::kFive>(ctl, ring, cf, P.fn, x, bias, par + kParFcB + P.f0, wave, lane, a.err, failed, out);
            release_to(ctl, cb + P.o_fc2, wave);
            stores_done();
            cbar(ctl, gen, a.err, failed);  // the staging area is written by the next phase
        }

        stamp(l, 5);

        // ------------------------------------------------ mlp.c_proj + residual -> next h
        // The staging area takes half of each sequence's 5120 activations at a time: every
        // row's first two chunks are multiplied with activations 0-2559, then its last two with
        // 2560-5119, the accumulators carried across (the loaders stream the chunks in that
        // order).  Up to 3 sequences, the second half's polls are in flight during the first
        // half's products (at 4 they would not fit in registers).
        {
            const int tid = opaque_tid(), lane = tid & 63, wave = tid >> 6;
            const int cg = cb + P.o_fc2;
            constexpr int NH = kFfn / kCT / 2;   // activations per thread, sequence and half
            constexpr int RW = kResidMax / kCW;  // rows per wave at most
            const uint32_t e = ep(l, kEpFf);
            auto hidx = [&](int h, int (&idx)[NH]) {
#pragma unroll
                for (int i = 0; i < NH; ++i) idx[i] = kXff + kStageF * h + tid + kCT * i;
            };
            XRead<NH> xr[B];
            auto issue = [&](int h) {
                int idx[NH];
                bool use[NH];
                hidx(h, idx);
#pragma unroll
                for (int i = 0; i < NH; ++i) use[i] = true;
#pragma unroll
                for (int q = 0; q < B; ++q) xr[q].issue(XR(q), idx, use, e);
            };
            auto stage_half = [&](int h) {
                int idx[NH];
                hidx(h, idx);
#pragma unroll
                for (int q = 0; q < B; ++q) {
                    float v[NH];
                    xr[q].wait(XR(q), idx, e, v, a.err, failed);
#pragma unroll
                    for (int i = 0; i < NH; ++i) sm.stage[q][tid + kCT * i] = v[i];
                }
            };
            float acc[RW][B];
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int q = 0; q < B; ++q) acc[r][q] = 0.0f;
            constexpr bool kEarly = B <= 3;
            issue(0);
            stage_half(0);
            if (kEarly) issue(1);
            cbar(ctl, gen, a.err, failed);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (h == 1) {
                    if (!kEarly) issue(1);
                    cbar(ctl, gen, a.err, failed);  // every wave is past the first half's activations
                    stage_half(1);
                    cbar(ctl, gen, a.err, failed);
                }
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    const int k = wave + kCW * r;
                    if (k < P.gn) {
                        const int c = cg + 2 * P.gn * h + 2 * k;
                        release_to(ctl, c, wave);
                        wide_half<B, RING>(ctl, ring, c, sm.stage, lane, a.err, failed, acc[r]);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const int k = wave + kCW * r;
                if (k < P.gn) {
                    float res[B];
#pragma unroll
                    for (int q = 0; q < B; ++q) res[q] = wave_sum(acc[r][q]);
                    if (lane == 0) {
                        const float b = par[kParFc2B + P.g0 + k];
#pragma unroll
                        for (int q = 0; q < B; ++q) xst_bcast(XW(q), kXh + P.g0 + k, ep(l + 1, kEpXh), sm.resid_m[q][k] + (res[q] + b));
                    }
                }
            }
            release_to(ctl, (l + 1) * P.layer_chunks, wave);
            stores_done();
            cbar(ctl, gen, a.err, failed);  // the staging area is written by the next phase
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
        XRead<5> xr[B];
#pragma unroll
        for (int q = 0; q < B; ++q) xr[q].issue(XR(q), idx, use, ep(a.layers, kEpXh));
        LnPar lf;
        lf.load(a.head + kHeadLnfW, a.head + kHeadLnfB, tid);
        LnPar fn;
        fn.load(a.head + kHeadFnW, a.head + kHeadFnB, tid);
        LaneBias<kGHead, false> bias;
        bias.load(a.head + kHeadBias + P.h0, P.hn, wave, lane);
#pragma unroll
        for (int q = 0; q < B; ++q) {
            float hv[5];
            xr[q].wait(XR(q), idx, ep(a.layers, kEpXh), hv, a.err, failed);
#pragma unroll
            for (int i = 0; i < 5; ++i) sm.stage[q][tid + 256 * i] = hv[i];
        }
        cbar(ctl, gen, a.err, failed);
        // ln_f into the second 1280 floats of the sequence's staging row, then final_norm back
        // into the first (the raw row is no longer read)
        ln_stage_rows<B>(sm.stage, 0, kWidth, lf, tid, lane, sm.lnst, ctl, gen, a.err, failed);
        cbar(ctl, gen, a.err, failed);
        ln_stage_rows<B>(sm.stage, kWidth, 0, fn, tid, lane, sm.lnst, ctl, gen, a.err, failed);
        cbar(ctl, gen, a.err, failed);
        const float* x[B];
#pragma unroll
        for (int q = 0; q < B; ++q) x[q] = sm.stage[q];
        auto out = [&](int k, float b, int q, float acc) { a.logits[static_cast<size_t>(q) * a.logit_stride + P.h0 + k] = acc + b; };
        gemv_rows_b<B, RING, C::kFive>(ctl, ring, chd, P.hn, x, bias, a.head + kHeadBias + P.h0, wave, lane, a.err, failed, out);
        release_to(ctl, total_chunks, wave);
    }
    stamp(a.layers, 6);
}

template <int B>
hipError_t launch_b(const StepArgs& a, int grid, hipStream_t s) {
    hipLaunchKernelGGL(step_batch_kernel<B>, dim3(grid), dim3(kST), 0, s, a);
    return hipGetLastError();
}
template <int B>
hipError_t occupancy_b(int* blocks_per_cu) {
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, step_batch_kernel<B>, kST, 0);
}

}  // namespace

// The merge of (sequence q, head h) runs on workgroup 20 q + h, and attn.c_proj / mlp.c_proj
// give a workgroup at most kResidMax rows.
bool step_batch_fits(int grid, int nseq) { return nseq >= 2 && nseq <= kStepBatchMax && grid >= kHeads * nseq && grid * kResidMax >= kWidth; }

hipError_t step_batch_occupancy(int nseq, int* blocks_per_cu) {
    switch (nseq) {
        case 2: return occupancy_b<2>(blocks_per_cu);
        case 3: return occupancy_b<3>(blocks_per_cu);
        case 4: return occupancy_b<4>(blocks_per_cu);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_step_batch(const StepArgs& a, int nseq, int grid, hipStream_t s) {
    // tile_rows forms 32-bit element offsets into slots 0 .. kStepBatchMax - 1 (of the launch's
    // KV base): the sequences' own, or those the row-owner table names
    if (nseq != a.nseq || static_cast<uint64_t>(kStepBatchMax) * a.kv_slot_stride >= 0xFFFFFFFFull) return hipErrorInvalidValue;
    switch (nseq) {
        case 2: return launch_b<2>(a, grid, s);
        case 3: return launch_b<3>(a, grid, s);
        case 4: return launch_b<4>(a, grid, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace itts

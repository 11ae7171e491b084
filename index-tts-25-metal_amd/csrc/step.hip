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
#include "kernels.h"

namespace itts {
namespace {

constexpr int kST = kStepThreads;  // 512
constexpr int kCT = 256;           // compute threads: waves 0..3
constexpr int kCW = kCT / 64;      // compute waves
constexpr int kLW = (kST - kCT) / 64;  // loader waves
constexpr int kLines = 5;          // 1 KB lines per chunk
constexpr int kChunkF = kLines * 256;  // floats per chunk (one 1280-wide row)
constexpr int kRing = 24;          // chunks in the LDS ring
// Chunks staged in registers per loader wave.  Measured on gfx950 (752 cached rows): 1 -> 713 us
// per step, 2 -> 634 us, 3 -> 650 us, 8 -> 659 us.  Fewer L2 misses in flight keep the memory-side
// queues short, and every hand-off (an agent-scope store and poll) waits in those queues.
constexpr int kSlots = 2;
// Weight stream loads: raw buffer loads (a wave-uniform base in the descriptor, 32-bit lane
// offsets, range-checked against the chunk's extent), non-temporal.  Measured 627 us per step
// against 634 us for global_load_dwordx4 ... nt of the same addresses.
constexpr int kCachePolicyNt = 2;     // cache-policy operand: nt
constexpr int kBufferDword3 = 0x00020000;  // descriptor word 3 of a raw 32-bit buffer on gfx9
constexpr int kKvRowsPerChunk = kChunkF / kHeadDim;  // 20 cached rows of one head
constexpr unsigned kSpinLimit = 1u << 20;     // global polls (~1 us each)
constexpr unsigned kLdsSpinLimit = 1u << 24;  // LDS polls (~0.1 us each)
static_assert(kCW == 4 && kLW == 4, "role split");

// Exchange layout (uint64 slots).
constexpr int kXh = 0;
constexpr int kXqkv = kXh + kWidth;
constexpr int kXattn = kXqkv + kQkv;
constexpr int kXhmid = kXattn + kWidth;
constexpr int kXff = kXhmid + kWidth;
constexpr int kXpart = kXff + kFfn;
static_assert(kXpart + kHeads * kAttnMaxSplits * 68 == kStepExchange, "exchange layout");
static_assert(kXpart == kStepBroadcast, "broadcast vectors come first");

enum Kind : uint32_t { kEpXh = 0, kEpQkv = 1, kEpPart = 2, kEpAttn = 3, kEpHmid = 4, kEpFf = 5 };

__device__ __forceinline__ uint64_t xld(const uint64_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// base + 32-bit unsigned element offset (a scalar base plus one VGPR per address)
__device__ __forceinline__ uint64_t xld(const uint64_t* base, int off) { return xld(base + static_cast<uint32_t>(off)); }
__device__ __forceinline__ void xst(uint64_t* p, uint32_t epoch, float v) {
    __hip_atomic_store(p, (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Copy r of broadcast slot i (i < kStepBroadcast).
__device__ __forceinline__ size_t xcopy(int r, int i) {
    return r == 0 ? static_cast<size_t>(i) : size_t(kStepExchange) + size_t(r - 1) * kStepCopyStride + i;
}
// A broadcast value goes to every copy.
__device__ __forceinline__ void xst_bcast(uint64_t* x, int i, uint32_t epoch, float v) {
#pragma unroll
    for (int r = 0; r < kStepCopies; ++r) xst(x + xcopy(r, i), epoch, v);
}

// N tagged values: issue() sends all loads, wait() retries the stale ones until their epoch
// is `e` (one retry loop for all N).  Splitting the two lets a wave do LDS work while the
// loads are in flight.  A bounded wait: past kSpinLimit retries the error flag is raised
// and the thread stops waiting for the rest of the launch.
template <int N>
struct XRead {
    uint64_t v[N];
    __device__ __forceinline__ void issue(const uint64_t* base, const int (&idx)[N], const bool (&use)[N], uint32_t e) {
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = use[i] ? xld(base, idx[i]) : (static_cast<uint64_t>(e) << 32);
    }
    __device__ __forceinline__ void wait(const uint64_t* base, const int (&idx)[N], uint32_t e, float (&out)[N], uint32_t* err,
                                         bool& failed) {
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
};
template <int N>
__device__ __forceinline__ void xread(const uint64_t* base, const int (&idx)[N], const bool (&use)[N], uint32_t e, float (&out)[N],
                                      uint32_t* err, bool& failed) {
    XRead<N> r;
    r.issue(base, idx, use, e);
    r.wait(base, idx, e, out, err, failed);
}

// A wave-uniform value through an empty asm: conditions derived from it are formed where
// they are used instead of being hoisted out of the layer loop into spilled registers.
__device__ __forceinline__ int opaque_s(int v) {
    asm volatile("" : "+s"(v));
    return v;
}
// threadIdx.x through an empty asm: per-thread offsets derived from it are recomputed in
// each phase instead of being hoisted out of the layer loop and held live across phases.
__device__ __forceinline__ int opaque_tid() {
    int t = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(t));
    return t;
}

// LDS hand-shake words.  A publish only has to follow this wave's earlier LDS accesses,
// so it waits lgkmcnt(0) and stores relaxed: a release store would also wait vmcnt(0),
// i.e. for every load in flight (a loader's whole pipeline of staged loads, or a compute
// wave's pending global stores).
constexpr int kWaitLgkm0 = 0xC07F;  // s_waitcnt lgkmcnt(0), vmcnt/expcnt untouched
constexpr int kWaitVm0 = 0x0F70;    // s_waitcnt vmcnt(0), lgkmcnt/expcnt untouched
// End of a phase that published hand-off values: wait until this wave's stores are
// acknowledged before it issues the next phase's polls and parameter loads.  Measured on
// gfx950: letting the next phase's loads queue behind the stores in flight lengthens the
// hand-off by more than the wait costs (0.8 vs 0.78 ms per step for the c_fc phase alone).
__device__ __forceinline__ void stores_done() { __builtin_amdgcn_s_waitcnt(kWaitVm0); }
__device__ __forceinline__ uint32_t lds_ld(const uint32_t* p) { return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP); }
__device__ __forceinline__ void lds_st(uint32_t* p, uint32_t v) {
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Ring hand-shake words and the compute-wave barrier counter (an LDS object apart from
// the ring).
struct alignas(16) Ctl {
    uint32_t done[kLW];  // loader w: 1 + last chunk index landed (its chunks are w, w+4, ...)
    uint32_t need[kCW];  // compute wave c: first chunk it may still read
    uint32_t bar;        // compute-wave barrier arrivals
};

// Barrier of the 4 compute waves (the loader waves never join it).
__device__ __forceinline__ void cbar(Ctl& ctl, uint32_t& gen, uint32_t* err, bool& failed) {
    gen += kCW;
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);  // this wave's LDS writes are done
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(&ctl.bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    unsigned spins = 0;
    while (lds_ld(&ctl.bar) < gen) {
        if (failed || ++spins > kLdsSpinLimit) {
            if (!failed) atomicOr(err, 1u);
            failed = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
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

// gamma/beta of this thread's 5 LayerNorm columns (tid + 256 i), loaded ahead of the input.
struct LnPar {
    float g[5], b[5];
    __device__ __forceinline__ void load(const float* __restrict__ gp, const float* __restrict__ bp, int tid) {
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            g[i] = gp[tid + 256 * i];
            b[i] = bp[tid + 256 * i];
        }
    }
};
// gamma/beta of this lane's 20 columns in the GEMV's lane order (4 (j*64 + lane) .. + 3).
struct LnParDot {
    float4 g[5], b[5];
    __device__ __forceinline__ void load(const float* __restrict__ gp, const float* __restrict__ bp, int lane) {
#pragma unroll
        for (int j = 0; j < 5; ++j) {
            g[j] = *reinterpret_cast<const float4*>(gp + (j * 64 + lane) * 4);
            b[j] = *reinterpret_cast<const float4*>(bp + (j * 64 + lane) * 4);
        }
    }
};

// Lane holding row k0 + 4 t's sum after wave_sum4 (rows k0 + 4 t, t = 0..3): lanes 0, 32,
// 16, 48 for t = 0, 1, 2, 3; for wave_sum2 (rows k0, k0 + 4): lanes 0 and 32.
__device__ __forceinline__ int row_of_lane4(int lane) { return (lane >> 5) + 2 * ((lane >> 4) & 1); }

// Bias of the row this lane will hold in each of a wave's first NG row groups of a phase
// slice (group g = rows wave + G g + 4 t, G = 16 for 1280-wide rows in groups of four, 8 for
// 5120-wide rows in pairs), loaded while the wave waits for the phase's input so that no row
// waits on a dependent HBM load.  Later groups load their bias when used.
template <int NG, bool kWide>
struct LaneBias {
    float v[NG];
    __device__ __forceinline__ void load(const float* __restrict__ b, int cnt, int wave, int lane) {
        const bool holder = kWide ? (lane & 31) == 0 : (lane & 15) == 0;
        const int t = kWide ? lane >> 5 : row_of_lane4(lane);
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            const int k = wave + (kWide ? 8 : 16) * g + 4 * t;
            v[g] = holder && k < cnt ? b[k] : 0.0f;
        }
    }
};

__device__ __forceinline__ int live_splits_dev(int L, int max_splits) {
    return min(max_splits, max(1, (L + kAttnSplitRows - 1) / kAttnSplitRows));
}

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

// Loader wave lw streams chunks lw, lw + 4, lw + 8, ... of the workgroup's sequence.  Each
// chunk is loaded into registers (kSlots chunks in flight or waiting per wave) and copied
// into its ring slot once every compute wave is past the chunk that used the slot before,
// so HBM keeps streaming while the ring is full and the compute waves wait for a hand-off.
// The loads are unconditional (past the end they re-read the first line of the weights), so
// every chunk issues exactly 5 loads and the compiler's vmcnt waits before each copy leave
// the younger kSlots - 1 chunks in flight.
__device__ __forceinline__ void run_loader(const StepArgs& a, const Plan& P, float* ring, Ctl& ctl, int lw, int lane) {
    const float* __restrict__ W = static_cast<const float*>(a.w);
    const int total = a.layers * P.layer_chunks + P.hn;
    const int owned = total > lw ? (total - lw + kLW - 1) / kLW : 0;
    bool failed = false;
    int cl = P.layer_chunks > 0 ? 0 : a.layers, cr = lw;  // (layer, chunk in layer) of the next chunk to load
    auto norm = [&]() {
        while (cl < a.layers && cr >= P.layer_chunks) {
            cr -= P.layer_chunks;
            ++cl;
        }
    };
    norm();
    typedef float v4f __attribute__((ext_vector_type(4)));  // plain vector type: the slots stay in registers
    v4f slot[kSlots][kLines];
    auto load = [&](v4f(&d)[kLines], int j) {
        const float* base = W;
        uint32_t extent = kChunkF * 4, off[kLines];
        if (j < owned) {
            chunk_src(a, P, W, cl, cr, lane, base, extent, off);
            cr += kLW;
            norm();
        } else {
#pragma unroll
            for (int k = 0; k < kLines; ++k) off[k] = static_cast<uint32_t>(lane * 16);
        }
        // the descriptor base: both halves made scalar and widened as unsigned (readfirstlane
        // returns int, whose sign would otherwise spread into the high half)
        const uint64_t bu = reinterpret_cast<uint64_t>(base);
        const uint32_t blo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(bu))));
        const uint32_t bhi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(bu >> 32))));
        const uint64_t bb = (static_cast<uint64_t>(bhi) << 32) | static_cast<uint64_t>(blo);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(bb), 0,
                                                                           static_cast<int>(__builtin_amdgcn_readfirstlane(static_cast<int>(extent))), kBufferDword3);
#pragma unroll
        for (int k = 0; k < kLines; ++k) d[k] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off[k]), 0, kCachePolicyNt));
    };
#pragma unroll
    for (int s = 0; s < kSlots; ++s) load(slot[s], s);
    uint32_t lim = kRing;  // chunks below lim may be written: min(need) + kRing
    for (int j0 = 0; j0 < owned; j0 += kSlots) {
#pragma unroll
        for (int s = 0; s < kSlots; ++s) {
            const int j = j0 + s;
            if (j < owned) {
                const uint32_t c = static_cast<uint32_t>(lw + kLW * j);
                unsigned spins = 0;
                while (c >= lim) {
                    uint32_t m = lds_ld(&ctl.need[0]);
#pragma unroll
                    for (int i = 1; i < kCW; ++i) m = min(m, lds_ld(&ctl.need[i]));
                    lim = m + kRing;
                    if (c < lim) break;
                    if (failed || ++spins > kLdsSpinLimit) {
                        if (!failed) atomicOr(a.err, 1u);
                        failed = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
                float* dst = ring + (c % kRing) * kChunkF + lane * 4;
#pragma unroll
                for (int k = 0; k < kLines; ++k) *reinterpret_cast<v4f*>(dst + k * 256) = slot[s][k];
                if (lane == 0) lds_st(&ctl.done[lw], c + 1);
            }
            load(slot[s], j + kSlots);
        }
    }
}

// ------------------------------------------------------------------ compute waves

// Wait until chunk c is in the ring (need[] unchanged).
__device__ __forceinline__ const float* wait_chunk(Ctl& ctl, const float* ring, int c, uint32_t* err, bool& failed) {
    unsigned spins = 0;
    while (lds_ld(&ctl.done[c % kLW]) <= static_cast<uint32_t>(c)) {
        if (failed || ++spins > kLdsSpinLimit) {
            if (!failed) atomicOr(err, 1u);
            failed = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    return ring + (c % kRing) * kChunkF;
}
// Wait until chunks c .. c + 3 (one per loader) are all in the ring: one 16-byte read of
// the four done[] words per poll.
__device__ __forceinline__ void wait_run4(Ctl& ctl, int c, uint32_t* err, bool& failed) {
    unsigned spins = 0;
    while (true) {
        // one ds_read_b128 (volatile: re-read every poll); the ring reads that follow are
        // issued only after the branch on this value, and LDS serves a wave's reads in order
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 d = *reinterpret_cast<const volatile u32x4*>(ctl.done);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        const uint32_t dd[4] = {d.x, d.y, d.z, d.w};
        bool ok = true;
#pragma unroll
        for (int m = 0; m < 4; ++m) ok &= dd[(c + m) % kLW] > static_cast<uint32_t>(c + m);
        if (ok) break;
        if (failed || ++spins > kLdsSpinLimit) {
            if (!failed) atomicOr(err, 1u);
            failed = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}
__device__ __forceinline__ void release_to(Ctl& ctl, int c, int wave) {
    if ((threadIdx.x & 63) == 0) lds_st(&ctl.need[wave], static_cast<uint32_t>(c));
}

// acc += dot(chunk, x) for one 1280-float chunk, in the multi-kernel GEMV's order: lane l
// takes 16-byte pieces j*64 + l, j ascending, components x, y, z, w.
__device__ __forceinline__ float dot_chunk(const float* ch, const float* xs, int lane, float acc) {
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        const float4 x4 = *reinterpret_cast<const float4*>(xs + (j * 64 + lane) * 4);
        const float4 w4 = *reinterpret_cast<const float4*>(ch + (j * 64 + lane) * 4);
        acc = __builtin_fmaf(w4.x, x4.x, acc);
        acc = __builtin_fmaf(w4.y, x4.y, acc);
        acc = __builtin_fmaf(w4.z, x4.z, acc);
        acc = __builtin_fmaf(w4.w, x4.w, acc);
    }
    return acc;
}

// A 1280-wide input vector in registers, in the GEMV's lane order: x[j] = floats
// 4 (j*64 + lane) .. +3.  Loaded once per phase and reused by every row group.
struct XRow {
    float4 x[5];
    __device__ __forceinline__ void load(const float* xs, int lane) {
#pragma unroll
        for (int j = 0; j < 5; ++j) x[j] = *reinterpret_cast<const float4*>(xs + (j * 64 + lane) * 4);
    }
};

// x = LayerNorm(row) in the GEMV's lane order, from the raw row in LDS and its statistics.
__device__ __forceinline__ void ln_to_xrow(const float* row, int lane, float mean, float inv, const LnParDot& p, XRow& xr) {
#pragma unroll
    for (int j = 0; j < 5; ++j) {
        const float4 r = *reinterpret_cast<const float4*>(row + (j * 64 + lane) * 4);
        xr.x[j].x = ln_apply(r.x, mean, inv, p.g[j].x, p.b[j].x);
        xr.x[j].y = ln_apply(r.y, mean, inv, p.g[j].y, p.b[j].y);
        xr.x[j].z = ln_apply(r.z, mean, inv, p.g[j].z, p.b[j].z);
        xr.x[j].w = ln_apply(r.w, mean, inv, p.g[j].w, p.b[j].w);
    }
}

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
    (void)wait_chunk(ctl, ring, c0 + k0 + 4 * (nt - 1), err, failed);
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

__global__ __launch_bounds__(kST) void step_kernel(StepArgs a) {
    __shared__ float ring[kRing * kChunkF];
    __shared__ Ctl ctl;
    __shared__ Smem sm;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const SeqState st = *a.state;
    if (!st.active) return;
    if (tid < kLW) ctl.done[tid] = 0;
    if (tid < kCW) ctl.need[tid] = 0;
    if (tid == 0) ctl.bar = 0;
    __syncthreads();  // the only barrier of the whole workgroup; roles split below

    Plan P;
    P.init(st.n, a.splits);
    const int total_chunks = a.layers * P.layer_chunks + P.hn;

    // ================================================================ loaders
    if (wave >= kCW) {
        run_loader(a, P, ring, ctl, __builtin_amdgcn_readfirstlane(wave - kCW), lane);
        return;
    }

    // ================================================================ compute waves
    bool failed = false;
    uint32_t gen = 0;
    uint64_t* __restrict__ X = a.xch;                             // copy 0: written by producers, partials
    const uint64_t* __restrict__ XB = a.xch + xcopy(P.b % kStepCopies, 0);  // this workgroup's copy for reading
    const uint32_t e0 = a.epoch;
    auto ep = [&](int l, uint32_t kind) { return e0 + 8u * static_cast<uint32_t>(l) + kind; };
    const uint32_t n = P.n;

    for (int l = 0; l < a.layers; ++l) {
        const float* __restrict__ par = a.params + static_cast<size_t>(l) * kParLayer;
        const size_t kvl = static_cast<size_t>(l) * a.kv_layer_stride;
        const int cb = l * P.layer_chunks;  // first chunk of this layer

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
            xr.issue(XB, idx, use, ep(l, kEpXh));
            LnParDot ln;
            ln.load(par + kParLn1W, par + kParLn1B, lane);
            LaneBias<kGQkv, false> bias;
            bias.load(par + kParQkvB + P.q0, P.qn, wave, lane);
            float hv[5];
            if (l == 0) {
                // h = mel_emb[token] + mel_pos[position] (gpt.cpp:79-85, kernels.metal:1310-1324)
#pragma unroll
                for (int i = 0; i < 5; ++i) {
                    const int c = tid + 256 * i;
                    hv[i] = a.mel_emb[static_cast<size_t>(st.token) * kWidth + c] + a.mel_pos[static_cast<size_t>(st.position) * kWidth + c];
                }
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
                // 8 arithmetic slots as attention_kernel; a tile has <= 64 rows here (KV capacity
                // <= 4096, checked on the host), so only slots 0..3 can hold a row and slots
                // 4..7 stay constant zeros (-inf scores) exactly as in the multi-kernel path.
                constexpr int PER = kAttnMaxChunk / 16;
                constexpr int PERL = 4;
                float4 k4[PER], v4[PER];
#pragma unroll
                for (int i = 0; i < PER; ++i) {
                    k4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                    v4[i] = k4[i];
                }
                // q and, in the tile holding it, the row appended by this step (row n): loads in
                // flight while the cached rows move from the ring to registers
                const int dn = static_cast<int>(n) - t0 - g;
                const int i_new = (act && static_cast<int>(n) < p1 && dn >= 0 && (dn & 15) == 0 && (dn >> 4) < PERL) ? (dn >> 4) : -1;
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
                // cached rows from the ring; need stays at the tile's first chunk until its rows
                // are in registers
                for (int j = 0; j < 2 * kc; ++j) (void)wait_chunk(ctl, ring, ca + j, a.err, failed);
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
                    d = sum16_up(d);
                    const bool valid = i < PERL && act && t0 + g + 16 * i < p1;
                    sc[i] = valid ? d * 0.125f : -INFINITY;
                    mloc = fmaxf(mloc, sc[i]);
                }
                const float wm = wave_max(mloc);
                if (lane == 0) sm.redm[wave] = wm;
                cbar(ctl, gen, a.err, failed);
                const float M = fmaxf(fmaxf(sm.redm[0], sm.redm[1]), fmaxf(sm.redm[2], sm.redm[3]));
                float lsum = 0.0f;
                float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int i = 0; i < PER; ++i) {
                    const bool valid = i < PERL && act && t0 + g + 16 * i < p1;
                    const float e = valid ? expf(sc[i] - M) : 0.0f;
                    lsum += e;
                    acc.x = __builtin_fmaf(e, v4[i].x, acc.x);
                    acc.y = __builtin_fmaf(e, v4[i].y, acc.y);
                    acc.z = __builtin_fmaf(e, v4[i].z, acc.z);
                    acc.w = __builtin_fmaf(e, v4[i].w, acc.w);
                }
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
    }

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
        auto out = [&](int k, float b, float acc) { a.logits[P.h0 + k] = acc + b; };
        gemv_rows(ctl, ring, chd, P.hn, x, bias, a.head + kHeadBias + P.h0, wave, lane, a.err, failed, out);
        release_to(ctl, total_chunks, wave);
    }
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

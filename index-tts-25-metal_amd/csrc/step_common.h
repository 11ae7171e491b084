// Pieces shared by the persistent decode-step kernels (step.hip: one sequence;
// step_batch.hip: 2-4 sequences): launch shape and chunking constants, the tagged
// exchange between workgroups, the LDS hand-shake words of the loader/compute split, the
// compute-wave barrier, and the LayerNorm and GEMV input helpers.  Every function is an
// inline device function; the kernels include this header inside their own namespaces.
#pragma once
#include "kernels.h"

namespace itts {
namespace stepc {

constexpr int kST = kStepThreads;  // 512
constexpr int kCT = 256;           // compute threads: waves 0..3
constexpr int kCW = kCT / 64;      // compute waves
constexpr int kLW = (kST - kCT) / 64;  // loader waves
constexpr int kLines = 5;          // 1 KB lines per chunk
constexpr int kChunkF = kLines * 256;  // floats per chunk (one 1280-wide row)
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
// Sleep (64 * kPollDelay clocks, about 0.5 us) before a phase's first poll of its input
// vector.  The producers of that vector finish 1-3 us after this workgroup ends its own
// previous phase, and every poll round is a memory-side request per element still missing,
// so rounds issued before the data can exist only add to the queues that the hand-offs and
// the weight stream share (one more unit of hand-off polling made a 752-row step 18% slower).
// Measured (step at 752 cached rows): no sleep 624 us, 8 -> 607, 20 -> 587, 28 -> 594,
// 40 -> 611; a sleep before the attention tiles' q poll and the merge's poll gained nothing.
constexpr int kPollDelay = 20;
constexpr unsigned kLdsSpinLimit = 1u << 24;  // LDS polls (~0.1 us each)
static_assert(kCW == 4 && kLW == 4, "role split");

// Exchange layout (uint64 slots).
constexpr int kXh = 0;
constexpr int kXqkv = kXh + kWidth;
constexpr int kXattn = kXqkv + kQkv;
constexpr int kXhmid = kXattn + kWidth;
constexpr int kXff = kXhmid + kWidth;
constexpr int kXpart = kXff + kFfn;
constexpr int kXlogit = kXpart + kHeads * kAttnMaxSplits * 68;
static_assert(kXlogit + kMelVocab == kStepExchange, "exchange layout");
static_assert(kXpart == kStepBroadcast, "broadcast vectors come first");

enum Kind : uint32_t { kEpXh = 0, kEpQkv = 1, kEpPart = 2, kEpAttn = 3, kEpHmid = 4, kEpFf = 5, kEpLogit = 6 };

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

__device__ __forceinline__ void poll_delay() { __builtin_amdgcn_s_sleep(kPollDelay); }

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
    uint32_t go;         // step.hip: set once layer 0's input row has arrived; loaders start then
    uint32_t last;       // step.hip: this workgroup was the last to finish its mel_head rows
};

// A loader wave's wait for ctl.go (bounded like every wait of the step kernels).
__device__ __forceinline__ void wait_go(Ctl& ctl, uint32_t* err) {
    unsigned spins = 0;
    while (lds_ld(&ctl.go) == 0) {
        if (++spins > kLdsSpinLimit) {
            atomicOr(err, 1u);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

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

// lane_value, ln_layout_load, ln_stats and ln_apply live in common.h.

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

__device__ __forceinline__ int live_splits_dev(int L, int max_splits) { return attn_splits(L, max_splits); }


// Wait until chunk c is in a ring of RING chunks (need[] unchanged).
template <int RING>
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
    return ring + (c % RING) * kChunkF;
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

// Loader wave lw streams chunks lw, lw + 4, lw + 8, ... of the workgroup's sequence.  Each
// chunk is loaded into registers (kSlots chunks in flight or waiting per wave) and copied
// into its ring slot once every compute wave is past the chunk that used the slot before,
// so HBM keeps streaming while the ring is full and the compute waves wait for a hand-off.
// The loads are unconditional (past the end they re-read the first line of the weights), so
// every chunk issues exactly 5 loads and the compiler's vmcnt waits before each copy leave
// the younger kSlots - 1 chunks in flight.
// RING: chunks in the ring; src(l, r, base, extent, off) gives chunk r of layer l (l == layers:
// chunk r of the head rows) as chunk_src does; layer_chunks and head_chunks size the stream.
template <int RING, class Src>
__device__ __forceinline__ void run_loader(const StepArgs& a, int layer_chunks, int head_chunks, float* ring, Ctl& ctl, int lw, int lane,
                                           Src src) {
    const float* __restrict__ W = static_cast<const float*>(a.w);
    const int total = a.layers * layer_chunks + head_chunks;
    const int owned = total > lw ? (total - lw + kLW - 1) / kLW : 0;
    bool failed = false;
    int cl = layer_chunks > 0 ? 0 : a.layers, cr = lw;  // (layer, chunk in layer) of the next chunk to load
    auto norm = [&]() {
        while (cl < a.layers && cr >= layer_chunks) {
            cr -= layer_chunks;
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
            src(cl, cr, base, extent, off);
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
    uint32_t lim = RING;  // chunks below lim may be written: min(need) + RING
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
                    lim = m + RING;
                    if (c < lim) break;
                    if (failed || ++spins > kLdsSpinLimit) {
                        if (!failed) atomicOr(a.err, 1u);
                        failed = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
                float* dst = ring + (c % RING) * kChunkF + lane * 4;
#pragma unroll
                for (int k = 0; k < kLines; ++k) *reinterpret_cast<v4f*>(dst + k * 256) = slot[s][k];
                if (lane == 0) lds_st(&ctl.done[lw], c + 1);
            }
            load(slot[s], j + kSlots);
        }
    }
}

}  // namespace stepc
}  // namespace itts

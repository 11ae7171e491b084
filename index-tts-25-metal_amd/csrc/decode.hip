// Decode-step kernels: LayerNorm-fused FP32/BF16 GEMV family and split-KV decode
// attention, for 1..10 sequences per launch.
//
// GEMV (replaces mit2_linear_gemv_f32, kernels.metal:1054-1080, plus the separate
// layernorm / gelu / add / kv-store / build-current dispatches of gpt.cpp:99-118):
//   * weights row-major [out][in]; each 64-lane wave owns RPW whole rows and streams
//     them with 128-bit (fp32) or 64-bit (bf16) non-temporal loads, all issued before
//     the prologue so the LayerNorm overlaps the weight fetch;
//   * lane l multiplies the 16-byte chunks l, l+64, ... of a row with the matching x
//     chunks, one FMA chain per (row, sequence), then a fixed xor-butterfly wave sum:
//     no atomics, so results are deterministic and identical for every batch size;
//   * the prologue computes LayerNorm(s) of the input row per workgroup (the row is
//     5 KB, cheaper to recompute than to synchronise on); the epilogue adds the bias
//     after the reduction (kernels.metal:1077-1078) and fuses the GELU, the residual
//     add, the q write and the in-place K/V append at cache row n.
// Attention (replaces mit2_gpt_cached_attention_resident_f32, kernels.metal:2064-2145):
//   * grid (splits, 20 heads, batch); a workgroup takes <= 128 consecutive cache rows
//     of one head, 16 lanes per row (one float4 of the 64-dim row each), loads all K
//     and V float4s up front, forms scores (q.k)*rsqrt(64), a max-subtracted exp and a
//     partial sum of weights and weighted V;
//   * a second small kernel merges the splits of each head with the usual rescaling
//     exp(m_s - M) and writes out = sum(w v) / sum(w); the kernel boundary orders the
//     two passes, so no workgroup needs a device-scope fence or atomic.
#include <type_traits>

#include "kernels.h"

namespace itts {
namespace {

constexpr int kNW = 4;  // waves per GEMV workgroup with a LayerNorm prologue (ln_block's layout)

// Splits actually used for L keys (attn_splits).
__device__ __forceinline__ int live_splits(int L, int max_splits) { return attn_splits(L, max_splits); }

// The prologue of a batched GEMV for layer 0's embedding row and the head, once per
// sequence: xn[b] = LayerNorm(s) of sequence b's input row (kProEmbedLn: of h = mel_emb[token]
// + mel_pos[position], also written to h_out).  ln_block<1, 5> is the batch-1 prologue's own
// reduction, so xn[b] holds exactly the values gemv_kernel<.., B = 1, ..> forms in its
// registers.  The per-layer ln_1 and ln_2 are formed inside the batched GEMV instead
// (kProStagedLn: from the staged rows in LDS, while the weights are in flight), which saves
// this launch: 3.3 us per LayerNorm at 8 sequences.
// One wave per sequence: lane l holds columns 64 w + l + 256 i (w < 4, i < 5), the values
// ln_block<1, 5>'s thread 64 w + l holds, and ln_stats forms the statistics in that kernel's
// order, so no barrier is needed.  Gamma and beta are requested with the row, before any store.
template <int PRO>
__global__ __launch_bounds__(64) void ln_seq_kernel(GemvArgs a) {
    const int b = blockIdx.x, lane = threadIdx.x;
    float v[4][5], g[4][5], be[4][5];
    constexpr int NL = PRO == kProLn2 ? 2 : 1;
    float g2[NL][4][5], be2[NL][4][5];
    if constexpr (PRO == kProEmbedLn) {
        const bool live = b < a.nseq;
        const uint32_t tok = live ? a.state[b].token : 0u, pos = live ? a.state[b].position : 0u;
#pragma unroll
        for (int w = 0; w < 4; ++w)
#pragma unroll
            for (int i = 0; i < 5; ++i) {
                const int c = 64 * w + lane + 256 * i;
                v[w][i] = a.mel_emb[static_cast<size_t>(tok) * kWidth + c] + a.mel_pos[static_cast<size_t>(pos) * kWidth + c];
            }
    } else {
#pragma unroll
        for (int w = 0; w < 4; ++w)
#pragma unroll
            for (int i = 0; i < 5; ++i) v[w][i] = a.x[b * a.x_stride + 64 * w + lane + 256 * i];
    }
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int c = 64 * w + lane + 256 * i;
            g[w][i] = a.ln_w[c];
            be[w][i] = a.ln_b[c];
            if constexpr (PRO == kProLn2) {
                g2[0][w][i] = a.ln2_w[c];
                be2[0][w][i] = a.ln2_b[c];
            }
        }
    if constexpr (PRO == kProEmbedLn) {
#pragma unroll
        for (int w = 0; w < 4; ++w)
#pragma unroll
            for (int i = 0; i < 5; ++i) a.h_out[b * kWidth + 64 * w + lane + 256 * i] = v[w][i];
    }
    float mean, inv;
    ln_stats(v, mean, inv);
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int i = 0; i < 5; ++i) v[w][i] = ln_apply(v[w][i], mean, inv, g[w][i], be[w][i]);
    if constexpr (PRO == kProLn2) {
        ln_stats(v, mean, inv);
#pragma unroll
        for (int w = 0; w < 4; ++w)
#pragma unroll
            for (int i = 0; i < 5; ++i) v[w][i] = ln_apply(v[w][i], mean, inv, g2[0][w][i], be2[0][w][i]);
    }
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int i = 0; i < 5; ++i) a.xn[b * kWidth + 64 * w + lane + 256 * i] = v[w][i];
}

// NW waves per workgroup: 4 with a LayerNorm prologue or no input staging; a staged batched
// launch may take 5, so 1280 or 5120 rows make exactly 256 or 512 workgroups and no CU runs
// a workgroup more than the others.
template <int COLS, int RPW, int B, typename WT, int PRO, int EPI, int NW = kNW>
__global__ __launch_bounds__(64 * NW) void gemv_kernel(GemvArgs a) {
    constexpr int J = COLS / 256;  // 16-byte chunks per lane per row
    constexpr int PER = kWidth / 256;
    static_assert(PRO == kProNone || PRO == kProStaged || COLS == kWidth, "LayerNorm prologue is 1280 wide");
    constexpr bool STAGED = PRO == kProStaged || PRO == kProStagedLn;
    static_assert(NW == kNW || STAGED, "only a staged GEMV takes another wave count");
    constexpr int TPB = 64 * NW;
    static_assert(kWidth % TPB == 0, "thread count divides the 1280-column chunk");
    using LD = WLoad<WT>;
    using VT = typename LD::vec;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = (blockIdx.x * NW + wave) * RPW;

    // Prologue input first, so waiting on it does not wait on the weight stream.
    float hv[B][PER];
    if constexpr (PRO == kProLn || PRO == kProLn2) {
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int i = 0; i < PER; ++i) hv[b][i] = a.x[b * a.x_stride + tid + 256 * i];
    } else if constexpr (PRO == kProEmbedLn) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const bool live = b < a.nseq;
            const uint32_t tok = live ? a.state[b].token : 0u, pos = live ? a.state[b].position : 0u;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int c = tid + 256 * i;
                hv[b][i] = a.mel_emb[static_cast<size_t>(tok) * kWidth + c] + a.mel_pos[static_cast<size_t>(pos) * kWidth + c];
            }
        }
    }

    // Staged input: its first 1280 columns requested before the weights too (loads complete in
    // order, so a later request would wait for the whole weight fetch).  16-byte pieces: piece
    // f < B * 320 is columns 4 (f % 320) .. of sequence f / 320.
    // (5120-wide rows, whose four chunks would otherwise hold too many registers at once: 4-byte
    // pieces, thread t taking columns t + TPB i of each sequence.  Holding a second chunk in
    // registers spilled at 8 sequences and measured slower.)
    constexpr bool WIDE = COLS > kWidth;
    constexpr int NCH = COLS / kWidth;             // 1280-column chunks per row
    constexpr int PX = kWidth / TPB;               // columns per thread, sequence and chunk (wide rows)
    constexpr int XF = kWidth / 4;                  // 16-byte pieces per sequence and chunk
    constexpr int NX = WIDE ? B * PX : (B * XF + TPB - 1) / TPB;  // pieces per thread
    using XP = typename std::conditional<WIDE, float, float4>::type;
    // Up to 4 sequences, 5120-wide rows are staged whole: every chunk's pieces requested up
    // front and stored before one barrier, instead of a barrier per chunk (the LDS holds
    // B x 5120 floats, 82 KB at 4).
    constexpr bool FULL = STAGED && WIDE && B <= 4;
    constexpr int NXR = FULL ? NCH * NX : NX;
    XP xr[STAGED ? NXR : 1];
    auto x_piece = [&](int q, int i) -> XP {       // piece tid + TPB i of chunk q
        const int f = tid + TPB * i;
        if constexpr (WIDE) {  // i = b * PX + k: column tid + TPB k of sequence b
            return a.x[(i / PX) * a.x_stride + q * kWidth + tid + TPB * (i % PX)];
        } else {
            return f < B * XF ? *reinterpret_cast<const float4*>(a.x + (f / XF) * a.x_stride + q * kWidth + (f % XF) * 4)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    if constexpr (STAGED) {
#pragma unroll
        for (int i = 0; i < NXR; ++i) xr[i] = x_piece(i / NX, i % NX);
    }
    // kProStagedLn: gamma and beta of the columns t + TPB k this thread normalises, also ahead
    // of the weights.
    constexpr int GC = PRO == kProStagedLn ? kWidth / TPB : 1;
    float gv[GC], bv[GC];
    if constexpr (PRO == kProStagedLn) {
#pragma unroll
        for (int k = 0; k < GC; ++k) {
            gv[k] = a.ln_w[tid + TPB * k];
            bv[k] = a.ln_b[tid + TPB * k];
        }
    }

    const WT* __restrict__ w = static_cast<const WT*>(a.w);
    VT wv[RPW][J];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = row0 + r;
        const int rr = row < a.rows ? row : a.rows - 1;  // clamp: loads stay in bounds, result discarded
#pragma unroll
        for (int j = 0; j < J; ++j) wv[r][j] = LD::load(w, static_cast<size_t>(rr) * (COLS / 4) + j * 64 + lane);
    }
    // The epilogue's (row, sequence) pair of this lane (see the wave_sum4 layout below), and its
    // bias and residual, requested behind the weights so the epilogue does not wait for them.
    constexpr int NV = RPW * B, NK = (NV + 3) / 4;
    const int lw = lane & 15, lg = lane >> 4;
    const int i = 4 * lw + ((lg == 1) ? 2 : (lg == 2) ? 1 : lg);
    const int er = (i < NV ? i : 0) / B, eb = (i < NV ? i : 0) % B;
    const int erow = min(row0 + er, a.rows - 1);  // in bounds; unused when past the rows
    const float ebias = a.bias[erow];
    float eresid = 0.0f;
    if constexpr (EPI == kEpiResid) eresid = a.resid[eb * a.out_stride + erow];
    // Whether any sequence is still decoding.  A replay after every sequence finished still
    // streams the weights once, but stores nothing.
    //   * 8 or more sequences: one vector load (lane b < B reads sequence b's flag) whose answer
    //     is needed only before the stores, when every load has landed.  Read as scalar loads
    //     behind the b < nseq tests, each flag was a round trip of its own, and the eight or
    //     ten of them outlasted the weight stream (batch 8: 6720 -> 6802 decode tokens/s).
    //   * fewer: those scalar loads, read only now that the weights are requested, return within
    //     the weight stream; the vote measured slower there (3 beams: 3415 -> 3368 tokens/s).
    constexpr bool kVote = B >= 8;
    const bool fl_live = kVote && lane < B && lane < a.nseq;
    uint32_t fl = 0;
    if constexpr (kVote) {
        fl = a.state[fl_live ? lane : 0].active;
    } else {
        uint32_t any = 0;
#pragma unroll
        for (int b = 0; b < B; ++b)
            if (b < a.nseq) any |= a.state[b].active;
        if (!any) return;
    }

    __shared__ float xs[PRO == kProNone ? 4 : (FULL ? NCH : STAGED && COLS > kWidth ? 2 : 1) * B * kWidth];
    __shared__ float red[B * kNW];
    if constexpr (PRO != kProNone && !STAGED) {
        if constexpr (PRO == kProEmbedLn) {
            if (blockIdx.x == 0) {
#pragma unroll
                for (int b = 0; b < B; ++b)
#pragma unroll
                    for (int i = 0; i < PER; ++i) a.h_out[b * kWidth + tid + 256 * i] = hv[b][i];
            }
        }
        ln_block<B, PER>(hv, a.ln_w, a.ln_b, red);
        if constexpr (PRO == kProLn2) ln_block<B, PER>(hv, a.ln2_w, a.ln2_b, red);
#pragma unroll
        for (int b = 0; b < B; ++b)
#pragma unroll
            for (int i = 0; i < PER; ++i) xs[b * kWidth + tid + 256 * i] = hv[b][i];
        __syncthreads();
    }

    float acc[RPW][B];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[r][b] = 0.0f;
    if constexpr (STAGED) {
        // x through LDS, 1280 columns at a time (two buffers when there are several chunks):
        // chunk q + 1 is loaded into registers while chunk q's FMAs run.  Per (row, sequence)
        // the FMA chain runs over j in order, as below.
        if constexpr (FULL) {
#pragma unroll
            for (int i = 0; i < NXR; ++i) {
                const int q = i / NX, k = i % NX;
                xs[q * B * kWidth + (k / PX) * kWidth + tid + TPB * (k % PX)] = xr[i];
            }
            __syncthreads();
        }
#pragma unroll
        for (int q = 0; q < NCH; ++q) {
            float* xq = xs + (FULL ? q : (q & 1)) * B * kWidth;
            if constexpr (!FULL) {
#pragma unroll
                for (int i = 0; i < NX; ++i) {
                    const int f = tid + TPB * i;
                    if (WIDE || f < B * XF) {
                        if constexpr (WIDE) {
                            xq[(i / PX) * kWidth + tid + TPB * (i % PX)] = xr[i];
                        } else {
                            *reinterpret_cast<float4*>(xq + (f / XF) * kWidth + (f % XF) * 4) = xr[i];
                        }
                    }
                }
                __syncthreads();
            }
            if constexpr (PRO == kProStagedLn) {
                // Each sequence's mean and 1 / sqrt(var + eps) by one wave, in ln_block<1, 5>'s
                // order (ln_stats), then every element normalised in place, as ln_block does:
                // the rows equal what ln_seq_kernel writes, bit for bit.
                __shared__ float lnst[B][2];
                for (int b = wave; b < B; b += NW) {  // wave-uniform: ln_stats needs all 64 lanes
                    float v[4][5];
                    ln_layout_load(xq + b * kWidth, lane, v);
                    float mean, inv;
                    ln_stats(v, mean, inv);
                    if (lane == 0) {
                        lnst[b][0] = mean;
                        lnst[b][1] = inv;
                    }
                }
                __syncthreads();
#pragma unroll
                for (int b = 0; b < B; ++b)
#pragma unroll
                    for (int k = 0; k < GC; ++k) {
                        float& e = xq[b * kWidth + tid + TPB * k];
                        e = ln_apply(e, lnst[b][0], lnst[b][1], gv[k], bv[k]);
                    }
                __syncthreads();
            }
            if (!FULL && q + 1 < NCH) {
#pragma unroll
                for (int i = 0; i < NX; ++i) xr[i] = x_piece(q + 1, i);
            }
#pragma unroll
            for (int jj = 0; jj < kWidth / 256; ++jj) {
                const int j = q * (kWidth / 256) + jj;
                float4 xv[B];
#pragma unroll
                for (int b = 0; b < B; ++b) xv[b] = *reinterpret_cast<const float4*>(xq + b * kWidth + (jj * 64 + lane) * 4);
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const float4 w4 = LD::to_f4(wv[r][j]);
#pragma unroll
                    for (int b = 0; b < B; ++b) {
                        acc[r][b] = __builtin_fmaf(w4.x, xv[b].x, acc[r][b]);
                        acc[r][b] = __builtin_fmaf(w4.y, xv[b].y, acc[r][b]);
                        acc[r][b] = __builtin_fmaf(w4.z, xv[b].z, acc[r][b]);
                        acc[r][b] = __builtin_fmaf(w4.w, xv[b].w, acc[r][b]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < (STAGED ? 0 : J); ++j) {
        float4 xv[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            if constexpr (PRO == kProNone)
                xv[b] = *reinterpret_cast<const float4*>(a.x + b * a.x_stride + (j * 64 + lane) * 4);
            else
                xv[b] = *reinterpret_cast<const float4*>(xs + b * kWidth + (j * 64 + lane) * 4);
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const float4 w4 = LD::to_f4(wv[r][j]);
#pragma unroll
            for (int b = 0; b < B; ++b) {
                acc[r][b] = __builtin_fmaf(w4.x, xv[b].x, acc[r][b]);
                acc[r][b] = __builtin_fmaf(w4.y, xv[b].y, acc[r][b]);
                acc[r][b] = __builtin_fmaf(w4.z, xv[b].z, acc[r][b]);
                acc[r][b] = __builtin_fmaf(w4.w, xv[b].w, acc[r][b]);
            }
        }
    }
    // The RPW * B sums, four at a time: wave_sum4(a, b, c, d) leaves sum(a) in lanes 0-15,
    // sum(c) in 16-31, sum(b) in 32-47 and sum(d) in 48-63, with wave_sum's pairings, so each
    // sum is bitwise the one wave_sum gives.  Lane L then owns accumulator
    // i = 4 (L & 15) + {0, 2, 1, 3}[L >> 4] (one (row, sequence) pair per lane, no loop over
    // the pairs).
    auto accv = [&](int k) -> float { return k < NV ? acc[k / B][k % B] : 0.0f; };
    float red4[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) red4[k] = wave_sum4(accv(4 * k), accv(4 * k + 1), accv(4 * k + 2), accv(4 * k + 3));
    float sum = red4[0];
#pragma unroll
    for (int k = 1; k < NK; ++k) sum = lw == k ? red4[k] : sum;
    if (kVote && !__any(fl_live && fl != 0)) return;  // every lane of the wave votes, before any leaves
    if (lw >= NK || i >= NV) return;
    const int b = eb;
    const int row = row0 + er;
    if (row >= a.rows) return;
    const float v = sum + ebias;
    if constexpr (EPI == kEpiQkv) {
        if (row < kWidth) {
            a.q[b * kWidth + row] = v;
        } else if (b < a.nseq && a.state[b].active) {
            const int rr = row - kWidth;
            const bool is_v = rr >= kWidth;
            const int c = is_v ? rr - kWidth : rr;
            const size_t off = static_cast<size_t>(b) * a.kv_slot_stride + a.kv_layer_off + (is_v ? a.kv_v_off : 0) +
                               (static_cast<size_t>(c >> 6) * a.kv_cap + a.state[b].n) * kHeadDim + (c & 63);
            a.kv[off] = v;
        }
    } else if constexpr (EPI == kEpiResid) {
        a.out[b * a.out_stride + row] = eresid + v;
    } else if constexpr (EPI == kEpiGelu) {
        a.out[b * a.out_stride + row] = gelu_f(v);
    } else {
        a.out[b * a.out_stride + row] = v;
    }
}

template <int COLS, int RPW, int PRO, int EPI, int B, int NW>
hipError_t launch_b(const GemvArgs& a, bool bf16, hipStream_t s) {
    const int rows_per_wg = NW * RPW;
    const dim3 grid((a.rows + rows_per_wg - 1) / rows_per_wg);
    if (bf16)
        hipLaunchKernelGGL((gemv_kernel<COLS, RPW, B, uint16_t, PRO, EPI, NW>), grid, dim3(64 * NW), 0, s, a);
    else
        hipLaunchKernelGGL((gemv_kernel<COLS, RPW, B, float, PRO, EPI, NW>), grid, dim3(64 * NW), 0, s, a);
    return hipGetLastError();
}

template <int COLS, int RPW, int PRO, int EPI, int NW = kNW>
hipError_t launch_gemv(const GemvArgs& a, int batch, bool bf16, hipStream_t s) {
    switch (gemv_batch_bucket(batch)) {
        case 1: return launch_b<COLS, RPW, PRO, EPI, 1, kNW>(a, bf16, s);
        case 2: return launch_b<COLS, RPW, PRO, EPI, 2, NW>(a, bf16, s);
        case 3: return launch_b<COLS, RPW, PRO, EPI, 3, NW>(a, bf16, s);
        case 4: return launch_b<COLS, RPW, PRO, EPI, 4, NW>(a, bf16, s);
        case 8: return launch_b<COLS, RPW, PRO, EPI, 8, NW>(a, bf16, s);
        case 10: return launch_b<COLS, RPW, PRO, EPI, 10, NW>(a, bf16, s);
        default: return hipErrorInvalidValue;
    }
}

// ------------------------------------------------------------------ attention

// One (sequence b, head h, split s) tile of the split pass.
template <int PER>
__device__ __forceinline__ void attention_tile(const AttnArgs& a, int b, int h, int s, int L, int S);

// The grid is a fixed kAttnGrid workgroups (a captured graph replays it whatever the cache
// lengths are); they walk this step's live tiles t = blockIdx.x, blockIdx.x + gridDim.x, ...
// in the order (sequence, split, head), so no workgroup is launched for a split beyond a
// sequence's live ones.
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a) {
    int off[kMaxBatch + 1];  // first tile of each sequence
    int Ls[kMaxBatch];
    // Every sequence's flag and length requested at once (slots past nseq read slot 0's, then
    // ignored), so the tile walk waits for one round trip instead of one per sequence.
    uint32_t act[kMaxBatch], cached[kMaxBatch];
#pragma unroll
    for (int b = 0; b < kMaxBatch; ++b) {
        const int bb = b < a.nseq ? b : 0;
        act[b] = a.state[bb].active;
        cached[b] = a.state[bb].n;
    }
    off[0] = 0;
#pragma unroll
    for (int b = 0; b < kMaxBatch; ++b) {
        const bool live = b < a.nseq && act[b] != 0;
        Ls[b] = live ? static_cast<int>(cached[b]) + 1 : 0;  // cached rows + the row appended by this step
        off[b + 1] = off[b] + (live ? kHeads * live_splits(Ls[b], a.splits) : 0);
    }
    for (int t = blockIdx.x; t < off[kMaxBatch]; t += gridDim.x) {
        int b = 0;
#pragma unroll
        for (int q = 1; q < kMaxBatch; ++q) b += t >= off[q] ? 1 : 0;
        const int r = t - off[b];
        const int S = live_splits(Ls[b], a.splits);
        // Tiles of at most 64 rows (every cache up to 768 rows) run the code with 4 row slots per
        // 16-lane group; the other slots' zero weights would leave every sum unchanged.
        if ((Ls[b] + S - 1) / S <= 64)
            attention_tile<kAttnMaxChunk / 32>(a, b, r % kHeads, r / kHeads, Ls[b], S);
        else
            attention_tile<kAttnMaxChunk / 16>(a, b, r % kHeads, r / kHeads, Ls[b], S);
        __syncthreads();  // the tile's LDS (redm, reds, accs) is reused by the next one
    }
}

template <int PER>
__device__ __forceinline__ void attention_tile(const AttnArgs& a, int b, int h, int s, int L, int S) {
    const int chunk = (L + S - 1) / S;
    const int p0 = s * chunk;
    const int p1 = min(L, p0 + chunk);
    const int t = threadIdx.x, g = t >> 4, sub = t & 15, lane = t & 63, wave = t >> 6;
    const float4 q4 = *reinterpret_cast<const float4*>(a.q + b * kWidth + h * kHeadDim + sub * 4);

    // Every row's owner slot (beams) is requested before any K/V load, and no load sits under a
    // per-row branch: rows past the tile read its first row (in bounds) and are zeroed after.  The K/V
    // address of a row depends on its owner and loads complete in order, so reading the owner
    // row by row made each row wait for every earlier row's K/V as well (one memory round trip
    // per row); the branches around the loads also cost waits for reused registers.
    const int pz = p0 < L ? p0 : L - 1;  // a row of the cache (the tile's first)
    uint32_t slot[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int p = p0 + g + 16 * i, pc = p < p1 ? p : pz;
        slot[i] = a.table ? a.table[static_cast<size_t>(b) * a.kv_cap + pc] : static_cast<uint32_t>(b);
    }
    float4 k4[PER], v4[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int p = p0 + g + 16 * i, pc = p < p1 ? p : pz;
        const size_t base = static_cast<size_t>(slot[i]) * a.kv_slot_stride + a.kv_layer_off +
                            (static_cast<size_t>(h) * a.kv_cap + pc) * kHeadDim + sub * 4;
        k4[i] = *reinterpret_cast<const float4*>(a.kv + base);
        v4[i] = *reinterpret_cast<const float4*>(a.kv + base + a.kv_v_off);
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        if (!(p0 + g + 16 * i < p1)) {
            k4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            v4[i] = k4[i];
        }
    }
    float sc[PER];
    float mloc = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        float d = q4.x * k4[i].x;
        d = __builtin_fmaf(q4.y, k4[i].y, d);
        d = __builtin_fmaf(q4.z, k4[i].z, d);
        d = __builtin_fmaf(q4.w, k4[i].w, d);
        d = sum16_up(d);
        const bool valid = p0 + g + 16 * i < p1;
        sc[i] = valid ? d * 0.125f : -INFINITY;
        mloc = fmaxf(mloc, sc[i]);
    }
    __shared__ float redm[4], reds[4];
    __shared__ float accs[16][kHeadDim + 4];
    const float wm = wave_max(mloc);
    if (lane == 0) redm[wave] = wm;
    __syncthreads();
    const float M = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
    float lsum = 0.0f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const bool valid = p0 + g + 16 * i < p1;
        const float e = valid ? expf(sc[i] - M) : 0.0f;
        lsum += e;
        acc.x = __builtin_fmaf(e, v4[i].x, acc.x);
        acc.y = __builtin_fmaf(e, v4[i].y, acc.y);
        acc.z = __builtin_fmaf(e, v4[i].z, acc.z);
        acc.w = __builtin_fmaf(e, v4[i].w, acc.w);
    }
    const float ws = wave_sum(sub == 0 ? lsum : 0.0f);
    if (lane == 0) reds[wave] = ws;
    accs[g][sub * 4 + 0] = acc.x;
    accs[g][sub * 4 + 1] = acc.y;
    accs[g][sub * 4 + 2] = acc.z;
    accs[g][sub * 4 + 3] = acc.w;
    __syncthreads();
    float* part = a.partial + (static_cast<size_t>(b * kHeads + h) * a.splits + s) * 68;
    if (t < kHeadDim) {
        float tot = 0.0f;
#pragma unroll
        for (int gg = 0; gg < 16; ++gg) tot += accs[gg][t];
        part[4 + t] = tot;
        if (t == 0) {
            part[0] = M;
            part[1] = ((reds[0] + reds[1]) + reds[2]) + reds[3];
        }
    }
}

// Merge of the splits of one (sequence, head): out = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M).
// The splits are taken as four chains, chain w holding splits w, w+4, ...; each chain's weighted
// sums run in split order, then the four chains' sums are added in chain order.
//   * at most 16 splits (caches up to 1024 rows): one wave runs all four chains, every load
//     issued before the first use, with no LDS and no barrier;
//   * more: wave w of four runs chain w, and the chains meet through LDS.
// Both give the same operations in the same order, so the same bits.
constexpr int kMergeOneWave = 16;
__global__ __launch_bounds__(256) void attention_merge_kernel(AttnArgs a) {
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (b >= a.nseq || !a.state[b].active) return;
    const int S = live_splits(static_cast<int>(a.state[b].n) + 1, a.splits);
    const float* pb = a.partial + static_cast<size_t>(b * kHeads + h) * a.splits * 68;
    if (S <= kMergeOneWave) {
        if (wave != 0) return;  // waves 1-3 have nothing to do on this path
        constexpr int PC = kMergeOneWave / 4;  // splits per chain
        float mk[4][PC], lk[4][PC], ak[4][PC];
#pragma unroll
        for (int w = 0; w < 4; ++w)
#pragma unroll
            for (int i = 0; i < PC; ++i) {
                const int k = w + 4 * i;
                const bool ok = k < S;
                mk[w][i] = ok ? pb[k * 68] : -INFINITY;
                lk[w][i] = ok ? pb[k * 68 + 1] : 0.0f;
                ak[w][i] = ok ? pb[k * 68 + 4 + lane] : 0.0f;
            }
        float wm[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            float m = -INFINITY;
#pragma unroll
            for (int i = 0; i < PC; ++i) m = fmaxf(m, mk[w][i]);
            wm[w] = m;
        }
        const float mg = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
        float den[4], num[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            den[w] = 0.0f;
            num[w] = 0.0f;
#pragma unroll
            for (int i = 0; i < PC; ++i) {
                const float wgt = mk[w][i] == -INFINITY ? 0.0f : expf(mk[w][i] - mg);
                den[w] = __builtin_fmaf(lk[w][i], wgt, den[w]);
                num[w] = __builtin_fmaf(ak[w][i], wgt, num[w]);
            }
            // The four-wave form's chains always end with empty slots (each adds +0, which turns
            // a -0 sum into +0): one such step here keeps even the sign of a zero the same.
            den[w] = __builtin_fmaf(0.0f, 0.0f, den[w]);
            num[w] = __builtin_fmaf(0.0f, 0.0f, num[w]);
        }
        const float d = ((den[0] + den[1]) + den[2]) + den[3];
        const float n = ((num[0] + num[1]) + num[2]) + num[3];
        a.out[b * kWidth + h * kHeadDim + lane] = n / d;
        return;
    }
    constexpr int PW = kAttnMaxSplits / 4;
    float mk[PW], lk[PW], ak[PW];
#pragma unroll
    for (int i = 0; i < PW; ++i) {
        const int k = wave + 4 * i;
        const bool ok = k < S;
        mk[i] = ok ? pb[k * 68] : -INFINITY;
        lk[i] = ok ? pb[k * 68 + 1] : 0.0f;
        ak[i] = ok ? pb[k * 68 + 4 + lane] : 0.0f;
    }
    __shared__ float wm[4], wden[4], wnum[4][kHeadDim];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PW; ++i) m = fmaxf(m, mk[i]);
    if (lane == 0) wm[wave] = m;
    __syncthreads();
    const float mg = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    float den = 0.0f, num = 0.0f;
#pragma unroll
    for (int i = 0; i < PW; ++i) {
        const float wgt = mk[i] == -INFINITY ? 0.0f : expf(mk[i] - mg);
        den = __builtin_fmaf(lk[i], wgt, den);
        num = __builtin_fmaf(ak[i], wgt, num);
    }
    wnum[wave][lane] = num;
    if (lane == 0) wden[wave] = den;
    __syncthreads();
    if (wave == 0) {
        const float d = ((wden[0] + wden[1]) + wden[2]) + wden[3];
        const float n = ((wnum[0][lane] + wnum[1][lane]) + wnum[2][lane]) + wnum[3][lane];
        a.out[b * kWidth + h * kHeadDim + lane] = n / d;
    }
}

}  // namespace

int gemv_batch_bucket(int batch) {
    for (int v : kGemvBatches)
        if (batch <= v) return v;
    return -1;
}

// Batches of 2 or more: the LayerNorm'd inputs are formed once (ln_seq_kernel), and the
// GEMV reads them (or its plain input) through LDS (kProStaged).  At batch 1 the GEMV forms
// the LayerNorm itself, with the same reduction, so every batch size gives the same bits.
template <int PRO>
hipError_t launch_ln_seq(const GemvArgs& a, int batch, hipStream_t s) {
    if (!a.xn) return hipErrorInvalidValue;
    hipLaunchKernelGGL((ln_seq_kernel<PRO>), dim3(gemv_batch_bucket(batch)), dim3(64), 0, s, a);
    return hipGetLastError();
}
GemvArgs staged_on_xn(const GemvArgs& a) {
    GemvArgs b = a;
    b.x = a.xn;
    b.x_stride = kWidth;
    return b;
}

// Rows per wave: chosen so every launch has >= 256 workgroups.  Batched attn.c_proj, mlp.c_fc
// and mlp.c_proj take workgroups of 5 waves: 256, 512 and 256 of them, an equal share per CU
// (with 4 waves, 320, 640 and 320: a quarter or half of the CUs ran one more).
hipError_t launch_gemv_qkv(const GemvArgs& a, int batch, bool bf16, bool embed, hipStream_t s) {
    if (batch >= 2 && !embed) return launch_gemv<kWidth, 2, kProStagedLn, kEpiQkv>(a, batch, bf16, s);
    if (batch >= 2) {
        const hipError_t e = launch_ln_seq<kProEmbedLn>(a, batch, s);
        if (e != hipSuccess) return e;
        return launch_gemv<kWidth, 2, kProStaged, kEpiQkv>(staged_on_xn(a), batch, bf16, s);
    }
    return embed ? launch_gemv<kWidth, 2, kProEmbedLn, kEpiQkv>(a, batch, bf16, s)
                 : launch_gemv<kWidth, 2, kProLn, kEpiQkv>(a, batch, bf16, s);
}
hipError_t launch_gemv_proj(const GemvArgs& a, int batch, bool bf16, hipStream_t s) {
    if (batch >= 2) return launch_gemv<kWidth, 1, kProStaged, kEpiResid, 5>(a, batch, bf16, s);
    return launch_gemv<kWidth, 1, kProNone, kEpiResid>(a, batch, bf16, s);
}
hipError_t launch_gemv_fc(const GemvArgs& a, int batch, bool bf16, hipStream_t s) {
    if (batch >= 2) return launch_gemv<kWidth, 2, kProStagedLn, kEpiGelu, 5>(a, batch, bf16, s);
    return launch_gemv<kWidth, 2, kProLn, kEpiGelu>(a, batch, bf16, s);
}
hipError_t launch_gemv_fc2(const GemvArgs& a, int batch, bool bf16, hipStream_t s) {
    if (batch >= 2) return launch_gemv<kFfn, 1, kProStaged, kEpiResid, 5>(a, batch, bf16, s);
    return launch_gemv<kFfn, 1, kProNone, kEpiResid>(a, batch, bf16, s);
}
hipError_t launch_gemv_head(const GemvArgs& a, int batch, bool bf16, hipStream_t s) {
    if (batch >= 2) {
        const hipError_t e = launch_ln_seq<kProLn2>(a, batch, s);
        if (e != hipSuccess) return e;
        return launch_gemv<kWidth, 2, kProStaged, kEpiLogits>(staged_on_xn(a), batch, bf16, s);
    }
    return launch_gemv<kWidth, 2, kProLn2, kEpiLogits>(a, batch, bf16, s);
}

hipError_t launch_attention(const AttnArgs& a, int batch, hipStream_t s) {
    if (a.nseq > kMaxBatch) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attention_kernel, dim3(std::min(kAttnGrid, a.splits * kHeads * batch)), dim3(256), 0, s, a);
    hipLaunchKernelGGL(attention_merge_kernel, dim3(kHeads, batch), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace itts

// Launch-argument structs and host launch wrappers of every HIP kernel of the
// GPT semantic-token loop.  Kernels live in decode.hip, sampler.hip, prefill.hip
// and util.hip; the runtime (runtime.hip) only calls the wrappers below.
#pragma once
#include "common.h"

namespace itts {

// ------------------------------------------------------------------ decode GEMV
enum Prologue : int {
    kProNone = 0,     // x read from global as is
    kProLn = 1,       // x = LayerNorm(x_in)
    kProEmbedLn = 2,  // h = mel_emb[token] + mel_pos[position] (written out), x = LayerNorm(h)
    kProLn2 = 3,      // x = LayerNorm_b(LayerNorm_a(x_in)) (ln_f then final_norm)
    kProStaged = 4,   // x read from global as is, through LDS in 1280-column chunks (batches)
    kProStagedLn = 5, // kProStaged, then x = LayerNorm(x_in) per sequence in LDS (batches)
};
enum Epilogue : int {
    kEpiQkv = 0,     // q row / K,V cache append at row n
    kEpiResid = 1,   // out = resid + (dot + bias)
    kEpiGelu = 2,    // out = gelu(dot + bias)
    kEpiLogits = 3,  // out = dot + bias
};

struct GemvArgs {
    const void* w;          // [rows][cols] row-major, fp32 or bf16
    const float* bias;      // [rows]
    const float* x;         // input rows [batch][x_stride]
    int x_stride;
    int rows;
    const float* ln_w;      // LayerNorm (first) gamma/beta
    const float* ln_b;
    const float* ln2_w;     // second LayerNorm (kProLn2)
    const float* ln2_b;
    const float* resid;     // kEpiResid input [batch][out_stride]
    float* out;             // [batch][out_stride]
    int out_stride;
    // kEpiQkv
    float* q;               // [batch][1280]
    float* kv;              // cache base
    size_t kv_slot_stride;  // floats per sequence slot
    size_t kv_layer_off;    // floats from slot base to this layer's K block
    size_t kv_v_off;        // floats from the K block to the V block
    uint32_t kv_cap;        // rows per (slot, layer, head)
    // kProEmbedLn
    const float* mel_emb;
    const float* mel_pos;
    float* h_out;           // [batch][1280]
    const SeqState* state;  // [batch]
    int nseq;               // sequences with state entries (<= batch template)
    // batches of 2 or more, layer 0's embedding row and the head: the LayerNorm'd input rows
    // [batch][1280], formed once per launch by a small kernel instead of in every GEMV workgroup
    float* xn;
};

// Batch templates instantiated for the decode GEMVs; the runtime pads a batch up
// to the next of these (extra slots stay inactive).
constexpr int kGemvBatches[] = {1, 2, 3, 4, 8, 10};
int gemv_batch_bucket(int batch);

hipError_t launch_gemv_qkv(const GemvArgs& a, int batch, bool bf16, bool embed, hipStream_t s);
hipError_t launch_gemv_proj(const GemvArgs& a, int batch, bool bf16, hipStream_t s);
hipError_t launch_gemv_fc(const GemvArgs& a, int batch, bool bf16, hipStream_t s);
hipError_t launch_gemv_fc2(const GemvArgs& a, int batch, bool bf16, hipStream_t s);
hipError_t launch_gemv_head(const GemvArgs& a, int batch, bool bf16, hipStream_t s);

// ------------------------------------------------------------------ decode attention
struct AttnArgs {
    const float* q;         // [batch][1280]
    const float* kv;
    size_t kv_slot_stride;
    size_t kv_layer_off;
    size_t kv_v_off;
    uint32_t kv_cap;
    const uint8_t* table;   // beam row-owner table [batch][kv_cap] (slot holding each row) or null
    float* partial;         // [batch][20][splits][68]: m, l, -, -, acc[64]
    float* out;             // [batch][1280]
    const SeqState* state;
    int nseq;               // sequences with state entries; slots >= nseq are padding
    int splits;
};
constexpr int kAttnMaxChunk = 128;   // rows per split at most
constexpr int kAttnSplitRows = 64;   // target rows per split, up to kAttnRoundSplits splits
constexpr int kAttnMaxSplits = 64;   // splits per (sequence, head) at most
constexpr int kAttnRoundSplits = 12;  // 20 heads x 12 splits: one round of a 256-workgroup grid
// Splits of the attention over L keys (at most max_splits, which the host sizes so that no
// split exceeds kAttnMaxChunk rows): about kAttnSplitRows rows each while that takes at most
// kAttnRoundSplits splits, else kAttnRoundSplits splits or, past 12 * 128 keys, splits of up
// to kAttnMaxChunk rows.  Every attention path (decode.hip, step.hip, step_batch.hip) uses
// this rule, so their tiles and merges are the same.
__host__ __device__ inline int attn_splits(int L, int max_splits) {
    const int fine = (L + kAttnSplitRows - 1) / kAttnSplitRows;
    const int coarse = (L + kAttnMaxChunk - 1) / kAttnMaxChunk;
    int s = fine <= kAttnRoundSplits ? fine : (coarse > kAttnRoundSplits ? coarse : kAttnRoundSplits);
    if (s < 1) s = 1;
    return s < max_splits ? s : max_splits;
}
// Split pass (kAttnGrid workgroups walking the live (sequence, split, head) tiles) then
// merge pass (grid 20 x batch).
constexpr int kAttnGrid = 1024;
hipError_t launch_attention(const AttnArgs& a, int batch, hipStream_t s);

// ------------------------------------------------------------------ sampler
enum SampleMode : int {
    kModeDecode = 0,      // processors from state options + seen mask, choose, advance state
    kModeProcessors = 1,  // processors only, write processed scores to out_scores
    kModeDraw = 2,        // logits are already processed: draw `draws` tokens with state.rng
};
struct SampleArgs {
    const float* logits;    // [batch][logit_stride]
    int logit_stride;
    SeqState* state;        // [batch]
    uint8_t* seen;          // [batch][8194] repetition-penalty set
    uint32_t* codes;        // [batch][code_stride]
    int code_stride;
    double* probs;          // [batch][8194] scratch
    uint64_t* sortbuf;      // [batch][16384] scratch (large survivor sets)
    float* out_scores;      // kModeProcessors output [batch][8194]
    uint32_t* out_tokens;   // kModeDraw output
    int draws;
    int mode;
    uint32_t* status;       // [batch] 0 ok, else error code (see sampler.hip)
};
hipError_t launch_sampler(const SampleArgs& a, int batch, hipStream_t s);

// ------------------------------------------------------------------ persistent decode step
// One launch per token for a single sequence (step.hip): grid = one 512-thread
// workgroup per CU, all resident together; workgroups hand vectors over through the exchange buffer
// (tagged 64-bit slots, kStepExchangeTotal of them, zero-initialised once).
constexpr int kStepThreads = 512;
// (the last kMelVocab slots: the logits, read by the fused sampling tail)
constexpr int kStepExchange = kWidth + kQkv + kWidth + kWidth + kFfn + kHeads * kAttnMaxSplits * 68 + kMelVocab;
// The vectors every workgroup reads (h, q|k|v, attention output, hmid, FFN activations:
// the first kStepBroadcast slots) are also written to kStepCopies - 1 further copies
// after the kStepExchange slots, kStepCopyStride apart, and workgroup b reads copy
// b % kStepCopies, so the polling threads spread over more memory channels.  Measured at
// 752 cached rows: polling from a phase's first cycle, 4 copies were 2-4% faster per step
// than 1 and 8 no better than 4; with the poll delay (step_common.h) 2 copies take 580 us,
// 1 copy 580-581 and 4 copies 591 (fewer stores per value), and the batch step is no slower.
constexpr int kStepBroadcast = kWidth + kQkv + kWidth + kWidth + kFfn;
constexpr int kStepCopies = 2;
constexpr int kStepCopyStride = kStepBroadcast + 256;
constexpr size_t kStepExchangeTotal = size_t(kStepExchange) + size_t(kStepCopies - 1) * kStepCopyStride;

struct StepArgs {
    const void* w;            // weight slab, fp32 or bf16
    size_t layer_stride;      // elements per layer block (c_attn, c_proj, c_fc, mlp.c_proj)
    size_t off_head;          // element offset of mel_head
    const float* params;      // [layers][kParLayer]
    const float* head;        // [kHeadPar]
    const float* mel_emb;
    const float* mel_pos;
    float* kv;                // cache of sequence slot 0
    size_t kv_layer_stride;   // floats per layer
    size_t kv_v_off;
    uint32_t kv_cap;
    int layers;
    int splits;               // attention splits at most (as the multi-kernel path)
    const SeqState* state;    // sequence 0
    uint64_t* xch;            // exchange slots
    float* logits;            // [8194]
    uint32_t epoch;           // tag base of this launch (fresh per launch, never 0)
    uint32_t* err;            // set to 1 when a hand-off wait gives up
    // batch step (step_batch.hip): sequences state[0..nseq), KV slots kv + q * kv_slot_stride,
    // logits rows logits + q * logit_stride, exchange regions xch + q * kStepExchangeTotal
    int nseq;
    size_t kv_slot_stride;
    int logit_stride;
    const uint8_t* table;     // beam row-owner table [nseq][kv_cap] (slot holding each row) or null
    // fused sampling tail (step.hip decode steps; null otherwise): after its mel_head rows each
    // workgroup counts itself in *tail; the last one samples the next token with `sample`
    // (kModeDecode, sequence 0) in place of a separate sampler launch, and resets *tail to 0
    uint32_t* tail;
    SampleArgs sample;
    // measurement only (step.hip; null otherwise): workgroup b's clock at the phase ends of
    // layer l, stamps[(b * (layers + 1) + l) * 8 + k], k = 0 layer start, 1 c_attn, 2 attention
    // tiles, 3 merge, 4 attn.c_proj, 5 mlp.c_fc, 6 mlp.c_proj (l = layers: 0 head start, 6 head end)
    uint64_t* stamps;
};
constexpr int kStepStampsPerLayer = 8;
bool step_fits(int grid);
hipError_t step_occupancy(bool bf16, int* blocks_per_cu);
hipError_t launch_step(const StepArgs& a, int grid, bool bf16, hipStream_t s);
// Persistent step for 2..kStepBatchMax sequences (FP32 weights, no beam row-owner table).
constexpr int kStepBatchMax = 4;
bool step_batch_fits(int grid, int nseq);
hipError_t step_batch_occupancy(int nseq, int* blocks_per_cu);
hipError_t launch_step_batch(const StepArgs& a, int nseq, int grid, hipStream_t s);


// ------------------------------------------------------------------ beam search
constexpr int kMaxBeamTake = 2 * kMaxBatch;
struct BeamCand {
    uint32_t parent, token;
    float score;
    uint32_t _pad;
};
struct BeamArgs {
    const float* logits;      // [parents][8194]
    const uint8_t* seen;      // [parents][8194] repetition sets
    const float* beam_score;  // [parents]
    float* all_scores;        // [parents][8194] out of beam_scores, in of beam_select
    double* probs;            // scratch, >= parents * 8194
    uint32_t* list;           // scratch, >= parents * 8194
    uint32_t* status;         // [0] select, [1 + p] scores of parent p
    uint64_t* rng;            // SplitMix64 state of the search
    BeamCand* cand;           // [take]
    int parents, take, do_sample, suppress_stop;
    float temperature, top_p, penalty;
    uint32_t top_k, num_beams;
    const uint32_t* parents_dev;  // the step's parent count on the device (<= parents), or null: parents
    BeamCand* host_cand;          // pinned host copies of cand[0..take) and status[0..parents], written
    uint32_t* host_status;        // by beam_select once it is done (null: none)
};
hipError_t launch_beam_scores(const BeamArgs& a, hipStream_t s);
hipError_t launch_beam_select(const BeamArgs& a, hipStream_t s);
// Children of a beam step on the device (gpt_sampling.cpp:229-236), then the reorder of
// their cached rows' owners and repetition sets, in one launch.
// - Children: from the ranked candidates, skipping stop tokens, the first `beams` become
//   children 0, 1, ... with parent[c], token[c], score[c] (the next step's parent scores)
//   and state[c] (tmpl with n, position and token[c]).  Slots without a child, and every
//   slot when a candidate is out of range (a code >= 8192 or a parent >= *parents_dev: the
//   host raises at that step), are inactive with parent 0 and token 0.  *parents_dev
//   becomes the child count, at least 1.
// - Reorder: every slot's table row (rows 0..n-1) and repetition set are staged, then child
//   c takes parent[c]'s, owns row n itself and adds token[c] to its set.
struct BeamAdvanceArgs {
    const BeamCand* cand;
    int take, beams;
    uint32_t* parents_dev;
    uint32_t *parent, *token;
    float* score;
    SeqState* state;
    const SeqState* tmpl;
    uint32_t n, position, cap;
    uint8_t *table, *table_tmp;  // [beams][cap] row owners
    uint8_t *seen, *seen_tmp;    // [beams][8194] repetition sets
};
hipError_t launch_beam_advance(const BeamAdvanceArgs& a, hipStream_t s);

// ------------------------------------------------------------------ prefill
struct LnRowsArgs {
    const float* x;
    float* y;
    const float* w;
    const float* b;
    int rows;
};
hipError_t launch_ln_rows(const LnRowsArgs& a, hipStream_t s);

// kGemmStore: c[M][N] = dot + bias.  kGemmSwiglu: output columns come in (gate, up) pairs
// 2i, 2i + 1; c[M][N / 2] gets silu(gate) * up (the Qwen MLP with interleaved weight rows).
enum GemmEpi : int { kGemmQkv = 0, kGemmResid = 1, kGemmGelu = 2, kGemmStore = 3, kGemmSwiglu = 4 };
struct GemmArgs {
    const float* a;         // [M][K]
    const void* w;          // [N][K] fp32 or bf16
    const float* bias;      // [N]
    int M, N, K;
    float* c;               // [M][N] (kGemmResid: read-modify-write residual)
    // kGemmQkv: q rows to c ([M][1280]); K/V to the cache of row_slot[m] at row_pos[m]
    float* kv;
    size_t kv_slot_stride, kv_layer_off, kv_v_off;
    uint32_t kv_cap;
    const uint32_t* row_slot;
    const uint32_t* row_pos;
    // split-K: at most `splits` K ranges (multiples of 128); launch_gemm picks the row
    // blocking and the split count from an estimate of the time.  The partial tiles go to
    // ws[splits][M][N] and a second kernel adds them in split order.
    int splits;             // 1: no split
    float* ws;
    // kGemmResid with ln_out (N = 1280): also ln_out[m] = LayerNorm(c[m]; ln_w, ln_b), the
    // next LayerNorm of the residual stream (kernels.metal:618-669), folded into the split-K
    // reduce when there is one
    const float* ln_w;
    const float* ln_b;
    float* ln_out;
};
// The workspace holds kGemmWsFloats floats, which bounds splits * M * N.
constexpr int kGemmMaxSplits = 16;
constexpr size_t kGemmWsFloats = size_t(512) * 64 * 64;
// The split count launch_gemm would use for this shape (callers pass it in GemmArgs.splits;
// 1 forbids splitting).
int gemm_splits(int M, int N, int K);
hipError_t launch_gemm(const GemmArgs& a, int epi, bool bf16, hipStream_t s);

struct CausalArgs {
    const float* q;         // [M][1280]
    const float* kv;
    size_t kv_slot_stride, kv_layer_off, kv_v_off;
    uint32_t kv_cap;
    const uint32_t* row_slot;
    const uint32_t* row_pos;
    float* out;             // [M][1280]
    int M;
};
hipError_t launch_causal_attention(const CausalArgs& a, hipStream_t s);

// ------------------------------------------------------------------ utilities
// dst[out][in] = src[in][out] (Conv1D -> row-major GEMV layout), fp32 or bf16 (RNE).
hipError_t launch_transpose(const float* src, void* dst, int in, int out, bool bf16, hipStream_t s);
hipError_t launch_convert(const float* src, void* dst, size_t n, bool bf16, hipStream_t s);
// Prefix text rows (gpt.cpp:57-69): out[r] = text_emb[ids[r]] + text_pos[r] + lang_emb[lang]; last row mel start.
hipError_t launch_text_rows(const float* text_emb, const float* text_pos, const float* lang_emb, const float* mel_emb,
                            const float* mel_pos, const uint32_t* ids, int n_ids, uint32_t language, float* out,
                            hipStream_t s);
// Speaker conditioning row (gpt.cpp:53-54): out = (bias + W speaker) + emotion.
hipError_t launch_speaker_row(const float* w, const float* b, const float* speaker, const float* emotion, float* out,
                              hipStream_t s);
// seen[b][i] = (i == 1 || i == 8192) for sequences b < nseq: the history {1, 8192}.
hipError_t launch_seen_reset(uint8_t* seen, int nseq, hipStream_t s);
// Prefill rows of one sequence in slot 0: row_slot[r] = 0, row_pos[r] = r (r < rows),
// last_rows[0] = rows - 1, last_rows[1..kMaxBatch) = 0.
hipError_t launch_prefill_rows_one(uint32_t* row_slot, uint32_t* row_pos, uint32_t* last_rows, uint32_t rows, hipStream_t s);
// Copy row src_rows[b] of x into h[b] (last prefix row of each sequence).
hipError_t launch_gather_rows(const float* x, const uint32_t* src_rows, float* h, int batch, hipStream_t s);

}  // namespace itts

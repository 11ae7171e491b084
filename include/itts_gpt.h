/* itts_gpt.h — C ABI of the MI355X-native IndexTTS 2.5 GPT semantic-token loop.
 *
 * The reference has no FFI: its callers link the C++ class itts25::GptDecoder
 * (include/itts25/gpt.hpp:19-43).  This header is the boundary that class is
 * rebuilt on; index-tts-25-metal_amd/cpp/itts25/gpt.hpp keeps the reference's C++
 * signatures on top of it, and the Python binding (index-tts-25-metal_amd/itts_gpt.py)
 * binds it with ctypes.  Plain pointers and sizes only; all pointers are host
 * pointers unless a name says otherwise.
 *
 * Status codes mirror the reference's exception kinds:
 *   ITTS_OK 0, ITTS_EINVAL -1 (std::invalid_argument), ITTS_ERUNTIME -2
 *   (std::runtime_error), ITTS_ELOGIC -3 (std::logic_error).  The message of the
 *   last failure on a handle is returned by itts_gpt_last_error(handle); failures
 *   of itts_gpt_create are reported by itts_gpt_last_error(NULL) (thread local).
 *
 * Threading: one handle = one HIP stream; a handle is not reentrant (as the
 * reference decoder is not, gpt.hpp:22).  Distinct handles may be used from
 * distinct threads.
 */
#ifndef ITTS_GPT_H
#define ITTS_GPT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ITTS_OK 0
#define ITTS_EINVAL (-1)
#define ITTS_ERUNTIME (-2)
#define ITTS_ELOGIC (-3)

#define ITTS_MEL_VOCAB 8194u
#define ITTS_MEL_START 8192u
#define ITTS_MEL_STOP 8193u
#define ITTS_MAX_BATCH 10u

/* One named host tensor, in the reference bundle's names and HF layouts
 * (Conv1D weights [in, out]; mel_head and spk_emb_proj [out, in]).
 * Replaces itts25::Weights::get/info (include/itts25/weights.hpp:9-10). */
typedef struct {
    const char* name;
    const float* data;
    int64_t shape[4];
    int32_t ndim;
    int32_t _pad;
} itts_tensor;

#define ITTS_WEIGHTS_F32 0u
#define ITTS_WEIGHTS_BF16 1u

typedef struct {
    uint32_t kv_capacity;  /* KV rows per sequence; 0 -> 4096 (gpt.cpp:7)            */
    uint32_t max_batch;    /* sequences for generate_batch / beams; 0 -> 1, <= 10     */
    uint32_t weight_dtype; /* ITTS_WEIGHTS_F32 or ITTS_WEIGHTS_BF16 (fp32 accumulate) */
    uint32_t flags;        /* reserved, 0                                             */
} itts_gpt_config;

/* Field meaning of itts25::GenerationOptions (include/itts25/gpt.hpp:7-16), plus
 * suppress_stop: when non-zero, raw logits 8192 and 8193 are set to -inf before
 * any processor so a fixed number of codes is produced (benchmarks; default 0;
 * no reference counterpart). */
typedef struct {
    int32_t do_sample;
    uint32_t _pad0;
    uint64_t seed;
    float temperature;
    uint32_t top_k;
    float top_p;
    float repetition_penalty;
    uint32_t num_beams;
    float length_penalty;
    uint32_t suppress_stop;
    uint32_t _pad1;
} itts_gen_options;

/* Defaults of itts25::GenerationOptions (gpt.hpp:7-16). */
void itts_gen_options_default(itts_gen_options* o);

typedef struct itts_gpt itts_gpt;
typedef struct itts_gpt_state itts_gpt_state;

/* GptDecoder::GptDecoder (gpt.cpp:8-23): checks shapes, uploads weights (Conv1D
 * weights transposed to [out, in] on the device), allocates the KV cache. */
int itts_gpt_create(const itts_tensor* tensors, int32_t count, const itts_gpt_config* cfg, itts_gpt** out);
void itts_gpt_destroy(itts_gpt* h);

/* ---- MIT2 weight bundles (the reference's model format) ----------------------
 * A directory (manifest.json + weights file) or a single file (weights stream +
 * manifest + "MIT2VOIC" footer), memory-mapped.  itts_bundle_open performs the
 * checks of mit2::Bundle::Bundle (vendor/metal-runtime/bundle.cpp:150-266) and of
 * itts25::Weights::Weights (src/weights.cpp:9-28; require_model: the manifest names
 * target "index-tts2.5"), with the same messages, reported by
 * itts_bundle_last_error() (thread local; all are ITTS_ERUNTIME, as the reference's
 * std::runtime_error).  Tensor data pointers stay valid until itts_bundle_close. */
typedef struct itts_bundle itts_bundle;
#define ITTS_DTYPE_F32 0u
#define ITTS_DTYPE_U32 1u
typedef struct {
    const char* name;  /* owned by the bundle */
    const void* data;  /* mapped bytes (host memory) */
    int64_t shape[8];
    int32_t ndim;
    uint32_t dtype;    /* ITTS_DTYPE_F32 or ITTS_DTYPE_U32 */
    uint64_t offset;   /* byte offset in the weights stream */
    uint64_t nbytes;
} itts_bundle_tensor;
int itts_bundle_open(const char* path, int32_t require_model, itts_bundle** out);
void itts_bundle_close(itts_bundle* b);
const char* itts_bundle_last_error(void);
int32_t itts_bundle_count(const itts_bundle* b);
/* mit2::Bundle::tensors()[index] */
int itts_bundle_tensor_at(const itts_bundle* b, int32_t index, itts_bundle_tensor* out);
/* itts25::Weights::info (weights.cpp:29-33): "Missing tensor: <name>" when absent. */
int itts_bundle_find(const itts_bundle* b, const char* name, itts_bundle_tensor* out);
/* GptDecoder(Weights&, ...) (gpt.cpp:8-23) on a bundle: the GPT tensors by their
 * reference names, uploaded straight from the mapping (f32 only, "Expected float32:
 * <name>" otherwise).  Failures are reported by itts_gpt_last_error(NULL). */
int itts_gpt_create_from_bundle(const itts_bundle* b, const itts_gpt_config* cfg, itts_gpt** out);
const char* itts_gpt_last_error(const itts_gpt* h);

/* GptDecoder::prepare (gpt.cpp:42-71): speaker[192], emotion[1280]; writes the
 * prefix (rows x 1280) into prefix_out, which holds capacity_rows rows. */
int itts_gpt_prepare(itts_gpt* h, const float* speaker, const float* emotion, const uint32_t* text, uint32_t n_text,
                     uint32_t language, float* prefix_out, uint32_t capacity_rows, uint32_t* rows);
/* Same prefix with caller-given conditioning rows in place of the reference's
 * [spk_proj(speaker) + emotion, 0, 0] block (gpt.cpp:53-56). */
int itts_gpt_prepare_cond(itts_gpt* h, const float* cond, uint32_t n_cond, const uint32_t* text, uint32_t n_text,
                          uint32_t language, float* prefix_out, uint32_t capacity_rows, uint32_t* rows);

/* GptDecoder::prefill (gpt.cpp:72-78): logits[8194] of the last prefix row. */
int itts_gpt_prefill(itts_gpt* h, const float* prefix, uint32_t rows, float* logits);
/* GptDecoder::step (gpt.cpp:79-85). */
int itts_gpt_step(itts_gpt* h, uint32_t code, uint32_t position, float* logits);
/* GptDecoder::cached_tokens (gpt.hpp:31). */
uint32_t itts_gpt_cached_tokens(const itts_gpt* h);

/* GptDecoder::checkpoint / restore (gpt.cpp:86-87): a device copy of the cached
 * KV rows.  A state is released with itts_gpt_state_release. */
int itts_gpt_checkpoint(itts_gpt* h, itts_gpt_state** out);
int itts_gpt_restore(itts_gpt* h, const itts_gpt_state* state);
uint32_t itts_gpt_state_tokens(const itts_gpt_state* state);
void itts_gpt_state_release(itts_gpt_state* state);

/* GptDecoder::generate (gpt_sampling.cpp:168-245): codes_out holds max_tokens. */
int itts_gpt_generate(itts_gpt* h, const float* prefix, uint32_t rows, const itts_gen_options* options,
                      uint32_t max_tokens, uint32_t* codes_out, uint32_t* n_codes, int32_t* stopped);

/* No counterpart in the reference: itts_gpt_generate (one sequence, num_beams 1) for callers
 * that cannot allocate device memory (tight serving loops, harnesses that forbid hipMalloc).
 * It calls no hipMalloc/hipFree: the prefill activations live in a 28 MiB device array of
 * the library (one per GPU, held until the process ends) instead of buffers grown per call,
 * and a decode graph not captured yet is replaced by eager launches of the same kernels.
 * Same kernels, same codes as itts_gpt_generate.  Limits (ITTS_EINVAL): prefix rows <= 512,
 * num_beams == 1.  Calls on one GPU share that array: within a process they are serialised
 * by a lock; the array keeps the last call's contents. */
int itts_gpt_generate_noalloc(itts_gpt* h, const float* prefix, uint32_t rows, const itts_gen_options* options,
                              uint32_t max_tokens, uint32_t* codes_out, uint32_t* n_codes, int32_t* stopped);

/* No counterpart in the reference: a diagnostic count, process-wide, of the device and
 * pinned-host allocations and graph instantiations the GPT decoders have made.  A call that
 * leaves it unchanged allocated nothing (the check on itts_gpt_generate_noalloc). */
uint64_t itts_gpt_alloc_events(void);

/* Independent requests decoded together (no reference counterpart: the reference
 * runs one request at a time, http.cpp:57).  Sequence b's prefix is prefixes[b]
 * (rows[b] x 1280); each follows generate()'s semantics with options[b].
 * codes_out is [batch][max_tokens]. */
int itts_gpt_generate_batch(itts_gpt* h, uint32_t batch, const float* const* prefixes, const uint32_t* rows,
                            const itts_gen_options* options, uint32_t max_tokens, uint32_t* codes_out,
                            uint32_t* n_codes, int32_t* stopped);

/* The GPT part of NativeRuntime::synthesize's segment loop (src/native_runtime.cpp:98-99),
 * for all of one request's text segments at once.  For segment i:
 *   prefix_i = prepare(speaker, emotion, ids_i, language)   (gpt.cpp:42-71)
 *   result_i = generate(prefix_i, options with seed + i, max_tokens)
 * where ids_i is the next id_counts[i] entries of ids (segments back to back).  Every
 * segment is checked in order, with prepare's and generate's messages, before any work
 * starts.  The prefixes are built on the device, and the segments are decoded together
 * up to max_batch at a time.  With num_beams > 1 they are decoded one at a time.  The
 * codes equal those of the sequential loop.  codes_out is [n_segments][max_tokens].
 * Afterwards cached_tokens() is that of the first segment of the last decoded group. */
int itts_gpt_generate_segments(itts_gpt* h, const float* speaker, const float* emotion, const uint32_t* ids,
                               const uint32_t* id_counts, uint32_t n_segments, uint32_t language,
                               const itts_gen_options* options, uint32_t max_tokens, uint32_t* codes_out,
                               uint32_t* n_codes, int32_t* stopped);
/* Same, with caller-given conditioning rows (n_cond x 1280) in place of the
 * [spk_proj(speaker) + emotion, 0, 0] block, as itts_gpt_prepare_cond. */
int itts_gpt_generate_segments_cond(itts_gpt* h, const float* cond, uint32_t n_cond, const uint32_t* ids,
                                    const uint32_t* id_counts, uint32_t n_segments, uint32_t language,
                                    const itts_gen_options* options, uint32_t max_tokens, uint32_t* codes_out,
                                    uint32_t* n_codes, int32_t* stopped);

/* apply_gpt_sampling_processors (gpt_sampling.cpp:28-128), run on the device. */
int itts_gpt_apply_processors(itts_gpt* h, const float* logits, uint32_t vocab, const uint32_t* history,
                              uint32_t n_history, const itts_gen_options* options, float* out);
/* sample_gpt_token_from_logits (gpt_sampling.cpp:130-165), run on the device with
 * the SplitMix64 state *rng_state (advanced in place), `draws` times. */
int itts_gpt_sample(itts_gpt* h, const float* processed, uint32_t vocab, uint64_t* rng_state, uint32_t draws,
                    uint32_t* tokens);

/* Timing of the last prefill / generate call on the handle's stream, from HIP
 * events (milliseconds).  decode_path: which kernels ran the last decode step or
 * generate loop, ITTS_PATH_MULTI (one launch per GEMV / attention pass, replayed
 * from a captured graph) or ITTS_PATH_STEP (one persistent launch per token). */
#define ITTS_PATH_MULTI 0u
#define ITTS_PATH_STEP 1u
typedef struct {
    float prefill_ms;
    float decode_ms;
    uint32_t decode_steps;
    uint32_t decode_path;
} itts_gpt_timing;
int itts_gpt_last_timing(const itts_gpt* h, itts_gpt_timing* out);

/* Measurement hook (no reference counterpart): launches one decode kernel kind
 * `iters` times back to back on the handle's stream, layer i % layers for launch i, and
 * returns the mean launch duration from HIP events and the algorithmic bytes moved per
 * launch.  which: 0 c_attn GEMV (+LayerNorm, K/V append), 1 attn.c_proj GEMV (+residual),
 * 2 mlp.c_fc GEMV (+LayerNorm, GELU), 3 mlp.c_proj GEMV (+residual), 4 mel_head GEMV
 * (+ln_f, final_norm), 5 decode attention, 6 the persistent whole-step kernel (batch 1,
 * FP32 weights only), 7 a 256 MiB device-to-device copy (reference for traffic counters).
 * Attention and the step kernel run with `cached_rows` rows in the cache (0 -> 752).
 * which | ITTS_BENCH_ONE_LAYER: every launch uses layer 0's weights, so after the first
 * launch they are served from the memory-side cache (the cost of a launch without HBM). */
#define ITTS_BENCH_ONE_LAYER 0x100
int itts_gpt_bench_kernel(itts_gpt* h, int32_t which, uint32_t batch, uint32_t cached_rows, uint32_t iters, float* avg_ms,
                          double* bytes_per_launch);

/* Measurement hook (no reference counterpart): where the persistent batch-1 step kernel's
 * time goes at `cached_rows` cached rows (0 -> 752), from clock stamps the kernel writes at
 * each phase end, averaged over `iters` launches.  phase_us[0] is the mean layer time;
 * phase_us[1..6] the mean share of each phase of a layer on the critical path (c_attn +
 * K/V append, attention tiles, split merge, attn.c_proj, mlp.c_fc, mlp.c_proj), measured
 * from the last workgroup to finish the previous phase to the last to finish this one;
 * phase_us[7] the head (ln_f, final_norm, mel_head).  FP32 decoders with the persistent
 * path only. */
int itts_gpt_step_phases(itts_gpt* h, uint32_t cached_rows, uint32_t iters, float* phase_us);
/* The same for the persistent batch step kernel with `nseq` (2-4) sequences, each at
 * `cached_rows` cached rows: the forward that batches of 2-4 and beam search run when the
 * decoder was created with max_batch >= nseq and ITTS_GPT_PERSISTENT_BATCH=1 (else the
 * call fails with an invalid-argument status). */
int itts_gpt_step_phases_batch(itts_gpt* h, uint32_t nseq, uint32_t cached_rows, uint32_t iters, float* phase_us);

/* ---- EnhancedCodec (src/codec.cpp), the consumer of the semantic codes ----------
 * The decode path of itts25::EnhancedCodec (include/itts25/codec.hpp:11-17) on the
 * MI355X: codes -> [2T][1024] time-major features.  encode() is not provided. */
typedef struct itts_codec itts_codec;
/* EnhancedCodec::EnhancedCodec (codec.cpp:5-20): the decode path's tensors by their
 * reference names (codebook, out_project, codec.decoder.*, codec.up), with the
 * reference's "Unsupported 2.5 codec shape: <name>" check (ITTS_ERUNTIME).  Failures are
 * reported by itts_codec_last_error(NULL) (thread local). */
int itts_codec_create(const itts_tensor* tensors, int32_t count, itts_codec** out);
/* The same from a MIT2 bundle's codec.* tensors (f32), uploaded from the mapping. */
int itts_codec_create_from_bundle(const itts_bundle* b, itts_codec** out);
void itts_codec_destroy(itts_codec* c);
const char* itts_codec_last_error(const itts_codec* c);
/* EnhancedCodec::decode (codec.cpp:64-72): n codes in [0, 8192), 1 <= n <= 5000
 * ("Codec expects 1..5000 code IDs in [0,8192)", ITTS_EINVAL); out holds 2n x 1024. */
int itts_codec_decode(itts_codec* c, const uint32_t* codes, uint32_t n, float* out);
/* Measurement hook (no reference counterpart): mean duration of the device work of a
 * decode of n codes over `iters` back-to-back runs (HIP events), and its GEMM FLOPs. */
int itts_codec_bench(itts_codec* c, uint32_t n, uint32_t iters, float* avg_ms, double* flops);

/* Verification hook (no reference counterpart): the device expf / exp / logf that the
 * sampler and beam kernels use in place of the reference's libm calls
 * (gpt_sampling.cpp:96, :144, :207-210), evaluated on the float inputs whose bit patterns
 * are first_bits + i * stride, i < count (<= 2^28).  ITTS_LIBM_EXP takes each float widened
 * to double and writes doubles; the others write floats.  out is host memory. */
#define ITTS_LIBM_EXPF 0
#define ITTS_LIBM_EXP 1
#define ITTS_LIBM_LOGF 2
int itts_libm_eval(int32_t fn, uint64_t first_bits, uint64_t stride, uint64_t count, void* out);
/* Verification hook (no reference counterpart): out[r] = the float sum, in index order, of
 * row r of values (rows x 8194 floats, each >= 0 or NaN), as the beam scores form the
 * log-softmax denominator (gpt_sampling.cpp:208), with the same device code.  values and
 * out are host memory; rows <= 65536. */
int itts_chain_sum_eval(const float* values, uint32_t rows, float* out);

/* Deterministic N(mean, std^2) fill for synthetic weights and inputs: value i is
 * a Box-Muller transform of two SplitMix64 outputs keyed by (seed, i), so the
 * result does not depend on thread count.  Host only. */
void itts_synthetic_normal(float* out, size_t n, uint64_t seed, float mean, float stddev);

#ifdef __cplusplus
}
#endif
#endif

/* C ABI of the MI355X-native Qwen3-0.6B emotion-text decoder.
 *
 * Replaces itts25::QwenDecoder (include/itts25/qwen.hpp:5-18, src/qwen.cpp:5-49), the
 * greedy decoder that turns an emotion description into the emotion vector's text.  The
 * status codes, itts_tensor and itts_bundle are those of itts_gpt.h.  A handle owns the
 * device weights, a 4096-row KV cache and one HIP stream; it is not reentrant (the
 * reference decoder is not either).  Messages of failed calls are reported by
 * itts_qwen_last_error(handle), those of itts_qwen_create* by itts_qwen_last_error(NULL)
 * (thread local).
 */
#ifndef ITTS_QWEN_H
#define ITTS_QWEN_H

#include <stddef.h>
#include <stdint.h>

#include "itts_gpt.h"

#ifdef __cplusplus
extern "C" {
#endif

#define ITTS_QWEN_VOCAB 151936u
#define ITTS_QWEN_EOS 151643u
#define ITTS_QWEN_LAYERS 28u

typedef struct itts_qwen itts_qwen;

typedef struct {
    uint32_t layers; /* decoder layers; 0 -> 28, the reference's (qwen.cpp:8) */
    uint32_t flags;  /* reserved, 0 */
} itts_qwen_config;

/* QwenDecoder::QwenDecoder (qwen.cpp:5-15): the tensors by their reference names
 * (qwen.model.embed_tokens.weight, qwen.model.layers.<i>.*, qwen.model.norm.weight), f32.
 * "Unsupported Qwen shape: <name>" (ITTS_EINVAL) for a tensor of another shape and
 * "Missing tensor: <name>" (ITTS_ERUNTIME) for an absent one, as Weights::info
 * (weights.cpp:29-33); the norm weights, which the reference reads at run time, are checked
 * here too. */
int itts_qwen_create(const itts_tensor* tensors, int32_t count, const itts_qwen_config* cfg, itts_qwen** out);
/* The same from a MIT2 bundle's qwen.* tensors (f32), uploaded from the mapping. */
int itts_qwen_create_from_bundle(const itts_bundle* b, const itts_qwen_config* cfg, itts_qwen** out);
void itts_qwen_destroy(itts_qwen* q);
const char* itts_qwen_last_error(const itts_qwen* q);

/* QwenDecoder::prefill (qwen.cpp:20): 1..3072 ids < 151936 ("Qwen prompt capacity is 3072
 * tokens", "Invalid Qwen token"; ITTS_EINVAL); the cache restarts at the prompt.  logits
 * (host) receives the 151936 logits of the last id. */
int itts_qwen_prefill(itts_qwen* q, const uint32_t* ids, uint32_t n, float* logits);
/* QwenDecoder::step (qwen.cpp:21): one id at the next cache row ("Qwen cache capacity
 * exceeded" before a prefill or at 4096 rows, then "Invalid Qwen token"; ITTS_EINVAL). */
int itts_qwen_step(itts_qwen* q, uint32_t id, float* logits);
/* QwenDecoder::generate (qwen.cpp:46-49): prefill, then greedy steps on the device (the
 * argmax picks the first index of the maximum, kernels.metal:1269-1305) until EOS 151643,
 * which is included.  out (host) holds `maximum` ids; *count receives the number written,
 * also when the call fails with "Qwen did not reach EOS within 1024 generated tokens"
 * (ITTS_ERUNTIME) after `maximum` ids.  Checked first: 1 <= maximum <= 1024 and
 * n + maximum <= 4096 ("Qwen generation capacity exceeded"), then the prompt as prefill's. */
int itts_qwen_generate(itts_qwen* q, const uint32_t* ids, uint32_t n, uint32_t maximum, uint32_t* out, uint32_t* count);
/* QwenDecoder::submissions (qwen.hpp:11): forward passes run so far (a prefill or one step
 * each), the reference's count of command buffers. */
uint64_t itts_qwen_submissions(const itts_qwen* q);

/* Measurement hook (no reference counterpart): HIP-event time of a prefill of `prompt`
 * synthetic ids, and the mean time of `iters` decode steps starting at `cached_rows`
 * cache rows (cached_rows + iters + 2 <= 4096); the cache contents are whatever a previous
 * call left. */
int itts_qwen_bench(itts_qwen* q, uint32_t prompt, uint32_t cached_rows, uint32_t iters, float* prefill_ms, float* step_us);

#ifdef __cplusplus
}
#endif
#endif

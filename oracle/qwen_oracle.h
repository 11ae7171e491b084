/* CPU oracle for the Qwen3-0.6B emotion-text decoder (itts25::QwenDecoder).
 *
 * TEST INFRASTRUCTURE ONLY.  A plain FP32 C++ restatement of src/qwen.cpp:5-49 and
 * of the Metal ops it calls; the HIP path is compared against it.  Nothing in the
 * product links it.
 *
 * Pinning (what checks each function, other than retyping it):
 *   orc_qwen_prefill / orc_qwen_step
 *       Hugging Face transformers' Qwen3ForCausalLM (an independent implementation of
 *       the same architecture), run in float64 on the same weights: last-row logits of
 *       a prefill and teacher-forced step logits (tests/test_qwen_oracle.py).  Each
 *       mistake that orc_qwen_set_mutation plants (GQA head mapping, RoPE rotation
 *       sign, a skipped q/k norm, RoPE without the cache offset, SiLU on the wrong
 *       half) must fail that comparison.  KV invariant: prefill(n) + step == the last
 *       row of prefill(n + 1).
 *   orc_qwen_generate
 *       greedy: each token is the first index of the maximum of the teacher-forced
 *       logits; EOS handling and capacity errors by their closed forms.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#include "gpt_oracle.h"

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QWEN_VOCAB 151936u
#define ORC_QWEN_EOS 151643u

typedef struct orc_qwen orc_qwen;

/* QwenDecoder::QwenDecoder (qwen.cpp:5-15) with `layers` decoder layers (the reference
 * has 28).  Copies the tensors.  NULL with err filled on a missing or ill-shaped tensor
 * ("Missing tensor: <name>", "Unsupported Qwen shape: <name>"). */
orc_qwen* orc_qwen_create(const orc_tensor* tensors, int32_t count, uint32_t layers, char* err, size_t err_len);
void orc_qwen_destroy(orc_qwen* m);
uint32_t orc_qwen_cached(const orc_qwen* m);

/* qwen.cpp:20-22.  logits holds 151936 floats.  0, or -1 invalid_argument / -2
 * runtime_error with orc_last_error() holding the reference's message. */
int orc_qwen_prefill(orc_qwen* m, const uint32_t* ids, uint32_t n, float* logits);
int orc_qwen_step(orc_qwen* m, uint32_t id, float* logits);
/* qwen.cpp:46-49: out holds `maximum` tokens; *count is set to the tokens produced, also
 * when the call ends with "Qwen did not reach EOS within 1024 generated tokens" (-2). */
int orc_qwen_generate(orc_qwen* m, const uint32_t* ids, uint32_t n, uint32_t maximum, uint32_t* out, uint32_t* count);
/* Row `pos` of the K (is_v = 0) or V cache of `layer` (1024 floats: 8 heads x 128). */
int orc_qwen_kv_row(const orc_qwen* m, uint32_t layer, int32_t is_v, uint32_t pos, float* out);

/* Test hook: plants a known mistake in the forward (0 = none; 1 = query head h reads kv
 * head h % 8; 2 = RoPE rotation with the opposite sign; 3 = q_norm/k_norm skipped; 4 =
 * RoPE positions without the cache offset; 5 = SiLU applied to up instead of gate). */
void orc_qwen_set_mutation(orc_qwen* m, int32_t mutation);

#ifdef __cplusplus
}
#endif

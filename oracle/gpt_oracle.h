/* CPU oracle for the IndexTTS 2.5 GPT semantic-token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain FP32 C++ restatement of the
 * reference op sequence (src/gpt.cpp:42-125) and of its sampler / generation
 * loop (src/gpt_sampling.cpp:11-245).  The HIP path is compared against it, and it is
 * the timed CPU baseline; nothing in the product links it.
 *
 * Pinning (what checks each function, other than retyping it):
 *   orc_splitmix_*        published SplitMix64 test vectors; the reference's own
 *                         sampler compiled from its sources (oracle/_ref).
 *   orc_processors        oracle/_ref (reference gpt_sampling.cpp compiled as is)
 *                         on random and tie-heavy logits; brute-force tie cases.
 *   orc_sample            oracle/_ref, same inputs and RNG stream.
 *   orc_prefill/orc_step  an independent float64 numpy forward on small shapes;
 *                         KV-cache invariants (step-by-step == full recompute;
 *                         prefill last row == stepping from one row).
 *   orc_prepare_*         exact gather-and-add identities.
 *   orc_generate          greedy reduces to argmax of teacher-forced logits;
 *                         sampled path == processors + sample per step (_ref).
 *   orc_generate (beams)  exhaustive search on a bias-only head, where beam search
 *                         must return the best hypothesis (tests/beam_brute.py), and a
 *                         hand-derived case for the -1e9 initial beam scores
 *                         (tests/test_beam_oracle.py).
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    const char* name;
    const float* data;
    int64_t shape[4];
    int32_t ndim;
    int32_t _pad;
} orc_tensor;

/* Same field meaning as itts25::GenerationOptions (include/itts25/gpt.hpp:7-16)
 * plus suppress_stop: when non-zero, raw logits 8192 and 8193 are set to -inf
 * before any processor (fixed-length benchmark runs only; default off). */
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
} orc_options;

typedef struct orc_model orc_model;

/* Returns NULL and fills err (if given) on a missing/ill-shaped tensor. */
orc_model* orc_create(const orc_tensor* tensors, int32_t count, uint32_t kv_capacity, char* err, size_t err_len);
void orc_destroy(orc_model* m);
uint32_t orc_width(const orc_model* m);
uint32_t orc_cached_tokens(const orc_model* m);

/* Prefix builders (gpt.cpp:42-71).  orc_prepare_ref follows the reference exactly
 * (speaker[192] -> spk_emb_proj, + emotion, two zero rows).  orc_prepare_cond
 * takes the conditioning rows directly (synthetic latents).  Output rows are
 * returned through *rows; prefix_out must hold (n_cond + n_text + 3) * width. */
int orc_prepare_ref(orc_model* m, const float* speaker, const float* emotion, const uint32_t* text, uint32_t n_text,
                    uint32_t language, float* prefix_out, uint32_t* rows);
int orc_prepare_cond(orc_model* m, const float* cond, uint32_t n_cond, const uint32_t* text, uint32_t n_text,
                     uint32_t language, float* prefix_out, uint32_t* rows);

/* gpt.cpp:72-85: prefill resets the cache; step appends one row. */
int orc_prefill(orc_model* m, const float* prefix, uint32_t rows, float* logits);
int orc_step(orc_model* m, uint32_t code, uint32_t position, float* logits);
/* gpt.cpp:86-87: a copy of the cached K/V rows, and its restore (NULL on error). */
typedef struct orc_state orc_state;
orc_state* orc_checkpoint(const orc_model* m);
int orc_restore(orc_model* m, const orc_state* st);
void orc_state_free(orc_state* st);
/* Read back the K or V row `pos` of layer `layer` (width floats). */
int orc_kv_row(const orc_model* m, uint32_t layer, int32_t is_v, uint32_t pos, float* out);

/* gpt_sampling.cpp:28-128 and 130-165. */
int orc_processors(const float* logits, uint32_t vocab, const uint32_t* history, uint32_t n_history,
                   const orc_options* opt, float* out);
int orc_sample(const float* processed, uint32_t vocab, uint64_t* rng_state, uint32_t* token);
uint64_t orc_splitmix_next(uint64_t* state);
double orc_splitmix_unit(uint64_t* state);

/* gpt_sampling.cpp:168-245.  codes_out holds max_tokens entries. */
int orc_generate(orc_model* m, const float* prefix, uint32_t rows, const orc_options* opt, uint32_t max_tokens,
                 uint32_t* codes_out, uint32_t* n_codes, int32_t* stopped);

/* The C library's expf(x) (fn 0), exp((double)x) (fn 1) or logf(x) (fn 2) on the float
 * inputs with bit patterns first + i * stride, i < count: the libm calls of
 * gpt_sampling.cpp:96, :144, :207-210, for comparison with the device's. */
void orc_libm_eval(int32_t fn, uint64_t first, uint64_t stride, uint64_t count, void* out);

/* Elementwise pieces exposed for kernel-level tests. */
float orc_gelu(float v);
void orc_layernorm(const float* x, const float* g, const float* b, uint32_t width, float eps, float* out);

const char* orc_last_error(void);

#ifdef __cplusplus
}
#endif

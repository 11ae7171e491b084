// Drop-in replacement of the reference's include/itts25/gpt.hpp (lines 7-43): same
// types, member functions, arguments and exception kinds, implemented over the HIP C ABI
// (include/itts_gpt.h).  The constructor keeps the reference's two-argument form so
// `GptDecoder gpt_(weights_, metal_)` (src/pipeline.cpp:12) compiles unchanged: it reads
// the GPT tensors from any Weights type with the reference's info(name).shape / get(name)
// interface (include/itts25/weights.hpp:9-10); the device context argument is not used
// (the decoder owns its HIP stream).
#pragma once
#include <cstdint>
#include <memory>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "itts_gpt.h"
#include "itts25/bundle_weights.hpp"

namespace itts25 {

struct GenerationOptions {
    bool do_sample = true;
    uint64_t seed = 20261002;
    float temperature = 0.8f;
    uint32_t top_k = 30;
    float top_p = 0.8f;
    float repetition_penalty = 10.0f;
    uint32_t num_beams = 1;
    float length_penalty = 0;
};
struct GenerationResult {
    std::vector<uint32_t> codes;
    bool stopped = false;
};
struct GptKvSnapshot;  // device copy of the cached KV rows
struct GptState {
    uint32_t tokens = 0;
    std::shared_ptr<GptKvSnapshot> kv;
};

// gpt_sampling.cpp:28-128, run on the device.
std::vector<float> apply_gpt_sampling_processors(const std::vector<float>& logits, const std::vector<uint32_t>& history,
                                                 const GenerationOptions& options);

class GptDecoder {
public:
    struct Tensor {
        std::string name;
        std::vector<int64_t> shape;
        const std::vector<float>* data;
    };

    // The reference accepts num_beams up to 10 on any decoder (gpt_sampling.cpp:172-173),
    // so the reference-form constructor provisions 10 KV slots (10 x 503 MB at capacity 4096).
    // Weights types: the reference's Weights (its bundle().root() names the MIT2 bundle,
    // which is re-opened here and uploaded straight from the mapping), this library's
    // BundleWeights (the same, from its open bundle), or any type with info()/get() (the
    // tensors are taken through get()).
    template <class AnyWeights, class Context>
    GptDecoder(AnyWeights& weights, Context& /*device context, unused*/) : handle_(create(weights)) {}
    static constexpr itts_gpt_config kReferenceConfig{4096, ITTS_MAX_BATCH, ITTS_WEIGHTS_F32, 0};
    explicit GptDecoder(const std::vector<Tensor>& tensors, const itts_gpt_config* config = nullptr);
    GptDecoder(const itts_bundle* bundle, const itts_gpt_config* config);
    ~GptDecoder();
    GptDecoder(const GptDecoder&) = delete;
    GptDecoder& operator=(const GptDecoder&) = delete;

    std::vector<float> prepare(const std::vector<float>& speaker, const std::vector<float>& emotion,
                               const std::vector<uint32_t>& text, uint32_t language);
    std::vector<float> prefill(const std::vector<float>& prefix);
    std::vector<float> step(uint32_t code, uint32_t position);
    GenerationResult generate(const std::vector<float>& prefix, const GenerationOptions& options, uint32_t max_tokens = 1500);
    // The GPT part of NativeRuntime::synthesize's segment loop (src/native_runtime.cpp:98-99)
    // for all of a request's text segments at once: result i equals
    // generate(prepare(speaker, emotion, segments[i], language), options with seed + i,
    // max_tokens).  No counterpart among the reference's members: it replaces that loop's
    // prepare/generate calls, decoding the segments together on the device.
    std::vector<GenerationResult> generate_segments(const std::vector<float>& speaker, const std::vector<float>& emotion,
                                                    const std::vector<std::vector<uint32_t>>& segments, uint32_t language,
                                                    const GenerationOptions& options, uint32_t max_tokens = 1500);
    GptState checkpoint() const;
    void restore(const GptState& state);
    uint32_t cached_tokens() const;

private:
    itts_gpt* handle_ = nullptr;

    template <class W, class = void>
    struct has_handle : std::false_type {};
    template <class W>
    struct has_handle<W, std::void_t<decltype(std::declval<const W&>().handle())>> : std::true_type {};
    template <class W, class = void>
    struct has_bundle_root : std::false_type {};
    template <class W>
    struct has_bundle_root<W, std::void_t<decltype(std::string(std::declval<W&>().bundle().root()))>> : std::true_type {};

    static itts_gpt* create_from_bundle(const itts_bundle* bundle, const itts_gpt_config* config);
    static itts_gpt* create_from_path(const std::string& bundle_path, const itts_gpt_config* config);
    static itts_gpt* create_from_tensors(const std::vector<Tensor>& tensors, const itts_gpt_config* config);
    template <class W>
    static itts_gpt* create(W& w) {
        if constexpr (has_handle<W>::value) return create_from_bundle(w.handle(), &kReferenceConfig);
        else if constexpr (has_bundle_root<W>::value) return create_from_path(std::string(w.bundle().root()), &kReferenceConfig);
        else return create_from_tensors(collect(w), &kReferenceConfig);
    }
    template <class AnyWeights>
    static std::vector<Tensor> collect(AnyWeights& w) {
        std::vector<Tensor> out;
        auto add = [&](const std::string& name) { out.push_back({name, w.info(name).shape, &w.get(name)}); };
        for (const char* n : {"gpt.spk_emb_proj.weight", "gpt.spk_emb_proj.bias", "gpt.text_embedding.weight",
                              "gpt.text_pos_embedding.emb.weight", "gpt.lang_embedding.weight", "gpt.mel_embedding.weight",
                              "gpt.mel_pos_embedding.emb.weight", "gpt.gpt.ln_f.weight", "gpt.gpt.ln_f.bias",
                              "gpt.final_norm.weight", "gpt.final_norm.bias", "gpt.mel_head.weight", "gpt.mel_head.bias"})
            add(n);
        for (uint32_t i = 0; i < 24; ++i) {
            const std::string p = "gpt.gpt.h." + std::to_string(i);
            for (const char* n : {".ln_1.weight", ".ln_1.bias", ".attn.c_attn.weight", ".attn.c_attn.bias", ".attn.c_proj.weight",
                                  ".attn.c_proj.bias", ".ln_2.weight", ".ln_2.bias", ".mlp.c_fc.weight", ".mlp.c_fc.bias",
                                  ".mlp.c_proj.weight", ".mlp.c_proj.bias"})
                add(p + n);
        }
        return out;
    }
    void check(int status) const;
};

}  // namespace itts25

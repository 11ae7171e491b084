// itts25::GptDecoder over the HIP C ABI (include/itts_gpt.h).  Same member semantics,
// error kinds and messages as the reference's src/gpt.cpp:42-125 and
// src/gpt_sampling.cpp:168-245; the math runs in libitts_gpt.so on the MI355X.
#include "itts25/gpt.hpp"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <stdexcept>

namespace itts25 {

struct GptKvSnapshot {
    itts_gpt_state* state = nullptr;
    ~GptKvSnapshot() { itts_gpt_state_release(state); }
};

namespace {

[[noreturn]] void rethrow(int status, const char* message) {
    const std::string m = message ? message : "";
    if (status == ITTS_EINVAL) throw std::invalid_argument(m);
    if (status == ITTS_ERUNTIME) throw std::runtime_error(m);
    throw std::logic_error(m);
}

itts_gen_options to_c(const GenerationOptions& o) {
    itts_gen_options c;
    itts_gen_options_default(&c);
    c.do_sample = o.do_sample ? 1 : 0;
    c.seed = o.seed;
    c.temperature = o.temperature;
    c.top_k = o.top_k;
    c.top_p = o.top_p;
    c.repetition_penalty = o.repetition_penalty;
    c.num_beams = o.num_beams;
    c.length_penalty = o.length_penalty;
    return c;
}

itts_gpt* sampler_handle() {
    static std::once_flag once;
    static itts_gpt* h = nullptr;
    std::call_once(once, [] {
        if (itts_gpt_create(nullptr, 0, nullptr, &h) != ITTS_OK) rethrow(ITTS_ERUNTIME, itts_gpt_last_error(nullptr));
    });
    return h;
}

}  // namespace

std::vector<float> apply_gpt_sampling_processors(const std::vector<float>& logits, const std::vector<uint32_t>& history,
                                                 const GenerationOptions& options) {
    itts_gpt* h = sampler_handle();
    std::vector<float> out(logits.size());
    const itts_gen_options c = to_c(options);
    const int st = itts_gpt_apply_processors(h, logits.data(), static_cast<uint32_t>(logits.size()), history.data(),
                                             static_cast<uint32_t>(history.size()), &c, out.data());
    if (st != ITTS_OK) rethrow(st, itts_gpt_last_error(h));
    return out;
}

itts_gpt* GptDecoder::create_from_tensors(const std::vector<Tensor>& tensors, const itts_gpt_config* config) {
    std::vector<itts_tensor> table;
    table.reserve(tensors.size());
    for (const auto& t : tensors) {
        itts_tensor e{};
        e.name = t.name.c_str();
        e.data = t.data->data();
        e.ndim = static_cast<int32_t>(t.shape.size());
        for (size_t i = 0; i < t.shape.size() && i < 4; ++i) e.shape[i] = t.shape[i];
        table.push_back(e);
    }
    itts_gpt* h = nullptr;
    const int st = itts_gpt_create(table.data(), static_cast<int32_t>(table.size()), config, &h);
    if (st != ITTS_OK) rethrow(st, itts_gpt_last_error(nullptr));
    return h;
}

itts_gpt* GptDecoder::create_from_bundle(const itts_bundle* bundle, const itts_gpt_config* config) {
    itts_gpt* h = nullptr;
    const int st = itts_gpt_create_from_bundle(bundle, config, &h);
    if (st != ITTS_OK) rethrow(st, itts_gpt_last_error(nullptr));
    return h;
}

itts_gpt* GptDecoder::create_from_path(const std::string& bundle_path, const itts_gpt_config* config) {
    // the caller's Weights has already checked the model bundle (weights.cpp:10-28)
    itts_bundle* b = nullptr;
    if (itts_bundle_open(bundle_path.c_str(), 0, &b) != ITTS_OK) throw std::runtime_error(itts_bundle_last_error());
    itts_gpt* h = nullptr;
    const int st = itts_gpt_create_from_bundle(b, config, &h);
    itts_bundle_close(b);  // the decoder holds device copies
    if (st != ITTS_OK) rethrow(st, itts_gpt_last_error(nullptr));
    return h;
}

GptDecoder::GptDecoder(const std::vector<Tensor>& tensors, const itts_gpt_config* config)
    : handle_(create_from_tensors(tensors, config)) {}

GptDecoder::GptDecoder(const itts_bundle* bundle, const itts_gpt_config* config) : handle_(create_from_bundle(bundle, config)) {}

GptDecoder::~GptDecoder() { itts_gpt_destroy(handle_); }

// ------------------------------------------------------------------ BundleWeights (weights.cpp:9-49)

BundleWeights::BundleWeights(const std::string& path, bool require_model) {
    if (itts_bundle_open(path.c_str(), require_model ? 1 : 0, &bundle_) != ITTS_OK) throw std::runtime_error(itts_bundle_last_error());
}

BundleWeights::~BundleWeights() { itts_bundle_close(bundle_); }

const TensorInfo& BundleWeights::info(const std::string& name) const {
    const auto found = infos_.find(name);
    if (found != infos_.end()) return found->second;
    itts_bundle_tensor t{};
    if (itts_bundle_find(bundle_, name.c_str(), &t) != ITTS_OK) throw std::runtime_error(itts_bundle_last_error());
    TensorInfo i;
    i.name = t.name;
    i.shape.assign(t.shape, t.shape + t.ndim);
    i.dtype = t.dtype == ITTS_DTYPE_F32 ? "f32" : "u32";
    i.offset = t.offset;
    i.nbytes = t.nbytes;
    return infos_.emplace(name, std::move(i)).first->second;
}

const std::vector<float>& BundleWeights::get(const std::string& name) {
    const auto found = cache_.find(name);
    if (found != cache_.end()) return found->second;
    itts_bundle_tensor t{};
    if (itts_bundle_find(bundle_, name.c_str(), &t) != ITTS_OK) throw std::runtime_error(itts_bundle_last_error());
    if (t.dtype != ITTS_DTYPE_F32) throw std::runtime_error("Expected float32: " + name);
    const float* p = static_cast<const float*>(t.data);
    return cache_.emplace(name, std::vector<float>(p, p + t.nbytes / sizeof(float))).first->second;
}

std::vector<uint32_t> BundleWeights::ids(const std::string& name) const {
    itts_bundle_tensor t{};
    if (itts_bundle_find(bundle_, name.c_str(), &t) != ITTS_OK) throw std::runtime_error(itts_bundle_last_error());
    if (t.dtype != ITTS_DTYPE_U32) throw std::runtime_error("Expected uint32: " + name);
    const uint32_t* p = static_cast<const uint32_t*>(t.data);
    return std::vector<uint32_t>(p, p + t.nbytes / sizeof(uint32_t));
}

void GptDecoder::check(int status) const {
    if (status != ITTS_OK) rethrow(status, itts_gpt_last_error(handle_));
}

std::vector<float> GptDecoder::prepare(const std::vector<float>& speaker, const std::vector<float>& emotion,
                                       const std::vector<uint32_t>& text, uint32_t language) {
    if (speaker.size() != 192 || emotion.size() != 1280) throw std::invalid_argument("Invalid GPT conditioning dimensions");
    const uint32_t cap = static_cast<uint32_t>(text.size()) + 6;
    std::vector<float> out(static_cast<size_t>(cap) * 1280);
    uint32_t rows = 0;
    check(itts_gpt_prepare(handle_, speaker.data(), emotion.data(), text.data(), static_cast<uint32_t>(text.size()), language,
                           out.data(), cap, &rows));
    out.resize(static_cast<size_t>(rows) * 1280);
    return out;
}

std::vector<float> GptDecoder::prefill(const std::vector<float>& prefix) {
    if (prefix.empty() || prefix.size() % 1280 || prefix.size() / 1280 > 1024)
        throw std::invalid_argument("Invalid GPT prefill dimensions");
    std::vector<float> logits(ITTS_MEL_VOCAB);
    check(itts_gpt_prefill(handle_, prefix.data(), static_cast<uint32_t>(prefix.size() / 1280), logits.data()));
    return logits;
}

std::vector<float> GptDecoder::step(uint32_t code, uint32_t position) {
    std::vector<float> logits(ITTS_MEL_VOCAB);
    check(itts_gpt_step(handle_, code, position, logits.data()));
    return logits;
}

GenerationResult GptDecoder::generate(const std::vector<float>& prefix, const GenerationOptions& options, uint32_t max_tokens) {
    if (prefix.empty() || prefix.size() % 1280) throw std::invalid_argument("Invalid GPT prefill dimensions");
    const itts_gen_options c = to_c(options);
    std::vector<uint32_t> codes(max_tokens ? max_tokens : 1);
    uint32_t n = 0;
    int32_t stopped = 0;
    check(itts_gpt_generate(handle_, prefix.data(), static_cast<uint32_t>(prefix.size() / 1280), &c, max_tokens, codes.data(), &n,
                            &stopped));
    codes.resize(n);
    return {std::move(codes), stopped != 0};
}

std::vector<GenerationResult> GptDecoder::generate_segments(const std::vector<float>& speaker, const std::vector<float>& emotion,
                                                            const std::vector<std::vector<uint32_t>>& segments, uint32_t language,
                                                            const GenerationOptions& options, uint32_t max_tokens) {
    if (speaker.size() != 192 || emotion.size() != 1280) throw std::invalid_argument("Invalid GPT conditioning dimensions");
    std::vector<uint32_t> ids, counts;
    for (const auto& seg : segments) {
        ids.insert(ids.end(), seg.begin(), seg.end());
        counts.push_back(static_cast<uint32_t>(seg.size()));
    }
    const itts_gen_options c = to_c(options);
    const size_t n = segments.size(), stride = max_tokens ? max_tokens : 1;
    std::vector<uint32_t> codes(std::max<size_t>(n, 1) * stride), lengths(std::max<size_t>(n, 1));
    std::vector<int32_t> stopped(std::max<size_t>(n, 1));
    check(itts_gpt_generate_segments(handle_, speaker.data(), emotion.data(), ids.data(), counts.data(), static_cast<uint32_t>(n),
                                     language, &c, max_tokens, codes.data(), lengths.data(), stopped.data()));
    std::vector<GenerationResult> out(n);
    for (size_t i = 0; i < n; ++i) {
        out[i].codes.assign(codes.begin() + i * stride, codes.begin() + i * stride + lengths[i]);
        out[i].stopped = stopped[i] != 0;
    }
    return out;
}

GptState GptDecoder::checkpoint() const {
    auto snap = std::make_shared<GptKvSnapshot>();
    check(itts_gpt_checkpoint(handle_, &snap->state));
    return {itts_gpt_state_tokens(snap->state), snap};
}

void GptDecoder::restore(const GptState& state) {
    if (!state.kv) throw std::invalid_argument("Invalid KV restore");
    check(itts_gpt_restore(handle_, state.kv->state));
}

uint32_t GptDecoder::cached_tokens() const { return itts_gpt_cached_tokens(handle_); }

}  // namespace itts25

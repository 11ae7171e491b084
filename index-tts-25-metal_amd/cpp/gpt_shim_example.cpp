// Example caller of the drop-in itts25::GptDecoder, written the way the reference's
// pipeline holds it (src/pipeline.cpp:12, 23-25): a Weights object with info()/get(),
// a device-context object, prepare -> generate.  `gpt_shim_example run` uses a synthetic
// weight table; `gpt_shim_example bundle <dir>` loads a MIT2 bundle through itts25::BundleWeights;
// both execute on the GPU.  Without arguments it only checks that the shim links.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <map>
#include <string>
#include <vector>

#include "itts25/codec.hpp"
#include "itts25/gpt.hpp"
#include "itts25/qwen.hpp"

namespace {
struct TensorInfo {
    std::vector<int64_t> shape;
};
struct TableWeights {  // the reference Weights interface (include/itts25/weights.hpp:9-10)
    std::map<std::string, TensorInfo> infos;
    std::map<std::string, std::vector<float>> data;
    const TensorInfo& info(const std::string& n) const { return infos.at(n); }
    const std::vector<float>& get(const std::string& n) { return data.at(n); }
    void add(const std::string& n, std::vector<int64_t> shape, float mean, float sd, uint64_t seed) {
        size_t count = 1;
        for (auto s : shape) count *= static_cast<size_t>(s);
        std::vector<float> v(count);
        itts_synthetic_normal(v.data(), count, seed, mean, sd);
        infos[n] = {shape};
        data[n] = std::move(v);
    }
};
struct DeviceContext {};
}  // namespace

// `gpt_shim_example bundle <dir>`: the reference pipeline's construction
// (src/pipeline.cpp:12; a Weights over the bundle, then GptDecoder gpt_(weights_, metal_)) on
// a MIT2 bundle, then the same prepare -> greedy generate as `run`, printing the codes.
// The shape of the reference's Weights as GptDecoder sees it: info/get plus bundle().root()
// naming the MIT2 bundle (include/itts25/weights.hpp, include/mit2/bundle.hpp).  Its get()
// is never called: the decoder re-opens bundle().root() and uploads from the mapping.
struct RefStyleWeights {
    struct Bundle {
        std::string path;
        const std::string& root() const { return path; }
    } b;
    itts25::BundleWeights inner;
    explicit RefStyleWeights(const char* p) : b{p}, inner(p) {}
    const Bundle& bundle() const { return b; }
    const itts25::TensorInfo& info(const std::string& n) const { return inner.info(n); }
    const std::vector<float>& get(const std::string&) { throw std::logic_error("get() should not be needed"); }
};

template <class W>
int run_bundle_with(W& w) {
    DeviceContext ctx;
    itts25::GptDecoder gpt(w, ctx);
    std::vector<float> speaker(192, 0.1f), emotion(1280, 0.05f);
    auto prefix = gpt.prepare(speaker, emotion, {5, 17, 300, 1, 0, 42}, 3);
    itts25::GenerationOptions opt;
    opt.do_sample = false;
    opt.repetition_penalty = 1;
    auto r = gpt.generate(prefix, opt, 8);
    std::printf("{\"rows\":%zu,\"codes\":[", prefix.size() / 1280);
    for (size_t i = 0; i < r.codes.size(); ++i) std::printf("%s%u", i ? "," : "", r.codes[i]);
    std::printf("],\"stopped\":%d,\"spk_shape\":[%lld,%lld]}\n", r.stopped ? 1 : 0,
                static_cast<long long>(w.info("gpt.spk_emb_proj.weight").shape[0]),
                static_cast<long long>(w.info("gpt.spk_emb_proj.weight").shape[1]));
    return 0;
}

// `gpt_shim_example qwen|qwenref|qwentable <dir> <prompt ids...>`: QwenDecoder the way
// src/main.cpp:160-166 drives it (prefill, three steps, generate), from BundleWeights, from a
// reference-style Weights (bundle().root()), or from a plain info()/get() table filled from
// the bundle.  Prints the prefill's argmax and logit sum, the steps' argmaxes, the generated
// ids, the failure of a generate that stops one id short of EOS, and the submissions.
template <class W>
int run_qwen_with(W& w, const std::vector<uint32_t>& prompt) {
    itts25::QwenDecoder qwen(w);
    const auto logits = qwen.prefill(prompt);
    auto argmax = [](const std::vector<float>& x) { return static_cast<long>(std::max_element(x.begin(), x.end()) - x.begin()); };
    double sum = 0;
    for (float v : logits) sum += v;
    std::printf("{\"prefill_argmax\":%ld,\"prefill_sum\":%.9g,\"steps\":[", argmax(logits), sum);
    for (uint32_t i = 1; i <= 3; ++i) std::printf("%s%ld", i > 1 ? "," : "", argmax(qwen.step(prompt[i % prompt.size()])));
    const auto ids = qwen.generate(prompt, 12);
    std::printf("],\"generated\":[");
    for (size_t i = 0; i < ids.size(); ++i) std::printf("%s%u", i ? "," : "", ids[i]);
    std::string short_error = "none";
    try {
        qwen.generate(prompt, static_cast<uint32_t>(ids.size() - 1));
    } catch (const std::runtime_error& e) {
        short_error = e.what();
    }
    std::printf("],\"short_error\":\"%s\",\"submissions\":%llu}\n", short_error.c_str(),
                static_cast<unsigned long long>(qwen.submissions()));
    return 0;
}

int run_qwen(const char* mode, const char* path, const std::vector<uint32_t>& prompt) {
    if (std::strcmp(mode, "qwenref") == 0) {
        RefStyleWeights w(path);
        return run_qwen_with(w, prompt);
    }
    itts25::BundleWeights b(path);
    if (std::strcmp(mode, "qwen") == 0) return run_qwen_with(b, prompt);
    TableWeights t;  // info()/get() only
    {
        std::vector<std::string> names{"qwen.model.embed_tokens.weight", "qwen.model.norm.weight"};
        for (unsigned l = 0; l < ITTS_QWEN_LAYERS; ++l) {
            const std::string p = "qwen.model.layers." + std::to_string(l);
            for (const char* s : {".self_attn.q_proj.weight", ".self_attn.k_proj.weight", ".self_attn.v_proj.weight",
                                  ".self_attn.o_proj.weight", ".self_attn.q_norm.weight", ".self_attn.k_norm.weight",
                                  ".mlp.gate_proj.weight", ".mlp.up_proj.weight", ".mlp.down_proj.weight",
                                  ".input_layernorm.weight", ".post_attention_layernorm.weight"})
                names.push_back(p + s);
        }
        for (const auto& n : names) {
            t.infos[n] = {b.info(n).shape};
            t.data[n] = b.get(n);
        }
    }
    return run_qwen_with(t, prompt);
}

int run_bundle(const char* path, bool ref_style) {
    if (ref_style) {
        RefStyleWeights w(path);
        return run_bundle_with(w);
    }
    itts25::BundleWeights w(path);
    return run_bundle_with(w);
}

// `gpt_shim_example gpt_test <model bundle> <fixture bundle>`: the reference's gpt_test
// (src/main.cpp:31-66) as a caller of this drop-in: the model and its single-file fixture
// through BundleWeights (Weights(model), fixture(golden, false)), then prepare for five
// languages, prefill, four steps, greedy and 3-beam generation, each compared with the
// fixture the way main.cpp's compare (19-30) and check_logits (40-47) do.  One JSON line
// per case, as gpt_test prints them; exit status 0 when every case passes.
bool compare(const std::string& name, const std::vector<float>& actual, const std::vector<float>& expected,
             float tolerance = 1e-4f, double rms_tolerance = 1e-5) {
    if (actual.size() != expected.size()) throw std::runtime_error("Output shape mismatch: " + name);
    double sum = 0, square = 0;
    float peak = 0;
    for (size_t i = 0; i < actual.size(); i++) {
        if (!std::isfinite(actual[i]) || !std::isfinite(expected[i])) throw std::runtime_error("Non-finite output: " + name);
        const auto d = std::abs(actual[i] - expected[i]);
        peak = std::max(peak, d);
        sum += d;
        square += d * d;
    }
    const double mean = sum / actual.size(), rmse = std::sqrt(square / actual.size());
    const bool pass = peak < tolerance && rmse < rms_tolerance;
    std::printf("{\"case\":\"%s\",\"max_abs_error\":%g,\"mean_abs_error\":%g,\"rmse\":%g,\"pass\":%s}\n", name.c_str(), peak, mean,
                rmse, pass ? "true" : "false");
    return pass;
}

int run_gpt_test(const char* model, const char* golden) {
    itts25::BundleWeights weights(model), fixture(golden, false);
    DeviceContext metal;
    itts25::GptDecoder gpt(weights, metal);
    bool pass = true;
    std::vector<float> chinese;
    for (const auto* lang : {"ZH", "EN", "JA", "ES", "AR"}) {
        const auto name = std::string("prefix.") + lang;
        auto prefix = gpt.prepare(fixture.get("speaker"), fixture.get("emotion"), fixture.ids(name + ".tokens"),
                                  fixture.ids(name + ".language")[0]);
        pass = compare(name, prefix, fixture.get(name + ".embeddings")) && pass;
        if (std::string(lang) == "ZH") chinese = std::move(prefix);
    }
    auto check_logits = [&](const std::string& name, const std::vector<float>& logits) {
        const auto& ref = fixture.get(name + ".logits");
        auto argmax = [](const std::vector<float>& x) { return std::max_element(x.begin(), x.end()) - x.begin(); };
        const bool match = argmax(logits) == argmax(ref);
        std::printf("{\"case\":\"%s.argmax\",\"exact_match\":%s}\n", name.c_str(), match ? "true" : "false");
        return compare(name, logits, ref, 1e-4f, 2e-5) && match;
    };
    pass = check_logits("decode.prefill", gpt.prefill(chinese)) && pass;
    for (uint32_t i = 1; i <= 4; i++) {
        auto name = "decode." + std::to_string(i);
        pass = check_logits(name, gpt.step(fixture.ids(name + ".code")[0], i)) && pass;
    }
    itts25::GenerationOptions config;
    config.do_sample = false;
    config.repetition_penalty = 1;
    auto generated = gpt.generate(chinese, config, 8);
    auto expected_codes = fixture.ids("generation.greedy.codes");
    if (!expected_codes.empty() && expected_codes.back() == 8193) expected_codes.pop_back();
    const bool generated_match = generated.codes == expected_codes;
    pass = generated_match && pass;
    std::printf("{\"case\":\"generation.greedy\",\"exact_match\":%s}\n", generated_match ? "true" : "false");
    config.num_beams = 3;
    auto beam = gpt.generate(chinese, config, 8);
    auto expected_beam = fixture.ids("generation.beam.codes");
    if (!expected_beam.empty() && expected_beam.back() == 8193) expected_beam.pop_back();
    const bool beam_match = beam.codes == expected_beam;
    pass = beam_match && pass;
    std::printf("{\"case\":\"generation.beam\",\"exact_match\":%s}\n", beam_match ? "true" : "false");
    std::printf("{\"stage\":\"gpt_2.5\",\"cached_tokens\":%u,\"pass\":%s}\n", gpt.cached_tokens(), pass ? "true" : "false");
    return pass ? 0 : 1;
}

int main(int argc, char** argv) {
    if (argc >= 4 && std::strcmp(argv[1], "gpt_test") == 0) return run_gpt_test(argv[2], argv[3]);
    if (argc >= 3 && std::strcmp(argv[1], "bundle") == 0) return run_bundle(argv[2], false);
    if (argc >= 3 && std::strcmp(argv[1], "refbundle") == 0) return run_bundle(argv[2], true);
    if (argc >= 4 && std::strncmp(argv[1], "qwen", 4) == 0) {
        std::vector<uint32_t> prompt;
        for (int i = 3; i < argc; ++i) prompt.push_back(static_cast<uint32_t>(std::strtoul(argv[i], nullptr, 10)));
        return run_qwen(argv[1], argv[2], prompt);
    }
    if (argc < 2 || std::strcmp(argv[1], "run") != 0) {
        std::printf("gpt shim linked\n");
        return 0;
    }
    TableWeights w;
    uint64_t seed = 1;
    w.add("gpt.spk_emb_proj.weight", {1280, 192}, 0, 0.02f, seed++);
    w.add("gpt.spk_emb_proj.bias", {1280}, 0, 0.02f, seed++);
    w.add("gpt.text_embedding.weight", {12000, 1280}, 0, 0.02f, seed++);
    w.add("gpt.text_pos_embedding.emb.weight", {602, 1280}, 0, 0.02f, seed++);
    w.add("gpt.lang_embedding.weight", {107, 1280}, 0, 0.02f, seed++);
    w.add("gpt.mel_embedding.weight", {8194, 1280}, 0, 0.02f, seed++);
    w.add("gpt.mel_pos_embedding.emb.weight", {1815, 1280}, 0, 0.02f, seed++);
    for (const char* n : {"gpt.gpt.ln_f", "gpt.final_norm"}) {
        w.add(std::string(n) + ".weight", {1280}, 1, 0, seed++);
        w.add(std::string(n) + ".bias", {1280}, 0, 0, seed++);
    }
    w.add("gpt.mel_head.weight", {8194, 1280}, 0, 0.02f, seed++);
    w.add("gpt.mel_head.bias", {8194}, 0, 0.02f, seed++);
    for (int i = 0; i < 24; ++i) {
        const std::string p = "gpt.gpt.h." + std::to_string(i);
        w.add(p + ".ln_1.weight", {1280}, 1, 0, seed++);
        w.add(p + ".ln_1.bias", {1280}, 0, 0, seed++);
        w.add(p + ".attn.c_attn.weight", {1280, 3840}, 0, 0.02f, seed++);
        w.add(p + ".attn.c_attn.bias", {3840}, 0, 0.02f, seed++);
        w.add(p + ".attn.c_proj.weight", {1280, 1280}, 0, 0.02f, seed++);
        w.add(p + ".attn.c_proj.bias", {1280}, 0, 0.02f, seed++);
        w.add(p + ".ln_2.weight", {1280}, 1, 0, seed++);
        w.add(p + ".ln_2.bias", {1280}, 0, 0, seed++);
        w.add(p + ".mlp.c_fc.weight", {1280, 5120}, 0, 0.02f, seed++);
        w.add(p + ".mlp.c_fc.bias", {5120}, 0, 0.02f, seed++);
        w.add(p + ".mlp.c_proj.weight", {5120, 1280}, 0, 0.02f, seed++);
        w.add(p + ".mlp.c_proj.bias", {1280}, 0, 0.02f, seed++);
    }
    DeviceContext ctx;
    itts25::GptDecoder gpt(w, ctx);
    std::vector<float> speaker(192, 0.1f), emotion(1280, 0.05f);
    auto prefix = gpt.prepare(speaker, emotion, {5, 17, 300, 1, 0, 42}, 3);
    itts25::GenerationOptions opt;
    opt.do_sample = false;
    opt.repetition_penalty = 1;
    auto r = gpt.generate(prefix, opt, 8);
    std::printf("{\"rows\":%zu,\"codes\":%zu,\"stopped\":%d,\"cached\":%u}\n", prefix.size() / 1280, r.codes.size(),
                r.stopped ? 1 : 0, gpt.cached_tokens());
    try {
        gpt.step(9000, 2);
        return 1;
    } catch (const std::invalid_argument&) {
    }
    opt.num_beams = 3;  // beam search through the reference-form decoder (10 beam slots)
    auto rb = gpt.generate(prefix, opt, 6);
    std::printf("{\"beam_codes\":%zu,\"beam_stopped\":%d}\n", rb.codes.size(), rb.stopped ? 1 : 0);
    auto scores = itts25::apply_gpt_sampling_processors(std::vector<float>(8194, 0.5f), {1, 8192}, itts25::GenerationOptions{});
    std::printf("{\"processed\":%zu}\n", scores.size());
    // NativeRuntime's segment loop (native_runtime.cpp:98-99) in one call, against the loop itself
    const std::vector<std::vector<uint32_t>> segments{{5, 17, 300}, {42, 43, 44, 45, 46}, {7}};
    itts25::GenerationOptions so;
    so.seed = 11;
    so.top_k = 0;
    auto batched = gpt.generate_segments(speaker, emotion, segments, 3, so, 10);
    bool same = batched.size() == segments.size();
    for (size_t i = 0; same && i < segments.size(); ++i) {
        auto o = so;
        o.seed += i;
        auto single = gpt.generate(gpt.prepare(speaker, emotion, segments[i], 3), o, 10);
        same = single.codes == batched[i].codes && single.stopped == batched[i].stopped;
    }
    std::printf("{\"segments\":%zu,\"segments_equal_loop\":%d}\n", batched.size(), same ? 1 : 0);
    // The codes' consumer through the reference's construction (native_runtime.cpp:30, 100):
    // EnhancedCodec codec_(weights_, metal_); codec_.decode(generated.codes).
    const std::string q = "codec.quantizer.quantizers.0", d = "codec.decoder.0";
    w.add(q + ".codebook.weight", {8192, 8}, 0, 1, seed++);
    w.add(q + ".out_project.weight", {1024, 8}, 0, 0.02f, seed++);
    w.add(q + ".out_project.bias", {1024}, 0, 0.02f, seed++);
    w.add(d + ".embed.weight", {384, 1024, 7}, 0, 0.02f, seed++);
    w.add(d + ".embed.bias", {384}, 0, 0.02f, seed++);
    w.add(d + ".norm.weight", {384}, 1, 0.1f, seed++);
    w.add(d + ".norm.bias", {384}, 0, 0.1f, seed++);
    for (int i = 0; i < 12; ++i) {
        const std::string l = d + ".convnext." + std::to_string(i);
        w.add(l + ".dwconv.weight", {384, 1, 7}, 0, 0.02f, seed++);
        w.add(l + ".dwconv.bias", {384}, 0, 0.02f, seed++);
        w.add(l + ".norm.weight", {384}, 1, 0.1f, seed++);
        w.add(l + ".norm.bias", {384}, 0, 0.1f, seed++);
        w.add(l + ".pwconv1.weight", {2048, 384}, 0, 0.02f, seed++);
        w.add(l + ".pwconv1.bias", {2048}, 0, 0.02f, seed++);
        w.add(l + ".pwconv2.weight", {384, 2048}, 0, 0.02f, seed++);
        w.add(l + ".pwconv2.bias", {384}, 0, 0.02f, seed++);
        w.add(l + ".gamma", {384}, 0.5f, 0.1f, seed++);
    }
    w.add(d + ".final_layer_norm.weight", {384}, 1, 0.1f, seed++);
    w.add(d + ".final_layer_norm.bias", {384}, 0, 0.1f, seed++);
    w.add("codec.decoder.1.weight", {1024, 384}, 0, 0.02f, seed++);
    w.add("codec.decoder.1.bias", {1024}, 0, 0.02f, seed++);
    w.add("codec.up.weight", {1024, 1024, 3}, 0, 0.02f, seed++);
    w.add("codec.up.bias", {1024}, 0, 0.02f, seed++);
    itts25::EnhancedCodec codec(w, ctx);
    const std::vector<uint32_t> codes = batched[0].codes.empty() ? std::vector<uint32_t>{1, 2, 3} : batched[0].codes;
    const auto features = codec.decode(codes);
    bool finite = true;
    for (float v : features) finite = finite && std::isfinite(v);
    bool refused = false;
    try {
        codec.decode({8192});
    } catch (const std::invalid_argument&) {
        refused = true;
    }
    std::printf("{\"codec_values\":%zu,\"codec_codes\":%zu,\"codec_finite\":%d,\"codec_refuses_8192\":%d}\n", features.size(),
                codes.size(), finite ? 1 : 0, refused ? 1 : 0);
    return 0;
}

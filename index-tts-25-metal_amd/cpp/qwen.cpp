// itts25::QwenDecoder over the HIP C ABI (include/itts_qwen.h): the reference's src/qwen.cpp
// (lines 5-49) with the math in libitts_gpt.so on the MI355X.
#include "itts25/qwen.hpp"

#include <stdexcept>

namespace itts25 {

namespace {
[[noreturn]] void qwen_rethrow(int status, const char* message) {
    const std::string m = message ? message : "";
    if (status == ITTS_EINVAL) throw std::invalid_argument(m);
    if (status == ITTS_ERUNTIME) throw std::runtime_error(m);
    throw std::logic_error(m);
}
}  // namespace

// The tensors of qwen.cpp:7-13 in its check order, then the norm weights run() reads.
std::vector<std::string> QwenDecoder::tensor_names() {
    std::vector<std::string> n{"qwen.model.embed_tokens.weight"};
    for (unsigned i = 0; i < ITTS_QWEN_LAYERS; ++i) {
        const std::string p = "qwen.model.layers." + std::to_string(i);
        for (const char* s : {".self_attn.q_proj.weight", ".self_attn.k_proj.weight", ".self_attn.v_proj.weight",
                              ".self_attn.o_proj.weight", ".self_attn.q_norm.weight", ".self_attn.k_norm.weight",
                              ".mlp.gate_proj.weight", ".mlp.up_proj.weight", ".mlp.down_proj.weight"})
            n.push_back(p + s);
    }
    for (unsigned i = 0; i < ITTS_QWEN_LAYERS; ++i) {
        const std::string p = "qwen.model.layers." + std::to_string(i);
        n.push_back(p + ".input_layernorm.weight");
        n.push_back(p + ".post_attention_layernorm.weight");
    }
    n.push_back("qwen.model.norm.weight");
    return n;
}

itts_qwen* QwenDecoder::create_from_tensors(const std::vector<Tensor>& tensors) {
    std::vector<itts_tensor> table;
    for (const auto& t : tensors) {
        itts_tensor e{};
        e.name = t.name.c_str();
        e.data = t.data->data();
        e.ndim = static_cast<int32_t>(t.shape.size());
        for (size_t i = 0; i < t.shape.size() && i < 4; ++i) e.shape[i] = t.shape[i];
        table.push_back(e);
    }
    itts_qwen* q = nullptr;
    const int st = itts_qwen_create(table.data(), static_cast<int32_t>(table.size()), nullptr, &q);
    if (st != ITTS_OK) qwen_rethrow(st, itts_qwen_last_error(nullptr));
    return q;
}

itts_qwen* QwenDecoder::create_from_bundle(const itts_bundle* bundle) {
    itts_qwen* q = nullptr;
    const int st = itts_qwen_create_from_bundle(bundle, nullptr, &q);
    if (st != ITTS_OK) qwen_rethrow(st, itts_qwen_last_error(nullptr));
    return q;
}

itts_qwen* QwenDecoder::create_from_path(const std::string& bundle_path) {
    itts_bundle* b = nullptr;
    if (itts_bundle_open(bundle_path.c_str(), 0, &b) != ITTS_OK) throw std::runtime_error(itts_bundle_last_error());
    itts_qwen* q = nullptr;
    const int st = itts_qwen_create_from_bundle(b, nullptr, &q);
    itts_bundle_close(b);  // the decoder holds device copies
    if (st != ITTS_OK) qwen_rethrow(st, itts_qwen_last_error(nullptr));
    return q;
}

QwenDecoder::~QwenDecoder() { itts_qwen_destroy(handle_); }

std::vector<float> QwenDecoder::prefill(const std::vector<uint32_t>& ids) {
    std::vector<float> out(ITTS_QWEN_VOCAB);
    const int st = itts_qwen_prefill(handle_, ids.data(), static_cast<uint32_t>(ids.size()), out.data());
    if (st != ITTS_OK) qwen_rethrow(st, itts_qwen_last_error(handle_));
    return out;
}

std::vector<float> QwenDecoder::step(uint32_t id) {
    std::vector<float> out(ITTS_QWEN_VOCAB);
    const int st = itts_qwen_step(handle_, id, out.data());
    if (st != ITTS_OK) qwen_rethrow(st, itts_qwen_last_error(handle_));
    return out;
}

std::vector<uint32_t> QwenDecoder::generate(const std::vector<uint32_t>& ids, uint32_t maximum) {
    std::vector<uint32_t> out(maximum ? maximum : 1);
    uint32_t count = 0;
    const int st = itts_qwen_generate(handle_, ids.data(), static_cast<uint32_t>(ids.size()), maximum, out.data(), &count);
    if (st != ITTS_OK) qwen_rethrow(st, itts_qwen_last_error(handle_));
    out.resize(count);
    return out;
}

}  // namespace itts25

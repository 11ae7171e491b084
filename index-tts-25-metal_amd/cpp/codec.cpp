// itts25::EnhancedCodec (decode path) over the HIP C ABI (include/itts_gpt.h): the reference's
// src/codec.cpp:5-20 and 57-72 with the math in libitts_gpt.so on the MI355X.
#include "itts25/codec.hpp"

#include <stdexcept>

namespace itts25 {

namespace {
[[noreturn]] void codec_rethrow(int status, const char* message) {
    const std::string m = message ? message : "";
    if (status == ITTS_EINVAL) throw std::invalid_argument(m);
    if (status == ITTS_ERUNTIME) throw std::runtime_error(m);
    throw std::logic_error(m);
}
}  // namespace

std::vector<std::string> EnhancedCodec::tensor_names() {
    const std::string q = "codec.quantizer.quantizers.0", d = "codec.decoder.0";
    std::vector<std::string> n{q + ".codebook.weight", q + ".out_project.weight", q + ".out_project.bias", d + ".embed.weight",
                               d + ".embed.bias",      d + ".norm.weight",        d + ".norm.bias"};
    for (int i = 0; i < 12; ++i) {
        const std::string l = d + ".convnext." + std::to_string(i);
        for (const char* s : {".dwconv.weight", ".dwconv.bias", ".norm.weight", ".norm.bias", ".pwconv1.weight", ".pwconv1.bias",
                              ".pwconv2.weight", ".pwconv2.bias", ".gamma"})
            n.push_back(l + s);
    }
    for (const char* s : {"codec.decoder.0.final_layer_norm.weight", "codec.decoder.0.final_layer_norm.bias", "codec.decoder.1.weight",
                          "codec.decoder.1.bias", "codec.up.weight", "codec.up.bias"})
        n.push_back(s);
    return n;
}

itts_codec* EnhancedCodec::create_from_tensors(const std::vector<Tensor>& tensors) {
    std::vector<itts_tensor> table;
    for (const auto& t : tensors) {
        itts_tensor e{};
        e.name = t.name.c_str();
        e.data = t.data->data();
        e.ndim = static_cast<int32_t>(t.shape.size());
        for (size_t i = 0; i < t.shape.size() && i < 4; ++i) e.shape[i] = t.shape[i];
        table.push_back(e);
    }
    itts_codec* c = nullptr;
    const int st = itts_codec_create(table.data(), static_cast<int32_t>(table.size()), &c);
    if (st != ITTS_OK) codec_rethrow(st, itts_codec_last_error(nullptr));
    return c;
}

itts_codec* EnhancedCodec::create_from_bundle(const itts_bundle* bundle) {
    itts_codec* c = nullptr;
    const int st = itts_codec_create_from_bundle(bundle, &c);
    if (st != ITTS_OK) codec_rethrow(st, itts_codec_last_error(nullptr));
    return c;
}

itts_codec* EnhancedCodec::create_from_path(const std::string& bundle_path) {
    itts_bundle* b = nullptr;
    if (itts_bundle_open(bundle_path.c_str(), 0, &b) != ITTS_OK) throw std::runtime_error(itts_bundle_last_error());
    itts_codec* c = nullptr;
    const int st = itts_codec_create_from_bundle(b, &c);
    itts_bundle_close(b);  // the codec holds device copies
    if (st != ITTS_OK) codec_rethrow(st, itts_codec_last_error(nullptr));
    return c;
}

EnhancedCodec::~EnhancedCodec() { itts_codec_destroy(handle_); }

std::vector<float> EnhancedCodec::decode(const std::vector<uint32_t>& codes) {
    std::vector<float> out(codes.size() * 2 * 1024);
    const int st = itts_codec_decode(handle_, codes.data(), static_cast<uint32_t>(codes.size()), out.empty() ? nullptr : out.data());
    if (st != ITTS_OK) codec_rethrow(st, itts_codec_last_error(handle_));
    return out;
}

EncodedSemantic EnhancedCodec::encode(const std::vector<float>&, uint32_t) {
    throw std::logic_error("EnhancedCodec::encode is not provided by this library (decode path only)");
}

}  // namespace itts25

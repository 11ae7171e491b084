// Drop-in for the decode path of the reference's include/itts25/codec.hpp (lines 7-28):
// itts25::EnhancedCodec with the reference's constructor form, so `codec_(weights_, metal_)`
// (src/native_runtime.cpp:30) compiles unchanged, and decode() (codec.cpp:64-72) running on
// the MI355X over the C ABI (include/itts_gpt.h, itts_codec_*).  encode() is declared for
// source compatibility and throws std::logic_error: this library provides the decode path.
#pragma once
#include <cstdint>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "itts_gpt.h"
#include "itts25/bundle_weights.hpp"

namespace itts25 {

struct EncodedSemantic {
    std::vector<uint32_t> codes;
    std::vector<float> projected;  // time-major [codes.size(), 1024]
};

class EnhancedCodec {
public:
    // Weights types as GptDecoder's constructor takes them: the reference's Weights (its
    // bundle().root() names the MIT2 bundle, re-opened here), BundleWeights, or any type with
    // info()/get() (the codec.* tensors are taken through get()).
    template <class AnyWeights, class Context>
    EnhancedCodec(AnyWeights& weights, Context& /*device context, unused*/) : handle_(create(weights)) {}
    ~EnhancedCodec();
    EnhancedCodec(const EnhancedCodec&) = delete;
    EnhancedCodec& operator=(const EnhancedCodec&) = delete;

    std::vector<float> decode(const std::vector<uint32_t>& codes);  // [2*T,1024]
    EncodedSemantic encode(const std::vector<float>& features, uint32_t tokens);
    uint64_t extra_gpu_submissions() const { return 0; }

private:
    itts_codec* handle_ = nullptr;

    template <class W, class = void>
    struct has_handle : std::false_type {};
    template <class W>
    struct has_handle<W, std::void_t<decltype(std::declval<const W&>().handle())>> : std::true_type {};
    template <class W, class = void>
    struct has_bundle_root : std::false_type {};
    template <class W>
    struct has_bundle_root<W, std::void_t<decltype(std::string(std::declval<W&>().bundle().root()))>> : std::true_type {};

    struct Tensor {
        std::string name;
        std::vector<int64_t> shape;
        const std::vector<float>* data;
    };
    static itts_codec* create_from_bundle(const itts_bundle* bundle);
    static itts_codec* create_from_path(const std::string& bundle_path);
    static itts_codec* create_from_tensors(const std::vector<Tensor>& tensors);
    static std::vector<std::string> tensor_names();
    template <class W>
    static itts_codec* create(W& w) {
        if constexpr (has_handle<W>::value) return create_from_bundle(w.handle());
        else if constexpr (has_bundle_root<W>::value) return create_from_path(std::string(w.bundle().root()));
        else {
            std::vector<Tensor> t;
            for (const auto& n : tensor_names()) t.push_back({n, w.info(n).shape, &w.get(n)});
            return create_from_tensors(t);
        }
    }
};

}  // namespace itts25

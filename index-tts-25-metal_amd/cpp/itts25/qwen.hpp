// Drop-in replacement of the reference's include/itts25/qwen.hpp (lines 5-18):
// itts25::QwenDecoder with the same members, arguments and exception kinds, running on the
// MI355X over the C ABI (include/itts_qwen.h).  The constructor takes any Weights type the
// way the reference's `QwenDecoder qwen(weights)` (src/main.cpp:160) and
// `std::make_unique<QwenDecoder>(weights_)` (src/native_runtime.cpp:50) pass it: the
// reference's Weights (its bundle().root() names the MIT2 bundle, re-opened here),
// BundleWeights, or any type with info(name).shape / get(name).
#pragma once
#include <cstdint>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "itts_qwen.h"
#include "itts25/bundle_weights.hpp"

namespace itts25 {

class QwenDecoder {
public:
    template <class AnyWeights>
    explicit QwenDecoder(AnyWeights& weights) : handle_(create(weights)) {}
    ~QwenDecoder();
    QwenDecoder(const QwenDecoder&) = delete;
    QwenDecoder& operator=(const QwenDecoder&) = delete;

    std::vector<float> prefill(const std::vector<uint32_t>& ids);
    std::vector<float> step(uint32_t id);
    std::vector<uint32_t> generate(const std::vector<uint32_t>& ids, uint32_t maximum = 1024);
    uint64_t submissions() const { return itts_qwen_submissions(handle_); }

private:
    itts_qwen* handle_ = nullptr;

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
    static itts_qwen* create_from_bundle(const itts_bundle* bundle);
    static itts_qwen* create_from_path(const std::string& bundle_path);
    static itts_qwen* create_from_tensors(const std::vector<Tensor>& tensors);
    static std::vector<std::string> tensor_names();
    template <class W>
    static itts_qwen* create(W& w) {
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

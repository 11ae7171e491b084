// A MIT2-bundle Weights for callers without the reference's Metal runtime: the interface of
// the reference's itts25::Weights (include/itts25/weights.hpp, src/weights.cpp:9-49) --
// constructor, get, info, ids, same checks and exception messages -- implemented over the
// C ABI's bundle reader (include/itts_gpt.h, itts_bundle_*).  It has its own name so it
// never shadows the reference's Weights, which the rest of the reference pipeline keeps
// using.  A GptDecoder built from it takes the tensors straight from the bundle's mapping.
#pragma once
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "itts_gpt.h"

namespace itts25 {

// The fields of mit2::TensorInfo (include/mit2/bundle.hpp) a caller of Weights reads.
struct TensorInfo {
    std::string name;
    std::vector<int64_t> shape;
    std::string dtype;  // "f32" or "u32"
    uint64_t offset = 0;
    uint64_t nbytes = 0;
};

class BundleWeights {
public:
    // Opens a bundle directory or single-file bundle; require_model: the manifest must
    // name target "index-tts2.5" (weights.cpp:10-14).  std::runtime_error on failure.
    explicit BundleWeights(const std::string& path, bool require_model = true);
    ~BundleWeights();
    BundleWeights(const BundleWeights&) = delete;
    BundleWeights& operator=(const BundleWeights&) = delete;

    const std::vector<float>& get(const std::string& name);     // f32 tensor, cached host copy
    const TensorInfo& info(const std::string& name) const;      // "Missing tensor: <name>"
    std::vector<uint32_t> ids(const std::string& name) const;   // u32 tensor
    const itts_bundle* handle() const { return bundle_; }

private:
    itts_bundle* bundle_ = nullptr;
    std::unordered_map<std::string, std::vector<float>> cache_;
    mutable std::unordered_map<std::string, TensorInfo> infos_;
};

}  // namespace itts25

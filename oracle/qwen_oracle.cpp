// CPU oracle for the Qwen3-0.6B emotion-text decoder.
//
// TEST INFRASTRUCTURE ONLY: tests/ load this library to compare the HIP path against.
// The product never links it.
//
// Follows, op for op:
//   src/qwen.cpp:5-15    constructor shape checks
//   src/qwen.cpp:20-22   prefill (capacity, fresh cache, run(ids, 0)) / step (cache check)
//   src/qwen.cpp:23-45   run: embedding rows; per layer RMSNorm -> q/k/v projections ->
//                        per-head q_norm / k_norm -> RoPE -> causal GQA attention ->
//                        o_proj + residual -> RMSNorm -> SiLU(gate) * up -> down + residual;
//                        final RMSNorm of the last row; logits through the tied embedding
//   src/qwen.cpp:46-49   greedy generate until EOS 151643
// Per-op math follows vendor/metal-runtime/metal/kernels.metal:
//   995-1030   RMSNorm: x * rsqrt(sum(x^2) / width + eps) * gamma, eps 1e-6
//   3111-3115  RoPE: angle = (offset + t) * 1e6^(-(d % 64) / 64), rotate-half
//   3116-3118  K/V rows stored at cache rows offset .. offset + t - 1
//   3119-3129  attention: score = q.k * 0.08838834764831844 over keys 0 .. offset + query,
//              kv head = head / 2, max-subtracted exp, value = sum((p / sum) * v)
//   363-374    SiLU-mul: (v / (1 + exp(-v))) * u
//   1269-1305  argmax: the first index of the maximum (NaN never wins)
// The linears add the zero bias the reference passes (qwen.cpp:17-19).  Sums inside a dot
// product are sequential here; the GPU uses its own order, so parity is tolerance based.
#include "qwen_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

std::string& orc_error_message();

namespace {

constexpr uint32_t kV = ORC_QWEN_VOCAB;
constexpr uint32_t kD = 1024;       // hidden width
constexpr uint32_t kQ = 2048;       // 16 query heads x 128
constexpr uint32_t kKV = 1024;      // 8 kv heads x 128
constexpr uint32_t kF = 3072;       // MLP width
constexpr uint32_t kHd = 128;
constexpr uint32_t kCap = 4096;     // gptKvCacheCreate(28, 4096, 1024)
constexpr uint32_t kPrompt = 3072;
constexpr uint32_t kMaxGen = 1024;
constexpr float kEps = 1e-6f;

struct QLayer {
    std::vector<float> q, k, v, o, gate, up, down, in_ln, post_ln, q_norm, k_norm;
};

// y[o] = W[o] . x + 0 for `rows` outputs of width `cols`, for each of t input rows.
void linear(const float* W, uint32_t rows, uint32_t cols, const float* X, uint32_t t, float* Y) {
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < static_cast<int64_t>(rows); ++o) {
        const float* w = W + static_cast<size_t>(o) * cols;
        for (uint32_t r = 0; r < t; ++r) {
            const float* x = X + static_cast<size_t>(r) * cols;
            float acc = 0.0f;
            for (uint32_t c = 0; c < cols; ++c) acc += w[c] * x[c];
            Y[static_cast<size_t>(r) * rows + o] = acc + 0.0f;
        }
    }
}

void rmsnorm_rows(const float* X, uint32_t rows, uint32_t width, const float* g, float* Y) {
    for (uint32_t r = 0; r < rows; ++r) {
        const float* x = X + static_cast<size_t>(r) * width;
        float ss = 0.0f;
        for (uint32_t i = 0; i < width; ++i) ss += x[i] * x[i];
        const float inv = 1.0f / std::sqrt(ss / static_cast<float>(width) + kEps);
        float* y = Y + static_cast<size_t>(r) * width;
        for (uint32_t i = 0; i < width; ++i) y[i] = x[i] * inv * g[i];
    }
}

}  // namespace

struct orc_qwen {
    uint32_t layers = 0;
    std::vector<float> embed, norm;
    std::vector<QLayer> L;
    std::vector<float> kc, vc;  // [layer][row][1024]
    std::vector<float> inv_freq;
    uint32_t cached = 0, selected = 0;
    int32_t mutation = 0;

    void rope(float* X, uint32_t t, uint32_t heads, uint32_t offset) const {
        std::vector<float> row(kHd);
        for (uint32_t r = 0; r < t; ++r) {
            const float pos = static_cast<float>((mutation == 4 ? 0u : offset) + r);
            for (uint32_t h = 0; h < heads; ++h) {
                float* x = X + (static_cast<size_t>(r) * heads + h) * kHd;
                std::copy(x, x + kHd, row.begin());
                for (uint32_t d = 0; d < kHd; ++d) {
                    const float angle = pos * inv_freq[d % 64];
                    float rotated = d < 64 ? -row[d + 64] : row[d - 64];
                    if (mutation == 2) rotated = -rotated;
                    x[d] = row[d] * std::cos(angle) + rotated * std::sin(angle);
                }
            }
        }
    }

    // qwen.cpp:23-45 for the t tokens `ids` at cache rows offset..; returns the logits of
    // the last one (and sets `selected` to their argmax).
    std::vector<float> run(const std::vector<uint32_t>& ids, uint32_t offset) {
        for (uint32_t id : ids)
            if (id >= kV) throw std::invalid_argument("Invalid Qwen token");
        const uint32_t t = static_cast<uint32_t>(ids.size());
        if (offset + t > kCap) throw std::invalid_argument("Invalid Qwen attention cache");
        std::vector<float> H(static_cast<size_t>(t) * kD), Xn(H.size()), Q(static_cast<size_t>(t) * kQ),
            K(static_cast<size_t>(t) * kKV), Vv(K.size()), A(Q.size()), P(H.size()), G(static_cast<size_t>(t) * kF),
            U(G.size());
        for (uint32_t r = 0; r < t; ++r)
            std::copy(embed.begin() + static_cast<size_t>(ids[r]) * kD, embed.begin() + static_cast<size_t>(ids[r] + 1) * kD,
                      H.begin() + static_cast<size_t>(r) * kD);
        for (uint32_t l = 0; l < layers; ++l) {
            const QLayer& w = L[l];
            rmsnorm_rows(H.data(), t, kD, w.in_ln.data(), Xn.data());
            linear(w.q.data(), kQ, kD, Xn.data(), t, Q.data());
            linear(w.k.data(), kKV, kD, Xn.data(), t, K.data());
            linear(w.v.data(), kKV, kD, Xn.data(), t, Vv.data());
            if (mutation != 3) {
                rmsnorm_rows(Q.data(), t * 16, kHd, w.q_norm.data(), Q.data());
                rmsnorm_rows(K.data(), t * 8, kHd, w.k_norm.data(), K.data());
            }
            rope(Q.data(), t, 16, offset);
            rope(K.data(), t, 8, offset);
            float* kl = kc.data() + static_cast<size_t>(l) * kCap * kKV;
            float* vl = vc.data() + static_cast<size_t>(l) * kCap * kKV;
            std::copy(K.begin(), K.end(), kl + static_cast<size_t>(offset) * kKV);
            std::copy(Vv.begin(), Vv.end(), vl + static_cast<size_t>(offset) * kKV);
#pragma omp parallel for collapse(2) schedule(static)
            for (int64_t qi = 0; qi < static_cast<int64_t>(t); ++qi)
                for (int64_t h = 0; h < 16; ++h) {
                    const uint32_t count = offset + static_cast<uint32_t>(qi) + 1;
                    const uint32_t kvh = mutation == 1 ? static_cast<uint32_t>(h) % 8 : static_cast<uint32_t>(h) / 2;
                    const float* q = Q.data() + static_cast<size_t>(qi) * kQ + h * kHd;
                    std::vector<float> s(count);
                    float peak = -INFINITY;
                    for (uint32_t key = 0; key < count; ++key) {
                        const float* k = kl + static_cast<size_t>(key) * kKV + kvh * kHd;
                        float dot = 0.0f;
                        for (uint32_t d = 0; d < kHd; ++d) dot += q[d] * k[d];
                        s[key] = dot * 0.08838834764831844f;
                        peak = std::max(peak, s[key]);
                    }
                    float sum = 0.0f;
                    for (uint32_t key = 0; key < count; ++key) {
                        s[key] = std::exp(s[key] - peak);
                        sum += s[key];
                    }
                    float* out = A.data() + static_cast<size_t>(qi) * kQ + h * kHd;
                    for (uint32_t d = 0; d < kHd; ++d) {
                        float value = 0.0f;
                        for (uint32_t key = 0; key < count; ++key) value += (s[key] / sum) * vl[static_cast<size_t>(key) * kKV + kvh * kHd + d];
                        out[d] = value;
                    }
                }
            linear(w.o.data(), kD, kQ, A.data(), t, P.data());
            for (size_t i = 0; i < H.size(); ++i) H[i] = H[i] + P[i];
            rmsnorm_rows(H.data(), t, kD, w.post_ln.data(), Xn.data());
            linear(w.gate.data(), kF, kD, Xn.data(), t, G.data());
            linear(w.up.data(), kF, kD, Xn.data(), t, U.data());
            for (size_t i = 0; i < G.size(); ++i) {
                const float a = mutation == 5 ? U[i] : G[i], b = mutation == 5 ? G[i] : U[i];
                G[i] = (a / (1.0f + std::exp(-a))) * b;
            }
            linear(w.down.data(), kD, kF, G.data(), t, P.data());
            for (size_t i = 0; i < H.size(); ++i) H[i] = H[i] + P[i];
        }
        std::vector<float> last(kD), logits(kV);
        rmsnorm_rows(H.data() + static_cast<size_t>(t - 1) * kD, 1, kD, norm.data(), last.data());
        linear(embed.data(), kV, kD, last.data(), 1, logits.data());
        float bv = -INFINITY;
        uint32_t bi = 0;
        for (uint32_t i = 0; i < kV; ++i)
            if (logits[i] > bv) {
                bv = logits[i];
                bi = i;
            }
        selected = bi;
        return logits;
    }
};

namespace {

template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::invalid_argument& e) {
        orc_error_message() = e.what();
        return -1;
    } catch (const std::runtime_error& e) {
        orc_error_message() = e.what();
        return -2;
    } catch (const std::exception& e) {
        orc_error_message() = e.what();
        return -3;
    }
}

}  // namespace

extern "C" {

orc_qwen* orc_qwen_create(const orc_tensor* tensors, int32_t count, uint32_t layers, char* err, size_t err_len) {
    std::unordered_map<std::string, const orc_tensor*> by;
    for (int32_t i = 0; i < count; ++i) by[tensors[i].name] = &tensors[i];
    auto m = new orc_qwen();
    try {
        auto get = [&](const std::string& name, std::vector<int64_t> shape) {
            auto it = by.find(name);
            if (it == by.end()) throw std::runtime_error("Missing tensor: " + name);
            const orc_tensor* t = it->second;
            if (std::vector<int64_t>(t->shape, t->shape + t->ndim) != shape) throw std::invalid_argument("Unsupported Qwen shape: " + name);
            size_t n = 1;
            for (int64_t s : shape) n *= static_cast<size_t>(s);
            return std::vector<float>(t->data, t->data + n);
        };
        m->layers = layers;
        m->embed = get("qwen.model.embed_tokens.weight", {kV, kD});
        m->L.resize(layers);
        for (uint32_t i = 0; i < layers; ++i) {
            const std::string p = "qwen.model.layers." + std::to_string(i);
            QLayer& w = m->L[i];
            w.q = get(p + ".self_attn.q_proj.weight", {kQ, kD});
            w.k = get(p + ".self_attn.k_proj.weight", {kKV, kD});
            w.v = get(p + ".self_attn.v_proj.weight", {kKV, kD});
            w.o = get(p + ".self_attn.o_proj.weight", {kD, kQ});
            w.q_norm = get(p + ".self_attn.q_norm.weight", {kHd});
            w.k_norm = get(p + ".self_attn.k_norm.weight", {kHd});
            w.gate = get(p + ".mlp.gate_proj.weight", {kF, kD});
            w.up = get(p + ".mlp.up_proj.weight", {kF, kD});
            w.down = get(p + ".mlp.down_proj.weight", {kD, kF});
            w.in_ln = get(p + ".input_layernorm.weight", {kD});
            w.post_ln = get(p + ".post_attention_layernorm.weight", {kD});
        }
        m->norm = get("qwen.model.norm.weight", {kD});
        m->kc.assign(static_cast<size_t>(layers) * kCap * kKV, 0.0f);
        m->vc.assign(m->kc.size(), 0.0f);
        m->inv_freq.resize(64);
        for (uint32_t j = 0; j < 64; ++j) m->inv_freq[j] = std::pow(1000000.0f, -static_cast<float>(j) / 64.0f);
    } catch (const std::exception& e) {
        if (err && err_len) {
            std::strncpy(err, e.what(), err_len - 1);
            err[err_len - 1] = 0;
        }
        delete m;
        return nullptr;
    }
    return m;
}

void orc_qwen_destroy(orc_qwen* m) { delete m; }
uint32_t orc_qwen_cached(const orc_qwen* m) { return m->cached; }
void orc_qwen_set_mutation(orc_qwen* m, int32_t mutation) { m->mutation = mutation; }

int orc_qwen_prefill(orc_qwen* m, const uint32_t* ids, uint32_t n, float* logits) {
    return guarded([&] {
        if (n == 0 || n > kPrompt) throw std::invalid_argument("Qwen prompt capacity is 3072 tokens");
        std::fill(m->kc.begin(), m->kc.end(), 0.0f);
        std::fill(m->vc.begin(), m->vc.end(), 0.0f);
        auto out = m->run(std::vector<uint32_t>(ids, ids + n), 0);
        m->cached = n;
        std::copy(out.begin(), out.end(), logits);
    });
}

int orc_qwen_step(orc_qwen* m, uint32_t id, float* logits) {
    return guarded([&] {
        if (!m->cached || m->cached >= kCap) throw std::invalid_argument("Qwen cache capacity exceeded");
        auto out = m->run({id}, m->cached);
        m->cached++;
        std::copy(out.begin(), out.end(), logits);
    });
}

int orc_qwen_generate(orc_qwen* m, const uint32_t* ids, uint32_t n, uint32_t maximum, uint32_t* out, uint32_t* count) {
    *count = 0;
    return guarded([&] {
        if (!maximum || maximum > kMaxGen || static_cast<uint64_t>(n) + maximum > kCap)
            throw std::invalid_argument("Qwen generation capacity exceeded");
        if (n == 0 || n > kPrompt) throw std::invalid_argument("Qwen prompt capacity is 3072 tokens");
        std::fill(m->kc.begin(), m->kc.end(), 0.0f);
        std::fill(m->vc.begin(), m->vc.end(), 0.0f);
        m->run(std::vector<uint32_t>(ids, ids + n), 0);
        m->cached = n;
        for (uint32_t i = 0; i < maximum; ++i) {
            const uint32_t id = m->selected;
            out[(*count)++] = id;
            if (id == ORC_QWEN_EOS) return;
            if (i + 1 < maximum) {
                m->run({id}, m->cached);
                m->cached++;
            }
        }
        throw std::runtime_error("Qwen did not reach EOS within 1024 generated tokens");
    });
}

int orc_qwen_kv_row(const orc_qwen* m, uint32_t layer, int32_t is_v, uint32_t pos, float* out) {
    if (layer >= m->layers || pos >= kCap) return -1;
    const std::vector<float>& c = is_v ? m->vc : m->kc;
    const float* src = c.data() + (static_cast<size_t>(layer) * kCap + pos) * kKV;
    std::copy(src, src + kKV, out);
    return 0;
}

}  // extern "C"

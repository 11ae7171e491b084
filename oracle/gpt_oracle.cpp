// CPU oracle for the IndexTTS 2.5 GPT semantic-token loop.
//
// TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's CPU
// baseline leg load this library to compare the HIP path against.  The product never
// links it.
//
// Follows, op for op:
//   src/gpt.cpp:42-71    prefix construction (prepare)
//   src/gpt.cpp:72-87    prefill / step / checkpoint / restore
//   src/gpt.cpp:88-125   the per-layer forward (pre-LN GPT-2 block, ln_f, final_norm, mel_head)
//   src/gpt_sampling.cpp:11-26    SplitMix64
//   src/gpt_sampling.cpp:28-128   repetition penalty -> temperature -> top-k -> top-p
//   src/gpt_sampling.cpp:130-165  categorical sampling
//   src/gpt_sampling.cpp:168-245  greedy/sampled loop and beam search
// Per-op math follows vendor/metal-runtime/metal/kernels.metal:
//   486-503 (tanh GELU with +-10 clamp), 618-669 (two-pass LayerNorm, biased variance),
//   1054-1080 (GEMV: dot, then + bias), 2064-2145 (decode attention, max-subtracted exp,
//   division by the sum at the end), 2249-2292 (causal prefill attention), 1310-1324
//   (mel_emb[code] + mel_pos[position]).
// Summation order inside a dot product is sequential here; the GPU path uses its
// own order, so forward parity is tolerance based (logits 1e-3 abs / 1e-4 rel).
#include "gpt_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <limits>
#include <memory>
#include <numeric>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

thread_local std::string g_err;

constexpr uint32_t kHeadDim = 64;
constexpr uint32_t kMelVocab = 8194;
constexpr uint32_t kMelStart = 8192;
constexpr uint32_t kMelStop = 8193;

struct Layer {
    const float *ln1_w, *ln1_b, *attn_w, *attn_b, *proj_w, *proj_b;
    const float *ln2_w, *ln2_b, *fc_w, *fc_b, *fc2_w, *fc2_b;
};

struct Snapshot {
    uint32_t tokens = 0;
    std::vector<float> kv;  // [layer][K|V][tokens][width]
};

}  // namespace

// The thread's last error message, shared with the Qwen oracle (qwen_oracle.cpp).
std::string& orc_error_message() { return g_err; }

struct orc_model {
    uint32_t width = 0, heads = 0, ffn = 0, layers = 0, cap = 0;
    uint32_t text_vocab = 0, lang_vocab = 0, text_pos_rows = 0, mel_pos_rows = 0;
    const float *spk_w = nullptr, *spk_b = nullptr;
    const float *text_emb = nullptr, *text_pos = nullptr, *lang_emb = nullptr;
    const float *mel_emb = nullptr, *mel_pos = nullptr;
    const float *lnf_w = nullptr, *lnf_b = nullptr, *fn_w = nullptr, *fn_b = nullptr;
    const float *head_w = nullptr, *head_b = nullptr;
    std::vector<Layer> L;
    std::vector<std::vector<float>> K, V;  // per layer [cap][width]
    uint32_t cached = 0;
};

namespace {

// ---------------------------------------------------------------- primitives

// y[t][j] = (sum_i x[t][i] * W[i][j]) + b[j]; W in HF Conv1D layout [in][out].
// gpt.cpp:24-37 transposes to [out][in] and runs y = W x + b (kernels.metal:1054-1080).
void conv1d(const float* x, uint32_t T, uint32_t in, const float* W, const float* b, uint32_t out, float* y) {
    constexpr uint32_t JB = 64;
    const int64_t nblk = (out + JB - 1) / JB;
#pragma omp parallel
    {
        std::vector<float> acc(static_cast<size_t>(T) * JB);
#pragma omp for schedule(static)
        for (int64_t blk = 0; blk < nblk; ++blk) {
            const uint32_t j0 = static_cast<uint32_t>(blk) * JB;
            const uint32_t jn = std::min(JB, out - j0);
            std::fill(acc.begin(), acc.end(), 0.0f);
            for (uint32_t i = 0; i < in; ++i) {
                const float* wr = W + static_cast<size_t>(i) * out + j0;
                for (uint32_t t = 0; t < T; ++t) {
                    const float xv = x[static_cast<size_t>(t) * in + i];
                    float* a = &acc[static_cast<size_t>(t) * JB];
                    for (uint32_t j = 0; j < jn; ++j) a[j] += xv * wr[j];
                }
            }
            for (uint32_t t = 0; t < T; ++t)
                for (uint32_t j = 0; j < jn; ++j)
                    y[static_cast<size_t>(t) * out + j0 + j] = acc[static_cast<size_t>(t) * JB + j] + b[j0 + j];
        }
    }
}

// y[j] = dot(W[j][:], x) + b[j]; W in [out][in] layout (nn.Linear, mel_head: gpt.cpp:122).
void linear_rows(const float* x, uint32_t in, const float* W, const float* b, uint32_t out, float* y) {
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < static_cast<int64_t>(out); ++j) {
        const float* w = W + static_cast<size_t>(j) * in;
        float acc = 0.0f;
        for (uint32_t i = 0; i < in; ++i) acc += w[i] * x[i];
        y[j] = acc + b[j];
    }
}

// kernels.metal:618-669: mean, biased variance, 1/sqrt(var + eps), (x-mean)*inv*g + b.
void layernorm(const float* x, const float* g, const float* b, uint32_t width, float eps, float* out) {
    float sum = 0.0f;
    for (uint32_t i = 0; i < width; ++i) sum += x[i];
    const float mean = sum / static_cast<float>(width);
    float var = 0.0f;
    for (uint32_t i = 0; i < width; ++i) {
        const float d = x[i] - mean;
        var += d * d;
    }
    const float inv = 1.0f / std::sqrt(var / static_cast<float>(width) + eps);
    for (uint32_t i = 0; i < width; ++i) out[i] = (x[i] - mean) * inv * g[i] + b[i];
}

// kernels.metal:486-503.
float gelu(float v) {
    const float c = 0.7978845608028654f;
    if (v > 10.0f) return v;
    if (v < -10.0f) return 0.0f;
    return 0.5f * v * (1.0f + std::tanh(c * (v + 0.044715f * v * v * v)));
}

// Attention of one query row against keys 0..n_keys-1 of one head.
// kernels.metal:2064-2145: score = (q.k) * rsqrt(64); w = exp(score - max); out = sum(w v) / sum(w).
void attend(const float* q, const float* Kb, const float* Vb, size_t row_stride, uint32_t n_keys, float* out,
            std::vector<float>& scores) {
    const float scale = 1.0f / std::sqrt(static_cast<float>(kHeadDim));
    scores.resize(n_keys);
    float mx = -std::numeric_limits<float>::infinity();
    for (uint32_t t = 0; t < n_keys; ++t) {
        const float* k = Kb + static_cast<size_t>(t) * row_stride;
        float s = 0.0f;
        for (uint32_t d = 0; d < kHeadDim; ++d) s += q[d] * k[d];
        s *= scale;
        scores[t] = s;
        mx = std::max(mx, s);
    }
    float denom = 0.0f;
    for (uint32_t t = 0; t < n_keys; ++t) {
        scores[t] = std::exp(scores[t] - mx);
        denom += scores[t];
    }
    for (uint32_t d = 0; d < kHeadDim; ++d) {
        float acc = 0.0f;
        for (uint32_t t = 0; t < n_keys; ++t) acc += scores[t] * Vb[static_cast<size_t>(t) * row_stride + d];
        out[d] = acc / denom;
    }
}

// ---------------------------------------------------------------- forward (gpt.cpp:88-125)

std::vector<float> run(orc_model& m, const float* input, uint32_t t, bool initial) {
    const uint32_t W = m.width, F = m.ffn;
    std::vector<float> hidden(input, input + static_cast<size_t>(t) * W);
    std::vector<float> xn(static_cast<size_t>(t) * W), qkv(static_cast<size_t>(t) * 3 * W);
    std::vector<float> att(static_cast<size_t>(t) * W), tmp(static_cast<size_t>(t) * W);
    std::vector<float> ff(static_cast<size_t>(t) * F);
    const uint32_t base = initial ? 0 : m.cached;  // first cache row written by this call
    for (uint32_t l = 0; l < m.layers; ++l) {
        const Layer& p = m.L[l];
        for (uint32_t r = 0; r < t; ++r) layernorm(&hidden[r * W], p.ln1_w, p.ln1_b, W, 1e-5f, &xn[r * W]);
        conv1d(xn.data(), t, W, p.attn_w, p.attn_b, 3 * W, qkv.data());
        // KV store (kernels.metal:1250-1266) / in-place append (kernels.metal:2087-2092).
        for (uint32_t r = 0; r < t; ++r) {
            std::memcpy(&m.K[l][static_cast<size_t>(base + r) * W], &qkv[static_cast<size_t>(r) * 3 * W + W], W * 4);
            std::memcpy(&m.V[l][static_cast<size_t>(base + r) * W], &qkv[static_cast<size_t>(r) * 3 * W + 2 * W], W * 4);
        }
        const int64_t jobs = static_cast<int64_t>(t) * m.heads;
#pragma omp parallel
        {
            std::vector<float> scores;
#pragma omp for schedule(dynamic, 4)
            for (int64_t job = 0; job < jobs; ++job) {
                const uint32_t r = static_cast<uint32_t>(job / m.heads), h = static_cast<uint32_t>(job % m.heads);
                const uint32_t n_keys = base + r + 1;  // causal: keys 0..query
                attend(&qkv[static_cast<size_t>(r) * 3 * W + h * kHeadDim], &m.K[l][h * kHeadDim], &m.V[l][h * kHeadDim],
                       W, n_keys, &att[static_cast<size_t>(r) * W + h * kHeadDim], scores);
            }
        }
        conv1d(att.data(), t, W, p.proj_w, p.proj_b, W, tmp.data());
        for (size_t i = 0; i < hidden.size(); ++i) hidden[i] = hidden[i] + tmp[i];  // residual (add_f32_pass)
        for (uint32_t r = 0; r < t; ++r) layernorm(&hidden[r * W], p.ln2_w, p.ln2_b, W, 1e-5f, &xn[r * W]);
        conv1d(xn.data(), t, W, p.fc_w, p.fc_b, F, ff.data());
        for (auto& v : ff) v = gelu(v);
        conv1d(ff.data(), t, F, p.fc2_w, p.fc2_b, W, tmp.data());
        for (size_t i = 0; i < hidden.size(); ++i) hidden[i] = hidden[i] + tmp[i];
    }
    std::vector<float> last(hidden.end() - W, hidden.end()), a(W), b(W);
    layernorm(last.data(), m.lnf_w, m.lnf_b, W, 1e-5f, a.data());
    layernorm(a.data(), m.fn_w, m.fn_b, W, 1e-5f, b.data());
    std::vector<float> logits(kMelVocab);
    linear_rows(b.data(), W, m.head_w, m.head_b, kMelVocab, logits.data());
    return logits;
}

std::vector<float> prefill(orc_model& m, const float* prefix, size_t count) {
    if (count == 0 || count % m.width || count / m.width > 1024 || count / m.width > m.cap)
        throw std::invalid_argument("Invalid GPT prefill dimensions");
    const uint32_t t = static_cast<uint32_t>(count / m.width);
    auto logits = run(m, prefix, t, true);
    m.cached = t;
    return logits;
}

std::vector<float> step(orc_model& m, uint32_t code, uint32_t position) {
    if (!m.cached || m.cached >= m.cap || code >= kMelVocab || position >= m.mel_pos_rows)
        throw std::invalid_argument("GPT step requires valid cache, code and position");
    // gpt_build_current (kernels.metal:1310-1324).
    std::vector<float> x(m.width);
    for (uint32_t i = 0; i < m.width; ++i)
        x[i] = m.mel_emb[static_cast<size_t>(code) * m.width + i] + m.mel_pos[static_cast<size_t>(position) * m.width + i];
    auto logits = run(m, x.data(), 1, false);
    m.cached++;
    return logits;
}

std::shared_ptr<Snapshot> checkpoint(const orc_model& m) {
    auto s = std::make_shared<Snapshot>();
    s->tokens = m.cached;
    const size_t row = static_cast<size_t>(m.cached) * m.width;
    s->kv.resize(row * 2 * m.layers);
    for (uint32_t l = 0; l < m.layers; ++l) {
        std::memcpy(&s->kv[(2 * l) * row], m.K[l].data(), row * 4);
        std::memcpy(&s->kv[(2 * l + 1) * row], m.V[l].data(), row * 4);
    }
    return s;
}

void restore(orc_model& m, const Snapshot& s) {
    const size_t row = static_cast<size_t>(s.tokens) * m.width;
    for (uint32_t l = 0; l < m.layers; ++l) {
        std::memcpy(m.K[l].data(), &s.kv[(2 * l) * row], row * 4);
        std::memcpy(m.V[l].data(), &s.kv[(2 * l + 1) * row], row * 4);
    }
    m.cached = s.tokens;
}

// ---------------------------------------------------------------- sampling (gpt_sampling.cpp)

struct SplitMix64 {
    uint64_t state;
    uint64_t next_u64() {
        uint64_t z = (state += 0x9E3779B97F4A7C15ULL);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        return z ^ (z >> 31);
    }
    double next_unit() { return static_cast<double>(next_u64() >> 11) * (1.0 / 9007199254740992.0); }
};

std::vector<float> processors(const std::vector<float>& logits, const std::vector<uint32_t>& history, const orc_options& c) {
    std::vector<float> s = logits;
    constexpr float neg_inf = -std::numeric_limits<float>::infinity();
    if (c.repetition_penalty != 1.0f) {
        if (c.repetition_penalty <= 0.0f) throw std::runtime_error("GPT repetition penalty must be positive");
        std::vector<uint8_t> seen(s.size(), 0);
        for (uint32_t tok : history) {
            if (tok >= s.size() || seen[tok]) continue;
            seen[tok] = 1;
            s[tok] = s[tok] < 0.0f ? s[tok] * c.repetition_penalty : s[tok] / c.repetition_penalty;
        }
    }
    if (c.temperature <= 0.0f) throw std::runtime_error("GPT sampling temperature must be positive");
    if (c.temperature != 1.0f)
        for (float& v : s) v /= c.temperature;
    if (c.top_k > 0 && c.top_k < s.size()) {
        std::vector<float> sorted = s;
        const size_t kth = static_cast<size_t>(std::max(c.top_k, c.num_beams > 1 ? 2u : 1u) - 1);
        std::nth_element(sorted.begin(), sorted.begin() + kth, sorted.end(), std::greater<float>());
        const float pivot = sorted[kth];
        for (float& v : s)
            if (v < pivot) v = neg_inf;
    }
    if (c.top_p < 1.0f) {
        if (c.top_p <= 0.0f) throw std::runtime_error("GPT top_p must be in (0, 1]");
        std::vector<size_t> order(s.size());
        std::iota(order.begin(), order.end(), size_t(0));
        std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return s[a] == s[b] ? a < b : s[a] < s[b]; });
        float mx = neg_inf;
        for (float v : s)
            if (std::isfinite(v)) mx = std::max(mx, v);
        if (!std::isfinite(mx)) throw std::runtime_error("GPT top_p filtering removed all logits");
        double total = 0.0;
        std::vector<double> probs(s.size(), 0.0);
        for (size_t i = 0; i < s.size(); ++i)
            if (std::isfinite(s[i])) {
                probs[i] = std::exp(static_cast<double>(s[i] - mx));
                total += probs[i];
            }
        if (total <= 0.0) throw std::runtime_error("GPT sampling probability mass is zero");
        double cumulative = 0.0;
        std::vector<uint8_t> remove(s.size(), 0);
        const double threshold = 1.0 - static_cast<double>(c.top_p);
        size_t finite_seen = 0;
        for (size_t idx : order) {
            if (!std::isfinite(s[idx])) {
                remove[idx] = 1;
                continue;
            }
            ++finite_seen;
            cumulative += probs[idx] / total;
            if (cumulative <= threshold) remove[idx] = 1;
        }
        if (finite_seen > 0) {
            const size_t keep = std::min(order.size(), c.num_beams > 1 ? size_t(2) : size_t(1));
            for (size_t i = 0; i < keep; ++i) remove[order[order.size() - 1 - i]] = 0;
        }
        for (size_t i = 0; i < s.size(); ++i)
            if (remove[i]) s[i] = neg_inf;
    }
    return s;
}

uint32_t sample(const std::vector<float>& p, SplitMix64& rng) {
    float mx = -std::numeric_limits<float>::infinity();
    for (float v : p)
        if (std::isfinite(v)) mx = std::max(mx, v);
    if (!std::isfinite(mx)) throw std::runtime_error("GPT sampling received no finite logits");
    double total = 0.0;
    std::vector<double> probs(p.size(), 0.0);
    for (size_t i = 0; i < p.size(); ++i)
        if (std::isfinite(p[i])) {
            probs[i] = std::exp(static_cast<double>(p[i] - mx));
            total += probs[i];
        }
    if (total <= 0.0) throw std::runtime_error("GPT sampling probability mass is zero");
    const double target = rng.next_unit() * total;
    double cumulative = 0.0;
    uint32_t last_finite = 0;
    for (uint32_t i = 0; i < probs.size(); ++i) {
        if (probs[i] <= 0.0) continue;
        last_finite = i;
        cumulative += probs[i];
        if (target < cumulative) return i;
    }
    return last_finite;
}

void suppress(std::vector<float>& logits, const orc_options& c) {
    if (!c.suppress_stop) return;
    logits[kMelStart] = -std::numeric_limits<float>::infinity();
    logits[kMelStop] = -std::numeric_limits<float>::infinity();
}

struct GenResult {
    std::vector<uint32_t> codes;
    bool stopped = false;
};

GenResult generate_beams(orc_model& m, const std::vector<float>& prefix, const orc_options& config, uint32_t maximum) {
    struct Beam {
        std::vector<uint32_t> codes;
        float score = 0;
        std::vector<float> logits;
        std::shared_ptr<Snapshot> state;
    };
    struct Finished {
        std::vector<uint32_t> codes;
        double score;
        bool eos;
    };
    struct Candidate {
        uint32_t parent, token;
        float score;
    };
    SplitMix64 random{config.seed};
    std::vector<Finished> finished;
    Beam initial;
    initial.logits = prefill(m, prefix.data(), prefix.size());
    suppress(initial.logits, config);
    initial.state = checkpoint(m);
    std::vector<Beam> beams(config.num_beams, initial);
    for (uint32_t i = 1; i < beams.size(); ++i) beams[i].score = -1e9f;
    auto finish = [&](const Beam& beam, float score, uint32_t length, bool eos) {
        finished.push_back({beam.codes, score / std::pow(static_cast<double>(std::max(length, 1u)), config.length_penalty), eos});
        // <= num_beams + 1 <= 11 entries: libc++'s std::sort keeps equal elements in order there.
        std::stable_sort(finished.begin(), finished.end(), [](const auto& a, const auto& b) { return a.score > b.score; });
        if (finished.size() > config.num_beams) finished.resize(config.num_beams);
    };
    for (uint32_t step_index = 0; step_index < maximum; ++step_index) {
        std::vector<Candidate> candidates;
        std::vector<float> all_scores;
        for (uint32_t parent = 0; parent < beams.size(); ++parent) {
            auto log_probs = beams[parent].logits;
            float peak = *std::max_element(log_probs.begin(), log_probs.end()), sum = 0;
            for (auto v : log_probs) sum += std::exp(v - peak);
            const float log_sum = peak + std::log(sum);
            for (auto& v : log_probs) v -= log_sum;
            std::vector<uint32_t> history{1, kMelStart};
            history.insert(history.end(), beams[parent].codes.begin(), beams[parent].codes.end());
            auto scores = processors(log_probs, history, config);
            for (auto& v : scores) v += beams[parent].score;
            all_scores.insert(all_scores.end(), scores.begin(), scores.end());
        }
        const uint32_t take = 2 * config.num_beams;
        if (config.do_sample) {
            auto available = all_scores;
            for (uint32_t i = 0; i < take; ++i) {
                const uint32_t id = sample(available, random);
                candidates.push_back({id / kMelVocab, id % kMelVocab, all_scores[id]});
                available[id] = -std::numeric_limits<float>::infinity();
            }
        } else {
            std::vector<uint32_t> order(all_scores.size());
            std::iota(order.begin(), order.end(), 0u);
            std::partial_sort(order.begin(), order.begin() + take, order.end(), [&](auto a, auto b) {
                return all_scores[a] == all_scores[b] ? a < b : all_scores[a] > all_scores[b];
            });
            for (uint32_t i = 0; i < take; ++i) {
                const auto id = order[i];
                candidates.push_back({id / kMelVocab, id % kMelVocab, all_scores[id]});
            }
        }
        // The reference uses std::sort here, built with AppleClang 17 / libc++
        // (docs/standalone-build.txt:1), whose std::sort sorts fewer than 24 elements with
        // stable sorting networks (2..5) and an insertion sort: for take = 2*num_beams <= 20
        // that is the stable order.
        std::stable_sort(candidates.begin(), candidates.end(), [](const auto& a, const auto& b) { return a.score > b.score; });
        std::vector<Beam> next;
        for (uint32_t rank = 0; rank < candidates.size(); ++rank) {
            const auto cand = candidates[rank];
            const auto& parent = beams[cand.parent];
            if (cand.token == kMelStop) {
                if (rank < config.num_beams) finish(parent, cand.score, step_index + 1, true);
                continue;
            }
            if (cand.token >= kMelStart) throw std::runtime_error("Beam generated invalid semantic code");
            Beam child;
            child.codes = parent.codes;
            child.codes.push_back(cand.token);
            child.score = cand.score;
            if (step_index + 1 < maximum) {
                restore(m, *parent.state);
                child.logits = step(m, cand.token, step_index + 2);
                suppress(child.logits, config);
                child.state = checkpoint(m);
            }
            next.push_back(std::move(child));
            if (next.size() == config.num_beams) break;
        }
        if (next.empty()) break;
        beams = std::move(next);
        if (finished.size() == config.num_beams &&
            finished.back().score >= candidates[0].score / std::pow(static_cast<double>(step_index + 1), config.length_penalty)) {
            beams.clear();
            break;
        }
    }
    for (const auto& beam : beams) finish(beam, beam.score, static_cast<uint32_t>(beam.codes.size()), false);
    if (finished.empty()) throw std::runtime_error("Beam search produced no hypotheses");
    return {std::move(finished[0].codes), finished[0].eos};
}

GenResult generate(orc_model& m, const std::vector<float>& prefix, const orc_options& options, uint32_t maximum) {
    if (!maximum || maximum + 1 >= m.mel_pos_rows || prefix.size() / m.width + maximum >= m.cap)
        throw std::invalid_argument("GPT generation capacity exceeded");
    orc_options config = options;
    if (!config.do_sample) {
        config.temperature = 1;
        config.top_k = 0;
        config.top_p = 1;
    }
    if (!std::isfinite(config.temperature) || !std::isfinite(config.top_p) || !std::isfinite(config.repetition_penalty) ||
        config.temperature <= 0 || config.top_p <= 0 || config.top_p > 1 || config.repetition_penalty <= 0)
        throw std::invalid_argument("Invalid GPT generation parameters");
    if (!config.num_beams || config.num_beams > 10 || !std::isfinite(config.length_penalty))
        throw std::invalid_argument("Invalid beam search configuration");
    if (config.num_beams > 1) return generate_beams(m, prefix, config, maximum);
    SplitMix64 random{config.seed};
    GenResult result;
    std::vector<uint32_t> history{1, kMelStart};
    auto logits = prefill(m, prefix.data(), prefix.size());
    suppress(logits, config);
    for (uint32_t i = 0; i < maximum; ++i) {
        auto scores = processors(logits, history, config);
        const uint32_t token = config.do_sample ? sample(scores, random)
                                                : static_cast<uint32_t>(std::max_element(scores.begin(), scores.end()) - scores.begin());
        if (token == kMelStop) {
            result.stopped = true;
            break;
        }
        if (token >= kMelStart) throw std::runtime_error("GPT generated invalid semantic code");
        result.codes.push_back(token);
        history.push_back(token);
        if (i + 1 < maximum) {
            logits = step(m, token, i + 2);
            suppress(logits, config);
        }
    }
    return result;
}

// Prefix rows after the conditioning block (gpt.cpp:44-50, 57-69).
std::vector<float> text_rows(const orc_model& m, const uint32_t* text, uint32_t n_text, uint32_t language) {
    std::vector<uint32_t> ids{0};
    for (uint32_t i = 0; i < n_text; ++i) {
        if (text[i] >= m.text_vocab) throw std::invalid_argument("Text token is outside 2.5 vocabulary");
        if (text[i] != 0 && text[i] != 1) ids.push_back(text[i]);
    }
    ids.push_back(1);
    if (ids.size() > m.text_pos_rows) throw std::invalid_argument("Text segment exceeds GPT position capacity");
    const uint32_t W = m.width;
    std::vector<float> out(static_cast<size_t>(ids.size() + 1) * W);
    for (size_t r = 0; r < ids.size(); ++r)
        for (uint32_t c = 0; c < W; ++c)
            out[r * W + c] = (m.text_emb[static_cast<size_t>(ids[r]) * W + c] + m.text_pos[r * W + c]) +
                             m.lang_emb[static_cast<size_t>(language) * W + c];
    for (uint32_t c = 0; c < W; ++c)
        out[ids.size() * W + c] = m.mel_emb[static_cast<size_t>(kMelStart) * W + c] + m.mel_pos[c];
    return out;
}

template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::invalid_argument& e) {
        g_err = e.what();
        return -1;
    } catch (const std::runtime_error& e) {
        g_err = e.what();
        return -2;
    } catch (const std::exception& e) {
        g_err = e.what();
        return -3;
    }
}

}  // namespace

extern "C" {

orc_model* orc_create(const orc_tensor* tensors, int32_t count, uint32_t kv_capacity, char* err, size_t err_len) {
    std::unordered_map<std::string, const orc_tensor*> by;
    for (int32_t i = 0; i < count; ++i) by[tensors[i].name] = &tensors[i];
    auto fail = [&](const std::string& msg) -> orc_model* {
        if (err && err_len) {
            std::strncpy(err, msg.c_str(), err_len - 1);
            err[err_len - 1] = 0;
        }
        return nullptr;
    };
    auto get = [&](const std::string& name, std::vector<int64_t> shape, bool optional = false) -> const float* {
        auto it = by.find(name);
        if (it == by.end()) {
            if (optional) return nullptr;
            throw std::runtime_error("Missing tensor: " + name);
        }
        const orc_tensor* t = it->second;
        std::vector<int64_t> s(t->shape, t->shape + t->ndim);
        for (size_t i = 0; i < shape.size(); ++i)
            if (shape[i] < 0) shape[i] = i < s.size() ? s[i] : -1;
        if (s != shape) throw std::runtime_error("Unsupported GPT shape: " + name);
        return t->data;
    };
    auto m = std::make_unique<orc_model>();
    try {
        auto it = by.find("gpt.mel_embedding.weight");
        if (it == by.end()) throw std::runtime_error("Missing tensor: gpt.mel_embedding.weight");
        m->width = static_cast<uint32_t>(it->second->shape[1]);
        if (m->width % kHeadDim) throw std::runtime_error("Unsupported GPT width");
        m->heads = m->width / kHeadDim;
        const int64_t W = m->width;
        m->mel_emb = get("gpt.mel_embedding.weight", {kMelVocab, W});
        m->mel_pos = get("gpt.mel_pos_embedding.emb.weight", {-1, W});
        m->mel_pos_rows = static_cast<uint32_t>(by["gpt.mel_pos_embedding.emb.weight"]->shape[0]);
        m->text_emb = get("gpt.text_embedding.weight", {-1, W});
        m->text_vocab = static_cast<uint32_t>(by["gpt.text_embedding.weight"]->shape[0]);
        m->text_pos = get("gpt.text_pos_embedding.emb.weight", {-1, W});
        m->text_pos_rows = static_cast<uint32_t>(by["gpt.text_pos_embedding.emb.weight"]->shape[0]);
        m->lang_emb = get("gpt.lang_embedding.weight", {-1, W});
        m->lang_vocab = static_cast<uint32_t>(by["gpt.lang_embedding.weight"]->shape[0]);
        m->spk_w = get("gpt.spk_emb_proj.weight", {W, 192}, true);
        m->spk_b = get("gpt.spk_emb_proj.bias", {W}, true);
        m->lnf_w = get("gpt.gpt.ln_f.weight", {W});
        m->lnf_b = get("gpt.gpt.ln_f.bias", {W});
        m->fn_w = get("gpt.final_norm.weight", {W});
        m->fn_b = get("gpt.final_norm.bias", {W});
        m->head_w = get("gpt.mel_head.weight", {kMelVocab, W});
        m->head_b = get("gpt.mel_head.bias", {kMelVocab});
        auto fc = by.find("gpt.gpt.h.0.mlp.c_fc.weight");
        if (fc == by.end()) throw std::runtime_error("Missing tensor: gpt.gpt.h.0.mlp.c_fc.weight");
        m->ffn = static_cast<uint32_t>(fc->second->shape[1]);
        const int64_t F = m->ffn;
        for (uint32_t l = 0;; ++l) {
            const std::string p = "gpt.gpt.h." + std::to_string(l);
            if (!by.count(p + ".attn.c_attn.weight")) break;
            Layer L;
            L.ln1_w = get(p + ".ln_1.weight", {W});
            L.ln1_b = get(p + ".ln_1.bias", {W});
            L.attn_w = get(p + ".attn.c_attn.weight", {W, 3 * W});
            L.attn_b = get(p + ".attn.c_attn.bias", {3 * W});
            L.proj_w = get(p + ".attn.c_proj.weight", {W, W});
            L.proj_b = get(p + ".attn.c_proj.bias", {W});
            L.ln2_w = get(p + ".ln_2.weight", {W});
            L.ln2_b = get(p + ".ln_2.bias", {W});
            L.fc_w = get(p + ".mlp.c_fc.weight", {W, F});
            L.fc_b = get(p + ".mlp.c_fc.bias", {F});
            L.fc2_w = get(p + ".mlp.c_proj.weight", {F, W});
            L.fc2_b = get(p + ".mlp.c_proj.bias", {W});
            m->L.push_back(L);
        }
        m->layers = static_cast<uint32_t>(m->L.size());
        if (!m->layers) throw std::runtime_error("GPT has no layers");
        m->cap = kv_capacity ? kv_capacity : 4096;
        m->K.assign(m->layers, std::vector<float>(static_cast<size_t>(m->cap) * W));
        m->V.assign(m->layers, std::vector<float>(static_cast<size_t>(m->cap) * W));
    } catch (const std::exception& e) {
        return fail(e.what());
    }
    return m.release();
}

void orc_destroy(orc_model* m) { delete m; }
uint32_t orc_width(const orc_model* m) { return m->width; }
uint32_t orc_cached_tokens(const orc_model* m) { return m->cached; }
const char* orc_last_error(void) { return g_err.c_str(); }

int orc_prepare_ref(orc_model* m, const float* speaker, const float* emotion, const uint32_t* text, uint32_t n_text,
                    uint32_t language, float* prefix_out, uint32_t* rows) {
    return guarded([&] {
        if (!m->spk_w || !speaker || !emotion || language >= m->lang_vocab)
            throw std::invalid_argument("Invalid GPT conditioning dimensions");
        const uint32_t W = m->width;
        // linear_rows_f32_rowmajor (kernels.metal:1352-1374): acc = bias, then += w*x.
        std::vector<float> cond(static_cast<size_t>(3) * W, 0.0f);
        for (uint32_t r = 0; r < W; ++r) {
            float acc = m->spk_b[r];
            for (uint32_t c = 0; c < 192; ++c) acc += m->spk_w[static_cast<size_t>(r) * 192 + c] * speaker[c];
            cond[r] = acc + emotion[r];
        }
        auto tail = text_rows(*m, text, n_text, language);
        std::memcpy(prefix_out, cond.data(), cond.size() * 4);
        std::memcpy(prefix_out + cond.size(), tail.data(), tail.size() * 4);
        *rows = static_cast<uint32_t>((cond.size() + tail.size()) / W);
    });
}

int orc_prepare_cond(orc_model* m, const float* cond, uint32_t n_cond, const uint32_t* text, uint32_t n_text,
                     uint32_t language, float* prefix_out, uint32_t* rows) {
    return guarded([&] {
        if (!n_cond || language >= m->lang_vocab) throw std::invalid_argument("Invalid GPT conditioning dimensions");
        const uint32_t W = m->width;
        auto tail = text_rows(*m, text, n_text, language);
        std::memcpy(prefix_out, cond, static_cast<size_t>(n_cond) * W * 4);
        std::memcpy(prefix_out + static_cast<size_t>(n_cond) * W, tail.data(), tail.size() * 4);
        *rows = static_cast<uint32_t>(n_cond + tail.size() / W);
    });
}

int orc_prefill(orc_model* m, const float* prefix, uint32_t rows, float* logits) {
    return guarded([&] {
        auto out = prefill(*m, prefix, static_cast<size_t>(rows) * m->width);
        std::memcpy(logits, out.data(), out.size() * 4);
    });
}

int orc_step(orc_model* m, uint32_t code, uint32_t position, float* logits) {
    return guarded([&] {
        auto out = step(*m, code, position);
        std::memcpy(logits, out.data(), out.size() * 4);
    });
}

int orc_kv_row(const orc_model* m, uint32_t layer, int32_t is_v, uint32_t pos, float* out) {
    return guarded([&] {
        if (layer >= m->layers || pos >= m->cap) throw std::invalid_argument("Invalid KV row");
        const auto& src = is_v ? m->V[layer] : m->K[layer];
        std::memcpy(out, &src[static_cast<size_t>(pos) * m->width], m->width * 4);
    });
}

struct orc_state {
    std::shared_ptr<Snapshot> s;
};

orc_state* orc_checkpoint(const orc_model* m) {
    orc_state* out = nullptr;
    (void)guarded([&] {
        if (!m->cached) throw std::invalid_argument("Invalid KV snapshot");
        out = new orc_state{checkpoint(*m)};
    });
    return out;
}

int orc_restore(orc_model* m, const orc_state* st) {
    return guarded([&] {
        if (!st || !st->s || !st->s->tokens) throw std::invalid_argument("Invalid KV restore");
        restore(*m, *st->s);
    });
}

void orc_state_free(orc_state* st) { delete st; }

int orc_processors(const float* logits, uint32_t vocab, const uint32_t* history, uint32_t n_history,
                   const orc_options* opt, float* out) {
    return guarded([&] {
        std::vector<float> l(logits, logits + vocab);
        std::vector<uint32_t> h(history, history + n_history);
        auto s = processors(l, h, *opt);
        std::memcpy(out, s.data(), s.size() * 4);
    });
}

int orc_sample(const float* processed, uint32_t vocab, uint64_t* rng_state, uint32_t* token) {
    return guarded([&] {
        SplitMix64 r{*rng_state};
        *token = sample(std::vector<float>(processed, processed + vocab), r);
        *rng_state = r.state;
    });
}

uint64_t orc_splitmix_next(uint64_t* state) {
    SplitMix64 r{*state};
    const uint64_t v = r.next_u64();
    *state = r.state;
    return v;
}

double orc_splitmix_unit(uint64_t* state) {
    SplitMix64 r{*state};
    const double v = r.next_unit();
    *state = r.state;
    return v;
}

int orc_generate(orc_model* m, const float* prefix, uint32_t rows, const orc_options* opt, uint32_t max_tokens,
                 uint32_t* codes_out, uint32_t* n_codes, int32_t* stopped) {
    return guarded([&] {
        std::vector<float> p(prefix, prefix + static_cast<size_t>(rows) * m->width);
        auto r = generate(*m, p, *opt, max_tokens);
        std::copy(r.codes.begin(), r.codes.end(), codes_out);
        *n_codes = static_cast<uint32_t>(r.codes.size());
        *stopped = r.stopped ? 1 : 0;
    });
}

void orc_libm_eval(int32_t fn, uint64_t first, uint64_t stride, uint64_t count, void* out) {
#pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < count; ++i) {
        const uint32_t b = static_cast<uint32_t>(first + i * stride);
        float x;
        std::memcpy(&x, &b, 4);
        if (fn == 0)
            static_cast<float*>(out)[i] = expf(x);
        else if (fn == 1)
            static_cast<double*>(out)[i] = exp(static_cast<double>(x));
        else
            static_cast<float*>(out)[i] = logf(x);
    }
}

float orc_gelu(float v) { return gelu(v); }
void orc_layernorm(const float* x, const float* g, const float* b, uint32_t width, float eps, float* out) {
    layernorm(x, g, b, width, eps, out);
}

}  // extern "C"

// Driver around the reference's own sampler source (src/gpt_sampling.cpp), compiled
// where it lies under the reference tree by oracle/Makefile (target `ref`) into
// oracle/_ref/ref_sampling.  TEST INFRASTRUCTURE ONLY: it exists to check the
// oracle's restatement of apply_gpt_sampling_processors (gpt_sampling.cpp:28-128),
// sample_gpt_token_from_logits (:130-165) and SplitMix64 (:11-26) on the same inputs.
//
// The reference translation unit also defines GptDecoder::generate/generate_beams,
// which call Metal-backed members that cannot be built here; they are never called,
// and the link leaves those symbols unresolved on purpose.
//
// Protocol (little-endian binary, stdin -> stdout), repeated until EOF:
//   u32 op                     1 = processors, 2 = sample
//   op 1: u32 vocab, u32 n_hist, f32 temperature, u32 top_k, f32 top_p, f32 penalty,
//         u32 num_beams, f32 logits[vocab], u32 history[n_hist]
//         -> i32 status, f32 scores[vocab] (status 0) or u32 len + message
//   op 2: u32 vocab, u64 seed, u32 draws, f32 processed[vocab]
//         -> i32 status, u32 tokens[draws], u64 final_state
#include REF_SAMPLING_SOURCE

#include <cstdio>
#include <cstring>
#include <exception>
#include <vector>

namespace {
template <class T>
bool rd(T* v, size_t n = 1) {
    return std::fread(v, sizeof(T), n, stdin) == n;
}
template <class T>
void wr(const T* v, size_t n = 1) {
    std::fwrite(v, sizeof(T), n, stdout);
}
void fail(const char* msg) {
    const int32_t st = 1;
    const uint32_t len = static_cast<uint32_t>(std::strlen(msg));
    wr(&st);
    wr(&len);
    wr(msg, len);
}
}  // namespace

int main() {
    uint32_t op;
    while (rd(&op)) {
        if (op == 1) {
            uint32_t vocab, n_hist, top_k, beams;
            float temperature, top_p, penalty;
            if (!rd(&vocab) || !rd(&n_hist) || !rd(&temperature) || !rd(&top_k) || !rd(&top_p) || !rd(&penalty) || !rd(&beams))
                return 2;
            std::vector<float> logits(vocab);
            std::vector<uint32_t> history(n_hist);
            if (!rd(logits.data(), vocab) || (n_hist && !rd(history.data(), n_hist))) return 2;
            itts25::GenerationOptions o;
            o.temperature = temperature;
            o.top_k = top_k;
            o.top_p = top_p;
            o.repetition_penalty = penalty;
            o.num_beams = beams;
            try {
                auto s = itts25::apply_gpt_sampling_processors(logits, history, o);
                const int32_t st = 0;
                wr(&st);
                wr(s.data(), s.size());
            } catch (const std::exception& e) {
                fail(e.what());
            }
        } else if (op == 2) {
            uint32_t vocab, draws;
            uint64_t seed;
            if (!rd(&vocab) || !rd(&seed) || !rd(&draws)) return 2;
            std::vector<float> p(vocab);
            if (!rd(p.data(), vocab)) return 2;
            itts25::SplitMix64 rng(seed);
            try {
                std::vector<uint32_t> out(draws);
                for (uint32_t i = 0; i < draws; ++i) out[i] = itts25::sample_gpt_token_from_logits(p, rng);
                const int32_t st = 0;
                wr(&st);
                wr(out.data(), out.size());
                wr(&rng.state);
            } catch (const std::exception& e) {
                fail(e.what());
            }
        } else {
            return 3;
        }
        std::fflush(stdout);
    }
    return 0;
}

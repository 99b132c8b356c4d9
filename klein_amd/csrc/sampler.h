// klein::Sampler on the MI355X sampler — the same public interface as klein's src/sampler.h:13-38.
//
// SamplerParams is unchanged (fields, order, defaults). Sampler keeps explicit Sampler(const SamplerParams&),
// reset(), accept(int32_t), sample(const float*, int) and params(), with the reference's semantics: one
// mt19937_64 draw per non-greedy sample (none when temperature <= 0), seed 0 meaning std::random_device.
// sample() takes a device pointer (read in place) or a host pointer (copied first). verify() adds the
// engine's 4-row verify/accept loop (src/engine.cpp:563-575) as one GPU step. A failing GPU call prints the
// error and exits, as klein's fatal() does (src/common.cpp:30-39).
#pragma once

#include <cstdint>
#include <random>
#include <vector>

#include "klein_sampler.h"

namespace klein {

struct SamplerParams {
    float temperature = 1.0f;   // <= 0: greedy
    int top_k = 20;             // <= 0: no limit
    float top_p = 0.95f;
    float min_p = 0.0f;
    float presence_penalty = 0.0f;
    float frequency_penalty = 0.0f;
    float repetition_penalty = 1.0f;
    uint64_t seed = 0;          // 0: random
};

class Sampler {
public:
    explicit Sampler(const SamplerParams& p);
    ~Sampler();
    Sampler(const Sampler&) = delete;
    Sampler& operator=(const Sampler&) = delete;
    void reset();
    void accept(int32_t token);
    int32_t sample(const float* logits, int n_vocab);
    const SamplerParams& params() const { return p_; }

    // The verify loop of Engine::generate in one call: rows 0..nb-1 of `logits` (row i at logits + i*n_vocab),
    // drafts[i] = batch[i+1]. Writes the emitted tokens to tokens[0..accepted], accepts them into the history
    // and returns `accepted`. Consumes accepted+1 draws of the generator when temperature > 0.
    int verify(const float* logits, int n_vocab, int nb, const int32_t* drafts, int32_t* tokens);

private:
    void ensure(int n_vocab);
    double draw_peek(std::mt19937_64& g) const;

    SamplerParams p_;
    std::mt19937_64 rng_;
    kls_handle h_ = nullptr;
    int n_vocab_ = 0;
    std::vector<int32_t> early_;  // accepted before the vocabulary size was known
};

}  // namespace klein

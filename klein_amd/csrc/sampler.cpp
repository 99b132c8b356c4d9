// klein::Sampler over the C ABI of the MI355X sampler (klein_sampler.h). Mirrors src/sampler.cpp:11-89.
#include "sampler.h"

#include <cstdio>
#include <cstdlib>
#include <limits>

namespace klein {

namespace {

[[noreturn]] void fatal_status(const char* what, int st) {
    std::fprintf(stderr, "error: %s: %s (%s)\n", what, kls_status_string(st), kls_last_error());
    std::exit(1);
}

kls_params to_c(const SamplerParams& p) {
    return kls_params{p.temperature, p.top_k, p.top_p, p.min_p, p.presence_penalty, p.frequency_penalty,
                      p.repetition_penalty, p.seed};
}

// The uniform std::uniform_real_distribution<double> draws from the engine (libstdc++: generate_canonical).
double canonical(std::mt19937_64& g) { return std::generate_canonical<double, std::numeric_limits<double>::digits>(g); }

}  // namespace

// sampler.cpp:11 — seed 0 draws a seed from std::random_device
Sampler::Sampler(const SamplerParams& p) : p_(p), rng_(p.seed ? p.seed : std::random_device{}()) {}

Sampler::~Sampler() {
    if (h_) kls_destroy(h_);
}

void Sampler::ensure(int n_vocab) {
    if (h_ && n_vocab == n_vocab_) return;
    if (h_) {  // a different vocabulary: start a new handle carrying the history over is not possible; refuse
        std::fprintf(stderr, "error: Sampler used with n_vocab %d after %d\n", n_vocab, n_vocab_);
        std::exit(1);
    }
    const kls_params cp = to_c(p_);
    if (int st = kls_create(&cp, n_vocab, 16, &h_)) fatal_status("kls_create", st);
    n_vocab_ = n_vocab;
    for (int32_t t : early_)
        if (int st = kls_accept(h_, t)) fatal_status("kls_accept", st);
    early_.clear();
}

// sampler.cpp:13
void Sampler::reset() {
    early_.clear();
    if (h_)
        if (int st = kls_reset(h_)) fatal_status("kls_reset", st);
}

// sampler.cpp:15
void Sampler::accept(int32_t token) {
    if (!h_) {
        early_.push_back(token);
        return;
    }
    if (int st = kls_accept(h_, token)) fatal_status("kls_accept", st);
}

double Sampler::draw_peek(std::mt19937_64& g) const { return canonical(g); }

// sampler.cpp:17-89; the draw's uniform comes from this sampler's generator, one per non-greedy call
int32_t Sampler::sample(const float* logits, int n_vocab) {
    ensure(n_vocab);
    const double u = p_.temperature > 0.0f ? canonical(rng_) : 0.0;
    int32_t t = 0;
    if (int st = kls_sample(h_, logits, n_vocab, u, &t)) fatal_status("kls_sample", st);
    return t;
}

// engine.cpp:563-575: row i uses the (i+1)-th draw; rows after a rejection are never sampled, so only
// accepted+1 draws are consumed.
int Sampler::verify(const float* logits, int n_vocab, int nb, const int32_t* drafts, int32_t* tokens) {
    ensure(n_vocab);
    double u[16] = {0};
    if (nb > 16) fatal_status("verify", KLS_ERR_RANGE);
    if (p_.temperature > 0.0f) {
        std::mt19937_64 peek = rng_;
        for (int i = 0; i < nb; ++i) u[i] = draw_peek(peek);
    }
    int32_t acc = 0;
    if (int st = kls_verify(h_, logits, nb, drafts, u, tokens, &acc, nullptr)) fatal_status("kls_verify", st);
    if (p_.temperature > 0.0f) rng_.discard((unsigned long long) acc + 1);
    return acc;
}

}  // namespace klein

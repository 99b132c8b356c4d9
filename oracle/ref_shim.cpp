// ORACLE — test infrastructure only (the CPU baseline of bench.py and the tests load it; the product never does).
//
// A C-ABI shim around the reference's own klein::Sampler (src/sampler.h:25-38), compiled together with the
// reference's src/sampler.cpp straight from /root/reference by oracle/Makefile into oracle/_ref/. The shim
// only forwards calls: construction with SamplerParams (sampler.h:13-22, sampler.cpp:11), reset (:13),
// accept (:15), sample (:17-89). It lets the tests check the restatement in sampler_oracle.cpp bit for bit and
// lets bench.py time the reference sampler itself on the host cores.
#include <chrono>
#include <cstdint>
#include <thread>
#include <vector>

#include "sampler.h"

extern "C" {

struct ref_params {  // same layout as orc_params, plus the seed
    float temperature;
    int32_t top_k;
    float top_p;
    float min_p;
    float presence_penalty;
    float frequency_penalty;
    float repetition_penalty;
    uint64_t seed;
};

void* ref_create(const ref_params* p) {
    klein::SamplerParams sp;
    sp.temperature = p->temperature;
    sp.top_k = p->top_k;
    sp.top_p = p->top_p;
    sp.min_p = p->min_p;
    sp.presence_penalty = p->presence_penalty;
    sp.frequency_penalty = p->frequency_penalty;
    sp.repetition_penalty = p->repetition_penalty;
    sp.seed = p->seed;
    return new klein::Sampler(sp);
}

void ref_destroy(void* s) { delete static_cast<klein::Sampler*>(s); }
void ref_reset(void* s) { static_cast<klein::Sampler*>(s)->reset(); }
void ref_accept(void* s, int32_t t) { static_cast<klein::Sampler*>(s)->accept(t); }
int32_t ref_sample(void* s, const float* logits, int n_vocab) {
    return static_cast<klein::Sampler*>(s)->sample(logits, n_vocab);
}

// The verify loop of Engine::generate (src/engine.cpp:563-575, without the caller-side stop conditions) driven
// through the reference Sampler: sample row i, accept it, continue while drafts[i] matches. Returns accepted.
int ref_verify(void* s, const float* logits, int n_vocab, int nb, const int32_t* drafts, int32_t* out_tokens) {
    auto* smp = static_cast<klein::Sampler*>(s);
    int accepted = 0;
    for (int i = 0; i < nb; ++i) {
        const int32_t t = smp->sample(logits + (size_t) i * n_vocab, n_vocab);
        smp->accept(t);
        out_tokens[i] = t;
        if (i + 1 < nb && drafts[i] == t) {
            accepted = i + 1;
            continue;
        }
        accepted = i;
        break;
    }
    for (int i = accepted + 1; i < nb; ++i) out_tokens[i] = -1;
    return accepted;
}

// Seconds for `reps` sample() calls cycling over n_rows rows, on the calling thread.
double ref_time_rows(void* s, const float* logits, int n_vocab, int n_rows, int reps, int32_t* sink) {
    auto* smp = static_cast<klein::Sampler*>(s);
    int32_t acc = 0;
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < reps; ++i) acc += smp->sample(logits + (size_t) (i % n_rows) * n_vocab, n_vocab);
    const auto t1 = std::chrono::steady_clock::now();
    if (sink) *sink = acc;
    return std::chrono::duration<double>(t1 - t0).count();
}

// Seconds for every one of n_rows rows to be sampled `reps` times with one Sampler per row, one std::thread per
// sampler, at most n_threads at a time (rows are dealt round-robin to the threads).
double ref_time_rows_threads(void* const* samplers, const float* logits, int n_vocab, int n_rows, int reps,
                             int n_threads) {
    if (n_threads < 1) n_threads = 1;
    const auto t0 = std::chrono::steady_clock::now();
    std::vector<std::thread> th;
    for (int t = 0; t < n_threads; ++t)
        th.emplace_back([=] {
            for (int rep = 0; rep < reps; ++rep)
                for (int r = t; r < n_rows; r += n_threads)
                    static_cast<klein::Sampler*>(samplers[r])->sample(logits + (size_t) r * n_vocab, n_vocab);
        });
    for (auto& x : th) x.join();
    const auto t1 = std::chrono::steady_clock::now();
    return std::chrono::duration<double>(t1 - t0).count();
}

}  // extern "C"

// Drives the C++ drop-in klein::Sampler (klein_amd/csrc/sampler.h, the interface of klein's src/sampler.h) through
// fixed scenarios on the GPU and records everything the reference needs to replay them: the parameters, every
// row of logits, the drafts, and the tokens the drop-in returned. tests/test_gpu_dropin.py replays each scenario
// with the reference's own Sampler (same seed, so the same mt19937_64 draws) and compares token for token.
//
// usage: dropin_check OUT_DIR    (writes OUT_DIR/scenario_<n>.bin and OUT_DIR/scenario_<n>.txt)
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <random>
#include <string>
#include <vector>

#include "sampler.h"

namespace {

struct Scenario {
    klein::SamplerParams p;
    int V;
    int samples;   // sample() + accept() steps
    int verifies;  // 4-row verify() steps
};

// Rows ~ N(0, 1.5) with 50 head tokens near 8, from a fixed generator (the values are written out, so the
// replay does not depend on how they were made).
void fill_row(std::mt19937_64& g, float* row, int V) {
    std::normal_distribution<float> n(0.0f, 1.5f);
    for (int i = 0; i < V; ++i) row[i] = n(g);
    std::uniform_int_distribution<int> pick(0, V - 1);
    std::normal_distribution<float> head(8.0f, 2.0f);
    for (int j = 0; j < 50 && j < V; ++j) row[pick(g)] = head(g);
}

int argmax(const float* row, int V) {
    int b = 0;
    for (int i = 1; i < V; ++i)
        if (row[i] > row[b]) b = i;
    return b;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s OUT_DIR\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    std::vector<Scenario> sc;
    {
        Scenario s{};
        s.p.temperature = 0.6f; s.p.top_k = 20; s.p.top_p = 0.95f; s.p.seed = 7;
        s.V = 248320; s.samples = 6; s.verifies = 4;
        sc.push_back(s);
    }
    {
        Scenario s{};
        s.p.temperature = 1.0f; s.p.top_k = 40; s.p.top_p = 0.95f; s.p.min_p = 0.05f;
        s.p.repetition_penalty = 1.1f; s.p.presence_penalty = 0.5f; s.p.frequency_penalty = 0.2f; s.p.seed = 11;
        s.V = 248320; s.samples = 6; s.verifies = 4;
        sc.push_back(s);
    }
    {
        Scenario s{};
        s.p.temperature = 0.0f; s.p.presence_penalty = 0.3f; s.p.seed = 3;
        s.V = 70001; s.samples = 4; s.verifies = 2;
        sc.push_back(s);
    }
    {
        Scenario s{};
        s.p.temperature = 0.9f; s.p.top_k = 0; s.p.top_p = 0.9f; s.p.repetition_penalty = 1.2f; s.p.seed = 5;
        s.V = 5000; s.samples = 4; s.verifies = 2;
        sc.push_back(s);
    }
    {
        Scenario s{};  // top-k 300: the mid path
        s.p.temperature = 0.8f; s.p.top_k = 300; s.p.top_p = 0.97f; s.p.min_p = 0.01f;
        s.p.repetition_penalty = 1.05f; s.p.presence_penalty = 0.2f; s.p.seed = 9;
        s.V = 248320; s.samples = 4; s.verifies = 3;
        sc.push_back(s);
    }
    std::mt19937_64 gen(20261201);
    for (size_t n = 0; n < sc.size(); ++n) {
        const Scenario& s = sc[n];
        klein::Sampler S(s.p);
        std::FILE* fb = std::fopen((dir + "/scenario_" + std::to_string(n) + ".bin").c_str(), "wb");
        std::FILE* ft = std::fopen((dir + "/scenario_" + std::to_string(n) + ".txt").c_str(), "w");
        if (!fb || !ft) return 3;
        std::fprintf(ft, "params %.9g %d %.9g %.9g %.9g %.9g %.9g %llu V %d\n", s.p.temperature, s.p.top_k,
                     s.p.top_p, s.p.min_p, s.p.presence_penalty, s.p.frequency_penalty, s.p.repetition_penalty,
                     (unsigned long long) s.p.seed, s.V);
        std::vector<float> rows((size_t) 4 * s.V);
        for (int t = 0; t < s.samples; ++t) {
            fill_row(gen, rows.data(), s.V);
            std::fwrite(rows.data(), sizeof(float), s.V, fb);
            const int32_t tok = S.sample(rows.data(), s.V);
            S.accept(tok);
            std::fprintf(ft, "sample %d\n", tok);
        }
        for (int t = 0; t < s.verifies; ++t) {
            int32_t drafts[3], toks[4];
            for (int r = 0; r < 4; ++r) fill_row(gen, rows.data() + (size_t) r * s.V, s.V);
            for (int r = 0; r < 3; ++r) drafts[r] = argmax(rows.data() + (size_t) r * s.V, s.V);  // often accepted
            std::fwrite(rows.data(), sizeof(float), (size_t) 4 * s.V, fb);
            const int acc = S.verify(rows.data(), s.V, 4, drafts, toks);
            std::fprintf(ft, "verify %d %d %d %d accepted %d", drafts[0], drafts[1], drafts[2], 0, acc);
            for (int i = 0; i <= acc; ++i) std::fprintf(ft, " %d", toks[i]);
            std::fprintf(ft, "\n");
        }
        std::fclose(fb);
        std::fclose(ft);
    }
    std::printf("dropin_check: %zu scenarios written to %s\n", sc.size(), dir.c_str());
    return 0;
}

// ORACLE — test infrastructure only. Nothing in the product links, loads or calls this file; only the tests,
// the smoke check and the CPU-baseline leg of bench.py do, and only as the checker.
//
// A CPU restatement of klein's token sampler (src/sampler.cpp:11-89) and of the MTP verify accept rule
// (src/engine.cpp:563-575), with the draw's uniform injected so that CPU and GPU see the same draws.
// Every function cites the reference lines it follows. The arithmetic is kept in the reference's order and
// precision: f32 penalties with separate roundings (built without -march, so no FMA contraction, as the
// reference's klein_core), std::exp(float) from the host libm, sequential double sums, and
// std::partial_sort over vector<pair<float,int32_t>> with the value-only comparator.
//
// Pinning (what checks each function; the tests under tests/ run these):
//   orc_sample (mode 0)  : bit-for-bit against the reference's own sampler.cpp compiled from its sources
//                          (oracle/_ref, when /root/reference exists) and the committed golden fixtures;
//                          closed forms (greedy == first argmax; top_k=1 == greedy; p sums to ~1; T->0 limit).
//   orc_sample (mode 1)  : equal to mode 0 whenever the top-(k+1) values are distinct; on planted ties, the
//                          lower id wins (closed form).
//   orc_verify           : closed form of engine.cpp:564-574 replayed with per-row orc_sample calls.
//   orc_uniforms         : C++ standard KAT (10000th output of mt19937_64 = 9981545732273789042) and the
//                          reference's own draws (oracle/_ref with the same seed).
//   orc_expf_glibc       : exhaustive comparison against the host libm expf over every float in [-110, 89].
//   orc_ppl_row          : closed forms in float64 (numpy logsumexp and the KL sum) to rounding, the first-maximum
//                          rule on planted ties, and the NaN / infinity cases (tests/test_oracle.py).
//   orc_argmax           : the library call itself (std::max_element, as engine.cpp:414); checked against the
//                          textbook loop on small rows and the closed form (first index of the largest value
//                          among numbers; a NaN first element wins) on planted ties, NaNs and infinities.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <random>
#include <thread>
#include <utility>
#include <vector>

extern "C" {

// Mirrors klein::SamplerParams (src/sampler.h:13-22), without the seed (the uniform is injected).
struct orc_params {
    float temperature;
    int32_t top_k;
    float top_p;
    float min_p;
    float presence_penalty;
    float frequency_penalty;
    float repetition_penalty;
};

}  // extern "C"

namespace {

using Cand = std::pair<float, int32_t>;

// The penalty lambda of src/sampler.cpp:18-29. `counts` is a dense per-id count array (the reference keeps an
// unordered_map<int32_t,int>; a lookup that finds nothing and a zero count are the same case here).
struct Logit {
    const float* logits;
    const int32_t* counts;
    const orc_params* p;
    bool penalize;
    float operator()(int32_t id) const {
        float l = logits[id];
        if (penalize && counts && counts[id] > 0) {
            if (p->repetition_penalty != 1.0f) l = l > 0 ? l / p->repetition_penalty : l * p->repetition_penalty;
            const float f = p->frequency_penalty * (float) counts[id];
            const float t = p->presence_penalty + f;
            l = l - t;
        }
        return l;
    }
};

// One Sampler::sample call (src/sampler.cpp:17-89) with the draw's uniform `u` given.
// mode 0: the reference's std::partial_sort with `a.first > b.first` (its tie order);
// mode 1: the total order (value descending, id ascending), i.e. on equal values the lower id wins.
int32_t sample_row(const float* logits, int n_vocab, const orc_params* p, const int32_t* counts, double u, int mode,
                   std::vector<Cand>& cand, int32_t* out_ids, float* out_probs, int cap, int* out_k, int* out_kept) {
    const bool penalize = p->presence_penalty != 0.0f || p->frequency_penalty != 0.0f || p->repetition_penalty != 1.0f;
    const Logit logit{logits, counts, p, penalize};
    if (out_k) *out_k = 0;
    if (out_kept) *out_kept = 0;

    if (p->temperature <= 0.0f) {  // greedy, src/sampler.cpp:31-39: strict '>' so the first (lowest) id wins ties
        int32_t best = 0;
        float bl = -INFINITY;
        for (int32_t i = 0; i < n_vocab; ++i) {
            const float l = logit(i);
            if (l > bl) {
                bl = l;
                best = i;
            }
        }
        return best;
    }

    // top-k over the penalized logits, src/sampler.cpp:42-51
    const int k = (p->top_k > 0 && p->top_k < n_vocab) ? p->top_k : n_vocab;
    cand.resize(n_vocab);
    for (int32_t i = 0; i < n_vocab; ++i) cand[i] = Cand(logit(i), i);
    if (mode == 0) {
        auto cmp = [](const Cand& a, const Cand& b) { return a.first > b.first; };
        if (k < n_vocab) {
            std::partial_sort(cand.begin(), cand.begin() + k, cand.end(), cmp);
            cand.resize(k);
        } else {
            std::sort(cand.begin(), cand.end(), cmp);
        }
    } else {
        auto cmp = [](const Cand& a, const Cand& b) { return a.first > b.first || (a.first == b.first && a.second < b.second); };
        std::partial_sort(cand.begin(), cand.begin() + k, cand.end(), cmp);
        cand.resize(k);
    }

    // softmax with temperature, src/sampler.cpp:53-60: f32 subtract and divide, libm expf, double running sum
    const float maxl = cand[0].first;
    double sum = 0.0;
    for (auto& c : cand) {
        const float x = (c.first - maxl) / p->temperature;
        c.first = std::exp(x);
        sum += c.first;
    }
    for (auto& c : cand) c.first = (float) (c.first / sum);
    if (out_k) *out_k = (int) cand.size();
    for (int i = 0; i < (int) cand.size() && i < cap; ++i) {
        if (out_ids) out_ids[i] = cand[i].second;
        if (out_probs) out_probs[i] = cand[i].first;
    }

    // min-p, src/sampler.cpp:62-68
    if (p->min_p > 0.0f) {
        const float thr = cand[0].first * p->min_p;
        size_t n = 1;
        while (n < cand.size() && cand[n].first >= thr) ++n;
        cand.resize(n);
    }
    // top-p, src/sampler.cpp:69-79 (cumulative double sum, no renormalisation)
    if (p->top_p < 1.0f) {
        double cum = 0.0;
        size_t n = 0;
        while (n < cand.size()) {
            cum += cand[n].first;
            ++n;
            if (cum >= p->top_p) break;
        }
        cand.resize(std::max<size_t>(n, 1));
    }
    if (out_kept) *out_kept = (int) cand.size();

    // draw, src/sampler.cpp:80-88: total in double, r = u*(total-0)+0 as libstdc++'s uniform_real_distribution
    double total = 0.0;
    for (auto& c : cand) total += c.first;
    double r = (u * (total - 0.0)) + 0.0;
    for (auto& c : cand) {
        r -= c.first;
        if (r <= 0.0) return c.second;
    }
    return cand.back().second;
}

}  // namespace

extern "C" {

// Sampler::sample for one row. `counts` (nullable) is a dense array of n_vocab per-id history counts.
// Optional outputs: the sorted top-k ids and their softmax probabilities (before min-p/top-p truncation), k,
// and the number of candidates kept for the draw.
int32_t orc_sample(const float* logits, int n_vocab, const orc_params* p, const int32_t* counts, double u, int mode,
                   int32_t* out_ids, float* out_probs, int cap, int* out_k, int* out_kept) {
    std::vector<Cand> cand;
    return sample_row(logits, n_vocab, p, counts, u, mode, cand, out_ids, out_probs, cap, out_k, out_kept);
}

// The verify/accept loop of Engine::generate (src/engine.cpp:563-575) without the caller-side stop conditions:
// row i is sampled with the history after accept(t_0..t_{i-1}) and draft batch[i+1] = drafts[i] is accepted
// while it equals t_i. `counts` is updated in place with every sampled token (accept(), engine.cpp:567).
// Returns `accepted`; out_tokens[0..accepted] are the emitted tokens.
int orc_verify(const float* logits, int n_vocab, int nb, const int32_t* drafts, const orc_params* p, int32_t* counts,
               const double* u, int mode, int32_t* out_tokens) {
    std::vector<Cand> cand;
    int accepted = 0;
    for (int i = 0; i < nb; ++i) {
        const int32_t t = sample_row(logits + (size_t) i * n_vocab, n_vocab, p, counts, u[i], mode, cand, nullptr,
                                     nullptr, 0, nullptr, nullptr);
        if (counts) counts[t]++;
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

// The uniforms the reference's draws consume: std::uniform_real_distribution<double> over mt19937_64(seed)
// (src/sampler.cpp:11,82-83) maps each engine output x to generate_canonical<double,53>: double(x) / 2^64,
// clamped below 1. `skip` outputs are discarded first. Uses the host std library directly.
void orc_uniforms(uint64_t seed, uint64_t skip, int n, double* out) {
    std::mt19937_64 rng(seed);
    rng.discard(skip);
    for (int i = 0; i < n; ++i) out[i] = std::generate_canonical<double, std::numeric_limits<double>::digits>(rng);
}

// n-th output (1-based) of mt19937_64 seeded with `seed` (default_seed = 5489 gives the standard's KAT).
uint64_t orc_mt64_nth(uint64_t seed, uint64_t n) {
    std::mt19937_64 rng(seed);
    if (n > 1) rng.discard(n - 1);
    return rng();
}

float orc_libm_expf(float x) { return std::exp(x); }

// --- expf restatement: the table-driven method of the ARM optimized-routines / glibc >= 2.27 expf
// (Szabolcs Nagy): x*32/ln2 = k + r, exp(x) = 2^(k/32) * 2^(r/32), 2^(r/32) by a cubic in r, all in double,
// rounded once to float. The table holds round-to-nearest 2^(i/32) with (i << 47) subtracted from the bits so
// that k can be added into the exponent field. This is the formulation the GPU uses, written in the
// fused-multiply-add form; tests compare it exhaustively with the host libm.
static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

float orc_expf_glibc(float x) {
    uint32_t ux;
    std::memcpy(&ux, &x, 4);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {  // |x| >= 88 or x is nan
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double) x;
    double kd = std::fma(inv_ln2_32, xd, shift);
    uint64_t ki;
    std::memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = std::fma(inv_ln2_32, xd, -kd);
    uint64_t t = kExp2Tab[ki % 32];
    t += ki << 47;
    double s;
    std::memcpy(&s, &t, 8);
    const double z = std::fma(c0, r, c1);
    const double r2 = r * r;
    double y = std::fma(c2, r, 1.0);
    y = std::fma(z, r2, y);
    y = y * s;
    return (float) y;
}

// Counts floats with bit patterns in [lo, hi] (inclusive, as uint32; NaNs skipped) whose restated expf differs
// in any bit from the host libm's. Runs on `nthreads` host threads.
long long orc_expf_check(uint32_t lo, uint32_t hi, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    std::atomic<long long> bad{0};
    std::vector<std::thread> th;
    const uint64_t span = (uint64_t) hi - lo + 1;
    for (int t = 0; t < nthreads; ++t) {
        th.emplace_back([&, t] {
            const uint64_t a = lo + span * t / nthreads, b = lo + span * (t + 1) / nthreads;
            long long local = 0;
            for (uint64_t u = a; u < b; ++u) {
                const uint32_t bits = (uint32_t) u;
                float x;
                std::memcpy(&x, &bits, 4);
                if (std::isnan(x)) continue;
                const float r0 = std::exp(x), r1 = orc_expf_glibc(x);
                uint32_t b0, b1;
                std::memcpy(&b0, &r0, 4);
                std::memcpy(&b1, &r1, 4);
                local += (b0 != b1);
            }
            bad += local;
        });
    }
    for (auto& x : th) x.join();
    return bad.load();
}

// Compares `n` device-computed expf results for the consecutive float bit patterns starting at `lo` with the host
// libm. Returns the number of bitwise mismatches and the first mismatching input (bits) through `first_bad`.
long long orc_expf_compare(uint32_t lo, const float* gpu, long long n, int nthreads, uint32_t* first_bad) {
    if (nthreads < 1) nthreads = 1;
    std::vector<long long> bad(nthreads, 0);
    std::vector<uint64_t> first(nthreads, UINT64_MAX);
    std::vector<std::thread> th;
    for (int t = 0; t < nthreads; ++t) {
        th.emplace_back([&, t] {
            const long long a = n * t / nthreads, b = n * (t + 1) / nthreads;
            for (long long i = a; i < b; ++i) {
                const uint32_t bits = lo + (uint32_t) i;
                float x;
                std::memcpy(&x, &bits, 4);
                if (std::isnan(x)) continue;
                const float r0 = std::exp(x);
                uint32_t b0, b1;
                std::memcpy(&b0, &r0, 4);
                std::memcpy(&b1, &gpu[i], 4);
                if (b0 != b1) {
                    bad[t]++;
                    if (first[t] == UINT64_MAX) first[t] = bits;
                }
            }
        });
    }
    for (auto& x : th) x.join();
    long long total = 0;
    uint64_t f = UINT64_MAX;
    for (int t = 0; t < nthreads; ++t) {
        total += bad[t];
        f = std::min(f, first[t]);
    }
    if (first_bad) *first_bad = (uint32_t) (f == UINT64_MAX ? 0 : f);
    return total;
}

// The per-token scoring of cmd_ppl (src/main.cpp:308-327) for one row of logits with target `target`:
// out[0] = lse, out[1] = nll, and with a base row of log-probabilities (nullable) out[2] = kl, out[3] = base
// nll; tops[0] = imax, tops[1] = ibase. Same operations, types and order as the reference loop.
void orc_ppl_row(const float* l, int n_vocab, int target, const float* blp, double* out, int32_t* tops) {
    float mx = l[0];  // main.cpp:308-311
    int imax = 0;
    for (int v = 1; v < n_vocab; ++v)
        if (l[v] > mx) {
            mx = l[v];
            imax = v;
        }
    double sum = 0.0;  // :312-313
    for (int v = 0; v < n_vocab; ++v) sum += std::exp((double) l[v] - mx);
    const double lse = mx + std::log(sum);  // :314
    out[0] = lse;
    out[1] = lse - l[target];  // :315
    tops[0] = imax;
    if (blp) {
        out[3] = -blp[target];  // :319
        double kl = 0.0;        // :320-325
        int ibase = 0;
        for (int v = 0; v < n_vocab; ++v) {
            if (blp[v] > blp[ibase]) ibase = v;
            if (blp[v] > -16.0f) kl += std::exp((double) blp[v]) * (blp[v] - (l[v] - lse));
        }
        out[2] = kl;
        tops[1] = ibase;
    }
}

// Engine::mtp_draft_token (src/engine.cpp:413-415): the index std::max_element returns over one row.
int32_t orc_argmax(const float* logits, int n) { return (int32_t) (std::max_element(logits, logits + n) - logits); }

// Times `reps` Sampler::sample calls on `n_rows` rows of logits (row r at logits + r*n_vocab), cycling through the
// rows, on one host thread; returns total seconds. Used for the CPU baseline when the reference build is absent.
double orc_time_rows(const float* logits, int n_vocab, int n_rows, const orc_params* p, const int32_t* counts,
                     int reps, int32_t* sink) {
    std::vector<Cand> cand;
    cand.reserve(n_vocab);
    const auto t0 = std::chrono::steady_clock::now();
    int32_t acc = 0;
    for (int i = 0; i < reps; ++i)
        acc += sample_row(logits + (size_t) (i % n_rows) * n_vocab, n_vocab, p, counts, 0.5, 0, cand, nullptr, nullptr,
                          0, nullptr, nullptr);
    const auto t1 = std::chrono::steady_clock::now();
    if (sink) *sink = acc;
    return std::chrono::duration<double>(t1 - t0).count();
}

}  // extern "C"

// Per-token scores of klein's perplexity / KL-divergence loop (src/main.cpp:308-327) on gfx950.
//
// For each row of logits l (one token position) and its target t the reference computes, in double:
//   mx   = l[0], raised by every later l[v] > mx (the first largest; imax its index)
//   lse  = mx + log(sum_v exp((double) l[v] - mx))                     nll = lse - l[t]
// and, against a row of base log-probabilities b:
//   kl   = sum_{v: b[v] > -16} exp((double) b[v]) * (b[v] - (l[v] - lse))
//   ibase = the first largest b (same rule), nll_base = -b[t].
// The kernel reads every logit (and base entry) once: a workgroup of 256 threads per (row, segment) keeps a
// running maximum with a rescaled double sum (the sum relative to the maximum so far), the first-maximum keys,
// and the KL sums split as kl = A + lse * B with A = sum e^b (b - l) and B = sum e^b (both free of lse), so one
// pass suffices; the row's last workgroup (ticket) combines the segments. The sums run in a different order
// than the reference's sequential loop, so results agree to rounding (about 1e-15 relative for lse), not bit for
// bit. NaN and infinities follow the reference: any NaN logit, or an infinite maximum, makes lse NaN (a term
// exp(NaN) or exp(inf - inf) enters its sum); -inf logits add exp(-inf) = 0.
#include <type_traits>

#include "kls_internal.h"

namespace kls {
namespace {

constexpr int PPL_WG = 256;
constexpr int PPL_NW = PPL_WG / 64;

// value descending, id ascending; NaN maps to 0 (no candidate), -0 is folded onto +0 (they compare equal)
__device__ __forceinline__ uint64_t num_key(float v, int id) {
    if (v != v) return 0ull;
    uint32_t u = __float_as_uint(v);
    if (v == 0.0f) u = 0u;
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t) o << 32) | (uint64_t) (~(uint32_t) id);
}

__device__ __forceinline__ int key_index(uint64_t k) { return (int) ~(uint32_t) k; }

__device__ __forceinline__ float key_value(uint64_t k) {
    const uint32_t o = (uint32_t) (k >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

// exp in double for the sums, by Tang's table-driven method (ACM TOMS 15(2), 1989): k = nearest integer to
// x*256/ln2 (the fused add of 1.5*2^52 rounds the product to an integer in the low word), r = x - k*ln2/256 (a
// 33-bit leading part of ln2/256, so k times it is exact for every |k| < 2^20, plus the remainder), and
// exp(x) = 2^(k>>8) * 2^((k&255)/256) * exp(r), with 2^(j/256) from a table of the correctly rounded values and
// exp(r) - 1 by its Taylor polynomial to r^4 (|r| <= ln2/512, so the next term is below 4e-17). Within 1.25 ulp
// (1.09 at worst over 2,500 points, against 0.97 for a 64-entry table with the polynomial to r^6).
// x is clamped to [-800, 710] (results 0 and inf there, as exp's); the callers never pass NaN.
__device__ const double kExp256Tab[256] = {
    0x1.0000000000000p+0, 0x1.00b1afa5abcbfp+0, 0x1.0163da9fb3335p+0, 0x1.02168143b0281p+0,
    0x1.02c9a3e778061p+0, 0x1.037d42e11bbccp+0, 0x1.04315e86e7f85p+0, 0x1.04e5f72f654b1p+0,
    0x1.059b0d3158574p+0, 0x1.0650a0e3c1f89p+0, 0x1.0706b29ddf6dep+0, 0x1.07bd42b72a836p+0,
    0x1.0874518759bc8p+0, 0x1.092bdf66607e0p+0, 0x1.09e3ecac6f383p+0, 0x1.0a9c79b1f3919p+0,
    0x1.0b5586cf9890fp+0, 0x1.0c0f145e46c85p+0, 0x1.0cc922b7247f7p+0, 0x1.0d83b23395decp+0,
    0x1.0e3ec32d3d1a2p+0, 0x1.0efa55fdfa9c5p+0, 0x1.0fb66affed31bp+0, 0x1.1073028d7233ep+0,
    0x1.11301d0125b51p+0, 0x1.11edbab5e2ab6p+0, 0x1.12abdc06c31ccp+0, 0x1.136a814f204abp+0,
    0x1.1429aaea92de0p+0, 0x1.14e95934f312ep+0, 0x1.15a98c8a58e51p+0, 0x1.166a45471c3c2p+0,
    0x1.172b83c7d517bp+0, 0x1.17ed48695bbc0p+0, 0x1.18af9388c8deap+0, 0x1.1972658375d2fp+0,
    0x1.1a35beb6fcb75p+0, 0x1.1af99f8138a1cp+0, 0x1.1bbe084045cd4p+0, 0x1.1c82f95281c6bp+0,
    0x1.1d4873168b9aap+0, 0x1.1e0e75eb44027p+0, 0x1.1ed5022fcd91dp+0, 0x1.1f9c18438ce4dp+0,
    0x1.2063b88628cd6p+0, 0x1.212be3578a819p+0, 0x1.21f49917ddc96p+0, 0x1.22bdda27912d1p+0,
    0x1.2387a6e756238p+0, 0x1.2451ffb82140ap+0, 0x1.251ce4fb2a63fp+0, 0x1.25e85711ece75p+0,
    0x1.26b4565e27cddp+0, 0x1.2780e341ddf29p+0, 0x1.284dfe1f56381p+0, 0x1.291ba7591bb70p+0,
    0x1.29e9df51fdee1p+0, 0x1.2ab8a66d10f13p+0, 0x1.2b87fd0dad990p+0, 0x1.2c57e39771b2fp+0,
    0x1.2d285a6e4030bp+0, 0x1.2df961f641589p+0, 0x1.2ecafa93e2f56p+0, 0x1.2f9d24abd886bp+0,
    0x1.306fe0a31b715p+0, 0x1.31432edeeb2fdp+0, 0x1.32170fc4cd831p+0, 0x1.32eb83ba8ea32p+0,
    0x1.33c08b26416ffp+0, 0x1.3496266e3fa2dp+0, 0x1.356c55f929ff1p+0, 0x1.36431a2de883bp+0,
    0x1.371a7373aa9cbp+0, 0x1.37f26231e754ap+0, 0x1.38cae6d05d866p+0, 0x1.39a401b7140efp+0,
    0x1.3a7db34e59ff7p+0, 0x1.3b57fbfec6cf4p+0, 0x1.3c32dc313a8e5p+0, 0x1.3d0e544ede173p+0,
    0x1.3dea64c123422p+0, 0x1.3ec70df1c5175p+0, 0x1.3fa4504ac801cp+0, 0x1.40822c367a024p+0,
    0x1.4160a21f72e2ap+0, 0x1.423fb2709468ap+0, 0x1.431f5d950a897p+0, 0x1.43ffa3f84b9d4p+0,
    0x1.44e086061892dp+0, 0x1.45c2042a7d232p+0, 0x1.46a41ed1d0057p+0, 0x1.4786d668b3237p+0,
    0x1.486a2b5c13cd0p+0, 0x1.494e1e192aed2p+0, 0x1.4a32af0d7d3dep+0, 0x1.4b17dea6db7d7p+0,
    0x1.4bfdad5362a27p+0, 0x1.4ce41b817c114p+0, 0x1.4dcb299fddd0dp+0, 0x1.4eb2d81d8abffp+0,
    0x1.4f9b2769d2ca7p+0, 0x1.508417f4531eep+0, 0x1.516daa2cf6642p+0, 0x1.5257de83f4eefp+0,
    0x1.5342b569d4f82p+0, 0x1.542e2f4f6ad27p+0, 0x1.551a4ca5d920fp+0, 0x1.56070dde910d2p+0,
    0x1.56f4736b527dap+0, 0x1.57e27dbe2c4cfp+0, 0x1.58d12d497c7fdp+0, 0x1.59c0827ff07ccp+0,
    0x1.5ab07dd485429p+0, 0x1.5ba11fba87a03p+0, 0x1.5c9268a5946b7p+0, 0x1.5d84590998b93p+0,
    0x1.5e76f15ad2148p+0, 0x1.5f6a320dceb71p+0, 0x1.605e1b976dc09p+0, 0x1.6152ae6cdf6f4p+0,
    0x1.6247eb03a5585p+0, 0x1.633dd1d1929fdp+0, 0x1.6434634ccc320p+0, 0x1.652b9febc8fb7p+0,
    0x1.6623882552225p+0, 0x1.671c1c70833f6p+0, 0x1.68155d44ca973p+0, 0x1.690f4b19e9538p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6b052fa75173ep+0, 0x1.6c012750bdabfp+0, 0x1.6cfdcddd47645p+0,
    0x1.6dfb23c651a2fp+0, 0x1.6ef9298593ae5p+0, 0x1.6ff7df9519484p+0, 0x1.70f7466f42e87p+0,
    0x1.71f75e8ec5f74p+0, 0x1.72f8286ead08ap+0, 0x1.73f9a48a58174p+0, 0x1.74fbd35d7cbfdp+0,
    0x1.75feb564267c9p+0, 0x1.77024b1ab6e09p+0, 0x1.780694fde5d3fp+0, 0x1.790b938ac1cf6p+0,
    0x1.7a11473eb0187p+0, 0x1.7b17b0976cfdbp+0, 0x1.7c1ed0130c132p+0, 0x1.7d26a62ff86f0p+0,
    0x1.7e2f336cf4e62p+0, 0x1.7f3878491c491p+0, 0x1.80427543e1a12p+0, 0x1.814d2add106d9p+0,
    0x1.82589994cce13p+0, 0x1.8364c1eb941f7p+0, 0x1.8471a4623c7adp+0, 0x1.857f4179f5b21p+0,
    0x1.868d99b4492edp+0, 0x1.879cad931a436p+0, 0x1.88ac7d98a6699p+0, 0x1.89bd0a478580fp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8be05bad61778p+0, 0x1.8cf3216b5448cp+0, 0x1.8e06a5e0866d9p+0,
    0x1.8f1ae99157736p+0, 0x1.902fed0282c8ap+0, 0x1.9145b0b91ffc6p+0, 0x1.925c353aa2fe2p+0,
    0x1.93737b0cdc5e5p+0, 0x1.948b82b5f98e5p+0, 0x1.95a44cbc8520fp+0, 0x1.96bdd9a7670b3p+0,
    0x1.97d829fde4e50p+0, 0x1.98f33e47a22a2p+0, 0x1.9a0f170ca07bap+0, 0x1.9b2bb4d53fe0dp+0,
    0x1.9c49182a3f090p+0, 0x1.9d674194bb8d5p+0, 0x1.9e86319e32323p+0, 0x1.9fa5e8d07f29ep+0,
    0x1.a0c667b5de565p+0, 0x1.a1e7aed8eb8bbp+0, 0x1.a309bec4a2d33p+0, 0x1.a42c980460ad8p+0,
    0x1.a5503b23e255dp+0, 0x1.a674a8af46052p+0, 0x1.a799e1330b358p+0, 0x1.a8bfe53c12e59p+0,
    0x1.a9e6b5579fdbfp+0, 0x1.ab0e521356ebap+0, 0x1.ac36bbfd3f37ap+0, 0x1.ad5ff3a3c2774p+0,
    0x1.ae89f995ad3adp+0, 0x1.afb4ce622f2ffp+0, 0x1.b0e07298db666p+0, 0x1.b20ce6c9a8952p+0,
    0x1.b33a2b84f15fbp+0, 0x1.b468415b749b1p+0, 0x1.b59728de5593ap+0, 0x1.b6c6e29f1c52ap+0,
    0x1.b7f76f2fb5e47p+0, 0x1.b928cf22749e4p+0, 0x1.ba5b030a1064ap+0, 0x1.bb8e0b79a6f1fp+0,
    0x1.bcc1e904bc1d2p+0, 0x1.bdf69c3f3a207p+0, 0x1.bf2c25bd71e09p+0, 0x1.c06286141b33dp+0,
    0x1.c199bdd85529cp+0, 0x1.c2d1cd9fa652cp+0, 0x1.c40ab5fffd07ap+0, 0x1.c544778fafb22p+0,
    0x1.c67f12e57d14bp+0, 0x1.c7ba88988c933p+0, 0x1.c8f6d9406e7b5p+0, 0x1.ca3405751c4dbp+0,
    0x1.cb720dcef9069p+0, 0x1.ccb0f2e6d1675p+0, 0x1.cdf0b555dc3fap+0, 0x1.cf3155b5bab74p+0,
    0x1.d072d4a07897cp+0, 0x1.d1b532b08c968p+0, 0x1.d2f87080d89f2p+0, 0x1.d43c8eacaa1d6p+0,
    0x1.d5818dcfba487p+0, 0x1.d6c76e862e6d3p+0, 0x1.d80e316c98398p+0, 0x1.d955d71ff6075p+0,
    0x1.da9e603db3285p+0, 0x1.dbe7cd63a8315p+0, 0x1.dd321f301b460p+0, 0x1.de7d5641c0658p+0,
    0x1.dfc97337b9b5fp+0, 0x1.e11676b197d17p+0, 0x1.e264614f5a129p+0, 0x1.e3b333b16ee12p+0,
    0x1.e502ee78b3ff6p+0, 0x1.e653924676d76p+0, 0x1.e7a51fbc74c83p+0, 0x1.e8f7977cdb740p+0,
    0x1.ea4afa2a490dap+0, 0x1.eb9f4867cca6ep+0, 0x1.ecf482d8e67f1p+0, 0x1.ee4aaa2188510p+0,
    0x1.efa1bee615a27p+0, 0x1.f0f9c1cb6412ap+0, 0x1.f252b376bba97p+0, 0x1.f3ac948dd7274p+0,
    0x1.f50765b6e4540p+0, 0x1.f6632798844f8p+0, 0x1.f7bfdad9cbe14p+0, 0x1.f91d802243c89p+0,
    0x1.fa7c1819e90d8p+0, 0x1.fbdba3692d514p+0, 0x1.fd3c22b8f71f1p+0, 0x1.fe9d96b2a23d9p+0};

// (LO / HI: whether the argument can lie below -800 / above 710; callers whose argument cannot skip that clamp)
template <bool LO = true, bool HI = true>
__device__ __forceinline__ double exp_tab(double x, const double* tab) {
    if (LO) x = fmax(x, -800.0);
    if (HI) x = fmin(x, 710.0);
    constexpr double kShift = 0x1.8p52;
    const double t1 = fma(x, 0x1.71547652b82fep+8, kShift);
    const int k = (int) (uint32_t) __double_as_longlong(t1);  // (two's complement in the low word)
    const double kd = t1 - kShift;
    const double r = fma(-kd, 0x1.473de6af278edp-42, fma(-kd, 0x1.62e42fef00000p-9, x));
    const double q = fma(r, fma(r, 1.0 / 24, 1.0 / 6), 0.5);
    const double p = fma(r * r, q, r);
    const double t = tab[k & 255];
    return ldexp(fma(t, p, t), k >> 8);
}

// A running maximum m of the finite logits seen and s = sum over them of exp(x - m).
struct RunSum {
    float m = -INFINITY;
    double s = 0.0;
    __device__ __forceinline__ void add(float x, const double* tab) {
        if (!(x - x == 0.0f)) return;  // NaN and infinities are accounted for by the flags
        if (x > m) {
            s = s * exp_tab((double) m - (double) x, tab);  // (0 while m is -inf: the clamp gives exp(-800))
            m = x;
        }
        s += exp_tab((double) x - (double) m, tab);
    }
    __device__ __forceinline__ void merge(float m2, double s2) {
        const float mm = fmaxf(m, m2);
        if (mm == -INFINITY) return;
        s = (m == -INFINITY ? 0.0 : s * exp((double) m - (double) mm)) +
            (m2 == -INFINITY ? 0.0 : s2 * exp((double) m2 - (double) mm));
        m = mm;
    }
};

template <typename T>
__device__ __forceinline__ T shfl_x(T v, int mask) {
    return __shfl_xor(v, mask, 64);
}

__device__ __forceinline__ uint64_t shfl_x64(uint64_t v, int mask) {
    const uint32_t lo = (uint32_t) __shfl_xor((int) (uint32_t) v, mask, 64);
    const uint32_t hi = (uint32_t) __shfl_xor((int) (uint32_t) (v >> 32), mask, 64);
    return ((uint64_t) hi << 32) | lo;
}

struct Partial {
    uint64_t key = 0ull, bkey = 0ull;
    uint32_t nan = 0u;
    RunSum r;
    double a = 0.0, b = 0.0;
    __device__ __forceinline__ void merge(const Partial& o) {
        key = key > o.key ? key : o.key;
        bkey = bkey > o.bkey ? bkey : o.bkey;
        nan |= o.nan;
        r.merge(o.r.m, o.r.s);
        a += o.a;
        b += o.b;
    }
    __device__ __forceinline__ Partial xor_lane(int mask) const {
        Partial o;
        o.key = shfl_x64(key, mask);
        o.bkey = shfl_x64(bkey, mask);
        o.nan = (uint32_t) __shfl_xor((int) nan, mask, 64);
        o.r.m = shfl_x(r.m, mask);
        o.r.s = shfl_x(r.s, mask);
        o.a = shfl_x(a, mask);
        o.b = shfl_x(b, mask);
        return o;
    }
};

__device__ __forceinline__ Partial wave_reduce(Partial p) {
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) p.merge(p.xor_lane(mask));
    return p;  // (every lane holds the wave's result; the order of merges is fixed)
}

// A segment's record in the row's scratch: 8 words.
__device__ __forceinline__ void put_rec(uint64_t* r, const Partial& p) {
    const uint64_t w[8] = {p.key, p.bkey, p.nan, (uint64_t) __float_as_uint(p.r.m),
                           (uint64_t) __double_as_longlong(p.r.s), (uint64_t) __double_as_longlong(p.a),
                           (uint64_t) __double_as_longlong(p.b), 0ull};
#pragma unroll
    for (int i = 0; i < 8; ++i) __hip_atomic_store(&r[i], w[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ Partial get_rec(const uint64_t* r) {
    uint64_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = __hip_atomic_load(&r[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    Partial p;
    p.key = w[0];
    p.bkey = w[1];
    p.nan = (uint32_t) w[2];
    p.r.m = __uint_as_float((uint32_t) w[3]);
    p.r.s = __longlong_as_double((long long) w[4]);
    p.a = __longlong_as_double((long long) w[5]);
    p.b = __longlong_as_double((long long) w[6]);
    return p;
}

__shared__ uint64_t s_ppl[PPL_NW][8];
__shared__ double s_exp256[256];
__shared__ int s_ppl_last;

__global__ __launch_bounds__(PPL_WG) void ppl_kernel(PplArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row = blockIdx.x / a.segs, seg = blockIdx.x - row * a.segs;
    const int lo = seg * a.seg_len, hi = min(a.V, lo + a.seg_len);
    const float* __restrict__ L = a.logits + (int64_t) row * a.row_stride;
    const float* __restrict__ B = a.base ? a.base + (int64_t) row * a.base_stride : nullptr;
    static_assert(PPL_WG == 256, "one table entry per thread");
    s_exp256[tid] = kExp256Tab[tid];
    __syncthreads();
    Partial p;
    // Thread t holds ids s0 + e (e < 4) of each step, s0 = lo + 4*(t + j*WG): float4 loads when the rows are
    // 16-byte aligned. Per thread the ids ascend, so the first maximum is kept with a strict '>'. The running
    // maximum moves once per step (its rescaling exp is not per logit), and excluded or non-finite terms enter
    // as exp of the clamp, 0.
    const bool vec = ((reinterpret_cast<uintptr_t>(L) | (B ? reinterpret_cast<uintptr_t>(B) : 0)) & 15u) == 0;
    float bx = -INFINITY, bb = -INFINITY;  // first maxima (logits, base) and their ids (INT_MAX: none yet)
    int ix = 0x7fffffff, ib = 0x7fffffff;
    // one float4 of each row per thread and step
    auto load = [&](int i0, float (&xv)[4], float (&bv)[4]) {
        if (vec && i0 + 3 < hi) {
            const float4 q = *reinterpret_cast<const float4*>(L + i0);
            xv[0] = q.x, xv[1] = q.y, xv[2] = q.z, xv[3] = q.w;
            if (B) {
                const float4 r = *reinterpret_cast<const float4*>(B + i0);
                bv[0] = r.x, bv[1] = r.y, bv[2] = r.z, bv[3] = r.w;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool in = i0 + e < hi;
                xv[e] = in ? L[i0 + e] : -INFINITY;
                if (B) bv[e] = in ? B[i0 + e] : -INFINITY;
            }
        }
    };
    // The work of one step: ids s0 + e of the logits xv and base entries bv; FULL: every id is in the segment.
    // First maxima move by selects (strict '>' over ascending ids, or the first id while none is held).
    auto step = [&](auto full, int s0, const float (&xv)[4], const float (&bv)[4]) {
        constexpr bool FULL = decltype(full)::value;
        float cm = p.r.m;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool in = FULL || s0 + e < hi;
            const float x = xv[e];
            const bool up = in && (x > bx || (ix == 0x7fffffff && x == bx));
            bx = up ? x : bx;
            ix = up ? s0 + e : ix;
            p.nan |= (in && x != x) ? 1u : 0u;
            if (x - x == 0.0f) cm = fmaxf(cm, x);  // (out-of-segment slots are -inf)
        }
        if (cm > p.r.m) {
            p.r.s = p.r.s * exp_tab<true, false>((double) p.r.m - (double) cm, s_exp256);  // (<= 0, or -inf)
            p.r.m = cm;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float x = xv[e];
            p.r.s += exp_tab<true, false>(x - x == 0.0f ? (double) x - (double) p.r.m : -800.0, s_exp256);  // (<= 0)
        }
        if (B) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool in = FULL || s0 + e < hi;
                const float b = bv[e], x = xv[e];
                const bool up = in && (b > bb || (ib == 0x7fffffff && b == bb));
                bb = up ? b : bb;
                ib = up ? s0 + e : ib;
                const bool term = in && b > -16.0f;
                const double eb = exp_tab<false, true>(term ? (double) b : -800.0, s_exp256);  // (above -16, or -800)
                p.a += term ? eb * ((double) b - (double) x) : 0.0;
                p.b += eb;
            }
        }
    };
    // Steps of PPL_WG float4s wholly inside the segment (16-byte aligned rows): float4 loads, the next step's
    // issued before this step's work; then the rest of the segment (or all of it) with per-id checks.
    constexpr int STEP = 4 * PPL_WG;
    const int nfull = vec ? (hi - lo) / STEP : 0;
    float xn[4], bn[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    if (nfull > 0) load(lo + 4 * tid, xn, bn);
    for (int j = 0; j < nfull; ++j) {
        float xv[4], bv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = xn[e], bv[e] = bn[e];
        if (j + 1 < nfull) load(lo + (j + 1) * STEP + 4 * tid, xn, bn);
        step(std::true_type{}, lo + j * STEP + 4 * tid, xv, bv);
    }
    for (int s0 = lo + nfull * STEP + 4 * tid; s0 - 4 * tid < hi; s0 += STEP) {
        float xv[4], bv[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        load(s0, xv, bv);
        step(std::false_type{}, s0, xv, bv);
    }
    p.key = ix == 0x7fffffff ? 0ull : num_key(bx, ix);
    p.bkey = ib == 0x7fffffff ? 0ull : num_key(bb, ib);
    p = wave_reduce(p);
    if (lane == 0) {
        uint64_t* r = &s_ppl[wave][0];
        r[0] = p.key;
        r[1] = p.bkey;
        r[2] = p.nan;
        r[3] = __float_as_uint(p.r.m);
        r[4] = (uint64_t) __double_as_longlong(p.r.s);
        r[5] = (uint64_t) __double_as_longlong(p.a);
        r[6] = (uint64_t) __double_as_longlong(p.b);
    }
    __syncthreads();
    uint64_t* rec = a.scratch + ((int64_t) row * a.segs + seg) * KCAP;
    if (tid == 0) {
        Partial q;
        for (int w = 0; w < PPL_NW; ++w) {
            Partial o;
            o.key = s_ppl[w][0];
            o.bkey = s_ppl[w][1];
            o.nan = (uint32_t) s_ppl[w][2];
            o.r.m = __uint_as_float((uint32_t) s_ppl[w][3]);
            o.r.s = __longlong_as_double((long long) s_ppl[w][4]);
            o.a = __longlong_as_double((long long) s_ppl[w][5]);
            o.b = __longlong_as_double((long long) s_ppl[w][6]);
            q.merge(o);
        }
        put_rec(rec, q);
        // the record is acknowledged before the ticket: the last workgroup reads it after its own increment
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        const uint32_t prev = atomicAdd(&a.ticket[row], 1u);
        s_ppl_last = prev == (uint32_t) (a.segs - 1);
    }
    __syncthreads();
    if (!s_ppl_last || wave != 0) return;
    // the row's last workgroup: wave 0 combines the segment records (lane s holds segment s, in a fixed order)
    const uint64_t* recs = a.scratch + (int64_t) row * a.segs * KCAP;
    Partial q;
    for (int s0 = 0; s0 < a.segs; s0 += 64) {
        Partial o;
        if (s0 + lane < a.segs) o = get_rec(recs + (int64_t) (s0 + lane) * KCAP);
        q.merge(wave_reduce(o));
    }
    if (lane != 0) return;
    const float l0 = L[0];
    const bool nan0 = l0 != l0;
    const float mx = key_value(q.key);
    double lse;
    if (q.nan || q.key == 0ull || !(mx - mx == 0.0f))
        lse = __longlong_as_double(0x7ff8000000000000ll);  // a NaN or an infinite maximum: the reference's NaN
    else
        lse = (double) mx + log(q.r.s * exp((double) q.r.m - (double) mx));
    const int t = a.targets ? a.targets[row] : -1;
    const bool tin = t >= 0 && t < a.V;
    if (a.out_lse) a.out_lse[row] = lse;
    if (a.out_nll) a.out_nll[row] = tin ? lse - (double) L[t] : __longlong_as_double(0x7ff8000000000000ll);
    if (a.out_top) a.out_top[row] = (nan0 || q.key == 0ull) ? 0 : key_index(q.key);
    if (B) {
        const float b0 = B[0];
        if (a.out_kl) a.out_kl[row] = q.b == 0.0 ? 0.0 : q.a + lse * q.b;  // (no term: the reference's 0)
        if (a.out_base_top) a.out_base_top[row] = (b0 != b0 || q.bkey == 0ull) ? 0 : key_index(q.bkey);
        if (a.out_nll_base) a.out_nll_base[row] = tin ? -(double) B[t] : __longlong_as_double(0x7ff8000000000000ll);
    }
    a.ticket[row] = 0u;  // (for the next launch)
}

}  // namespace

int ppl_segments(int V, int rows, int* seg_len) {
    // 256-thread workgroups over 2048..16384 ids: the longest whose grid still gives every CU a few
    int sl = 16384;
    while (sl > 2048 && (long long) rows * ((V + sl - 1) / sl) < 1024) sl >>= 1;
    *seg_len = sl;
    return (V + sl - 1) / sl;
}

hipError_t launch_ppl(const PplArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(ppl_kernel, dim3(a.n_rows * a.segs), dim3(PPL_WG), 0, s, a);
    return hipGetLastError();
}

}  // namespace kls

// HIP kernels of the gfx950 token sampler.
//
// One fused kernel samples a batch of rows (klein src/sampler.cpp:17-89 per row, plus the verify accept rule of
// src/engine.cpp:563-575 across rows). The grid is a list of (row, segment) work items; a workgroup of NW waves
// (NW = 4 for short segments, 16 for long ones) holds one segment of one row (NW*64 threads x EPT logits) in
// registers after a single coalesced HBM read:
//   * penalties (sampler.cpp:18-29) are applied in-register by the one lane holding each id, from a count table
//     of the segment's history ids staged in LDS; nothing is written to the logits or any global buffer;
//   * greedy (sampler.cpp:31-39) keeps a per-lane (max, first id) and reduces across lanes and segments;
//   * top-k (sampler.cpp:42-51): lanes contribute their largest logits (all 256 lanes of a 4-wave workgroup, the
//     512 lanes of waves 0..7 of a 16-wave one); the k-th largest of those distinct logits is a lower bound of
//     the segment's k-th largest value, and with the best bound
//     other workgroups of the row have published, one float compare per logit rejects nearly everything. The
//     few survivors are ordered by a 64-bit key (value descending, id ascending) with wave64 bitonic networks
//     built from DPP and permlane swaps;
//   * the last workgroup of a row (ticket counter) merges the segment candidate lists into the row's sorted
//     top-k and runs the O(k) tail on one wave: softmax with temperature (expf bit-identical to the host
//     glibc's, double sums), min-p, top-p and the draw (sampler.cpp:53-88);
//   * in a verify step each row publishes its token (device memory and pinned host memory) and the workgroup
//     that completes the step's last row forms the accepted prefix (a 64-bit step counter carries every row's
//     draft mismatch bit), so `accepted` is in device memory for the consumers that follow on the stream.
// Ticket counters and published bounds are reset by their last user, so launches replay from a captured graph
// without memset nodes.
#include "kls_internal.h"

namespace kls {
namespace {

constexpr int CW = 128;  // candidate slots per wave in LDS

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Buffer resource word 3 for raw (stride 0) 32-bit data on gfx9-family parts, and the non-temporal load policy.
constexpr int kRawBufferFlags = 0x00020000;
constexpr int kNonTemporal = 2;

// Workgroup memory of the sampling kernel, one set per workgroup width, addressed directly (no generic
// pointers into LDS).
extern __shared__ __align__(16) uint32_t s_cnt[];    // with penalties: the segment's history counts
template <int NW> __shared__ uint64_t s_cand[NW][CW];  // per-wave candidate regions
template <int NW> __shared__ uint64_t s_list[NW][64];  // per-wave sorted lists
template <int NW> __shared__ uint64_t s_red[NW];
template <int NW> __shared__ uint32_t s_q[NW];
template <int NW> __shared__ int s_n[NW];
template <int NW> __shared__ uint32_t s_mx[NW][64];    // per-wave sorted lane maxima
template <int NW> __shared__ uint32_t s_mx4[4][64];    // their merges in groups of four waves
__shared__ int s_last;
__shared__ int s_counted;  // waves done counting the history (lazy top-k rows)
// 16-wave top-k segments: arrivals at the early bound (per group of four waves, then group merges), the bound
// and its ready flag
__shared__ int s_arr[4];
__shared__ uint32_t s_qe;
__shared__ int s_qready;


// ---------------------------------------------------------------------------------------------------------
// keys: order-preserving 32-bit image of the f32 value in the high word, ~id in the low word, so that a larger
// 64-bit key means a larger value or, on equal values, a lower id. -0 is folded onto +0 (the reference's
// comparator treats them as equal); NaN maps to 0, below every number.
__device__ __forceinline__ uint32_t ord_f32(float v) {
    uint32_t u = __float_as_uint(v);
    if (v == 0.0f) u = 0u;
    if (v != v) return 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float unord_f32(uint32_t o) {
    const uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
    return __uint_as_float(u);
}

__device__ __forceinline__ uint64_t mk_key(float v, int id) {
    return ((uint64_t) ord_f32(v) << 32) | (uint64_t) (~(uint32_t) id);
}

__device__ __forceinline__ int key_id(uint64_t k) { return (int) ~(uint32_t) k; }

// mk_key for a value known not to be NaN (-0 + 0 = +0 folds the zeros)
__device__ __forceinline__ uint64_t mk_key_num(float v, int id) {
    const uint32_t u = __float_as_uint(v + 0.0f);
    const uint32_t o = u ^ ((uint32_t) ((int32_t) u >> 31) | 0x80000000u);
    return ((uint64_t) o << 32) | (uint64_t) (~(uint32_t) id);
}

// Largest float f such that every value image >= o has value >= f.
__device__ __forceinline__ float floor32(uint32_t o) { return o == 0u ? -INFINITY : unord_f32(o); }
__device__ __forceinline__ float floor64(uint64_t k) { return floor32((uint32_t) (k >> 32)); }

__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Device-scope (all XCDs) relaxed store / load: written through to, and read from, the device coherence point.
__device__ __forceinline__ void store_dev(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_dev(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until every memory operation this wave issued has completed (device-scope stores acknowledged).
__device__ __forceinline__ void wait_stores() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ uint64_t min64(uint64_t a, uint64_t b) { return a > b ? b : a; }

// Signalling between the waves of one workgroup through LDS flags and counters. The LDS serves each wave's
// operations in order, so the LDS writes a wave made before raising a flag are seen by a wave that has seen the
// flag and reads after it. Release or acquire orderings at workgroup scope would also make the wave wait for its
// outstanding global loads (s_waitcnt vmcnt(0)), which drains a stream of logit loads still in flight; these wait
// for the wave's LDS operations only (lgkmcnt(0)) and keep the compiler from moving memory operations across.
__device__ __forceinline__ void lds_wait() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt and expcnt not waited for
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ int lds_raise(int* p, int v) {
    lds_wait();
    const int old = __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return old;
}
__device__ __forceinline__ void lds_publish(int* p, int v) {
    lds_wait();
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ int lds_peek(const int* p) {
    const int v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    return v;
}

// ---------------------------------------------------------------------------------------------------------
// wave64 cross-lane exchange with lane ^ M: DPP within rows of 16 lanes, permlane swaps across rows.
// Every cross-lane read (DPP, permlane, readlane, ballot) runs in wave-uniform control flow with all 64 lanes
// active, and its result is consumed outside lane-divergent branches: inside such a branch the compiler may
// compute the inputs for the active lanes only.
template <int CTRL>
__device__ __forceinline__ int dpp(int x) {
    return __builtin_amdgcn_mov_dpp(x, CTRL, 0xf, 0xf, false);
}

template <int M>
__device__ __forceinline__ int xor_lane(int x, int lane) {
    if constexpr (M == 1) {
        return dpp<0xB1>(x);  // quad_perm [1,0,3,2]
    } else if constexpr (M == 2) {
        return dpp<0x4E>(x);  // quad_perm [2,3,0,1]
    } else if constexpr (M == 4) {
        return dpp<0x141>(dpp<0x1B>(x));  // quad_perm [3,2,1,0] then row_half_mirror: i ^ 3 ^ 7
    } else if constexpr (M == 8) {
        return dpp<0x128>(x);  // row_ror:8
    } else if constexpr (M == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);  // {[r0 r0 r2 r2], [r1 r1 r3 r3]}
        return (lane & 16) ? (int) p[0] : (int) p[1];
    } else {
        static_assert(M == 32, "xor distance");
        const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);  // {[lo lo], [hi hi]}
        return (lane & 32) ? (int) p[0] : (int) p[1];
    }
}

template <int M>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t x, int lane) {
    const uint32_t lo = (uint32_t) xor_lane<M>((int) (uint32_t) x, lane);
    const uint32_t hi = (uint32_t) xor_lane<M>((int) (uint32_t) (x >> 32), lane);
    return ((uint64_t) hi << 32) | lo;
}

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }
__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }
__device__ __forceinline__ int mbcnt(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t) (m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t) m, 0u));
}

__device__ __forceinline__ uint64_t rdlane64(uint64_t x, int l) {
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) x, l);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readlane((int) (uint32_t) (x >> 32), l);
    return ((uint64_t) hi << 32) | lo;
}
__device__ __forceinline__ float rdlanef(float x, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}
__device__ __forceinline__ int rdlanei(int x, int l) { return __builtin_amdgcn_readlane(x, l); }

// Lanes that keep the larger key in a compare-exchange step of a bitonic network (block size SIZE, partner
// lane ^ STRIDE; DESC: blocks sorted descending at the end), as a wave-uniform 64-bit mask. Wave lanes are
// numbered 0..63, so the mask is a constant and each step's direction logic is one scalar XOR.
template <int SIZE, int STRIDE, bool DESC>
constexpr uint64_t keep_max_lanes() {
    uint64_t m = 0;
    for (int l = 0; l < 64; ++l) {
        const bool up = ((l & SIZE) == 0) == DESC;
        const bool lower = (l & STRIDE) == 0;
        if (lower == up) m |= 1ull << l;
    }
    return m;
}

// Both lanes of every pair (lane, lane ^ M), M = 16 or 32, get {lower lane's x, upper lane's x}.
template <int M>
__device__ __forceinline__ auto swap_rows(uint32_t x) {
    if constexpr (M == 16) {
        return __builtin_amdgcn_permlane16_swap(x, x, false, false);
    } else {
        static_assert(M == 32, "row distance");
        return __builtin_amdgcn_permlane32_swap(x, x, false, false);
    }
}

// One compare-exchange step. With DPP partners (STRIDE < 16) a lane takes its partner's key y when
// (y > x) == keep-max; permlane swaps (STRIDE 16, 32) give both lanes of a pair the pair's lower-lane key a and
// upper-lane key b, and a lane takes a when (a > b) == keep-max. (Equal keys: either choice is the same key.)
template <int SIZE, int STRIDE, bool DESC, typename T>
__device__ __forceinline__ T bitonic_step_t(T x, int lane) {
    const bool km = __builtin_amdgcn_inverse_ballot_w64(keep_max_lanes<SIZE, STRIDE, DESC>());
    if constexpr (STRIDE < 16) {
        T y;
        if constexpr (sizeof(T) == 8) {
            y = xor_lane64<STRIDE>(x, lane);
        } else {
            y = (T) xor_lane<STRIDE>((int) x, lane);
        }
        return ((y > x) == km) ? y : x;
    } else {
        T a, b;
        if constexpr (sizeof(T) == 8) {
            const auto pl = swap_rows<STRIDE>((uint32_t) x);
            const auto ph = swap_rows<STRIDE>((uint32_t) (x >> 32));
            a = ((uint64_t) ph[0] << 32) | pl[0];
            b = ((uint64_t) ph[1] << 32) | pl[1];
        } else {
            const auto p = swap_rows<STRIDE>(x);
            a = p[0];
            b = p[1];
        }
        return ((a > b) == km) ? a : b;
    }
}

template <int SIZE, int STRIDE, bool DESC>
__device__ __forceinline__ uint64_t bitonic_step(uint64_t x, int lane) {
    return bitonic_step_t<SIZE, STRIDE, DESC, uint64_t>(x, lane);
}

template <int SIZE, bool DESC>
__device__ __forceinline__ uint64_t bitonic_stage(uint64_t x, int lane) {
    if constexpr (SIZE >= 64) x = bitonic_step<SIZE, 32, DESC>(x, lane);
    if constexpr (SIZE >= 32) x = bitonic_step<SIZE, 16, DESC>(x, lane);
    if constexpr (SIZE >= 16) x = bitonic_step<SIZE, 8, DESC>(x, lane);
    if constexpr (SIZE >= 8) x = bitonic_step<SIZE, 4, DESC>(x, lane);
    if constexpr (SIZE >= 4) x = bitonic_step<SIZE, 2, DESC>(x, lane);
    return bitonic_step<SIZE, 1, DESC>(x, lane);
}

// Sorts one key per lane across the wave (DESC: lane 0 holds the largest).
template <bool DESC>
__device__ __forceinline__ uint64_t sort64(uint64_t x, int lane) {
    x = bitonic_stage<2, DESC>(x, lane);
    x = bitonic_stage<4, DESC>(x, lane);
    x = bitonic_stage<8, DESC>(x, lane);
    x = bitonic_stage<16, DESC>(x, lane);
    x = bitonic_stage<32, DESC>(x, lane);
    return bitonic_stage<64, DESC>(x, lane);
}

// Top 64 of a descending list `a` and an ascending list `b`, descending.
__device__ __forceinline__ uint64_t merge64(uint64_t a, uint64_t b, int lane) {
    return bitonic_stage<64, true>(max64(a, b), lane);  // max of desc and asc is bitonic
}

template <int SIZE, int STRIDE, bool DESC>
__device__ __forceinline__ uint32_t bitonic_step32(uint32_t x, int lane) {
    return bitonic_step_t<SIZE, STRIDE, DESC, uint32_t>(x, lane);
}

template <int SIZE, bool DESC>
__device__ __forceinline__ uint32_t bitonic_stage32(uint32_t x, int lane) {
    if constexpr (SIZE >= 64) x = bitonic_step32<SIZE, 32, DESC>(x, lane);
    if constexpr (SIZE >= 32) x = bitonic_step32<SIZE, 16, DESC>(x, lane);
    if constexpr (SIZE >= 16) x = bitonic_step32<SIZE, 8, DESC>(x, lane);
    if constexpr (SIZE >= 8) x = bitonic_step32<SIZE, 4, DESC>(x, lane);
    if constexpr (SIZE >= 4) x = bitonic_step32<SIZE, 2, DESC>(x, lane);
    return bitonic_step32<SIZE, 1, DESC>(x, lane);
}

// Sorts one 32-bit value per lane across the wave (DESC: lane 0 holds the largest).
template <bool DESC>
__device__ __forceinline__ uint32_t sort32(uint32_t x, int lane) {
    x = bitonic_stage32<2, DESC>(x, lane);
    x = bitonic_stage32<4, DESC>(x, lane);
    x = bitonic_stage32<8, DESC>(x, lane);
    x = bitonic_stage32<16, DESC>(x, lane);
    x = bitonic_stage32<32, DESC>(x, lane);
    return bitonic_stage32<64, DESC>(x, lane);
}

// Top 64 of a descending list `a` and an ascending list `b`, descending.
__device__ __forceinline__ uint32_t merge32(uint32_t a, uint32_t b, int lane) {
    return bitonic_stage32<64, true>(max(a, b), lane);
}


// Inserts the wave-uniform key x into the descending list held one key per lane (keys distinct; the smallest
// falls off): lanes below x's position keep theirs, the rest shift down one lane (DPP wave_shr:1).
__device__ __forceinline__ uint64_t insert64(uint64_t lst, uint64_t x, int lane) {
    const int pos = __popcll(ballot(lst > x));
    const uint32_t lo = (uint32_t) __builtin_amdgcn_mov_dpp((int) (uint32_t) lst, 0x138, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_mov_dpp((int) (uint32_t) (lst >> 32), 0x138, 0xf, 0xf, false);
    const uint64_t sh = ((uint64_t) hi << 32) | lo;
    return lane < pos ? lst : (lane == pos ? x : sh);
}

__device__ __forceinline__ uint64_t wave_max64(uint64_t x, int lane) {
    x = max64(x, xor_lane64<32>(x, lane));
    x = max64(x, xor_lane64<16>(x, lane));
    x = max64(x, xor_lane64<8>(x, lane));
    x = max64(x, xor_lane64<4>(x, lane));
    x = max64(x, xor_lane64<2>(x, lane));
    return max64(x, xor_lane64<1>(x, lane));
}

// ---------------------------------------------------------------------------------------------------------
// expf, bit-identical to the host glibc's (>= 2.27, x86-64 FMA variant) on every input: the table-driven
// method of ARM's optimized-routines (Szabolcs Nagy): x*32/ln2 = k + r, exp(x) = 2^(k/32) * 2^(r/32), with
// 2^(r/32) from a cubic in r, evaluated in double and rounded once to float. tab[i] = bits(RN(2^(i/32))) - i<<47.
__device__ const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

__device__ __forceinline__ float expf_glibc(float x) {
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88 or nan
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double) x;
    double kd = __builtin_fma(inv_ln2_32, xd, shift);
    const uint64_t ki = (uint64_t) __double_as_longlong(kd);
    kd = __dsub_rn(kd, shift);
    const double r = __builtin_fma(inv_ln2_32, xd, -kd);
    const uint64_t t = kExp2Tab[ki & 31u] + (ki << 47);
    const double s = __longlong_as_double((long long) t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = __dmul_rn(r, r);
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = __dmul_rn(y, s);
    return __double2float_rn(y);
}

// expf_glibc with the table in registers: lane l of `tab` holds kExp2Tab[l & 31], read across lanes
// (ds_bpermute), so every lane of the wave must call it; the special cases are selected after.
__device__ __forceinline__ float expf_glibc_tab(float x, uint64_t tab) {
    const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double) x;
    double kd = __builtin_fma(inv_ln2_32, xd, shift);
    const uint64_t ki = (uint64_t) __double_as_longlong(kd);
    kd = __dsub_rn(kd, shift);
    const double r = __builtin_fma(inv_ln2_32, xd, -kd);
    const int src = (int) (ki & 31u) << 2;
    const uint32_t lo = (uint32_t) __builtin_amdgcn_ds_bpermute(src, (int) (uint32_t) tab);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_ds_bpermute(src, (int) (uint32_t) (tab >> 32));
    const uint64_t t = (((uint64_t) hi << 32) | lo) + (ki << 47);
    const double s = __longlong_as_double((long long) t);
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = __dmul_rn(r, r);
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = __dmul_rn(y, s);
    float res = __double2float_rn(y);
    const uint32_t ux = __float_as_uint(x);
    if (((ux >> 20) & 0x7ffu) >= 0x42bu) {  // |x| >= 88 or nan: as expf_glibc
        if (ux == 0xff800000u) res = 0.0f;
        else if (((ux >> 20) & 0x7ffu) >= 0x7f8u) res = x + x;
        else if (x > 0x1.62e42ep6f) res = __uint_as_float(0x7f800000u);
        else if (x < -0x1.9fe368p6f) res = 0.0f;
    }
    return res;
}

// Penalty of src/sampler.cpp:24-25 for an id seen `c` > 0 times: repetition first (l > 0 ? l / rep : l * rep),
// then l - (presence + frequency * (float)c), each operation rounded separately (no contraction). Branch-free:
// with a repetition penalty of 1 both forms give l, as the reference's skipped step leaves it. The quotient is
// RN_f32(l * (1/rep in double)): exact for every float l. Why: the double product's relative error is below
// 2^-51.9, while a quotient of two floats that is not a float lies more than 2^-49 (relative) from every midpoint
// between floats (the midpoint m = M 2^e, M odd with 25 bits, makes l - rep*m a nonzero multiple of 2^e*ulp), so
// rounding the product to float cannot cross one. Specials agree too (0, inf, NaN operands and rep = 0 or inf).
__device__ __forceinline__ float penalize(float l, uint32_t c, const SamplingParams& p) {
    const float d = __double2float_rn(__dmul_rn((double) l, p.inv_repetition));
    const float m = __fmul_rn(l, p.repetition);
    l = l > 0.0f ? d : m;
    const float f = __fmul_rn(p.frequency, __uint2float_rn(c));
    const float t = __fadd_rn(p.presence, f);
    return __fsub_rn(l, t);
}

// ---------------------------------------------------------------------------------------------------------
// History counts in LDS. A table covers the ids [tlo, thi) of a segment. Entry i counts id tlo + i: a 32-bit
// word each, or (C16) a 16-bit half of word i/2, bits 16*(i%2) up, which halves the table of a long segment.
// 16-bit counts are exact while a row's history holds fewer than 65536 ids; longer histories take 32-bit
// tables over half a segment at a time.

// The 16-byte aligned body of the raw history prefetched ahead of the second half of the logits, per thread.
constexpr int HR = 4;

template <bool C16>
__device__ __forceinline__ void cnt_add(int id, int tlo, int thi, uint32_t w) {
    const uint32_t i = (uint32_t) id - (uint32_t) tlo;  // ids below tlo wrap to large values
    if (i < (uint32_t) (thi - tlo)) {
        if (C16)
            atomicAdd(&s_cnt[i >> 1], w << ((i & 1u) << 4));
        else
            atomicAdd(&s_cnt[i], w);
    }
}

// Clears the first `words` words of the table (rounded up to 4: segments are multiples of 1024 ids) with threads
// tid = 0..WG-1.
template <int WG>
__device__ __forceinline__ void cnt_zero(int words, int tid = (int) threadIdx.x) {
    const int n4 = (words + 3) & ~3;
    for (int i = 4 * tid; i < n4; i += 4 * WG) *reinterpret_cast<uint4*>(s_cnt + i) = make_uint4(0u, 0u, 0u, 0u);
}

// Where a row's raw history lies: ids [s0, s1) of hist_ids; [b0, b1) is its 16-byte aligned body (empty when the
// array itself is not 16-byte aligned), of which each thread prefetched HR int4 starting at b0.
struct RawHistory {
    int s0 = 0, b0 = 0, b1 = 0, s1 = 0;
};

// Counts every history id in [tlo, thi) into the table: the prefetched int4s, the rest of a raw history, a
// bucketed history, and the extra lists.
// Without PREF the whole raw history is read from memory (hq unused).
// The counting threads are tid = 0..WG-1 (the workgroup's threads, or a subset of its waves).
template <int WG, bool C16, bool PREF>
__device__ __forceinline__ void count_history(const RowsArgs& a, int row, int tlo, int thi, const int4 (&hq)[HR],
                                              const RawHistory& rh, int tid) {
    if (a.hist_off) {
        if (PREF) {
#pragma unroll
            for (int r = 0; r < HR; ++r) {
                cnt_add<C16>(hq[r].x, tlo, thi, 1u);
                cnt_add<C16>(hq[r].y, tlo, thi, 1u);
                cnt_add<C16>(hq[r].z, tlo, thi, 1u);
                cnt_add<C16>(hq[r].w, tlo, thi, 1u);
            }
        }
        for (int j = rh.s0 + tid; j < rh.b0; j += WG) cnt_add<C16>(a.hist_ids[j], tlo, thi, 1u);
        for (int j = rh.b0 + 4 * ((PREF ? HR * WG : 0) + tid); j < rh.b1; j += 4 * WG) {
            const int4 q = *reinterpret_cast<const int4*>(a.hist_ids + j);
            cnt_add<C16>(q.x, tlo, thi, 1u);
            cnt_add<C16>(q.y, tlo, thi, 1u);
            cnt_add<C16>(q.z, tlo, thi, 1u);
            cnt_add<C16>(q.w, tlo, thi, 1u);
        }
        for (int j = rh.b1 + tid; j < rh.s1; j += WG) cnt_add<C16>(a.hist_ids[j], tlo, thi, 1u);
    } else if (a.hist_boff) {
        // bucketed unique ids with counts: read the buckets that overlap [tlo, thi)
        const int bb0 = tlo >> a.bucket_shift;
        const int bb1 = min(a.n_buckets, (thi + (1 << a.bucket_shift) - 1) >> a.bucket_shift);
        const int s0 = max(a.hist_boff[bb0], 0), s1 = a.hist_boff[bb1];
        for (int j = s0 + tid; j < s1; j += WG) cnt_add<C16>(a.hist_ids[j], tlo, thi, (uint32_t) a.hist_w[j]);
    }
    if (a.extra_a) {
        const int na = min(max(*a.extra_a_n, 0), PENDING_CAP);
        for (int j = tid; j < na; j += WG) cnt_add<C16>(a.extra_a[j], tlo, thi, 1u);
    }
    if (a.extra_b) {
        const int nb = min(row * a.extra_b_step, VERIFY_MAX_ROWS);
        for (int j = tid; j < nb; j += WG) cnt_add<C16>(a.extra_b[j], tlo, thi, 1u);
    }
}

// The history counts of the four ids lo + 4*(i*WG + tid) + e from the table over [tlo, ...); 0 past hi (unless
// INR: every id is below hi).
template <int WG, bool C16, bool INR>
__device__ __forceinline__ void group_counts(uint32_t (&c)[4], int i, int lo, int hi, int tlo, float dep = 0.0f) {
    const int id0 = lo + 4 * (i * WG + (int) threadIdx.x);
    if (!INR && id0 >= hi) {
        c[0] = c[1] = c[2] = c[3] = 0u;
        return;
    }
    int t = id0 - tlo;  // a multiple of 4
    // The read waits for `dep` (the caller's running result over the previous groups): the scheduler would
    // otherwise hoist every group's read ahead of the data and hold all their flags at once.
    asm volatile("" : "+v"(t) : "v"(dep));
    if (C16) {
        const uint2 q = *reinterpret_cast<const uint2*>(s_cnt + (t >> 1));
        c[0] = q.x & 0xffffu;
        c[1] = q.x >> 16;
        c[2] = q.y & 0xffffu;
        c[3] = q.y >> 16;
    } else {
        const uint4 q = *reinterpret_cast<const uint4*>(s_cnt + t);
        c[0] = q.x;
        c[1] = q.y;
        c[2] = q.z;
        c[3] = q.w;
    }
#pragma unroll
    for (int e = 1; e < 4; ++e)
        if (!INR && id0 + e >= hi) c[e] = 0u;
}

// Applies the table's counts to the four logits of group i this thread holds (ids lo + 4*(i*WG + tid) + e).
// Nearly every wave-wide group holds some history id, so the penalty is computed for all four logits and
// selected where the count is nonzero (no divergent branches). INR: every id is below hi.
template <int WG, int EPT, bool C16, bool INR>
__device__ __forceinline__ void apply_group(float (&v)[EPT], int i, int lo, int hi, int tlo, const SamplingParams& p) {
    uint32_t c[4];
    group_counts<WG, C16, INR>(c, i, lo, hi, tlo);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float x = v[4 * i + e];
        const float y = penalize(x, c[e], p);
        v[4 * i + e] = c[e] != 0u ? y : x;
    }
}

template <int WG, int EPT, bool C16, bool INR, int I0, int I1>
__device__ __forceinline__ void apply_counts(float (&v)[EPT], int lo, int hi, int tlo, const SamplingParams& p) {
#pragma unroll
    for (int i = I0; i < I1; ++i) apply_group<WG, EPT, C16, INR>(v, i, lo, hi, tlo, p);
}

// ---------------------------------------------------------------------------------------------------------
// Candidate lists. Survivors of the filter are appended to the wave's LDS region. The workgroup's regions are
// then read as one list in chunks of 64: one chunk is sorted once; more are sorted by one wave each and merged.
// Regions that fill up are folded (sort + bitonic merge) on the slow paths only.

// Descending top-64 of `lst` (descending; ignored when !have) and the n keys of the wave's region.
template <int NW>
__device__ __forceinline__ uint64_t fold_region(int wave, int n, uint64_t lst, bool have, int lane) {
    for (int c0 = 0; c0 < n; c0 += 64) {
        const uint64_t key = (c0 + lane < n) ? s_cand<NW>[wave][c0 + lane] : 0ull;
        if (!have) {
            lst = sort64<true>(key, lane);
            have = true;
        } else {
            lst = merge64(lst, sort64<false>(key, lane), lane);
        }
    }
    return have ? lst : 0ull;
}

// Appends the keys of `pass` lanes to the wave's region; records an overflow instead of folding.
template <int NW>
struct WaveCollect {
    int n = 0;
    bool overflow = false;
    __device__ __forceinline__ void offer(int wave, bool pass, uint64_t key) {
        const uint64_t m = ballot(pass);
        if (!m) return;
        const int c = __popcll(m);
        if (n + c > CW) {
            overflow = true;
            return;
        }
        if (pass) s_cand<NW>[wave][n + mbcnt(m)] = key;
        n += c;
    }
};

// A wave's descending top-64 over a stream of offers, folding its region whenever it fills (slow paths).
template <int NW>
struct WaveTopK {
    uint64_t lst = 0ull;
    bool have = false;
    int n = 0;
    uint64_t own = 0ull;  // lst's k-th key (0 while fewer than k)
    __device__ __forceinline__ void offer(int wave, bool pass, uint64_t key, int k, int lane) {
        const uint64_t m = ballot(pass);
        if (!m) return;
        const int c = __popcll(m);
        if (n + c > CW) {
            __builtin_amdgcn_wave_barrier();
            lst = fold_region<NW>(wave, n, lst, have, lane);
            have = true;
            n = 0;
            own = rdlane64(lst, k - 1);
            __builtin_amdgcn_wave_barrier();
        }
        if (pass) s_cand<NW>[wave][n + mbcnt(m)] = key;
        n += c;
    }
    __device__ __forceinline__ uint64_t finish(int wave, int lane) {
        __builtin_amdgcn_wave_barrier();
        return fold_region<NW>(wave, n, lst, have, lane);
    }
};

// Wave 0's descending top-64 of the lists in s_list[0..n) (other waves return 0).
template <int NW>
__device__ __forceinline__ uint64_t merge_lists(int n, int lane, int wave) {
    if (wave != 0) return 0ull;
    uint64_t lst = s_list<NW>[0][lane];
    for (int o = 1; o < n; ++o) lst = merge64(lst, s_list<NW>[o][63 - lane], lane);
    return lst;
}

// The workgroup's descending top-64 of what its waves collected, in wave 0 (other waves get 0). Returns false
// (in every thread) if a region overflowed.
// Publishes the waves' region counts (-1: overflow) and reads them all back; returns false if any overflowed.
template <int NW>
__device__ __forceinline__ bool region_counts(const WaveCollect<NW>& w, int lane, int wave, int (&cnt)[NW], int* total) {
    if (lane == 0) s_n<NW>[wave] = w.overflow ? -1 : w.n;
    __syncthreads();
    bool bad = false;
    *total = 0;
#pragma unroll
    for (int r = 0; r < NW; ++r) {
        cnt[r] = s_n<NW>[r];
        bad |= cnt[r] < 0;
        *total += cnt[r];
    }
    return !bad;
}

// The workgroup's descending top-64 of the regions (cnt[r] keys in region r), in wave 0 (others get 0).
template <int NW>
__device__ __forceinline__ uint64_t select_regions(const int (&cnt)[NW], int total, int lane, int wave) {
    const int nc = (total + 63) >> 6;
    if (nc > NW) {
        // more chunks than waves: every wave folds its own region, wave 0 merges the lists
        const uint64_t lst = fold_region<NW>(wave, s_n<NW>[wave], 0ull, false, lane);
        s_list<NW>[wave][lane] = lst;
        __syncthreads();
        return merge_lists<NW>(NW, lane, wave);
    }
    // entry j of the concatenated regions: find its region, then one read
    auto entry = [&](int j) {
        int r = 0, base = 0, end = cnt[0];
#pragma unroll
        for (int q = 1; q < NW; ++q) {
            const bool past = j >= end;
            r = past ? q : r;
            base = past ? end : base;
            end += cnt[q];
        }
        return j < total ? s_cand<NW>[r][j - base] : 0ull;
    };
    const int extra = total - 64;
    if (extra > 0 && extra <= 16) {
        // a few keys past one chunk: wave 0 sorts the first 64 and inserts the others one at a time
        if (wave != 0) return 0ull;
        uint64_t lst = sort64<true>(entry(lane), lane);
        const uint64_t ex = entry(64 + lane);
        for (int t = 0; t < extra; ++t) lst = insert64(lst, rdlane64(ex, t), lane);
        return lst;
    }
    uint64_t lst = 0ull;
    if (wave < nc) lst = sort64<true>(entry(64 * wave + lane), lane);  // chunk `wave`
    if (nc <= 1) return wave == 0 ? lst : 0ull;
    if (wave < nc) s_list<NW>[wave][lane] = lst;
    __syncthreads();
    return merge_lists<NW>(nc, lane, wave);
}

// The workgroup's descending top-64 of what its waves collected, in wave 0 (other waves get 0). Returns false
// (in every thread) if a region overflowed.
template <int NW>
__device__ __forceinline__ bool wg_select(const WaveCollect<NW>& w, int lane, int wave, uint64_t* out) {
    int cnt[NW], total;
    *out = 0ull;
    if (!region_counts<NW>(w, lane, wave, cnt, &total)) return false;
    *out = select_regions<NW>(cnt, total, lane, wave);
    return true;
}

// Scans ids [slo, shi) into the waves' exact lists (slow path), with penalties from the table over [tlo, ...).
template <int NW, bool C16>
__device__ __forceinline__ void scan_exact(WaveTopK<NW>& w, const RowsArgs& a, const float* __restrict__ L, int slo,
                                           int shi, bool pen, int tlo, uint64_t t_row, int lane, int wave) {
    constexpr int WG = NW * 64;
    for (int base = slo + 4 * (wave * 64 + lane); base - 4 * lane < shi; base += 4 * WG) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int id = base + e;
            float x = __uint_as_float(0x7fc00000u);
            if (id < shi) {
                x = L[id];
                if (pen) {
                    const uint32_t i = (uint32_t) (id - tlo);
                    const uint32_t c = C16 ? (s_cnt[i >> 1] >> ((i & 1u) << 4)) & 0xffffu : s_cnt[i];
                    if (c != 0u) x = penalize(x, c, a.p);
                }
            }
            const uint64_t key = x == x ? mk_key(x, id) : 0ull;
            w.offer(wave, key != 0ull && key > max64(t_row, w.own), key, a.p.k, lane);
        }
    }
}

// Slow path of a segment (a region overflowed, e.g. many logits equal to the bound): re-read the segment and
// keep exact per-wave lists with folding, then merge. With `wide` counts the history is staged again, half a
// segment at a time. Returns the top-64 in wave 0.
// The table, when present, covers the ids from lb (<= lo) on.
template <int NW, int SEG, bool C16>
__device__ __forceinline__ uint64_t segment_slow(const RowsArgs& a, const float* __restrict__ L, int row, int lo, int hi,
                                                 int lb, bool pen, bool wide, const RawHistory& rh, uint64_t t_row,
                                                 int lane, int wave) {
    constexpr int WG = NW * 64;
    WaveTopK<NW> w;
    if (!pen || !wide) {
        scan_exact<NW, C16>(w, a, L, lo, hi, pen, lb, t_row, lane, wave);
    } else {
#pragma unroll 1
        for (int h = 0; h < 2; ++h) {
            const int wlo = max(lo, lb + h * (SEG / 2)), whi = min(hi, lb + (h + 1) * (SEG / 2));
            if (wlo >= whi) continue;  // uniform
            __syncthreads();
            cnt_zero<WG>(whi - wlo);
            __syncthreads();
            const int4 none[HR] = {};
            count_history<WG, false, false>(a, row, wlo, whi, none, rh, (int) threadIdx.x);
            __syncthreads();
            scan_exact<NW, false>(w, a, L, wlo, whi, true, wlo, t_row, lane, wave);
        }
    }
    s_list<NW>[wave][lane] = w.finish(wave, lane);
    __syncthreads();
    return merge_lists<NW>(NW, lane, wave);
}

// Slow path of the row merge: every segment list entry at or above `ts`, folded exactly.
template <int NW>
__device__ __forceinline__ uint64_t merge_slow(const uint64_t* cand, int segs, int k, uint64_t ts, int lane, int wave) {
    WaveTopK<NW> w;
    for (int s = wave; s < segs; s += NW) {
        const uint64_t key = lane < k ? load_dev(&cand[(int64_t) s * KCAP + lane]) : 0ull;
        w.offer(wave, key != 0ull && key >= ts && key > w.own, key, k, lane);
    }
    s_list<NW>[wave][lane] = w.finish(wave, lane);
    __syncthreads();
    return merge_lists<NW>(NW, lane, wave);
}


// ---------------------------------------------------------------------------------------------------------
// The O(k) tail of src/sampler.cpp:53-88 on one wave: lane i holds the i-th candidate (value descending, id
// ascending) for i < kk.
//
// The reference accumulates in double, sequentially: the softmax total, the top-p cumulative sum, the draw's
// total and the draw's running subtraction. When every addend is a multiple of a power of two small enough that
// no partial sum needs more than 53 bits, each of those sums is exact, hence equal to the exact sum in any order:
// e_i >= 2^-23 (e_0 = 1, kk <= 64: partial sums < 2^7, multiples of 2^-46) and p_i >= 2^-28 (partial sums < 2,
// multiples of 2^-51). Then the softmax total is a tree reduction, the cumulative sums are a wave prefix scan, and
// the draw's subtraction r_i = r - cum_i is exact until it first reaches <= 0 (rounding keeps the sign), so the
// drawn candidate is the first i with cum_i >= r. Otherwise the sums run as sequential register chains.

__device__ __forceinline__ double wave_sum_f64(double x, int lane) {
    uint64_t b = __builtin_bit_cast(uint64_t, x);
    b = __builtin_bit_cast(uint64_t, __builtin_bit_cast(double, b) + __builtin_bit_cast(double, xor_lane64<32>(b, lane)));
    b = __builtin_bit_cast(uint64_t, __builtin_bit_cast(double, b) + __builtin_bit_cast(double, xor_lane64<16>(b, lane)));
    b = __builtin_bit_cast(uint64_t, __builtin_bit_cast(double, b) + __builtin_bit_cast(double, xor_lane64<8>(b, lane)));
    b = __builtin_bit_cast(uint64_t, __builtin_bit_cast(double, b) + __builtin_bit_cast(double, xor_lane64<4>(b, lane)));
    b = __builtin_bit_cast(uint64_t, __builtin_bit_cast(double, b) + __builtin_bit_cast(double, xor_lane64<2>(b, lane)));
    b = __builtin_bit_cast(uint64_t, __builtin_bit_cast(double, b) + __builtin_bit_cast(double, xor_lane64<1>(b, lane)));
    return __builtin_bit_cast(double, b);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_f64(double x) {
    const uint64_t b = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) (uint32_t) b, CTRL, ROWS, 0xf, false);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) (uint32_t) (b >> 32), CTRL, ROWS, 0xf, false);
    return __builtin_bit_cast(double, ((uint64_t) hi << 32) | lo);  // 0.0 where the source lane is outside the row
}

// Integer forms of wave_sum_f64 above and wave_scan_f64 below (every lane active): the wave's total in every
// lane, and the inclusive prefix sum across the wave.
__device__ __forceinline__ int wave_sum_i32(int x, int lane) {
    x += xor_lane<32>(x, lane);
    x += xor_lane<16>(x, lane);
    x += xor_lane<8>(x, lane);
    x += xor_lane<4>(x, lane);
    x += xor_lane<2>(x, lane);
    return x + xor_lane<1>(x, lane);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_i32(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, ROWS, 0xf, false);  // 0 where the source lane is outside the row
}

__device__ __forceinline__ int wave_scan_i32(int x) {
    x += dpp_i32<0x111, 0xf>(x);
    x += dpp_i32<0x112, 0xf>(x);
    x += dpp_i32<0x114, 0xf>(x);
    x += dpp_i32<0x118, 0xf>(x);
    x += dpp_i32<0x142, 0xa>(x);
    x += dpp_i32<0x143, 0xc>(x);
    return x;
}

// Inclusive prefix sum across the wave (row_shr within rows of 16, then row broadcasts of lanes 15 and 31).
__device__ __forceinline__ double wave_scan_f64(double x) {
    x += dpp_f64<0x111, 0xf>(x);
    x += dpp_f64<0x112, 0xf>(x);
    x += dpp_f64<0x114, 0xf>(x);
    x += dpp_f64<0x118, 0xf>(x);
    x += dpp_f64<0x142, 0xa>(x);
    x += dpp_f64<0x143, 0xc>(x);
    return x;
}

__device__ __forceinline__ double rdlaned(double x, int l) {
    return __builtin_bit_cast(double, rdlane64(__builtin_bit_cast(uint64_t, x), l));
}

// Sequential chains in reference order; lane i keeps the i-th partial result.
__device__ __forceinline__ double chain_sum(float e, int kk) {
    double sum = 0.0;
    for (int i = 0; i < kk; ++i) sum = __dadd_rn(sum, (double) rdlanef(e, i));
    return sum;
}

__device__ __forceinline__ double chain_prefix(float p, int n, int lane) {
    double cum = 0.0, mine = 0.0;
    for (int i = 0; i < n; ++i) {
        cum = __dadd_rn(cum, (double) rdlanef(p, i));
        mine = lane == i ? cum : mine;
    }
    return mine;
}

__device__ __forceinline__ double chain_draw(double r, float p, int n, int lane) {
    double mine = 1.0;
    for (int i = 0; i < n; ++i) {
        r = __dsub_rn(r, (double) rdlanef(p, i));
        mine = lane == i ? r : mine;
    }
    return mine;
}

// exp_tab: lane l holds kExp2Tab[l & 31] (loaded ahead by the caller).
__device__ int sample_tail(uint64_t lst, int kk, const SamplingParams p, double u, uint64_t exp_tab, int lane,
                           float* dbg_probs, int32_t* dbg_meta) {
    if (kk == 0) return 0;
    const bool act = lane < kk;
    const float v = act ? unord_f32((uint32_t) (lst >> 32)) : 0.0f;
    const int id = act ? key_id(lst) : -1;
    // softmax with temperature (:53-60)
    const float maxl = rdlanef(v, 0);
    const float x = __fdiv_rn(__fsub_rn(v, maxl), p.temperature);
    const float ex = expf_glibc_tab(x, exp_tab);  // (all lanes)
    const float e = act ? ex : 0.0f;
    const bool exact_e = ballot(act && e < 0x1p-23f) == 0ull;
    const double sum = exact_e ? wave_sum_f64((double) e, lane) : chain_sum(e, kk);
    const float pr = act ? __double2float_rn(__ddiv_rn((double) e, sum)) : 0.0f;
    int n = kk;
    // min-p (:62-68): keep the prefix while p >= p0*min_p
    if (p.min_p > 0.0f) {
        const float thr = __fmul_rn(rdlanef(pr, 0), p.min_p);
        const uint64_t fail = ballot(act && lane >= 1 && !(pr >= thr));
        if (fail) n = __builtin_ctzll(fail);
    }
    // top-p (:69-79): cum_i = (...((0 + p0) + p1) ...) + p_i, stop at the first cum_i >= top_p; the draw total
    // (:80-81) is the same chain over the kept prefix, cum_{n-1}
    const bool exact_p = ballot(lane < n && pr < 0x1p-28f) == 0ull;
    const double cum = exact_p ? wave_scan_f64(lane < n ? (double) pr : 0.0) : chain_prefix(pr, n, lane);
    if (p.top_p < 1.0f) {
        const uint64_t hit = ballot(lane < n && cum >= (double) p.top_p);
        if (hit) n = __builtin_ctzll(hit) + 1;
    }
    const double total = rdlaned(cum, n - 1);
    // draw (:82-88): r = u*(total-0)+0 as std::uniform_real_distribution<double>(0, total); r -= p_i until <= 0
    const double r = __dadd_rn(__dmul_rn(u, __dsub_rn(total, 0.0)), 0.0);
    uint64_t hit;
    if (exact_p)
        hit = ballot(lane < n && cum >= r);
    else
        hit = ballot(lane < n && chain_draw(r, pr, n, lane) <= 0.0);
    const int tok = rdlanei(id, hit ? __builtin_ctzll(hit) : n - 1);
    if (dbg_probs) dbg_probs[lane] = pr;
    if (dbg_meta && lane == 0) {
        dbg_meta[0] = kk;
        dbg_meta[1] = n;
    }
    return tok;
}

// Reports that an internal wait of this launch gave up (its results are then not trusted): the host turns a
// nonzero word into an error.
__device__ __forceinline__ void report_fault(const RowsArgs& a, uint32_t code) {
    if (a.fault) __hip_atomic_store(a.fault, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Publishes row `row`'s token: device output, and for the host one 64-bit word (sequence number, token).
// `seq` is the call's sequence number (read_call: the call block is host memory); `draft` the draft
// this row's token is compared with in a verify step (src/engine.cpp:571: batch[row + 1]; unused for the last
// row). Called by one lane.
__device__ __forceinline__ void publish(const RowsArgs& a, int row, int tok, uint32_t seq, int32_t draft) {
    a.out_tokens[row] = tok;
    a.row_ticket[row] = 0u;
    if (a.share_bounds) a.row_thr[row] = 0ull;
    // (the step counter first: waiting for its return then does not wait for a store to host memory)
    int acc = -1;
    if (a.step_word) {
        // engine.cpp:564-575: drafts are accepted while batch[i + 1] == t_i. Row r (< nb - 1) sets bit r when its
        // token differs from its draft; bit nb - 1 stands for the end of the batch, so accepted = the lowest set
        // bit of the union. The count in the high word tells the last row apart.
        const uint64_t mine = (1ull << 32) | ((row + 1 < a.n_rows && tok != draft) ? (1ull << row) : 0ull);
        const uint64_t prev = __hip_atomic_fetch_add(a.step_word, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((uint32_t) (prev >> 32) == (uint32_t) (a.n_rows - 1)) {
            acc = __builtin_ctz((uint32_t) (prev | mine) | (1u << (a.n_rows - 1)));
            *a.out_accepted = acc;
            __hip_atomic_store(a.step_word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (a.host_res && row < VERIFY_MAX_ROWS) {
        __hip_atomic_store(&a.host_res->row_word[row], ((uint64_t) seq << 32) | (uint32_t) tok, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
        if (acc >= 0)
            __hip_atomic_store(&a.host_res->step_word, ((uint64_t) seq << 32) | (uint32_t) acc, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// What a row's last workgroup needs from the call block (pinned host memory for steps over the handle's history):
// the sequence number to publish, the row's draft and uniform. The workgroup's last wave reads them (scalar
// loads) once it has issued all its logit loads, and hands them to wave 0 through LDS before a barrier that
// precedes the tail. Issued at kernel start, the same loads held the workgroup's first barrier (whose wait on the
// scalar/LDS counter includes them) for a PCIe round trip before most logits were requested; as system-scope
// vector loads they were slower still. Measured on the 4-row verify step: 14.1 us at kernel start, 9.8 us here,
// 9.6 us with no host reads at all.
struct CallIn {
    uint32_t seq;
    int32_t draft;
    double u;
};

__shared__ CallIn s_cin;

template <bool GREEDY>
__device__ __forceinline__ CallIn read_call(const RowsArgs& a, int row) {
    CallIn c{0u, -1, 0.0};
    if (a.host_res) c.seq = a.call->seq;
    if (a.step_word && row + 1 < a.n_rows) c.draft = a.call->drafts[row];
    if (!GREEDY) c.u = a.u[row];
    return c;
}

// The row's last workgroup, wave 0 (all lanes), with at most 8 segments: the lists (each sorted, the first k
// entries valid) are merged as a tree, pairs, then pairs of pairs; every lane loads from every list slot
// (clamped to the row's lists; entries past k are stale and zeroed), so the loads are issued together. Odd lists
// are read reversed (ascending); results are merged descending where they are a left operand, ascending where a
// right one. Then the tail (sampler.cpp:53-88) and the row's token.
__device__ __forceinline__ void merge_few_tail(const RowsArgs& a, int row, const uint64_t* cand, int k, uint32_t seq,
                                               int32_t draft, double u_row, int lane) {
    const uint64_t exp_tab = kExp2Tab[lane & 31];
    uint64_t lk[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) lk[s] = load_dev(&cand[(int64_t) min(s, a.segs - 1) * KCAP + ((s & 1) ? 63 - lane : lane)]);
#pragma unroll
    for (int s = 0; s < 8; ++s) lk[s] = (s < a.segs && ((s & 1) ? 63 - lane : lane) < k) ? lk[s] : 0ull;
    uint64_t lst = a.segs > 1 ? bitonic_stage<64, true>(max64(lk[0], lk[1]), lane) : lk[0];
    if (a.segs > 2) {
        const uint64_t m23 = bitonic_stage<64, false>(max64(lk[2], lk[3]), lane);
        if (a.segs > 4) {
            const uint64_t m45 = bitonic_stage<64, true>(max64(lk[4], lk[5]), lane);
            const uint64_t m67 = bitonic_stage<64, false>(max64(lk[6], lk[7]), lane);
            const uint64_t m0123 = bitonic_stage<64, true>(max64(lst, m23), lane);
            const uint64_t m4567 = bitonic_stage<64, false>(max64(m45, m67), lane);
            lst = bitonic_stage<64, true>(max64(m0123, m4567), lane);
        } else {
            lst = bitonic_stage<64, true>(max64(lst, m23), lane);
        }
    }
    const int kk = min(k, (int) __popcll(ballot(lst != 0ull && lane < k)));
    if (a.dbg_keys) a.dbg_keys[row * KCAP + lane] = lane < kk ? lst : 0ull;
    const int tok = sample_tail(lst, kk, a.p, u_row, exp_tab, lane, a.dbg_probs ? a.dbg_probs + row * KCAP : nullptr,
                                a.dbg_meta ? a.dbg_meta + row * 2 : nullptr);
    if (lane == 0) publish(a, row, tok, seq, draft);
}

// Loads this thread's logits of groups I0 <= i < I1: ids lb + 4*(i*WG + tid) + e.
//  * FULL: every group is a whole aligned float4 inside the row, read through the buffer resource `seg` (base =
//    logit lb) with one offset register for all groups;
//  * otherwise each float4 is checked against hi (NaN past it) and misaligned rows load scalars.
template <bool FULL, int WG, int EPT, int I0, int I1>
__device__ __forceinline__ void load_groups(float (&v)[EPT], bool vec, __amdgpu_buffer_rsrc_t seg,
                                            const float* __restrict__ L, int lb, int hi) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = I0; i < I1; ++i) {
        if constexpr (FULL) {
            const u32x4 f = __builtin_amdgcn_raw_buffer_load_b128(seg, tid * 16, i * WG * 16, kNonTemporal);
            v[4 * i + 0] = __uint_as_float(f[0]);
            v[4 * i + 1] = __uint_as_float(f[1]);
            v[4 * i + 2] = __uint_as_float(f[2]);
            v[4 * i + 3] = __uint_as_float(f[3]);
        } else {
            const int base = lb + 4 * (i * WG + tid);
            if (vec && base + 3 < hi) {
                const f32x4 f = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(L + base));
                v[4 * i + 0] = f[0];
                v[4 * i + 1] = f[1];
                v[4 * i + 2] = f[2];
                v[4 * i + 3] = f[3];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * i + e] = (base + e < hi) ? L[base + e] : __uint_as_float(0x7fc00000u);
            }
        }
    }
}

template <bool GREEDY, bool PENALIZE, bool FULL, int NW, int EPT>
__global__ __launch_bounds__(NW * 64) void rows_kernel(RowsArgs a) {
    constexpr int WG = NW * 64;
    constexpr int SEG = WG * EPT;
    constexpr int NV = EPT / 4;    // float4 per thread
    constexpr bool C16 = NW > 4;   // 16-bit history counts (segments of 16384 ids and more)
    static_assert(NW == 4 || NW == 16, "workgroup width");
    static_assert(!C16 || NV % 2 == 0, "half-segment windows");
    const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    // Work item of this workgroup. Workgroups are dealt round-robin to the 8 XCDs (workgroup i on XCD i % 8);
    // with xcd_map, XCD x takes a contiguous block of (row, segment) items, so a row's segments (and the reads
    // of its history) mostly share one L2. Padding workgroups leave before any synchronization.
    int item = blockIdx.x;
    if (a.xcd_map) {
        const int per = (a.n_rows * a.segs + 7) >> 3;
        item = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    }
    if (item >= a.n_rows * a.segs) return;
    // (uniform; readfirstlane keeps the row and the addresses derived from it in scalar registers)
    const int row = __builtin_amdgcn_readfirstlane(item / a.segs), seg = item - row * a.segs;
    const int lo = seg * SEG;
    const int hi = min(a.V, lo + SEG);
    // FULL (V >= SEG, aligned rows, V % 4 == 0): every workgroup reads SEG whole float4s; the row's last segment
    // is shifted down to end at V, so it also holds `skip` ids below lo (the previous segment's). Those take part
    // in the maximum and the bound (real logits of the row: a bound that k held logits reach is one that k logits
    // of the row reach, and a repeated maximum is harmless) but are never offered as candidates, so each id is
    // listed by one segment only. lb is the first id held.
    const int lb = FULL ? min(lo, a.V - SEG) : lo;
    const int skip = lo - lb;  // leading ids held but not owned (uniform)
    const float* __restrict__ L = a.logits + (int64_t) row * a.row_stride;
    const bool vec = ((a.row_stride & 3) == 0) && ((reinterpret_cast<uintptr_t>(a.logits) & 15u) == 0);
    const int k = a.p.k;
    uint64_t* seg_out = a.seg_cand + ((int64_t) row * a.segs + seg) * KCAP;
    // what the row's last workgroup will need from host memory (the pinned call block, for graph-replayed
    // steps), read now so that its latency is hidden behind the segment's
    // greedy rows as std::max_element (engine.cpp:414): the running maximum starts at the first logit and only
    // '<' replaces it, so a NaN there is the result; otherwise the result is sampler.cpp's greedy id
    const float l0 = (GREEDY && a.first_nan) ? L[0] : 0.0f;
    const bool nan_first = l0 != l0;
    // a bound other workgroups of the row published (large grids only): read before the logits arrive
    const uint64_t t_row =
        a.share_bounds ? __hip_atomic_load(&a.row_thr[row], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;

    // ---- one coalesced read of the segment: thread t holds ids lb + 4*(i*WG + t) + e, in three batches. With
    // penalties the row's raw history is prefetched (into registers) after the first groups of logits (its wait
    // covers those only: loads complete in order) and counted into the LDS table while the middle of the segment
    // is in flight; the last quarter is issued after the count, so the prefetched ids and the whole segment are
    // never held at once.
    const __amdgpu_buffer_rsrc_t seg_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(L + lb), (short) 0, SEG * 4, kRawBufferFlags);
    // 16-wave top-k segments take their bound from waves 0..7 (the early bound, below); its LDS counters are
    // cleared before the barrier that follows the first batch (without penalties: one float4 per thread)
    constexpr bool EARLY = !GREEDY && NW == 16;
    constexpr int Q1 = PENALIZE ? (NV >= 8 ? 2 : NV >= 2 ? 1 : 0) : EARLY ? 1 : NV;
    constexpr int Q3 = PENALIZE ? NV - NV / 4 : Q1;
    float v[EPT];
    RawHistory rh;
    bool wide = false;
    // Penalties that never raise a logit (rep >= 1, presence >= 0, frequency >= 0: penalized <= raw for every
    // id) are applied lazily. Greedy rows penalize a history logit when its raw value beats the running maximum;
    // top-k rows scan raw logits and penalize afterwards only the lane maxima and the logits that pass the bound.
    const bool late = !GREEDY && PENALIZE && a.p.lazy;
    // (the row's history bounds are read first: their latency overlaps the first batch and the table clearing)
    if (PENALIZE && a.hist_off) {
        rh.s0 = max(a.hist_off[row], 0);
        rh.s1 = max(a.hist_off[row + 1], rh.s0);
    }
    load_groups<FULL, WG, EPT, 0, Q1>(v, vec, seg_rsrc, L, lb, hi);
    if (PENALIZE) {
        // cleared whatever the table's width turns out to be (wide tables are cleared again per half)
        cnt_zero<WG>(C16 ? (hi - lb + 1) / 2 : hi - lb);
        if (tid == 0) {
            s_counted = 0;  // (ordered before every increment by the barrier below)
            if (EARLY) {
                s_arr[0] = s_arr[1] = s_arr[2] = s_arr[3] = 0;
                s_qready = 0;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        int4 hq[HR];
#pragma unroll
        for (int r = 0; r < HR; ++r) hq[r] = make_int4(-1, -1, -1, -1);
        if (a.hist_off) {
            const bool hv = (reinterpret_cast<uintptr_t>(a.hist_ids) & 15u) == 0;
            rh.b0 = hv ? min(rh.s1, (rh.s0 + 3) & ~3) : rh.s1;
            rh.b1 = hv ? max(rh.b0, rh.s1 & ~3) : rh.s1;
#pragma unroll
            for (int r = 0; r < HR; ++r) {
                const int j = rh.b0 + 4 * (r * WG + tid);
                if (j < rh.b1) hq[r] = *reinterpret_cast<const int4*>(a.hist_ids + j);
            }
        }
        // counts reach 65536 only with that many history ids in the row (extras included)
        const int extra = (a.extra_a ? PENDING_CAP : 0) + (a.extra_b ? VERIFY_MAX_ROWS : 0);
        wide = C16 && (a.count_wide != 0 || (rh.s1 - rh.s0) + extra >= 65536);
        // (the barrier comes before the rest of the segment: every wave reaches it having issued few loads; a
        // wave whose loads wait for issue slots would hold the others here)
        __syncthreads();  // table zeroed
        // Lazy 16-wave rows: waves 4..15, whose loads wait behind the first group's anyway, count before
        // issuing the middle batch, so that the table is complete (and the early bound can form) sooner.
        const bool count_first = late && NW == 16 && wave >= 4;
        if (!count_first) load_groups<FULL, WG, EPT, Q1, Q3>(v, vec, seg_rsrc, L, lb, hi);
        if (!wide) {
            count_history<WG, C16, true>(a, row, lb, hi, hq, rh, (int) threadIdx.x);
            // (before the last batch, for the same reason; late counts are first read after the scan, once
            // every wave has announced its count: LDS operations of a wave complete in order)
            if (!late) {
                __syncthreads();  // table complete
            } else {
                if (lane == 0) lds_raise(&s_counted, 1);
                __builtin_amdgcn_sched_barrier(0);  // (the last batch stays after the count)
            }
        }
        if (count_first) load_groups<FULL, WG, EPT, Q1, Q3>(v, vec, seg_rsrc, L, lb, hi);
    } else if (EARLY) {
        if (tid == 0) {
            s_arr[0] = s_arr[1] = s_arr[2] = s_arr[3] = 0;
            s_qready = 0;
        }
        __syncthreads();  // counters cleared
    }
    load_groups<FULL, WG, EPT, Q3, NV>(v, vec, seg_rsrc, L, lb, hi);
    const CallIn cin = wave == NW - 1 ? read_call<GREEDY>(a, row) : CallIn{0u, -1, 0.0};  // (to LDS below)
    // with penalties (16-bit or narrow tables) the counts are applied group by group as the logits are first
    // used (or lazily), below; wide counts are applied here, half a segment at a time
    const bool pen_now = PENALIZE && !wide && !a.p.lazy;
    const bool pen_lazy = PENALIZE && !wide && a.p.lazy;
    if (PENALIZE && wide) {
        if constexpr (C16) {
            // 32-bit counts over half a segment at a time, the history read again from memory
            const int4 none[HR] = {};
            const int mid = min(hi, lb + SEG / 2);
            cnt_zero<WG>(mid - lb);
            __syncthreads();
            count_history<WG, false, false>(a, row, lb, mid, none, rh, (int) threadIdx.x);
            __syncthreads();
            apply_counts<WG, EPT, false, FULL, 0, NV / 2>(v, lb, hi, lb, a.p);
            if (mid < hi) {
                __syncthreads();
                cnt_zero<WG>(hi - mid);
                __syncthreads();
                count_history<WG, false, false>(a, row, mid, hi, none, rh, (int) threadIdx.x);
                __syncthreads();
                apply_counts<WG, EPT, false, FULL, NV / 2, NV>(v, lb, hi, mid, a.p);
            }
        }
    }

    if (GREEDY) {
        // src/sampler.cpp:31-39: a thread's ids ascend with (i, e), so strict '>' keeps the lowest id.
        float best_v = -INFINITY;
        int best_id = 0;
        uint32_t cn[4] = {0u, 0u, 0u, 0u};  // lazy: group i+1's counts, read while group i is worked on
        if (pen_lazy) group_counts<WG, C16, FULL>(cn, 0, lb, hi, lb, best_v);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if (pen_now) apply_group<WG, EPT, C16, FULL>(v, i, lb, hi, lb, a.p);
            const uint32_t c[4] = {cn[0], cn[1], cn[2], cn[3]};
            if (pen_lazy && i + 1 < NV) group_counts<WG, C16, FULL>(cn, i + 1, lb, hi, lb, best_v);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float x = v[4 * i + e];
                if (x > best_v && c[e] != 0u) x = penalize(x, c[e], a.p);  // lazy: penalized <= raw
                if (x > best_v) {
                    best_v = x;
                    best_id = lb + 4 * (i * WG + tid) + e;
                }
            }
        }
        uint64_t key = best_v > -INFINITY ? mk_key(best_v, best_id) : 0ull;
        key = wave_max64(key, lane);
        if (lane == 0) s_red<NW>[wave] = key;
        if (wave == NW - 1 && lane == 0) s_cin = cin;
        __syncthreads();
        if (tid == 0) {
            uint64_t m = s_red<NW>[0];
#pragma unroll
            for (int o = 1; o < NW; ++o) m = max64(m, s_red<NW>[o]);
            store_dev(&seg_out[0], m);
        }
    } else {
        // ---- lower bound of the segment's k-th value: every lane contributes its largest logit (NaN counts as
        // -inf and never reaches a bound); the k-th largest of these lane maxima (logits at distinct positions)
        // is reached by at least k logits of the segment. Each wave sorts its lane maxima and keeps its top 64,
        // and the waves' lists are merged (in groups of four for 16 waves). The second largest, m2, is kept for
        // the filter, which skips a lane whose m2 falls below the bound (only its maximum can survive).
        // (canonicalized values: signaling NaNs quieted, so max ignores a NaN and med3 keeps m2, and every NaN fails
        // the filter's compares; med3(m1, m2, x) = max(m2, min(m1, x)) for m1 >= m2)
        float m1 = -INFINITY, m2 = -INFINITY;
        int s1 = 0;  // slot 4*i+e of m1 (its first occurrence)
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if (pen_now) apply_group<WG, EPT, C16, FULL>(v, i, lb, hi, lb, a.p);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float x = __builtin_canonicalizef(v[4 * i + e]);
                v[4 * i + e] = x;
                s1 = x > m1 ? 4 * i + e : s1;
                m2 = __builtin_amdgcn_fmed3f(m1, m2, x);
                m1 = __builtin_fmaxf(m1, x);
                // (kept as register updates: otherwise the compiler defers them and holds every partial maximum)
                asm volatile("" : "+v"(s1), "+v"(m2));
            }
        }
        // lazy: the lane's contribution to the bound is its maximum's penalized value (a logit of the lane
        // that reaches it); m2 stays raw, an upper bound of every other penalized logit of the lane
        if (pen_lazy) {
            // table complete: every wave has counted (each does so right after issuing its loads, whatever the
            // others do, so the wait ends; the bound on it is a guard only)
            bool counted = false;
            for (int spin = 0; spin < a.spin_limit && !counted; ++spin) {
                counted = lds_peek(&s_counted) >= NW;
                if (!counted) __builtin_amdgcn_s_sleep(1);
            }
            if (!counted && lane == 0) report_fault(a, FAULT_COUNT_WAIT);
            if (m1 > -INFINITY) {
                const int off = 4 * ((s1 >> 2) * WG + tid) + (s1 & 3);
                const uint32_t c = C16 ? (s_cnt[off >> 1] >> ((off & 1) << 4)) & 0xffffu : s_cnt[off];
                if (c != 0u) m1 = penalize(m1, c, a.p);
            }
        }
        uint32_t gl;
        if constexpr (NW == 4) {
            // 4 waves: each sorts its lane maxima, every wave merges the four lists
            s_mx<NW>[wave][lane] = sort32<true>(ord_f32(m1), lane);
            __syncthreads();
            gl = s_mx<NW>[0][lane];
#pragma unroll
            for (int o = 1; o < NW; ++o) gl = merge32(gl, s_mx<NW>[o][63 - lane], lane);
        } else {
            // 16 waves: the early bound, from the lane maxima of the first eg groups of four waves alone (waves
            // 0..7: 512 distinct logits of the segment, so still reached by k of them). Those waves receive their
            // logits first (loads issue wave by wave), so the bound is usually ready when the later waves finish
            // their scan, and they filter at once (measured on the 64-row batch: 0.75 µs less than with waves
            // 0..11 without penalties, 0.25 µs less with them, where waves 4..15 count the history first). Each
            // early wave sorts its lane maxima; the last of each group of four to arrive merges the group's lists,
            // the last group to finish merges the groups' and publishes the k-th value. No wave waits before it
            // has contributed, so every wait below ends.
            constexpr int eg = 2;
            if (wave < 4 * eg) {
                const int g = wave >> 2;
                s_mx<NW>[wave][lane] = sort32<true>(ord_f32(m1), lane);
                int n = 0;
                if (lane == 0) n = lds_raise(&s_arr[g], 1);
                if (rdlanei(n, 0) == 3) {
                    gl = s_mx<NW>[4 * g][lane];
#pragma unroll
                    for (int o = 1; o < 4; ++o) gl = merge32(gl, s_mx<NW>[4 * g + o][63 - lane], lane);
                    s_mx4<NW>[g][lane] = gl;
                    n = 0;
                    if (lane == 0) n = lds_raise(&s_arr[3], 1);
                    if (rdlanei(n, 0) == eg - 1) {
#pragma unroll
                        for (int o = 0; o < 3; ++o)
                            if (o < eg && o != g) gl = merge32(gl, s_mx4<NW>[o][63 - lane], lane);
                        const uint32_t qw = (uint32_t) rdlanei((int) gl, k - 1);  // all lanes active
                        if (lane == 0) {
                            s_qe = qw;
                            lds_publish(&s_qready, 1);
                        }
                    }
                }
            }
            // (the bound on the wait is a guard only: if it expires the launch reports a fault)
            bool ready = false;
            for (int spin = 0; spin < a.spin_limit && !ready; ++spin) {
                ready = lds_peek(&s_qready) != 0;
                if (!ready) __builtin_amdgcn_s_sleep(1);
            }
            if (!ready && lane == 0) report_fault(a, FAULT_BOUND_WAIT);
            gl = s_qe;
        }
        const uint32_t q = NW == 4 ? (uint32_t) rdlanei((int) gl, k - 1) : gl;  // all lanes active
        const float t_f = fmaxf(floor32(q), floor64(t_row));

        // ---- filter: survivors go to the wave's LDS region. A lane whose second largest (raw) logit is below the
        // bound holds at most one survivor, its maximum at slot s1 (penalized, lazily), offered directly; the other
        // lanes' logits are tested one by one (lazily penalized when their raw value passes).
        WaveCollect<NW> w;
        const bool multi = m2 >= t_f;
        {
            const int slot = 4 * ((s1 >> 2) * WG + tid) + (s1 & 3);
            const bool pass = !multi && m1 >= t_f && slot >= skip;
            if (ballot(pass)) {
                const uint64_t key = mk_key_num(m1, lb + slot);
                w.offer(wave, pass && key > t_row, key);
            }
        }
        // Lanes with more: one at a time, the lane's EPT logits pass through the wave's (idle) list row in LDS,
        // so that every lane of the wave tests one of them.
        float* const buf = reinterpret_cast<float*>(&s_list<NW>[wave][0]);
        static_assert(EPT * sizeof(float) <= sizeof(s_list<NW>[0]), "transpose row");
        for (uint64_t mm = ballot(multi); mm != 0ull; mm &= mm - 1) {
            const int l = (int) __builtin_ctzll(mm);  // uniform
            if (lane == l) {
#pragma unroll
                for (int i = 0; i < NV; ++i)
                    *reinterpret_cast<float4*>(buf + 4 * i) = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
            }
            __builtin_amdgcn_wave_barrier();
            const int sl = min(lane, EPT - 1);  // slot of the source lane
            float x = buf[sl];
            const int off = 4 * ((sl >> 2) * WG + wave * 64 + l) + (sl & 3);  // its id - lb
            if (pen_lazy && x >= t_f) {
                const uint32_t c = C16 ? (s_cnt[off >> 1] >> ((off & 1) << 4)) & 0xffffu : s_cnt[off];
                if (c != 0u) x = penalize(x, c, a.p);  // lazy: test the penalized value
            }
            const uint64_t key = mk_key_num(x, lb + off);  // (used only where x passes: not NaN)
            w.offer(wave, lane < EPT && x >= t_f && off >= skip && key > t_row, key);
            __builtin_amdgcn_wave_barrier();
        }
        uint64_t lst;
        if (wave == NW - 1 && lane == 0) s_cin = cin;  // (read by wave 0 after wg_select's barrier)
        if (!wg_select<NW>(w, lane, wave, &lst))
            lst = segment_slow<NW, SEG, C16>(a, L, row, lo, hi, lb, PENALIZE, wide, rh, t_row, lane, wave);
        if (wave == 0) {
            if (lane < k) store_dev(&seg_out[lane], lst);
            if (a.share_bounds) {
                const uint64_t own = rdlane64(lst, k - 1);
                if (lane == 0 && own > t_row) atomicMax((unsigned long long*) &a.row_thr[row], (unsigned long long) own);
            }
        }
    }

    // ---- the last workgroup of the row merges the segment results. Hand-off: the segment results above were
    // written (by wave 0, which also takes the ticket) with device-scope stores; the wave waits for them to be
    // acknowledged before the ticket increment, and the last workgroup reads them with device-scope loads after
    // its increment returned. With few segments wave 0 does all of it alone (no barrier).
    const uint64_t* cand = a.seg_cand + (int64_t) row * a.segs * KCAP;
    if (GREEDY ? a.segs <= 64 : a.segs <= 8) {
        if (wave != 0) return;
        const CallIn c0 = s_cin;
        const uint32_t seq = c0.seq;
        const int32_t draft = c0.draft;
        const double u_row = c0.u;
        wait_stores();
        uint32_t prev = 0u;
        if (lane == 0) prev = atomicAdd(&a.row_ticket[row], 1u);
        if ((uint32_t) rdlanei((int) prev, 0) != (uint32_t) (a.segs - 1)) return;
        if (GREEDY) {
            uint64_t m = load_dev(&cand[(int64_t) min(lane, a.segs - 1) * KCAP]);
            m = wave_max64(lane < a.segs ? m : 0ull, lane);
            if (lane == 0) {
                if (a.dbg_meta) {
                    a.dbg_meta[row * 2] = 0;
                    a.dbg_meta[row * 2 + 1] = 0;
                }
                publish(a, row, nan_first ? 0 : m ? key_id(m) : 0, seq, draft);  // all -inf / NaN: id 0
            }
            return;
        }
        merge_few_tail(a, row, cand, k, seq, draft, u_row, lane);
        return;
    }
    __syncthreads();
    if (tid == 0) {
        wait_stores();
        const uint32_t prev = atomicAdd(&a.row_ticket[row], 1u);
        s_last = (prev == (uint32_t) (a.segs - 1));
    }
    __syncthreads();
    if (!s_last) return;
    const CallIn c0 = s_cin;
    const uint32_t seq = c0.seq;
    const int32_t draft = c0.draft;
    const double u_row = c0.u;

    if (GREEDY) {
        uint64_t m = 0ull;
        for (int s = tid; s < a.segs; s += WG) m = max64(m, load_dev(&cand[(int64_t) s * KCAP]));
        m = wave_max64(m, lane);
        if (lane == 0) s_red<NW>[wave] = m;
        __syncthreads();
        if (tid != 0) return;
#pragma unroll
        for (int o = 0; o < NW; ++o) m = max64(m, s_red<NW>[o]);
        if (a.dbg_meta) {
            a.dbg_meta[row * 2] = 0;
            a.dbg_meta[row * 2 + 1] = 0;
        }
        publish(a, row, nan_first ? 0 : m ? key_id(m) : 0, seq, draft);  // all -inf / NaN: id 0
        return;
    }

    // Lower bound of the row's k-th value from the heads of the segment lists: H = the first J = ceil(k/segs)
    // entries of every list (J*segs >= k distinct logits). With |H| <= 64 the bound is the k-th largest value in H;
    // otherwise H is dealt round-robin to the waves and the bound is the smallest of the waves'
    // ceil(k/NW)-th largest values. Either way at least k logits reach it, so the row's top-k are among the list
    // entries at or above it. Up to 16*NW lists stay in registers (16 per wave) while the bound is formed.
    constexpr int RB = 16;
    const int J = (k + a.segs - 1) / a.segs;
    const int nH = min(a.segs * J, WG);
    const bool one = nH <= 64;
    const int h = one ? (wave == 0 ? lane : WG) : lane * NW + wave;
    // (loads clamped to the row's lists and issued together; what is out of range is zeroed after)
    const uint64_t exp_tab = kExp2Tab[lane & 31];
    const int hc = min(h, nH - 1);
    uint64_t hv = load_dev(&cand[(int64_t) (hc / J) * KCAP + hc % J]);
    const bool inreg = a.segs <= NW * RB;
    uint64_t key[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) key[r] = load_dev(&cand[(int64_t) min(wave + NW * r, a.segs - 1) * KCAP + lane]);
#pragma unroll
    for (int r = 0; r < RB; ++r) key[r] = (inreg && wave + NW * r < a.segs && lane < k) ? key[r] : 0ull;
    hv = h < nH ? hv : 0ull;
    const uint32_t sv = sort32<true>((uint32_t) (hv >> 32), lane);
    const uint32_t qw = (uint32_t) rdlanei((int) sv, (one ? k : (k + NW - 1) / NW) - 1);  // all lanes active
    if (lane == 0) s_q<NW>[wave] = (one && wave != 0) ? 0xffffffffu : qw;
    __syncthreads();
    uint32_t qm = s_q<NW>[0];
#pragma unroll
    for (int o = 1; o < NW; ++o) qm = min(qm, s_q<NW>[o]);
    const uint64_t ts = (uint64_t) qm << 32;
    WaveCollect<NW> w;
    if (inreg) {
#pragma unroll
        for (int r = 0; r < RB; ++r) w.offer(wave, key[r] != 0ull && key[r] >= ts, key[r]);
    } else {
        for (int s0 = wave; s0 < a.segs; s0 += NW * RB) {
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const int s = s0 + NW * r;
                key[r] = (s < a.segs && lane < k) ? load_dev(&cand[(int64_t) s * KCAP + lane]) : 0ull;
            }
#pragma unroll
            for (int r = 0; r < RB; ++r) w.offer(wave, key[r] != 0ull && key[r] >= ts, key[r]);
        }
    }
    uint64_t lst;
    if (!wg_select<NW>(w, lane, wave, &lst)) {
        __syncthreads();
        lst = merge_slow<NW>(cand, a.segs, k, ts, lane, wave);
    }
    if (wave != 0) return;
    const int kk = min(k, (int) __popcll(ballot(lst != 0ull && lane < k)));
    if (a.dbg_keys) a.dbg_keys[row * KCAP + lane] = lane < kk ? lst : 0ull;
    const int tok = sample_tail(lst, kk, a.p, u_row, exp_tab, lane, a.dbg_probs ? a.dbg_probs + row * KCAP : nullptr,
                                a.dbg_meta ? a.dbg_meta + row * 2 : nullptr);
    if (lane == 0) publish(a, row, tok, seq, draft);
}

__global__ void noop_kernel_impl(int) {}

__global__ void expf_table_kernel(uint32_t lo, long long n, float* out) {
    const long long i = (long long) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = expf_glibc(__uint_as_float(lo + (uint32_t) i));
}

// ---------------------------------------------------------------------------------------------------------
// Wide top-k (k above what the mid path holds, up to no limit; src/sampler.cpp:42-51): keys of every logit, one
// device-wide radix sort (kls_sort.hip), then the tail over the sorted keys.

constexpr int WIDE_WG = 256;
// ids per keys workgroup with penalties: 4,096 (32-bit history counts: 16 KB of LDS; every workgroup scans the
// row's history)
constexpr int WIDE_SEG = 4096;

// Keys of ids [lo, hi) of one row (workgroup = (row, segment)), every history count applied to its logit.
// TPW: sort tiles per workgroup (1: tiles of 4,096 keys, 2: of 2,048), whose counts of the sort's first digit the
// workgroup writes as the sort's histogram kernel would (its first histogram launch is then saved); 0: none (tiles
// of 8,192 keys span two workgroups).
template <int TPW>
__global__ __launch_bounds__(WIDE_WG) void wide_keys_kernel(RowsArgs a, WideArgs w) {
    static_assert(TPW == 0 || (TPW <= 2 && WIDE_SEG / TPW >= SORT_TILE_MIN), "whole sort tiles per workgroup");
    __shared__ uint32_t h[TPW > 0 ? TPW : 1][256];
    const int segs = (a.V + WIDE_SEG - 1) / WIDE_SEG;
    const int row = (int) blockIdx.x / segs, seg = (int) blockIdx.x - row * segs;
    const int lo = seg * WIDE_SEG, hi = min(a.V, lo + WIDE_SEG);
    const float* __restrict__ L = a.logits + (int64_t) row * a.row_stride;
    {
        RawHistory rh;
        if (a.hist_off) {
            rh.s0 = max(a.hist_off[row], 0);
            rh.s1 = max(a.hist_off[row + 1], rh.s0);
            const bool hv = (reinterpret_cast<uintptr_t>(a.hist_ids) & 15u) == 0;
            rh.b0 = hv ? min(rh.s1, (rh.s0 + 3) & ~3) : rh.s1;
            rh.b1 = hv ? max(rh.b0, rh.s1 & ~3) : rh.s1;
        }
        const int4 none[HR] = {};
        cnt_zero<WIDE_WG>(hi - lo);
        if (TPW > 0)
            for (int i = (int) threadIdx.x; i < TPW * 256; i += WIDE_WG) (&h[0][0])[i] = 0u;
        __syncthreads();
        count_history<WIDE_WG, false, false>(a, row, lo, hi, none, rh, (int) threadIdx.x);
        __syncthreads();
    }
    const int ib = w.id_bits;

    const uint32_t idm = (1u << ib) - 1u;
    uint64_t* __restrict__ out = w.keys + (int64_t) row * a.V;
    // the thread's logits are loaded together (a loop of load, wait, store took one memory latency per id)
    constexpr int PT = WIDE_SEG / WIDE_WG;
    float v[PT];
#pragma unroll
    for (int j = 0; j < PT; ++j) {
        const int id = lo + (int) threadIdx.x + j * WIDE_WG;
        v[j] = id < hi ? L[id] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < PT; ++j) {
        const int id = lo + (int) threadIdx.x + j * WIDE_WG;
        if (id < hi) {
            float x = v[j];
            const uint32_t c = s_cnt[id - lo];
            if (c != 0u) x = penalize(x, c, a.p);
            const uint32_t o = ord_f32(x);
            out[id] = ((uint64_t) o << ib) | (uint64_t) (~(uint32_t) id & idm);
            // (the tile of id within the workgroup is j * WIDE_WG / tile: a constant of the unrolled loop)
            if (TPW > 0) atomicAdd(&h[TPW > 1 ? j * WIDE_WG * TPW / WIDE_SEG : 0][255u - (o & 255u)], 1u);
        }
    }
    if (TPW > 0) {
        __syncthreads();
        constexpr int TILE = WIDE_SEG / (TPW > 0 ? TPW : 1);
        const int tiles = (a.V + TILE - 1) / TILE;  // the row's tiles
        for (int i = (int) threadIdx.x; i < TPW * 256; i += WIDE_WG) {
            const int t = seg * TPW + i / 256;
            if (t < tiles) w.counts[((size_t) row * tiles + t) * 256 + (i & 255)] = (&h[0][0])[i];
        }
    }
}

// Keys of one sort tile of one row (TILE ids) without penalties, as wide_keys_kernel writes them, and the tile's
// counts of the sort's first digit (bits [id_bits, id_bits + 8) of a key: the value image's low 8 bits), laid out
// as the sort's histogram kernel lays them out (counts[(row * tiles + tile) * 256 + 255 - digit]), so that the
// sort's first histogram launch, and its read of every key, are saved (one row of 248,320 ids: 82.3 -> 80.2 us per
// step; 4 rows 117.9 -> 116.1 us). PT = TILE / 1024 logits per thread (2 to 8), loaded together.
constexpr int WKH_WG = 1024;
template <int TILE>
__global__ __launch_bounds__(WKH_WG) void wide_keys_hist_kernel(RowsArgs a, WideArgs w) {
    constexpr int PT = TILE / WKH_WG;
    __shared__ uint32_t h[256];
    const int tid = (int) threadIdx.x;
    const int tiles = (a.V + TILE - 1) / TILE;
    const int row = (int) blockIdx.x / tiles, lo = ((int) blockIdx.x - row * tiles) * TILE;
    const int n = min(TILE, a.V - lo);
    const float* __restrict__ L = a.logits + (int64_t) row * a.row_stride + lo;
    float v[PT];
#pragma unroll
    for (int j = 0; j < PT; ++j) {
        const int i = tid + j * WKH_WG;
        v[j] = i < n ? L[i] : 0.0f;
    }
    if (tid < 256) h[tid] = 0u;
    __syncthreads();
    const int ib = w.id_bits;
    const uint32_t idm = (1u << ib) - 1u;
    uint64_t* __restrict__ out = w.keys + (int64_t) row * a.V + lo;
#pragma unroll
    for (int j = 0; j < PT; ++j) {
        const int i = tid + j * WKH_WG;
        if (i < n) {
            const uint32_t o = ord_f32(v[j]);
            out[i] = ((uint64_t) o << ib) | (uint64_t) (~(uint32_t) (lo + i) & idm);
            atomicAdd(&h[255u - (o & 255u)], 1u);
        }
    }
    __syncthreads();
    if (tid < 256) w.counts[(size_t) blockIdx.x * 256 + tid] = h[tid];
}

// The tail over sorted candidates (sorted_tail below) runs on one workgroup of TAIL_WG threads per row.
constexpr int TAIL_WG = 1024;
__shared__ int s_wide_n;  // kk, then the min-p length

// ---- Exact parallel replay of a sequential double sum: acc <- RN(acc + t_i), i = 0, 1, ... in order.
// While acc > 0 stays in one binade [2^E, 2^(E+1)) every value on the way is A * u with u = 2^(E-52) and A an
// integer in [2^52, 2^53), and RN(A*u + t) = (A + d)*u where, writing t/u = f + phi (f integer, 0 <= phi < 1),
// d = f when phi < 1/2, f + 1 when phi > 1/2, and at a tie (phi = 1/2) whichever of f, f + 1 makes A + d even.
// So each term is a map of the parity of A: (d for parity 0, d for parity 1, parity after each). Maps compose
// associatively, so a workgroup scans a block of terms at a time (replay_sum: TAIL_WG threads, one or two terms
// each; the wide tail's map kernels: a chunk of WT_CHUNK) and knows every A on the way. A term
// whose exact sum could leave the binade (A + f < 2^52, or A + f >= 2^53 - 1, or t/u huge) is added with the real
// double addition instead, and the scan restarts after it in the new binade; so is every term while acc is 0 or
// subnormal. Identical results to the sequential loop, in one workgroup step per block and per binade change.
// Increments are integers held in doubles: while no term leaves the binade every increment and every partial
// count is below 2^53 in magnitude, so the double arithmetic on them is exact (and full rate, with no integer
// conversions); past a term that leaves the binade the values are discarded anyway.
struct ParMap {
    double d0, d1;  // increments (in units of u) for incoming parity 0 / 1
    uint32_t p;     // bit 0: parity after, from parity 0; bit 1: from parity 1
};

__device__ __forceinline__ ParMap par_identity() { return ParMap{0.0, 0.0, 2u}; }

// Parity of an integer-valued double below 2^53 in magnitude (0 or 1).
__device__ __forceinline__ uint32_t dparity(double x) { return (uint32_t) (x - 2.0 * floor(0.5 * x)); }

// e first, then l
__device__ __forceinline__ ParMap par_compose(const ParMap& e, const ParMap& l) {
    const uint32_t e0 = e.p & 1u, e1 = (e.p >> 1) & 1u, l0 = l.p & 1u, l1 = (l.p >> 1) & 1u;
    ParMap c;
    c.d0 = e.d0 + (e0 ? l.d1 : l.d0);
    c.d1 = e.d1 + (e1 ? l.d1 : l.d0);
    c.p = (e0 ? l1 : l0) | ((e1 ? l1 : l0) << 1);
    return c;
}

// A map moved across lanes by DPP control CTRL (rows ROWS enabled); lanes with no source (or a disabled row)
// get the identity map.
template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_d0(double x) {
    const uint64_t v = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) (uint32_t) v, CTRL, ROWS, 0xf, false);
    const uint32_t hi = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) (uint32_t) (v >> 32), CTRL, ROWS, 0xf, false);
    return __builtin_bit_cast(double, ((uint64_t) hi << 32) | lo);  // (0.0 where there is no source)
}

template <int CTRL, int ROWS>
__device__ __forceinline__ ParMap dpp_map(const ParMap& m) {
    return ParMap{dpp_d0<CTRL, ROWS>(m.d0), dpp_d0<CTRL, ROWS>(m.d1),
                  (uint32_t) __builtin_amdgcn_update_dpp(2, (int) m.p, CTRL, ROWS, 0xf, false)};
}

// Inclusive scan of the maps across lanes in lane order (earlier lanes' terms first): row_shr 1, 2, 4, 8 within
// rows of 16, then row_bcast 15 and 31 (as wave_scan_f64). ROWS16: lanes 0..15 only (a scan of one row).
template <bool ROWS16>
__device__ __forceinline__ ParMap wave_scan_map(ParMap x) {
    x = par_compose(dpp_map<0x111, 0xf>(x), x);
    x = par_compose(dpp_map<0x112, 0xf>(x), x);
    x = par_compose(dpp_map<0x114, 0xf>(x), x);
    x = par_compose(dpp_map<0x118, 0xf>(x), x);
    if (!ROWS16) {
        x = par_compose(dpp_map<0x142, 0xa>(x), x);
        x = par_compose(dpp_map<0x143, 0xc>(x), x);
    }
    return x;
}

__device__ __forceinline__ ParMap rdlane_map(const ParMap& m, int l) {
    return ParMap{rdlaned(m.d0, l), rdlaned(m.d1, l), (uint32_t) __builtin_amdgcn_readlane((int) m.p, l)};
}

__shared__ ParMap s_rp_wave[TAIL_WG / 64];
__shared__ int s_rp_first;
__shared__ double s_rp_acc;
__shared__ int s_rp_next, s_rp_stop;

// The map of one term t in the binade of 2^E (f: its integer part in units of u; cross: too large to map: any
// |t/u| >= 2^53 takes the sum out of the binade).
__device__ __forceinline__ ParMap term_map(double t, int E, double* f, bool* cross) {
    const double q = ldexp(t, 52 - E);
    ParMap m = par_identity();
    *f = 0.0;
    *cross = false;
    if (!(fabs(q) < 0x1p53)) {
        *cross = true;  // (handled by the real addition; the map is not used past it)
        return m;
    }
    const double fl = floor(q);
    *f = fl;
    const double ph = q - fl;  // exact
    const uint32_t pf = dparity(fl);
    if (ph == 0.5) {
        m.d0 = fl + (double) pf;          // (A + d even from either parity)
        m.d1 = fl + (double) (1u - pf);
        m.p = 0u;
    } else {
        const double d = fl + (ph > 0.5 ? 1.0 : 0.0);
        const uint32_t pd = ph > 0.5 ? 1u - pf : pf;
        m.d0 = m.d1 = d;
        m.p = pd | ((1u - pd) << 1);
    }
    return m;
}

// Replays the chain over t[0..n) from `acc` with the whole workgroup (every thread calls it, uniformly);
// stop(acc, i) is evaluated on each partial result after term i, and the first i for which it holds ends the
// chain (returned in *stopped, else -1). Returns the last partial result.
// RP_PT terms per thread in one block: thread tid loads RP_PT consecutive terms into registers (the loads issued
// together, so a block waits for one memory latency, not one per term), composes their maps, and the workgroup
// scans the threads' maps, so a block covers TAIL_WG * RP_PT terms with one scan and two barriers; each thread
// then walks its own terms from the scanned prefix to find the first that leaves the binade or meets the stop.
// 1 suits chains of at most TAIL_WG terms (no serial walk: the mid path's tail and the wide tail's chunks), 2
// chains of up to 2 * TAIL_WG terms.
// NEG: the chain adds -t_i (the draw's subtractions) instead of t_i.
template <int RP_PT, bool NEG = false, typename F>
__device__ double replay_sum(const double* __restrict__ t, int n, double acc, F stop, int* stopped) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr double TWO52 = 0x1p52, TWO53 = 0x1p53;
    int i = 0, st = -1;
    while (i < n) {
        if (!(acc >= 0x1p-1000 && acc <= 0x1.fffffffffffffp+1023)) {
            // zero, negative, subnormal, tiny, infinite or NaN: one real addition (every thread the same)
            acc = __dadd_rn(acc, NEG ? -t[i] : t[i]);
            if (stop(acc, i)) {
                st = i;
                break;
            }
            ++i;
            continue;
        }
        int E;
        (void) frexp(acc, &E);  // acc in [2^(E-1), 2^E)
        E -= 1;
        const double u = ldexp(1.0, E - 52);
        const double A0 = ldexp(acc, 52 - E);  // (an integer in [2^52, 2^53))
        const uint32_t pi0 = dparity(A0);
        const int j0 = i + tid * RP_PT;
        // a wave past the block's terms (uniform in the wave) loads, maps and walks nothing: it holds
        // identities and takes the barriers and the block's total with the others
        const bool live = i + wave * 64 * RP_PT < n;
        double tv[RP_PT];  // this thread's terms (addresses clamped to the chain; terms past it are not used)
        ParMap M = par_identity();
        if (live) {
#pragma unroll
            for (int q = 0; q < RP_PT; ++q) tv[q] = NEG ? -t[min(j0 + q, n - 1)] : t[min(j0 + q, n - 1)];
            // the composed map of this thread's terms
#pragma unroll
            for (int q = 0; q < RP_PT; ++q) {
                double f;
                bool c;
                const ParMap m = term_map(tv[q], E, &f, &c);
                if (j0 + q < n) M = par_compose(M, m);
            }
        }
        // workgroup scan of the threads' maps: each wave's (DPP), then the waves' totals (a 16-lane DPP scan
        // that every wave runs on the totals it reads back)
        ParMap x = par_identity(), xe = par_identity();
        if (live) {
            x = wave_scan_map<false>(M);
            xe = dpp_map<0x138, 0xf>(x);  // wave_shr:1: the maps before this lane (lane 0: identity)
        }
        if (lane == 63) s_rp_wave[wave] = x;
        if (tid == 0) s_rp_first = 0x7fffffff;
        __syncthreads();
        const ParMap wt = wave_scan_map<true>(lane < TAIL_WG / 64 ? s_rp_wave[lane & (TAIL_WG / 64 - 1)] : par_identity());
        const ParMap pre = wave == 0 ? par_identity() : rdlane_map(wt, wave - 1);
        const ParMap tot_all = rdlane_map(wt, TAIL_WG / 64 - 1);
        // this thread's terms in order, from the maps of every term before them in this block
        ParMap X = par_compose(pre, xe);
        int hq = -1;
        bool h_cross = false;
        double h_A = 0.0, h_t = 0.0, h_nxt = 0.0;
#pragma unroll
        for (int q = 0; q < RP_PT; ++q) {
            const int j = j0 + q;
            if (live && hq < 0 && j < n) {
                const double tj = tv[q];
                double f;
                bool cross;
                const ParMap m = term_map(tj, E, &f, &cross);
                const double Aj = A0 + (pi0 ? X.d1 : X.d0);
                const uint32_t pij = pi0 ? ((X.p >> 1) & 1u) : (X.p & 1u);
                const double dj = pij ? m.d1 : m.d0;
                if (!cross) cross = (Aj + f < TWO52) || (Aj + f >= TWO53 - 1.0);
                const double nxt = (Aj + dj) * u;  // (exact when no earlier term crossed)
                if (cross || stop(nxt, j)) {
                    hq = q;
                    h_cross = cross;
                    h_A = Aj;
                    h_t = tj;
                    h_nxt = nxt;
                } else {
                    X = par_compose(X, m);
                }
            }
        }
        if (hq >= 0) atomicMin(&s_rp_first, j0 + hq - i);
        __syncthreads();
        const int first = s_rp_first;
        if (first == 0x7fffffff) {
            // no term left the binade or stopped: the block's total
            acc = (A0 + (pi0 ? tot_all.d1 : tot_all.d0)) * u;
            i += TAIL_WG * RP_PT;
        } else {
            if (hq >= 0 && j0 + hq - i == first) {
                // (the thread that holds the first such term)
                const int j = j0 + hq;
                double r;
                int s2 = -1;
                if (h_cross) {
                    r = __dadd_rn(h_A * u, h_t);
                    if (stop(r, j)) s2 = j;
                } else {
                    r = h_nxt;
                    s2 = j;
                }
                s_rp_acc = r;
                s_rp_next = j + 1;
                s_rp_stop = s2;
            }
            __syncthreads();
            acc = s_rp_acc;
            i = s_rp_next;
            st = s_rp_stop;
            if (st >= 0) break;
        }
        __syncthreads();  // (the LDS words are rewritten by the next block)
    }
    *stopped = st;
    return acc;
}

// Test hook: replay_sum over t[0..n) from acc0 (2 terms per thread above TAIL_WG terms, as the wide tail's
// replayed chunks, else 1, as the mid path's tail); mode 0 never stops, 1 stops at acc >= thr, 2 at acc <= 0.
// out[0] = the result, out[1] = the stop index (-1: none).
__global__ __launch_bounds__(TAIL_WG) void sum_replay_kernel(const double* t, int n, double acc0, int mode, double thr,
                                                             double* out) {
    int st;
    const auto stop = [mode, thr](double acc, int) { return mode == 1 ? acc >= thr : mode == 2 ? acc <= 0.0 : false; };
    // (the tails' choices of terms per thread)
    const double r = n > TAIL_WG ? replay_sum<2>(t, n, acc0, stop, &st) : replay_sum<1>(t, n, acc0, stop, &st);
    if (threadIdx.x == 0) {
        out[0] = r;
        out[1] = (double) st;
    }
}

// ---- Exact parallel forms of the tail's sums (one candidate per thread). The reference's chains add floats (e_i,
// then p_i) in double. Every float term is a multiple of 2^g, g = the exponent of the least positive term - 23
// (2^-149 for a subnormal least term); while a partial sum stays below 2^(g + 53) it is a multiple of 2^g with at
// most 53 significant bits, so it is exact. Hence, when the whole sum is below 2^(g + 53), every partial sum in
// any order is exact: the total is a tree reduction and the cumulative sums are a prefix scan. The test uses the
// tree total with a factor-two margin (its rounding error, when there is any, is far below that).
__shared__ double s_tx_sum[TAIL_WG / 64], s_tx_min[TAIL_WG / 64], s_tx_tot[TAIL_WG / 64], s_tx_pmin[TAIL_WG / 64];
__shared__ int s_tx_mp[TAIL_WG / 64], s_tx_tp[TAIL_WG / 64], s_tx_dr[TAIL_WG / 64];

// Least positive x across the wave (+inf when none).
__device__ __forceinline__ double wave_min_pos(double x, int lane) {
    uint64_t b = __builtin_bit_cast(uint64_t, x > 0.0 ? x : (double) INFINITY);
    b = min64(b, xor_lane64<32>(b, lane));  // (positive doubles order as their bit patterns)
    b = min64(b, xor_lane64<16>(b, lane));
    b = min64(b, xor_lane64<8>(b, lane));
    b = min64(b, xor_lane64<4>(b, lane));
    b = min64(b, xor_lane64<2>(b, lane));
    b = min64(b, xor_lane64<1>(b, lane));
    return __builtin_bit_cast(double, b);
}

// The condition above for float terms whose least positive value is mn and whose tree total is tot.
__device__ __forceinline__ bool sums_exact(double mn, double tot) {
    if (!(mn < (double) INFINITY)) return true;  // no positive term: every partial sum is 0
    int e;
    (void) frexp(mn, &e);                        // mn in [2^(e-1), 2^e)
    const int g = max(e - 1 - 23, -149);
    return tot < ldexp(1.0, g + 52);
}

// The tail's sums with one candidate per thread (kk <= TAIL_WG, t[i] = e_i), four barriers: the softmax total
// and its least term; p_i, the min-p cut, the cumulative sums, their total and least term; the top-p stop
// (t[i] <- cum_i); the draw. Returns the drawn candidate with *n_kept and this thread's p_i, or -1 (t untouched)
// when a chain is not exact in every order and must be replayed. The exactness of the cumulative chain is
// judged over all kk terms, which covers the kept prefix.
// Waves past the candidates (wave * 64 >= kk) only post neutral values (sum 0, least term +inf, no index) and
// take the barriers and the workgroup-wide decisions with the others; the caller uses the result on wave 0.
__device__ int tail_exact(double* t, int kk, const SamplingParams& p, double u, int lane, int wave, int* n_kept,
                          float* p_mine) {
    const int tid = (int) threadIdx.x;
    const bool in = tid < kk;
    const bool live = wave * 64 < kk;  // (uniform in the wave)
    double e = 0.0;
    if (live) {
        e = in ? t[tid] : 0.0;
        const double sw = wave_sum_f64(e, lane), mw = wave_min_pos(e, lane);
        if (lane == 0) {
            s_tx_sum[wave] = sw;
            s_tx_min[wave] = mw;
        }
    } else if (lane == 0) {
        s_tx_sum[wave] = 0.0;
        s_tx_min[wave] = (double) INFINITY;
    }
    __syncthreads();
    double sum = 0.0, mn = (double) INFINITY;
#pragma unroll
    for (int w = 0; w < TAIL_WG / 64; ++w) {
        sum += s_tx_sum[w];
        mn = fmin(mn, s_tx_min[w]);
    }
    if (!sums_exact(mn, sum)) return -1;
    // p_i (:60) and min-p (:62-68): the first i >= 1 with p_i < p_0 * min_p ends the list
    float pf = 0.0f;
    double cw = 0.0;
    if (live) {
        pf = in ? __double2float_rn(__ddiv_rn(e, sum)) : 0.0f;
        const float thr = __fmul_rn(__double2float_rn(__ddiv_rn(t[0], sum)), p.min_p);
        const uint64_t bm = ballot(p.min_p > 0.0f && in && tid >= 1 && !(pf >= thr));
        const double x = in ? (double) pf : 0.0;
        cw = wave_scan_f64(x);
        const double tw = rdlaned(cw, 63), mw = wave_min_pos(x, lane);
        if (lane == 0) {
            s_tx_tot[wave] = tw;
            s_tx_pmin[wave] = mw;
            s_tx_mp[wave] = bm ? wave * 64 + __builtin_ctzll(bm) : 0x7fffffff;
        }
    } else if (lane == 0) {
        s_tx_tot[wave] = 0.0;
        s_tx_pmin[wave] = (double) INFINITY;
        s_tx_mp[wave] = 0x7fffffff;
    }
    __syncthreads();
    double before = 0.0, tot = 0.0, pmn = (double) INFINITY;
    int n = kk;
#pragma unroll
    for (int w = 0; w < TAIL_WG / 64; ++w) {
        const double v = s_tx_tot[w];
        before += w < wave ? v : 0.0;
        tot += v;
        pmn = fmin(pmn, s_tx_pmin[w]);
        n = min(n, s_tx_mp[w]);
    }
    if (!sums_exact(pmn, tot)) return -1;
    // top-p (:69-79): the first i with cum_i >= top_p keeps i + 1; the draw total (:80-81) is cum_{n-1}
    const double cum = before + cw;
    if (live) {
        if (in) t[tid] = cum;  // (every thread read e_0 before the barrier above)
        const uint64_t bt = ballot(tid < n && cum >= (double) p.top_p);
        if (lane == 0) s_tx_tp[wave] = bt ? wave * 64 + __builtin_ctzll(bt) : 0x7fffffff;
    } else if (lane == 0) {
        s_tx_tp[wave] = 0x7fffffff;
    }
    __syncthreads();
    if (p.top_p < 1.0f) {
        int f = 0x7fffffff;
#pragma unroll
        for (int w = 0; w < TAIL_WG / 64; ++w) f = min(f, s_tx_tp[w]);
        if (f != 0x7fffffff) n = f + 1;
    }
    // draw (:82-88): r = u*(total-0)+0; r - cum_i is exact while positive and keeps its sign at the step where it
    // reaches <= 0, so the drawn candidate is the first i with cum_i >= r (the last kept if none)
    if (live) {
        const double r0 = __dadd_rn(__dmul_rn(u, __dsub_rn(t[n - 1], 0.0)), 0.0);
        const uint64_t bd = ballot(tid < n && cum >= r0);
        if (lane == 0) s_tx_dr[wave] = bd ? wave * 64 + __builtin_ctzll(bd) : 0x7fffffff;
    } else if (lane == 0) {
        s_tx_dr[wave] = 0x7fffffff;
    }
    __syncthreads();
    int f = 0x7fffffff;
#pragma unroll
    for (int w = 0; w < TAIL_WG / 64; ++w) f = min(f, s_tx_dr[w]);
    *n_kept = n;
    *p_mine = pf;
    return f != 0x7fffffff ? f : n - 1;
}

// Key layouts the tail reads: the wide path's packed keys, and the fast path's (value image << 32 | ~id).
struct WideKeyFmt {
    int ib;          // id bits
    uint64_t vmask;  // value and id fields
    uint32_t idm;    // id field
    __device__ uint32_t img(uint64_t k) const { return (uint32_t) ((k & vmask) >> ib); }
    __device__ int id(uint64_t k) const { return (int) (~(uint32_t) k & idm); }
};
struct FastKeyFmt {
    __device__ uint32_t img(uint64_t k) const { return (uint32_t) (k >> 32); }
    __device__ int id(uint64_t k) const { return (int) ~(uint32_t) k; }
};

// The tail of src/sampler.cpp:53-88 over a row's sorted keys K (value descending, id ascending; the first
// k <= TAIL_WG are the candidates, ended early by the first key of value image 0, a NaN), with the whole
// workgroup (TAIL_WG threads, one candidate each, uniform control flow): the per-candidate terms (e_i, then p_i)
// go to t[0..k) as doubles, and every sum is the reference's sequential double chain: tail_exact when the
// candidates meet the exactness condition above, else replayed exactly (replay_sum). Publishes the row's token.
template <typename Fmt>
__device__ void sorted_tail(const RowsArgs& a, int row, const uint64_t* K, int k, double* t, const CallIn& cin,
                            const Fmt& fmt) {
    const int tid = (int) threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const SamplingParams p = a.p;
    const uint32_t seq = cin.seq;
    const int32_t draft = cin.draft;
    const uint32_t o0 = k > 0 ? fmt.img(K[0]) : 0u;
    if (o0 == 0u) {  // no number in the row: the fast path's empty candidate list
        if (wave == 0) {
            if (a.dbg_keys) a.dbg_keys[row * KCAP + lane] = 0ull;
            if (lane == 0) {
                if (a.dbg_meta) {
                    a.dbg_meta[row * 2] = 0;
                    a.dbg_meta[row * 2 + 1] = 0;
                }
                publish(a, row, 0, seq, draft);
            }
        }
        return;
    }
    const float maxl = unord_f32(o0);
    // e_i (:55-58) of every candidate, and kk: the first NaN key ends the candidates
    if (tid == 0) s_wide_n = k;
    __syncthreads();
    if (wave * 64 < k) {  // (waves past the candidates have no term)
        const uint32_t o = fmt.img(K[min(tid, k - 1)]);
        const float e = expf_glibc_tab(__fdiv_rn(__fsub_rn(unord_f32(o), maxl), p.temperature), kExp2Tab[lane & 31]);
        if (tid < k) {
            if (o == 0u) atomicMin(&s_wide_n, tid);
            t[tid] = (double) e;
        }
    }
    __syncthreads();
    const int kk = s_wide_n;
    int n = 0;
    float dbg_p = 0.0f;
    int idx = tail_exact(t, kk, p, cin.u, lane, wave, &n, &dbg_p);
    const bool act = lane < kk;
    if (idx < 0) {
        // the chains replayed exactly in reference order: the softmax total (:58)
        int st;
        const auto never = [](double, int) { return false; };
        const double sum = replay_sum<1>(t, kk, 0.0, never, &st);
        // p_i (:60), and min-p (:62-68): the first candidate i >= 1 with p_i < p_0 * min_p ends the list
        const double e0 = (double) expf_glibc(__fdiv_rn(__fsub_rn(maxl, maxl), p.temperature));
        const float thr = __fmul_rn(__double2float_rn(__ddiv_rn(e0, sum)), p.min_p);
        if (tid == 0) s_wide_n = kk;
        __syncthreads();
        if (tid < kk) {
            const float pi = __double2float_rn(__ddiv_rn(t[tid], sum));
            if (p.min_p > 0.0f && tid >= 1 && !(pi >= thr)) atomicMin(&s_wide_n, tid);
            t[tid] = (double) pi;
        }
        __syncthreads();
        n = s_wide_n;
        dbg_p = act ? (float) t[lane] : 0.0f;
        // top-p (:69-79): cum over the candidates until it reaches top_p; the draw total (:80-81) is the same
        // chain over the kept ones
        double total;
        if (p.top_p < 1.0f) {
            const double tp = (double) p.top_p;
            const auto reach = [tp](double acc, int) { return acc >= tp; };
            total = replay_sum<1>(t, n, 0.0, reach, &st);
            n = st >= 0 ? st + 1 : n;
        } else {
            total = replay_sum<1>(t, n, 0.0, never, &st);
        }
        // draw (:82-88): r = u*(total-0)+0, then r -= p_i until r <= 0 (else the last kept candidate); as a
        // chain of additions of -p_i (exactly the subtractions)
        const double r0 = __dadd_rn(__dmul_rn(cin.u, __dsub_rn(total, 0.0)), 0.0);
        const auto spent = [](double r, int) { return r <= 0.0; };
        replay_sum<1, true>(t, n, r0, spent, &st);
        idx = st >= 0 ? st : n - 1;
    }
    if (wave != 0) return;
    const int tok = fmt.id(K[idx]);
    const uint64_t kl = act ? K[lane] : 0ull;
    if (a.dbg_keys) a.dbg_keys[row * KCAP + lane] = act ? ((uint64_t) fmt.img(kl) << 32) | (uint64_t) ~(uint32_t) fmt.id(kl) : 0ull;
    if (a.dbg_probs) a.dbg_probs[row * KCAP + lane] = dbg_p;
    if (lane == 0) {
        if (a.dbg_meta) {
            a.dbg_meta[row * 2] = kk;
            a.dbg_meta[row * 2 + 1] = n;
        }
        publish(a, row, tok, seq, draft);
    }
}

// ---- The wide path's tail (src/sampler.cpp:53-88 over every sorted candidate) on many workgroups. Its three
// double chains (the softmax total, the top-p cumulative sum with the draw's total, the draw's subtractions) are
// cut into chunks of WT_CHUNK terms, and each chain runs as:
//   * a map kernel (workgroup = (row, chunk)): every term's place in the chain from an approximate prefix (the
//     earlier chunks' term sums and a scan of the chunk's own, added in any order). A term whose approximate
//     partial results before and after it, widened by a margin, lie in one binade [2^E, 2^(E+1)) (and, for
//     top-p, below the stop) has exact partial results there too and does not meet the stop: its map in that
//     binade (term_map) is valid. The chunk is cut into segments, in order: maximal runs of such terms in one
//     binade, composed to one map (a segmented scan), and every other term on its own (binade crossings, the
//     stop, the start from 0). Terms whose approximate partial result before them is past the stop by the
//     margin are left out (the exact chain has stopped before them). A chunk of more than WT_SEGS segments is
//     recorded as one segment to replay;
//   * a resolve kernel (one workgroup per row): from the chain's exact start, the segments in order: runs of
//     mapped segments of one binade are applied as one composed map (64 at a time), a single term is added, a
//     segment to replay goes through replay_sum; a mapped segment whose composed results reach the stop, or that
//     the exact partial result enters outside its binade, is replayed term by term.
// The margin: with M = |start| + the sum of the chain's |terms|, every rounded partial result of the reference's
// chain is within j * 2^-53 * M of the exact partial sum after j terms, and the approximate prefix within
// (chunks + 2 * WT_CHUNK + 16) * 2^-53 * M of it (additions of same-signed values in any order); the margin is
// (n + chunks + 2 * WT_CHUNK + 64) * 2^-50 * M, more than eight times their sum. A composed result outside its
// binade would be a broken bound and is reported as a fault.
// Chunk kernels: WT_WG threads, WT_PT terms each (i = lo + q * WT_WG + tid for the term passes; consecutive
// runs lo + tid * WT_PT + q where maps are composed in order).
constexpr int WT_WG = 256, WT_PT = WT_CHUNK / WT_WG;
constexpr int WT_FLAT = 1400;  // segment records a resolve kernel holds in LDS at once
static_assert(WT_FLAT >= WT_SEGS, "a window holds at least one chunk's segments");
constexpr int WT_RP = WT_CHUNK > TAIL_WG ? 2 : 1;  // replay_sum terms per thread: a replayed segment (at most a chunk) is one block
static_assert(WT_CHUNK <= WT_RP * TAIL_WG, "a chunk is one replay_sum block of one or two terms per thread");
// segment codes of a term on its own / past n or past the stop
constexpr int CODE_HARD = -0x7fffffff, CODE_NONE = -0x7ffffffe;

__shared__ double s_wt_red[2][WT_WG / 64];
__shared__ ParMap s_wt_map[WT_WG / 64];
__shared__ int s_wt_code[WT_WG / 64], s_wt_head[WT_WG / 64], s_wt_hcnt[WT_WG / 64];
__shared__ WideSeg s_wt_seg[WT_SEGS];
__shared__ int s_wt_start[WT_SEGS];
__shared__ WideSeg s_wt_flat[WT_FLAT];
__shared__ double s_wt_acc;                               // the resolve walk's state, handed between waves
__shared__ int s_wt_i, s_wt_st, s_wt_rs, s_wt_re;
__shared__ int s_wt_off[TAIL_WG + 1];
__shared__ uint16_t s_wt_rc[WT_FLAT];  // the window's chunk (from cb) of each record
static_assert(TAIL_WG <= 65536, "a window's chunk index fits 16 bits");
__shared__ int s_wt_wsum[TAIL_WG / 64];

// Composition for a segmented scan: bit 2 of p marks a map that starts a segment (nothing before it applies).
__device__ __forceinline__ ParMap seg_compose(const ParMap& e, const ParMap& l) {
    if (l.p & 4u) return l;
    ParMap c = par_compose(e, l);
    c.p |= e.p & 4u;
    return c;
}
__device__ __forceinline__ ParMap wave_seg_scan(ParMap x) {
    x = seg_compose(dpp_map<0x111, 0xf>(x), x);
    x = seg_compose(dpp_map<0x112, 0xf>(x), x);
    x = seg_compose(dpp_map<0x114, 0xf>(x), x);
    x = seg_compose(dpp_map<0x118, 0xf>(x), x);
    x = seg_compose(dpp_map<0x142, 0xa>(x), x);
    x = seg_compose(dpp_map<0x143, 0xc>(x), x);
    return x;
}

__device__ __forceinline__ WideKeyFmt wide_fmt(const WideArgs& w) {
    return WideKeyFmt{w.id_bits, (1ull << (32 + w.id_bits)) - 1ull, (1u << w.id_bits) - 1u};
}
// a row's terms: its part of the (free after the sort) unsorted key buffer
__device__ __forceinline__ double* wide_terms(const RowsArgs& a, const WideArgs& w, int row) {
    return reinterpret_cast<double*>(w.keys + (int64_t) row * a.V);
}

// Sum of x over the chunk workgroup, in every thread (slot: which LDS row to use).
__device__ __forceinline__ double wt_sum(double x, int slot, int lane, int wave) {
    x = wave_sum_f64(x, lane);
    if (lane == 0) s_wt_red[slot][wave] = x;
    __syncthreads();
    double s = 0.0;
#pragma unroll
    for (int o = 0; o < WT_WG / 64; ++o) s += s_wt_red[slot][o];
    return s;
}

// Chain PH of a row: 0 the softmax total over the kk candidates from 0 (:58); 1 the cumulative sum over the n_mp
// kept by min-p from 0, stopping where it reaches top_p when top_p < 1 (:69-81); 2 the draw over the n_top kept,
// r0 - p_0 - p_1 - ..., stopping at r <= 0 (:82-88).
template <int PH>
struct WtChain {
    int n;
    double a0;
    int mode;    // 0: no stop, 1: stop at acc >= thr, 2: stop at acc <= 0
    double thr;
    static constexpr bool NEG = PH == 2;
    __device__ WtChain(const RowsArgs& a, const WideRow& rs) {
        n = PH == 0 ? rs.kk : PH == 1 ? rs.n_mp : rs.n_top;
        a0 = PH == 2 ? rs.r0 : 0.0;
        mode = PH == 2 ? 2 : (PH == 1 && a.p.top_p < 1.0f) ? 1 : 0;
        thr = (double) a.p.top_p;
    }
};

// e_i (:55-58) of the row's first w.k sorted keys, their chunk sums, and the candidate count kk (the first NaN key
// ends the candidates: written by the one thread whose key is the first NaN, or holds the last key if none is).
__global__ __launch_bounds__(WT_WG) void wt_terms_kernel(RowsArgs a, WideArgs w) {
    const int row = (int) blockIdx.x / w.chunks, c = (int) blockIdx.x - row * w.chunks;
    const int tid = (int) threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const WideKeyFmt fmt = wide_fmt(w);
    const uint64_t* K = w.sorted + (int64_t) row * a.V;
    double* t = wide_terms(a, w, row);
    const int k = w.k, lo = c * WT_CHUNK;
    const uint64_t etab = kExp2Tab[lane & 31];
    uint32_t o[WT_PT];
#pragma unroll
    for (int q = 0; q < WT_PT; ++q) o[q] = fmt.img(K[min(lo + q * WT_WG + tid, k - 1)]);
    const float maxl = unord_f32(fmt.img(K[0]));
    double s = 0.0;
#pragma unroll
    for (int q = 0; q < WT_PT; ++q) {
        const int i = lo + q * WT_WG + tid;
        const float e = expf_glibc_tab(__fdiv_rn(__fsub_rn(unord_f32(o[q]), maxl), a.p.temperature), etab);
        if (i < k) {
            const double ed = o[q] != 0u ? (double) e : 0.0;
            t[i] = ed;
            s += ed;
            if (o[q] == 0u ? (i == 0 || fmt.img(K[i - 1]) != 0u) : i == k - 1)
                w.rowst[row].kk = o[q] == 0u ? i : k;
        }
    }
    s = wt_sum(s, 0, lane, wave);
    if (tid == 0) w.part[(int64_t) row * w.chunks + c] = s;
}

// p_i = (float) (e_i / sum) (:60) in place, min-p (:62-68: n_mp lowered to the first i >= 1 with p_i < p_0 *
// min_p; the resolve of chain 0 set it to kk), and the chunk sums of the p_i.
__global__ __launch_bounds__(WT_WG) void wt_probs_kernel(RowsArgs a, WideArgs w) {
    const int row = (int) blockIdx.x / w.chunks, c = (int) blockIdx.x - row * w.chunks;
    const int tid = (int) threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const WideKeyFmt fmt = wide_fmt(w);
    const int kk = w.rowst[row].kk, lo = c * WT_CHUNK;
    if (lo >= kk) return;  // (uniform)
    const double sum = w.rowst[row].sum;
    double* t = wide_terms(a, w, row);
    double e[WT_PT];
#pragma unroll
    for (int q = 0; q < WT_PT; ++q) e[q] = t[min(lo + q * WT_WG + tid, kk - 1)];
    const float maxl = unord_f32(fmt.img(w.sorted[(int64_t) row * a.V]));
    const double e0 = (double) expf_glibc(__fdiv_rn(__fsub_rn(maxl, maxl), a.p.temperature));
    const float thr = __fmul_rn(__double2float_rn(__ddiv_rn(e0, sum)), a.p.min_p);
    double s = 0.0;
    int fail = 0x7fffffff;
#pragma unroll
    for (int q = 0; q < WT_PT; ++q) {
        const int i = lo + q * WT_WG + tid;
        if (i < kk) {
            const float pi = __double2float_rn(__ddiv_rn(e[q], sum));
            if (a.p.min_p > 0.0f && i >= 1 && !(pi >= thr)) fail = min(fail, i);
            t[i] = (double) pi;
            s += (double) pi;
        }
    }
    s = wt_sum(s, 0, lane, wave);
    const uint64_t fb = ballot(fail != 0x7fffffff);
    if (fb) {
        int m = fail;
        m = min(m, xor_lane<32>(m, lane));
        m = min(m, xor_lane<16>(m, lane));
        m = min(m, xor_lane<8>(m, lane));
        m = min(m, xor_lane<4>(m, lane));
        m = min(m, xor_lane<2>(m, lane));
        m = min(m, xor_lane<1>(m, lane));
        if (lane == 0) atomicMin(&w.rowst[row].n_mp, m);
    }
    if (tid == 0) w.part[(int64_t) row * w.chunks + c] = s;
}

// The segments of a chunk of chain PH (see above).
template <int PH>
__global__ __launch_bounds__(WT_WG) void wt_maps_kernel(RowsArgs a, WideArgs w) {
    const int row = (int) blockIdx.x / w.chunks, c = (int) blockIdx.x - row * w.chunks;
    const int tid = (int) threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const WtChain<PH> ch(a, w.rowst[row]);
    const int n = ch.n, lo = c * WT_CHUNK;
    if (lo >= n) return;  // (uniform)
    const int nc = (n + WT_CHUNK - 1) / WT_CHUNK, last = min(n, lo + WT_CHUNK) - 1;
    const double* t = wide_terms(a, w, row);
    const int j0 = lo + tid * WT_PT;
    double sv[WT_PT];  // the terms as the chain adds them (0 past n)
    static_assert(WT_PT % 2 == 0, "pairs of terms");
    if (j0 + WT_PT <= n && (reinterpret_cast<uintptr_t>(t) & 15u) == 0) {
        // 16-byte loads (j0 is a multiple of WT_PT; the row's terms start 16-byte aligned when V is even)
#pragma unroll
        for (int q = 0; q < WT_PT; q += 2) {
            const double2 x = *reinterpret_cast<const double2*>(t + j0 + q);
            sv[q] = ch.NEG ? -x.x : x.x;
            sv[q + 1] = ch.NEG ? -x.y : x.y;
        }
    } else {
#pragma unroll
        for (int q = 0; q < WT_PT; ++q) {
            const double x = t[min(j0 + q, n - 1)];
            sv[q] = j0 + q < n ? (ch.NEG ? -x : x) : 0.0;
        }
    }
    // approximate partial results: the earlier chunks' sums, then an exclusive scan of the threads' sums
    double pre = 0.0, all = 0.0, own = 0.0;
    for (int j = tid; j < nc; j += WT_WG) {
        const double v = w.part[(int64_t) row * w.chunks + j];
        pre += j < c ? v : 0.0;
        all += v;
    }
#pragma unroll
    for (int q = 0; q < WT_PT; ++q) own += sv[q];
    pre = wt_sum(pre, 0, lane, wave);
    all = wt_sum(all, 1, lane, wave);
    const double incl = wave_scan_f64(own);
    __syncthreads();  // (the sums' LDS rows are reused)
    if (lane == 63) s_wt_red[0][wave] = incl;
    __syncthreads();
    double run = (ch.NEG ? ch.a0 - pre : ch.a0 + pre) + (incl - own);
#pragma unroll
    for (int o = 0; o < WT_WG / 64; ++o) run += o < wave ? s_wt_red[0][o] : 0.0;
    const double margin = (fabs(ch.a0) + all) * ((double) n + (double) nc + 2.0 * WT_CHUNK + 64.0) * 0x1p-50;
    // each term's binade (code: E) when its map is valid, else CODE_HARD
    ParMap m[WT_PT];
    int code[WT_PT];
#pragma unroll
    for (int q = 0; q < WT_PT; ++q) {
        const double before = run, after = run + sv[q];
        run = after;
        const double lb = fmin(before, after) - margin, hb = fmax(before, after) + margin;
        int E = 0;
        bool easy = lb >= 0x1p-1000 && hb <= 0x1p1000;  // (false for NaN)
        if (easy) {
            (void) frexp(lb, &E);
            E -= 1;  // lb in [2^E, 2^(E+1))
            easy = hb < ldexp(1.0, E + 1) && !(ch.mode == 1 && !(hb < ch.thr));
        }
        double f;
        bool cr;
        m[q] = term_map(sv[q], E, &f, &cr);
        const bool past = (ch.mode == 1 && before - margin >= ch.thr) || (ch.mode == 2 && before + margin <= 0.0);
        code[q] = (j0 + q >= n || past) ? CODE_NONE : (easy && !cr) ? E : CODE_HARD;
    }
    // segment heads: the chunk's first term, a term on its own, and a term after one or in another binade
    int prev = __builtin_amdgcn_update_dpp(0, code[WT_PT - 1], 0x138, 0xf, 0xf, false);  // wave_shr:1 (lane 0: below)
    if (lane == 63) s_wt_code[wave] = code[WT_PT - 1];
    bool head[WT_PT];
    int hc = 0;
    __syncthreads();
    if (lane == 0) prev = wave > 0 ? s_wt_code[wave - 1] : CODE_NONE;
#pragma unroll
    for (int q = 0; q < WT_PT; ++q) {
        const int pc = q == 0 ? prev : code[q - 1];
        head[q] = code[q] != CODE_NONE && ((tid == 0 && q == 0) || code[q] == CODE_HARD || pc != code[q]);
        hc += head[q] ? 1 : 0;
    }
    // whether the next term starts a segment or is left out (for a thread's last term: the next thread's first)
    const int brk0 = (head[0] || code[0] == CODE_NONE) ? 1 : 0;
    int nh = __builtin_amdgcn_update_dpp(0, brk0, 0x130, 0xf, 0xf, false);  // wave_shl:1 (lane 63: below)
    if (lane == 0) s_wt_head[wave] = brk0;
    // segment ordinals: an inclusive scan of the heads
    const int hi = wave_scan_i32(hc);
    if (lane == 63) s_wt_hcnt[wave] = hi;
    // segmented scan of the maps: each thread's summary, then the wave's and the waves'
    ParMap T = par_identity();
#pragma unroll
    for (int q = 0; q < WT_PT; ++q) {
        ParMap x = code[q] > CODE_NONE ? m[q] : par_identity();
        if (head[q]) x.p |= 4u;
        T = seg_compose(T, x);
    }
    const ParMap ti = wave_seg_scan(T);
    const ParMap te = dpp_map<0x138, 0xf>(ti);  // wave_shr:1: the threads before this one (lane 0: identity)
    if (lane == 63) s_wt_map[wave] = ti;
    __syncthreads();
    if (lane == 63) nh = wave + 1 < WT_WG / 64 ? s_wt_head[wave + 1] : 1;
    int hbase = hi - hc, htot = 0;
    ParMap win = par_identity();
#pragma unroll
    for (int o = 0; o < WT_WG / 64; ++o) {
        const int v = s_wt_hcnt[o];
        hbase += o < wave ? v : 0;
        htot += v;
        if (o < wave) win = seg_compose(win, s_wt_map[o]);
    }
    const bool over = htot > w.seg_cap;  // (uniform)
    if (!over) {
        // each segment's record at its last term (its start at its head)
        ParMap R = seg_compose(win, te);
        int ord = hbase - 1;
#pragma unroll
        for (int q = 0; q < WT_PT; ++q) {
            const int j = j0 + q;
            if (code[q] != CODE_NONE) {
                if (head[q]) {
                    ++ord;
                    R = par_identity();
                    s_wt_start[ord] = j;
                }
                if (code[q] != CODE_HARD) R = par_compose(R, m[q]);
                const bool ends = j == last || (q + 1 < WT_PT ? head[q + 1] || code[q + 1] == CODE_NONE : nh != 0);
                if (ends) {
                    WideSeg r;
                    r.kind = code[q] == CODE_HARD ? WS_TERM : WS_MAP;
                    r.d0 = code[q] == CODE_HARD ? sv[q] : R.d0;
                    r.d1 = R.d1;
                    r.p = R.p & 3u;
                    r.E = code[q] == CODE_HARD ? 0 : code[q];
                    r.start = 0;
                    r.end = j + 1;
                    r.pad = 0;
                    s_wt_seg[ord] = r;
                }
            }
        }
    }
    __syncthreads();
    WideSeg* out = w.seg + ((int64_t) row * w.chunks + c) * WT_SEGS;
    if (over) {
        if (tid == 0) out[0] = WideSeg{0.0, 0.0, 2u, 0, WS_REPLAY, lo, last + 1, 0};
    } else if (tid < htot) {
        WideSeg r = s_wt_seg[tid];
        r.start = s_wt_start[tid];
        out[tid] = r;
    }
    if (tid == 0) w.nseg[(int64_t) row * w.chunks + c] = over ? 1 : htot;
}

__device__ __forceinline__ bool in_binade(double x, int E) {
    int e;
    (void) frexp(x, &e);
    return x >= 0x1p-1000 && x <= 0x1p1000 && e - 1 == E;
}

// Chain PH of one row from its exact start, with the whole workgroup (uniform control flow): returns the last
// partial result and the stop index (-1: none).
template <int PH, typename F>
__device__ double wt_resolve(const RowsArgs& a, const WideArgs& w, int row, const WtChain<PH>& ch, F stop,
                             int* stopped) {
    const int tid = (int) threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = ch.n, nc = (n + WT_CHUNK - 1) / WT_CHUNK;
    const double* t = wide_terms(a, w, row);
    const WideSeg* seg = w.seg + (int64_t) row * w.chunks * WT_SEGS;
    const int32_t* nseg = w.nseg + (int64_t) row * w.chunks;
    double acc = ch.a0;
    int st = -1;
    for (int cb = 0; cb < nc && st < 0;) {
        // a window of chunks [cb, ce) whose segments fit in LDS: the segment counts of up to TAIL_WG chunks,
        // scanned (s_wt_off: the chunks' first records), then as many chunks as fit (at least one)
        __syncthreads();
        const int cnt = cb + tid < nc ? nseg[cb + tid] : 0;
        int cs = wave_scan_i32(cnt);  // inclusive scan of the counts
        if (lane == 63) s_wt_wsum[wave] = cs;
        __syncthreads();
#pragma unroll
        for (int o = 0; o < TAIL_WG / 64; ++o) cs += o < wave ? s_wt_wsum[o] : 0;
        s_wt_off[tid + 1] = cs;
        if (tid == 0) s_wt_off[0] = 0;
        const int fit = __syncthreads_count(cb + tid < nc && cs <= WT_FLAT);
        const int ce = cb + max(fit, 1), wn = s_wt_off[ce - cb];
        // each chunk of the window marks its records with its index (s_wt_off[tid + 1] <= wn <= WT_FLAT), so that
        // a record finds its chunk with one LDS read instead of a binary search over the offsets
        if (tid < ce - cb)
            for (int r = s_wt_off[tid]; r < s_wt_off[tid + 1]; ++r) s_wt_rc[r] = (uint16_t) tid;
        __syncthreads();
        for (int r = tid; r < wn; r += TAIL_WG) {
            const int c = s_wt_rc[r];
            s_wt_flat[r] = seg[(int64_t) (cb + c) * WT_SEGS + (r - s_wt_off[c])];
        }
        __syncthreads();
        cb = ce;
        // wave 0 walks the window's records; the workgroup joins it for a replay (replay_sum)
        int i = 0;
        while (true) {  // (uniform)
            if (wave == 0) {
                int rs = -1, re = -1;
                while (i < wn && st < 0) {
                    const WideSeg r = s_wt_flat[i];
                    if (r.kind == WS_MAP && in_binade(acc, r.E)) {
                        // a run of mapped segments of r's binade (at most 64): each lane's inclusive result
                        const WideSeg q = i + lane < wn ? s_wt_flat[i + lane] : WideSeg{0.0, 0.0, 2u, 0, 0, 0, 0, 0};
                        const uint64_t rm = ballot(i + lane < wn && q.kind == WS_MAP && q.E == r.E);
                        const int len = ~rm ? (int) __builtin_ctzll(~rm) : 64;  // >= 1
                        ParMap x = lane < len ? ParMap{q.d0, q.d1, q.p} : par_identity();
                        if (len > 1) x = wave_scan_map<false>(x);
                        const double A = ldexp(acc, 52 - r.E);
                        const double Al = A + (dparity(A) ? x.d1 : x.d0);
                        const double accl = ldexp(Al, r.E - 52);
                        if (ballot(lane < len && !(Al >= 0x1p52 && Al < 0x1p53)) && lane == 0) report_fault(a, FAULT_WIDE_MAP);
                        const uint64_t hit = ballot(lane < len && stop(accl, 0));
                        if (!hit) {
                            acc = rdlaned(accl, len - 1);
                            i += len;
                            continue;
                        }
                        // the stop lies in segment l of the run: replay it from the result before it
                        const int l = (int) __builtin_ctzll(hit);
                        const WideSeg h = s_wt_flat[i + l];
                        acc = l > 0 ? rdlaned(accl, l - 1) : acc;
                        rs = h.start;
                        re = h.end;
                        i += l + 1;
                        break;
                    } else if (r.kind == WS_TERM) {
                        acc = __dadd_rn(acc, r.d0);
                        if (stop(acc, r.start)) st = r.start;
                        ++i;
                    } else {  // a segment to replay, or a mapped one entered outside its binade
                        rs = r.start;
                        re = r.end;
                        ++i;
                        break;
                    }
                }
                if (lane == 0) {
                    s_wt_acc = acc;
                    s_wt_i = i;
                    s_wt_st = st;
                    s_wt_rs = rs;
                    s_wt_re = re;
                }
            }
            __syncthreads();
            acc = s_wt_acc;
            i = s_wt_i;
            st = s_wt_st;
            const int rs = s_wt_rs, re = s_wt_re;
            __syncthreads();  // (read before wave 0 rewrites them)
            if (rs < 0) break;  // the window is walked, or the chain stopped
            int s2;
            acc = replay_sum<WT_RP, WtChain<PH>::NEG>(t + rs, re - rs, acc, stop, &s2);
            if (s2 >= 0) {
                st = rs + s2;
                break;
            }
        }
    }
    *stopped = st;
    return acc;
}

// Resolves chain PH of each row (one workgroup per row) and hands its results to the next kernels; the last
// publishes the row's token.
template <int PH>
__global__ __launch_bounds__(TAIL_WG) void wt_resolve_kernel(RowsArgs a, WideArgs w) {
    const int row = (int) blockIdx.x, tid = (int) threadIdx.x, lane = lane_id(), wave = tid >> 6;
    WideRow* rs = w.rowst + row;
    const WtChain<PH> ch(a, *rs);
    // the call block (pinned host memory) read at the start: its round trip overlaps the chain's first loads
    const CallIn cin = PH > 0 ? read_call<false>(a, row) : CallIn{0u, -1, 0.0};
    int st = -1;
    double acc = ch.a0;
    if (ch.n > 0) {
        if (ch.mode == 1) {
            const double thr = ch.thr;
            acc = wt_resolve<PH>(a, w, row, ch, [thr](double x, int) { return x >= thr; }, &st);
        } else if (ch.mode == 2) {
            acc = wt_resolve<PH>(a, w, row, ch, [](double x, int) { return x <= 0.0; }, &st);
        } else {
            acc = wt_resolve<PH>(a, w, row, ch, [](double, int) { return false; }, &st);
        }
    }
    if (tid != 0 && PH != 2) return;
    if (PH == 0) {
        rs->sum = acc;
        rs->n_mp = ch.n;  // (min-p lowers it)
    } else if (PH == 1) {
        // top-p (:70-79) keeps up to the stop; the draw's total (:80-81) is the chain's result there
        const int n_top = st >= 0 ? st + 1 : ch.n;
        const double u = cin.u;
        rs->n_top = n_top;
        rs->total = acc;
        rs->r0 = __dadd_rn(__dmul_rn(u, __dsub_rn(acc, 0.0)), 0.0);
    } else {
        if (wave != 0) return;
        const WideKeyFmt fmt = wide_fmt(w);
        const uint64_t* K = w.sorted + (int64_t) row * a.V;
        const int kk = rs->kk, n_top = ch.n;
        const int idx = st >= 0 ? st : n_top - 1;
        const int tok = kk > 0 ? fmt.id(K[idx]) : 0;  // no number in the row: the fast path's empty list
        const bool act = lane < kk;
        const uint64_t kl = act ? K[lane] : 0ull;
        if (a.dbg_keys) a.dbg_keys[row * KCAP + lane] = act ? ((uint64_t) fmt.img(kl) << 32) | (uint64_t) ~(uint32_t) fmt.id(kl) : 0ull;
        if (a.dbg_probs) a.dbg_probs[row * KCAP + lane] = act ? (float) wide_terms(a, w, row)[lane] : 0.0f;
        if (lane == 0) {
            if (a.dbg_meta) {
                a.dbg_meta[row * 2] = kk;
                a.dbg_meta[row * 2 + 1] = kk > 0 ? n_top : 0;
            }
            publish(a, row, tok, cin.seq, cin.draft);
        }
    }
}

// ---------------------------------------------------------------------------------------------------------
// Mid top-k (KCAP < k <= MID_KMAX; src/sampler.cpp:42-51) in one launch. Workgroup = (row, segment of MID_SEG
// ids), 16 waves, 32 logits per thread held in registers:
//   1. the history counts are applied to every logit (a 32-bit LDS table over the segment);
//   2. a bound reached by at least ks = min(k, segment length) logits of the segment: each wave takes the
//      ceil(ks/16)-th largest of its lanes' two largest values (128 distinct logits), and the smallest of the 16
//      waves' values has at least 16 * ceil(ks/16) >= ks logits at or above it, so the segment's top ks are all
//      at or above it (with fewer numbers than that the bound is 0 and every number qualifies);
//   3. with more than m.cap keys at or above it (ties at the bound), the key threshold is bisected until between
//      ks and m.cap keys reach it (keys are distinct, so such a threshold exists);
//   4. the keys that reach it are appended to the row's buffer (space taken with a device-scope counter), so the
//      buffer holds every key of the row's top k;
//   5. the row's last workgroup (ticket) holds the buffer in registers (16 keys per thread), forms the same
//      bound for k over it when it holds more than 2k + 256 keys (bisected down to MID_SORT keys if needed),
//      sorts the keys that reach it in LDS and runs sorted_tail over the first k.
// Counters are left zero for the next launch (the ticket by publish, the buffer's counter by the last workgroup).
constexpr int MID_NW = 16, MID_WG = MID_NW * 64, MID_EPT = 32, MID_RK = MID_ROWCAP / MID_WG;
constexpr int MID_SORT = 4096;  // keys the row's sort holds
constexpr int MID_BIGK = 256;   // top-k above this takes the kernel with the register-templated sort
static_assert(MID_WG * MID_EPT == MID_SEG, "segment length");
static_assert(MID_WG == TAIL_WG, "the row's tail runs on the mid workgroup");
static_assert(MID_KMAX <= TAIL_WG, "sorted_tail holds one candidate per thread");
static_assert(MID_KMAX <= MID_NW * 64, "a wave's bound index is at most 64");
static_assert(MID_SORT == 4 * MID_WG && MID_SORT >= MID_KMAX, "the sort's layout");

__shared__ uint32_t s_mid_w[MID_NW];  // per-wave bounds
__shared__ int s_mid_c[2][MID_NW];    // per-wave counts (two sets, used alternately)
__shared__ int s_mid_base;

// The j-th largest (1 <= j <= 64) of the 128 values m1, m2 of the wave's lanes (value images, m2 <= m1 in each
// lane); 0 when fewer than j are nonzero. It is the largest t that at least j of the values reach, built from
// the top bit down: per bit two compares, whose lane masks are the ballots, and scalar counts (a chain of 32
// short steps; two 64-lane bitonic sorts and a merge were 48 dependent cross-lane steps).
__device__ __forceinline__ uint32_t wave_top2_kth(uint32_t m1, uint32_t m2, int j, int lane) {
    (void) lane;
    uint32_t t = 0u;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
        const uint32_t c = t | (1u << b);
        const int n = __popcll(ballot(m1 >= c)) + __popcll(ballot(m2 >= c));
        t = n >= j ? c : t;
    }
    return t;
}

// Workgroup sum of c (every thread calls it). `par` alternates the LDS slots, so one barrier per call suffices:
// a thread writes a slot again only after a later call's barrier, which every thread passes after its reads.
__device__ __forceinline__ int mid_sum(int c, int lane, int wave, int& par) {
    const int x = wave_sum_i32(c, lane);
    if (lane == 0) s_mid_c[par][wave] = x;
    __syncthreads();
    int tot = 0;
#pragma unroll
    for (int w = 0; w < MID_NW; ++w) tot += s_mid_c[par][w];
    par ^= 1;
    return tot;
}

// Exclusive prefix of c over the workgroup's threads (thread order), and the total.
__device__ __forceinline__ int mid_prefix(int c, int lane, int wave, int& par, int* total) {
    const int x = wave_scan_i32(c);
    if (lane == 63) s_mid_c[par][wave] = x;
    __syncthreads();
    int tot = 0, before = 0;
#pragma unroll
    for (int w = 0; w < MID_NW; ++w) {
        const int sw = s_mid_c[par][w];
        tot += sw;
        before += w < wave ? sw : 0;
    }
    par ^= 1;
    *total = tot;
    return before + x - c;
}

// A key threshold reached by between `need` and `cap` keys of the workgroup (1 <= need <= cap), given `lo`, one
// reached by more than cap: bisection over (lo, 2^64 - 2] with workgroup counts, cnt(t) = this thread's keys
// >= t. Invariants: more than cap keys reach lo, fewer than need reach hi + 1; distinct keys make the count
// fall by at most one per step of t, so the interval never closes before a threshold is found, and halving a
// 64-bit interval finds it within 64 rounds. Past that (not reachable) the launch reports a fault and the
// threshold lets nothing through.
template <typename F>
__device__ __forceinline__ uint64_t mid_narrow(const RowsArgs& a, F cnt, uint64_t lo, int need, int cap, int lane,
                                               int wave, int& par) {
    uint64_t hi = ~0ull - 1ull;  // no key reaches 2^64 - 1 (the largest value image is that of +inf)
    for (int it = 0; it < 66; ++it) {
        const uint64_t mid = lo + (hi - lo) / 2 + 1;
        const int c = mid_sum(cnt(mid), lane, wave, par);
        if (c > cap)
            lo = mid;
        else if (c < need)
            hi = mid - 1;
        else
            return mid;
    }
    if (threadIdx.x == 0) report_fault(a, FAULT_NARROW);
    return ~0ull;
}

// Sorts S[0..P) descending with the workgroup, S = the first MID_SORT keys of the LDS words s_cnt (P a power of
// two in [64, MID_SORT]; the next MID_SORT keys, U, serve the exchanges). Element i lives in lane i % 64 of wave
// (i / 64) % 16, register i / 1024: strides below 64 are bitonic steps across lanes, strides of 1024 and 2048
// compare a thread's own registers, and strides 64..512 go through LDS, the two halves alternating so that each
// such step needs one barrier. Returns the offset in keys (0: S, MID_SORT: U) of the half that holds the result
// (after a barrier). Every access indexes s_cnt itself, so it compiles to LDS instructions: a pointer chosen
// between the halves at run time would be a generic address, and generic (FLAT) accesses to LDS take the
// vector memory path (each exchange step then cost ~0.5 us more).
__device__ __forceinline__ int mid_sort(int P, int lane, int wave) {
    constexpr int R = MID_SORT / MID_WG;
    uint64_t* const L = reinterpret_cast<uint64_t*>(s_cnt);
    const int nch = P >> 6;  // chunks of 64
    uint64_t x[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int c = r * MID_NW + wave;
        x[r] = c < nch ? L[c * 64 + lane] : 0ull;
        // chunks alternately descending and ascending: every block of 128 is then bitonic
        if (c < nch) x[r] = (c & 1) ? sort64<false>(x[r], lane) : sort64<true>(x[r], lane);
    }
    int bo = MID_SORT;  // the half the next exchange writes (U first, then alternating)
    for (int size = 128; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride >= 64; stride >>= 1) {
            if (stride >= MID_WG) {
                const int rs = stride / MID_WG;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int c = r * MID_NW + wave;
                    if ((r & rs) == 0 && c < nch) {
                        const int r2 = r | rs;
                        const bool desc = ((c * 64) & size) == 0;
                        const uint64_t mx = max64(x[r], x[r2]), mn = min64(x[r], x[r2]);
                        x[r] = desc ? mx : mn;
                        x[r2] = desc ? mn : mx;
                    }
                }
            } else {
                const int b = bo;
                bo ^= MID_SORT;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int c = r * MID_NW + wave;
                    if (c < nch) L[b + c * 64 + lane] = x[r];
                }
                __syncthreads();
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int c = r * MID_NW + wave;
                    if (c < nch) {
                        const int i = c * 64 + lane;
                        const uint64_t y = L[b + (i ^ stride)];
                        const bool lower = (i & stride) == 0, desc = (i & size) == 0;
                        x[r] = (lower == desc) ? max64(x[r], y) : min64(x[r], y);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int c = r * MID_NW + wave;
            if (c < nch) x[r] = ((c * 64) & size) == 0 ? bitonic_stage<64, true>(x[r], lane) : bitonic_stage<64, false>(x[r], lane);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int c = r * MID_NW + wave;
        if (c < nch) L[bo + c * 64 + lane] = x[r];
    }
    __syncthreads();
    return bo;
}

// The same sort with the registers that hold elements as a template parameter (NR = P / 1024, at least 1; with 1,
// the waves past P / 64 hold none and only take the barriers): every register is live, so an exchange's LDS reads
// are issued together and waited for once, where the form above makes each register's test its own block with its
// own wait (2,048 keys timed alone: 9.6 against 13.4 us). It has its own kernel instantiation for large top-k: in
// the same kernel as the form above it changed the compiler's schedule of the segment phase and cost small k more
// than it saved.
template <int NR>
__device__ __forceinline__ int mid_sort_r(int P, int lane, int wave) {
    static_assert(NR >= 1 && NR * MID_WG <= MID_SORT, "registers per thread");
    uint64_t* const L = reinterpret_cast<uint64_t*>(s_cnt);
    const bool act = NR > 1 || wave < (P >> 6);  // (uniform in the wave)
    uint64_t x[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) x[r] = act ? L[(r * MID_NW + wave) * 64 + lane] : 0ull;
    if (act) {
        // chunks alternately descending and ascending: every block of 128 is then bitonic
#pragma unroll
        for (int r = 0; r < NR; ++r)
            x[r] = ((r * MID_NW + wave) & 1) ? sort64<false>(x[r], lane) : sort64<true>(x[r], lane);
    }
    int bo = MID_SORT;  // the half the next exchange writes (U first, then alternating)
    for (int size = 128; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride >= 64; stride >>= 1) {
            if (stride >= MID_WG) {
                const int rs = stride / MID_WG;
#pragma unroll
                for (int r = 0; r < NR; ++r) {
                    const int r2 = r | rs;
                    if ((r & rs) == 0 && r2 < NR) {
                        const bool desc = (((r * MID_NW + wave) * 64) & size) == 0;
                        const uint64_t mx = max64(x[r], x[r2]), mn = min64(x[r], x[r2]);
                        x[r] = desc ? mx : mn;
                        x[r2] = desc ? mn : mx;
                    }
                }
            } else {
                const int b = bo;
                bo ^= MID_SORT;
                if (act) {
#pragma unroll
                    for (int r = 0; r < NR; ++r) L[b + (r * MID_NW + wave) * 64 + lane] = x[r];
                }
                __syncthreads();
                if (act) {
                    uint64_t y[NR];
#pragma unroll
                    for (int r = 0; r < NR; ++r) y[r] = L[b + (((r * MID_NW + wave) * 64 + lane) ^ stride)];
#pragma unroll
                    for (int r = 0; r < NR; ++r) {
                        const int i = (r * MID_NW + wave) * 64 + lane;
                        const bool lower = (i & stride) == 0, desc = (i & size) == 0;
                        x[r] = (lower == desc) ? max64(x[r], y[r]) : min64(x[r], y[r]);
                    }
                }
            }
        }
        if (act) {
#pragma unroll
            for (int r = 0; r < NR; ++r)
                x[r] = (((r * MID_NW + wave) * 64) & size) == 0 ? bitonic_stage<64, true>(x[r], lane)
                                                                 : bitonic_stage<64, false>(x[r], lane);
        }
    }
    if (act) {
#pragma unroll
        for (int r = 0; r < NR; ++r) L[bo + (r * MID_NW + wave) * 64 + lane] = x[r];
    }
    __syncthreads();
    return bo;
}

__device__ __forceinline__ int mid_sort_big(int P, int lane, int wave) {
    static_assert(MID_SORT == 4 * MID_WG, "at most four registers per thread");
    return P > 2 * MID_WG ? mid_sort_r<4>(P, lane, wave)
                          : P > MID_WG ? mid_sort_r<2>(P, lane, wave) : mid_sort_r<1>(P, lane, wave);
}

template <bool PENALIZE, bool BIGK>
__global__ __launch_bounds__(MID_WG) void mid_kernel(RowsArgs a, MidArgs m) {
    constexpr int WG = MID_WG, EPT = MID_EPT, NV = EPT / 4;
    const int tid = (int) threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const int segs = a.segs;
    const int row = (int) blockIdx.x / segs, seg = (int) blockIdx.x - row * segs;
    const int lo = seg * MID_SEG, hi = min(a.V, lo + MID_SEG);
    const float* __restrict__ L = a.logits + (int64_t) row * a.row_stride;
    const bool vec = (reinterpret_cast<uintptr_t>(L) & 15u) == 0;
    // logit (i, e) of this thread: id lo + 4*(i*WG + tid) + e; NaN past the segment (never a candidate)
    float v[EPT];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int b = lo + 4 * (i * WG + tid);
        if (vec && b + 3 < hi) {
            const f32x4 f = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(L + b));
            v[4 * i + 0] = f[0];
            v[4 * i + 1] = f[1];
            v[4 * i + 2] = f[2];
            v[4 * i + 3] = f[3];
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * i + e] = b + e < hi ? L[b + e] : __uint_as_float(0x7fc00000u);
        }
    }
    // what the row's last workgroup needs from the call block (pinned host memory for graph-replayed steps), read
    // by every workgroup once its logit loads are issued: the PCIe round trip then ends before the first barrier
    // (which comes after the logits) instead of holding the last workgroup's first wait
    const CallIn cin = read_call<false>(a, row);
    if (PENALIZE) {
        RawHistory rh;
        if (a.hist_off) {
            rh.s0 = max(a.hist_off[row], 0);
            rh.s1 = max(a.hist_off[row + 1], rh.s0);
            const bool hv = (reinterpret_cast<uintptr_t>(a.hist_ids) & 15u) == 0;
            rh.b0 = hv ? min(rh.s1, (rh.s0 + 3) & ~3) : rh.s1;
            rh.b1 = hv ? max(rh.b0, rh.s1 & ~3) : rh.s1;
        }
        const int4 none[HR] = {};
        cnt_zero<WG>(hi - lo, tid);
        __syncthreads();
        count_history<WG, false, false>(a, row, lo, hi, none, rh, tid);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int id = lo + 4 * (i * WG + tid) + e;
                if (id < hi) {
                    const uint32_t c = s_cnt[id - lo];
                    if (c != 0u) v[4 * i + e] = penalize(v[4 * i + e], c, a.p);
                }
            }
        }
    }
    int par = 0;
    const int ks = min(m.k, hi - lo);
    uint32_t m1 = 0u, m2 = 0u;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const uint32_t o = ord_f32(v[j]);
        m2 = max(m2, min(m1, o));
        m1 = max(m1, o);
    }
    const uint32_t tw = wave_top2_kth(m1, m2, (ks + MID_NW - 1) / MID_NW, lane);
    if (lane == 0) s_mid_w[wave] = tw;
    __syncthreads();
    uint32_t bnd = 0xffffffffu;
#pragma unroll
    for (int w = 0; w < MID_NW; ++w) bnd = min(bnd, s_mid_w[w]);
    uint64_t T = (uint64_t) max(bnd, 1u) << 32;  // (numbers only: NaN keys are below 2^32)
    auto cnt = [&](uint64_t t) {
        int c = 0;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) c += mk_key(v[4 * i + e], lo + 4 * (i * WG + tid) + e) >= t ? 1 : 0;
        }
        return c;
    };
    int total;
    int off = mid_prefix(cnt(T), lane, wave, par, &total);
    if (total > m.cap) {
        T = mid_narrow(a, cnt, T, ks, m.cap, lane, wave, par);
        off = mid_prefix(cnt(T), lane, wave, par, &total);
    }
    if (tid == 0) s_mid_base = (int) atomicAdd(&m.fill[row], (uint32_t) total);
    __syncthreads();
    uint64_t* const buf = m.buf + (int64_t) row * MID_ROWCAP;
    // The keys are placed in LDS in thread order first (the count table and the sort space are free here), then
    // written to the row's buffer with neighbouring threads on neighbouring slots: straight from the registers,
    // each thread's 32 conditional stores were 32 store instructions per wave for a few keys each, all waited for
    // before the ticket. A few keys (at most 256: the extra barrier costs more than the stores save), or no room
    // in LDS (one segment, a larger cap), are stored directly.
    constexpr int STAGE = PENALIZE ? MID_SEG * (int) sizeof(uint32_t) / 8 : 2 * MID_SORT;  // keys the LDS holds
    if (total > 256 && total <= STAGE) {  // (uniform)
        uint64_t* const stage = reinterpret_cast<uint64_t*>(s_cnt);
        int o = off;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint64_t key = mk_key(v[4 * i + e], lo + 4 * (i * WG + tid) + e);
                if (key >= T) stage[o++] = key;
            }
        }
        __syncthreads();
        for (int j = tid; j < total; j += WG)
            if (s_mid_base + j < MID_ROWCAP) store_dev(&buf[s_mid_base + j], stage[j]);
    } else {
        int o = s_mid_base + off;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint64_t key = mk_key(v[4 * i + e], lo + 4 * (i * WG + tid) + e);
                if (key >= T) {
                    if (o < MID_ROWCAP) store_dev(&buf[o], key);
                    ++o;
                }
            }
        }
    }
    wait_stores();
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(&a.row_ticket[row], 1u) == (uint32_t) (segs - 1);
    __syncthreads();
    if (!s_last) return;

    // ---- the row's last workgroup
    if (tid == 0)
        s_mid_base = (int) __hip_atomic_exchange(&m.fill[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int N = min(s_mid_base, MID_ROWCAP);
    const int k = m.k;
    // Key g of the buffer sits in register g / WG of thread g % WG (the loads issued together). Only the first
    // RV registers hold keys; the loops over them end at the first group of four past RV (a scalar bound: the
    // workgroup's one CU issues every instruction of all 16 waves, so registers that hold nothing would still
    // cost issue slots, and a branch per register costs more than it saves).
    const int RV = __builtin_amdgcn_readfirstlane((N + WG - 1) / WG);
    static_assert(MID_RK % 4 == 0, "groups of four registers");
    uint64_t rk[MID_RK];
#pragma unroll
    for (int r = 0; r < MID_RK; ++r) {
        const int g = tid + r * WG;
        rk[r] = g < N ? load_dev(&buf[g]) : 0ull;
    }
    auto cnt2 = [&](uint64_t t) {
        int c = 0;
#pragma unroll
        for (int r = 0; r < MID_RK; ++r) {
            if (r % 4 == 0 && r >= RV) break;
            c += rk[r] >= t ? 1 : 0;
        }
        return c;
    };
    uint64_t T2 = 1ull;  // (every buffered key: all are numbers)
    if (N > 2 * k + 256) {  // (always when N > MID_SORT)
        uint32_t q1 = 0u, q2 = 0u;
#pragma unroll
        for (int r = 0; r < MID_RK; ++r) {
            if (r % 4 == 0 && r >= RV) break;
            const uint32_t ov = (uint32_t) (rk[r] >> 32);
            q2 = max(q2, min(q1, ov));
            q1 = max(q1, ov);
        }
        const uint32_t tw2 = wave_top2_kth(q1, q2, (k + MID_NW - 1) / MID_NW, lane);
        if (lane == 0) s_mid_w[wave] = tw2;
        __syncthreads();
        uint32_t b2 = 0xffffffffu;
#pragma unroll
        for (int w = 0; w < MID_NW; ++w) b2 = min(b2, s_mid_w[w]);
        T2 = (uint64_t) max(b2, 1u) << 32;
        if (mid_sum(cnt2(T2), lane, wave, par) > MID_SORT) T2 = mid_narrow(a, cnt2, T2, k, MID_SORT, lane, wave, par);
    }
    int n2;
    int o2 = mid_prefix(cnt2(T2), lane, wave, par, &n2);
    n2 = min(n2, MID_SORT);
    uint64_t* const S = reinterpret_cast<uint64_t*>(s_cnt);  // (the count table is no longer needed)
    int P = 64;
    while (P < n2) P <<= 1;
    for (int i = n2 + tid; i < P; i += WG) S[i] = 0ull;
#pragma unroll
    for (int r = 0; r < MID_RK; ++r) {
        if (r % 4 == 0 && r >= RV) break;
        if (rk[r] >= T2) {
            if (o2 < MID_SORT) S[o2] = rk[r];
            ++o2;
        }
    }
    __syncthreads();
    // (top-k <= 256: the one-register form up to 1,024 keys, else the generic one; together they add less code to
    // this kernel than the templated forms, whose size changed the segment phase's schedule)
    int ko;
    if constexpr (BIGK) ko = mid_sort_big(P, lane, wave);
    else ko = P <= MID_WG ? mid_sort_r<1>(P, lane, wave) : mid_sort(P, lane, wave);
    sorted_tail(a, row, S + ko, min(k, n2), reinterpret_cast<double*>(S + (MID_SORT - ko)), cin, FastKeyFmt{});
}

// LDS of the history count table: 4 bytes per id for 4-wave workgroups, 2 for 16-wave ones.
template <bool P, int NW, int EPT>
constexpr size_t table_bytes() {
    return P ? (size_t) NW * 64 * EPT * (NW > 4 ? 2 : 4) : 0;
}

template <bool G, bool P, bool F, int NW, int EPT>
hipError_t launch_cfg(const RowsArgs& a, hipStream_t s) {
    constexpr size_t lds = table_bytes<P, NW, EPT>();
    hipLaunchKernelGGL((rows_kernel<G, P, F, NW, EPT>), dim3(rows_grid(a)), dim3(NW * 64), lds, s, a);
    return hipGetLastError();
}

template <bool G, bool P, bool F>
hipError_t launch_gpf(const RowsArgs& a, hipStream_t s) {
    switch (a.seg_len) {
        case 1024: return launch_cfg<G, P, F, 4, 4>(a, s);
        case 2048: return launch_cfg<G, P, F, 4, 8>(a, s);
        case 4096: return launch_cfg<G, P, F, 4, 16>(a, s);
        case 8192: return launch_cfg<G, P, F, 4, 32>(a, s);
        case 16384: return launch_cfg<G, P, F, 16, 16>(a, s);
        case 32768: return launch_cfg<G, P, F, 16, 32>(a, s);
        case 65536: return launch_cfg<G, P, F, 16, 64>(a, s);
        default: return hipErrorInvalidValue;
    }
}

template <bool G, bool P>
hipError_t launch_gp(const RowsArgs& a, hipStream_t s) {
    return rows_full(a.logits, a.row_stride, a.V, a.seg_len) ? launch_gpf<G, P, true>(a, s)
                                                               : launch_gpf<G, P, false>(a, s);
}

template <bool G, bool P, bool F, int NW, int EPT>
hipError_t allow_lds() {
    constexpr size_t b = table_bytes<P, NW, EPT>();
    if (b <= 65536) return hipSuccess;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&rows_kernel<G, P, F, NW, EPT>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int) b);
}

}  // namespace

int rows_grid(const RowsArgs& a) {
    const int w = a.n_rows * a.segs;
    return a.xcd_map ? ((w + 7) & ~7) : w;
}

hipError_t prepare_rows_kernels() {
    hipError_t e = allow_lds<false, true, false, 16, 64>();
    if (e == hipSuccess) e = allow_lds<true, true, false, 16, 64>();
    if (e == hipSuccess) e = allow_lds<false, true, true, 16, 64>();
    if (e == hipSuccess) e = allow_lds<true, true, true, 16, 64>();
    return e;
}

hipError_t launch_rows(const RowsArgs& a, bool greedy, bool penalize, hipStream_t s) {
    if (a.p.k < 1 || a.p.k > KCAP) return hipErrorInvalidValue;
    if (greedy) return penalize ? launch_gp<true, true>(a, s) : launch_gp<true, false>(a, s);
    return penalize ? launch_gp<false, true>(a, s) : launch_gp<false, false>(a, s);
}

int wide_id_bits(int V) {
    int b = 1;
    while (b < 31 && (1ll << b) < (long long) V) ++b;
    return b;
}

hipError_t launch_wide(const RowsArgs& a, const WideArgs& w, bool penalize, hipStream_t s) {
    if (w.k <= KCAP || w.k > a.V || w.chunks != (w.k + WT_CHUNK - 1) / WT_CHUNK) return hipErrorInvalidValue;
    const int tile = sort_tile_keys(a.n_rows, (size_t) a.V);
    if (penalize) {
        const dim3 g((unsigned) (a.n_rows * ((a.V + WIDE_SEG - 1) / WIDE_SEG)));
        constexpr size_t lds = WIDE_SEG * sizeof(uint32_t);
        if (tile == WIDE_SEG) hipLaunchKernelGGL(wide_keys_kernel<1>, g, dim3(WIDE_WG), lds, s, a, w);
        else if (tile == WIDE_SEG / 2) hipLaunchKernelGGL(wide_keys_kernel<2>, g, dim3(WIDE_WG), lds, s, a, w);
        else hipLaunchKernelGGL(wide_keys_kernel<0>, g, dim3(WIDE_WG), lds, s, a, w);
    } else {
        // one workgroup per sort tile, which also counts the sort's first digit
        const dim3 g((unsigned) (a.n_rows * ((a.V + tile - 1) / tile)));
        if (tile == 8192) hipLaunchKernelGGL(wide_keys_hist_kernel<8192>, g, dim3(WKH_WG), 0, s, a, w);
        else if (tile == 4096) hipLaunchKernelGGL(wide_keys_hist_kernel<4096>, g, dim3(WKH_WG), 0, s, a, w);
        else hipLaunchKernelGGL(wide_keys_hist_kernel<SORT_TILE_MIN>, g, dim3(WKH_WG), 0, s, a, w);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    uint64_t* sorted = nullptr;
    // Each row's keys are sorted on their own. They are written in id order and the sort is stable, so sorting on
    // the value field alone leaves equal values in ascending id order, as the id field would: its passes are
    // skipped (4 passes of 8 bits).
    const bool counted = !penalize || tile <= WIDE_SEG;  // the keys kernel wrote the first pass's counts
    e = sort_keys_desc(w.keys, w.sorted, a.n_rows, (size_t) a.V, w.id_bits, 32 + w.id_bits, w.counts, counted,
                       &sorted, s);
    if (e != hipSuccess) return e;
    // the tail reads the sorted buffer and keeps its terms in the other one: the three chains, each mapped per
    // chunk and resolved per row
    WideArgs t = w;
    t.sorted = sorted;
    t.keys = sorted == w.keys ? w.sorted : w.keys;
    const dim3 gc((unsigned) (a.n_rows * w.chunks)), gr((unsigned) a.n_rows);
    hipLaunchKernelGGL(wt_terms_kernel, gc, dim3(WT_WG), 0, s, a, t);
    hipLaunchKernelGGL(wt_maps_kernel<0>, gc, dim3(WT_WG), 0, s, a, t);
    hipLaunchKernelGGL(wt_resolve_kernel<0>, gr, dim3(TAIL_WG), 0, s, a, t);
    hipLaunchKernelGGL(wt_probs_kernel, gc, dim3(WT_WG), 0, s, a, t);
    hipLaunchKernelGGL(wt_maps_kernel<1>, gc, dim3(WT_WG), 0, s, a, t);
    hipLaunchKernelGGL(wt_resolve_kernel<1>, gr, dim3(TAIL_WG), 0, s, a, t);
    hipLaunchKernelGGL(wt_maps_kernel<2>, gc, dim3(WT_WG), 0, s, a, t);
    hipLaunchKernelGGL(wt_resolve_kernel<2>, gr, dim3(TAIL_WG), 0, s, a, t);
    return hipGetLastError();
}

hipError_t launch_mid(const RowsArgs& a, const MidArgs& m, bool penalize, hipStream_t s) {
    if (m.k <= KCAP || m.k > MID_KMAX || a.segs != mid_segments(a.V) || m.cap < m.k ||
        (int64_t) m.cap * a.segs > MID_ROWCAP)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned) (a.n_rows * a.segs));
    // top-k above MID_BIGK: the instantiation with the register-templated sort (k = 512 / 1,024: -1.0 / -2.2 us;
    // at k = 65 / 256 that instantiation is 0.9 / 0.2 us slower, its segment phase scheduled differently)
    const size_t lp = MID_SEG * sizeof(uint32_t), ln = 2 * MID_SORT * sizeof(uint64_t);
    if (m.k > MID_BIGK) {
        if (penalize) hipLaunchKernelGGL((mid_kernel<true, true>), grid, dim3(MID_WG), lp, s, a, m);
        else hipLaunchKernelGGL((mid_kernel<false, true>), grid, dim3(MID_WG), ln, s, a, m);
    } else {
        if (penalize) hipLaunchKernelGGL((mid_kernel<true, false>), grid, dim3(MID_WG), lp, s, a, m);
        else hipLaunchKernelGGL((mid_kernel<false, false>), grid, dim3(MID_WG), ln, s, a, m);
    }
    return hipGetLastError();
}

hipError_t prepare_mid_kernels() {
    const int lp = (int) (MID_SEG * sizeof(uint32_t)), ln = (int) (2 * MID_SORT * sizeof(uint64_t));
    const void* k[4] = {reinterpret_cast<const void*>(&mid_kernel<true, false>),
                        reinterpret_cast<const void*>(&mid_kernel<true, true>),
                        reinterpret_cast<const void*>(&mid_kernel<false, false>),
                        reinterpret_cast<const void*>(&mid_kernel<false, true>)};
    const int lds[4] = {lp, lp, ln, ln};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 4 && e == hipSuccess; ++i)
        e = hipFuncSetAttribute(k[i], hipFuncAttributeMaxDynamicSharedMemorySize, lds[i]);
    return e;
}

hipError_t launch_sum_replay(const double* t, int n, double acc0, int mode, double thr, double* out, hipStream_t s) {
    hipLaunchKernelGGL(sum_replay_kernel, dim3(1), dim3(TAIL_WG), 0, s, t, n, acc0, mode, thr, out);
    return hipGetLastError();
}

const void* noop_kernel() { return reinterpret_cast<const void*>(&noop_kernel_impl); }

hipError_t launch_expf_table(uint32_t lo, long long n, float* out, hipStream_t s) {
    const int threads = 256;
    const long long blocks = (n + threads - 1) / threads;
    hipLaunchKernelGGL(expf_table_kernel, dim3((unsigned) blocks), dim3(threads), 0, s, lo, n, out);
    return hipGetLastError();
}

}  // namespace kls

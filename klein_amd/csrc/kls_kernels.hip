// HIP kernels of the gfx950 token sampler.
//
// One fused kernel samples a batch of rows (klein src/sampler.cpp:17-89 per row, plus the verify accept rule of
// src/engine.cpp:563-575 across rows). Grid = (segments, rows). A workgroup of 4 waves holds one segment of one
// row (256 threads x EPT logits) in registers after a single coalesced HBM read:
//   * penalties (sampler.cpp:18-29) are applied in-register by the one lane holding each id, from a count table
//     of the segment's history ids staged in LDS; nothing is written to the logits or any global buffer;
//   * greedy (sampler.cpp:31-39) keeps a per-lane (max, first id) and reduces across lanes and segments;
//   * top-k (sampler.cpp:42-51): a lower bound of the row's k-th largest value is formed from the lane maxima
//     (each wave's ceil(k/4)-th largest lane maximum; the smallest of the four, so at least k logits of the
//     segment reach it) and from the best bound other workgroups of the row have published; one float compare
//     per logit rejects nearly everything, and the few survivors are ordered by a 64-bit key (value
//     descending, id ascending) with wave64 bitonic networks built from DPP and permlane swaps;
//   * the last workgroup of a row (ticket counter) merges the segment candidate lists into the row's sorted
//     top-k and runs the O(k) tail on one wave: softmax with temperature (expf bit-identical to the host
//     glibc's, sequential double sum), min-p, top-p and the draw (sampler.cpp:53-88);
//   * in a verify step the last row to finish computes the accepted-prefix length.
// Ticket counters and published bounds are reset by their last user, so launches replay from a captured graph
// without memset nodes.
#include "kls_internal.h"

namespace kls {
namespace {

constexpr int WG = 256;
constexpr int NW = WG / 64;
constexpr int CW = 128;  // candidate slots per wave in LDS

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Workgroup memory of the sampling kernel, addressed directly (no generic pointers into LDS).
extern __shared__ __align__(16) uint32_t s_cnt[];  // with penalties: the segment's history counts
__shared__ uint64_t s_cand[NW][CW];                // per-wave candidate regions
__shared__ uint64_t s_list[NW][64];                // per-wave sorted lists
__shared__ uint64_t s_red[NW];
__shared__ uint32_t s_q[NW];
__shared__ int s_n[NW];
__shared__ int s_last;

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

// ---------------------------------------------------------------------------------------------------------
// wave64 cross-lane exchange with lane ^ M: DPP within rows of 16 lanes, permlane swaps across rows.
// Every cross-lane read (DPP, permlane, readlane, ballot) runs in wave-uniform control flow with all 64 lanes
// active, and its result is consumed outside lane-divergent branches: inside such a branch the compiler may
// compute the inputs for the active lanes only.
template <int CTRL>
__device__ __forceinline__ int dpp(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, false);
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

// One compare-exchange step of a bitonic network over one 64-bit key per lane.
template <int SIZE, int STRIDE, bool DESC>
__device__ __forceinline__ uint64_t bitonic_step(uint64_t x, int lane) {
    const uint64_t y = xor_lane64<STRIDE>(x, lane);
    const bool up = (((lane & SIZE) == 0) == DESC);
    const bool lower = (lane & STRIDE) == 0;
    return (lower == up) ? max64(x, y) : min64(x, y);
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

template <int SIZE, int STRIDE>
__device__ __forceinline__ uint32_t bitonic_step32(uint32_t x, int lane) {
    const uint32_t y = (uint32_t) xor_lane<STRIDE>((int) x, lane);
    const bool up = ((lane & SIZE) == 0);
    const bool lower = (lane & STRIDE) == 0;
    return (lower == up) ? max(x, y) : min(x, y);
}

template <int SIZE>
__device__ __forceinline__ uint32_t bitonic_stage32(uint32_t x, int lane) {
    if constexpr (SIZE >= 64) x = bitonic_step32<SIZE, 32>(x, lane);
    if constexpr (SIZE >= 32) x = bitonic_step32<SIZE, 16>(x, lane);
    if constexpr (SIZE >= 16) x = bitonic_step32<SIZE, 8>(x, lane);
    if constexpr (SIZE >= 8) x = bitonic_step32<SIZE, 4>(x, lane);
    if constexpr (SIZE >= 4) x = bitonic_step32<SIZE, 2>(x, lane);
    return bitonic_step32<SIZE, 1>(x, lane);
}

// Descending sort of one 32-bit value per lane.
__device__ __forceinline__ uint32_t sort32_desc(uint32_t x, int lane) {
    x = bitonic_stage32<2>(x, lane);
    x = bitonic_stage32<4>(x, lane);
    x = bitonic_stage32<8>(x, lane);
    x = bitonic_stage32<16>(x, lane);
    x = bitonic_stage32<32>(x, lane);
    return bitonic_stage32<64>(x, lane);
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

// Penalty of src/sampler.cpp:24-25 for an id seen `c` > 0 times: repetition first, then
// l - (presence + frequency * (float)c), each operation rounded separately (no contraction).
__device__ __forceinline__ float penalize(float l, uint32_t c, const SamplingParams& p) {
    if (p.repetition != 1.0f) l = l > 0.0f ? __fdiv_rn(l, p.repetition) : __fmul_rn(l, p.repetition);
    const float f = __fmul_rn(p.frequency, __uint2float_rn(c));
    const float t = __fadd_rn(p.presence, f);
    return __fsub_rn(l, t);
}

// Counts the history ids that fall in [lo, hi) into the LDS table s_cnt[0 .. hi-lo).
__device__ __forceinline__ void stage_history(const RowsArgs& a, int row, int lo, int hi) {
    const int tid = threadIdx.x;
    const int n4 = (hi - lo + 3) & ~3;  // <= seg_len: the table is zeroed in 16-byte stores
    for (int i = 4 * tid; i < n4; i += 4 * WG) *reinterpret_cast<uint4*>(s_cnt + i) = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
    if (a.hist_boff) {
        // bucketed unique ids with counts: read the buckets that overlap [lo, hi)
        const int b0 = lo >> a.bucket_shift;
        const int b1 = min(a.n_buckets, (hi + (1 << a.bucket_shift) - 1) >> a.bucket_shift);
        const int s0 = max(a.hist_boff[b0], 0), s1 = a.hist_boff[b1];
        for (int j = s0 + tid; j < s1; j += WG) {
            const int id = a.hist_ids[j];
            if (id >= lo && id < hi) atomicAdd(&s_cnt[id - lo], (uint32_t) a.hist_w[j]);
        }
    } else if (a.hist_off) {
        // raw ids of this row: every workgroup of the row scans them (from L2) and keeps those in its segment
        const int s0 = max(a.hist_off[row], 0), s1 = a.hist_off[row + 1];
        const int head = min(s1, (s0 + 3) & ~3), body = head + (max(s1 - head, 0) & ~3);
        for (int j = s0 + tid; j < head; j += WG) {
            const int id = a.hist_ids[j];
            if (id >= lo && id < hi) atomicAdd(&s_cnt[id - lo], 1u);
        }
        for (int j = head + 4 * tid; j < body; j += 4 * WG) {
            const int4 q = *reinterpret_cast<const int4*>(a.hist_ids + j);
            if (q.x >= lo && q.x < hi) atomicAdd(&s_cnt[q.x - lo], 1u);
            if (q.y >= lo && q.y < hi) atomicAdd(&s_cnt[q.y - lo], 1u);
            if (q.z >= lo && q.z < hi) atomicAdd(&s_cnt[q.z - lo], 1u);
            if (q.w >= lo && q.w < hi) atomicAdd(&s_cnt[q.w - lo], 1u);
        }
        for (int j = max(body, head) + tid; j < s1; j += WG) {
            const int id = a.hist_ids[j];
            if (id >= lo && id < hi) atomicAdd(&s_cnt[id - lo], 1u);
        }
    }
    if (a.extra_a) {
        const int na = min(max(*a.extra_a_n, 0), PENDING_CAP);
        for (int j = tid; j < na; j += WG) {
            const int id = a.extra_a[j];
            if (id >= lo && id < hi) atomicAdd(&s_cnt[id - lo], 1u);
        }
    }
    if (a.extra_b) {
        const int nb = min(row * a.extra_b_step, VERIFY_MAX_ROWS);
        for (int j = tid; j < nb; j += WG) {
            const int id = a.extra_b[j];
            if (id >= lo && id < hi) atomicAdd(&s_cnt[id - lo], 1u);
        }
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------------------------------------
// Candidate lists. Fast path: survivors of the filter are appended to the wave's LDS region and, when the four
// regions together hold at most 64 keys, sorted once. Larger sets are folded chunk by chunk (sort + bitonic
// merge). The fold lives out of line: it is the only large network, and the streaming loops stay small.

// Descending top-64 of `lst` (descending; ignored when !have) and the n keys of the wave's region.
__device__ __forceinline__ uint64_t fold_region(int wave, int n, uint64_t lst, bool have, int lane) {
    for (int c0 = 0; c0 < n; c0 += 64) {
        const uint64_t key = (c0 + lane < n) ? s_cand[wave][c0 + lane] : 0ull;
        if (!have) {
            lst = sort64<true>(key, lane);
            have = true;
        } else {
            lst = merge64(lst, sort64<false>(key, lane), lane);
        }
    }
    return have ? lst : 0ull;
}

__device__ __forceinline__ uint64_t sort_desc(uint64_t key, int lane) { return sort64<true>(key, lane); }

__device__ __forceinline__ uint64_t merge_desc_asc(uint64_t a, uint64_t b, int lane) { return merge64(a, b, lane); }

// Appends the keys of `pass` lanes to the wave's region; records an overflow instead of folding.
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
        if (pass) s_cand[wave][n + mbcnt(m)] = key;
        n += c;
    }
};

// A wave's descending top-64 over a stream of offers, folding its region whenever it fills (slow paths).
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
            lst = fold_region(wave, n, lst, have, lane);
            have = true;
            n = 0;
            own = rdlane64(lst, k - 1);
            __builtin_amdgcn_wave_barrier();
        }
        if (pass) s_cand[wave][n + mbcnt(m)] = key;
        n += c;
    }
    __device__ __forceinline__ uint64_t finish(int wave, int lane) {
        __builtin_amdgcn_wave_barrier();
        return fold_region(wave, n, lst, have, lane);
    }
};

// The workgroup's descending top-64 of what its waves collected, in wave 0 (other waves get 0); keys below
// `floor_key` are dropped. Returns false (in every thread) if a region overflowed.
__device__ __forceinline__ bool wg_select(const WaveCollect& w, uint64_t floor_key, int lane, int wave, uint64_t* out) {
    if (lane == 0) s_n[wave] = w.overflow ? -1 : w.n;
    __syncthreads();
    const int n0 = s_n[0], n1 = s_n[1], n2 = s_n[2], n3 = s_n[3];
    *out = 0ull;
    if ((n0 | n1 | n2 | n3) < 0) return false;
    if (n0 + n1 + n2 + n3 <= 64) {
        if (wave == 0) {
            uint64_t key = 0ull;
            if (lane < n0)
                key = s_cand[0][lane];
            else if (lane < n0 + n1)
                key = s_cand[1][lane - n0];
            else if (lane < n0 + n1 + n2)
                key = s_cand[2][lane - n0 - n1];
            else if (lane < n0 + n1 + n2 + n3)
                key = s_cand[3][lane - n0 - n1 - n2];
            *out = sort_desc(key < floor_key ? 0ull : key, lane);
        }
        return true;
    }
    uint64_t lst = fold_region(wave, s_n[wave], 0ull, false, lane);
    s_list[wave][lane] = lst >= floor_key ? lst : 0ull;
    __syncthreads();
    if (wave == 0) {
        lst = s_list[0][lane];
#pragma unroll
        for (int o = 1; o < NW; ++o) lst = merge_desc_asc(lst, s_list[o][63 - lane], lane);
        *out = lst;
    }
    return true;
}

// Slow path of a segment (a region overflowed, e.g. many logits equal to the bound): re-read the segment and
// keep exact per-wave lists with folding, then merge. Returns the top-64 in wave 0.
__device__ __forceinline__ uint64_t segment_slow(const RowsArgs& a, const float* __restrict__ L, int lo, int hi, bool pen,
                                                 uint64_t t_row, int lane, int wave) {
    const int k = a.p.k;
    WaveTopK w;
    for (int base = lo + 4 * (wave * 64 + lane); base - 4 * lane < hi; base += 4 * WG) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int id = base + e;
            float x = __uint_as_float(0x7fc00000u);
            if (id < hi) {
                x = L[id];
                if (pen && s_cnt[id - lo] != 0u) x = penalize(x, s_cnt[id - lo], a.p);
            }
            const uint64_t key = x == x ? mk_key(x, id) : 0ull;
            w.offer(wave, key != 0ull && key > max64(t_row, w.own), key, k, lane);
        }
    }
    uint64_t lst = w.finish(wave, lane);
    s_list[wave][lane] = lst;
    __syncthreads();
    if (wave != 0) return 0ull;
    lst = s_list[0][lane];
    for (int o = 1; o < NW; ++o) lst = merge_desc_asc(lst, s_list[o][63 - lane], lane);
    return lst;
}

// Slow path of the row merge: every segment list entry at or above `ts`, folded exactly.
__device__ __forceinline__ uint64_t merge_slow(const uint64_t* cand, int segs, int k, uint64_t ts, int lane, int wave) {
    WaveTopK w;
    for (int s = wave; s < segs; s += NW) {
        const uint64_t key = lane < k ? load_dev(&cand[(int64_t) s * KCAP + lane]) : 0ull;
        w.offer(wave, key != 0ull && key >= ts && key > w.own, key, k, lane);
    }
    uint64_t lst = w.finish(wave, lane);
    s_list[wave][lane] = lst;
    __syncthreads();
    if (wave != 0) return 0ull;
    lst = s_list[0][lane];
    for (int o = 1; o < NW; ++o) lst = merge_desc_asc(lst, s_list[o][63 - lane], lane);
    return lst;
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

__device__ int sample_tail(uint64_t lst, int kk, const SamplingParams& p, double u, int lane, float* dbg_probs,
                           int32_t* dbg_meta) {
    if (kk == 0) return 0;
    const bool act = lane < kk;
    const float v = act ? unord_f32((uint32_t) (lst >> 32)) : 0.0f;
    const int id = act ? key_id(lst) : -1;
    // softmax with temperature (:53-60)
    const float maxl = rdlanef(v, 0);
    const float x = __fdiv_rn(__fsub_rn(v, maxl), p.temperature);
    const float e = act ? expf_glibc(x) : 0.0f;
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

// Publishes row `row`'s token: device output, and for the host one 64-bit word (sequence number, token).
__device__ __forceinline__ void publish(const RowsArgs& a, int row, int tok) {
    a.out_tokens[row] = tok;
    a.row_ticket[row] = 0u;
    if (a.share_bounds) a.row_thr[row] = 0ull;
    if (a.host_res && row < VERIFY_MAX_ROWS)
        __hip_atomic_store(&a.host_res->row_word[row], ((uint64_t) a.call->seq << 32) | (uint32_t) tok,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

template <bool GREEDY, bool PENALIZE, int EPT>
__global__ __launch_bounds__(WG) void rows_kernel(RowsArgs a) {
    constexpr int SEG = WG * EPT;
    constexpr int NV = EPT / 4;  // float4 per thread
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
    const int row = item / a.segs, seg = item - row * a.segs;
    const int lo = seg * SEG;
    const int hi = min(a.V, lo + SEG);
    const float* __restrict__ L = a.logits + (int64_t) row * a.row_stride;
    const bool vec = ((a.row_stride & 3) == 0) && ((reinterpret_cast<uintptr_t>(a.logits) & 15u) == 0);
    const int k = a.p.k;
    uint64_t* seg_out = a.seg_cand + ((int64_t) row * a.segs + seg) * KCAP;
    // a bound other workgroups of the row published (large grids only): read before the logits arrive
    const uint64_t t_row =
        a.share_bounds ? __hip_atomic_load(&a.row_thr[row], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;

    // ---- one coalesced read of the segment: thread t holds ids lo + 4*(i*256 + t) + e
    float v[EPT];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int base = lo + 4 * (i * WG + tid);
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
    if (PENALIZE) {
        stage_history(a, row, lo, hi);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int off = 4 * (i * WG + tid);
            if (lo + off >= hi) continue;
            uint32_t c[4];
            if (lo + off + 3 < hi) {
                const uint4 q = *reinterpret_cast<const uint4*>(s_cnt + off);
                c[0] = q.x;
                c[1] = q.y;
                c[2] = q.z;
                c[3] = q.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) c[e] = (lo + off + e < hi) ? s_cnt[off + e] : 0u;
            }
            if ((c[0] | c[1] | c[2] | c[3]) != 0u) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (c[e] != 0u) v[4 * i + e] = penalize(v[4 * i + e], c[e], a.p);
            }
        }
    }

    if (GREEDY) {
        // src/sampler.cpp:31-39: a thread's ids ascend with (i, e), so strict '>' keeps the lowest id.
        float best_v = -INFINITY;
        int best_id = 0;
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (v[4 * i + e] > best_v) {
                    best_v = v[4 * i + e];
                    best_id = lo + 4 * (i * WG + tid) + e;
                }
        uint64_t key = best_v > -INFINITY ? mk_key(best_v, best_id) : 0ull;
        key = wave_max64(key, lane);
        if (lane == 0) s_red[wave] = key;
        __syncthreads();
        if (tid == 0) store_dev(&seg_out[0], max64(max64(s_red[0], s_red[1]), max64(s_red[2], s_red[3])));
    } else {
        // ---- lower bound of the row's k-th value: each wave's ceil(k/4)-th largest lane maximum, smallest of
        // the four (at least 4*ceil(k/4) >= k logits of this segment reach it)
        // (per lane: the largest and second largest logit; the wave bound is the larger of the k4-th largest lane
        // maximum and the ceil(k4/2)-th largest second maximum, each reached by at least k4 logits; NaN counts
        // as -inf here and never reaches a bound)
        float m1 = -INFINITY, m2 = -INFINITY;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const float x = v[i] == v[i] ? v[i] : -INFINITY;
            m2 = fmaxf(m2, fminf(m1, x));
            m1 = fmaxf(m1, x);
        }
        const uint32_t s1 = sort32_desc(ord_f32(m1), lane);
        const uint32_t s2 = sort32_desc(ord_f32(m2), lane);
        const int k4 = (k + NW - 1) / NW;
        const uint32_t q1 = (uint32_t) __builtin_amdgcn_readlane((int) s1, k4 - 1);  // all lanes active
        const uint32_t q2 = (uint32_t) __builtin_amdgcn_readlane((int) s2, (k4 + 1) / 2 - 1);
        if (lane == 0) s_q[wave] = max(q1, q2);
        __syncthreads();
        const uint32_t q = min(min(s_q[0], s_q[1]), min(s_q[2], s_q[3]));
        const float t_f = fmaxf(floor32(q), floor64(t_row));

        // ---- filter: one compare per logit; survivors go to the wave's LDS region
        WaveCollect w;
#pragma unroll
        for (int i = 0; i < NV; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float x = v[4 * i + e];
                const bool pass = x >= t_f;
                if (ballot(pass)) {
                    const uint64_t key = mk_key(x, lo + 4 * (i * WG + tid) + e);
                    w.offer(wave, pass && key > t_row, key);
                }
            }
        uint64_t lst;
        if (!wg_select(w, 0ull, lane, wave, &lst)) lst = segment_slow(a, L, lo, hi, PENALIZE, t_row, lane, wave);
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
    // its increment returned.
    __syncthreads();
    if (tid == 0) {
        wait_stores();
        const uint32_t prev = atomicAdd(&a.row_ticket[row], 1u);
        s_last = (prev == (uint32_t) (a.segs - 1));
    }
    __syncthreads();
    if (!s_last) return;
    const uint64_t* cand = a.seg_cand + (int64_t) row * a.segs * KCAP;

    if (GREEDY) {
        uint64_t m = 0ull;
        for (int s = tid; s < a.segs; s += WG) m = max64(m, load_dev(&cand[(int64_t) s * KCAP]));
        m = wave_max64(m, lane);
        if (lane == 0) s_red[wave] = m;
        __syncthreads();
        if (tid != 0) return;
        m = max64(max64(s_red[0], s_red[1]), max64(s_red[2], s_red[3]));
        if (a.dbg_meta) {
            a.dbg_meta[row * 2] = 0;
            a.dbg_meta[row * 2 + 1] = 0;
        }
        publish(a, row, m ? key_id(m) : 0);  // all -inf / NaN: the reference returns id 0
        return;
    }

    // Lower bound of the row's k-th value from the heads of the segment lists: H = the first J = ceil(k/segs)
    // entries of every list (J*segs >= k distinct logits). With |H| <= 64 the bound is the k-th largest value in H;
    // otherwise H is dealt round-robin to the four waves and the bound is the smallest of the waves'
    // ceil(k/4)-th largest values. Either way at least k logits reach it, so the row's top-k are among the list
    // entries at or above it. Up to 64 lists stay in registers (16 per wave) while the bound is formed.
    constexpr int RB = 16;
    const int J = (k + a.segs - 1) / a.segs;
    const int nH = min(a.segs * J, WG);
    const bool one = nH <= 64;
    const int h = one ? (wave == 0 ? lane : WG) : lane * NW + wave;
    const uint64_t hv = h < nH ? load_dev(&cand[(int64_t) (h / J) * KCAP + h % J]) : 0ull;
    const bool inreg = a.segs <= NW * RB;
    uint64_t key[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int s = wave + NW * r;
        key[r] = (inreg && s < a.segs && lane < k) ? load_dev(&cand[(int64_t) s * KCAP + lane]) : 0ull;
    }
    const uint32_t sv = sort32_desc((uint32_t) (hv >> 32), lane);
    const uint32_t qw = (uint32_t) rdlanei((int) sv, (one ? k : (k + NW - 1) / NW) - 1);  // all lanes active
    if (lane == 0) s_q[wave] = (one && wave != 0) ? 0xffffffffu : qw;
    __syncthreads();
    const uint64_t ts = (uint64_t) min(min(s_q[0], s_q[1]), min(s_q[2], s_q[3])) << 32;
    WaveCollect w;
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
    if (!wg_select(w, 0ull, lane, wave, &lst)) {
        __syncthreads();
        lst = merge_slow(cand, a.segs, k, ts, lane, wave);
    }
    if (wave != 0) return;
    const int kk = min(k, (int) __popcll(ballot(lst != 0ull && lane < k)));
    if (a.dbg_keys) a.dbg_keys[row * KCAP + lane] = lane < kk ? lst : 0ull;
    const int tok = sample_tail(lst, kk, a.p, a.u[row], lane, a.dbg_probs ? a.dbg_probs + row * KCAP : nullptr,
                                a.dbg_meta ? a.dbg_meta + row * 2 : nullptr);
    if (lane == 0) publish(a, row, tok);
}

__global__ void expf_table_kernel(uint32_t lo, long long n, float* out) {
    const long long i = (long long) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = expf_glibc(__uint_as_float(lo + (uint32_t) i));
}

template <bool G, bool P>
hipError_t launch_ept(const RowsArgs& a, hipStream_t s) {
    const dim3 grid(rows_grid(a)), block(WG);
    const size_t lds = P ? (size_t) a.seg_len * sizeof(uint32_t) : 0;
    switch (a.seg_len) {
        case 1024: hipLaunchKernelGGL((rows_kernel<G, P, 4>), grid, block, lds, s, a); break;
        case 2048: hipLaunchKernelGGL((rows_kernel<G, P, 8>), grid, block, lds, s, a); break;
        case 4096: hipLaunchKernelGGL((rows_kernel<G, P, 16>), grid, block, lds, s, a); break;
        case 8192: hipLaunchKernelGGL((rows_kernel<G, P, 32>), grid, block, lds, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

int rows_grid(const RowsArgs& a) {
    const int w = a.n_rows * a.segs;
    return a.xcd_map ? ((w + 7) & ~7) : w;
}

hipError_t launch_rows(const RowsArgs& a, bool greedy, bool penalize, hipStream_t s) {
    if (a.p.k < 1 || a.p.k > KCAP) return hipErrorInvalidValue;
    if (greedy) return penalize ? launch_ept<true, true>(a, s) : launch_ept<true, false>(a, s);
    return penalize ? launch_ept<false, true>(a, s) : launch_ept<false, false>(a, s);
}

hipError_t launch_expf_table(uint32_t lo, long long n, float* out, hipStream_t s) {
    const int threads = 256;
    const long long blocks = (n + threads - 1) / threads;
    hipLaunchKernelGGL(expf_table_kernel, dim3((unsigned) blocks), dim3(threads), 0, s, lo, n, out);
    return hipGetLastError();
}

}  // namespace kls

// HIP kernels of the gfx950 token sampler.
//
// One fused kernel samples a batch of rows (klein src/sampler.cpp:17-89 per row, plus the verify accept rule of
// src/engine.cpp:563-575 across rows). Grid = (segments, rows); a workgroup of 4 waves streams one segment of
// one row from HBM exactly once:
//   * penalties (sampler.cpp:18-29) are applied in-register by the one lane that streams each id, from a count
//     table of the segment's history ids staged in LDS (no atomics touch the logits or any global buffer);
//   * greedy (sampler.cpp:31-39) keeps a per-lane (max, first id) and reduces across lanes and segments;
//   * top-k (sampler.cpp:42-51) keeps a sorted 64-entry candidate list per wave, one entry per lane, ordered by
//     a 64-bit key (value descending, id ascending); elements below a running lower bound of the row's k-th key
//     are rejected with a single float compare. Lower bounds are shared between the waves of a workgroup
//     (LDS) and the workgroups of a row (a global max), so few elements ever reach the list;
//   * the last workgroup of a row (ticket counter) merges the segment lists into the row's sorted top-k and
//     runs the O(k) tail on one wave: softmax with temperature (bit-exact glibc expf restatement, sequential
//     double sum), min-p, top-p, and the draw (sampler.cpp:53-88);
//   * in a verify step, the last row to finish computes the accepted-prefix length.
// Ticket counters and shared bounds are reset by their last user, so the kernel can be replayed from a
// captured graph without memset nodes.
#include "kls_internal.h"

namespace kls {
namespace {

constexpr int WG = 256;
constexpr int NW = WG / 64;
constexpr int UNROLL = 4;      // tiles of 256 elements in flight per wave
constexpr int SERIAL_MAX = 6;  // up to this many candidates in a slot are inserted one by one

// ---------------------------------------------------------------------------------------------------------
// keys: 32-bit order-preserving image of the f32 value in the high word, ~id in the low word, so that a larger
// 64-bit key means a larger value or, on equal values, a lower id. -0 is folded onto +0 (the reference's
// comparator treats them as equal); NaN maps to the lowest value image.
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

// Largest float f such that every key >= `k` has value >= f (the pre-filter bound for a key threshold).
__device__ __forceinline__ float key_floor(uint64_t k) {
    const uint32_t hi = (uint32_t) (k >> 32);
    return hi == 0u ? -INFINITY : unord_f32(hi);
}

// ---------------------------------------------------------------------------------------------------------
// wave64 helpers
__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

__device__ __forceinline__ uint64_t bperm64(uint64_t x, int src_lane) {
    const int lo = __builtin_amdgcn_ds_bpermute(src_lane << 2, (int) (uint32_t) x);
    const int hi = __builtin_amdgcn_ds_bpermute(src_lane << 2, (int) (uint32_t) (x >> 32));
    return ((uint64_t) (uint32_t) hi << 32) | (uint32_t) lo;
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

__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t min64(uint64_t a, uint64_t b) { return a > b ? b : a; }

__device__ __forceinline__ uint64_t wave_max64(uint64_t x, int lane) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) x = max64(x, bperm64(x, lane ^ m));
    return x;
}

// Bitonic sort of one key per lane into descending order (lane 0 = largest).
__device__ __forceinline__ uint64_t sort64_desc(uint64_t x, int lane) {
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const uint64_t y = bperm64(x, lane ^ stride);
            const bool desc = (lane & size) == 0;
            const bool lower = (lane & stride) == 0;
            x = (lower == desc) ? max64(x, y) : min64(x, y);
        }
    }
    return x;
}

// Top 64 of two descending lists (one entry per lane each), descending.
__device__ __forceinline__ uint64_t merge64_desc(uint64_t a, uint64_t b, int lane) {
    uint64_t c = max64(a, bperm64(b, 63 - lane));  // bitonic: a descending, reversed b ascending
#pragma unroll
    for (int stride = 32; stride > 0; stride >>= 1) {
        const uint64_t y = bperm64(c, lane ^ stride);
        c = ((lane & stride) == 0) ? max64(c, y) : min64(c, y);
    }
    return c;
}

// Inserts key x (distinct from every entry) into a descending list; the smallest entry falls off.
__device__ __forceinline__ uint64_t insert64_desc(uint64_t lst, uint64_t x, int lane) {
    const int pos = __popcll(ballot(lst > x));
    const uint64_t up = bperm64(lst, lane - 1);
    return lane < pos ? lst : (lane == pos ? x : up);
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

// ---------------------------------------------------------------------------------------------------------
// Loads the 4 logits of one lane in one tile (element ids base..base+3); ids at or past `hi` read as NaN.
__device__ __forceinline__ void load4(const float* __restrict__ L, int base, int hi, bool vec, float (&v)[4]) {
    if (vec && base + 3 < hi) {
        const float4 f = *reinterpret_cast<const float4*>(L + base);
        v[0] = f.x;
        v[1] = f.y;
        v[2] = f.z;
        v[3] = f.w;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (base + e < hi) ? L[base + e] : __uint_as_float(0x7fc00000u);
    }
}

// Applies the penalties to the 4 logits at ids base..base+3 from the segment's LDS count table.
__device__ __forceinline__ void penalize4(const uint32_t* s_cnt, int lo, int base, int hi, const SamplingParams& p,
                                          float (&v)[4]) {
    uint32_t c[4];
    if (base + 3 < hi) {
        const uint4 q = *reinterpret_cast<const uint4*>(s_cnt + (base - lo));
        c[0] = q.x;
        c[1] = q.y;
        c[2] = q.z;
        c[3] = q.w;
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) c[e] = (base + e < hi) ? s_cnt[base + e - lo] : 0u;
    }
    if ((c[0] | c[1] | c[2] | c[3]) != 0u) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (c[e] != 0u) v[e] = penalize(v[e], c[e], p);
    }
}

// Adds history ids in [lo, hi) to the LDS count table.
__device__ __forceinline__ void stage_history(const RowsArgs& a, int row, int lo, int hi, uint32_t* s_cnt) {
    const int tid = threadIdx.x;
    for (int i = tid; i < hi - lo; i += WG) s_cnt[i] = 0u;
    __syncthreads();
    if (a.hist_boff) {
        const int32_t* bo = a.hist_boff + (int64_t) (a.hist_shared ? 0 : row) * (a.n_buckets + 1);
        const int b0 = lo >> a.bucket_shift;
        const int b1 = min(a.n_buckets, (hi + (1 << a.bucket_shift) - 1) >> a.bucket_shift);
        const int s0 = bo[b0], s1 = bo[b1];
        for (int j = max(s0, 0) + tid; j < min(s1, a.hist_cap); j += WG) {
            const int id = a.hist_ids[j];
            if (id >= lo && id < hi) atomicAdd(&s_cnt[id - lo], a.hist_w ? (uint32_t) a.hist_w[j] : 1u);
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

// The O(k) tail of src/sampler.cpp:53-88 on one wave. `lst` holds the row's candidates in descending key order,
// one per lane; the first kk are the top-k. Returns the drawn id (uniform across the wave).
__device__ int sample_tail(uint64_t lst, int kk, const SamplingParams& p, double u, int lane, float* dbg_probs,
                           int32_t* dbg_meta) {
    const bool act = lane < kk;
    const float v = act ? unord_f32((uint32_t) (lst >> 32)) : 0.0f;
    const int id = act ? key_id(lst) : -1;
    // softmax with temperature (:53-60)
    const float maxl = rdlanef(v, 0);
    const float x = __fdiv_rn(__fsub_rn(v, maxl), p.temperature);
    const float e = act ? expf_glibc(x) : 0.0f;
    double sum = 0.0;
    for (int i = 0; i < kk; ++i) sum = __dadd_rn(sum, (double) rdlanef(e, i));
    const float pr = act ? __double2float_rn(__ddiv_rn((double) e, sum)) : 0.0f;
    int n = kk;
    // min-p (:62-68): keep the prefix while p >= p0*min_p
    if (p.min_p > 0.0f) {
        const float thr = __fmul_rn(rdlanef(pr, 0), p.min_p);
        const uint64_t fail = ballot(act && lane >= 1 && !(pr >= thr));
        if (fail) n = __builtin_ctzll(fail);
    }
    // top-p (:69-79): sequential double cumulative sum, stop at the first cum >= top_p
    if (p.top_p < 1.0f) {
        double cum = 0.0;
        int m = 0;
        while (m < n) {
            cum = __dadd_rn(cum, (double) rdlanef(pr, m));
            ++m;
            if (cum >= (double) p.top_p) break;
        }
        n = max(m, 1);
    }
    // draw (:80-88) with r = u*(total-0)+0 as std::uniform_real_distribution<double>(0, total)
    double total = 0.0;
    for (int i = 0; i < n; ++i) total = __dadd_rn(total, (double) rdlanef(pr, i));
    double r = __dadd_rn(__dmul_rn(u, __dsub_rn(total, 0.0)), 0.0);
    int tok = rdlanei(id, n - 1);
    for (int i = 0; i < n; ++i) {
        r = __dsub_rn(r, (double) rdlanef(pr, i));
        if (r <= 0.0) {
            tok = rdlanei(id, i);
            break;
        }
    }
    if (dbg_probs) dbg_probs[lane] = pr;
    if (dbg_meta && lane == 0) {
        dbg_meta[0] = kk;
        dbg_meta[1] = n;
    }
    return tok;
}

// Verify step: after every row's token is final, the last row computes the accepted-prefix length
// (engine.cpp:571-573: accept draft i+1 while it equals t_i) and publishes tokens + count to the host block.
__device__ void finish_step(const RowsArgs& a) {
    __threadfence_system();
    const uint32_t prev = atomicAdd(a.step_ticket, 1u);
    if (prev != (uint32_t) (a.n_rows - 1)) return;
    *a.step_ticket = 0u;
    __threadfence();
    int acc = 0;
    if (a.drafts) {
        while (acc < a.n_rows - 1 &&
               __hip_atomic_load(&a.out_tokens[acc], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == a.drafts[acc])
            ++acc;
        *a.out_accepted = acc;
    }
    if (a.host_res) {
        for (int i = 0; i < a.n_rows && i < VERIFY_MAX_ROWS; ++i)
            a.host_res->tokens[i] = __hip_atomic_load(&a.out_tokens[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.host_res->accepted = acc;
        __threadfence_system();
        __hip_atomic_store(&a.host_res->seq, a.call ? a.call->seq : 0u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

template <bool GREEDY, bool PENALIZE>
__global__ __launch_bounds__(WG) void rows_kernel(RowsArgs a) {
    extern __shared__ __align__(16) uint32_t s_cnt[];  // PENALIZE: the segment's history counts
    __shared__ uint64_t s_list[NW][KCAP];
    __shared__ uint64_t s_red[NW];
    __shared__ volatile uint64_t s_thr[NW];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const int seg = blockIdx.x, row = blockIdx.y;
    const int lo = seg * a.seg_len;
    const int hi = min(a.V, lo + a.seg_len);
    const float* __restrict__ L = a.logits + (int64_t) row * a.row_stride;
    const bool vec = ((a.row_stride & 3) == 0) && ((reinterpret_cast<uintptr_t>(a.logits) & 15u) == 0);
    const int k = a.p.k;
    const int n_tiles = (hi - lo + 255) >> 8;
    uint64_t* seg_out = a.seg_cand + ((int64_t) row * a.segs + seg) * KCAP;

    if (PENALIZE) stage_history(a, row, lo, hi, s_cnt);

    if (GREEDY) {
        // src/sampler.cpp:31-39: per lane, ids ascend through the stream, so strict '>' keeps the lowest id.
        float best_v = -INFINITY;
        int best_id = 0;
        for (int t0 = wave; t0 < n_tiles; t0 += NW * UNROLL) {
            float v[UNROLL][4];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const int base = lo + (t0 + u * NW) * 256 + lane * 4;
                load4(L, base, (t0 + u * NW < n_tiles) ? hi : lo, vec, v[u]);
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const int base = lo + (t0 + u * NW) * 256 + lane * 4;
                if (PENALIZE) penalize4(s_cnt, lo, base, (t0 + u * NW < n_tiles) ? hi : lo, a.p, v[u]);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (v[u][e] > best_v) {
                        best_v = v[u][e];
                        best_id = base + e;
                    }
            }
        }
        uint64_t key = best_v > -INFINITY ? mk_key(best_v, best_id) : 0ull;
        key = wave_max64(key, lane);
        if (lane == 0) s_red[wave] = key;
        __syncthreads();
        if (tid == 0) {
            uint64_t m = s_red[0];
            for (int w = 1; w < NW; ++w) m = max64(m, s_red[w]);
            seg_out[0] = m;
        }
    } else {
        if (tid < NW) s_thr[tid] = 0ull;
        __syncthreads();
        uint64_t lst = 0ull;  // this wave's candidates, descending, one per lane
        uint64_t own = 0ull;  // key of this wave's k-th candidate (0 while fewer than k)
        uint64_t ext = 0ull;  // best lower bound published by other waves / workgroups of the row
        uint64_t pub_lds = 0ull, pub_glb = 0ull;
        float thr_f = -INFINITY;
        bool first = true;
        int group = 0;
        for (int t0 = wave; t0 < n_tiles; t0 += NW * UNROLL, ++group) {
            float v[UNROLL][4];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const int base = lo + (t0 + u * NW) * 256 + lane * 4;
                load4(L, base, (t0 + u * NW < n_tiles) ? hi : lo, vec, v[u]);
            }
            if (PENALIZE) {
#pragma unroll
                for (int u = 0; u < UNROLL; ++u) {
                    const int base = lo + (t0 + u * NW) * 256 + lane * 4;
                    penalize4(s_cnt, lo, base, (t0 + u * NW < n_tiles) ? hi : lo, a.p, v[u]);
                }
            }
            if (first) {
                // Warm-up bound: the k-th largest of the 64 lane maxima. At least k elements of this group are
                // >= it, so no element of the row's top-k is below it.
                first = false;
                float m = -INFINITY;
#pragma unroll
                for (int u = 0; u < UNROLL; ++u)
#pragma unroll
                    for (int e = 0; e < 4; ++e) m = fmaxf(m, v[u][e]);
                const uint64_t km = sort64_desc((uint64_t) ord_f32(m) << 32, lane);
                thr_f = fmaxf(thr_f, key_floor(rdlane64(km, k - 1)));
            }
            uint64_t msk[UNROLL][4];
            uint64_t any = 0ull;
#pragma unroll
            for (int u = 0; u < UNROLL; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    msk[u][e] = ballot(v[u][e] >= thr_f);
                    any |= msk[u][e];
                }
            if (any) {
                uint64_t thr = max64(own, ext);
#pragma unroll
                for (int u = 0; u < UNROLL; ++u) {
                    const int tbase = lo + (t0 + u * NW) * 256;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        uint64_t mm = msk[u][e];
                        if (!mm) continue;
                        if (__popcll(mm) <= SERIAL_MAX) {
                            while (mm) {
                                const int j = __builtin_ctzll(mm);
                                mm &= mm - 1;
                                const uint64_t key = mk_key(rdlanef(v[u][e], j), tbase + j * 4 + e);
                                if (key > thr) {
                                    lst = insert64_desc(lst, key, lane);
                                    own = rdlane64(lst, k - 1);
                                    thr = max64(own, ext);
                                }
                            }
                        } else {
                            uint64_t key = mk_key(v[u][e], tbase + lane * 4 + e);
                            key = ((mm >> lane) & 1ull) && key > thr ? key : 0ull;
                            lst = merge64_desc(lst, sort64_desc(key, lane), lane);
                            own = rdlane64(lst, k - 1);
                            thr = max64(own, ext);
                        }
                    }
                }
            }
            // share the bound: every group inside the workgroup, every 4th group across the row
            if (own > pub_lds) {
                if (lane == 0) s_thr[wave] = own;
                pub_lds = own;
            }
#pragma unroll
            for (int w = 0; w < NW; ++w) ext = max64(ext, s_thr[w]);
            if ((group & 3) == 3) {
                if (own > pub_glb) {
                    if (lane == 0) atomicMax((unsigned long long*) &a.row_thr[row], (unsigned long long) own);
                    pub_glb = own;
                }
                ext = max64(ext, __hip_atomic_load(&a.row_thr[row], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            }
            thr_f = fmaxf(thr_f, key_floor(max64(own, ext)));
        }
        s_list[wave][lane] = lst;
        __syncthreads();
        if (wave == 0) {
            for (int w = 1; w < NW; ++w) lst = merge64_desc(lst, s_list[w][lane], lane);
            seg_out[lane] = lane < k ? lst : 0ull;
            own = rdlane64(lst, k - 1);
            if (lane == 0 && own > pub_glb)
                atomicMax((unsigned long long*) &a.row_thr[row], (unsigned long long) own);
        }
    }

    // ---- last workgroup of the row merges the segment results
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        const uint32_t prev = atomicAdd(&a.row_ticket[row], 1u);
        s_last = (prev == (uint32_t) (a.segs - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const uint64_t* cand = a.seg_cand + (int64_t) row * a.segs * KCAP;

    if (GREEDY) {
        uint64_t m = 0ull;
        for (int s = tid; s < a.segs; s += WG)
            m = max64(m, __hip_atomic_load(&cand[(int64_t) s * KCAP], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        m = wave_max64(m, lane);
        if (lane == 0) s_red[wave] = m;
        __syncthreads();
        if (tid != 0) return;
        for (int w = 1; w < NW; ++w) m = max64(m, s_red[w]);
        m = max64(m, s_red[0]);
        const int tok = m ? key_id(m) : 0;  // all -inf / NaN: the reference returns id 0
        a.out_tokens[row] = tok;
        if (a.dbg_meta) {
            a.dbg_meta[row * 2] = 0;
            a.dbg_meta[row * 2 + 1] = 0;
        }
        a.row_ticket[row] = 0u;
        a.row_thr[row] = 0ull;
        finish_step(a);
        return;
    }

    // lower bound for the row's k-th key: the best k-th of any segment (or any published bound)
    uint64_t ts = 0ull;
    for (int s = tid; s < a.segs; s += WG)
        ts = max64(ts, __hip_atomic_load(&cand[(int64_t) s * KCAP + k - 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    ts = wave_max64(ts, lane);
    if (lane == 0) s_red[wave] = ts;
    __syncthreads();
    ts = max64(max64(s_red[0], s_red[1]), max64(s_red[2], s_red[3]));
    uint64_t lst = 0ull, own = 0ull;
    for (int s = wave; s < a.segs; s += NW) {
        const uint64_t key = lane < k ? __hip_atomic_load(&cand[(int64_t) s * KCAP + lane], __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT)
                                      : 0ull;
        const bool pass = key != 0ull && key >= ts && key > own;
        uint64_t mm = ballot(pass);
        if (!mm) continue;
        if (__popcll(mm) <= 4) {
            while (mm) {
                const int j = __builtin_ctzll(mm);
                mm &= mm - 1;
                const uint64_t x = rdlane64(key, j);
                if (x > own) {
                    lst = insert64_desc(lst, x, lane);
                    own = rdlane64(lst, k - 1);
                }
            }
        } else {
            lst = merge64_desc(lst, pass ? key : 0ull, lane);  // a passing set is a prefix of a sorted list
            own = rdlane64(lst, k - 1);
        }
    }
    s_list[wave][lane] = lst;
    __syncthreads();
    if (wave != 0) return;
    for (int w = 1; w < NW; ++w) lst = merge64_desc(lst, s_list[w][lane], lane);
    const int kk = min(k, (int) __popcll(ballot(lst != 0ull && lane < k)));
    if (a.dbg_keys) a.dbg_keys[row * KCAP + lane] = lane < kk ? lst : 0ull;
    const int tok = sample_tail(lst, kk, a.p, a.u[row], lane, a.dbg_probs ? a.dbg_probs + row * KCAP : nullptr,
                                a.dbg_meta ? a.dbg_meta + row * 2 : nullptr);
    if (lane == 0) {
        a.out_tokens[row] = tok;
        a.row_ticket[row] = 0u;
        a.row_thr[row] = 0ull;
        finish_step(a);
    }
}

// One workgroup per row: counting-sort the row's raw history ids into buckets of (1 << bucket_shift) ids and
// record the bucket offsets, so that the sampling kernel finds each segment's ids with two loads.
__global__ __launch_bounds__(1024) void partition_kernel(PartitionArgs a) {
    __shared__ uint32_t s_cnt[MAX_BUCKETS];
    __shared__ uint32_t s_wsum[16];
    const int row = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const int s = max(a.hist_off[row], 0), e = min(a.hist_off[row + 1], a.cap);
    for (int b = tid; b < MAX_BUCKETS; b += 1024) s_cnt[b] = 0u;
    __syncthreads();
    for (int j = s + tid; j < e; j += 1024) {
        const int id = a.hist_ids[j];
        if (id >= 0 && id < a.V) atomicAdd(&s_cnt[id >> a.bucket_shift], 1u);
    }
    __syncthreads();
    // exclusive scan of the bucket counts (one per thread)
    const uint32_t c = tid < a.n_buckets ? s_cnt[tid] : 0u;
    uint32_t incl = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t y = (uint32_t) __builtin_amdgcn_ds_bpermute((lane - d) << 2, (int) incl);
        if (lane >= d) incl += y;
    }
    if (lane == 63) s_wsum[wave] = incl;
    __syncthreads();
    uint32_t woff = 0;
    for (int w = 0; w < wave; ++w) woff += s_wsum[w];
    uint32_t total = 0;
    for (int w = 0; w < 16; ++w) total += s_wsum[w];
    const uint32_t excl = woff + incl - c;
    int32_t* bo = a.boff + (int64_t) row * (a.n_buckets + 1);
    if (tid < a.n_buckets) bo[tid] = s + (int) excl;
    if (tid == 0) bo[a.n_buckets] = s + (int) total;  // s + total <= e: only ids read from [s, e) are counted
    __syncthreads();
    if (tid < a.n_buckets) s_cnt[tid] = excl;
    __syncthreads();
    for (int j = s + tid; j < e; j += 1024) {
        const int id = a.hist_ids[j];
        if (id >= 0 && id < a.V) {
            const uint32_t pos = atomicAdd(&s_cnt[id >> a.bucket_shift], 1u);
            a.part_ids[s + (int) pos] = id;
        }
    }
}

__global__ void expf_table_kernel(uint32_t lo, long long n, float* out) {
    const long long i = (long long) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = expf_glibc(__uint_as_float(lo + (uint32_t) i));
}

}  // namespace

hipError_t launch_rows(const RowsArgs& a, bool greedy, bool penalize, hipStream_t s) {
    const dim3 grid(a.segs, a.n_rows), block(WG);
    const size_t lds = penalize ? (size_t) a.seg_len * sizeof(uint32_t) : 0;
    if (greedy) {
        if (penalize)
            hipLaunchKernelGGL((rows_kernel<true, true>), grid, block, lds, s, a);
        else
            hipLaunchKernelGGL((rows_kernel<true, false>), grid, block, lds, s, a);
    } else {
        if (penalize)
            hipLaunchKernelGGL((rows_kernel<false, true>), grid, block, lds, s, a);
        else
            hipLaunchKernelGGL((rows_kernel<false, false>), grid, block, lds, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_partition(const PartitionArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(partition_kernel, dim3(a.n_rows), dim3(1024), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_expf_table(uint32_t lo, long long n, float* out, hipStream_t s) {
    const int threads = 256;
    const long long blocks = (n + threads - 1) / threads;
    hipLaunchKernelGGL(expf_table_kernel, dim3((unsigned) blocks), dim3(threads), 0, s, lo, n, out);
    return hipGetLastError();
}

}  // namespace kls

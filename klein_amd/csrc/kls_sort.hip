// Descending sort of the rows of 64-bit keys for the wide top-k path, each row on its own: a stable
// least-significant-digit radix sort, 8 bits per pass, two kernels per pass (no memset, so a pass can be captured
// in a graph). Every row is cut into tiles of 1024 * PER keys (PER = 2, 4 or 8 keys per thread, chosen per launch;
// the last tile partial); tile t of row r is workgroup r * tiles_per_row + t.
//   1. sort_hist_kernel: each tile counts its digits in LDS, written tile-major: counts[tile * 256 + digit];
//   2. sort_scatter_kernel: each tile finds where its keys of each digit start in its row (the row's keys of
//      smaller digits, then those of its digit in the row's earlier tiles: sums over the row's part of the count
//      table, read coalesced by four groups of 256 threads, and a scan over the 256 digit totals in LDS), ranks
//      its keys stably, places them in digit order in LDS and writes them from there, so that neighbouring
//      threads write neighbouring slots of each digit's run (written straight from the ranking, a wave's 64
//      keys of random low digits went to up to 64 cache lines).
// Descending order is ascending order of the inverted digit (255 - digit). Within a tile, key i of the tile is
// held by wave i / (64 PER), slot (i / 64) % PER, lane i % 64; a wave ranks its keys slot by slot: the lanes of a
// slot whose digits are equal are found with eight ballots, a key's rank is the wave's count of that digit so far
// plus the equal lanes below it, and the lowest of those lanes adds the group's size to the wave's count (the
// wave's LDS operations run in order). Then an exclusive prefix over the waves per digit gives every key its
// place: tile base of its digit + earlier waves' count + its rank in the wave.
#include "kls_internal.h"

namespace kls {
namespace {

constexpr int ST_WG = 1024, ST_NW = ST_WG / 64;
static_assert(2 * ST_WG == SORT_TILE_MIN, "the smallest tile: two keys per thread");

__device__ __forceinline__ uint32_t rdigit(uint64_t k, int shift) { return 255u - (uint32_t) ((k >> shift) & 255u); }

__device__ __forceinline__ uint64_t ballot64(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// Inclusive prefix sum across the wave, every lane active: row_shr 1, 2, 4, 8 within rows of 16 lanes, then the
// row broadcasts of lanes 15 and 31 (a source lane outside the row adds 0).
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return (uint32_t) __builtin_amdgcn_update_dpp(0, (int) x, CTRL, ROWS, 0xf, false);
}
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t x) {
    x += dpp_u32<0x111, 0xf>(x);
    x += dpp_u32<0x112, 0xf>(x);
    x += dpp_u32<0x114, 0xf>(x);
    x += dpp_u32<0x118, 0xf>(x);
    x += dpp_u32<0x142, 0xa>(x);
    x += dpp_u32<0x143, 0xc>(x);
    return x;
}

// Offset of key s of this thread in its tile (wave-major: each wave holds 64 * PER consecutive keys).
template <int PER>
__device__ __forceinline__ int tile_offset(int wave, int s, int lane) { return wave * (PER * 64) + s * 64 + lane; }

template <int PER>
__global__ __launch_bounds__(ST_WG) void sort_hist_kernel(const uint64_t* __restrict__ in, uint32_t row_len,
                                                          uint32_t tpr, int shift, uint32_t* __restrict__ counts) {
    // four sub-tables, picked by lane & 3 and padded apart, so that a wave's lanes with one digit (most keys share
    // a few digits in the sign and exponent passes) add to four addresses in four banks, not one
    constexpr int HC = 4, HP = 257;
    __shared__ uint32_t h[HC * HP];
    const int tid = (int) threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t row = blockIdx.x / tpr, t = blockIdx.x - row * tpr;
    constexpr int TILE = PER * ST_WG;
    const int lim = (int) min((uint32_t) TILE, row_len - t * TILE);  // keys in this tile
    const uint64_t* __restrict__ src = in + (size_t) row * row_len + (size_t) t * TILE;
    uint64_t k[PER];  // (loaded together, before the table is cleared)
#pragma unroll
    for (int s = 0; s < PER; ++s) {
        const int i = tile_offset<PER>(wave, s, lane);
        k[s] = i < lim ? src[i] : 0ull;
    }
    for (int i = tid; i < HC * HP; i += ST_WG) h[i] = 0u;
    __syncthreads();
    uint32_t* const hl = h + (lane & (HC - 1)) * HP;
#pragma unroll
    for (int s = 0; s < PER; ++s)
        if (tile_offset<PER>(wave, s, lane) < lim) atomicAdd(&hl[rdigit(k[s], shift)], 1u);
    __syncthreads();
    if (tid < 256) counts[(size_t) blockIdx.x * 256 + tid] = h[tid] + h[HP + tid] + h[2 * HP + tid] + h[3 * HP + tid];
}

constexpr int SC_UNROLL = 16;  // count-table rows in flight per thread

template <int PER>
__global__ __launch_bounds__(ST_WG) void sort_scatter_kernel(const uint64_t* __restrict__ in, uint64_t* __restrict__ out,
                                                             uint32_t row_len, uint32_t tpr, int shift,
                                                             const uint32_t* __restrict__ counts) {
    __shared__ uint32_t cw[ST_NW][256];  // per wave: digit counts so far, then the earlier waves' counts
    __shared__ uint32_t tb[256];         // this tile's first slot per digit
    __shared__ uint32_t part[2][4][256];  // the count sums of the four groups: earlier tiles, all tiles
    __shared__ uint32_t wsum[4], wsum2[4];
    __shared__ uint32_t ts[256];          // this tile's first slot per digit within the tile
    constexpr int TILE = PER * ST_WG;
    __shared__ uint64_t sk[TILE];         // the tile's keys in digit order
    const int tid = (int) threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t row = blockIdx.x / tpr, tile = blockIdx.x - row * tpr;  // (tile within the row)
    const int lim = (int) min((uint32_t) TILE, row_len - tile * TILE);
    const uint64_t* __restrict__ src = in + (size_t) row * row_len + (size_t) tile * TILE;
    uint64_t* __restrict__ dst = out + (size_t) row * row_len;
    const uint32_t* __restrict__ rc = counts + (size_t) row * tpr * 256;  // the row's part of the count table
    uint64_t k[PER];
#pragma unroll
    for (int s = 0; s < PER; ++s) {
        const int i = tile_offset<PER>(wave, s, lane);
        k[s] = i < lim ? src[i] : 0ull;
    }
    for (int i = tid; i < ST_NW * 256; i += ST_WG) (&cw[0][0])[i] = 0u;
    {
        // group g sums the row's tiles g, g + 4, ... of the count table for digit d
        const int g = tid >> 8, d = tid & 255;
        uint32_t before = 0u, all = 0u;
        for (uint32_t t0 = (uint32_t) g; t0 < tpr; t0 += 4 * SC_UNROLL) {
            uint32_t v[SC_UNROLL];
#pragma unroll
            for (int u = 0; u < SC_UNROLL; ++u) {
                const uint32_t t = t0 + 4u * u;
                v[u] = t < tpr ? rc[(size_t) t * 256 + d] : 0u;
            }
#pragma unroll
            for (int u = 0; u < SC_UNROLL; ++u) {
                all += v[u];
                before += t0 + 4u * u < tile ? v[u] : 0u;
            }
        }
        part[0][g][d] = before;
        part[1][g][d] = all;
    }
    __syncthreads();
    if (tid < 256) {
        // digit totals over every tile, scanned over the digits (4 waves of 64); plus the earlier tiles' counts
        const uint32_t before = part[0][0][tid] + part[0][1][tid] + part[0][2][tid] + part[0][3][tid];
        const uint32_t all = part[1][0][tid] + part[1][1][tid] + part[1][2][tid] + part[1][3][tid];
        const uint32_t x = wave_scan_u32(all);
        if (lane == 63) wsum[wave] = x;
        tb[tid] = x - all + before;  // (the earlier waves' totals are added below)
    }
    __syncthreads();
    if (tid < 256) {
        uint32_t add = 0u;
#pragma unroll
        for (int w = 0; w < 3; ++w) add += w < wave ? wsum[w] : 0u;
        tb[tid] += add;
    }
    const uint64_t below = (1ull << lane) - 1ull;
    uint32_t rk[PER];
#pragma unroll
    for (int s = 0; s < PER; ++s) {
        const bool valid = tile_offset<PER>(wave, s, lane) < lim;
        const uint32_t d = rdigit(k[s], shift);
        uint64_t same = ballot64(valid);  // (all lanes take part in every ballot)
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const bool bit = (d >> b) & 1u;
            const uint64_t m = ballot64(bit);
            same &= bit ? m : ~m;
        }
        const uint32_t before = (uint32_t) __popcll(same & below);
        const uint32_t prev = cw[wave][d];
        rk[s] = prev + before;
        if (valid && before == 0u) cw[wave][d] = prev + (uint32_t) __popcll(same);
    }
    __syncthreads();
    uint32_t tile_before = 0u;
    if (tid < 256) {
        // the earlier waves' counts per digit, and the tile's count of digit tid scanned over the digits
        uint32_t run = 0u;
#pragma unroll
        for (int w = 0; w < ST_NW; ++w) {
            const uint32_t v = cw[w][tid];
            cw[w][tid] = run;
            run += v;
        }
        const uint32_t x = wave_scan_u32(run);
        if (lane == 63) wsum2[wave] = x;
        tile_before = x - run;
    }
    __syncthreads();
    if (tid < 256) {
        uint32_t add = 0u;
#pragma unroll
        for (int w = 0; w < 3; ++w) add += w < wave ? wsum2[w] : 0u;
        ts[tid] = tile_before + add;
    }
    __syncthreads();
    // the tile's keys in digit order (stable: wave, then slot, then lane order within a digit)
#pragma unroll
    for (int s = 0; s < PER; ++s) {
        if (tile_offset<PER>(wave, s, lane) < lim) {
            const uint32_t d = rdigit(k[s], shift);
            sk[ts[d] + cw[wave][d] + rk[s]] = k[s];
        }
    }
    __syncthreads();
    // slot i of the tile goes to the row's slot of its digit: the digit's first row slot for this tile plus its
    // place in the digit's run
#pragma unroll
    for (int s = 0; s < PER; ++s) {
        const int i = s * ST_WG + tid;
        if (i < lim) {
            const uint64_t key = sk[i];
            const uint32_t d = rdigit(key, shift);
            const uint32_t pos = tb[d] + (uint32_t) i - ts[d];
            if (pos < row_len) dst[pos] = key;  // (always: the counts are the row's own)
        }
    }
}

template <int PER>
hipError_t sort_passes(uint64_t* a, uint64_t* b, int rows, size_t row_len, int begin_bit, int end_bit,
                       uint32_t* counts, bool first_counted, uint64_t** result, hipStream_t s) {
    const uint32_t tpr = (uint32_t) ((row_len + PER * ST_WG - 1) / (PER * ST_WG));
    const dim3 grid((unsigned) rows * tpr);
    uint64_t* src = a;
    uint64_t* dst = b;
    for (int shift = begin_bit; shift < end_bit; shift += 8) {
        if (!(first_counted && shift == begin_bit))
            hipLaunchKernelGGL(sort_hist_kernel<PER>, grid, dim3(ST_WG), 0, s, src, (uint32_t) row_len, tpr, shift,
                               counts);
        hipLaunchKernelGGL(sort_scatter_kernel<PER>, grid, dim3(ST_WG), 0, s, src, dst, (uint32_t) row_len, tpr,
                           shift, counts);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        uint64_t* t = src;
        src = dst;
        dst = t;
    }
    *result = src;
    return hipSuccess;
}

}  // namespace

// Keys per tile: the largest of 8,192 / 4,096 whose grid (rows x tiles) still covers the CUs (240 workgroups
// or more), else 2,048. Smaller tiles spread a pass over more CUs, larger ones sum fewer count-table rows per
// tile (248,320 keys, no top-k limit, device time per step: 4 rows 146.1 / 128.5 / 131.4 us and 1 row 116.7 /
// 98.8 / 93.9 us with 8,192 / 4,096 / 2,048 keys per tile).
int sort_tile_keys(int rows, size_t row_len) {
    for (int t = 8192; t > SORT_TILE_MIN; t >>= 1)
        if ((size_t) rows * ((row_len + t - 1) / t) >= 240) return t;
    return SORT_TILE_MIN;
}

hipError_t sort_keys_desc(uint64_t* a, uint64_t* b, int rows, size_t row_len, int begin_bit, int end_bit,
                          uint32_t* counts, bool first_counted, uint64_t** result, hipStream_t s) {
    if (rows < 1 || row_len == 0 || (size_t) rows * row_len >= (1ull << 32) || begin_bit < 0 ||
        end_bit <= begin_bit || end_bit > 64)
        return hipErrorInvalidValue;
    switch (sort_tile_keys(rows, row_len)) {
        case 8192: return sort_passes<8>(a, b, rows, row_len, begin_bit, end_bit, counts, first_counted, result, s);
        case 4096: return sort_passes<4>(a, b, rows, row_len, begin_bit, end_bit, counts, first_counted, result, s);
        default: return sort_passes<2>(a, b, rows, row_len, begin_bit, end_bit, counts, first_counted, result, s);
    }
}

}  // namespace kls

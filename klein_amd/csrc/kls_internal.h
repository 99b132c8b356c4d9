// Internal interface between the C-ABI layer (kls_api.cpp) and the HIP kernels (kls_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "klein_sampler.h"

namespace kls {

// Candidates kept per segment and per row on the fast path (one per lane of a wave64).
constexpr int KCAP = 64;
// Rows a verify step may carry (1 main + up to 15 drafts).
constexpr int VERIFY_MAX_ROWS = 16;
// History ids accepted since the last device upload that ride along with a call.
constexpr int PENDING_CAP = 256;
// Segments (vocabulary ids per workgroup): 256 threads x EPT elements, EPT in {4, 8, 16, 32} (1024..8192 ids,
// history counts in LDS at 4 B per id), or 1024 threads x {16, 32, 64} (16384..65536 ids, 2 B per id).
constexpr int SEG_MIN = 1024;
constexpr int SEG_WIDE = 16384;  // first length served by 1024-thread workgroups
constexpr int SEG_MAX = 65536;
// History bucket width: history lists are partitioned into buckets of (1 << bucket_shift) ids, and segments
// start on bucket boundaries so a workgroup finds its history slice with two loads.
constexpr int MIN_BUCKET_SHIFT = 10;
constexpr int MAX_BUCKETS = 1024;

// Per-call inputs a graph-captured step reads from pinned host memory (written by the host before launch).
struct CallBlock {
    double u[VERIFY_MAX_ROWS];
    int32_t drafts[VERIFY_MAX_ROWS];
    int32_t n_pending;
    uint32_t seq;
    int32_t pending[PENDING_CAP];
};

// Results a step writes back to pinned host memory: per row one 64-bit word, (sequence number << 32) | token,
// stored at once so the host sees either the old word or the new one; for a verify step one more word,
// (sequence number << 32) | accepted, written by the workgroup that completes the step's last row.
struct ResultBlock {
    uint64_t row_word[VERIFY_MAX_ROWS];
    uint64_t step_word;
    // nonzero: a kernel launched for this handle found an internal wait that did not end (the code names it);
    // set by the device, read and cleared by the host
    uint32_t fault;
};

// Fault codes (ResultBlock::fault).
constexpr uint32_t FAULT_COUNT_WAIT = 1;   // the history count table was not announced complete in time
constexpr uint32_t FAULT_BOUND_WAIT = 2;   // the early bound of a 16-wave segment was not published in time
constexpr uint32_t FAULT_NARROW = 3;       // a mid top-k threshold bisection did not end (not reachable)
constexpr uint32_t FAULT_WIDE_MAP = 4;     // a segment map of the wide tail left its binade (not reachable)

struct SamplingParams {
    float temperature;
    float top_p;
    float min_p;
    float presence;
    float frequency;
    float repetition;
    int32_t k;  // effective top-k (1..KCAP on the fast path)
    // 1 / repetition in double: RN_f32(l * inv_repetition) is RN_f32(l / repetition) for every float l (the
    // product's relative error, below 2^-51.9, is smaller than any quotient's distance to a rounding midpoint)
    double inv_repetition;
    int32_t lazy;  // penalties never raise a logit (repetition >= 1, presence >= 0, frequency >= 0)
};

struct RowsArgs {
    const float* logits;
    int64_t row_stride;  // floats between rows
    int32_t V;
    int32_t n_rows;
    int32_t segs;
    int32_t seg_len;  // ids per segment: workgroup threads x EPT
    int32_t xcd_map;  // 1: deal (row, segment) work so that a row's segments run on one XCD (see the kernel)
    SamplingParams p;

    // history, one of two forms (neither: no history):
    //  * bucketed (the handle's own history, shared by all rows): unique ids sorted into buckets of
    //    (1 << bucket_shift) ids with counts hist_w; hist_boff[b] = first entry of bucket b;
    //  * raw (the batch entry point): row r's ids are hist_ids[hist_off[r] .. hist_off[r+1]), repeats counted.
    const int32_t* hist_ids;
    const int32_t* hist_w;     // bucketed form: counts
    const int32_t* hist_boff;  // bucketed form: [n_buckets + 1]
    const int32_t* hist_off;   // raw form: [n_rows + 1]
    int32_t bucket_shift;
    int32_t n_buckets;
    int32_t count_wide;  // a history count may reach 65536 (16-bit count tables are then not used)
    // extra history ids counted on top: list A (count read from memory) for every row, list B's first
    // row*extra_b_step entries for row `row` (the verify step's drafts on the accepted path)
    const int32_t* extra_a;
    const int32_t* extra_a_n;
    const int32_t* extra_b;
    int32_t extra_b_step;

    const double* u;  // [n_rows]

    // scratch (self-resetting between launches)
    uint64_t* seg_cand;     // [n_rows][segs][KCAP]
    uint32_t* row_ticket;   // [n_rows]
    uint64_t* row_thr;      // [n_rows]
    int32_t share_bounds;   // publish / read per-row lower bounds across workgroups (large grids)
    int32_t first_nan;      // greedy rows as std::max_element: a NaN first logit is the result

    // outputs
    int32_t* out_tokens;    // [n_rows] device
    uint64_t* dbg_keys;     // [n_rows][KCAP] final sorted candidate keys
    float* dbg_probs;       // [n_rows][KCAP]
    int32_t* dbg_meta;      // [n_rows][2]: k, kept
    ResultBlock* host_res;  // pinned, may be NULL: tokens and per-row sequence numbers for the host
    const CallBlock* call;  // the sequence number to publish (with host_res), the drafts of a verify step
    // verify steps (src/engine.cpp:563-575): the accept prefix on the device. Each row's last workgroup adds
    // (1 << 32) | (mismatch of row r: 1 << r) to *step_word; the one that completes the count forms
    // accepted = the first row whose token differs from its draft (the last row if none), writes it to
    // *out_accepted and to host_res->step_word, and clears *step_word for the next launch. NULL: no accept.
    uint64_t* step_word;
    int32_t* out_accepted;
    uint32_t* fault;        // mapped pinned word, may be NULL: set when an internal wait gives up
    int32_t spin_limit;     // polls of an internal wait before it gives up (a guard: the waits always end)
};

constexpr int32_t DEFAULT_SPIN_LIMIT = 1 << 20;


// Wide top-k (k above KCAP, up to no limit; src/sampler.cpp:42-51): every logit of a row becomes one 64-bit key
//   (order-preserving image of the (penalized) value << id_bits) | (~id & id mask)
// in id order, and a stable descending sort of each row on the value field leaves the row's keys
// value-descending and, on equal values, id-ascending (the fast path's order). NaN maps to the value image 0,
// after every number. The sorted keys then go through the O(k) tail in reference order.
// The wide path's tail cuts each of its double chains into chunks of WT_CHUNK terms (kls_kernels.hip), and each
// chunk into at most WT_SEGS segments, recorded in order:
constexpr int WT_CHUNK = 1024, WT_SEGS = 64;
enum : int32_t {
    WS_MAP = 1,     // terms [start, end) composed to one parity map in the binade 2^E
    WS_TERM = 2,    // one term (d0, signed as the chain adds it) added on its own
    WS_REPLAY = 3,  // terms [start, end) replayed one by one (a chunk of more than WT_SEGS segments)
};
struct WideSeg {
    double d0, d1;  // WS_MAP: increments in units of 2^(E-52) from an incoming even / odd partial result
    uint32_t p;     // WS_MAP: parity after, bit 0 from even, bit 1 from odd
    int32_t E;
    int32_t kind;
    int32_t start, end;
    int32_t pad;
};
// a row's state between the tail's kernels
struct WideRow {
    int32_t kk;     // candidates: keys before the first NaN key
    int32_t n_mp;   // kept by min-p
    int32_t n_top;  // kept by top-p
    int32_t pad;
    double sum;     // softmax total
    double total;   // the draw's total
    double r0;      // the draw's start, u * total
};

struct WideArgs {
    uint64_t* keys;       // [n_rows * V]
    uint64_t* sorted;     // [n_rows * V] (the sort alternates between the two buffers)
    uint32_t* counts;     // the sort's digit counts: 256 * sort_tiles(max_rows * V)
    int32_t k;            // MID_KMAX < k <= V (or a k the mid path cannot hold)
    int32_t id_bits;      // ids are below 1 << id_bits
    int32_t chunks;       // chunks per row: ceil(k / WT_CHUNK)
    int32_t seg_cap;      // segments a chunk may leave (WT_SEGS; fewer only under a test layout)
    double* part;         // [max_rows * chunks] term sums of the chunks
    WideSeg* seg;         // [max_rows * chunks * WT_SEGS] the chunks' segments of the chain being resolved
    int32_t* nseg;        // [max_rows * chunks] segments per chunk
    WideRow* rowst;       // [max_rows]
};

// Mid top-k (KCAP < k <= MID_KMAX; src/sampler.cpp:42-51), one kernel: 1024-thread workgroups over segments of
// MID_SEG ids append the logits at or above a per-segment bound (every one of the segment's top-k among them) to
// the row's buffer of MID_ROWCAP keys (fast-path keys: value image << 32 | ~id); the row's last workgroup selects
// and sorts the row's top-k from it in LDS and runs the wide path's exact tail.
constexpr int MID_KMAX = 1024;
constexpr int MID_SEG = 32768;
constexpr int MID_ROWCAP = 16384;
struct MidArgs {
    uint64_t* buf;    // [n_rows][MID_ROWCAP]
    uint32_t* fill;   // [n_rows] keys appended so far (left zero)
    int32_t k;        // KCAP < k <= MID_KMAX
    int32_t cap;      // keys a segment may append: MID_ROWCAP / segments, at least k
};
// Segments of the mid path for V ids, and whether top-k k fits it.
inline int mid_segments(int V) { return (V + MID_SEG - 1) / MID_SEG; }
inline bool mid_fits(int V, int k) { return k > KCAP && k <= MID_KMAX && k <= MID_ROWCAP / mid_segments(V); }

// Per-token perplexity / KL-divergence scores (src/main.cpp:308-327; kls_ppl.hip). Row r of logits at
// logits + r*row_stride, of base log-probabilities (optional) at base + r*base_stride; outputs per row, each
// optional. Scratch: per (row, segment) a KCAP-word record; per row a ticket counter (left zero).
struct PplArgs {
    const float* logits;
    int64_t row_stride;
    const float* base;
    int64_t base_stride;
    const int32_t* targets;
    int32_t V;
    int32_t n_rows;
    int32_t segs;
    int32_t seg_len;
    uint64_t* scratch;
    uint32_t* ticket;
    double* out_lse;
    double* out_nll;
    int32_t* out_top;
    double* out_kl;
    double* out_nll_base;
    int32_t* out_base_top;
};
// The launch layout of rows_kernel for `rows` rows of V ids (kls_api.cpp): ids per segment and segments per row.
// seg_override (a power of two in [SEG_MIN, SEG_MAX], else 0) forces the length; target_wg and wide_target_wg
// are the grid sizes the choice aims at (defaults 128 and 320).
void choose_segments(int V, int rows, bool greedy, int seg_override, int target_wg, int wide_target_wg, int* seg_len,
                     int* segs);
// The kernels' whole-float4 form: every row starts on a 16-byte boundary, the stride and V are multiples of 4 and no
// segment is partial (V >= seg_len). Otherwise every float4 is checked against the segment's end.
inline bool rows_full(const float* logits, int64_t stride, int V, int seg_len) {
    return (stride & 3) == 0 && (reinterpret_cast<uintptr_t>(logits) & 15u) == 0 && (V & 3) == 0 && V >= seg_len;
}
// Greedy rows in the checked form (not rows_full) take at most 32,768-id segments: with 65,536 ids that kernel
// runs out of registers and spills (kls_api.cpp).
void fit_segments(bool greedy, const float* logits, int64_t stride, int V, int* seg_len, int* segs);
constexpr int DEFAULT_TARGET_WG = 128, DEFAULT_WIDE_TARGET_WG = 320;
// Grids of more (row, segment) workgroups than this share per-row running bounds through device memory.
constexpr int DEFAULT_SHARE_MIN_WG = 1024;
// Records the failure for kls_last_error (kls_api.cpp) and returns `status`.
int set_error(int status, const char* what, hipError_t e = hipSuccess);
// The kernel's parameter block for klein::SamplerParams p with effective top-k k (src/sampler.cpp:42).
SamplingParams sampling_params(const kls_params& p, int k);
int ppl_segments(int V, int rows, int* seg_len);  // segments per row (and their length) of a launch
hipError_t launch_ppl(const PplArgs& a, hipStream_t s);

// Launchers (kls_kernels.hip). Return hipSuccess or the launch error.
hipError_t launch_rows(const RowsArgs& a, bool greedy, bool penalize, hipStream_t s);
int rows_grid(const RowsArgs& a);  // workgroups launch_rows starts
hipError_t prepare_rows_kernels();  // once per device: LDS limits of the kernels with large count tables
hipError_t launch_expf_table(uint32_t lo, long long n, float* out, hipStream_t s);
// A kernel that does nothing (one wave): the body of the graph that prepares a stream for graph launches.
const void* noop_kernel();
// Test hook of the wide tail's exact sum replay (see kls_debug_sum_replay).
hipError_t launch_sum_replay(const double* t, int n, double acc0, int mode, double thr, double* out, hipStream_t s);
// Wide top-k: keys (with penalties from the history in `a`), the sort, the tail (tokens published as
// launch_rows does).
hipError_t launch_wide(const RowsArgs& a, const WideArgs& w, bool penalize, hipStream_t s);
int wide_id_bits(int V);  // key bits the ids of a V-entry vocabulary take
// Mid top-k: one kernel over a.n_rows rows of a.segs = mid_segments(V) segments (tokens published as launch_rows
// does).
hipError_t launch_mid(const RowsArgs& a, const MidArgs& m, bool penalize, hipStream_t s);
hipError_t prepare_mid_kernels();  // once per device: LDS limit of the kernel with a count table

// Descending sort of each of `rows` rows of row_len 64-bit keys (rows * row_len < 2^32; row r at r * row_len) on
// bits [begin_bit, end_bit) (kls_sort.hip): a stable radix sort, 8 bits per pass, alternating between the buffers
// a (the input) and b; *result is the one that holds the sorted keys. Keys equal on those bits keep their input
// order. counts: 256 * rows * sort_tiles(row_len) words of scratch (enough for every tile size the sort picks).
// Each row is cut into tiles of sort_tile_keys(rows, row_len) keys (2,048, 4,096 or 8,192), and a pass's counts
// are tile-major: counts[(r * tiles_per_row + t) * 256 + 255 - digit] for tile t of row r. first_counted: the
// caller has written the first pass's counts (bits [begin_bit, begin_bit + 8) of the keys in a) in that layout,
// and the first pass's histogram kernel is not launched.
constexpr int SORT_TILE_MIN = 2048;
inline size_t sort_tiles(size_t n) { return (n + SORT_TILE_MIN - 1) / SORT_TILE_MIN; }
int sort_tile_keys(int rows, size_t row_len);
hipError_t sort_keys_desc(uint64_t* a, uint64_t* b, int rows, size_t row_len, int begin_bit, int end_bit,
                          uint32_t* counts, bool first_counted, uint64_t** result, hipStream_t s);

}  // namespace kls

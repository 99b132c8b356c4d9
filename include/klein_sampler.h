/* klein_sampler.h — C ABI of the MI355X (gfx950) token sampler.
 *
 * Drop-in for klein's sampling path: klein::Sampler (src/sampler.h:25-38, src/sampler.cpp:11-89) and the MTP
 * verify accept loop of Engine::generate (src/engine.cpp:563-575). Plain C types and pointers only; every entry
 * point returns a status (KLS_OK = 0) and never throws. The C++ class klein::Sampler in klein_amd/csrc/sampler.h
 * keeps the reference's interface on top of these functions.
 *
 * Results equal the reference sampler's on the same logits and the same uniform draws: token ids, top-k id sets
 * and accepted-draft counts bit for bit (on equal values the lower id wins), probabilities to the bit as well.
 * The uniform `u` of a draw is the value std::uniform_real_distribution<double> would derive from the sampler's
 * mt19937_64 (libstdc++ generate_canonical: double(x) / 2^64, clamped below 1); the caller supplies it.
 */
#ifndef KLEIN_SAMPLER_H_
#define KLEIN_SAMPLER_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum kls_status {
    KLS_OK = 0,
    KLS_ERR_INVALID_ARG = 1, /* null pointer, n_vocab <= 0, n_vocab differing from the handle's, nb < 1 */
    KLS_ERR_RANGE = 2,       /* rows above the handle's capacity, a token id outside [0, n_vocab) */
    KLS_ERR_UNSUPPORTED = 3, /* a parameter combination this build does not implement */
    KLS_ERR_HIP = 4,         /* a HIP runtime call failed (the message names it: kls_last_error) */
    KLS_ERR_NO_DEVICE = 5,   /* no GPU visible */
    KLS_ERR_OOM = 6          /* device or pinned allocation failed */
};

/* klein::SamplerParams (src/sampler.h:13-22): same fields, order and defaults (temperature 1, top_k 20,
 * top_p 0.95, min_p 0, presence 0, frequency 0, repetition 1, seed 0). temperature <= 0 selects greedy;
 * top_k <= 0 or >= n_vocab means no limit. The seed is used by the C++ wrapper's mt19937_64 only. */
typedef struct kls_params {
    float temperature;
    int32_t top_k;
    float top_p;
    float min_p;
    float presence_penalty;
    float frequency_penalty;
    float repetition_penalty;
    uint64_t seed;
} kls_params;

typedef struct kls_sampler* kls_handle;

/* hipStream_t, passed as a plain pointer; NULL selects the library's own stream of the handle's device (one per
 * device, shared by every handle created on it; a blocking stream, so such calls are ordered with work on the
 * legacy default stream). */
typedef void* kls_stream;

/* Replaces Sampler::Sampler (src/sampler.cpp:11). Binds the current HIP device, allocates every buffer the
 * handle will use (no allocation happens in the calls below), and starts with an empty token history.
 * max_rows bounds the rows of kls_verify and kls_sample_batch. A top-k of 65 to 1024 takes the mid path: one
 * kernel, like top-k <= 64, with a 128 KB candidate buffer per row (vocabularies of up to 16384 / top_k segments
 * of 32768 ids: n_vocab <= 524,288 for every such top-k). A larger top-k (or no limit) takes a slower path
 * that keys and sorts every logit of a row (2 x 8 bytes per logit per row of device memory, plus ~6.2 KB per
 * 2,048 ids per row for the sort's digit counts and the tail's chunk records; a key kernel, a radix sort's passes and the tail's kernels,
 * captured together in a verify step's graph); it needs n_vocab * max_rows below 2^32 (KLS_ERR_UNSUPPORTED
 * otherwise). */
int kls_create(const kls_params* params, int n_vocab, int max_rows, kls_handle* out);

int kls_destroy(kls_handle h);

/* Replaces Sampler::reset (src/sampler.cpp:13): clears the token history. */
int kls_reset(kls_handle h);

/* Replaces Sampler::accept (src/sampler.cpp:15): counts one more occurrence of `token` for the penalties.
 * Calls that use the handle (this one included) are refused with KLS_ERR_INVALID_ARG while a verify step is in
 * flight (between kls_verify_enqueue and kls_verify_wait). The asynchronous calls that lend the handle's scratch
 * (kls_sample_batch, kls_argmax, kls_ppl_scores) are ordered after the handle's earlier launches when they come
 * on another stream. */
int kls_accept(kls_handle h, int32_t token);

/* Replaces Sampler::sample (src/sampler.cpp:17-89) for one row of n_vocab f32 logits. `logits` may be a device
 * pointer (read in place) or a host pointer (copied to the device first). `u` is the draw's uniform (ignored
 * when temperature <= 0). Penalties use the history given through kls_accept. Synchronous. */
int kls_sample(kls_handle h, const float* logits, int n_vocab, double u, int32_t* out_token);

/* Replaces the verify/accept loop of Engine::generate (src/engine.cpp:563-575). `logits` holds nb rows of
 * n_vocab f32 (row i at logits + i*n_vocab; device or host pointer); row 0 is the main position and rows
 * 1..nb-1 the draft positions. drafts[i] (i < nb-1) is the draft token batch[i+1]; u[i] the uniform of row i.
 * Row i is sampled with the history after accepting t_0..t_{i-1}; drafts are accepted while drafts[i] == t_i.
 * On return out_tokens[0..*out_accepted] are the emitted tokens (later entries are unspecified) and the
 * emitted tokens have been added to the history, as the engine's accept(t) calls do (engine.cpp:567).
 * The caller-side stops of the engine (end-of-generation token, n_predict, callback) stay with the caller.
 * The step runs as one hipGraph launch on `stream`; host-side inputs and outputs go through pinned memory. The
 * accepted count is formed on the device, by the workgroup that completes the last row, and also stays in
 * device memory with the tokens (kls_device_results) for work that follows on the stream. The first verify
 * step on a stream first runs a short series of empty graph launches through it (once per stream and process:
 * this ROCm's first graph launches on a stream cost several times the later ones). */
int kls_verify(kls_handle h, const float* logits, int nb, const int32_t* drafts, const double* u,
               int32_t* out_tokens, int32_t* out_accepted, kls_stream stream);

/* The two halves of kls_verify, for callers that overlap other host work with the step or bracket it with
 * stream events: kls_verify_enqueue launches the step on `stream` and returns; kls_verify_wait waits for its
 * results (spinning on the pinned result block) and then behaves as the end of kls_verify. One step may be in
 * flight per handle. No counterpart in the reference, whose loop is synchronous. */
int kls_verify_enqueue(kls_handle h, const float* logits, int nb, const int32_t* drafts, const double* u,
                       kls_stream stream);
int kls_verify_wait(kls_handle h, int32_t* out_tokens, int32_t* out_accepted);

/* No counterpart in the reference (whose results live on the host): the device buffers that hold the last
 * verify step's results, for consumers enqueued after it on the same stream: d_tokens[i] is row i's token
 * (i < nb), *d_accepted the accepted count. Valid for the handle's lifetime; overwritten by the next step
 * (kls_sample and kls_sample_batch without an output of their own write d_tokens too). Either pointer may be
 * NULL. */
int kls_device_results(kls_handle h, const int32_t** d_tokens, const int32_t** d_accepted);

/* No counterpart in the reference: reports (once) KLS_ERR_HIP if a kernel launched for this handle gave up an
 * internal wait since the last check, in which case that call's results are not valid. The synchronous calls
 * (kls_sample, kls_verify, kls_verify_wait) check by themselves after their step; callers of the asynchronous
 * ones check after synchronizing the stream (every call also checks on entry). */
int kls_check(kls_handle h);

/* Batched sampling of n_rows independent rows, all on the device, asynchronous on `stream` (no host sync).
 * Row r is at d_logits + r*row_stride floats; its token history is d_hist_ids[d_hist_off[r] .. d_hist_off[r+1])
 * (raw ids, repeats counted, ids outside [0, n_vocab) ignored; d_hist_off has n_rows+1 non-decreasing entries
 * that index d_hist_ids; NULL offsets = no history). d_u[r] is row r's uniform. Tokens are written to
 * d_out_tokens[r]. The handle's own history is not used or changed. Each row equals one Sampler::sample call on
 * that row after accept() of its history ids. */
int kls_sample_batch(kls_handle h, const float* d_logits, int n_rows, int64_t row_stride, const int32_t* d_hist_off,
                     const int32_t* d_hist_ids, const double* d_u, int32_t* d_out_tokens, kls_stream stream);

/* No counterpart in the reference: kls_sample_batch for callers that cannot allocate (code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc). It takes the parameters instead of a handle and
 * allocates nothing: the sampling kernel's scratch (per (row, segment) candidate lists, per-row tickets and
 * bounds, 515 KiB) is a static device array that each GPU holds for the life of the process, resolved with
 * hipGetSymbolAddress on the first call with that device current. Same inputs, outputs and results as
 * kls_sample_batch (stream NULL = the null stream). Limits: top-k at most 64 unless greedy (KLS_ERR_UNSUPPORTED
 * otherwise), n_rows <= KLS_NOALLOC_MAX_ROWS and n_rows x segments <= KLS_NOALLOC_MAX_WORKGROUPS (segments of
 * up to 65,536 ids: 4 per row at n_vocab = 248,320), else KLS_ERR_RANGE. Every call on one GPU shares the
 * array: calls that overlap on one GPU (other streams, other threads) race and must be serialized by the
 * caller; each call clears the rows' tickets and bounds with a small kernel before sampling. */
#define KLS_NOALLOC_MAX_ROWS 256
#define KLS_NOALLOC_MAX_WORKGROUPS 1024
int kls_sample_batch_noalloc(const kls_params* params, int n_vocab, const float* d_logits, int n_rows,
                             int64_t row_stride, const int32_t* d_hist_off, const int32_t* d_hist_ids,
                             const double* d_u, int32_t* d_out_tokens, kls_stream stream);

/* Replaces Engine::mtp_draft_token (src/engine.cpp:413-415): for each of n_rows rows of n_vocab f32 logits on
 * the device (row r at d_logits + r*row_stride), the index std::max_element returns: the first largest element
 * under '<', so a NaN never replaces the running maximum and a NaN first element is the result. Indices are
 * written to d_out[r]. Asynchronous on `stream`; the handle lends its scratch (n_rows <= max_rows, n_vocab equal
 * to the handle's) and its own history and parameters are not used. */
int kls_argmax(kls_handle h, const float* d_logits, int n_rows, int64_t row_stride, int32_t* d_out,
               kls_stream stream);

/* Replaces the per-token scoring of klein's perplexity / KL-divergence loop (src/main.cpp:308-327) for n_rows
 * rows of n_vocab f32 logits on the device (row r at d_logits + r*row_stride, target token d_targets[r]):
 *   d_lse[r] = mx + log(sum_v exp(l[v] - mx)), mx the first largest logit;  d_nll[r] = d_lse[r] - l[target];
 *   d_top[r] = the index of the first largest logit (std::max_element's rule, as the loop's own scan);
 * and, with a row of f32 base log-probabilities (d_base, row r at d_base + r*base_stride; NULL for none):
 *   d_kl[r] = sum over b[v] > -16 of exp(b[v]) * (b[v] - (l[v] - lse));  d_nll_base[r] = -b[target];
 *   d_base_top[r] = the index of the first largest b.
 * Every output pointer may be NULL (not written). Sums are in double but in another order than the reference's
 * sequential loop: values agree to rounding (~1e-15 relative for lse), indices exactly. A NaN logit or an
 * infinite maximum gives a NaN lse, as in the reference; a target outside [0, n_vocab) gives a NaN nll.
 * Asynchronous on `stream`; the handle lends its scratch (n_rows <= max_rows, n_vocab equal to the handle's). */
int kls_ppl_scores(kls_handle h, const float* d_logits, int n_rows, int64_t row_stride, const int32_t* d_targets,
                   const float* d_base, int64_t base_stride, double* d_lse, double* d_nll, int32_t* d_top,
                   double* d_kl, double* d_nll_base, int32_t* d_base_top, kls_stream stream);

/* ---- The verify step's consumer: the recurrent-state rollback (src/engine.cpp:578-583, src/state.cpp:162-184).
 *
 * Storage type of the rollback snapshots (StateConfig::snap_type, src/state.h:20). */
enum kls_snap_type { KLS_SNAP_F32 = 0, KLS_SNAP_F16 = 1, KLS_SNAP_BF16 = 2 };

/* The Gated DeltaNet recurrent state of one sequence as klein's State lays it out (src/state.h:45-46,
 * src/state.cpp:68-76), for each of n_layers recurrent layers l:
 *   conv[l]      n_snapshots slots of conv_row f32, slot i at byte offset i * conv_stride: slot 0 the current
 *                state, slot s the state s tokens back;
 *   ssm[l]       ssm_row f32: the current state;
 *   ssm_snap[l]  n_snapshots - 1 rows of ssm_row elements of snap_type, row i at byte offset i * snap_stride:
 *                row s - 1 the state s tokens back (unused when n_snapshots is 1).
 * The three arrays are host arrays of n_layers device pointers; the strides are ggml's nb[1]. */
typedef struct kls_recurrent_desc {
    int32_t n_layers;
    int32_t n_snapshots;
    int64_t conv_row;
    int64_t ssm_row;
    int64_t conv_stride;
    int64_t snap_stride;
    int32_t snap_type;
    float* const* conv;
    float* const* ssm;
    const void* const* ssm_snap;
} kls_recurrent_desc;

typedef struct kls_recurrent* kls_recurrent_handle;

/* No counterpart in the reference (its State owns the tensors): copies the layer pointer table to device
 * memory (the only allocation) for kls_rollback_recurrent. The state buffers stay the caller's. */
int kls_recurrent_create(const kls_recurrent_desc* desc, kls_recurrent_handle* out);
int kls_recurrent_destroy(kls_recurrent_handle r);

/* Replaces `rejected = (nb - 1) - accepted; if (rejected > 0) state->rollback_recurrent(gpu, rejected)` of
 * Engine::generate (src/engine.cpp:578-582) with State::rollback_recurrent (src/state.cpp:162-184): for every
 * layer, conv slot s is copied over slot 0 and snapshot row s - 1 is converted to f32 into ssm, s = rejected.
 * `accepted` is read from device memory (d_accepted: kls_device_results's, or any device int32) by the kernel,
 * so the call can be enqueued right after kls_verify_enqueue on the same stream, before the host knows the
 * result. One kernel launch over all layers, asynchronous on `stream` (NULL: the null stream). nb must not
 * exceed n_snapshots (KLS_ERR_RANGE; the reference asserts s < n_snapshots); an accepted value outside
 * [0, nb - 1] rolls nothing back. */
int kls_rollback_recurrent(kls_recurrent_handle r, const int32_t* d_accepted, int nb, kls_stream stream);

/* The sorted top-k candidates of `row` from the last completed call (kls_sample: row 0): ids, softmax
 * probabilities before min-p/top-p truncation (up to `cap`), k, and how many survived min-p/top-p.
 * Synchronizes the handle's stream. For tests and tooling; not needed on the sampling path. */
int kls_get_candidates(kls_handle h, int row, int32_t* ids, float* probs, int cap, int32_t* n_k, int32_t* n_kept);

/* Test hook, no counterpart in the reference: writes the sampler's expf of the n consecutive float bit
 * patterns lo, lo+1, ... to device memory `d_out`, asynchronously on `stream`, so tests can compare the device
 * exponential with the host libm's std::exp(float) (src/sampler.cpp:57) over whole ranges of inputs. */
int kls_debug_expf(uint32_t lo, long long n, float* d_out, kls_stream stream);

/* Test hook, no counterpart in the reference: overrides the launch layout the handle chooses (a field of 0 keeps
 * the default; xcd_map -1 keeps it): seg_len = vocabulary ids per workgroup (a power of two in [1024, 65536]),
 * target_wg / wide_target_wg = the grid sizes the segment choice aims at, share_min_wg = the grid size above
 * which workgroups of a row share a running bound through device memory, xcd_map = 1 to deal a row's segments
 * to one XCD, 0 for plain order. Results do not depend on the layout; tests use it to reach every code path.
 * wait_limit bounds the polls of the kernels' internal waits (0: the default, 2^20; negative: none, so such a
 * wait gives up at once and the call reports KLS_ERR_HIP): tests force the failure path with it. wide_segs caps
 * the segments a chunk of the wide top-k tail may leave (0: the default, 64; else 1..64): a chunk of more is
 * replayed term by term, which tests reach with it. */
typedef struct kls_debug_layout {
    int32_t seg_len;
    int32_t target_wg;
    int32_t wide_target_wg;
    int32_t share_min_wg;
    int32_t xcd_map;
    int32_t wait_limit;
    int32_t wide_segs;
} kls_debug_layout;
int kls_debug_set_layout(kls_handle h, const kls_debug_layout* layout);

/* Measurement hook, no counterpart in the reference: device time of the verify kernel as the last verify step's
 * graph runs it (same arguments: uniforms and drafts from the pinned call block, results published to pinned
 * memory), measured with HIP events on `stream` around `reps` launches of a graph of n back-to-back copies;
 * *out_us = microseconds per kernel. Needs a completed verify step on the handle (KLS_ERR_INVALID_ARG otherwise);
 * the handle's results are those of that step again afterwards. */
int kls_debug_time_verify(kls_handle h, int n, int reps, kls_stream stream, double* out_us);

/* Measurement hook, no counterpart in the reference: n_steps verify steps (kls_verify) back to back from C, as a
 * C++ engine's generation loop calls them (src/engine.cpp:563-575 runs once per step): step i samples the nb
 * rows at `logits` with drafts[i*(nb-1) ...] and u[i*nb ...] and writes out_tokens[i*nb ...] and
 * out_accepted[i]; out_step_ns[i] (may be NULL) receives the step's host wall time in nanoseconds (enqueue to
 * tokens on the host). Stops at the first step that fails and returns its status. */
int kls_debug_run_verify_steps(kls_handle h, const float* logits, int nb, int n_steps, const int32_t* drafts,
                               const double* u, int32_t* out_tokens, int32_t* out_accepted, int64_t* out_step_ns,
                               kls_stream stream);

/* Test hook, no counterpart in the reference: *out_path = the kernel path the handle's sampling calls take
 * (greedy and top-k <= 64: FAST; top-k 65..1024: MID; larger or no limit: WIDE). */
enum kls_path { KLS_PATH_FAST = 0, KLS_PATH_MID = 1, KLS_PATH_WIDE = 2 };
int kls_debug_path(kls_handle h, int32_t* out_path);

/* Test hook, no counterpart in the reference: the wide top-k tail's parallel replay of a sequential double sum
 * (src/sampler.cpp:58,70-77,84-87 accumulate this way; the block form that replays the wide tail's segments and
 * the mid path's tail) over the n device doubles d_terms from acc0:
 * acc = acc + d_terms[i] in order, stopping after the first i where (mode 1) acc >= thr or (mode 2) acc <= 0
 * (mode 0: never). d_out[0] receives the result, d_out[1] the stop index (-1: none). Asynchronous on `stream`. */
int kls_debug_sum_replay(const double* d_terms, int n, double acc0, int mode, double thr, double* d_out,
                         kls_stream stream);

/* Human-readable name of a status code. */
const char* kls_status_string(int status);

/* Thread-local text of the last failure on this thread (empty when none). */
const char* kls_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* KLEIN_SAMPLER_H_ */

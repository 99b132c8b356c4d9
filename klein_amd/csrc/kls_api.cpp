// C-ABI layer of the gfx950 token sampler (include/klein_sampler.h).
//
// A handle replaces one klein::Sampler (src/sampler.h:25-38): it holds the parameters, the token history
// (src/sampler.h:36, counts_), and every device / pinned buffer its calls use, all allocated in kls_create.
// The history lives on the host as the reference keeps it (id -> count) and on the device as a list of
// unique ids with counts, bucketed by id range; ids accepted since the last upload travel with each call in
// pinned memory and are counted on the device on top of the uploaded list, so an engine step uploads nothing.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "klein_sampler.h"
#include "kls_internal.h"

using namespace kls;

namespace {

thread_local std::string g_err;

int fail(int status, const char* what, hipError_t e = hipSuccess) {
    char buf[256];
    if (e != hipSuccess)
        snprintf(buf, sizeof buf, "%s: %s", what, hipGetErrorString(e));
    else
        snprintf(buf, sizeof buf, "%s", what);
    g_err = buf;
    return status;
}

#define KLS_HIP(expr)                                                        \
    do {                                                                     \
        hipError_t e_ = (expr);                                              \
        if (e_ != hipSuccess) return fail(KLS_ERR_HIP, #expr, e_);           \
    } while (0)

}  // namespace

namespace kls {

int set_error(int status, const char* what, hipError_t e) { return fail(status, what, e); }

// Segment length. First choice, for vocabularies of at least 16384 ids: 1024-thread workgroups over
// 16384..65536 whole ids, the shortest that leaves at most 8 segments per row (the row's last workgroup then
// merges the lists on one wave, without a barrier) and at most wide_target_wg workgroups (measured at V =
// 248,320: 32768 ids for 1 to 16 rows, 8.6-10.1 µs against 8.9-14.4 µs with 8192-id segments; 65536 for the
// 64-row batch). Greedy rows merge trivially and read faster from more workgroups, so they skip this choice.
// Otherwise short segments (256 threads x {4, 8, 16, 32} logits): the smallest length whose grid
// (rows x segments) stays within target_wg workgroups (128: half the CUs; every segment of a row then takes the
// row's ticket, and more segments wait longer on it than their shorter reads save), and for greedy rows at most
// kGreedySegs segments per row (one wave then merges the row's maxima without a barrier: the one-row draft
// argmax measured 3.5 us with 31 segments of 8192 ids, 3.6 with 61 of 4096, 4.4 with 122 of 2048). When even 8192 ids leave
// too many workgroups, 1024-thread workgroups over 16384..65536 ids (one per CU), the smallest length within
// wide_target_wg: every logit and the row's history are then read once per segment with the chip full.
constexpr int kGreedySegs = 32;  // at most this many segments per greedy row on the short-segment layouts
void choose_segments(int V, int rows, bool greedy, int seg_override, int target_wg, int wide_target_wg, int* seg_len,
                     int* segs) {
    auto grid = [&](int sl) { return (long long) rows * ((V + sl - 1) / sl); };
    int sl = SEG_MIN;
    const int o = seg_override;
    int few = 0;
    for (int l = SEG_WIDE; l <= SEG_MAX && !few && !greedy; l *= 2)
        if (V >= l && (V + l - 1) / l <= 8 && grid(l) <= wide_target_wg) few = l;
    if (o >= SEG_MIN && o <= SEG_MAX && (o & (o - 1)) == 0) {
        sl = o;
    } else if (few) {
        sl = few;
    } else {
        while (sl < SEG_WIDE / 2 && (grid(sl) > target_wg || (greedy && (V + sl - 1) / sl > kGreedySegs))) sl *= 2;
        if (grid(sl) > target_wg) {
            sl = SEG_WIDE;
            while (sl < SEG_MAX && grid(sl) > wide_target_wg) sl *= 2;
        }
    }
    *seg_len = sl;
    *segs = (V + sl - 1) / sl;
}

// Greedy rows in the checked (not whole-float4) form keep to 32,768-id segments: the 65,536-id form of that kernel
// needs more than the 128 registers a 1024-thread workgroup allows and spills (64 rows of 248,319 ids, row stride
// 248,320: 42.1 us against 23.8 us with penalties, 14.9 against 14.5 without). The sampling kernels' checked forms
// keep 65,536 (22.7 us against 30.9).
void fit_segments(bool greedy, const float* logits, int64_t stride, int V, int* seg_len, int* segs) {
    if (greedy && *seg_len > 32768 && !rows_full(logits, stride, V, *seg_len)) {
        *seg_len = 32768;
        *segs = (V + 32767) / 32768;
    }
}

SamplingParams sampling_params(const kls_params& p, int k) {
    return SamplingParams{p.temperature, p.top_p, p.min_p, p.presence_penalty, p.frequency_penalty,
                          p.repetition_penalty, std::min(k, KCAP), 1.0 / (double) p.repetition_penalty,
                          (p.repetition_penalty >= 1.0f && p.presence_penalty >= 0.0f && p.frequency_penalty >= 0.0f)
                              ? 1 : 0};
}

}  // namespace kls

struct kls_sampler {
    kls_params p{};
    SamplingParams sp{};
    bool greedy = false, penalize = false;
    int k = 0;
    int V = 0, max_rows = 0, device = 0;
    int bucket_shift = MIN_BUCKET_SHIFT, n_buckets = 0;
    // launch layout (defaults; kls_debug_set_layout overrides them for tests)
    int seg_len_override = 0, target_wg = DEFAULT_TARGET_WG, wide_target_wg = DEFAULT_WIDE_TARGET_WG;
    int share_min_wg = DEFAULT_SHARE_MIN_WG, xcd_map = 1;
    int spin_limit = DEFAULT_SPIN_LIMIT;
    hipStream_t stream = nullptr;  // the library's stream of this device (shared by handles; not destroyed)
    // ordering of launches that share the scratch: the stream of the last launch, and an event that makes a
    // launch on another stream wait for it
    hipStream_t last_stream = nullptr;
    hipEvent_t order_ev = nullptr;
    const void* dev_ptr = nullptr;  // the last logits pointer found to be device memory

    // token history: host copy (as the reference's counts_) + what has reached the device
    std::unordered_map<int32_t, int32_t> counts;
    std::vector<int32_t> pending;  // accepted since the last upload, in order
    int32_t* d_hist_ids = nullptr;  // [V] unique ids, bucketed
    int32_t* d_hist_w = nullptr;    // [V] counts
    int32_t* d_hist_boff = nullptr; // [n_buckets + 1]
    int32_t* h_stage = nullptr;     // pinned staging for uploads: 2*V + n_buckets + 1
    bool count_wide = false;        // a device count may reach 65536

    // scratch
    uint64_t* d_seg_cand = nullptr;
    uint32_t* d_row_ticket = nullptr;
    uint64_t* d_row_thr = nullptr;
    int32_t* d_tokens = nullptr;
    int32_t* d_accepted = nullptr;  // accepted count of the last verify step
    uint64_t* d_step = nullptr;     // the verify step's row counter and mismatch bits (left zero)
    uint64_t* d_dbg_keys = nullptr;
    float* d_dbg_probs = nullptr;
    int32_t* d_dbg_meta = nullptr;
    float* d_rows_buf = nullptr;  // host logits are copied here
    int max_segs = 0;

    // mid top-k (KCAP < k <= MID_KMAX, one kernel): the rows' candidate buffers
    bool mid = false;
    MidArgs m{};
    // wide top-k (larger k, or no limit): key buffers and the sort's scratch
    bool wide = false;
    WideArgs w{};

    // pinned host blocks
    CallBlock* call = nullptr;    // host view
    ResultBlock* res = nullptr;
    CallBlock* call_dev = nullptr;  // device views of the same mapped memory
    ResultBlock* res_dev = nullptr;
    int32_t tokens[VERIFY_MAX_ROWS] = {};  // tokens of the last completed step
    uint32_t seq = 0;

    // verify graph, keyed by what it bakes in
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;
    bool inflight = false;
    hipStream_t inflight_stream = nullptr;
    int inflight_rows = 0;
    bool inflight_verify = false;
    int32_t accepted = 0;  // accepted count of the last completed verify step (as the device formed it)
    const float* g_logits = nullptr;
    int g_rows = 0;
    bool g_count_wide = false;
    bool g_verify = false;          // the captured step is a verify step (else a one-row sample on the wide path)
    bool g_valid = false;
    RowsArgs g_args{};  // the arguments the verify graph was captured with
};

namespace {

bool is_device_ptr(const void* p) {
    hipPointerAttribute_t attr;
    const hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void) hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

// The engine passes the same logits buffer every step: the last pointer found to be device memory is
// remembered, so a step makes no pointer query.
bool is_device_logits(kls_sampler* h, const void* p) {
    if (p == h->dev_ptr) return true;
    if (!is_device_ptr(p)) return false;
    h->dev_ptr = p;
    return true;
}

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;                                 // guards everything below
hipStream_t g_stream[MAX_DEVICES] = {};          // the library's stream per device
hipGraphExec_t g_prep_exec[MAX_DEVICES] = {};    // a graph of one empty kernel per device
std::unordered_set<hipStream_t> g_graph_ready;   // streams that have carried PREP_LAUNCHES graph launches

// The library's own stream of `device` (created on first use, kept for the process): handles created without
// a caller stream share it, so a new handle costs no stream creation and starts on a stream that is ready for
// graph launches. A blocking stream: like work passed the NULL stream, it is ordered with the legacy default
// stream (a caller's buffers filled there are ready before a call reads or writes them).
hipError_t library_stream(int device, hipStream_t* out) {
    if (device < 0 || device >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_stream[device]) {
        const hipError_t e = hipStreamCreateWithFlags(&g_stream[device], hipStreamDefault);
        if (e != hipSuccess) {
            g_stream[device] = nullptr;
            return e;
        }
    }
    *out = g_stream[device];
    return hipSuccess;
}

// On this ROCm the first few dozen graph launches on a stream cost two to three times the host time of later
// ones (measured on MI355X with a one-kernel graph: ~40 us instead of ~16 us for the first 40 launches of a new
// stream; launches of another graph on the stream beforehand remove the difference, direct kernel launches and
// hipGraphUpload do not). Before the first verify step on a stream, PREP_LAUNCHES launches of a graph of one
// empty kernel go through it (~3 ms, once per stream and process).
constexpr int PREP_LAUNCHES = 128;

hipError_t prepare_graph_stream(int device, hipStream_t s) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_graph_ready.count(s)) return hipSuccess;
    hipError_t e;
    if (!g_prep_exec[device]) {
        hipGraph_t g = nullptr;
        if ((e = hipGraphCreate(&g, 0)) != hipSuccess) return e;
        int unused = 0;
        void* args[] = {&unused};
        hipKernelNodeParams np{};
        np.func = const_cast<void*>(noop_kernel());
        np.gridDim = dim3(1);
        np.blockDim = dim3(64);
        np.sharedMemBytes = 0;
        np.kernelParams = args;
        np.extra = nullptr;
        hipGraphNode_t node;
        e = hipGraphAddKernelNode(&node, g, nullptr, 0, &np);
        if (e == hipSuccess) e = hipGraphInstantiate(&g_prep_exec[device], g, nullptr, nullptr, 0);
        (void) hipGraphDestroy(g);
        if (e != hipSuccess) {
            g_prep_exec[device] = nullptr;
            return e;
        }
    }
    for (int i = 0; i < PREP_LAUNCHES; ++i)
        if ((e = hipGraphLaunch(g_prep_exec[device], s)) != hipSuccess) return e;
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
    g_graph_ready.insert(s);
    return hipSuccess;
}

void segments_for(const kls_sampler* h, int rows, bool greedy, int* seg_len, int* segs) {
    choose_segments(h->V, rows, greedy, h->seg_len_override, h->target_wg, h->wide_target_wg, seg_len, segs);
}

// Rebuilds the device history from the host counts (bucketed unique ids + counts) and clears `pending`.
int upload_history(kls_sampler* h, hipStream_t s) {
    std::vector<std::pair<int32_t, int32_t>> ent(h->counts.begin(), h->counts.end());
    std::sort(ent.begin(), ent.end());
    int32_t* ids = h->h_stage;
    int32_t* w = h->h_stage + h->V;
    int32_t* bo = h->h_stage + 2 * (size_t) h->V;
    const int n = (int) ent.size();
    int b = 0;
    int32_t max_count = 0;
    for (int i = 0; i < n; ++i) {
        ids[i] = ent[i].first;
        w[i] = ent[i].second;
        max_count = std::max(max_count, ent[i].second);
        const int bi = ent[i].first >> h->bucket_shift;
        while (b <= bi) bo[b++] = i;
    }
    while (b <= h->n_buckets) bo[b++] = n;
    // the copies read the pinned staging asynchronously: wait for them before the staging is reused
    if (n > 0) {
        KLS_HIP(hipMemcpyAsync(h->d_hist_ids, ids, sizeof(int32_t) * n, hipMemcpyHostToDevice, s));
        KLS_HIP(hipMemcpyAsync(h->d_hist_w, w, sizeof(int32_t) * n, hipMemcpyHostToDevice, s));
    }
    KLS_HIP(hipMemcpyAsync(h->d_hist_boff, bo, sizeof(int32_t) * (h->n_buckets + 1), hipMemcpyHostToDevice, s));
    KLS_HIP(hipStreamSynchronize(s));
    h->pending.clear();
    // counts on the device add at most the pending ids and a step's drafts to the uploaded ones; the captured
    // verify graph bakes the table width in, so a change of width invalidates it
    h->count_wide = (int64_t) max_count + PENDING_CAP + VERIFY_MAX_ROWS >= 65536;
    if (h->count_wide != h->g_count_wide) h->g_valid = false;
    return KLS_OK;
}

RowsArgs base_args(kls_sampler* h, const float* logits, int rows, int64_t stride, bool greedy) {
    RowsArgs a{};
    a.logits = logits;
    a.row_stride = stride;
    a.V = h->V;
    a.n_rows = rows;
    if (h->mid && !greedy) {
        a.seg_len = MID_SEG;
        a.segs = mid_segments(h->V);
    } else {
        segments_for(h, rows, greedy, &a.seg_len, &a.segs);
        if (!h->seg_len_override) fit_segments(greedy, logits, stride, h->V, &a.seg_len, &a.segs);
    }
    a.p = h->sp;
    a.bucket_shift = h->bucket_shift;
    a.n_buckets = h->n_buckets;
    a.seg_cand = h->d_seg_cand;
    a.row_ticket = h->d_row_ticket;
    a.row_thr = h->d_row_thr;
    a.share_bounds = (long long) rows * a.segs > h->share_min_wg ? 1 : 0;
    a.xcd_map = h->xcd_map;
    a.out_tokens = h->d_tokens;
    a.dbg_keys = h->d_dbg_keys;
    a.dbg_probs = h->d_dbg_probs;
    a.dbg_meta = h->d_dbg_meta;
    a.fault = &h->res_dev->fault;
    a.spin_limit = h->spin_limit;
    return a;
}

// Arguments of a step over the handle's own history: rows read their uniforms and drafts from the pinned call
// block, and count the handle's pending ids (and, for row i, drafts 0..i-1) on top of the uploaded history.
RowsArgs step_args(kls_sampler* h, const float* logits, int rows, bool verify) {
    RowsArgs a = base_args(h, logits, rows, h->V, h->greedy);
    if (h->penalize) {
        a.hist_ids = h->d_hist_ids;
        a.hist_w = h->d_hist_w;
        a.hist_boff = h->d_hist_boff;
        a.count_wide = h->count_wide ? 1 : 0;

        a.extra_a = h->call_dev->pending;
        a.extra_a_n = &h->call_dev->n_pending;
        a.extra_b = verify ? h->call_dev->drafts : nullptr;
        a.extra_b_step = verify ? 1 : 0;
    }
    a.u = h->call_dev->u;
    a.host_res = h->res_dev;
    a.call = h->call_dev;
    if (verify) {
        a.step_word = h->d_step;
        a.out_accepted = h->d_accepted;
    }
    return a;
}

// The sampling kernels of the handle's path over `a` (the fast path and the mid top-k path: one kernel each;
// the wide path: keys, the radix sort's passes, the tail). None of them sets memory with a memset, so a verify
// step of any path can be captured in a graph.
hipError_t launch_sampling(const kls_sampler* h, const RowsArgs& a, bool penalize, hipStream_t s) {
    if (h->wide) return launch_wide(a, h->w, penalize, s);
    if (h->mid) return launch_mid(a, h->m, penalize, s);
    return launch_rows(a, h->greedy, penalize, s);
}

int check_handle(kls_handle h) {
    if (!h) return fail(KLS_ERR_INVALID_ARG, "null handle");
    return KLS_OK;
}

// Turns a fault a kernel of this handle reported (an internal wait that gave up) into an error, once.
int check_fault(kls_sampler* h) {
    const uint32_t f = __atomic_load_n(&h->res->fault, __ATOMIC_ACQUIRE);
    if (f == 0u) return KLS_OK;
    __atomic_store_n(&h->res->fault, 0u, __ATOMIC_RELEASE);
    char buf[160];
    snprintf(buf, sizeof buf, "a sampling kernel of this handle gave up an internal wait (code %u): its results are "
                              "not valid", f);
    return fail(KLS_ERR_HIP, buf);
}

// Orders a launch on `s` after the handle's previous launches, which share its scratch: when the stream changes,
// `s` waits for everything enqueued on the previous one so far.
int order_on(kls_sampler* h, hipStream_t s) {
    if (h->last_stream && h->last_stream != s) {
        KLS_HIP(hipEventRecord(h->order_ev, h->last_stream));
        KLS_HIP(hipStreamWaitEvent(s, h->order_ev, 0));
    }
    h->last_stream = s;
    return KLS_OK;
}

// Entry checks of the asynchronous calls that lend the handle's scratch.
int check_async(kls_sampler* h, hipStream_t s) {
    if (h->inflight) return fail(KLS_ERR_INVALID_ARG, "a verify or sample step is in flight on this handle");
    if (int st = check_fault(h)) return st;
    return order_on(h, s);
}

// Brings the device history up to date before a step: pending ids ride in the call block up to its capacity.
int prepare_history(kls_sampler* h, hipStream_t s) {
    if (!h->penalize) return KLS_OK;
    if ((int) h->pending.size() > PENDING_CAP) {
        const int st = upload_history(h, s);
        if (st) return st;
    }
    h->call->n_pending = (int32_t) h->pending.size();
    std::copy(h->pending.begin(), h->pending.end(), h->call->pending);
    return KLS_OK;
}

// Enqueues one step over `rows` rows of the handle's history on `s`; results land in the pinned block. The
// caller has checked that no step is in flight and written the step's uniforms (and drafts) to the call block.
int enqueue_step(kls_sampler* h, const float* logits, int rows, bool verify, hipStream_t s) {
    if (int st = check_fault(h)) return st;
    if (int st = order_on(h, s)) return st;
    const float* dl = logits;
    if (!is_device_logits(h, logits)) {
        KLS_HIP(hipMemcpyAsync(h->d_rows_buf, logits, sizeof(float) * (size_t) rows * h->V, hipMemcpyHostToDevice, s));
        dl = h->d_rows_buf;
    }
    int st = prepare_history(h, s);
    if (st) return st;
    h->call->seq = ++h->seq;
    const RowsArgs a = step_args(h, dl, rows, verify);
    // A verify step is one graph launch; so is a sample on the wide path, whose keys, radix passes and tail are
    // many kernels (one graph launch costs the host less than their direct launches). A fast- or mid-path sample is
    // one kernel, launched directly. The graph is kept while the logits pointer, the row count and the kind of
    // step stay the same.
    if (verify || h->wide) {
        if (!h->g_valid || h->g_logits != dl || h->g_rows != rows || h->g_verify != verify) {
            // (a stale graph is replaced whether or not its teardown reports an error)
            if (h->gexec) (void) hipGraphExecDestroy(h->gexec);
            if (h->graph) (void) hipGraphDestroy(h->graph);
            h->gexec = nullptr;
            h->graph = nullptr;
            h->g_valid = false;
            hipStream_t cap = nullptr;
            KLS_HIP(hipStreamCreateWithFlags(&cap, hipStreamNonBlocking));
            const hipError_t be = hipStreamBeginCapture(cap, hipStreamCaptureModeRelaxed);
            const hipError_t le = be == hipSuccess ? launch_sampling(h, a, h->penalize, cap) : hipSuccess;
            hipGraph_t g = nullptr;
            const hipError_t ce = be == hipSuccess ? hipStreamEndCapture(cap, &g) : hipSuccess;
            (void) hipStreamDestroy(cap);
            if (be != hipSuccess) return fail(KLS_ERR_HIP, "hipStreamBeginCapture", be);
            if (le != hipSuccess) return fail(KLS_ERR_HIP, "sampling kernel (capture)", le);
            if (ce != hipSuccess) return fail(KLS_ERR_HIP, "hipStreamEndCapture", ce);
            h->graph = g;
            KLS_HIP(hipGraphInstantiate(&h->gexec, h->graph, nullptr, nullptr, 0));
            h->g_logits = dl;
            h->g_rows = rows;
            h->g_count_wide = h->count_wide;
            h->g_verify = verify;
            h->g_args = a;
            h->g_valid = true;
        }
        KLS_HIP(prepare_graph_stream(h->device, s));
        KLS_HIP(hipGraphLaunch(h->gexec, s));
    } else {
        KLS_HIP(launch_sampling(h, a, h->penalize, s));
    }
    h->inflight = true;
    h->inflight_stream = s;
    h->inflight_rows = rows;
    h->inflight_verify = verify;
    return KLS_OK;
}

// Waits for the in-flight step: spins on the sequence numbers the kernel publishes (a verify step's accepted
// count, then each row's token), falling back to a stream synchronization after 50 ms (queued work ahead of the
// step, or a failure).
int wait_step(kls_sampler* h) {
    if (!h->inflight) return fail(KLS_ERR_INVALID_ARG, "no step in flight on this handle");
    h->inflight = false;
    const uint32_t want = h->call->seq;
    const int rows = h->inflight_rows;
    const bool verify = h->inflight_verify;
    auto done = [&] {
        if (verify) {
            const uint64_t w = __atomic_load_n(&h->res->step_word, __ATOMIC_ACQUIRE);
            if ((uint32_t) (w >> 32) != want) return false;
            h->accepted = (int32_t) (uint32_t) w;
        }
        for (int r = 0; r < rows; ++r) {
            const uint64_t w = __atomic_load_n(&h->res->row_word[r], __ATOMIC_ACQUIRE);
            if ((uint32_t) (w >> 32) != want) return false;
            h->tokens[r] = (int32_t) (uint32_t) w;
        }
        return true;
    };
    const auto t0 = std::chrono::steady_clock::now();
    while (!done()) {
        if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(50)) {
            KLS_HIP(hipStreamSynchronize(h->inflight_stream));
            if (!done()) {
                if (int st = check_fault(h)) return st;
                return fail(KLS_ERR_HIP, "step result not published");
            }
            break;
        }
#if defined(__x86_64__)
        __builtin_ia32_pause();
#endif
    }
    return check_fault(h);
}

void add_history(kls_sampler* h, int32_t t) {
    h->counts[t]++;
    // (the device copy of the history is read only with penalties)
    if (h->penalize) h->pending.push_back(t);
}

}  // namespace

extern "C" {

const char* kls_status_string(int status) {
    switch (status) {
        case KLS_OK: return "ok";
        case KLS_ERR_INVALID_ARG: return "invalid argument";
        case KLS_ERR_RANGE: return "out of range";
        case KLS_ERR_UNSUPPORTED: return "unsupported";
        case KLS_ERR_HIP: return "HIP runtime error";
        case KLS_ERR_NO_DEVICE: return "no GPU device";
        case KLS_ERR_OOM: return "out of memory";
        default: return "unknown status";
    }
}

const char* kls_last_error(void) { return g_err.c_str(); }

int kls_destroy(kls_handle h) {
    if (!h) return fail(KLS_ERR_INVALID_ARG, "null handle");
    (void) hipSetDevice(h->device);
    // (the handle's work may be on any stream it was given: wait for the device)
    (void) hipDeviceSynchronize();
    if (h->gexec) (void) hipGraphExecDestroy(h->gexec);
    if (h->graph) (void) hipGraphDestroy(h->graph);
    void* dev[] = {h->d_hist_ids, h->d_hist_w, h->d_hist_boff, h->d_seg_cand,
                   h->d_row_ticket, h->d_row_thr, h->d_tokens, h->d_accepted,
                   h->d_step, h->d_dbg_keys, h->d_dbg_probs, h->d_dbg_meta,
                   h->d_rows_buf, h->w.keys, h->w.sorted, h->w.counts, h->w.part, h->w.seg, h->w.nseg, h->w.rowst,
                   h->m.buf, h->m.fill};
    for (void* p : dev)
        if (p) (void) hipFree(p);
    if (h->h_stage) (void) hipHostFree(h->h_stage);
    if (h->call) (void) hipHostFree(h->call);
    if (h->res) (void) hipHostFree(h->res);
    if (h->order_ev) (void) hipEventDestroy(h->order_ev);
    delete h;
    return KLS_OK;
}

int kls_create(const kls_params* params, int n_vocab, int max_rows, kls_handle* out) {
    if (!params || !out) return fail(KLS_ERR_INVALID_ARG, "null argument");
    *out = nullptr;
    if (n_vocab <= 0) return fail(KLS_ERR_INVALID_ARG, "n_vocab must be positive");
    if (max_rows < 1) return fail(KLS_ERR_INVALID_ARG, "max_rows must be positive");
    const int k = (params->top_k > 0 && params->top_k < n_vocab) ? params->top_k : n_vocab;
    // k above KCAP: the mid path up to MID_KMAX (while the rows' buffers hold every segment's share), else the
    // wide path, whose radix sort indexes the rows' keys with 32 bits
    const bool mid = params->temperature > 0.0f && mid_fits(n_vocab, k);
    const bool wide = params->temperature > 0.0f && k > KCAP && !mid;
    if (wide && (long long) n_vocab * max_rows >= (1ll << 32))
        return fail(KLS_ERR_UNSUPPORTED, "top-k above 64 with this many rows of this vocabulary");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
        (void) hipGetLastError();
        return fail(KLS_ERR_NO_DEVICE, "no GPU visible");
    }
    kls_sampler* h = new kls_sampler();
    h->p = *params;
    h->V = n_vocab;
    h->max_rows = max_rows;
    h->k = k;
    h->greedy = params->temperature <= 0.0f;
    h->mid = mid;
    h->wide = wide;
    h->penalize = params->presence_penalty != 0.0f || params->frequency_penalty != 0.0f ||
                  params->repetition_penalty != 1.0f;
    h->sp = sampling_params(*params, k);
    while (((n_vocab + (1 << h->bucket_shift) - 1) >> h->bucket_shift) > MAX_BUCKETS) h->bucket_shift++;
    h->n_buckets = (n_vocab + (1 << h->bucket_shift) - 1) >> h->bucket_shift;
    (void) hipGetDevice(&h->device);

    auto oom = [&](const char* what, hipError_t e) {
        kls_destroy(h);
        return fail(KLS_ERR_OOM, what, e);
    };
    hipError_t e;
    if ((e = library_stream(h->device, &h->stream)) != hipSuccess) {
        kls_destroy(h);
        return fail(KLS_ERR_HIP, "library stream", e);
    }
    if ((e = hipEventCreateWithFlags(&h->order_ev, hipEventDisableTiming)) != hipSuccess) return oom("event", e);
    if ((e = prepare_rows_kernels()) != hipSuccess || (mid && (e = prepare_mid_kernels()) != hipSuccess)) {
        kls_destroy(h);
        return fail(KLS_ERR_HIP, "kernel LDS limits", e);
    }
    h->max_segs = (n_vocab + SEG_MIN - 1) / SEG_MIN;
    const size_t R = (size_t) max_rows;
#define ALLOC(ptr, bytes) \
    if ((e = hipMalloc((void**) &(ptr), (bytes))) != hipSuccess) return oom(#ptr, e)
    ALLOC(h->d_hist_ids, sizeof(int32_t) * n_vocab);
    ALLOC(h->d_hist_w, sizeof(int32_t) * n_vocab);
    ALLOC(h->d_hist_boff, sizeof(int32_t) * (h->n_buckets + 1));
    ALLOC(h->d_seg_cand, sizeof(uint64_t) * R * h->max_segs * KCAP);
    ALLOC(h->d_row_ticket, sizeof(uint32_t) * R);
    ALLOC(h->d_row_thr, sizeof(uint64_t) * R);
    ALLOC(h->d_tokens, sizeof(int32_t) * R);
    ALLOC(h->d_accepted, sizeof(int32_t));
    ALLOC(h->d_step, sizeof(uint64_t));
    ALLOC(h->d_dbg_keys, sizeof(uint64_t) * R * KCAP);
    ALLOC(h->d_dbg_probs, sizeof(float) * R * KCAP);
    ALLOC(h->d_dbg_meta, sizeof(int32_t) * R * 2);
    ALLOC(h->d_rows_buf, sizeof(float) * R * n_vocab);
    if (mid) {
        h->m.k = k;
        h->m.cap = MID_ROWCAP / mid_segments(n_vocab);
        ALLOC(h->m.buf, sizeof(uint64_t) * R * MID_ROWCAP);
        ALLOC(h->m.fill, sizeof(uint32_t) * R);
    }
    if (wide) {
        h->w.k = k;
        h->w.id_bits = wide_id_bits(n_vocab);
        ALLOC(h->w.keys, sizeof(uint64_t) * R * n_vocab);
        ALLOC(h->w.sorted, sizeof(uint64_t) * R * n_vocab);
        ALLOC(h->w.counts, sizeof(uint32_t) * 256 * R * sort_tiles((size_t) n_vocab));
        h->w.chunks = (k + WT_CHUNK - 1) / WT_CHUNK;
        h->w.seg_cap = WT_SEGS;
        ALLOC(h->w.part, sizeof(double) * R * h->w.chunks);
        ALLOC(h->w.seg, sizeof(WideSeg) * R * h->w.chunks * WT_SEGS);
        ALLOC(h->w.nseg, sizeof(int32_t) * R * h->w.chunks);
        ALLOC(h->w.rowst, sizeof(WideRow) * R);
    }
#undef ALLOC
    if ((e = hipHostMalloc((void**) &h->h_stage, sizeof(int32_t) * (2 * (size_t) n_vocab + h->n_buckets + 1),
                           hipHostMallocDefault)) != hipSuccess)
        return oom("pinned staging", e);
    if ((e = hipHostMalloc((void**) &h->call, sizeof(CallBlock), hipHostMallocMapped | hipHostMallocCoherent)) !=
        hipSuccess)
        return oom("pinned call block", e);
    if ((e = hipHostMalloc((void**) &h->res, sizeof(ResultBlock), hipHostMallocMapped | hipHostMallocCoherent)) !=
        hipSuccess)
        return oom("pinned result block", e);
    if ((e = hipHostGetDevicePointer((void**) &h->call_dev, h->call, 0)) != hipSuccess) return oom("mapped call", e);
    if ((e = hipHostGetDevicePointer((void**) &h->res_dev, h->res, 0)) != hipSuccess) return oom("mapped res", e);
    std::memset(h->call, 0, sizeof(CallBlock));
    std::memset(h->res, 0, sizeof(ResultBlock));
    // zero the self-resetting counters and bounds once; the kernels leave them zero after every launch
    if ((e = hipMemsetAsync(h->d_row_ticket, 0, sizeof(uint32_t) * R, h->stream)) != hipSuccess) return oom("init", e);
    if ((e = hipMemsetAsync(h->d_row_thr, 0, sizeof(uint64_t) * R, h->stream)) != hipSuccess) return oom("init", e);
    if ((e = hipMemsetAsync(h->d_hist_boff, 0, sizeof(int32_t) * (h->n_buckets + 1), h->stream)) != hipSuccess)
        return oom("init", e);
    if ((e = hipMemsetAsync(h->d_step, 0, sizeof(uint64_t), h->stream)) != hipSuccess) return oom("init", e);
    if (mid && (e = hipMemsetAsync(h->m.fill, 0, sizeof(uint32_t) * R, h->stream)) != hipSuccess) return oom("init", e);
    if ((e = hipMemsetAsync(h->d_accepted, 0, sizeof(int32_t), h->stream)) != hipSuccess) return oom("init", e);
    if ((e = hipStreamSynchronize(h->stream)) != hipSuccess) return oom("init", e);
    *out = h;
    return KLS_OK;
}

int kls_reset(kls_handle h) {
    if (int st = check_handle(h)) return st;
    if (h->inflight) return fail(KLS_ERR_INVALID_ARG, "a step is in flight on this handle");
    h->counts.clear();
    h->pending.clear();
    (void) hipSetDevice(h->device);
    return h->penalize ? upload_history(h, h->stream) : KLS_OK;
}

int kls_accept(kls_handle h, int32_t token) {
    if (int st = check_handle(h)) return st;
    if (token < 0 || token >= h->V) return fail(KLS_ERR_RANGE, "token outside [0, n_vocab)");
    if (h->inflight) return fail(KLS_ERR_INVALID_ARG, "a step is in flight on this handle");
    add_history(h, token);
    return KLS_OK;
}

int kls_sample(kls_handle h, const float* logits, int n_vocab, double u, int32_t* out_token) {
    if (int st = check_handle(h)) return st;
    if (!logits || !out_token) return fail(KLS_ERR_INVALID_ARG, "null argument");
    if (n_vocab != h->V) return fail(KLS_ERR_INVALID_ARG, "n_vocab differs from the handle's");
    // (checked before the call block is written: a running step reads it)
    if (h->inflight) return fail(KLS_ERR_INVALID_ARG, "a step is already in flight on this handle");
    (void) hipSetDevice(h->device);
    h->call->u[0] = u;
    int st = enqueue_step(h, logits, 1, false, h->stream);
    if (!st) st = wait_step(h);
    if (st) return st;
    *out_token = h->tokens[0];
    return KLS_OK;
}

int kls_verify_enqueue(kls_handle h, const float* logits, int nb, const int32_t* drafts, const double* u,
                       kls_stream stream) {
    if (int st = check_handle(h)) return st;
    if (!logits || !u || (nb > 1 && !drafts)) return fail(KLS_ERR_INVALID_ARG, "null argument");
    if (nb < 1) return fail(KLS_ERR_INVALID_ARG, "nb must be at least 1");
    if (nb > h->max_rows || nb > VERIFY_MAX_ROWS) return fail(KLS_ERR_RANGE, "nb above the handle's capacity");
    // (checked before the call block is written: a running step reads it)
    if (h->inflight) return fail(KLS_ERR_INVALID_ARG, "a step is already in flight on this handle");
    (void) hipSetDevice(h->device);
    hipStream_t s = stream ? (hipStream_t) stream : h->stream;
    for (int i = 0; i < nb; ++i) h->call->u[i] = u[i];
    for (int i = 0; i + 1 < nb; ++i) h->call->drafts[i] = drafts[i];
    return enqueue_step(h, logits, nb, true, s);
}

int kls_verify_wait(kls_handle h, int32_t* out_tokens, int32_t* out_accepted) {
    if (int st = check_handle(h)) return st;
    if (!out_tokens || !out_accepted) return fail(KLS_ERR_INVALID_ARG, "null argument");
    if (h->inflight && !h->inflight_verify) return fail(KLS_ERR_INVALID_ARG, "no verify step in flight on this handle");
    const int nb = h->inflight_rows;
    if (int st = wait_step(h)) return st;
    // the accepted count as the device formed it (engine.cpp:564-575: drafts accepted while batch[i+1] == t_i)
    const int acc = h->accepted;
    if (acc < 0 || acc >= nb) return fail(KLS_ERR_HIP, "accepted count out of range");
    for (int i = 0; i < nb; ++i) out_tokens[i] = h->tokens[i];
    for (int i = 0; i <= acc; ++i) add_history(h, out_tokens[i]);
    *out_accepted = acc;
    return KLS_OK;
}

int kls_verify(kls_handle h, const float* logits, int nb, const int32_t* drafts, const double* u,
               int32_t* out_tokens, int32_t* out_accepted, kls_stream stream) {
    if (int st = check_handle(h)) return st;
    if (!out_tokens || !out_accepted) return fail(KLS_ERR_INVALID_ARG, "null argument");
    if (int st = kls_verify_enqueue(h, logits, nb, drafts, u, stream)) return st;
    return kls_verify_wait(h, out_tokens, out_accepted);
}

int kls_device_results(kls_handle h, const int32_t** d_tokens, const int32_t** d_accepted) {
    if (int st = check_handle(h)) return st;
    if (!d_tokens && !d_accepted) return fail(KLS_ERR_INVALID_ARG, "null argument");
    if (d_tokens) *d_tokens = h->d_tokens;
    if (d_accepted) *d_accepted = h->d_accepted;
    return KLS_OK;
}

int kls_check(kls_handle h) {
    if (int st = check_handle(h)) return st;
    return check_fault(h);
}

int kls_debug_set_layout(kls_handle h, const kls_debug_layout* l) {
    if (int st = check_handle(h)) return st;
    if (!l) return fail(KLS_ERR_INVALID_ARG, "null argument");
    if (h->inflight) return fail(KLS_ERR_INVALID_ARG, "a step is in flight on this handle");
    const int o = l->seg_len;
    if (o != 0 && (o < SEG_MIN || o > SEG_MAX || (o & (o - 1)) != 0))
        return fail(KLS_ERR_INVALID_ARG, "segment length must be 0 or a power of two in [1024, 65536]");
    if (l->target_wg < 0 || l->wide_target_wg < 0 || l->share_min_wg < 0 || l->xcd_map < -1 || l->xcd_map > 1 ||
        l->wide_segs < 0 || l->wide_segs > WT_SEGS)
        return fail(KLS_ERR_INVALID_ARG, "layout field out of range");
    h->seg_len_override = o;
    if (l->target_wg) h->target_wg = l->target_wg;
    if (l->wide_target_wg) h->wide_target_wg = l->wide_target_wg;
    if (l->share_min_wg) h->share_min_wg = l->share_min_wg;
    if (l->xcd_map >= 0) h->xcd_map = l->xcd_map;
    h->spin_limit = l->wait_limit == 0 ? DEFAULT_SPIN_LIMIT : l->wait_limit < 0 ? 0 : l->wait_limit;
    h->w.seg_cap = l->wide_segs == 0 ? WT_SEGS : l->wide_segs;
    h->g_valid = false;  // (the verify graph bakes the layout in)
    return KLS_OK;
}

int kls_sample_batch(kls_handle h, const float* d_logits, int n_rows, int64_t row_stride, const int32_t* d_hist_off,
                     const int32_t* d_hist_ids, const double* d_u, int32_t* d_out_tokens, kls_stream stream) {
    if (int st = check_handle(h)) return st;
    if (!d_logits || !d_out_tokens || (!h->greedy && !d_u)) return fail(KLS_ERR_INVALID_ARG, "null argument");
    if ((d_hist_off == nullptr) != (d_hist_ids == nullptr))
        return fail(KLS_ERR_INVALID_ARG, "history offsets and ids go together");
    if (n_rows < 1) return fail(KLS_ERR_INVALID_ARG, "n_rows must be positive");
    if (n_rows > h->max_rows) return fail(KLS_ERR_RANGE, "n_rows above the handle's capacity");
    if (row_stride < h->V) return fail(KLS_ERR_INVALID_ARG, "row_stride below n_vocab");
    (void) hipSetDevice(h->device);
    hipStream_t s = stream ? (hipStream_t) stream : h->stream;
    if (int st = check_async(h, s)) return st;
    RowsArgs a = base_args(h, d_logits, n_rows, row_stride, h->greedy);
    const bool pen = h->penalize && d_hist_off != nullptr;
    if (pen) {
        a.hist_ids = d_hist_ids;
        a.hist_off = d_hist_off;
    }
    a.u = d_u;
    a.out_tokens = d_out_tokens;
    KLS_HIP(launch_sampling(h, a, pen, s));
    return KLS_OK;
}

int kls_argmax(kls_handle h, const float* d_logits, int n_rows, int64_t row_stride, int32_t* d_out,
               kls_stream stream) {
    if (int st = check_handle(h)) return st;
    if (!d_logits || !d_out) return fail(KLS_ERR_INVALID_ARG, "null argument");
    if (n_rows < 1) return fail(KLS_ERR_INVALID_ARG, "n_rows must be positive");
    if (n_rows > h->max_rows) return fail(KLS_ERR_RANGE, "n_rows above the handle's capacity");
    if (row_stride < h->V) return fail(KLS_ERR_INVALID_ARG, "row_stride below n_vocab");
    (void) hipSetDevice(h->device);
    hipStream_t s = stream ? (hipStream_t) stream : h->stream;
    if (int st = check_async(h, s)) return st;
    RowsArgs a = base_args(h, d_logits, n_rows, row_stride, true);
    a.out_tokens = d_out;
    a.first_nan = 1;
    // (the greedy kernel: first maximum under '>' from -inf, plus the NaN-first case; no penalties)
    KLS_HIP(launch_rows(a, true, false, s));
    return KLS_OK;
}

int kls_ppl_scores(kls_handle h, const float* d_logits, int n_rows, int64_t row_stride, const int32_t* d_targets,
                   const float* d_base, int64_t base_stride, double* d_lse, double* d_nll, int32_t* d_top,
                   double* d_kl, double* d_nll_base, int32_t* d_base_top, kls_stream stream) {
    if (int st = check_handle(h)) return st;
    if (!d_logits) return fail(KLS_ERR_INVALID_ARG, "null logits");
    if (d_nll && !d_targets) return fail(KLS_ERR_INVALID_ARG, "nll needs targets");
    if ((d_kl || d_nll_base || d_base_top) && !d_base) return fail(KLS_ERR_INVALID_ARG, "KL outputs need a base row");
    if (d_nll_base && !d_targets) return fail(KLS_ERR_INVALID_ARG, "base nll needs targets");
    if (n_rows < 1) return fail(KLS_ERR_INVALID_ARG, "n_rows must be positive");
    if (n_rows > h->max_rows) return fail(KLS_ERR_RANGE, "n_rows above the handle's capacity");
    if (row_stride < h->V || (d_base && base_stride < h->V)) return fail(KLS_ERR_INVALID_ARG, "row stride below n_vocab");
    (void) hipSetDevice(h->device);
    hipStream_t s = stream ? (hipStream_t) stream : h->stream;
    if (int st = check_async(h, s)) return st;
    PplArgs a{};
    a.logits = d_logits;
    a.row_stride = row_stride;
    a.base = d_base;
    a.base_stride = base_stride;
    a.targets = d_targets;
    a.V = h->V;
    a.n_rows = n_rows;
    a.segs = ppl_segments(h->V, n_rows, &a.seg_len);
    if (a.segs > h->max_segs) return fail(KLS_ERR_UNSUPPORTED, "ppl segments exceed the scratch");
    a.scratch = h->d_seg_cand;
    a.ticket = h->d_row_ticket;
    a.out_lse = d_lse;
    a.out_nll = d_nll;
    a.out_top = d_top;
    a.out_kl = d_kl;
    a.out_nll_base = d_nll_base;
    a.out_base_top = d_base_top;
    KLS_HIP(launch_ppl(a, s));
    return KLS_OK;
}

int kls_get_candidates(kls_handle h, int row, int32_t* ids, float* probs, int cap, int32_t* n_k, int32_t* n_kept) {
    if (int st = check_handle(h)) return st;
    if (row < 0 || row >= h->max_rows) return fail(KLS_ERR_RANGE, "row outside the handle's capacity");
    if (cap < 0 || (cap > 0 && (!ids || !probs))) return fail(KLS_ERR_INVALID_ARG, "bad output buffers");
    if (h->inflight) return fail(KLS_ERR_INVALID_ARG, "a step is in flight on this handle");
    (void) hipSetDevice(h->device);
    KLS_HIP(hipDeviceSynchronize());
    uint64_t keys[KCAP];
    float pr[KCAP];
    int32_t meta[2];
    KLS_HIP(hipMemcpy(keys, h->d_dbg_keys + (size_t) row * KCAP, sizeof keys, hipMemcpyDeviceToHost));
    KLS_HIP(hipMemcpy(pr, h->d_dbg_probs + (size_t) row * KCAP, sizeof pr, hipMemcpyDeviceToHost));
    KLS_HIP(hipMemcpy(meta, h->d_dbg_meta + (size_t) row * 2, sizeof meta, hipMemcpyDeviceToHost));
    const int n = std::min(cap, std::min(meta[0], KCAP));
    for (int i = 0; i < n; ++i) {
        ids[i] = (int32_t) ~(uint32_t) keys[i];
        probs[i] = pr[i];
    }
    if (n_k) *n_k = meta[0];
    if (n_kept) *n_kept = meta[1];
    return KLS_OK;
}

int kls_debug_time_verify(kls_handle h, int n, int reps, kls_stream stream, double* out_us) {
    if (int st = check_handle(h)) return st;
    if (n < 1 || reps < 1 || !out_us) return fail(KLS_ERR_INVALID_ARG, "bad arguments");
    if (h->inflight) return fail(KLS_ERR_INVALID_ARG, "a step is in flight on this handle");
    if (!h->g_valid || !h->g_verify) return fail(KLS_ERR_INVALID_ARG, "no captured verify step on this handle");
    (void) hipSetDevice(h->device);
    hipStream_t s = stream ? (hipStream_t) stream : h->stream;
    if (int st = order_on(h, s)) return st;
    // n launches of the verify kernel with the captured step's arguments, captured back to back in one graph
    hipStream_t cap = nullptr;
    KLS_HIP(hipStreamCreateWithFlags(&cap, hipStreamNonBlocking));
    hipError_t e = hipStreamBeginCapture(cap, hipStreamCaptureModeRelaxed);
    for (int i = 0; i < n && e == hipSuccess; ++i) e = launch_sampling(h, h->g_args, h->penalize, cap);
    hipGraph_t g = nullptr;
    const hipError_t ce = hipStreamEndCapture(cap, &g);
    (void) hipStreamDestroy(cap);
    if (e != hipSuccess) return fail(KLS_ERR_HIP, "sampling kernel (capture)", e);
    if (ce != hipSuccess) return fail(KLS_ERR_HIP, "hipStreamEndCapture", ce);
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void) hipGraphDestroy(g);
    if (e != hipSuccess) return fail(KLS_ERR_HIP, "hipGraphInstantiate", e);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.0f;
    e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = prepare_graph_stream(h->device, s);
    if (e == hipSuccess) e = hipGraphLaunch(x, s);  // (once untimed)
    if (e == hipSuccess) e = hipEventRecord(e0, s);
    for (int r = 0; r < reps && e == hipSuccess; ++r) e = hipGraphLaunch(x, s);
    if (e == hipSuccess) e = hipEventRecord(e1, s);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) (void) hipEventDestroy(e0);
    if (e1) (void) hipEventDestroy(e1);
    (void) hipGraphExecDestroy(x);
    if (e != hipSuccess) return fail(KLS_ERR_HIP, "timed replay", e);
    *out_us = (double) ms * 1e3 / ((double) n * reps);
    return check_fault(h);
}

int kls_debug_run_verify_steps(kls_handle h, const float* logits, int nb, int n_steps, const int32_t* drafts,
                               const double* u, int32_t* out_tokens, int32_t* out_accepted, int64_t* out_step_ns,
                               kls_stream stream) {
    if (int st = check_handle(h)) return st;
    if (n_steps < 1 || nb < 1 || !drafts || !u || !out_tokens || !out_accepted)
        return fail(KLS_ERR_INVALID_ARG, "bad arguments");
    for (int i = 0; i < n_steps; ++i) {
        const auto t0 = std::chrono::steady_clock::now();
        const int st = kls_verify(h, logits, nb, drafts + (int64_t) i * (nb > 1 ? nb - 1 : 0), u + (int64_t) i * nb,
                                  out_tokens + (int64_t) i * nb, out_accepted + i, stream);
        const auto t1 = std::chrono::steady_clock::now();
        if (out_step_ns) out_step_ns[i] = std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count();
        if (st) return st;
    }
    return KLS_OK;
}

int kls_debug_path(kls_handle h, int32_t* out_path) {
    if (int st = check_handle(h)) return st;
    if (!out_path) return fail(KLS_ERR_INVALID_ARG, "null argument");
    *out_path = h->wide ? KLS_PATH_WIDE : h->mid ? KLS_PATH_MID : KLS_PATH_FAST;
    return KLS_OK;
}

int kls_debug_sum_replay(const double* d_terms, int n, double acc0, int mode, double thr, double* d_out,
                         kls_stream stream) {
    if ((!d_terms && n > 0) || !d_out || n < 0 || mode < 0 || mode > 2) return fail(KLS_ERR_INVALID_ARG, "bad arguments");
    KLS_HIP(launch_sum_replay(d_terms, n, acc0, mode, thr, d_out, (hipStream_t) stream));
    return KLS_OK;
}

// Test hook: expf of the consecutive float bit patterns lo, lo+1, ... (n of them) into device memory `out`.
int kls_debug_expf(uint32_t lo, long long n, float* out, kls_stream stream) {
    if (!out || n < 0) return fail(KLS_ERR_INVALID_ARG, "bad arguments");
    KLS_HIP(launch_expf_table(lo, n, out, (hipStream_t) stream));
    return KLS_OK;
}

}  // extern "C"

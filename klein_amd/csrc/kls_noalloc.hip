// kls_sample_batch_noalloc: the batched sampling entry point for callers that cannot allocate device memory
// (code under HIP graph capture, serving loops that forbid hipMalloc). It takes no handle: the scratch the
// sampling kernel needs (per (row, segment) candidate lists, per-row tickets and bounds) lives in the
// file-scope device array `scratch` below, resolved once per device with hipGetSymbolAddress.
#include <hip/hip_runtime.h>

#include <mutex>

#include "klein_sampler.h"
#include "kls_internal.h"

namespace kls {
namespace {

constexpr int NA_MAX_ROWS = KLS_NOALLOC_MAX_ROWS;
constexpr int NA_MAX_ITEMS = KLS_NOALLOC_MAX_WORKGROUPS;
constexpr size_t CAND_BYTES = (size_t) NA_MAX_ITEMS * KCAP * sizeof(uint64_t);   // 512 KiB
constexpr size_t TICKET_OFF = CAND_BYTES;
constexpr size_t THR_OFF = TICKET_OFF + (size_t) NA_MAX_ROWS * sizeof(uint32_t);
constexpr size_t SCRATCH_BYTES = THR_OFF + (size_t) NA_MAX_ROWS * sizeof(uint64_t);
static_assert(THR_OFF % 8 == 0, "bound words are 64-bit");

// Every GPU the library runs on holds its own copy until the process ends. Host code never uses this name as
// an address: it uses the per-device address that hipGetSymbolAddress returns (scratch_addr).
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void* scratch_addr[MAX_DEVICES] = {};

// Clears the tickets and bounds of rows [0, n): the kernel leaves them zero after a launch that completes, but
// the array keeps whatever the last call on this GPU left.
__global__ void clear_rows_kernel(uint32_t* ticket, uint64_t* thr, int n) {
    const int i = (int) (blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) {
        ticket[i] = 0u;
        thr[i] = 0ull;
    }
}

// The address of `scratch` on the current device, resolved (and the kernels' LDS limits set) on the first call
// with that device current.
hipError_t device_scratch(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!scratch_addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        if ((e = prepare_rows_kernels()) != hipSuccess) return e;
        scratch_addr[dev] = p;
    }
    *out = scratch_addr[dev];
    return hipSuccess;
}

}  // namespace
}  // namespace kls

using namespace kls;

extern "C" int kls_sample_batch_noalloc(const kls_params* params, int n_vocab, const float* d_logits, int n_rows,
                                        int64_t row_stride, const int32_t* d_hist_off, const int32_t* d_hist_ids,
                                        const double* d_u, int32_t* d_out_tokens, kls_stream stream) {
    if (!params || !d_logits || !d_out_tokens) return set_error(KLS_ERR_INVALID_ARG, "null argument");
    const bool greedy = params->temperature <= 0.0f;
    if (!greedy && !d_u) return set_error(KLS_ERR_INVALID_ARG, "null uniforms");
    if ((d_hist_off == nullptr) != (d_hist_ids == nullptr))
        return set_error(KLS_ERR_INVALID_ARG, "history offsets and ids go together");
    if (n_vocab <= 0) return set_error(KLS_ERR_INVALID_ARG, "n_vocab must be positive");
    if (n_rows < 1) return set_error(KLS_ERR_INVALID_ARG, "n_rows must be positive");
    if (row_stride < n_vocab) return set_error(KLS_ERR_INVALID_ARG, "row_stride below n_vocab");
    const int k = (params->top_k > 0 && params->top_k < n_vocab) ? params->top_k : n_vocab;
    if (!greedy && k > KCAP)
        return set_error(KLS_ERR_UNSUPPORTED, "top-k above 64 (or no limit) needs a handle (kls_sample_batch)");
    if (n_rows > NA_MAX_ROWS) return set_error(KLS_ERR_RANGE, "n_rows above KLS_NOALLOC_MAX_ROWS");
    int seg_len = 0, segs = 0;
    choose_segments(n_vocab, n_rows, greedy, 0, DEFAULT_TARGET_WG, DEFAULT_WIDE_TARGET_WG, &seg_len, &segs);
    if ((long long) n_rows * ((n_vocab + 32767) / 32768) <= NA_MAX_ITEMS)
        fit_segments(greedy, d_logits, row_stride, n_vocab, &seg_len, &segs);
    if ((long long) n_rows * segs > NA_MAX_ITEMS)
        return set_error(KLS_ERR_RANGE, "rows x segments above KLS_NOALLOC_MAX_WORKGROUPS");
    void* base = nullptr;
    if (hipError_t e = device_scratch(&base)) return set_error(KLS_ERR_HIP, "device scratch", e);
    unsigned char* b = static_cast<unsigned char*>(base);
    hipStream_t s = (hipStream_t) stream;

    RowsArgs a{};
    a.logits = d_logits;
    a.row_stride = row_stride;
    a.V = n_vocab;
    a.n_rows = n_rows;
    a.seg_len = seg_len;
    a.segs = segs;
    a.xcd_map = 1;
    a.p = sampling_params(*params, k);
    const bool pen = (params->presence_penalty != 0.0f || params->frequency_penalty != 0.0f ||
                      params->repetition_penalty != 1.0f) && d_hist_off != nullptr;
    if (pen) {
        a.hist_ids = d_hist_ids;
        a.hist_off = d_hist_off;
    }
    a.u = d_u;
    a.seg_cand = reinterpret_cast<uint64_t*>(b);
    a.row_ticket = reinterpret_cast<uint32_t*>(b + TICKET_OFF);
    a.row_thr = reinterpret_cast<uint64_t*>(b + THR_OFF);
    a.share_bounds = (long long) n_rows * segs > DEFAULT_SHARE_MIN_WG ? 1 : 0;
    a.out_tokens = d_out_tokens;
    a.spin_limit = DEFAULT_SPIN_LIMIT;
    hipLaunchKernelGGL(clear_rows_kernel, dim3((unsigned) ((n_rows + 255) / 256)), dim3(256), 0, s, a.row_ticket,
                       a.row_thr, n_rows);
    if (hipError_t e = hipGetLastError()) return set_error(KLS_ERR_HIP, "clear_rows_kernel", e);
    if (hipError_t e = launch_rows(a, greedy, pen, s)) return set_error(KLS_ERR_HIP, "launch_rows", e);
    return KLS_OK;
}

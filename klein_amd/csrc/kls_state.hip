// The verify step's consumer on the device: the DeltaNet recurrent-state rollback of klein's decode loop
// (src/engine.cpp:578-583: rejected = (nb - 1) - accepted; State::rollback_recurrent(gpu, rejected),
// src/state.cpp:162-184), driven by the accepted count the verify kernel leaves in device memory, so the step
// needs no host round trip before the next forward pass is enqueued.
//
// State layout (src/state.h:45-46, src/state.cpp:68-76), per recurrent layer:
//   conv     [conv_row f32] x n_snapshots slots: slot 0 the current state, slot s the state s tokens back;
//   ssm      [ssm_row f32]: the current state;
//   ssm_snap [ssm_row snap_type] x (n_snapshots - 1) rows: row s - 1 the state s tokens back.
// Rolling back s tokens copies conv slot s over slot 0 and converts snapshot row s - 1 into ssm (ggml_cpy from
// f16 / bf16 / f32 to f32: exact). One launch covers every layer: a 2-D grid of (unit block, layer), each thread
// moving 4 elements with a non-temporal load and a 16-byte store (the state is streamed once). Measured on
// MI355X at a 27B-class layout (238 MB moved): 40 us, 0.74 of the HBM peak; eight-element units with four units
// per thread reached 82 us (a wave's stores then cover every other 16 bytes of a line).
#include <hip/hip_runtime.h>

#include <cstring>
#include <vector>

#include "klein_sampler.h"
#include "kls_internal.h"

struct kls_recurrent {
    int device = 0;
    int n_layers = 0, n_snapshots = 0;
    int64_t conv_row = 0, ssm_row = 0, conv_stride = 0, snap_stride = 0;
    int snap_type = KLS_SNAP_F32;
    bool vec = false;              // every pointer, stride and row allows the 4-element path
    void** d_ptrs = nullptr;       // device: conv[n_layers], ssm[n_layers], ssm_snap[n_layers]
};

namespace kls {
namespace {

struct RollbackArgs {
    float* const* conv;
    float* const* ssm;
    const void* const* snap;
    const int32_t* accepted;
    int32_t nb;
    int64_t conv_row, ssm_row;
    int64_t conv_stride_f;   // floats between conv slots
    int64_t snap_stride_e;   // elements between snapshot rows
};

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// f16 -> f32, exact (every binary16 value is a binary32 value): the hardware conversion.
__device__ __forceinline__ float h2f(uint32_t h) { return (float) __builtin_bit_cast(_Float16, (uint16_t) h); }
// bf16 -> f32, exact: the bf16 bits are the high half of the f32 bits.
__device__ __forceinline__ float b2f(uint32_t b) { return __uint_as_float(b << 16); }

template <int SNAP>
__device__ __forceinline__ float snap_elem(const void* p, int64_t i) {
    if constexpr (SNAP == KLS_SNAP_F32) return static_cast<const float*>(p)[i];
    else if constexpr (SNAP == KLS_SNAP_F16) return h2f(static_cast<const uint16_t*>(p)[i]);
    else return b2f(static_cast<const uint16_t*>(p)[i]);
}

// grid.y = layer, grid.x * blockDim.x threads stride over the layer's units: conv units [0, cu) then ssm units.
// VEC: a unit is 4 elements (rows are multiples of 4 and every address is 16-byte aligned), so each store
// instruction of a wave writes 1 KB of consecutive f32 (whole cache lines); else 1 element.
template <int SNAP, bool VEC>
__global__ __launch_bounds__(256) void rollback_kernel(RollbackArgs a) {
    // engine.cpp:578: rejected = (nb - 1) - accepted (clamped: a value outside [0, nb - 1] moves nothing out of
    // bounds); state.cpp:163: nothing to do for s <= 0
    const int acc = *a.accepted;
    const int s = (acc >= 0 && acc < a.nb) ? (a.nb - 1) - acc : 0;
    if (s <= 0) return;
    const int layer = (int) blockIdx.y;
    constexpr int U = VEC ? 4 : 1;
    const int64_t cu = a.conv_row / U, su = a.ssm_row / U;
    float* const conv = a.conv[layer];
    float* const ssm = a.ssm[layer];
    const void* const snap = a.snap[layer];
    const float* const csrc = conv + (int64_t) s * a.conv_stride_f;  // state.cpp:177: conv slot s -> slot 0
    const int64_t sbase = (int64_t) (s - 1) * a.snap_stride_e;        // state.cpp:178: snapshot row s - 1 -> ssm
    const int64_t stride = (int64_t) gridDim.x * blockDim.x;
    for (int64_t u = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; u < cu + su; u += stride) {
        if (u < cu) {
            if constexpr (VEC) {
                const f32x4 x = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(csrc + 4 * u));
                *reinterpret_cast<f32x4*>(conv + 4 * u) = x;
            } else {
                conv[u] = csrc[u];
            }
        } else {
            const int64_t i = u - cu;
            if constexpr (VEC) {
                f32x4 y;
                if constexpr (SNAP == KLS_SNAP_F32) {
                    y = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(static_cast<const float*>(snap) + sbase + 4 * i));
                } else {
                    const u32x2 q = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(snap) + sbase + 4 * i));
                    if constexpr (SNAP == KLS_SNAP_F16)
                        y = f32x4{h2f(q[0] & 0xffffu), h2f(q[0] >> 16), h2f(q[1] & 0xffffu), h2f(q[1] >> 16)};
                    else
                        y = f32x4{b2f(q[0] & 0xffffu), b2f(q[0] >> 16), b2f(q[1] & 0xffffu), b2f(q[1] >> 16)};
                }
                *reinterpret_cast<f32x4*>(ssm + 4 * i) = y;
            } else {
                ssm[i] = snap_elem<SNAP>(snap, sbase + i);
            }
        }
    }
}

template <int SNAP>
hipError_t launch_snap(const RollbackArgs& a, bool vec, int n_layers, hipStream_t s) {
    const int64_t units = vec ? (a.conv_row + a.ssm_row) / 4 : a.conv_row + a.ssm_row;
    // one unit per thread (every load of the layer in flight at once), at most 65535 workgroups per layer; the
    // grid-stride loop covers larger layers
    const int64_t want = (units + 255) / 256;
    const unsigned gx = (unsigned) (want < 1 ? 1 : want > 65535 ? 65535 : want);
    const dim3 grid(gx, (unsigned) n_layers);
    if (vec)
        hipLaunchKernelGGL((rollback_kernel<SNAP, true>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((rollback_kernel<SNAP, false>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace kls

using namespace kls;

extern "C" {

int kls_recurrent_create(const kls_recurrent_desc* d, kls_recurrent_handle* out) {
    if (!d || !out) return set_error(KLS_ERR_INVALID_ARG, "null argument");
    *out = nullptr;
    if (d->n_layers < 1 || d->n_layers > 65535) return set_error(KLS_ERR_INVALID_ARG, "n_layers outside [1, 65535]");
    if (d->n_snapshots < 1) return set_error(KLS_ERR_INVALID_ARG, "n_snapshots must be positive");
    if (d->conv_row < 0 || d->ssm_row < 0) return set_error(KLS_ERR_INVALID_ARG, "negative row length");
    if (d->snap_type != KLS_SNAP_F32 && d->snap_type != KLS_SNAP_F16 && d->snap_type != KLS_SNAP_BF16)
        return set_error(KLS_ERR_INVALID_ARG, "unknown snapshot type");
    const int64_t esz = d->snap_type == KLS_SNAP_F32 ? 4 : 2;
    if (d->conv_stride < d->conv_row * 4 || d->conv_stride % 4 != 0)
        return set_error(KLS_ERR_INVALID_ARG, "conv_stride below the row or not a multiple of 4 bytes");
    if (d->n_snapshots > 1 && (d->snap_stride < d->ssm_row * esz || d->snap_stride % esz != 0))
        return set_error(KLS_ERR_INVALID_ARG, "snap_stride below the row or not a multiple of the element size");
    if (!d->conv || !d->ssm || (d->n_snapshots > 1 && !d->ssm_snap))
        return set_error(KLS_ERR_INVALID_ARG, "null pointer table");
    bool vec = d->conv_row % 4 == 0 && d->ssm_row % 4 == 0 && d->conv_stride % 16 == 0 &&
               (d->n_snapshots <= 1 || d->snap_stride % 16 == 0);
    std::vector<void*> tab(3 * (size_t) d->n_layers, nullptr);
    for (int l = 0; l < d->n_layers; ++l) {
        if (!d->conv[l] || !d->ssm[l] || (d->n_snapshots > 1 && !d->ssm_snap[l]))
            return set_error(KLS_ERR_INVALID_ARG, "null layer pointer");
        tab[l] = d->conv[l];
        tab[d->n_layers + l] = d->ssm[l];
        tab[2 * d->n_layers + l] = d->n_snapshots > 1 ? const_cast<void*>(d->ssm_snap[l]) : nullptr;
        vec = vec && aligned16(d->conv[l]) && aligned16(d->ssm[l]) && (d->n_snapshots <= 1 || aligned16(d->ssm_snap[l]));
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
        (void) hipGetLastError();
        return set_error(KLS_ERR_NO_DEVICE, "no GPU visible");
    }
    kls_recurrent* r = new kls_recurrent();
    (void) hipGetDevice(&r->device);
    r->n_layers = d->n_layers;
    r->n_snapshots = d->n_snapshots;
    r->conv_row = d->conv_row;
    r->ssm_row = d->ssm_row;
    r->conv_stride = d->conv_stride;
    r->snap_stride = d->snap_stride;
    r->snap_type = d->snap_type;
    r->vec = vec;
    hipError_t e = hipMalloc((void**) &r->d_ptrs, sizeof(void*) * tab.size());
    if (e != hipSuccess) {
        delete r;
        return set_error(KLS_ERR_OOM, "pointer table", e);
    }
    if ((e = hipMemcpy(r->d_ptrs, tab.data(), sizeof(void*) * tab.size(), hipMemcpyHostToDevice)) != hipSuccess) {
        (void) hipFree(r->d_ptrs);
        delete r;
        return set_error(KLS_ERR_HIP, "pointer table upload", e);
    }
    *out = r;
    return KLS_OK;
}

int kls_recurrent_destroy(kls_recurrent_handle r) {
    if (!r) return set_error(KLS_ERR_INVALID_ARG, "null handle");
    (void) hipSetDevice(r->device);
    (void) hipDeviceSynchronize();
    if (r->d_ptrs) (void) hipFree(r->d_ptrs);
    delete r;
    return KLS_OK;
}

int kls_rollback_recurrent(kls_recurrent_handle r, const int32_t* d_accepted, int nb, kls_stream stream) {
    if (!r) return set_error(KLS_ERR_INVALID_ARG, "null handle");
    if (!d_accepted) return set_error(KLS_ERR_INVALID_ARG, "null accepted count");
    if (nb < 1) return set_error(KLS_ERR_INVALID_ARG, "nb must be at least 1");
    // state.cpp:164: the rollback depth (at most nb - 1) must have a snapshot slot
    if (nb > r->n_snapshots) return set_error(KLS_ERR_RANGE, "nb above the state's snapshot slots");
    if (nb == 1) return KLS_OK;  // nothing can be rejected
    (void) hipSetDevice(r->device);
    RollbackArgs a{};
    a.conv = reinterpret_cast<float* const*>(r->d_ptrs);
    a.ssm = reinterpret_cast<float* const*>(r->d_ptrs + r->n_layers);
    a.snap = reinterpret_cast<const void* const*>(r->d_ptrs + 2 * r->n_layers);
    a.accepted = d_accepted;
    a.nb = nb;
    a.conv_row = r->conv_row;
    a.ssm_row = r->ssm_row;
    a.conv_stride_f = r->conv_stride / 4;
    a.snap_stride_e = r->snap_stride / (r->snap_type == KLS_SNAP_F32 ? 4 : 2);
    hipStream_t s = (hipStream_t) stream;
    hipError_t e;
    switch (r->snap_type) {
        case KLS_SNAP_F32: e = launch_snap<KLS_SNAP_F32>(a, r->vec, r->n_layers, s); break;
        case KLS_SNAP_F16: e = launch_snap<KLS_SNAP_F16>(a, r->vec, r->n_layers, s); break;
        default: e = launch_snap<KLS_SNAP_BF16>(a, r->vec, r->n_layers, s); break;
    }
    if (e != hipSuccess) return set_error(KLS_ERR_HIP, "rollback_kernel", e);
    return KLS_OK;
}

}  // extern "C"

"""ctypes bindings of the C ABI (include/klein_sampler.h) in klein_amd/lib/libklein_sampler.so.

The library is the only compute path: loading fails loudly when it is missing, and nothing falls back to a CPU
implementation."""
from __future__ import annotations

import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libklein_sampler.so")

KLS_OK = 0
KLS_ERR_INVALID_ARG = 1
KLS_ERR_RANGE = 2
KLS_ERR_UNSUPPORTED = 3
KLS_ERR_HIP = 4
KLS_ERR_NO_DEVICE = 5
KLS_ERR_OOM = 6

# every entry point include/klein_sampler.h declares
EXPORTS = ["kls_create", "kls_destroy", "kls_reset", "kls_accept", "kls_sample", "kls_verify", "kls_verify_enqueue",
           "kls_verify_wait", "kls_sample_batch", "kls_sample_batch_noalloc", "kls_argmax", "kls_ppl_scores",
           "kls_device_results", "kls_check", "kls_recurrent_create", "kls_recurrent_destroy",
           "kls_rollback_recurrent", "kls_get_candidates", "kls_debug_set_layout", "kls_debug_time_verify",
           "kls_debug_run_verify_steps", "kls_debug_path", "kls_debug_expf",
           "kls_debug_sum_replay", "kls_status_string", "kls_last_error"]


class KlsParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float), ("min_p", C.c_float),
                ("presence_penalty", C.c_float), ("frequency_penalty", C.c_float),
                ("repetition_penalty", C.c_float), ("seed", C.c_uint64)]


class KlsDebugLayout(C.Structure):
    _fields_ = [("seg_len", C.c_int32), ("target_wg", C.c_int32), ("wide_target_wg", C.c_int32),
                ("share_min_wg", C.c_int32), ("xcd_map", C.c_int32), ("wait_limit", C.c_int32),
                ("wide_segs", C.c_int32)]


class KlsRecurrentDesc(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("n_snapshots", C.c_int32), ("conv_row", C.c_int64),
                ("ssm_row", C.c_int64), ("conv_stride", C.c_int64), ("snap_stride", C.c_int64),
                ("snap_type", C.c_int32), ("conv", C.POINTER(C.c_void_p)), ("ssm", C.POINTER(C.c_void_p)),
                ("ssm_snap", C.POINTER(C.c_void_p))]


KLS_SNAP_F32, KLS_SNAP_F16, KLS_SNAP_BF16 = 0, 1, 2
KLS_PATH_FAST, KLS_PATH_MID, KLS_PATH_WIDE = 0, 1, 2


class KlsError(RuntimeError):
    def __init__(self, status: int, where: str, detail: str):
        super().__init__(f"{where}: {status_string(status)} ({detail})")
        self.status = status


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python klein_amd/build.py` "
                               "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        P, I32P, F32P, F64P = C.c_void_p, C.POINTER(C.c_int32), C.POINTER(C.c_float), C.POINTER(C.c_double)
        L.kls_create.argtypes = [C.POINTER(KlsParams), C.c_int, C.c_int, C.POINTER(C.c_void_p)]
        L.kls_destroy.argtypes = [P]
        L.kls_reset.argtypes = [P]
        L.kls_accept.argtypes = [P, C.c_int32]
        L.kls_sample.argtypes = [P, C.c_void_p, C.c_int, C.c_double, I32P]
        L.kls_verify.argtypes = [P, C.c_void_p, C.c_int, I32P, F64P, I32P, I32P, C.c_void_p]
        L.kls_verify_enqueue.argtypes = [P, C.c_void_p, C.c_int, I32P, F64P, C.c_void_p]
        L.kls_verify_wait.argtypes = [P, I32P, I32P]
        L.kls_sample_batch.argtypes = [P, C.c_void_p, C.c_int, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_void_p, C.c_void_p]
        L.kls_sample_batch_noalloc.argtypes = [C.POINTER(KlsParams), C.c_int, C.c_void_p, C.c_int, C.c_int64,
                                               C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        L.kls_recurrent_create.argtypes = [C.POINTER(KlsRecurrentDesc), C.POINTER(C.c_void_p)]
        L.kls_recurrent_destroy.argtypes = [P]
        L.kls_rollback_recurrent.argtypes = [P, C.c_void_p, C.c_int, C.c_void_p]
        L.kls_argmax.argtypes = [P, C.c_void_p, C.c_int, C.c_int64, C.c_void_p, C.c_void_p]
        L.kls_ppl_scores.argtypes = [P, C.c_void_p, C.c_int, C.c_int64, C.c_void_p, C.c_void_p, C.c_int64,
                                     C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_void_p]
        L.kls_get_candidates.argtypes = [P, C.c_int, I32P, F32P, C.c_int, I32P, I32P]
        L.kls_device_results.argtypes = [P, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)]
        L.kls_check.argtypes = [P]
        L.kls_debug_set_layout.argtypes = [P, C.POINTER(KlsDebugLayout)]
        L.kls_debug_time_verify.argtypes = [P, C.c_int, C.c_int, C.c_void_p, C.POINTER(C.c_double)]
        L.kls_debug_run_verify_steps.argtypes = [P, C.c_void_p, C.c_int, C.c_int, I32P, C.POINTER(C.c_double), I32P,
                                                 I32P, C.POINTER(C.c_int64), C.c_void_p]
        L.kls_debug_path.argtypes = [P, C.POINTER(C.c_int32)]
        L.kls_debug_expf.argtypes = [C.c_uint32, C.c_longlong, C.c_void_p, C.c_void_p]
        L.kls_debug_sum_replay.argtypes = [C.c_void_p, C.c_int, C.c_double, C.c_int, C.c_double, C.c_void_p,
                                           C.c_void_p]
        L.kls_status_string.restype = C.c_char_p
        L.kls_status_string.argtypes = [C.c_int]
        L.kls_last_error.restype = C.c_char_p
        L.kls_last_error.argtypes = []
        for name in EXPORTS:
            f = getattr(L, name)
            if f.restype is None or f.restype is C.c_int:
                if name not in ("kls_status_string", "kls_last_error"):
                    f.restype = C.c_int
        _lib = L
    return _lib


def status_string(st: int) -> str:
    return lib().kls_status_string(st).decode()


def check(st: int, where: str):
    if st != KLS_OK:
        raise KlsError(st, where, lib().kls_last_error().decode())

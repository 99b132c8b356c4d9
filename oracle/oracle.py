"""ORACLE — test infrastructure only: ctypes bindings of the CPU restatement (liboracle.so) and of the reference
sampler compiled from its own sources (_ref/libklein_ref.so). Only tests/, the smoke check and the CPU-baseline
leg of bench.py import this module, as the checker; the product never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libklein_ref.so")

MODE_STDLIB = 0   # std::partial_sort with the reference's value-only comparator (its tie order)
MODE_TOTAL = 1    # value descending, id ascending (lower id wins ties)


class OrcParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int32), ("top_p", C.c_float), ("min_p", C.c_float),
                ("presence_penalty", C.c_float), ("frequency_penalty", C.c_float),
                ("repetition_penalty", C.c_float)]


class RefParams(C.Structure):
    _fields_ = OrcParams._fields_ + [("seed", C.c_uint64)]


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _ip(a):
    return a.ctypes.data_as(C.POINTER(C.c_int32))


def _dp(a):
    return a.ctypes.data_as(C.POINTER(C.c_double))


def build():
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} is not built (run `make -C oracle`)")
        L = C.CDLL(LIB)
        L.orc_sample.restype = C.c_int32
        L.orc_sample.argtypes = [C.POINTER(C.c_float), C.c_int, C.POINTER(OrcParams), C.POINTER(C.c_int32),
                                 C.c_double, C.c_int, C.POINTER(C.c_int32), C.POINTER(C.c_float), C.c_int,
                                 C.POINTER(C.c_int), C.POINTER(C.c_int)]
        L.orc_verify.restype = C.c_int
        L.orc_verify.argtypes = [C.POINTER(C.c_float), C.c_int, C.c_int, C.POINTER(C.c_int32), C.POINTER(OrcParams),
                                 C.POINTER(C.c_int32), C.POINTER(C.c_double), C.c_int, C.POINTER(C.c_int32)]
        L.orc_uniforms.restype = None
        L.orc_uniforms.argtypes = [C.c_uint64, C.c_uint64, C.c_int, C.POINTER(C.c_double)]
        L.orc_mt64_nth.restype = C.c_uint64
        L.orc_mt64_nth.argtypes = [C.c_uint64, C.c_uint64]
        L.orc_libm_expf.restype = C.c_float
        L.orc_libm_expf.argtypes = [C.c_float]
        L.orc_expf_glibc.restype = C.c_float
        L.orc_expf_glibc.argtypes = [C.c_float]
        L.orc_expf_check.restype = C.c_longlong
        L.orc_expf_check.argtypes = [C.c_uint32, C.c_uint32, C.c_int]
        L.orc_expf_compare.restype = C.c_longlong
        L.orc_expf_compare.argtypes = [C.c_uint32, C.POINTER(C.c_float), C.c_longlong, C.c_int,
                                       C.POINTER(C.c_uint32)]
        L.orc_time_rows.restype = C.c_double
        L.orc_ppl_row.argtypes = [C.POINTER(C.c_float), C.c_int, C.c_int, C.POINTER(C.c_float),
                                  C.POINTER(C.c_double), C.POINTER(C.c_int32)]
        L.orc_argmax.argtypes = [C.POINTER(C.c_float), C.c_int]
        L.orc_argmax.restype = C.c_int32
        L.orc_time_rows.argtypes = [C.POINTER(C.c_float), C.c_int, C.c_int, C.POINTER(OrcParams),
                                    C.POINTER(C.c_int32), C.c_int, C.POINTER(C.c_int32)]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_LIB)


def ref():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"{REF_LIB} is not built (needs the reference sources)")
        L = C.CDLL(REF_LIB)
        L.ref_create.restype = C.c_void_p
        L.ref_create.argtypes = [C.POINTER(RefParams)]
        L.ref_destroy.argtypes = [C.c_void_p]
        L.ref_reset.argtypes = [C.c_void_p]
        L.ref_accept.argtypes = [C.c_void_p, C.c_int32]
        L.ref_sample.restype = C.c_int32
        L.ref_sample.argtypes = [C.c_void_p, C.POINTER(C.c_float), C.c_int]
        L.ref_verify.restype = C.c_int
        L.ref_verify.argtypes = [C.c_void_p, C.POINTER(C.c_float), C.c_int, C.c_int, C.POINTER(C.c_int32),
                                 C.POINTER(C.c_int32)]
        L.ref_time_rows.restype = C.c_double
        L.ref_time_rows.argtypes = [C.c_void_p, C.POINTER(C.c_float), C.c_int, C.c_int, C.c_int,
                                    C.POINTER(C.c_int32)]
        L.ref_time_rows_threads.restype = C.c_double
        L.ref_time_rows_threads.argtypes = [C.POINTER(C.c_void_p), C.POINTER(C.c_float), C.c_int, C.c_int, C.c_int,
                                            C.c_int]
        _ref = L
    return _ref


def params_struct(p) -> OrcParams:
    d = p if isinstance(p, dict) else p.as_dict()
    return OrcParams(d["temperature"], d["top_k"], d["top_p"], d["min_p"], d["presence_penalty"],
                     d["frequency_penalty"], d["repetition_penalty"])


def sample(logits_row: np.ndarray, p, u: float, counts: np.ndarray | None = None, mode: int = MODE_TOTAL,
           cap: int = 0):
    """One Sampler::sample (src/sampler.cpp:17-89) with injected uniform. Returns
    (token, topk_ids, topk_probs, n_kept); topk arrays hold min(k, cap) entries (cap 0 = k when k <= 4096)."""
    row = np.ascontiguousarray(logits_row, dtype=np.float32)
    V = row.shape[0]
    ps = params_struct(p)
    k = ps.top_k if 0 < ps.top_k < V else V
    if cap == 0:
        cap = min(k, 4096)
    ids = np.zeros(max(cap, 1), dtype=np.int32)
    probs = np.zeros(max(cap, 1), dtype=np.float32)
    cnt = None if counts is None else np.ascontiguousarray(counts, dtype=np.int32)
    nk, nkept = C.c_int(0), C.c_int(0)
    t = lib().orc_sample(_fp(row), V, C.byref(ps), None if cnt is None else _ip(cnt), float(u), mode, _ip(ids),
                         _fp(probs), cap, C.byref(nk), C.byref(nkept))
    n = min(nk.value, cap)
    return int(t), ids[:n].copy(), probs[:n].copy(), int(nkept.value)


def verify(logits: np.ndarray, drafts: np.ndarray, p, u: np.ndarray, counts: np.ndarray | None = None,
           mode: int = MODE_TOTAL):
    """The verify/accept loop of Engine::generate (src/engine.cpp:563-575). Returns (tokens, accepted, counts)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    nb, V = lg.shape
    dr = np.ascontiguousarray(drafts if drafts is not None else np.zeros(0), dtype=np.int32)
    if dr.shape[0] < max(nb - 1, 0):
        raise ValueError("need nb-1 drafts")
    uu = np.ascontiguousarray(u, dtype=np.float64)
    cnt = None if counts is None else np.ascontiguousarray(counts, dtype=np.int32).copy()
    toks = np.zeros(nb, dtype=np.int32)
    ps = params_struct(p)
    acc = lib().orc_verify(_fp(lg), V, nb, _ip(dr) if dr.size else None, C.byref(ps),
                           None if cnt is None else _ip(cnt), _dp(uu), mode, _ip(toks))
    return toks, int(acc), cnt


def ppl_row(logits_row: np.ndarray, target: int, base: np.ndarray | None = None) -> dict:
    """Per-token scoring of cmd_ppl (src/main.cpp:308-327): lse, nll, imax and, with base log-probabilities,
    kl, nll_base, ibase."""
    r = np.ascontiguousarray(logits_row, dtype=np.float32)
    b = None if base is None else np.ascontiguousarray(base, dtype=np.float32)
    out = np.zeros(4, dtype=np.float64)
    tops = np.zeros(2, dtype=np.int32)
    lib().orc_ppl_row(_fp(r), int(r.shape[0]), int(target), None if b is None else _fp(b), _dp(out), _ip(tops))
    d = dict(lse=float(out[0]), nll=float(out[1]), top=int(tops[0]))
    if b is not None:
        d.update(kl=float(out[2]), nll_base=float(out[3]), base_top=int(tops[1]))
    return d


def argmax(row: np.ndarray) -> int:
    """Engine::mtp_draft_token (src/engine.cpp:413-415): std::max_element's index over one row."""
    r = np.ascontiguousarray(row, dtype=np.float32)
    return int(lib().orc_argmax(_fp(r), int(r.shape[0])))


def uniforms(seed: int, n: int, skip: int = 0) -> np.ndarray:
    out = np.zeros(n, dtype=np.float64)
    lib().orc_uniforms(seed, skip, n, _dp(out))
    return out


class RefSampler:
    """The reference's own klein::Sampler (compiled from src/sampler.cpp) behind the shim."""

    def __init__(self, p):
        d = p if isinstance(p, dict) else p.as_dict()
        rp = RefParams(d["temperature"], d["top_k"], d["top_p"], d["min_p"], d["presence_penalty"],
                       d["frequency_penalty"], d["repetition_penalty"], d["seed"])
        self._L = ref()
        self._h = self._L.ref_create(C.byref(rp))

    def __del__(self):
        if getattr(self, "_h", None):
            self._L.ref_destroy(self._h)
            self._h = None

    def reset(self):
        self._L.ref_reset(self._h)

    def accept(self, t: int):
        self._L.ref_accept(self._h, int(t))

    def sample(self, row: np.ndarray) -> int:
        r = np.ascontiguousarray(row, dtype=np.float32)
        return int(self._L.ref_sample(self._h, _fp(r), r.shape[0]))

    def verify(self, logits: np.ndarray, drafts: np.ndarray):
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        nb, V = lg.shape
        dr = np.ascontiguousarray(drafts, dtype=np.int32)
        toks = np.zeros(nb, dtype=np.int32)
        acc = self._L.ref_verify(self._h, _fp(lg), V, nb, _ip(dr), _ip(toks))
        return toks, int(acc)


# ---- The verify step's consumer: the recurrent-state rollback (src/engine.cpp:578-583, src/state.cpp:162-184).

SNAP_F32, SNAP_F16, SNAP_BF16 = 0, 1, 2


def snap_to_f32(row: np.ndarray, snap_type: int) -> np.ndarray:
    """ggml_cpy of a snapshot row to f32 (src/state.cpp:178): f32 unchanged; f16 (uint16 bit patterns) through
    numpy's binary16 conversion; bf16 (uint16 bit patterns) as the high half of the f32 bits. All exact."""
    if snap_type == SNAP_F32:
        return np.array(row, dtype=np.float32)
    u = np.asarray(row, dtype=np.uint16)
    if snap_type == SNAP_F16:
        return u.view(np.float16).astype(np.float32)
    return (u.astype(np.uint32) << 16).view(np.float32)


def rollback_recurrent(conv: np.ndarray, ssm: np.ndarray, snap: np.ndarray | None, snap_type: int, accepted: int,
                       nb: int):
    """One layer of Engine::generate's rollback: rejected = (nb - 1) - accepted (src/engine.cpp:578), then
    State::rollback_recurrent(gpu, rejected) (src/state.cpp:162-184): nothing for s <= 0, else conv slot s over
    slot 0 (state.cpp:177) and snapshot row s - 1 converted into ssm (state.cpp:178). conv: [n_snapshots, conv_row]
    f32; ssm: [ssm_row] f32; snap: [n_snapshots - 1, ssm_row] (f32, or uint16 bits of f16 / bf16). Returns the new
    (conv, ssm) as copies."""
    conv = np.array(conv, dtype=np.float32, copy=True)
    ssm = np.array(ssm, dtype=np.float32, copy=True)
    s = (nb - 1) - accepted
    if s <= 0:
        return conv, ssm
    assert s < conv.shape[0], "state.cpp:164: s < n_snapshots"
    conv[0] = conv[s]
    ssm[:] = snap_to_f32(snap[s - 1], snap_type)
    return conv, ssm

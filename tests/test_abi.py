"""CPU checks of the C ABI library: it loads, exports every entry point include/klein_sampler.h declares, and
reports argument errors before touching a GPU. No compute call is made here."""
import ctypes as C
import os
import re

import pytest

from klein_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    syms = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            syms |= set(re.findall(r"^\s*(?:int|const char\*)\s+(kls_\w+)\s*\(", text, re.M))
    return syms


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    syms = declared_symbols()
    assert syms and syms == set(_lib.EXPORTS)
    for s in syms:
        assert hasattr(L, s), s


def test_status_strings():
    assert _lib.status_string(0) == "ok"
    assert _lib.status_string(_lib.KLS_ERR_RANGE) == "out of range"
    assert _lib.status_string(99) == "unknown status"


def _params(**kw):
    d = dict(temperature=1.0, top_k=20, top_p=0.95, min_p=0.0, presence_penalty=0.0, frequency_penalty=0.0,
             repetition_penalty=1.0, seed=0)
    d.update(kw)
    return _lib.KlsParams(*d.values())


def test_create_argument_errors():
    L = _lib.lib()
    h = C.c_void_p()
    assert L.kls_create(None, 100, 1, C.byref(h)) == _lib.KLS_ERR_INVALID_ARG
    p = _params()
    assert L.kls_create(C.byref(p), 0, 1, C.byref(h)) == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_create(C.byref(p), -5, 1, C.byref(h)) == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_create(C.byref(p), 100, 0, C.byref(h)) == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_create(C.byref(p), 100, 1, None) == _lib.KLS_ERR_INVALID_ARG
    assert b"n_vocab" in L.kls_last_error() or b"max_rows" in L.kls_last_error() or L.kls_last_error()


def test_null_handle_errors():
    L = _lib.lib()
    out = C.c_int32()
    assert L.kls_destroy(None) == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_reset(None) == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_accept(None, 3) == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_sample(None, None, 10, 0.5, C.byref(out)) == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_verify(None, None, 4, None, None, None, None, None) == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_sample_batch(None, None, 1, 10, None, None, None, None, None) == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_get_candidates(None, 0, None, None, 0, None, None) == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_debug_expf(0, 10, None, None) == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_debug_run_verify_steps(None, None, 4, 1, None, None, None, None, None, None) == \
        _lib.KLS_ERR_INVALID_ARG


def test_no_device_is_reported_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    L = _lib.lib()
    h = C.c_void_p()
    p = _params()
    assert L.kls_create(C.byref(p), 1000, 4, C.byref(h)) == _lib.KLS_ERR_NO_DEVICE


def test_noalloc_limits_reported_before_device_work():
    """kls_sample_batch_noalloc refuses what its static scratch cannot hold, before any HIP call (so also without a
    GPU): rows above KLS_NOALLOC_MAX_ROWS, rows x segments above KLS_NOALLOC_MAX_WORKGROUPS, top-k above 64."""
    L = _lib.lib()
    fake = C.c_void_p(0x1000)  # never dereferenced: the checks come first
    p = _params(top_k=20)
    args = lambda rows, V: (C.byref(p), V, fake, rows, V, None, None, fake, fake, None)  # noqa: E731
    assert L.kls_sample_batch_noalloc(*args(257, 248320)) == _lib.KLS_ERR_RANGE
    assert L.kls_sample_batch_noalloc(*args(256, 65536 * 5)) == _lib.KLS_ERR_RANGE
    pw = _params(top_k=65)
    assert L.kls_sample_batch_noalloc(C.byref(pw), 1000, fake, 1, 1000, None, None, fake, fake, None) == \
        _lib.KLS_ERR_UNSUPPORTED
    pn = _params(top_k=0)
    assert L.kls_sample_batch_noalloc(C.byref(pn), 1000, fake, 1, 1000, None, None, fake, fake, None) == \
        _lib.KLS_ERR_UNSUPPORTED
    assert L.kls_sample_batch_noalloc(None, 1000, fake, 1, 1000, None, None, fake, fake, None) == \
        _lib.KLS_ERR_INVALID_ARG
    assert L.kls_sample_batch_noalloc(C.byref(p), 1000, fake, 1, 999, None, None, fake, fake, None) == \
        _lib.KLS_ERR_INVALID_ARG


def test_recurrent_desc_errors_before_device_work():
    L = _lib.lib()
    h = C.c_void_p()
    P = C.c_void_p * 2
    arr = P(0x1000, 0x2000)
    ptr = C.cast(arr, C.POINTER(C.c_void_p))
    ok = dict(n_layers=2, n_snapshots=4, conv_row=64, ssm_row=128, conv_stride=256, snap_stride=256,
              snap_type=_lib.KLS_SNAP_F16, conv=ptr, ssm=ptr, ssm_snap=ptr)

    def make(**kw):
        d = dict(ok)
        d.update(kw)
        return _lib.KlsRecurrentDesc(*[d[f] for f, _ in _lib.KlsRecurrentDesc._fields_])

    assert L.kls_recurrent_create(None, C.byref(h)) == _lib.KLS_ERR_INVALID_ARG
    for bad in (dict(n_layers=0), dict(n_snapshots=0), dict(snap_type=7), dict(conv_stride=128),
                dict(snap_stride=100), dict(conv=None), dict(ssm_snap=None)):
        assert L.kls_recurrent_create(C.byref(make(**bad)), C.byref(h)) == _lib.KLS_ERR_INVALID_ARG, bad
    assert L.kls_rollback_recurrent(None, None, 4, None) == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_recurrent_destroy(None) == _lib.KLS_ERR_INVALID_ARG

"""Python mirror of klein::Sampler (src/sampler.h:25-38) over the gfx950 C ABI.

Same construction from SamplerParams, reset(), accept(token), sample(logits, n_vocab) and params(), with the
reference's draw stream (one mt19937_64 output per non-greedy sample), plus verify() for the engine's
verify/accept loop (src/engine.cpp:563-575) and sample_batch() for independent rows with their own histories.
Logits may be torch tensors on the GPU (read in place), or host arrays (copied to the device by the library).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .rng import MT19937_64, canonical
from .workloads import Params


def _ptr(x):
    """Address of a torch tensor or numpy array; keeps no copy."""
    if hasattr(x, "data_ptr"):
        return C.c_void_p(x.data_ptr())
    if isinstance(x, np.ndarray):
        if not x.flags["C_CONTIGUOUS"]:
            raise ValueError("logits must be C-contiguous")
        return C.c_void_p(x.ctypes.data)
    raise TypeError("expected a torch tensor or numpy array")


def _stream_ptr(stream):
    if stream is None:
        return None
    return C.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))


def _call_stream(stream, like):
    """The stream a device call runs on: `stream` if given; else, for torch tensor arguments, torch's current
    stream, so that the call is ordered with the torch work that makes and reads its buffers (as a torch op
    is); else NULL. (torch's default stream is the legacy default stream, handle 0: NULL then selects the
    library's stream, which is ordered with it.)"""
    if stream is not None:
        return _stream_ptr(stream)
    if hasattr(like, "data_ptr") and getattr(like, "is_cuda", False):
        import torch
        cs = torch.cuda.current_stream(like.device).cuda_stream
        return C.c_void_p(cs) if cs else None
    return None


class Sampler:
    """klein::Sampler. max_rows bounds verify()/sample_batch() rows."""

    def __init__(self, params: Params | None = None, n_vocab: int | None = None, max_rows: int = 16,
                 layout: dict | None = None, **kw):
        """layout: launch-layout overrides for tests (kls_debug_set_layout): seg_len, target_wg, wide_target_wg,
        share_min_wg, xcd_map. Results do not depend on them."""
        self._p = params if params is not None else Params(**kw)
        self._layout = dict(layout or {})
        import random
        self._rng = MT19937_64(self._p.seed if self._p.seed else random.SystemRandom().getrandbits(32))
        self._h = None
        self._n_vocab = None
        self._max_rows = max_rows
        self._early = []
        if n_vocab is not None:
            self._ensure(n_vocab)

    # -- lifetime
    def _ensure(self, n_vocab: int):
        if self._h is not None:
            if n_vocab != self._n_vocab:
                raise ValueError(f"n_vocab {n_vocab} differs from the sampler's {self._n_vocab}")
            return
        L = _lib.lib()
        p = self._p
        cp = _lib.KlsParams(p.temperature, p.top_k, p.top_p, p.min_p, p.presence_penalty, p.frequency_penalty,
                            p.repetition_penalty, p.seed)
        h = C.c_void_p()
        _lib.check(L.kls_create(C.byref(cp), int(n_vocab), int(self._max_rows), C.byref(h)), "kls_create")
        self._h = h
        self._n_vocab = int(n_vocab)
        if self._layout:
            self.set_layout(**self._layout)
        for t in self._early:
            _lib.check(L.kls_accept(self._h, int(t)), "kls_accept")
        self._early = []

    def set_layout(self, seg_len=0, target_wg=0, wide_target_wg=0, share_min_wg=0, xcd_map=-1, wait_limit=0,
                   wide_segs=0):
        """Test hook (kls_debug_set_layout): a field of 0 (xcd_map -1) keeps the default."""
        lay = _lib.KlsDebugLayout(int(seg_len), int(target_wg), int(wide_target_wg), int(share_min_wg), int(xcd_map),
                                  int(wait_limit), int(wide_segs))
        _lib.check(_lib.lib().kls_debug_set_layout(self._h, C.byref(lay)), "kls_debug_set_layout")

    def device_results(self):
        """(d_tokens, d_accepted) device addresses of the last verify step's results (kls_device_results)."""
        t, a = C.c_void_p(), C.c_void_p()
        _lib.check(_lib.lib().kls_device_results(self._h, C.byref(t), C.byref(a)), "kls_device_results")
        return t.value, a.value

    def check(self):
        """Raises if a kernel of this handle gave up an internal wait since the last check (kls_check)."""
        _lib.check(_lib.lib().kls_check(self._h), "kls_check")

    @property
    def path(self) -> str:
        """The kernel path of the handle's sampling calls: "fast", "mid" or "wide" (kls_debug_path)."""
        v = C.c_int32()
        _lib.check(_lib.lib().kls_debug_path(self._h, C.byref(v)), "kls_debug_path")
        return {_lib.KLS_PATH_FAST: "fast", _lib.KLS_PATH_MID: "mid", _lib.KLS_PATH_WIDE: "wide"}[v.value]

    def close(self):
        if self._h is not None:
            _lib.lib().kls_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- the reference interface
    def params(self) -> Params:
        return self._p

    def reset(self):
        self._early = []
        if self._h is not None:
            _lib.check(_lib.lib().kls_reset(self._h), "kls_reset")

    def accept(self, token: int):
        if self._h is None:
            self._early.append(int(token))
            return
        _lib.check(_lib.lib().kls_accept(self._h, int(token)), "kls_accept")

    def sample(self, logits, n_vocab: int | None = None, u: float | None = None) -> int:
        """One row. `u` overrides the draw (else the sampler's own mt19937_64 supplies it, as the reference)."""
        n = int(n_vocab if n_vocab is not None else logits.shape[-1])
        self._ensure(n)
        if u is None:
            u = canonical(self._rng) if self._p.temperature > 0 else 0.0
        out = C.c_int32()
        _lib.check(_lib.lib().kls_sample(self._h, _ptr(logits), n, float(u), C.byref(out)), "kls_sample")
        return int(out.value)

    # -- additions
    def verify(self, logits, drafts, u=None, stream=None):
        """The verify/accept loop: returns (tokens[0..accepted], accepted)."""
        nb, n = int(logits.shape[0]), int(logits.shape[1])
        self._ensure(n)
        dr = np.ascontiguousarray(np.asarray(drafts, dtype=np.int32).reshape(-1))
        if dr.shape[0] < nb - 1:
            raise ValueError("need nb-1 drafts")
        if u is None:
            if self._p.temperature > 0:
                peek = self._rng.copy()
                uu = np.array([canonical(peek) for _ in range(nb)], dtype=np.float64)
            else:
                uu = np.zeros(nb)
            consume = True
        else:
            uu = np.ascontiguousarray(u, dtype=np.float64)
            consume = False
        toks = np.zeros(nb, dtype=np.int32)
        acc = C.c_int32()
        if dr.size == 0:
            dr = np.zeros(1, dtype=np.int32)
        _lib.check(_lib.lib().kls_verify(self._h, _ptr(logits), nb, dr.ctypes.data_as(C.POINTER(C.c_int32)),
                                         uu.ctypes.data_as(C.POINTER(C.c_double)),
                                         toks.ctypes.data_as(C.POINTER(C.c_int32)), C.byref(acc),
                                         _call_stream(stream, logits)), "kls_verify")
        a = int(acc.value)
        if consume and self._p.temperature > 0:
            self._rng.discard(a + 1)
        return toks[:a + 1].copy(), a

    def sample_batch(self, logits, u, out_tokens, hist_off=None, hist_ids=None, stream=None):
        """Independent rows on the device (torch tensors): logits [rows, V] f32, u [rows] f64, out [rows] i32,
        optional CSR histories hist_off [rows+1] i32 / hist_ids i32. Asynchronous on `stream` (default: torch's
        current stream)."""
        rows, n = int(logits.shape[0]), int(logits.shape[1])
        self._ensure(n)
        stride = int(logits.stride(0)) if hasattr(logits, "stride") else n
        _lib.check(_lib.lib().kls_sample_batch(
            self._h, _ptr(logits), rows, stride, None if hist_off is None else _ptr(hist_off),
            None if hist_ids is None else _ptr(hist_ids), None if u is None else _ptr(u), _ptr(out_tokens),
            _call_stream(stream, out_tokens)), "kls_sample_batch")

    def argmax(self, logits, out, stream=None):
        """Engine::mtp_draft_token (src/engine.cpp:413-415) per row of the device tensor logits [rows, V] f32:
        std::max_element's index into out [rows] i32. Asynchronous on `stream`."""
        rows, n = int(logits.shape[0]), int(logits.shape[1])
        self._ensure(n)
        stride = int(logits.stride(0)) if hasattr(logits, "stride") else n
        _lib.check(_lib.lib().kls_argmax(self._h, _ptr(logits), rows, stride, _ptr(out), _call_stream(stream, out)),
                   "kls_argmax")

    def ppl_scores(self, logits, targets, base=None, stream=None):
        """cmd_ppl's per-token scores (src/main.cpp:308-327) for the device tensors logits [rows, V] f32 and
        targets [rows] i32, optionally base log-probabilities [rows, V] f32. Returns device tensors: lse, nll
        (f64), top (i32) and, with a base, kl, nll_base (f64) and base_top (i32). Asynchronous on `stream`."""
        import torch
        rows, n = int(logits.shape[0]), int(logits.shape[1])
        self._ensure(n)
        dev = logits.device
        out = dict(lse=torch.empty(rows, dtype=torch.float64, device=dev),
                   nll=torch.empty(rows, dtype=torch.float64, device=dev),
                   top=torch.empty(rows, dtype=torch.int32, device=dev))
        if base is not None:
            out.update(kl=torch.empty(rows, dtype=torch.float64, device=dev),
                       nll_base=torch.empty(rows, dtype=torch.float64, device=dev),
                       base_top=torch.empty(rows, dtype=torch.int32, device=dev))
        g = lambda k: _ptr(out[k]) if k in out else None
        _lib.check(_lib.lib().kls_ppl_scores(
            self._h, _ptr(logits), rows, int(logits.stride(0)), _ptr(targets),
            None if base is None else _ptr(base), int(base.stride(0)) if base is not None else 0,
            g("lse"), g("nll"), g("top"), g("kl"), g("nll_base"), g("base_top"), _call_stream(stream, logits)),
            "kls_ppl_scores")
        return out

    def candidates(self, row: int = 0, cap: int = 64):
        """(ids, probs, k, kept) of the last call's row: the sorted top-k and softmax probabilities."""
        ids = np.zeros(cap, dtype=np.int32)
        pr = np.zeros(cap, dtype=np.float32)
        nk, nkept = C.c_int32(), C.c_int32()
        _lib.check(_lib.lib().kls_get_candidates(self._h, int(row), ids.ctypes.data_as(C.POINTER(C.c_int32)),
                                                 pr.ctypes.data_as(C.POINTER(C.c_float)), cap, C.byref(nk),
                                                 C.byref(nkept)), "kls_get_candidates")
        n = min(int(nk.value), cap)
        return ids[:n].copy(), pr[:n].copy(), int(nk.value), int(nkept.value)


def debug_sum_replay(terms, acc0: float, mode: int = 0, thr: float = 0.0, stream=None):
    """The wide tail's exact replay of acc = acc + terms[i] (device float64 tensor), in order; mode 1 stops at
    acc >= thr, mode 2 at acc <= 0. Returns (result, stop index or -1)."""
    import torch
    out = torch.zeros(2, dtype=torch.float64, device=terms.device)
    _lib.check(_lib.lib().kls_debug_sum_replay(_ptr(terms), int(terms.numel()), float(acc0), int(mode), float(thr),
                                               _ptr(out), _call_stream(stream, out)), "kls_debug_sum_replay")
    r = out.cpu().numpy()
    return float(r[0]), int(r[1])


def debug_expf(lo_bits: int, out, stream=None):
    """Device expf of float bit patterns lo_bits .. lo_bits+len(out)-1 into the torch float32 tensor `out`."""
    _lib.check(_lib.lib().kls_debug_expf(int(lo_bits), int(out.numel()), _ptr(out), _call_stream(stream, out)),
               "kls_debug_expf")

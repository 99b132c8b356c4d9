"""kls_sample_batch_noalloc (the allocation-free batch entry point, scratch in a static device array) against
kls_sample_batch on the same inputs, bit for bit, on two calls in a row, the second smaller (fewer rows, a
smaller vocabulary, other parameters) so it runs over what the first left in the shared array; a few rows of
each are also checked against the oracle (src/sampler.cpp:17-89). Plus the size limits, reported before any
device work."""
import ctypes as C

import numpy as np
import pytest

from klein_amd import _lib
from klein_amd import workloads as W

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


def kparams(p):
    return _lib.KlsParams(p.temperature, p.top_k, p.top_p, p.min_p, p.presence_penalty, p.frequency_penalty,
                          p.repetition_penalty, p.seed)


def run_both(torch, K, x, hists, u, p):
    rows, V = x.shape
    d = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    du = torch.from_numpy(np.ascontiguousarray(u)).cuda()
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum([len(h) for h in hists])
    doff = torch.from_numpy(off).cuda()
    dids = torch.from_numpy(np.concatenate(hists).astype(np.int32) if off[-1] else np.zeros(1, np.int32)).cuda()
    S = K.Sampler(p, n_vocab=V, max_rows=rows)
    ref = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    S.sample_batch(d, du, ref, doff, dids)
    torch.cuda.synchronize()
    S.close()
    out = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
    cp = kparams(p)
    st = _lib.lib().kls_sample_batch_noalloc(C.byref(cp), V, C.c_void_p(d.data_ptr()), rows, V,
                                             C.c_void_p(doff.data_ptr()), C.c_void_p(dids.data_ptr()),
                                             C.c_void_p(du.data_ptr()), C.c_void_p(out.data_ptr()), None)
    _lib.check(st, "kls_sample_batch_noalloc")
    torch.cuda.synchronize()
    return ref.cpu().numpy(), out.cpu().numpy()


def test_noalloc_matches_handle_batch_twice(oracle_lib):
    import torch
    import klein_amd as K
    assert torch.cuda.is_available()
    O = oracle_lib
    # call 1: the 64-row batched workload (penalties over 16,384-id histories, top-k 64, top-p 0.9)
    w = W.batched()
    say("noalloc call 1: 64 x 248320")
    ref, got = run_both(torch, K, w.logits, w.histories, w.u, w.params)
    assert list(got) == list(ref)
    for r in (0, 17, 63):
        assert got[r] == O.sample(w.logits[r], w.params, w.u[r], W.counts_of(w.histories[r], w.vocab))[0]
    # call 2: smaller, over the same static array
    rng = np.random.default_rng(21)
    V, rows = 100000, 5
    x = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    hists = [rng.integers(0, V, 700).astype(np.int32) for _ in range(rows)]
    u = rng.random(rows)
    p = W.Params(temperature=0.7, top_k=20, top_p=0.8, presence_penalty=-0.3, repetition_penalty=0.9)
    say("noalloc call 2: 5 x 100000")
    ref, got = run_both(torch, K, x, hists, u, p)
    assert list(got) == list(ref)
    for r in range(rows):
        assert got[r] == O.sample(x[r], p, u[r], W.counts_of(hists[r], V))[0]

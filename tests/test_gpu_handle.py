"""GPU tests of the handle's own bookkeeping through the C ABI: the accept prefix formed on the device (and left in
device memory), the verify graph's key (the count-table width baked into a capture), calls refused while a step
is in flight, reset(), the launch layouts that only large grids or a test hook reach (bounds shared across
workgroups, plain workgroup order), the ordering of asynchronous calls on different streams, and the failure
path of the kernels' bounded internal waits (forced from the host with a zero poll limit). Tokens and accepted
counts are compared with the oracle (src/sampler.cpp:17-89, src/engine.cpp:563-575) bit for bit."""
import ctypes as C

import numpy as np
import pytest

from klein_amd import _lib
from klein_amd import workloads as W

pytestmark = pytest.mark.gpu

V = 248320


def say(*a):
    print("[case]", *a, flush=True)


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    torch.cuda.init()
    return torch


@pytest.fixture(scope="module")
def K():
    import klein_amd
    return klein_amd


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def read_device_i32(torch, ptr, n):
    """n int32 from a raw device address (hipMemcpy device -> host after a device synchronization)."""
    torch.cuda.synchronize()
    hip = C.CDLL("libamdhip64.so")
    out = np.zeros(n, np.int32)
    st = hip.hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), C.c_size_t(4 * n), C.c_int(2))
    assert st == 0
    return out


def oracle_drafts(O, x, p, u, counts, m, rng):
    """Drafts whose first m entries are the oracle's own tokens on the accepted path (so accepted >= m)."""
    drafts = rng.integers(0, x.shape[1], x.shape[0] - 1).astype(np.int32)
    c = None if counts is None else counts.copy()
    for i in range(m):
        drafts[i] = O.sample(x[i], p, u[i], c, O.MODE_TOTAL)[0]
        if c is not None:
            c[drafts[i]] += 1
    return drafts


def test_device_accept_prefix_and_results(torch_cuda, K, oracle_lib):
    """Every accepted count 0..nb-1 for nb = 1, 2, 4 and 16 rows; the device copy of accepted and tokens."""
    torch, O = torch_cuda, oracle_lib
    rng = np.random.default_rng(4)
    p = W.Params(temperature=0.6, top_k=20, top_p=0.95, seed=3)
    for nb in (1, 2, 4, 16):
        S = K.Sampler(p, n_vocab=V, max_rows=16)
        x, _ = W._head_rows(rng, nb, V)
        d = dev(torch, x)
        for m in sorted({min(v, nb - 1) for v in (0, 1, nb // 2, nb - 1)}):
            u = rng.random(nb)
            drafts = oracle_drafts(O, x, p, u, None, m, rng)
            say("nb", nb, "m", m)
            toks, acc = S.verify(d, drafts if nb > 1 else np.zeros(1, np.int32), u=u)
            ot, oa, _ = O.verify(x, drafts, p, u, None, O.MODE_TOTAL)
            assert acc == oa and acc >= m
            assert list(toks) == list(ot[:oa + 1])
            dt, da = S.device_results()
            assert read_device_i32(torch, da, 1)[0] == acc
            assert list(read_device_i32(torch, dt, acc + 1)) == list(ot[:oa + 1])
        S.close()


def test_step_loop_hook(torch_cuda, K, oracle_lib):
    """kls_debug_run_verify_steps (bench.py's timed loop): 12 verify steps with penalties run back to back from C,
    each step's history the tokens the earlier ones accepted; tokens and accepted counts against the oracle's chain
    of steps, and a wall time for every step."""
    torch, O = torch_cuda, oracle_lib
    rng = np.random.default_rng(21)
    p = W.Params(temperature=0.7, top_k=20, top_p=0.95, presence_penalty=0.4, frequency_penalty=0.1,
                 repetition_penalty=1.05, seed=9)
    nb, n = 4, 12
    x, _ = W._head_rows(rng, nb, V)
    d = dev(torch, x)
    counts = np.zeros(V, np.int32)
    drafts = np.zeros((n, nb - 1), np.int32)
    us = rng.random((n, nb))
    exp = []
    for i in range(n):
        drafts[i] = oracle_drafts(O, x, p, us[i], counts, i % nb, rng)
        ot, oa, counts = O.verify(x, drafts[i], p, us[i], counts, O.MODE_TOTAL)
        exp.append((oa, list(ot[:oa + 1])))
    S = K.Sampler(p, n_vocab=V)
    toks = np.zeros((n, nb), np.int32)
    acc = np.zeros(n, np.int32)
    ns = np.zeros(n, np.int64)
    I32P, F64P = C.POINTER(C.c_int32), C.POINTER(C.c_double)
    say("step loop", n)
    _lib.check(_lib.lib().kls_debug_run_verify_steps(
        S._h, C.c_void_p(d.data_ptr()), nb, n, np.ascontiguousarray(drafts).ctypes.data_as(I32P),
        np.ascontiguousarray(us).ctypes.data_as(F64P), toks.ctypes.data_as(I32P), acc.ctypes.data_as(I32P),
        ns.ctypes.data_as(C.POINTER(C.c_int64)), None), "kls_debug_run_verify_steps")
    for i in range(n):
        oa, ot = exp[i]
        assert acc[i] == oa and list(toks[i][:oa + 1]) == ot, i
        assert ns[i] > 0
    S.close()


def test_graph_recaptured_when_counts_widen(torch_cuda, K, oracle_lib):
    """A verify graph captured while the history's counts fit 16 bits must not be replayed once an id's count
    can reach 65536: the step after the widening upload matches the oracle (a stale 16-bit table would wrap the
    count of the repeated id and leave it nearly unpenalized)."""
    torch, O = torch_cuda, oracle_lib
    rng = np.random.default_rng(11)
    p = W.Params(temperature=0.6, top_k=20, top_p=0.95, presence_penalty=0.5, frequency_penalty=0.2,
                 repetition_penalty=1.1, seed=5)
    x, heads = W._head_rows(rng, 4, V)
    star = int(heads[0][0])
    x[:, star] = np.float32(30.0)  # the top logit of every row unless penalized
    d = dev(torch, x)
    S = K.Sampler(p, n_vocab=V)
    L = _lib.lib()
    counts = np.zeros(V, np.int32)
    for n in (65000, 560):  # 65000: counts fit the 16-bit table; 65560: they no longer do (wrapped: 24)
        for _ in range(n):
            st = L.kls_accept(S._h, star)
            if st:
                _lib.check(st, "kls_accept")
        counts[star] += n
        u = rng.random(4)
        drafts = rng.integers(0, V, 3).astype(np.int32)
        say("count", int(counts[star]))
        toks, acc = S.verify(d, drafts, u=u)
        ot, oa, counts = O.verify(x, drafts, p, u, counts, O.MODE_TOTAL)
        assert acc == oa and list(toks) == list(ot[:oa + 1]), int(counts[star])
        assert toks[0] != star
    S.close()


def test_second_enqueue_refused_without_side_effects(torch_cuda, K, oracle_lib):
    torch, O = torch_cuda, oracle_lib
    rng = np.random.default_rng(12)
    p = W.Params(temperature=0.7, top_k=20, top_p=0.9, seed=8)
    x, _ = W._head_rows(rng, 4, V)
    d = dev(torch, x)
    u = rng.random(4)
    drafts = oracle_drafts(O, x, p, u, None, 2, rng)
    S = K.Sampler(p, n_vocab=V)
    L = _lib.lib()
    I32, F64 = C.POINTER(C.c_int32), C.POINTER(C.c_double)
    dr = np.ascontiguousarray(drafts)
    uu = np.ascontiguousarray(u)
    say("enqueue")
    _lib.check(L.kls_verify_enqueue(S._h, C.c_void_p(d.data_ptr()), 4, dr.ctypes.data_as(I32),
                                    uu.ctypes.data_as(F64), None), "kls_verify_enqueue")
    other_d = np.array([1, 2, 3], np.int32)
    other_u = np.array([0.1, 0.2, 0.3, 0.4])
    st = L.kls_verify_enqueue(S._h, C.c_void_p(d.data_ptr()), 4, other_d.ctypes.data_as(I32),
                              other_u.ctypes.data_as(F64), None)
    assert st == _lib.KLS_ERR_INVALID_ARG
    assert L.kls_sample(S._h, C.c_void_p(d.data_ptr()), V, C.c_double(0.5), C.byref(C.c_int32())) == \
        _lib.KLS_ERR_INVALID_ARG
    assert L.kls_accept(S._h, 5) == _lib.KLS_ERR_INVALID_ARG
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    assert L.kls_argmax(S._h, C.c_void_p(d.data_ptr()), 1, V, C.c_void_p(out.data_ptr()), None) == \
        _lib.KLS_ERR_INVALID_ARG
    toks = np.zeros(4, np.int32)
    acc = C.c_int32()
    _lib.check(L.kls_verify_wait(S._h, toks.ctypes.data_as(I32), C.byref(acc)), "kls_verify_wait")
    ot, oa, _ = O.verify(x, drafts, p, u, None, O.MODE_TOTAL)
    assert acc.value == oa and list(toks[:oa + 1]) == list(ot[:oa + 1])
    S.close()


def test_reset_then_penalized_sampling(torch_cuda, K, oracle_lib):
    torch, O = torch_cuda, oracle_lib
    rng = np.random.default_rng(13)
    p = W.Params(temperature=1.0, top_k=40, top_p=0.95, min_p=0.05, presence_penalty=0.5, frequency_penalty=0.2,
                 repetition_penalty=1.1, seed=9)
    x, heads = W._head_rows(rng, 1, V)
    d = dev(torch, x[0])
    S = K.Sampler(p, n_vocab=V)
    hist = np.concatenate([np.repeat(heads[0][:10], 30), rng.integers(0, V, 500)]).astype(np.int32)
    for t in hist:
        S.accept(int(t))
    u = 0.37
    say("penalized before reset")
    assert S.sample(d, u=u) == O.sample(x[0], p, u, W.counts_of(hist, V), O.MODE_TOTAL)[0]
    S.reset()
    say("after reset")
    assert S.sample(d, u=u) == O.sample(x[0], p, u, np.zeros(V, np.int32), O.MODE_TOTAL)[0]
    hist2 = rng.integers(0, V, 300).astype(np.int32)
    for t in hist2:
        S.accept(int(t))
    say("new history after reset")
    assert S.sample(d, u=u) == O.sample(x[0], p, u, W.counts_of(hist2, V), O.MODE_TOTAL)[0]
    S.close()


@pytest.mark.parametrize("layout", [dict(share_min_wg=1), dict(xcd_map=0), dict(share_min_wg=1, xcd_map=0),
                                    dict(seg_len=1024, share_min_wg=1)])
def test_layouts_shared_bounds_and_plain_order(torch_cuda, K, oracle_lib, layout):
    """Batches and verify steps with per-row bounds shared through device memory (normally above 1,024
    workgroups) and with workgroups in plain order (no XCD dealing)."""
    torch, O = torch_cuda, oracle_lib
    rng = np.random.default_rng(14)
    rows = 6
    x, _ = W._head_rows(rng, rows, V)
    hists = [rng.integers(0, V, 2000).astype(np.int32) for _ in range(rows)]
    p = W.Params(temperature=1.0, top_k=64, top_p=0.9, presence_penalty=0.5, frequency_penalty=0.2,
                 repetition_penalty=1.1)
    S = K.Sampler(p, n_vocab=V, max_rows=rows, layout=layout)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum([len(h) for h in hists])
    u = rng.random(rows)
    out = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    say("batch", layout)
    S.sample_batch(dev(torch, x), dev(torch, u), out, dev(torch, off), dev(torch, np.concatenate(hists)))
    torch.cuda.synchronize()
    S.check()
    got = out.cpu().numpy()
    for r in range(rows):
        assert got[r] == O.sample(x[r], p, u[r], W.counts_of(hists[r], V), O.MODE_TOTAL)[0], (layout, r)
    S.close()
    pv = W.Params(temperature=0.6, top_k=20, top_p=0.95, presence_penalty=0.4, repetition_penalty=1.2, seed=2)
    S = K.Sampler(pv, n_vocab=V, layout=layout)
    h0 = rng.integers(0, V, 400).astype(np.int32)
    for t in h0:
        S.accept(int(t))
    counts = W.counts_of(h0, V)
    xv = x[:4].copy()
    dv = dev(torch, xv)
    for step in range(3):
        uv = rng.random(4)
        drafts = oracle_drafts(O, xv, pv, uv, counts, step, rng)
        say("verify", layout, step)
        toks, acc = S.verify(dv, drafts, u=uv)
        ot, oa, counts = O.verify(xv, drafts, pv, uv, counts, O.MODE_TOTAL)
        assert acc == oa and list(toks) == list(ot[:oa + 1]), (layout, step)
    S.close()


def test_async_calls_on_two_streams(torch_cuda, K, oracle_lib):
    """kls_sample_batch on one stream, then kls_argmax and kls_sample_batch on another, back to back on one handle:
    the later launches wait for the earlier ones (they share the handle's scratch)."""
    torch, O = torch_cuda, oracle_lib
    rng = np.random.default_rng(15)
    rows = 8
    x, _ = W._head_rows(rng, rows, V)
    d = dev(torch, x)
    p = W.Params(temperature=0.8, top_k=32, top_p=0.9)
    S = K.Sampler(p, n_vocab=V, max_rows=rows)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    u1, u2 = rng.random(rows), rng.random(rows)
    o1 = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    o2 = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    o3 = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    du1, du2 = dev(torch, u1), dev(torch, u2)
    torch.cuda.synchronize()
    for rep in range(5):
        say("two streams rep", rep)
        S.sample_batch(d, du1, o1, stream=sa)
        S.argmax(d, o2, stream=sb)
        S.sample_batch(d, du2, o3, stream=sb)
        torch.cuda.synchronize()
        S.check()
        assert list(o1.cpu().numpy()) == [O.sample(x[r], p, u1[r])[0] for r in range(rows)]
        assert list(o2.cpu().numpy()) == [O.argmax(x[r]) for r in range(rows)]
        assert list(o3.cpu().numpy()) == [O.sample(x[r], p, u2[r])[0] for r in range(rows)]
    S.close()


def test_internal_wait_failure_is_reported(torch_cuda, K, oracle_lib):
    """With a poll limit of zero (set from the host) the early-bound and count-table waits give up at once: the
    call must fail with KLS_ERR_HIP instead of returning tokens, report it once, add nothing to the history, and
    the handle works again with the default limit."""
    torch, O = torch_cuda, oracle_lib
    rng = np.random.default_rng(16)
    x, _ = W._head_rows(rng, 4, V)
    d = dev(torch, x)
    p = W.Params(temperature=0.6, top_k=20, top_p=0.95, presence_penalty=0.3, repetition_penalty=1.1, seed=4)
    S = K.Sampler(p, n_vocab=V, layout=dict(wait_limit=-1))
    hist = rng.integers(0, V, 100).astype(np.int32)
    for t in hist:
        S.accept(int(t))
    u = rng.random(4)
    drafts = oracle_drafts(O, x, p, u, W.counts_of(hist, V), 2, rng)
    say("forced give-up")
    with pytest.raises(_lib.KlsError) as ei:
        S.verify(d, drafts, u=u)
    assert ei.value.status == _lib.KLS_ERR_HIP
    S.check()  # reported once
    S.set_layout(wait_limit=0)
    say("default limit again")
    toks, acc = S.verify(d, drafts, u=u)
    ot, oa, _ = O.verify(x, drafts, p, u, W.counts_of(hist, V), O.MODE_TOTAL)
    assert acc == oa and list(toks) == list(ot[:oa + 1])
    S.close()

"""GPU parity of the mid top-k path (top_k 65..1024, src/sampler.cpp:42-51): one kernel that gathers every
segment's candidates above a bound into a per-row buffer, selects and sorts the row's top k in LDS and runs the
exact tail. Token ids, the first 64 candidates (ids and probabilities), the candidate count and the kept count
bit-exact against the oracle: ordinary rows at the largest and smallest k, vocabularies of one partial segment
to eight segments, penalties of both signs, exact ties (all-equal rows and bf16-valued rows, which force the
threshold bisection in the segments and in the row), infinities, and verify steps through the captured graph."""
import ctypes as C

import numpy as np
import pytest

from klein_amd import _lib
from klein_amd import workloads as W

pytestmark = pytest.mark.gpu


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


def head_rows(rng, rows, V, scale=1.5):
    x = (rng.standard_normal((rows, V)) * scale).astype(np.float32)
    for r in range(rows):
        heads = rng.choice(V, min(50, V), replace=False)
        x[r, heads] = (8 + 2 * rng.standard_normal(len(heads))).astype(np.float32)
        x[r, rng.choice(V, min(12, V), replace=False)] = np.float32(9.5)  # exact ties among the heads
    return x


def bf16_rows(rng, rows, V):
    """Logits rounded to bf16 (8 significant bits): thousands of exact ties around every rank."""
    x = (rng.standard_normal((rows, V)) * 2.0).astype(np.float32)
    return (x.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


def check_row(S, O, x, p, u, counts, r, label):
    t, oids, probs, kept = O.sample(x, p, float(u), counts, O.MODE_TOTAL, cap=64)
    gi, gp, gk, gkept = S.candidates(r)
    k_ref = p.top_k if 0 < p.top_k < x.shape[0] else x.shape[0]
    assert gk == k_ref, (label, r, gk, k_ref)
    assert list(gi) == list(oids), (label, r)
    assert gp.tobytes() == probs.tobytes(), (label, r)
    assert gkept == kept, (label, r, gkept, kept)
    return t


def run_batch(torch, K, O, x, p, u, hists=None, label=""):
    rows, V = x.shape
    S = K.Sampler(p, n_vocab=V, max_rows=rows)
    assert S.path == "mid", (label, S.path)
    out = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    if hists is not None:
        off = np.zeros(rows + 1, np.int32)
        off[1:] = np.cumsum([len(h) for h in hists])
        ids = np.concatenate(hists).astype(np.int32) if off[-1] else np.zeros(1, np.int32)
        S.sample_batch(dev(torch, x), dev(torch, u), out, dev(torch, off), dev(torch, ids))
    else:
        S.sample_batch(dev(torch, x), dev(torch, u), out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for r in range(rows):
        counts = W.counts_of(hists[r], V) if hists is not None else None
        t = check_row(S, O, x[r], p, u[r], counts, r, label)
        assert got[r] == t, (label, r, got[r], t)
    S.check()
    S.close()


# V, rows, k, temperature, top_p, min_p
ORDINARY = [
    (248320, 4, 65, 1.0, 0.95, 0.0),
    (248320, 4, 1024, 0.8, 1.0, 0.0),
    (248320, 2, 1000, 1.2, 0.9, 0.01),
    (70001, 3, 300, 1.0, 0.95, 0.0),      # three segments, the last partial
    (32768, 2, 777, 0.6, 0.99, 0.0),      # one whole segment
    (5000, 3, 1024, 2.0, 0.999, 0.0),     # one partial segment
    (100, 2, 0, 1.0, 1.0, 0.01),          # no limit on 100 ids: k = V = 100
]


@pytest.mark.parametrize("case", range(len(ORDINARY)))
def test_mid_ordinary_rows(torch_cuda, K, oracle_lib, case):
    V, rows, k, T, tp, mp = ORDINARY[case]
    rng = np.random.default_rng(1200 + case)
    x = head_rows(rng, rows, V)
    u = rng.random(rows)
    u[0] = 0.9999999
    p = W.Params(temperature=T, top_k=k, top_p=tp, min_p=mp)
    say("mid ordinary", case, "V", V, "k", k, "rows", rows)
    run_batch(torch_cuda, K, oracle_lib, x, p, u, label=f"ordinary{case}")


PENS = {
    1: dict(presence_penalty=0.5, frequency_penalty=0.2, repetition_penalty=1.1),
    2: dict(presence_penalty=-0.8, frequency_penalty=-0.1, repetition_penalty=0.7),
}


@pytest.mark.parametrize("pen", [1, 2])
def test_mid_penalties(torch_cuda, K, oracle_lib, pen):
    rng = np.random.default_rng(1300 + pen)
    V, rows, k = 248320, 3, 400
    x = head_rows(rng, rows, V)
    hists = []
    for r in range(rows):
        ranks = np.minimum(rng.zipf(1.1, 5000), V) - 1
        h = rng.permutation(V)[ranks].astype(np.int32)
        hists.append(np.concatenate([h, np.argsort(-x[r])[:600].astype(np.int32)]))  # heads through the penalties
    u = rng.random(rows)
    p = W.Params(temperature=0.9, top_k=k, top_p=0.95, min_p=0.0, **PENS[pen])
    say("mid penalties", pen)
    run_batch(torch_cuda, K, oracle_lib, x, p, u, hists, label=f"pen{pen}")


def test_mid_ties_and_infinities(torch_cuda, K, oracle_lib):
    """Rows whose segments and row buffer hold far more keys at the bound than the caps (bisection in both
    stages), bf16-valued rows, and rows of mostly -inf logits."""
    rng = np.random.default_rng(1400)
    V = 248320
    x = np.zeros((5, V), np.float32)                      # row 0: every logit equal
    x[1] = bf16_rows(rng, 1, V)[0]                        # row 1: bf16 values
    x[2] = -np.inf                                        # row 2: 700 finite logits, the rest -inf
    x[2, rng.choice(V, 700, replace=False)] = rng.standard_normal(700).astype(np.float32)
    x[3] = np.where(np.arange(V) % 5 == 0, np.float32(3.0), np.float32(1.0))  # two values, both tied in bulk
    x[4] = -np.inf                                        # row 4: every logit -inf but one
    x[4, 12345] = 0.0
    u = np.array([0.3, 0.77, 0.5, 0.999, 0.1])
    for k, tp in ((1000, 0.5), (130, 1.0)):
        p = W.Params(temperature=1.0, top_k=k, top_p=tp, min_p=0.0)
        say("mid ties, k", k)
        run_batch(torch_cuda, K, oracle_lib, x, p, u, label=f"ties{k}")


def test_mid_verify_steps_in_graph(torch_cuda, K, oracle_lib):
    """Verify steps with top-k 300 and penalties over the handle's history: the accepted prefix formed on the
    device, the step captured in one graph (kls_debug_time_verify replays it)."""
    O = oracle_lib
    torch = torch_cuda
    V = 248320
    rng = np.random.default_rng(1500)
    p = W.Params(temperature=0.7, top_k=300, top_p=0.9, min_p=0.0, presence_penalty=0.3, frequency_penalty=0.05,
                 repetition_penalty=1.05, seed=5)
    nb = 4
    S = K.Sampler(p, n_vocab=V, max_rows=nb)
    assert S.path == "mid"
    counts = np.zeros(V, np.int32)
    for t in rng.integers(0, V, 500):
        S.accept(int(t))
        counts[t] += 1
    x = dev(torch, head_rows(rng, nb, V))
    xh = x.cpu().numpy()
    for step in range(6):
        u = rng.random(nb)
        m = step % nb
        drafts = rng.integers(0, V, nb - 1).astype(np.int32)
        c = counts.copy()
        for i in range(m):
            drafts[i] = O.sample(xh[i], p, u[i], c, O.MODE_TOTAL)[0]
            c[drafts[i]] += 1
        say("mid verify", step, "m", m)
        toks, acc = S.verify(x, drafts, u=u)
        ot, oa, counts = O.verify(xh, drafts, p, u, counts, O.MODE_TOTAL)
        assert acc == oa and acc >= m and list(toks) == list(ot[:oa + 1]), (step, acc, oa)
    us = C.c_double()
    _lib.check(_lib.lib().kls_debug_time_verify(S._h, 2, 2, None, C.byref(us)), "kls_debug_time_verify")
    assert us.value > 0.0
    S.check()
    S.close()


def test_mid_paths_chosen(K):
    """Which path a handle takes: fast up to 64, mid up to 1024 where the buffers allow, wide beyond (no GPU
    work beyond the handle)."""
    for V, k, want in ((248320, 64, "fast"), (248320, 65, "mid"), (248320, 1024, "mid"), (248320, 1025, "wide"),
                       (248320, 0, "wide"), (1000, 0, "mid"), (600000, 1024, "wide"), (600000, 800, "mid")):
        S = K.Sampler(W.Params(temperature=1.0, top_k=k), n_vocab=V, max_rows=1)
        assert S.path == want, (V, k, S.path, want)
        S.close()

"""Randomized GPU parity sweep over every sampling path (src/sampler.cpp:17-89) through the batch entry point:
vocabularies from 1,000 to 248,320 ids, top-k from 1 to no limit (the fast, mid and wide paths), greedy and
temperatures 0.3 to 2.5, top-p and min-p on and off, penalties of both signs over Zipf histories, and rows of
normal, head-heavy, bf16-valued (ties) and partly -inf logits. Token ids bit-exact against the oracle, and for
sampled rows the candidate count, the first 64 candidates (ids and probabilities) and the kept count."""
import numpy as np
import pytest

from klein_amd import workloads as W

pytestmark = pytest.mark.gpu


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


PENS = [{}, dict(presence_penalty=0.5, frequency_penalty=0.2, repetition_penalty=1.1),
        dict(presence_penalty=-0.6, frequency_penalty=-0.1, repetition_penalty=0.8)]


def make_rows(rng, kind, rows, V):
    x = (rng.standard_normal((rows, V)) * rng.choice([0.5, 1.5, 3.0])).astype(np.float32)
    if kind == "heads":
        for r in range(rows):
            h = rng.choice(V, min(50, V), replace=False)
            x[r, h] = (8 + 2 * rng.standard_normal(len(h))).astype(np.float32)
    elif kind == "bf16":
        x = (x.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    elif kind == "ninf":
        x[rng.random((rows, V)) < 0.6] = -np.inf
    return x


@pytest.mark.parametrize("block", range(6))
def test_random_sweep(torch_cuda, K, oracle_lib, block):
    torch, O = torch_cuda, oracle_lib
    rng = np.random.default_rng(3100 + block)
    for case in range(20):
        V = int(rng.choice([1000, 4096, 5000, 32768, 70001, 248320]))
        k = int(rng.choice([0, 1, 2, 20, 64, 65, 130, 300, 1024, 1025, 3000, V // 2]))
        T = float(rng.choice([0.0, 0.3, 0.7, 1.0, 2.5]))
        tp = float(rng.choice([1.0, 0.99, 0.9, 0.5, 0.1]))
        mp = float(rng.choice([0.0, 0.0, 0.01, 0.1]))
        pen = int(rng.integers(3))
        rows = int(rng.choice([1, 2, 3]))
        kind = str(rng.choice(["normal", "heads", "bf16", "ninf"]))
        p = W.Params(temperature=T, top_k=k, top_p=tp, min_p=mp, **PENS[pen])
        label = f"block {block} case {case}: V {V} k {k} T {T} top_p {tp} min_p {mp} pen {pen} rows {rows} {kind}"
        print("[case]", label, flush=True)
        x = make_rows(rng, kind, rows, V)
        u = rng.random(rows)
        hists = []
        for _ in range(rows):
            n = int(rng.integers(0, 800)) if pen else 0
            ranks = np.minimum(rng.zipf(1.1, n), V) - 1
            hists.append(rng.permutation(V)[ranks].astype(np.int32))
        S = K.Sampler(p, n_vocab=V, max_rows=rows)
        out = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
        dx = torch.from_numpy(np.ascontiguousarray(x)).cuda()
        du = torch.from_numpy(u).cuda()
        if pen:
            off = np.zeros(rows + 1, np.int32)
            off[1:] = np.cumsum([len(h) for h in hists])
            ids = np.concatenate(hists).astype(np.int32) if off[-1] else np.zeros(1, np.int32)
            S.sample_batch(dx, du, out, torch.from_numpy(off).cuda(), torch.from_numpy(ids).cuda())
        else:
            S.sample_batch(dx, du, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        for r in range(rows):
            counts = W.counts_of(hists[r], V) if pen else None
            t, oids, probs, kept = O.sample(x[r], p, float(u[r]), counts, O.MODE_TOTAL, cap=64)
            assert got[r] == t, (label, r, got[r], t)
            if T > 0.0:
                gi, gp, gk, gkept = S.candidates(r)
                k_ref = k if 0 < k < V else V
                assert gk == k_ref or (kind == "ninf" and gk <= k_ref), (label, r, gk, k_ref)
                assert list(gi) == list(oids), (label, r)
                assert gp.tobytes() == probs.tobytes(), (label, r)
                assert gkept == kept, (label, r, gkept, kept)
        S.check()
        S.close()


@pytest.mark.parametrize("block", range(3))
def test_random_verify_sweep(torch_cuda, K, oracle_lib, block):
    """Verify steps (src/engine.cpp:563-575) over the handle's own history on every path: random nb, top-k,
    temperature, top-p, min-p and penalties; the first m drafts are the oracle's own tokens on the accepted path
    (so 0..nb-1 drafts are accepted); each step's tokens and accepted count against the oracle's chain."""
    torch, O = torch_cuda, oracle_lib
    rng = np.random.default_rng(3300 + block)
    for case in range(8):
        V = int(rng.choice([5000, 70001, 248320]))
        nb = int(rng.choice([1, 2, 4, 8]))
        k = int(rng.choice([1, 20, 64, 65, 300, 1024, 2000, 0]))
        T = float(rng.choice([0.0, 0.6, 1.0, 1.8]))
        tp = float(rng.choice([1.0, 0.95, 0.6]))
        mp = float(rng.choice([0.0, 0.05]))
        pen = int(rng.integers(3))
        p = W.Params(temperature=T, top_k=k, top_p=tp, min_p=mp, seed=int(rng.integers(1, 1000)), **PENS[pen])
        label = f"block {block} case {case}: V {V} nb {nb} k {k} T {T} top_p {tp} min_p {mp} pen {pen}"
        print("[case]", label, flush=True)
        x = make_rows(rng, str(rng.choice(["normal", "heads", "bf16"])), nb, V)
        d = torch.from_numpy(np.ascontiguousarray(x)).cuda()
        S = K.Sampler(p, n_vocab=V, max_rows=max(nb, 1))
        counts = np.zeros(V, np.int32)
        for t in rng.integers(0, V, int(rng.integers(0, 300))):
            S.accept(int(t))
            counts[t] += 1
        for step in range(3):
            u = rng.random(nb)
            m = int(rng.integers(0, nb))
            drafts = rng.integers(0, V, max(nb - 1, 1)).astype(np.int32)
            c = counts.copy()
            for i in range(min(m, nb - 1)):
                drafts[i] = O.sample(x[i], p, u[i], c if pen else None, O.MODE_TOTAL)[0]
                c[drafts[i]] += 1
            toks, acc = S.verify(d, drafts if nb > 1 else np.zeros(1, np.int32), u=u)
            ot, oa, counts = O.verify(x, drafts[:nb - 1] if nb > 1 else np.zeros(0, np.int32), p, u, counts,
                                      O.MODE_TOTAL)
            assert acc == oa and list(toks) == list(ot[:oa + 1]), (label, step, acc, oa)
        S.check()
        S.close()

"""GPU parity of every segment length the sampling kernel supports (256-thread workgroups over 1024..8192 ids,
1024-thread workgroups over 16384..65536 ids with 16-bit history counts), of the 32-bit fallback for histories
with 65536 or more ids in a row, and of verify steps wide enough to take the 1024-thread workgroups. Token ids
and candidate lists bit-exact against the oracle."""
import numpy as np
import pytest

from klein_amd import workloads as W

pytestmark = pytest.mark.gpu

SEG_LENS = (1024, 2048, 4096, 8192, 16384, 32768, 65536)


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


def head_rows(rng, rows, V):
    x = (rng.standard_normal((rows, V)) * 1.5).astype(np.float32)
    for r in range(rows):
        heads = rng.choice(V, min(50, V), replace=False)
        x[r, heads] = (8 + 2 * rng.standard_normal(len(heads))).astype(np.float32)
        if V > 100:
            x[r, rng.choice(V, 12, replace=False)] = np.float32(9.5)  # exact ties among the heads
    return x


def zipf_history(rng, V, n):
    if n == 0:
        return np.zeros(0, np.int32)
    ranks = np.minimum(rng.zipf(1.1, n), V) - 1
    perm = rng.permutation(V)
    return perm[ranks].astype(np.int32)


def check_batch(torch, K, O, x, p, hists, u, seg, label):
    rows, V = x.shape
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum([len(h) for h in hists])
    ids = np.concatenate(hists).astype(np.int32) if off[-1] else np.zeros(1, np.int32)
    S = K.Sampler(p, n_vocab=V, max_rows=rows, layout=dict(seg_len=seg) if seg else None)
    out = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    say(label, "seg", seg, "rows", rows, "V", V)
    S.sample_batch(dev(torch, x), dev(torch, u), out, dev(torch, off), dev(torch, ids))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    pen = p.presence_penalty != 0 or p.frequency_penalty != 0 or p.repetition_penalty != 1
    for r in range(rows):
        counts = W.counts_of(hists[r], V) if pen else None
        t, oids, probs, kept = O.sample(x[r], p, float(u[r]), counts, O.MODE_TOTAL)
        assert got[r] == t, (label, seg, r)
        if p.temperature > 0:
            gi, gp, gk, gkept = S.candidates(r)
            assert gk == len(oids), (label, seg, r)
            assert list(gi) == list(oids), (label, seg, r)
            assert gp.tobytes() == probs.tobytes(), (label, seg, r)
            assert gkept == kept, (label, seg, r)
    S.close()


BATCH_CASES = [
    # V, rows, temperature, top_k, penalties (0 none, 1 positive, 2 negative), history length
    (248320, 3, 1.0, 64, 1, 16384),
    (70001, 2, 0.7, 20, 2, 3000),
    (100000, 2, 0.0, 1, 1, 5000),
    (5000, 3, 1.0, 40, 0, 0),
    (131072, 2, 1.3, 7, 1, 0),
]


@pytest.mark.parametrize("seg", SEG_LENS)
def test_segment_lengths_batch(torch_cuda, K, oracle_lib, seg):
    torch = torch_cuda
    rng = np.random.default_rng(seg)
    for V, rows, T, k, pen, nh in BATCH_CASES:
        x = head_rows(rng, rows, V)
        pp = dict(temperature=T, top_k=k, top_p=0.9, min_p=0.0)
        if pen == 1:
            pp.update(presence_penalty=0.5, frequency_penalty=0.2, repetition_penalty=1.1)
        elif pen == 2:
            pp.update(presence_penalty=-0.8, frequency_penalty=-0.1, repetition_penalty=0.7)
        p = W.Params(**pp)
        hists = [zipf_history(rng, V, int(rng.integers(nh // 2, nh + 1)) if nh else 0) for _ in range(rows)]
        if pen and V > 1000:
            for r in range(rows):  # push some heads through the penalties
                hists[r] = np.concatenate([hists[r], np.argsort(-x[r])[:30].astype(np.int32)])
        u = rng.random(rows)
        u[0] = 0.9999999
        check_batch(torch, K, oracle_lib, x, p, hists, u, seg, f"V{V} T{T} k{k} pen{pen}")


def test_greedy_batch_rows_not_whole_float4s(torch_cuda, K, oracle_lib):
    """64 greedy rows with penalties whose logits are not whole float4s (V = 248,319, contiguous rows): the
    default layout keeps such greedy launches to 32,768-id segments (the 65,536-id form of that kernel spills
    registers); tokens against the oracle with the default layout and with 65,536-id segments forced."""
    torch = torch_cuda
    rng = np.random.default_rng(31)
    V, rows = 248319, 64
    x = head_rows(rng, rows, V)
    p = W.Params(temperature=0.0, presence_penalty=0.5, frequency_penalty=0.2, repetition_penalty=1.1)
    hists = [np.concatenate([zipf_history(rng, V, 4000), np.argsort(-x[r])[:20].astype(np.int32)])
             for r in range(rows)]
    for seg in (0, 65536):
        check_batch(torch, K, oracle_lib, x, p, hists, np.zeros(rows), seg, "greedy rows not whole float4s")


@pytest.mark.parametrize("seg", (16384, 65536, 4096))
def test_history_counts_above_16_bits(torch_cuda, K, oracle_lib, seg):
    """A row whose history holds 70,000 ids, one id 66,000 times: 16-bit count tables would wrap, so the kernel
    stages 32-bit counts half a segment at a time."""
    torch = torch_cuda
    rng = np.random.default_rng(4242)
    V, rows = 248320, 3
    x = head_rows(rng, rows, V)
    top = np.argsort(-x[0])[:8]
    h0 = np.concatenate([np.full(66000, top[0], np.int32), zipf_history(rng, V, 3990),
                         np.array(top[1:], np.int32), np.full(2, top[3], np.int32)])
    rng.shuffle(h0)
    h1 = zipf_history(rng, V, 800)
    h2 = np.concatenate([np.full(65536, 7, np.int32), np.array([np.argsort(-x[2])[0]], np.int32)])
    for pp in (dict(presence_penalty=0.1, frequency_penalty=1e-5, repetition_penalty=1.05),
               dict(presence_penalty=-0.2, frequency_penalty=-2e-6, repetition_penalty=0.9)):
        p = W.Params(temperature=1.0, top_k=64, top_p=0.95, **pp)
        u = rng.random(rows)
        check_batch(torch, K, oracle_lib, x, p, [h0, h1, h2], u, seg, "wide counts")
    p = W.Params(temperature=0.0, presence_penalty=0.1, frequency_penalty=1e-4)
    check_batch(torch, K, oracle_lib, x, p, [h0, h1, h2], np.zeros(rows), seg, "wide counts greedy")


@pytest.mark.parametrize("wide", (False, True))
def test_verify_16_rows_penalized(torch_cuda, K, oracle_lib, wide):
    """Verify steps of 16 rows run on 1024-thread workgroups with the handle's bucketed history, the pending ids
    and the drafts counted on the device; with `wide` one id has been accepted 65,600 times (32-bit counts)."""
    torch = torch_cuda
    O = oracle_lib
    V, nb = 248320, 16
    rng = np.random.default_rng(1616 + wide)
    p = W.Params(temperature=0.9, top_k=30, top_p=0.9, presence_penalty=0.4, frequency_penalty=0.1 if not wide else 1e-5,
                 repetition_penalty=1.15, seed=5)
    S = K.Sampler(p, n_vocab=V, max_rows=nb)
    counts = np.zeros(V, np.int32)
    hist = list(rng.integers(0, V, 700))
    if wide:
        hist += [4321] * 65600
    for t in hist:
        S.accept(int(t))
        counts[t] += 1
    buf = torch.empty((nb, V), dtype=torch.float32, device="cuda")
    from klein_amd.rng import MT19937_64, canonical
    g = MT19937_64(5)
    accs = []
    for step in range(6):
        x = head_rows(rng, nb, V)
        if wide:
            x[:, 4321] = np.float32(12.0)
        gp = g.copy()
        u = np.array([canonical(gp) for _ in range(nb)])
        m = int(rng.integers(0, nb))
        drafts = rng.integers(0, V, nb - 1).astype(np.int32)
        c = counts.copy()
        for i in range(m):
            drafts[i] = O.sample(x[i], p, u[i], c, O.MODE_TOTAL)[0]
            c[drafts[i]] += 1
        buf.copy_(torch.from_numpy(x))
        say("verify16 wide", wide, "step", step, "m", m)
        toks, acc = S.verify(buf, drafts)
        ot, oa, counts = O.verify(x, drafts, p, u, counts, O.MODE_TOTAL)
        assert acc == oa and list(toks) == list(ot[:oa + 1]), step
        g.discard(acc + 1)
        accs.append(acc)
    S.close()


@pytest.mark.parametrize("seg", (16384, 32768, 65536))
def test_penalized_top_logits(torch_cuda, K, oracle_lib, seg):
    """Penalties that can only lower logits (applied lazily) on 1024-thread segments, where the history holds a
    row's largest raw logits: every lane maximum that forms the bound is a history id (row 0: the 2000 largest,
    row 1: every other one of the 4000 largest, row 2: the 40 largest among Zipf ids), under heavy presence /
    frequency or repetition penalties. Tokens and candidate lists bit-exact against the oracle."""
    torch = torch_cuda
    rng = np.random.default_rng(seg + 7)
    V, rows = 248320, 3
    x = head_rows(rng, rows, V)
    order = np.argsort(-x, axis=1, kind="stable")
    hists = [order[0, :2000].astype(np.int32),                                    # every top logit penalized
             order[1, : 4000 : 2].astype(np.int32),                               # every other one
             np.concatenate([order[2, :40], zipf_history(rng, V, 8000)]).astype(np.int32)]
    for pp in (dict(presence_penalty=10.0, frequency_penalty=5.0, repetition_penalty=1.0),
               dict(presence_penalty=0.5, frequency_penalty=0.2, repetition_penalty=4.0)):
        for k in (64, 20, 1):
            p = W.Params(temperature=1.0, top_k=k, top_p=0.9, **pp)
            u = rng.random(rows)
            check_batch(torch, K, oracle_lib, x, p, hists, u, seg, f"top penalized k{k} {pp}")

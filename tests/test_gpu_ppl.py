"""GPU parity of the perplexity / KL-divergence scores (kls_ppl_scores; klein's cmd_ppl loop, src/main.cpp:308-327)
against the oracle's restatement of that loop: indices exact, lse / nll / kl to rounding (the kernel sums in
another order; tolerances written below), on the loop's 64-row pass, small passes (other segment lengths),
strided rows, and NaN / infinity / out-of-range cases."""
import numpy as np
import pytest

from klein_amd import workloads as W

pytestmark = pytest.mark.gpu

LSE_RTOL = 1e-13  # lse and nll, relative to |lse|
KL_RTOL = 1e-12   # kl, relative to the sum of its terms' magnitudes


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


def base_logprobs(rng, rows, V):
    z = rng.standard_normal((rows, V)) * 3.0
    z -= z.max(1, keepdims=True)
    return (z - np.log(np.exp(z).sum(1, keepdims=True))).astype(np.float32)


def run(torch, K, x, targets, base=None, pitch=None, max_rows=None):
    rows, V = x.shape
    pitch = pitch or V
    lx = np.zeros((rows, pitch), np.float32)
    lx[:, :V] = x
    dl = torch.from_numpy(lx).cuda()
    db = None
    if base is not None:
        bx = np.zeros((rows, pitch), np.float32)
        bx[:, :V] = base
        db = torch.from_numpy(bx).cuda()
    dt = torch.from_numpy(np.asarray(targets, np.int32)).cuda()
    S = K.Sampler(W.Params(), n_vocab=V, max_rows=max_rows or rows)
    out = S.ppl_scores(dl[:, :V], dt, None if db is None else db[:, :V])
    torch.cuda.synchronize()
    S.close()
    return {k: v.cpu().numpy() for k, v in out.items()}


def check(O, x, targets, got, base=None, label=""):
    for r in range(x.shape[0]):
        e = O.ppl_row(x[r], int(targets[r]) if 0 <= targets[r] < x.shape[1] else 0,
                      None if base is None else base[r])
        assert got["top"][r] == e["top"], (label, r)
        if np.isnan(e["lse"]):
            assert np.isnan(got["lse"][r]), (label, r)
        else:
            tol = LSE_RTOL * abs(e["lse"]) + 1e-14
            assert abs(got["lse"][r] - e["lse"]) <= tol, (label, r, got["lse"][r], e["lse"])
            if 0 <= targets[r] < x.shape[1]:
                assert got["nll"][r] == e["nll"] or abs(got["nll"][r] - e["nll"]) <= tol, (label, r)
        if not 0 <= targets[r] < x.shape[1]:
            assert np.isnan(got["nll"][r]), (label, r)
        if base is not None:
            assert got["base_top"][r] == e["base_top"], (label, r)
            b = base[r].astype(np.float64)
            m = base[r] > -16.0
            mag = float(np.sum(np.abs(np.exp(b[m]) * (b[m] - (x[r].astype(np.float64)[m] - e["lse"])))))
            if not np.isfinite(e["kl"]):
                assert got["kl"][r] == e["kl"] or (np.isnan(got["kl"][r]) and np.isnan(e["kl"])), (label, r)
            else:
                assert abs(got["kl"][r] - e["kl"]) <= KL_RTOL * mag + 1e-15, (label, r, got["kl"][r], e["kl"])
            if 0 <= targets[r] < x.shape[1]:
                assert got["nll_base"][r] == e["nll_base"], (label, r)


def test_ppl_pass_64_rows_with_base(torch_cuda, K, oracle_lib):
    """The loop's default pass (--ppl-batch 64) over the full vocabulary, with a KL base."""
    rng = np.random.default_rng(31)
    rows, V = 64, W.VOCAB
    x = (rng.standard_normal((rows, V)) * 1.5).astype(np.float32)
    for r in range(rows):
        x[r, rng.choice(V, 50, replace=False)] = (8 + 2 * rng.standard_normal(50)).astype(np.float32)
    x[5, [10, 20000]] = x[5].max() + 1  # a tie for the top
    base = base_logprobs(rng, rows, V)
    targets = rng.integers(0, V, rows).astype(np.int32)
    say("ppl 64 x", V, "with base")
    got = run(torch_cuda, K, x, targets, base)
    check(oracle_lib, x, targets, got, base, "64 rows")
    assert got["top"][5] == 10


@pytest.mark.parametrize("rows", [1, 3, 16])
def test_small_passes_strided(torch_cuda, K, oracle_lib, rows):
    rng = np.random.default_rng(40 + rows)
    V = W.VOCAB
    x = (rng.standard_normal((rows, V)) * 2.0).astype(np.float32)
    base = base_logprobs(rng, rows, V)
    targets = rng.integers(0, V, rows).astype(np.int32)
    say("ppl small pass", rows, "strided")
    got = run(torch_cuda, K, x, targets, base, pitch=V + 7)
    check(oracle_lib, x, targets, got, base, f"{rows} rows")


def test_nan_infinity_and_targets(torch_cuda, K, oracle_lib):
    rng = np.random.default_rng(50)
    V = 30000
    x = rng.standard_normal((8, V)).astype(np.float32)
    x[0, 0] = np.nan                   # NaN first: lse NaN, top 0
    x[1, 777] = np.nan                 # NaN elsewhere: lse NaN, top the first largest number
    x[2, :] = -np.inf                  # all -inf: lse NaN
    x[3, 123] = np.inf                 # +inf maximum: lse NaN, top 123
    x[4, rng.choice(V, 100, replace=False)] = -np.inf  # -inf entries add nothing
    x[5, :] = np.float32(0.5)          # all equal: top 0, lse = 0.5 + log(V)
    x[6, 3] = -np.inf                  # target logit -inf: nll +inf
    base = base_logprobs(rng, 8, V)
    base[7, 0] = np.nan                # base NaN first: base top 0
    targets = rng.integers(0, V, 8).astype(np.int32)
    targets[6] = 3
    targets[7] = V + 5                 # out of range: NaN nll
    say("ppl NaN / inf / targets")
    got = run(torch_cuda, K, x, targets, base)
    check(oracle_lib, x, targets, got, base, "specials")
    assert got["top"][0] == 0 and got["top"][3] == 123 and np.isinf(got["nll"][6])
    assert got["base_top"][7] == 0


def test_without_base_and_small_vocab(torch_cuda, K, oracle_lib):
    rng = np.random.default_rng(60)
    for V in (1, 5, 4097, 100003):
        x = rng.integers(-4, 4, (4, V)).astype(np.float32)  # ties
        targets = rng.integers(0, V, 4).astype(np.int32)
        say("ppl without base, vocabulary", V)
        got = run(torch_cuda, K, x, targets, None)
        check(oracle_lib, x, targets, got, None, f"V={V}")

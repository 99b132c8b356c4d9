"""GPU checks of the wide top-k tail's exact parallel replay of sequential double sums (the reference's softmax
total, top-p cumulative sum and draw, src/sampler.cpp:58,70-77,84-87, accumulate one term at a time in double):
the result and the stop index must equal a plain in-order loop of IEEE double additions (Python floats), bit for
bit, on inputs built to hit every branch: round-to-even ties on every term, many binade crossings up and down,
stops, huge and tiny terms, zero / subnormal / negative starting values, NaN and infinity. Chains of more than
1,024 terms run with 8 terms per thread, shorter ones with one (both forms are checked)."""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)


@pytest.fixture(scope="module")
def torch_cuda():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    torch.cuda.init()
    return torch


def loop(t, acc, mode=0, thr=0.0):
    for i, x in enumerate(t.tolist()):
        acc = acc + x
        if (mode == 1 and acc >= thr) or (mode == 2 and acc <= 0.0):
            return acc, i
    return acc, -1


def same(a, b):
    return (math.isnan(a) and math.isnan(b)) or a == b and math.copysign(1, a) == math.copysign(1, b)


def check(torch, t, acc0, mode=0, thr=0.0, label=""):
    import klein_amd
    d = torch.from_numpy(np.ascontiguousarray(t, dtype=np.float64)).cuda()
    got = klein_amd.debug_sum_replay(d, acc0, mode, thr)
    exp = loop(np.asarray(t, np.float64), float(acc0), mode, thr)
    assert got[1] == exp[1] and same(got[0], exp[0]), (label, got, exp)


def test_softmax_like_terms(torch_cuda):
    rng = np.random.default_rng(1)
    x = np.sort(rng.uniform(0, 40, 120000))
    t = np.exp(-x).astype(np.float32).astype(np.float64)  # float terms, descending, most below 2^-29
    t[0] = 1.0
    say("softmax-like", t.size)
    check(torch_cuda, t, 0.0, 0, label="softmax")


def test_ties_on_every_term(torch_cuda):
    rng = np.random.default_rng(2)
    t = (2 * rng.integers(0, 1 << 20, 60000) + 1).astype(np.float64) * 2.0 ** -53  # exact half-ulps of [1, 2)
    say("ties")
    check(torch_cuda, t, 1.0, 0, label="ties at 1")
    check(torch_cuda, t * 2.0 ** 10, 1024.0 + 2.0 ** -42, 0, label="ties at 1024, odd start")


def test_crossings_up_and_stops(torch_cuda):
    rng = np.random.default_rng(3)
    t = rng.uniform(0, 10, 70000)
    say("binades up")
    check(torch_cuda, t, 0.0, 0, label="up")
    check(torch_cuda, t, 0.0, 1, 123456.789, label="stop at threshold")
    p = np.sort(rng.dirichlet(np.full(5000, 0.3)))[::-1].astype(np.float32).astype(np.float64)
    check(torch_cuda, p, 0.0, 1, 0.95, label="top-p")


def test_draw_down_to_zero(torch_cuda):
    rng = np.random.default_rng(4)
    p = np.sort(rng.dirichlet(np.full(200000, 0.05)))[::-1].astype(np.float32).astype(np.float64)
    for u in (0.0, 0.3, 0.999999):
        r0 = u * float(np.sum(p))
        say("draw", u)
        check(torch_cuda, -p, r0, 2, label=f"draw {u}")
    check(torch_cuda, -p, 1e-300, 2, label="draw from a tiny start")


def test_mixed_magnitudes_and_starts(torch_cuda):
    rng = np.random.default_rng(5)
    t = rng.standard_normal(30000) * 10.0 ** rng.uniform(-20, 5, 30000)
    say("mixed")
    for acc0 in (0.0, 1e-300, -5.0, 3.0, 5e-324):
        check(torch_cuda, t, acc0, 0, label=f"mixed from {acc0}")
    t2 = np.abs(t)
    check(torch_cuda, t2, 0.0, 0, label="positive mixed")
    check(torch_cuda, t2[::-1].copy(), 0.0, 0, label="positive ascending")


def test_specials(torch_cuda):
    say("specials")
    check(torch_cuda, np.zeros(0), 0.7, 0, label="empty")
    check(torch_cuda, np.array([0.25]), 0.0, 0, label="one")
    check(torch_cuda, np.zeros(3000), 1.5, 0, label="zeros")
    t = np.full(5000, 1e-3)
    t[2500] = np.nan
    check(torch_cuda, t, 0.0, 0, label="NaN term")
    t[2500] = np.inf
    check(torch_cuda, t, 0.0, 0, label="inf term")
    check(torch_cuda, np.full(4000, 2.0 ** -60), 1.0, 0, label="below half an ulp")
    check(torch_cuda, np.full(4000, 2.0 ** -53), 1.0, 0, label="exactly half an ulp")


def test_short_chains(torch_cuda):
    """The one-term-per-thread form (chains of at most 1,024 terms, as the mid top-k tail replays): pieces of the
    patterns above, with ties, crossings, stops and a draw."""
    rng = np.random.default_rng(6)
    ties = (2 * rng.integers(0, 1 << 20, 1024) + 1).astype(np.float64) * 2.0 ** -53
    up = rng.uniform(0, 10, 1000)
    p = np.sort(rng.dirichlet(np.full(700, 0.3)))[::-1].astype(np.float32).astype(np.float64)
    mixed = rng.standard_normal(1024) * 10.0 ** rng.uniform(-20, 5, 1024)
    x = np.sort(rng.uniform(0, 40, 1024))
    soft = np.exp(-x).astype(np.float32).astype(np.float64)
    soft[0] = 1.0
    say("short chains")
    check(torch_cuda, ties, 1.0, 0, label="short ties")
    check(torch_cuda, up, 0.0, 0, label="short up")
    check(torch_cuda, up, 0.0, 1, 2500.5, label="short stop")
    check(torch_cuda, p, 0.0, 1, 0.95, label="short top-p")
    check(torch_cuda, -p, 0.37 * float(np.sum(p)), 2, label="short draw")
    check(torch_cuda, mixed, 3.0, 0, label="short mixed")
    check(torch_cuda, soft, 0.0, 0, label="short softmax")
    check(torch_cuda, soft[:1], 0.0, 0, label="one term")

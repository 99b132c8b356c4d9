"""CPU checks that pin the oracle (oracle/sampler_oracle.cpp): the reference's own sampler compiled from its
sources, the C++ standard's known answer for mt19937_64, the host libm exhaustively for expf, and closed forms."""
import json
import os

import numpy as np
import pytest

from klein_amd import workloads as W
from klein_amd.rng import MT19937_64, canonical

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_mt19937_64_kat(oracle_lib):
    # [rand.predef]: the 10000th consecutive invocation of a default-constructed mt19937_64 yields 9981545732273789042
    assert oracle_lib.lib().orc_mt64_nth(5489, 10000) == 9981545732273789042
    g = MT19937_64()
    g.discard(9999)
    assert g() == 9981545732273789042


def test_uniform_stream_matches_std(oracle_lib):
    for seed in (1, 42, 0xDEADBEEF, 2**63 + 5):
        g = MT19937_64(seed)
        ours = [canonical(g) for _ in range(100)]
        assert ours == list(oracle_lib.uniforms(seed, 100))
    # the clamp below 1: an engine output within 2^10 of 2^64 rounds to 2^64 as a double
    assert float(2**64 - 1) / 2**64 == 1.0


def test_expf_restatement_exhaustive(oracle_lib):
    """Every float in [-110, 89] (2.24e9 inputs): the table+polynomial expf equals the host libm's bit for bit."""
    import struct
    lo_neg = struct.unpack("<I", struct.pack("<f", -110.0))[0]
    hi_pos = struct.unpack("<I", struct.pack("<f", 89.0))[0]
    n = os.cpu_count() or 8
    bad = oracle_lib.lib().orc_expf_check(0x80000000, lo_neg, n) + oracle_lib.lib().orc_expf_check(0, hi_pos, n)
    assert bad == 0


def test_expf_restatement_specials(oracle_lib):
    L = oracle_lib.lib()
    for x in (0.0, -0.0, 1.0, -1.0, 88.0, 88.72283, 88.7229, -87.3, -103.97, -103.98, -104.0, float("-inf"),
              float("inf"), 1e-30, -1e-30):
        a, b = L.orc_expf_glibc(x), L.orc_libm_expf(x)
        assert (a == b) or (np.isnan(a) and np.isnan(b)), x
    assert np.isnan(L.orc_expf_glibc(float("nan")))


def _ref_or_skip(oracle_lib):
    if not oracle_lib.ref_available():
        pytest.skip("reference build (oracle/_ref) not present")
    return oracle_lib


RANDOM_PARAMS = [
    dict(temperature=0.0, top_k=20, top_p=0.95, min_p=0.0),
    dict(temperature=1.0, top_k=20, top_p=0.95, min_p=0.0),
    dict(temperature=0.7, top_k=20, top_p=0.8, min_p=0.0),
    dict(temperature=1.0, top_k=40, top_p=0.95, min_p=0.05, presence_penalty=0.5, frequency_penalty=0.2,
         repetition_penalty=1.1),
    dict(temperature=0.6, top_k=1, top_p=0.95),
    dict(temperature=1.3, top_k=64, top_p=1.0, min_p=0.1),
    dict(temperature=0.9, top_k=0, top_p=0.5),
    dict(temperature=1.0, top_k=7, top_p=0.95, presence_penalty=-0.7, repetition_penalty=0.8),
    dict(temperature=0.0, top_k=5, presence_penalty=1.5),
    dict(temperature=2.0, top_k=300, top_p=0.99, frequency_penalty=-0.3),
]


@pytest.mark.parametrize("pi", range(len(RANDOM_PARAMS)))
def test_oracle_equals_reference_build(oracle_lib, pi):
    """Restatement (std::partial_sort mode) == the reference's sampler.cpp compiled from its sources, token for
    token, with the reference drawing from its own mt19937_64 and the oracle fed the same stream's uniforms."""
    O = _ref_or_skip(oracle_lib)
    rng = np.random.default_rng(100 + pi)
    for trial in range(6):
        V = int(rng.choice([50, 333, 1000, 4099, 20000]))
        p = W.Params(**RANDOM_PARAMS[pi], seed=int(rng.integers(1, 2**63)))
        logits = (rng.standard_normal(V) * rng.uniform(0.5, 3)).astype(np.float32)
        if trial % 2:
            logits[rng.choice(V, 10, replace=False)] += 6
        hist = rng.integers(0, V, size=int(rng.integers(0, 300))).astype(np.int32)
        ref = O.RefSampler(p)
        for t in hist:
            ref.accept(int(t))
        counts = W.counts_of(hist, V)
        g = MT19937_64(p.seed)
        for step in range(3):
            row = (logits + np.float32(step) * rng.standard_normal(V).astype(np.float32)).astype(np.float32)
            r = ref.sample(row)
            u = canonical(g) if p.temperature > 0 else 0.0
            t, ids, probs, kept = O.sample(row, p, u, counts, O.MODE_STDLIB)
            assert t == r, (pi, trial, step)
            ref.accept(r)
            counts[r] += 1


def test_oracle_verify_equals_reference_build(oracle_lib):
    O = _ref_or_skip(oracle_lib)
    rng = np.random.default_rng(7)
    for trial in range(12):
        V = 3000
        p = W.Params(temperature=float(rng.choice([0.0, 0.6, 1.0])), top_k=int(rng.choice([1, 5, 20])), top_p=0.95,
                     presence_penalty=float(rng.choice([0.0, 0.5])), seed=int(rng.integers(1, 2**62)))
        logits = rng.standard_normal((4, V)).astype(np.float32) * 2
        # drafts that are often right: the argmax of each row, sometimes replaced
        drafts = np.argmax(logits[:3], axis=1).astype(np.int32)
        drafts[rng.random(3) < 0.3] = rng.integers(0, V)
        ref = O.RefSampler(p)
        hist = rng.integers(0, V, 50).astype(np.int32)
        for t in hist:
            ref.accept(int(t))
        rt, ra = ref.verify(logits, drafts)
        g = MT19937_64(p.seed)
        u = np.array([canonical(g) for _ in range(4)]) if p.temperature > 0 else np.zeros(4)
        ot, oa, _ = O.verify(logits, drafts, p, u, W.counts_of(hist, V), O.MODE_STDLIB)
        assert oa == ra and list(ot[:oa + 1]) == list(rt[:ra + 1]), trial


def test_greedy_closed_form(oracle_lib):
    rng = np.random.default_rng(3)
    for _ in range(20):
        V = int(rng.integers(1, 5000))
        x = rng.integers(-4, 4, V).astype(np.float32)  # many exact ties
        t, *_ = oracle_lib.sample(x, W.Params(temperature=0.0), 0.0)
        assert t == int(np.argmax(x))  # numpy returns the first maximal index
    x = np.full(10, -np.inf, dtype=np.float32)
    assert oracle_lib.sample(x, W.Params(temperature=0.0), 0.0)[0] == 0


def _max_element_loop(x):
    """The textbook std::max_element: the running maximum starts at element 0 and only '<' replaces it."""
    best = 0
    for i in range(1, len(x)):
        if x[best] < x[i]:
            best = i
    return best


def _max_element_closed(x):
    """Closed form: a NaN first element is the result; otherwise the first index of the largest number (NaNs
    never compare larger), and 0 when no element exceeds the first."""
    if np.isnan(x[0]):
        return 0
    num = np.where(np.isnan(x), -np.inf, x)
    m = num.max()
    return 0 if m <= x[0] else int(np.argmax(num == m))


def test_argmax_matches_textbook_loop_and_closed_form(oracle_lib):
    """Engine::mtp_draft_token (engine.cpp:413-415) = std::max_element: pinned by the loop definition on small
    rows and by the closed form on long ones, with planted ties, NaNs and infinities."""
    rng = np.random.default_rng(11)
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0], dtype=np.float32)
    for trial in range(400):
        V = int(rng.integers(1, 40))
        x = rng.integers(-3, 3, V).astype(np.float32)
        k = int(rng.integers(0, 4))
        if k:
            x[rng.integers(0, V, k)] = specials[rng.integers(0, len(specials), k)]
        got = oracle_lib.argmax(x)
        assert got == _max_element_loop(x) == _max_element_closed(x), (trial, x)
    for trial in range(20):
        V = int(rng.integers(1000, 300000))
        x = rng.standard_normal(V).astype(np.float32)
        x[rng.integers(0, V, 5)] = x.max()  # ties with the maximum
        if trial % 4 == 1:
            x[rng.integers(0, V, 50)] = np.nan
        if trial % 4 == 2:
            x[0] = np.nan
        if trial % 4 == 3:
            x[:] = -np.inf
        assert oracle_lib.argmax(x) == _max_element_closed(x), trial
    # (a dropped NaN-first rule or a '<=' comparison each fail one of these)
    assert oracle_lib.argmax(np.array([np.nan, 1.0, 2.0], np.float32)) == 0
    assert oracle_lib.argmax(np.array([1.0, 2.0, 2.0], np.float32)) == 1
    assert oracle_lib.argmax(np.array([-np.inf, np.nan, -np.inf], np.float32)) == 0


def _ppl_closed(l, t, b=None):
    """Float64 closed forms of the ppl scores: numpy's (pairwise) sums instead of the loop's sequential ones."""
    x = l.astype(np.float64)
    mx = float(l[0]) if np.isnan(l[0]) else float(np.nanmax(np.where(np.isnan(l), -np.inf, l)))
    with np.errstate(invalid="ignore", over="ignore"):
        lse = mx + np.log(np.sum(np.exp(x - mx)))
    d = dict(lse=lse, nll=lse - x[t], top=_max_element_closed(l))
    if b is not None:
        bb = b.astype(np.float64)
        m = b > -16.0
        terms = np.exp(bb[m]) * (bb[m] - (x[m] - lse))
        d.update(kl=float(np.sum(terms)), kl_mag=float(np.sum(np.abs(terms))), nll_base=-bb[t],
                 base_top=_max_element_closed(b))
    return d


def test_ppl_row_closed_forms(oracle_lib):
    """cmd_ppl's per-token scores (main.cpp:308-327): lse and nll against float64 logsumexp, kl against the
    float64 sum of its terms, both to rounding (a float exp, a dropped term or a sign error is far outside), the
    indices by the first-maximum rule, and the NaN / infinity outcomes."""
    rng = np.random.default_rng(21)
    for trial in range(12):
        V = int(rng.integers(2, 60000))
        l = (rng.standard_normal(V) * 2).astype(np.float32)
        l[rng.integers(0, V, 3)] = l.max()  # ties with the maximum
        z = (rng.standard_normal(V) * 3).astype(np.float64)
        b = (z - (z.max() + np.log(np.sum(np.exp(z - z.max()))))).astype(np.float32)  # base log-probabilities
        t = int(rng.integers(0, V))
        got = oracle_lib.ppl_row(l, t, b)
        exp = _ppl_closed(l, t, b)
        assert got["top"] == exp["top"] and got["base_top"] == exp["base_top"]
        assert abs(got["lse"] - exp["lse"]) <= 1e-12 * abs(exp["lse"]) + 1e-13
        assert abs(got["nll"] - exp["nll"]) <= 1e-12 * abs(exp["lse"]) + 1e-13
        assert abs(got["kl"] - exp["kl"]) <= 1e-12 * exp["kl_mag"] + 1e-15
        assert got["nll_base"] == exp["nll_base"]
    # NaN and infinities: the reference's arithmetic decides
    nan = np.float32(np.nan)
    r = oracle_lib.ppl_row(np.array([nan, 1, 2], np.float32), 1)
    assert np.isnan(r["lse"]) and r["top"] == 0
    r = oracle_lib.ppl_row(np.array([0, nan, 2], np.float32), 1)
    assert np.isnan(r["lse"]) and r["top"] == 2
    r = oracle_lib.ppl_row(np.array([-np.inf, -np.inf], np.float32), 0)
    assert np.isnan(r["lse"]) and r["top"] == 0
    r = oracle_lib.ppl_row(np.array([1, np.inf, 2], np.float32), 0)
    assert np.isnan(r["lse"]) and r["top"] == 1
    r = oracle_lib.ppl_row(np.array([-np.inf, 0.0, 0.0], np.float32), 1)
    assert r["lse"] == np.log(2.0) and r["top"] == 1 and r["nll"] == np.log(2.0)


def test_penalty_closed_form_brute_force(oracle_lib):
    """Tiny vocabulary: greedy over the penalized logits written out with explicit float32 roundings."""
    rng = np.random.default_rng(11)
    f32 = np.float32
    for _ in range(200):
        V = 12
        x = (rng.standard_normal(V) * 2).astype(f32)
        counts = rng.integers(0, 4, V).astype(np.int32)
        rep, pres, freq = f32(rng.choice([1.0, 1.1, 0.7])), f32(rng.choice([0, 0.5, -0.3])), f32(rng.choice([0, 0.2]))
        if rep == 1 and pres == 0 and freq == 0:
            pres = f32(0.25)
        y = x.copy()
        for i in range(V):
            if counts[i] > 0:
                l = x[i]
                if rep != f32(1):
                    l = f32(l / rep) if l > 0 else f32(l * rep)
                l = f32(l - f32(pres + f32(freq * f32(counts[i]))))
                y[i] = l
        p = W.Params(temperature=0.0, presence_penalty=float(pres), frequency_penalty=float(freq),
                     repetition_penalty=float(rep))
        assert oracle_lib.sample(x, p, 0.0, counts)[0] == int(np.argmax(y))


def test_softmax_topk_invariants(oracle_lib):
    rng = np.random.default_rng(5)
    V = 20000
    for _ in range(10):
        x = (rng.standard_normal(V) * 1.5).astype(np.float32)
        k = int(rng.integers(1, 65))
        p = W.Params(temperature=float(rng.uniform(0.3, 2)), top_k=k, top_p=1.0, min_p=0.0)
        t, ids, probs, kept = oracle_lib.sample(x, p, float(rng.random()))
        order = np.lexsort((np.arange(V), -x))  # value descending, id ascending
        assert list(ids) == list(order[:k])
        assert abs(float(np.sum(probs.astype(np.float64))) - 1.0) < 1e-5
        assert np.all(np.diff(probs) <= 0)
        assert kept == k  # top_p = 1 and min_p = 0 keep every candidate
        assert t in set(ids.tolist())
        # top_k = 1 is greedy
        assert oracle_lib.sample(x, W.Params(temperature=1.0, top_k=1), 0.7)[0] == int(np.argmax(x))
        # T -> 0+: all mass on the maximum
        assert oracle_lib.sample(x, W.Params(temperature=1e-6, top_k=k), 0.999)[0] == int(np.argmax(x))


def test_ties_lower_id_wins_in_total_order(oracle_lib):
    V = 1000
    x = np.zeros(V, dtype=np.float32)
    x[[900, 10, 500, 20]] = 5.0
    t, ids, probs, _ = oracle_lib.sample(x, W.Params(temperature=1.0, top_k=3, top_p=1.0), 0.0,
                                         mode=oracle_lib.MODE_TOTAL)
    assert list(ids) == [10, 20, 500]
    assert t == 10  # u = 0 draws the first candidate


def test_stdlib_tie_order_known_case(oracle_lib):
    """libstdc++ partial_sort on [5(id0), 5(id1), 9(id2)] with k=2 keeps ids [2, 0]. Observed through the
    reference build: seed 27's first draw (u = 0.99714) lands on the second candidate."""
    x = np.array([5.0, 5.0, 9.0], dtype=np.float32)
    p = W.Params(temperature=1.0, top_k=2, top_p=1.0, seed=27)
    u = oracle_lib.uniforms(27, 1)[0]
    assert u > 0.995
    t, ids, _, _ = oracle_lib.sample(x, p, u, mode=oracle_lib.MODE_STDLIB)
    assert list(ids) == [2, 0] and t == 0
    if oracle_lib.ref_available():
        assert oracle_lib.RefSampler(p).sample(x) == 0


def test_verify_accept_closed_form(oracle_lib):
    V = 500
    rng = np.random.default_rng(9)
    x = rng.standard_normal((4, V)).astype(np.float32)
    am = np.argmax(x, axis=1).astype(np.int32)
    greedy = W.Params(temperature=0.0)
    for n_right in range(4):
        drafts = am[:3].copy()
        if n_right < 3:
            drafts[n_right] = (am[n_right] + 1) % V
        toks, acc, _ = oracle_lib.verify(x, drafts, greedy, np.zeros(4))
        assert acc == n_right
        assert list(toks[:acc + 1]) == list(am[:acc + 1])


@pytest.mark.parametrize("name", ["greedy", "topk_topp", "penalties", "verify", "batched"])
def test_golden_fixtures(oracle_lib, name):
    """The committed fixtures (written from the reference build) still hold: same generator bytes, and the
    oracle reproduces the reference's tokens, accepted counts and its own recorded top-k/probabilities."""
    path = os.path.join(GOLDEN, f"{name}.json")
    if not os.path.exists(path):
        pytest.skip("fixture not generated")
    fx = json.load(open(path))
    w = W.BUILDERS[name](seed=fx["seed"])
    assert w.digest() == fx["logits_sha256"]
    p = W.Params(**fx["params"])
    for case in fx["cases"]:
        r = case["row"]
        counts = W.counts_of(w.histories[r], w.vocab) if w.histories else None
        if name == "verify":
            toks, acc, _ = oracle_lib.verify(w.logits, np.array(case["drafts"], np.int32), p,
                                             np.array(case["u"]), None, oracle_lib.MODE_STDLIB)
            assert acc == case["accepted"] and list(toks[:acc + 1]) == case["tokens"][:acc + 1]
            continue
        t, ids, probs, kept = oracle_lib.sample(w.logits[r], p, case["u"], counts, oracle_lib.MODE_STDLIB)
        assert t == case["token"]
        assert list(ids) == case["topk_ids"]
        assert [float(x) for x in probs] == case["topk_probs"]
        assert kept == case["kept"]


def _decode_binary16(u):
    """IEEE binary16 decoded from its fields with integer arithmetic (sign, 5-bit exponent, 10-bit fraction)."""
    sgn = -1.0 if u >> 15 else 1.0
    e, f = (u >> 10) & 0x1F, u & 0x3FF
    if e == 0:
        return sgn * f * 2.0 ** -24
    if e == 31:
        return sgn * float("inf") if f == 0 else float("nan")
    return sgn * (1024 + f) * 2.0 ** (e - 25)


def _decode_bfloat16(u):
    """bfloat16 decoded from its fields (sign, 8-bit exponent, 7-bit fraction)."""
    sgn = -1.0 if u >> 15 else 1.0
    e, f = (u >> 7) & 0xFF, u & 0x7F
    if e == 0:
        return sgn * f * 2.0 ** -133
    if e == 255:
        return sgn * float("inf") if f == 0 else float("nan")
    return sgn * (128 + f) * 2.0 ** (e - 134)


def test_snapshot_conversions_every_pattern(oracle_lib):
    """The oracle's f16 / bf16 -> f32 conversion of rollback snapshots against a field-by-field decode, on all
    65,536 bit patterns each (NaN patterns: NaN out)."""
    O = oracle_lib
    pats = np.arange(65536, dtype=np.uint32)
    for st, dec in ((O.SNAP_F16, _decode_binary16), (O.SNAP_BF16, _decode_bfloat16)):
        got = O.snap_to_f32(pats.astype(np.uint16), st)
        want = np.array([dec(int(u)) for u in pats], dtype=np.float64)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].astype(np.float64), want[~nan])


def test_rollback_closed_form(oracle_lib):
    """Slot i of conv holds 100 + i and snapshot row j holds (j + 1) / 2 (states i and j + 1 tokens back,
    src/state.h:45-46): rolling back after `accepted` of nb - 1 drafts leaves 100 + s in slot 0 and s / 2 in ssm,
    s = nb - 1 - accepted, the other slots untouched; s = 0 changes nothing."""
    O = oracle_lib
    nb, conv_row, ssm_row = 4, 6, 5
    conv = np.stack([np.full(conv_row, 100 + i, np.float32) for i in range(nb)])
    ssm = np.full(ssm_row, -7.0, np.float32)
    for st, enc in ((O.SNAP_F32, lambda v: np.float32(v)),
                    (O.SNAP_F16, lambda v: np.float16(v).view(np.uint16)),
                    (O.SNAP_BF16, lambda v: np.uint16(np.float32(v).view(np.uint32) >> 16))):
        snap = np.stack([np.full(ssm_row, enc((j + 1) / 2)) for j in range(nb - 1)])
        for acc in range(nb):
            c, m = O.rollback_recurrent(conv, ssm, snap, st, acc, nb)
            s = nb - 1 - acc
            assert np.all(c[1:] == conv[1:])
            if s == 0:
                assert np.all(c == conv) and np.all(m == ssm)
            else:
                assert np.all(c[0] == 100 + s) and np.all(m == s / 2)

"""CPU checks of the double-precision exp of the perplexity kernel (klein_amd/csrc/kls_ppl.hip, exp_tab).

The kernel restates Tang's table-driven exp (ACM TOMS 15(2), 1989): k = nearest integer to x*256/ln2, r = x -
k*ln2/256 with a two-part ln2/256, exp(x) = 2^(k>>8) * T[k & 255] * (1 + p(r)) with p the Taylor polynomial of
exp(r) - 1 to r^4. These tests read the table and constants from the kernel source and check them against
60-digit decimal arithmetic: every entry is the correctly rounded 2^(j/256), the leading part of ln2/256 is short
enough that k times it is exact, and the method (each fused multiply-add emulated exactly with rationals, one
rounding) is within 1.25 ulp of exp on points spread over the argument range, on integer multiples of ln2/256
(r = 0) and on the reduction's boundaries (|r| = ln2/512)."""
import math
import os
import re
from decimal import Decimal, getcontext
from fractions import Fraction

import numpy as np
import pytest

SRC = os.path.join(os.path.dirname(__file__), "..", "klein_amd", "csrc", "kls_ppl.hip")
getcontext().prec = 60
LN2 = Decimal(2).ln()


def source():
    return open(SRC).read()


def table():
    body = source().split("kExp256Tab[256] = {", 1)[1].split("};", 1)[0]
    vals = [float.fromhex(t) for t in re.findall(r"0x1\.[0-9a-f]+p[+-]\d+", body)]
    assert len(vals) == 256
    return vals


def constants():
    fn = source().split("double exp_tab(double x, const double* tab) {", 1)[1].split("}", 1)[0]
    hexes = [float.fromhex(t) for t in re.findall(r"0x1\.[0-9a-f]+p[+-]\d+", fn)]
    shift = float.fromhex(re.search(r"kShift = (0x1\.8p52)", fn).group(1))
    inv, lo, hi = hexes[0], hexes[1], hexes[2]
    return shift, inv, hi, lo


def rn(q):
    """Round a rational to the nearest double (ties to even)."""
    return float(q) if q == 0 else _rn(Fraction(q))


def _rn(q):
    f = float(q)  # Fraction.__float__ rounds correctly (ties to even)
    return f


def fma(a, b, c):
    return rn(Fraction(a) * Fraction(b) + Fraction(c))


def exp_tab(x, tab, shift, inv, hi, lo):
    x = min(max(x, -800.0), 710.0)
    t1 = fma(x, inv, shift)
    k = int(np.array(t1).view(np.int64) & 0xFFFFFFFF)
    k = k - (1 << 32) if k >= (1 << 31) else k
    kd = t1 - shift
    r = fma(-kd, lo, fma(-kd, hi, x))
    q = fma(r, fma(r, 1.0 / 24, 1.0 / 6), 0.5)
    p = fma(r * r, q, r)
    t = tab[k & 255]
    return math.ldexp(fma(t, p, t), k >> 8)


def ulps(got, x):
    exact = Decimal(x).exp()
    ref = float(exact)
    if ref == 0.0 or math.isinf(ref):
        return 0.0 if got == ref else math.inf
    return float(abs(Decimal(got) - exact) / Decimal(math.ulp(ref)))


def test_table_entries_correctly_rounded():
    tab = table()
    for j, t in enumerate(tab):
        exact = (LN2 * j / 256).exp()
        assert Decimal(t) - exact <= Decimal(math.ulp(t)) / 2, j
        assert exact - Decimal(t) <= Decimal(math.ulp(t)) / 2, j


def test_reduction_constants():
    shift, inv, hi, lo = constants()
    assert shift == 1.5 * 2.0 ** 52
    assert inv == float(256 / LN2)
    m, _ = math.frexp(hi)
    assert (m * 2 ** 33) == int(m * 2 ** 33), "leading part has at most 33 bits"
    # k*hi exact for |k| < 2^20 (the clamp keeps |x*256/ln2| below 3e5)
    assert abs(Decimal(hi) + Decimal(lo) - LN2 / 256) < Decimal(2) ** -95
    assert 800 * 256 / math.log(2) < 2 ** 20


@pytest.mark.parametrize("seed", [1, 2])
def test_within_an_ulp_and_a_quarter(seed):
    tab, (shift, inv, hi, lo) = table(), constants()
    rng = np.random.default_rng(seed)
    xs = list(rng.uniform(-30.0, 0.0, 300)) + list(rng.uniform(-745.0, 709.0, 150)) + list(rng.uniform(-1, 1, 100))
    step = math.log(2) / 256
    xs += [j * step for j in range(-600, 600, 37)]                     # r = 0
    xs += [(j + 0.5) * step for j in range(-600, 600, 41)]             # |r| at the boundary
    xs += [-0.0, 0.0, 1e-300, -1e-300, 709.7, -744.0, -800.0, -1e6]
    worst = 0.0
    for x in xs:
        u = ulps(exp_tab(float(x), tab, shift, inv, hi, lo), float(x))
        worst = max(worst, u)
        assert u <= 1.25, (x, u)
    assert worst > 0.0  # the check compares real results


def test_planted_mistake_is_caught():
    """A table entry off by one ulp, or a dropped polynomial term, is detected."""
    tab, (shift, inv, hi, lo) = table(), constants()
    bad = list(tab)
    bad[77] = math.nextafter(bad[77], 3.0)
    with pytest.raises(AssertionError):
        for j, t in enumerate(bad):
            exact = (LN2 * j / 256).exp()
            assert abs(Decimal(t) - exact) <= Decimal(math.ulp(t)) / 2, j

    def short(x):  # polynomial to r^3 only
        x = min(max(x, -800.0), 710.0)
        t1 = fma(x, inv, shift)
        k = int(np.array(t1).view(np.int64) & 0xFFFFFFFF)
        k = k - (1 << 32) if k >= (1 << 31) else k
        kd = t1 - shift
        r = fma(-kd, lo, fma(-kd, hi, x))
        p = fma(r * r, fma(r, 1.0 / 6, 0.5), r)
        return math.ldexp(fma(tab[k & 255], p, tab[k & 255]), k >> 8)

    assert max(ulps(short(x), x) for x in [(j + 0.5) * math.log(2) / 256 for j in range(-50, 50, 7)]) > 1.25

"""CPU checks of the arithmetic identities the sampling kernel relies on (no GPU needed).

The repetition penalty divides a logit by `rep` (src/sampler.cpp:24: `l > 0 ? l / rep : l * rep`, in float). The
kernel computes the quotient as RN_f32(l * (1/rep in double)) instead of an IEEE float division; the identity holds
for every float l because the double product's relative error (< 2^-51.9) is smaller than the distance (> 2^-49
relative) from any float quotient to a midpoint between floats. These tests check it against numpy's IEEE float32
division: whole binades, the subnormal range, random bit patterns over all exponents, many divisors, and the
special operands."""
import numpy as np

FLT_MAX = np.finfo(np.float32).max


def kernel_div(a, rep):
    inv = 1.0 / np.float64(np.float32(rep))
    with np.errstate(all="ignore"):
        return (a.astype(np.float64) * inv).astype(np.float32)


def ieee_div(a, rep):
    with np.errstate(all="ignore"):
        return a / np.float32(rep)


def same(x, y):
    xb, yb = x.view(np.uint32), y.view(np.uint32)
    nan = np.isnan(x) & np.isnan(y)
    return np.all((xb == yb) | nan)


def bits_range(lo, hi):
    return np.arange(lo, hi, dtype=np.uint32).view(np.float32)


REPS = [1.1, 0.7, 1.2, 1.05, 0.9, 1.15, 1.3, 2.0, 0.5, 3.0, 1e-3, 1e3, 1.0000001, 0.99999994, 7.0, 1.0 / 3.0,
        np.float32(1e-40), float(FLT_MAX), 1.5e-38]


def test_whole_binades_and_subnormals():
    one_two = bits_range(0x3F800000, 0x40000000)  # [1, 2): every significand
    for rep in (1.1, 0.7, 1.3):
        assert same(kernel_div(one_two, rep), ieee_div(one_two, rep)), rep
    sub = bits_range(1, 0x00800000)  # every positive subnormal
    for rep in (1.1, 0.9):
        assert same(kernel_div(sub, rep), ieee_div(sub, rep)), rep
        assert same(kernel_div(-sub, rep), ieee_div(-sub, rep)), rep


def test_random_patterns_many_divisors():
    rng = np.random.default_rng(123)
    reps = [np.float32(r) for r in REPS] + [np.float32(np.exp(rng.uniform(np.log(1e-3), np.log(1e3)))) for _ in range(40)]
    for rep in reps:
        bits = rng.integers(0, 0x7F800000, 1 << 20, dtype=np.uint32)
        a = bits.view(np.float32)
        a = np.concatenate([a, -a])
        assert same(kernel_div(a, rep), ieee_div(a, rep)), float(rep)


def test_special_operands():
    a = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, FLT_MAX, -FLT_MAX, 1e-45, -1e-45, 1.0, -1.0],
                 dtype=np.float32)
    for rep in (1.1, 0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -2.5, FLT_MAX):
        assert same(kernel_div(a, rep), ieee_div(a, rep)), rep


def test_planted_mistake_is_caught():
    """The comparison is sensitive: a single-precision reciprocal (a plausible shortcut) fails it."""
    rng = np.random.default_rng(5)
    a = rng.integers(0x3F800000, 0x40000000, 1 << 16, dtype=np.uint32).view(np.float32)
    rep = np.float32(1.1)
    single = (a * (np.float32(1.0) / rep)).astype(np.float32)
    assert not same(single, ieee_div(a, rep))

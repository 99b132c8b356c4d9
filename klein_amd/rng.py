"""The draw stream of klein's Sampler: std::mt19937_64 (src/sampler.h:35, seeded at src/sampler.cpp:11) and the
uniform std::uniform_real_distribution<double> derives from one engine output (libstdc++ generate_canonical:
double(x) / 2^64, clamped below 1)."""
from __future__ import annotations

import math

_MASK = (1 << 64) - 1
_N, _M = 312, 156
_MATRIX_A = 0xB5026F5AA96619E9
_UPPER, _LOWER = 0xFFFFFFFF80000000, 0x7FFFFFFF


class MT19937_64:
    """The 64-bit Mersenne Twister of the C++ standard ([rand.predef] mt19937_64)."""

    def __init__(self, seed: int = 5489):
        mt = [0] * _N
        mt[0] = seed & _MASK
        for i in range(1, _N):
            mt[i] = (6364136223846793005 * (mt[i - 1] ^ (mt[i - 1] >> 62)) + i) & _MASK
        self._mt = mt
        self._i = _N

    def _twist(self):
        mt = self._mt
        for i in range(_N):
            x = (mt[i] & _UPPER) | (mt[(i + 1) % _N] & _LOWER)
            xa = x >> 1
            if x & 1:
                xa ^= _MATRIX_A
            mt[i] = mt[(i + _M) % _N] ^ xa
        self._i = 0

    def __call__(self) -> int:
        if self._i >= _N:
            self._twist()
        y = self._mt[self._i]
        self._i += 1
        y ^= (y >> 29) & 0x5555555555555555
        y ^= (y << 17) & 0x71D67FFFEDA60000
        y ^= (y << 37) & 0xFFF7EEE000000000
        y ^= y >> 43
        return y & _MASK

    def discard(self, n: int):
        for _ in range(n):
            self()

    def copy(self) -> "MT19937_64":
        c = MT19937_64.__new__(MT19937_64)
        c._mt = list(self._mt)
        c._i = self._i
        return c


def canonical(g: MT19937_64) -> float:
    """generate_canonical<double, 53>: one engine output x -> double(x) / 2^64 (round to nearest), below 1."""
    u = float(g()) / 18446744073709551616.0
    return u if u < 1.0 else math.nextafter(1.0, 0.0)

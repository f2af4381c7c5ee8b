"""The launch-time division of the head-row kernels (FastDiv in
csrc/h3_common.hpp): q = (n * m) >> (31 + s), m = ceil(2^(31 + s) / d),
s = ceil(log2 d), claimed exact for every n < 2^31, and formed on the device as
mulhi(2n, m) >> s (mulhi: the high 32 bits of the 64-bit product). Checked against integer
division over every divisor up to 4096 plus large ones, at the dividends where
an error would first show (just below and at each multiple of d near 2^31,
and small n). CPU only."""
from __future__ import annotations

import random


def magic(d: int):
    s = 0
    while (1 << s) < d:
        s += 1
    return ((1 << (31 + s)) + d - 1) // d, 31 + s


def fast_div(n: int, m: int, shift: int) -> int:
    assert 0 <= n < (1 << 31) and shift >= 31
    mulhi = ((n << 1) * m) >> 32  # v_mul_hi_u32 of 2n (< 2^32) and m
    return mulhi >> (shift - 31)


def test_magic_fits_32_bits_and_divides_exactly():
    rng = random.Random(0)
    divisors = list(range(1, 4097)) + [rng.randrange(4097, 1 << 31) for _ in range(2000)] + [(1 << 31) - 1, 1 << 30]
    top = (1 << 31) - 1
    for d in divisors:
        m, shift = magic(d)
        assert 0 < m < (1 << 32), d
        k = top // d
        samples = {0, 1, d - 1, d, d + 1, top, top - 1, k * d, k * d - 1, (k - 1) * d, (k - 1) * d - 1}
        samples |= {rng.randrange(0, 1 << 31) for _ in range(8)}
        for n in samples:
            if 0 <= n <= top:
                assert fast_div(n, m, shift) == n // d, (n, d)


def test_exhaustive_small_dividends_for_head_counts():
    """Every n < 2^16 for the divisors head-row splits use (P * Hs, Hs)."""
    for d in (1, 2, 3, 4, 7, 8, 12, 14, 28, 42, 56, 112):
        m, shift = magic(d)
        assert all(fast_div(n, m, shift) == n // d for n in range(1 << 16)), d

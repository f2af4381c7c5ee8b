"""The head-row reciprocal table (build_rsqrt_table / rsqrt_bf16 in
csrc/h3_pointwise.hip): for a bf16 var = 1.m x 2^(2k + p),
bf16(1 / sqrt(var)) with IEEE fp32 sqrt and division equals
T[p][m] x 2^-k, T[p][m] = bf16(1 / sqrt(1.m x 2^p)). Checked over every
positive normal bf16 value with numpy's IEEE fp32 arithmetic. CPU only."""
from __future__ import annotations

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (round to nearest even) -> fp32, for finite x."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def rsqrt_ieee(v: np.ndarray) -> np.ndarray:
    return np.float32(1.0) / np.sqrt(v.astype(np.float32))


def test_table_times_power_of_two_is_the_ieee_sequence():
    e = np.arange(1, 255, dtype=np.uint32)
    m = np.arange(128, dtype=np.uint32)
    bits = ((e[:, None] << 23) | (m[None, :] << 16)).reshape(-1)
    var = bits.view(np.float32)
    exact = bf16_round(rsqrt_ieee(var))
    table = bf16_round(rsqrt_ieee(((np.uint32(127) + (np.arange(256) >> 7).astype(np.uint32)) << 23
                                   | ((np.arange(256) & 127).astype(np.uint32) << 16)).view(np.float32)))
    ee = (bits >> 23).astype(np.int64) - 127
    p = ee & 1
    k = (ee - p) >> 1
    idx = (p << 7) | ((bits >> 16) & 127).astype(np.int64)
    fast = np.ldexp(table[idx], -k).astype(np.float32)
    assert np.array_equal(fast.view(np.uint32), exact.view(np.uint32))

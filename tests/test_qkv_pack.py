"""q/k norm + RoPE and the v pack of one head group in one launch
(launch_h3_qkv_norm_rope_pack), in the layout of InfiniLM's sequence-parallel
attention: by-rank views of the fused [T, 3, P * Hs, 128] projection in,
permuted [P, T, Hs, 128] send buffers out, the RoPE cache rows gathered by
token position (patches/InfiniLM.patch:1071-1110).

CPU: the by-rank views address the projection as the reference's as_strided
does; the oracle's composition reduces to qk_norm_rope on the gathered rows.
GPU: bitwise against the oracle and against the reference's sequence of
separate launches (gather, q launch, k launch, v copy), over shapes that take
both launch shapes, a generic-stride layout and clamped positions.
"""
from __future__ import annotations

import pytest
import torch

from conftest import assert_bitwise

BF = torch.bfloat16


def randn(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(BF)


def test_qkv_by_rank_views(pkg):
    """Part i of the projection, head (p, h) of token t, is projected[t, i, p * Hs + h]
    (patches/InfiniLM.patch:1089-1097)."""
    T, P, Hs, D = 5, 3, 2, 8
    projected = torch.arange(T * 3 * P * Hs * D, dtype=torch.float32).view(T, 3, P * Hs, D)
    views = pkg.qkv_by_rank(projected, P)
    for i, view in enumerate(views):
        assert view.shape == (T, P, Hs, D)
        for t in range(T):
            for p in range(P):
                for h in range(Hs):
                    assert torch.equal(view[t, p, h], projected[t, i, p * Hs + h])
    with pytest.raises(ValueError):
        pkg.qkv_by_rank(projected, 4)


def test_oracle_pack_is_gather_then_qk_norm_rope(oracle):
    gen = torch.Generator().manual_seed(1)
    T, P, Hs = 12, 2, 3
    q, k, v = (randn(gen, T, P, Hs, 128, scale=2.0) for _ in range(3))
    wq, wk = ((randn(gen, 128, scale=0.1) + 1).to(BF) for _ in range(2))
    pos = oracle.grid_positions(2, 3, 4)
    cache = oracle.rope_cache(pos, oracle.rope_powers())
    order = torch.randperm(T, generator=gen)
    q_out, k_out, v_out = oracle.qkv_norm_rope_pack(q, k, v, wq, wk, 1e-6, cache, order)
    assert_bitwise(q_out, oracle.qk_norm_rope(q, wq, 1e-6, cache[order, :48], cache[order, 48:]), "q")
    assert_bitwise(k_out, oracle.qk_norm_rope(k, wk, 1e-6, cache[order, :48], cache[order, 48:]), "k")
    assert_bitwise(v_out, v, "v")
    # Identity positions: the gather is the cache itself.
    q_id, _, _ = oracle.qkv_norm_rope_pack(q, k, v, wq, wk, 1e-6, cache, torch.arange(T))
    assert_bitwise(q_id, oracle.qk_norm_rope(q, wq, 1e-6, cache[:T, :48], cache[:T, 48:]), "identity gather")


def _case(T, P, Hs, seed, device, N=None):
    gen = torch.Generator().manual_seed(seed)
    projected = randn(gen, T, 3, P * Hs, 128, scale=2.0)
    wq, wk = ((randn(gen, 128, scale=0.1) + 1).to(BF) for _ in range(2))
    N = N or T
    from oracle import h3_oracle as oracle
    side = max(1, round(N ** (1 / 3)))
    pos = oracle.grid_positions(side, side, (N + side * side - 1) // (side * side))[:N]
    cache = oracle.rope_cache(pos, oracle.rope_powers())
    positions = torch.randint(0, N, (T,), generator=gen)
    return projected, wq, wk, cache, positions


@pytest.mark.gpu
@pytest.mark.parametrize("T,P,Hs", [(77, 4, 3), (1024, 2, 7), (8192, 1, 14), (300, 8, 1)],
                         ids=["77x4x3", "1024x2x7", "8192x1x14", "300x8x1"])
def test_qkv_pack_production_layout(pkg, oracle, device, T, P, Hs):
    projected, wq, wk, cache, positions = _case(T, P, Hs, T + P, device)
    q, k, v = pkg.qkv_by_rank(projected, P)
    ref = oracle.qkv_norm_rope_pack(q, k, v, wq, wk, 1e-6, cache, positions)
    pd, wqd, wkd, cd, posd = (t.to(device) for t in (projected, wq, wk, cache, positions))
    qd, kd, vd = pkg.qkv_by_rank(pd, P)
    send = [torch.full((P, T, Hs, 128), float("nan"), dtype=BF, device=device) for _ in range(3)]
    outs = [s.permute(1, 0, 2, 3) for s in send]
    pkg.make_qkv_norm_rope_pack()(qd, kd, vd, wqd, wkd, 1e-6, cd, posd, *outs)
    torch.cuda.synchronize()
    for name, got, want in zip("qkv", outs, ref):
        assert_bitwise(got, want, f"{name} {T}x{P}x{Hs}")
    # The reference's sequence: gather the cache rows, one q/k launch each, copy v.
    rows = cd[posd]
    cos, sin = rows[:, :48].contiguous(), rows[:, 48:].contiguous()
    sep = [torch.full((P, T, Hs, 128), float("nan"), dtype=BF, device=device).permute(1, 0, 2, 3)
           for _ in range(2)]
    k_qk = pkg.make_qk_norm_rope()
    k_qk(qd, wqd, 1e-6, cos, sin, sep[0])
    k_qk(kd, wkd, 1e-6, cos, sin, sep[1])
    torch.cuda.synchronize()
    assert_bitwise(outs[0], sep[0], "fused vs separate q")
    assert_bitwise(outs[1], sep[1], "fused vs separate k")
    assert torch.equal(send[2].permute(1, 0, 2, 3).cpu().view(torch.int16), vd.cpu().view(torch.int16))


@pytest.mark.gpu
def test_qkv_pack_generic_strides_and_clamped_positions(pkg, oracle, device):
    """Element path (inner stride 2), int32 positions, positions outside the
    cache clamped to its first / last row."""
    T, P, Hs, N = 50, 2, 3, 40
    projected, wq, wk, cache, _ = _case(T, P, Hs, 7, device, N=N)
    gen = torch.Generator().manual_seed(8)
    positions = torch.randint(-5, N + 5, (T,), generator=gen)
    wide = torch.zeros(T, 3, P * Hs, 256, dtype=BF)
    wide[..., ::2] = projected
    q, k, v = pkg.qkv_by_rank(projected, P)
    ref = oracle.qkv_norm_rope_pack(q, k, v, wq, wk, 1e-6, cache, positions.clamp(0, N - 1))
    qd, kd, vd = pkg.qkv_by_rank(wide.to(device)[..., ::2], P)
    outs = [torch.full((T, P, Hs, 256), float("nan"), dtype=BF, device=device)[..., 1::2] for _ in range(3)]
    pkg.make_qkv_norm_rope_pack()(qd, kd, vd, wq.to(device), wk.to(device), 1e-6, cache.to(device),
                                  positions.to(torch.int32).to(device), *outs)
    torch.cuda.synchronize()
    for name, got, want in zip("qkv", outs, ref):
        assert_bitwise(got, want, f"strided {name}")

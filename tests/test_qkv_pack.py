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

import math
import re
from pathlib import Path

import numpy as np
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


# ------------------------------------------------------------------ fp8 epilogue


def test_qk_fp8_bound_holds_on_adversarial_inputs(oracle):
    """|qk_norm_rope(x)| <= fp32(sqrt(128) * 1.03125) * max|w| for inputs that
    put all of a head's energy in one channel or one rotated pair, at angles
    that keep it there, and for random heads; and the bound is tight within
    10% (a one-hot pass-through channel reaches sqrt(128) * w)."""
    gen = torch.Generator().manual_seed(11)
    rows = []
    for i in range(128):  # one-hot heads, each sign
        for sign in (1.0, -1.0):
            x = torch.zeros(128)
            x[i] = sign * 3.0
            rows.append(x)
    for i in range(48):  # energy split over a rotate-half pair
        x = torch.zeros(128)
        x[i], x[i + 48] = 2.0, -2.0
        rows.append(x)
    rows += list(torch.randn(64, 128, generator=gen) * 4)
    x = torch.stack(rows).to(BF).view(-1, 1, 1, 128)
    T = x.shape[0]
    for w in ((torch.rand(128, generator=gen) * 0.5 + 0.75).to(BF), torch.ones(128, dtype=BF),
              (torch.randn(128, generator=gen) * 2).to(BF)):
        for theta in (0.0, math.pi / 4, math.pi / 2, 1.0, 2.5):
            cos = torch.full((T, 48), math.cos(theta)).to(BF)
            sin = torch.full((T, 48), math.sin(theta)).to(BF)
            y = oracle.qk_norm_rope(x, w, 1e-6, cos, sin).float()
            _, bound = oracle.qk_fp8_descale(w)
            assert float(y.abs().max()) <= float(bound), (theta, float(y.abs().max()), float(bound))
        # Tightness: one-hot at the largest-|w| pass-through channel, angle 0.
        j = 96 + int(w[96:].float().abs().argmax())
        xh = torch.zeros(1, 1, 1, 128)
        xh[..., j] = 1.0
        y = oracle.qk_norm_rope(xh.to(BF), w, 1e-6, cos[:1] * 0 + 1, sin[:1] * 0).float()
        assert float(y.abs().max()) >= 0.9 * math.sqrt(128) * float(w[96:].float().abs().max())


def test_kernel_bound_constant_is_the_oracles():
    text = (Path(__file__).resolve().parents[1] / "minimaxh3_on_k100-ai_amd" / "csrc" / "h3_pointwise.hip").read_text()
    literal = re.search(r"kQkFp8BoundPerWeight = ([0-9.]+)f", text).group(1)
    assert np.float32(float(literal)) == np.float32(math.sqrt(128) * 1.03125)


@pytest.mark.gpu
@pytest.mark.parametrize("T,P,Hs", [(1024, 2, 7), (8192, 1, 14), (77, 4, 3)], ids=["1024x2x7", "8192x1x14", "77x4x3"])
def test_qkv_pack_fp8_codes(pkg, oracle, device, T, P, Hs):
    projected, wq, wk, cache, positions = _case(T, P, Hs, 3 * T + P, device)
    wk = (wk.float() * 1.7).to(BF)  # a different bound for k
    q, k, v = pkg.qkv_by_rank(projected, P)
    q8_ref, k8_ref, v_ref, qd_ref, kd_ref = oracle.qkv_norm_rope_pack_fp8(q, k, v, wq, wk, 1e-6, cache, positions)
    qd, kd, vd = pkg.qkv_by_rank(projected.to(device), P)
    codes = [torch.zeros(P, T, Hs, 128, dtype=torch.float8_e4m3fn, device=device) for _ in range(2)]
    q8, k8 = (c.permute(1, 0, 2, 3) for c in codes)
    v_out = torch.full((T, P, Hs, 128), float("nan"), dtype=BF, device=device)
    q_descale = torch.zeros(P * Hs, device=device)
    k_descale = torch.zeros(P * Hs, device=device)
    pkg.make_qkv_norm_rope_pack_fp8()(qd, kd, vd, wq.to(device), wk.to(device), 1e-6, cache.to(device),
                                      positions.to(device), q8, k8, v_out, q_descale, k_descale)
    torch.cuda.synchronize()
    assert torch.equal(q8.cpu().view(torch.uint8), q8_ref.view(torch.uint8))
    assert torch.equal(k8.cpu().view(torch.uint8), k8_ref.view(torch.uint8))
    assert_bitwise(v_out, v_ref, "v")
    assert torch.equal(q_descale.cpu(), qd_ref.expand(P * Hs))
    assert torch.equal(k_descale.cpu(), kd_ref.expand(P * Hs))


@pytest.mark.gpu
@pytest.mark.parametrize("T,P,Hs", [(1024, 2, 7), (8192, 1, 14), (77, 4, 3), (5, 1, 1), (1, 4, 33)],
                         ids=["1024x2x7", "8192x1x14", "77x4x3", "5x1x1", "1x4x33-fewer-batches-than-heads"])
def test_qkv_pack_fp8_vamax(pkg, oracle, device, T, P, Hs):
    """The pack with V's amax folded into slots: q8 / k8 / v / descales as the
    plain fp8 pack, the maximum over each head's slots equals the oracle's
    amax of |v| over that head's rows, and V quantised from the slots equals
    the oracle's per-head quantisation bitwise (codes and descales), in the
    V^T layout the fp8 attention reads. One head gets a large outlier so its
    amax is a single element somewhere in the middle of the rows. Launches
    with at least one V block per head pin V's blocks to heads (their own
    kernel instantiation); 1x4x33 has 9 batches of 16 rows for 132 heads and
    takes the other path (V's maxima folded in LDS, then atomically)."""
    projected, wq, wk, cache, positions = _case(T, P, Hs, 7 * T + P, device)
    projected[T // 2, 2, P * Hs - 1, 17] = -37.0
    q, k, v = pkg.qkv_by_rank(projected, P)
    q8_ref, k8_ref, v_ref, qd_ref, kd_ref = oracle.qkv_norm_rope_pack_fp8(q, k, v, wq, wk, 1e-6, cache, positions)
    qd, kd, vd = pkg.qkv_by_rank(projected.to(device), P)
    q8 = torch.zeros(T, P, Hs, 128, dtype=torch.float8_e4m3fn, device=device)
    k8 = torch.zeros_like(q8)
    v_out = torch.empty(T, P, Hs, 128, dtype=BF, device=device)
    q_descale, k_descale = torch.zeros(P * Hs, device=device), torch.zeros(P * Hs, device=device)
    v_amax = torch.full((P * Hs, pkg._lib.AMAX_SLOTS), float("nan"), device=device)
    pkg.make_qkv_norm_rope_pack_fp8_vamax()(qd, kd, vd, wq.to(device), wk.to(device), 1e-6, cache.to(device),
                                            positions.to(device), q8, k8, v_out, q_descale, k_descale, v_amax)
    torch.cuda.synchronize()
    assert torch.equal(q8.cpu().view(torch.uint8), q8_ref.view(torch.uint8))
    assert torch.equal(k8.cpu().view(torch.uint8), k8_ref.view(torch.uint8))
    assert_bitwise(v_out, v_ref, "v")
    assert torch.equal(q_descale.cpu(), qd_ref.expand(P * Hs))
    assert torch.equal(k_descale.cpu(), kd_ref.expand(P * Hs))
    amax_ref = oracle.v_amax_per_head(v)  # head p * Hs + h
    assert torch.equal(v_amax.cpu().amax(dim=1), amax_ref)
    assert float(v_amax.cpu().max()) == 37.0
    # Quantise each rank's V from its slots, in the [1, Hs, T, 128] attention view.
    for p in range(P):
        vp = v_out[:, p].unsqueeze(0).transpose(1, 2)
        v8, v_descale = pkg.quantize_fp8_per_head(vp, transposed=True,
                                                  amax_slots=v_amax[p * Hs:(p + 1) * Hs].contiguous())
        torch.cuda.synchronize()
        ref8, refd = oracle.quantize_fp8_per_head(v_ref[:, p].unsqueeze(0).transpose(1, 2))
        assert torch.equal(v_descale.cpu(), refd)
        assert torch.equal(v8.cpu().view(torch.uint8), ref8.view(torch.uint8))


@pytest.mark.gpu
@pytest.mark.parametrize("T,P,Hs", [(1024, 2, 7), (8192, 1, 14), (77, 4, 3), (1, 4, 33)],
                         ids=["1024x2x7", "8192x1x14", "77x4x3", "1x4x33-fewer-batches-than-heads"])
def test_qkv_pack_fp8x2_vamax(pkg, oracle, device, T, P, Hs):
    """The pack with two-term q and k codes: hi codes, lo codes and descales
    bitwise equal to the oracle's qkv_norm_rope_pack_fp8_two_term (the hi
    codes also equal the one-term pack's), v bitwise, V's slots as in the
    one-term pack; the lo outputs are permuted send-buffer views like the hi
    ones."""
    projected, wq, wk, cache, positions = _case(T, P, Hs, 11 * T + P, device)
    q, k, v = pkg.qkv_by_rank(projected, P)
    rq8, rql, rk8, rkl, rv, rqd, rkd = oracle.qkv_norm_rope_pack_fp8_two_term(q, k, v, wq, wk, 1e-6, cache, positions)
    q1, k1, _, _, _ = oracle.qkv_norm_rope_pack_fp8(q, k, v, wq, wk, 1e-6, cache, positions)
    assert torch.equal(rq8.view(torch.uint8), q1.view(torch.uint8))
    qd, kd, vd = pkg.qkv_by_rank(projected.to(device), P)
    codes = torch.full((4, P, T, Hs, 128), 0x7F, dtype=torch.uint8, device=device)  # hi/lo of q/k, send layout
    views = [codes[i].permute(1, 0, 2, 3) for i in range(4)]  # [T, P, Hs, 128]
    v_out = torch.empty(T, P, Hs, 128, dtype=BF, device=device)
    q_descale, k_descale = torch.zeros(P * Hs, device=device), torch.zeros(P * Hs, device=device)
    v_amax = torch.full((P * Hs, pkg._lib.AMAX_SLOTS), float("nan"), device=device)
    pkg.make_qkv_norm_rope_pack_fp8x2_vamax()(qd, kd, vd, wq.to(device), wk.to(device), 1e-6, cache.to(device),
                                              positions.to(device), views[0], views[1], views[2], views[3], v_out,
                                              q_descale, k_descale, v_amax)
    torch.cuda.synchronize()
    for got, ref in zip(views, (rq8, rql, rk8, rkl)):
        assert torch.equal(got.cpu(), ref.view(torch.uint8))
    assert_bitwise(v_out, rv, "v")
    assert torch.equal(q_descale.cpu(), rqd.expand(P * Hs)) and torch.equal(k_descale.cpu(), rkd.expand(P * Hs))
    assert torch.equal(v_amax.cpu().amax(dim=1), oracle.v_amax_per_head(v))
    assert int((views[1].cpu() != 0).sum()) > views[1].numel() // 2  # the lo codes carry the residuals


@pytest.mark.gpu
def test_qkv_pack_fp8x2_feeds_fp8x2_attention(pkg, oracle, device):
    """The fp8 configuration's pipeline on one rank: the two-term pack (q, k
    codes and V's amax slots), V^T quantised from the slots, the two-term
    attention; within relative RMS 5e-2 of fp32 attention on the packed bf16
    q, k, v, and within 4e-3 of the oracle's emulation of the same codes."""
    T, P, Hs = 4096, 1, 4
    projected, wq, wk, cache, positions = _case(T, P, Hs, 5, device)
    q, k, v = pkg.qkv_by_rank(projected.to(device), P)
    q8, ql, k8, kl = (torch.empty(T, P, Hs, 128, dtype=torch.float8_e4m3fn, device=device) for _ in range(4))
    v_out = torch.empty(T, P, Hs, 128, dtype=BF, device=device)
    qd, kd = torch.empty(Hs, device=device), torch.empty(Hs, device=device)
    slots = torch.empty(Hs, pkg._lib.AMAX_SLOTS, device=device)
    pkg.make_qkv_norm_rope_pack_fp8x2_vamax()(q, k, v, wq.to(device), wk.to(device), 1e-6, cache.to(device),
                                              positions.to(device), q8, ql, k8, kl, v_out, qd, kd, slots)
    bhsd = lambda t: t[:, 0].unsqueeze(0).transpose(1, 2)  # noqa: E731  [T, 1, Hs, 128] -> [1, Hs, T, 128]
    v8, vd = pkg.quantize_fp8_per_head(bhsd(v_out), transposed=True, amax_slots=slots)
    out = torch.empty(1, Hs, T, 128, dtype=BF, device=device)
    scale = 128 ** -0.5
    pkg.make_attention_fp8x2()(bhsd(q8), bhsd(ql), bhsd(k8), bhsd(kl), v8, qd, kd, vd, scale, out)
    torch.cuda.synchronize()
    qn, kn, vn = (bhsd(t).cpu() for t in oracle.qkv_norm_rope_pack(*(x.cpu() for x in (q, k, v)), wq, wk, 1e-6,
                                                                    cache, positions))
    ref = oracle.attention(qn, kn, vn, scale)
    rel = float((out.cpu().double() - ref.double()).norm() / ref.double().norm())
    assert rel <= 5e-2, rel
    emu = oracle.attention_fp8_emulated(bhsd(q8).cpu(), bhsd(k8).cpu(), oracle.quantize_fp8_per_head(vn)[0], qd.cpu(),
                                        kd.cpu(), vd.cpu(), scale,
                                        lo_terms=(bhsd(ql).cpu(), qd.cpu() / 16, bhsd(kl).cpu(), kd.cpu() / 16))
    rel_emu = float((out.cpu().double() - emu.double()).norm() / emu.double().norm())
    print(f"EMU pack pipeline: rel {rel_emu:.3e}", flush=True)
    assert rel_emu <= 4e-3, rel_emu  # measured 1.7e-3 on an MI355X


@pytest.mark.gpu
def test_qkv_pack_fp8_tiny_weight(pkg, oracle, device):
    """A q weight of order 1e-38 puts 448 / bound past fp32's range: the
    epilogue takes the (y 2^64) * (448 / (bound 2^64)) form, as the oracle does
    (bitwise codes and descales); k keeps an ordinary weight."""
    T, P, Hs = 256, 1, 3
    projected, wq, wk, cache, positions = _case(T, P, Hs, 5, device)
    wq = (wq.float() * 1e-38).to(BF)
    q, k, v = pkg.qkv_by_rank(projected, P)
    q8_ref, k8_ref, v_ref, qd_ref, kd_ref = oracle.qkv_norm_rope_pack_fp8(q, k, v, wq, wk, 1e-6, cache, positions)
    assert not torch.isnan(q8_ref.float()).any() and float(q8_ref.float().abs().max()) > 0
    qd, kd, vd = pkg.qkv_by_rank(projected.to(device), P)
    q8 = torch.zeros(T, P, Hs, 128, dtype=torch.float8_e4m3fn, device=device)
    k8 = torch.zeros_like(q8)
    v_out = torch.empty(T, P, Hs, 128, dtype=BF, device=device)
    q_descale, k_descale = torch.zeros(P * Hs, device=device), torch.zeros(P * Hs, device=device)
    pkg.make_qkv_norm_rope_pack_fp8()(qd, kd, vd, wq.to(device), wk.to(device), 1e-6, cache.to(device),
                                      positions.to(device), q8, k8, v_out, q_descale, k_descale)
    torch.cuda.synchronize()
    assert torch.equal(q8.cpu().view(torch.uint8), q8_ref.view(torch.uint8))
    assert torch.equal(k8.cpu().view(torch.uint8), k8_ref.view(torch.uint8))
    assert torch.equal(q_descale.cpu(), qd_ref.expand(P * Hs))
    assert torch.equal(k_descale.cpu(), kd_ref.expand(P * Hs))


@pytest.mark.gpu
def test_qkv_pack_fp8_feeds_fp8_attention(pkg, oracle, device):
    """Producer q8 / k8 (weight-bound scales) and the quantiser's v8 into the
    all-fp8 attention lose no accuracy against absmax-scaled q8 / k8 of the same
    bf16 values through the same kernel (relative RMS against fp32 attention
    within 2e-3 of it). The all-fp8 recipe itself sits at about 5.3e-2 on these
    RMSNorm'd inputs for both scalings (the CPU emulation gives the same
    figure), above the fp8 configuration's 5e-2 bar, so only the equivalence
    is asserted for it; the fp8 P.V variant meets the bar."""
    T, H = 2048, 4
    projected, wq, wk, cache, positions = _case(T, 1, H, 99, device)
    qd, kd, vd = pkg.qkv_by_rank(projected.to(device), 1)
    wqd, wkd, cd, pd = wq.to(device), wk.to(device), cache.to(device), positions.to(device)
    q8 = torch.empty(1, H, T, 128, dtype=torch.float8_e4m3fn, device=device)
    k8 = torch.empty_like(q8)
    v_out = torch.empty(1, T, H, 128, dtype=BF, device=device)
    q_descale, k_descale = torch.empty(H, device=device), torch.empty(H, device=device)
    # [T, 1, H, 128] views of the [1, H, T, 128] attention layouts.
    as_tph = lambda t: t[0].permute(1, 0, 2).unsqueeze(1)  # noqa: E731
    pkg.make_qkv_norm_rope_pack_fp8()(qd, kd, vd, wqd, wkd, 1e-6, cd, pd, as_tph(q8), as_tph(k8),
                                      v_out.view(T, 1, H, 128), q_descale, k_descale)
    qb, kb = torch.empty(T, 1, H, 128, dtype=BF, device=device), torch.empty(T, 1, H, 128, dtype=BF, device=device)
    pkg.make_qkv_norm_rope_pack()(qd, kd, vd, wqd, wkd, 1e-6, cd, pd, qb, kb, torch.empty_like(qb))
    to_bhsd = lambda t: t.view(1, T, H, 128).transpose(1, 2)  # noqa: E731
    v = to_bhsd(v_out)
    v8, v_descale = pkg.quantize_fp8_per_head(v, transposed=True)
    qa, qad = pkg.quantize_fp8_per_head(to_bhsd(qb))
    ka, kad = pkg.quantize_fp8_per_head(to_bhsd(kb))
    scale = 128 ** -0.5
    out, out_amax, out_pv = (torch.empty(1, H, T, 128, dtype=BF, device=device) for _ in range(3))
    pkg.make_attention_fp8()(q8, k8, v8, q_descale, k_descale, v_descale, scale, out)
    pkg.make_attention_fp8()(qa, ka, v8, qad, kad, v_descale, scale, out_amax)
    pkg.make_attention_fp8pv()(to_bhsd(qb), to_bhsd(kb), v8, v_descale, scale, out_pv)
    torch.cuda.synchronize()
    ref = oracle.attention(to_bhsd(qb).cpu(), to_bhsd(kb).cpu(), v.cpu(), scale, dtype=torch.float32).double()

    def rel(o):
        return float((o.cpu().double() - ref).norm() / ref.norm())

    r_prod, r_amax, r_pv = rel(out), rel(out_amax), rel(out_pv)
    assert r_prod <= r_amax + 2e-3, (r_prod, r_amax)
    assert r_pv <= 5e-2, r_pv


@pytest.mark.gpu
def test_qkv_pack_fp8_nan_and_inf_rows(pkg, oracle, device):
    """A q head row holding a NaN and a k head row holding +inf: RMSNorm makes
    the first all NaN and the second NaN where the infinite square meets 0 (as
    in the reference's chain); their fp8 codes are NaN codes in kernel and
    oracle alike (the saturation keeps NaN), every other code bitwise, one-term
    and two-term packs."""
    T, P, Hs = 77, 2, 3
    projected, wq, wk, cache, positions = _case(T, P, Hs, 4242, device)
    projected[5, 0, 1, 9] = float("nan")        # a q head row
    projected[11, 1, 2, 100] = float("inf")     # a k head row
    q, k, v = pkg.qkv_by_rank(projected, P)
    q8_ref, k8_ref, _, _, _ = oracle.qkv_norm_rope_pack_fp8(q, k, v, wq, wk, 1e-6, cache, positions)
    rq8, rql, rk8, rkl, _, _, _ = oracle.qkv_norm_rope_pack_fp8_two_term(q, k, v, wq, wk, 1e-6, cache, positions)
    qd, kd, vd = pkg.qkv_by_rank(projected.to(device), P)

    def same(got, ref):
        g, r = got.cpu().view(torch.uint8), ref.view(torch.uint8)
        g_nan, r_nan = (g & 0x7F) == 0x7F, (r & 0x7F) == 0x7F
        return torch.equal(g_nan, r_nan) and torch.equal(g[~g_nan], r[~r_nan]) and bool(r_nan.any())

    codes = [torch.zeros(P, T, Hs, 128, dtype=torch.float8_e4m3fn, device=device) for _ in range(2)]
    q8, k8 = (c.permute(1, 0, 2, 3) for c in codes)
    v_out = torch.empty(T, P, Hs, 128, dtype=BF, device=device)
    qs, ks = torch.zeros(P * Hs, device=device), torch.zeros(P * Hs, device=device)
    pkg.make_qkv_norm_rope_pack_fp8()(qd, kd, vd, wq.to(device), wk.to(device), 1e-6, cache.to(device),
                                      positions.to(device), q8, k8, v_out, qs, ks)
    torch.cuda.synchronize()
    assert same(q8, q8_ref) and same(k8, k8_ref)
    codes2 = torch.zeros((4, P, T, Hs, 128), dtype=torch.uint8, device=device)
    views = [codes2[i].permute(1, 0, 2, 3) for i in range(4)]
    v_amax = torch.zeros((P * Hs, pkg._lib.AMAX_SLOTS), device=device)
    pkg.make_qkv_norm_rope_pack_fp8x2_vamax()(qd, kd, vd, wq.to(device), wk.to(device), 1e-6, cache.to(device),
                                              positions.to(device), views[0], views[1], views[2], views[3], v_out,
                                              qs, ks, v_amax)
    torch.cuda.synchronize()
    for got, ref in zip(views, (rq8, rql, rk8, rkl)):
        assert same(got, ref)

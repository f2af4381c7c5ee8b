"""AdaLN rows per token: the DiT block's three AdaLN sites over all tokens in
one launch each (launch_h3_*_indexed), against the reference's call pattern of
one launch per run-length segment of the AdaLN indices on broadcast views of
the segment's modulation row (patches/InfiniLM.patch:1353-1397, segments built
at :1765-1793).

CPU: the oracle's segment builder on known answers; the per-segment loops
(the reference's pattern) equal the per-token gather forms bitwise, and a
planted wrong row is caught; the host-side index handling.
GPU: every indexed kernel is bitwise the oracle and bitwise the per-segment
launches of the non-indexed kernels, over index patterns (runs, alternating,
random, one row), widths that take each kernel path, batch > 1, strided
views, tables as column blocks of the [R, 6 W] modulation matrix, and
out-of-range indices (clamped by the kernel when the host check is off).
"""
from __future__ import annotations

import pytest
import torch

from conftest import assert_bitwise

BF = torch.bfloat16


def randn(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(BF)


def index_pattern(kind: str, B: int, S: int, R: int, gen) -> torch.Tensor:
    """int64 [B, S] row indices into R table rows."""
    if kind == "runs":  # a few long runs, e.g. the modalities of a sequence
        cuts = sorted(torch.randint(1, max(S, 2), (3,), generator=gen).tolist())
        rows = torch.empty(S, dtype=torch.int64)
        bounds = [0, *cuts, S]
        for i in range(len(bounds) - 1):
            rows[bounds[i]:bounds[i + 1]] = (i * 7 + 1) % R
        return rows.expand(B, S).clone()
    if kind == "alternating":
        return (torch.arange(B * S, dtype=torch.int64) % R).view(B, S)
    if kind == "random":
        return torch.randint(0, R, (B, S), generator=gen, dtype=torch.int64)
    if kind == "one":
        return torch.zeros(B, S, dtype=torch.int64)
    raise ValueError(kind)


# ------------------------------------------------------------------ CPU: oracle


def test_adaln_segments_known_answers(oracle):
    assert oracle.adaln_segments(torch.tensor([], dtype=torch.int64)) == []
    assert oracle.adaln_segments(torch.tensor([3])) == [(0, 1, 3)]
    assert oracle.adaln_segments(torch.tensor([0, 0, 1, 1, 1, 0])) == [(0, 2, 0), (2, 3, 1), (5, 1, 0)]
    assert oracle.adaln_segments(torch.tensor([2, 1, 2, 1])) == [(0, 1, 2), (1, 1, 1), (2, 1, 2), (3, 1, 1)]
    assert oracle.adaln_segments(torch.tensor([5] * 9, dtype=torch.int32)) == [(0, 9, 5)]


@pytest.mark.parametrize("kind", ["runs", "alternating", "random", "one"])
def test_adaln_segments_cover_in_maximal_runs(oracle, kind):
    gen = torch.Generator().manual_seed(1)
    idx = index_pattern(kind, 1, 300, 4, gen)[0]
    segs = oracle.adaln_segments(idx)
    assert segs[0][0] == 0 and sum(n for _, n, _ in segs) == 300
    for (s0, n0, r0), (s1, _, r1) in zip(segs, segs[1:]):
        assert s1 == s0 + n0 and r1 != r0  # contiguous, and no two neighbours share a row
    for start, length, row in segs:
        assert bool((idx[start:start + length] == row).all())


@pytest.mark.parametrize("kind", ["runs", "alternating", "random", "one"])
def test_segment_loops_equal_per_token_forms(oracle, kind):
    gen = torch.Generator().manual_seed(2)
    S, W, R = 97, 256, 5
    x, y = randn(gen, 1, S, W, scale=3.0), randn(gen, 1, S, W)
    w = (randn(gen, W, scale=0.1) + 1).to(BF)
    tables = [randn(gen, R, W, scale=0.5) for _ in range(3)]  # gate, scale, shift
    idx = index_pattern(kind, 1, S, R, gen)
    segs = oracle.adaln_segments(idx)
    assert_bitwise(oracle.rms_modulate_segments(x, w, 1e-6, tables[1], tables[2], segs),
                   oracle.rms_modulate_indexed(x, w, 1e-6, tables[1], tables[2], idx), "rms_modulate")
    res_s, out_s = oracle.gated_residual_rms_modulate_segments(x, tables[0], y, w, 1e-6, tables[1], tables[2], segs)
    res_i, out_i = oracle.gated_residual_rms_modulate_indexed(x, tables[0], y, w, 1e-6, tables[1], tables[2], idx)
    assert_bitwise(res_s, res_i, "residual")
    assert_bitwise(out_s, out_i, "gated rms_modulate")
    assert_bitwise(oracle.gated_residual_segments(x, tables[0], y, segs),
                   oracle.gated_residual_indexed(x, tables[0], y, idx), "gated residual")


def test_a_wrong_segment_row_is_detected(oracle):
    """A planted mistake in the segment list (one run given the next row)
    changes exactly that run's tokens."""
    gen = torch.Generator().manual_seed(3)
    S, W, R = 64, 128, 3
    x = randn(gen, 1, S, W, scale=2.0)
    w = (randn(gen, W, scale=0.1) + 1).to(BF)
    sc, sh = randn(gen, R, W, scale=0.5), randn(gen, R, W, scale=0.5)
    idx = torch.tensor([0] * 20 + [1] * 30 + [2] * 14).view(1, S)
    segs = oracle.adaln_segments(idx)
    wrong = list(segs)
    wrong[1] = (segs[1][0], segs[1][1], (segs[1][2] + 1) % R)
    good = oracle.rms_modulate_indexed(x, w, 1e-6, sc, sh, idx)
    bad = oracle.rms_modulate_segments(x, w, 1e-6, sc, sh, wrong)
    differs = (good.view(torch.int16) != bad.view(torch.int16)).any(dim=-1)[0]
    assert not bool(differs[:20].any()) and not bool(differs[50:].any())
    assert bool(differs[20:50].all())


# ------------------------------------------------------------------ CPU: host logic


def test_modulation_columns_order(pkg):
    """Column block i of the [R, 6 W] modulation matrix is the i-th of shift_msa,
    scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp (patches/InfiniLM.patch:1375)."""
    R, W = 3, 16
    modulation = torch.arange(6, dtype=torch.float32).repeat_interleave(W).repeat(R, 1)
    modulation = modulation + 10 * torch.arange(R, dtype=torch.float32)[:, None]
    cols = pkg.modulation_columns(modulation, W)
    names = ["shift_msa", "scale_msa", "gate_msa", "shift_mlp", "scale_mlp", "gate_mlp"]
    assert list(cols) == names
    for i, name in enumerate(names):
        assert cols[name].shape == (R, W)
        assert cols[name].data_ptr() == modulation.data_ptr() + i * W * 4  # a view, no copy
        assert torch.equal(cols[name], i + 10 * torch.arange(R, dtype=torch.float32)[:, None].expand(R, W))
    with pytest.raises(ValueError):
        pkg.modulation_columns(modulation, W + 1)


def test_token_index_host_checks(pkg):
    from importlib import import_module
    pw = import_module(pkg.__name__ + ".h3_pointwise")
    x = torch.zeros(1, 5, 8)
    out = pw._token_index(torch.tensor([0, 1, 1, 2, 0], dtype=torch.int32), x, 3, True)
    assert out.dtype == torch.int64 and out.shape == (1, 5) and out.tolist() == [[0, 1, 1, 2, 0]]
    with pytest.raises(ValueError, match="out of range"):
        pw._token_index(torch.tensor([0, 1, 3, 2, 0]), x, 3, True)
    with pytest.raises(ValueError, match="out of range"):
        pw._token_index(torch.tensor([0, -1, 0, 0, 0]), x, 3, True)
    assert pw._token_index(torch.tensor([0, 9, 0, 0, 0]), x, 3, False).tolist() == [[0, 9, 0, 0, 0]]
    with pytest.raises(ValueError, match="int32 or int64"):
        pw._token_index(torch.zeros(5), x, 3, True)
    with pytest.raises(ValueError, match=r"\[B, S\]"):
        pw._token_index(torch.zeros(4, dtype=torch.int64), x, 3, True)
    x2 = torch.zeros(2, 5, 8)
    with pytest.raises(ValueError, match=r"\[B, S\]"):
        pw._token_index(torch.zeros(5, dtype=torch.int64), x2, 3, True)


# ------------------------------------------------------------------ GPU: kernels

# (B, S, W): widths through every kernel path of the indexed RMS family --
# W = 128 / 12 (row-group lanes kernel, vector and element paths), 520, 3072,
# 5376, 7168 (rms_stream_kernel, 1 to 4 groups per thread), 8200 and 16384
# (block kernel).
CASES = [(1, 300, 128), (1, 77, 12), (1, 700, 520), (2, 150, 3072), (1, 1500, 5376), (1, 613, 7168),
         (1, 9, 8200), (1, 5, 16384)]
KINDS = ["runs", "alternating", "random", "one"]


def _inputs(B, S, W, R, kind, seed, device):
    gen = torch.Generator().manual_seed(seed)
    x, y = randn(gen, B, S, W, scale=3.0), randn(gen, B, S, W)
    w = (randn(gen, W, scale=0.1) + 1).to(BF)
    modulation = randn(gen, R, 6 * W, scale=0.5)
    idx = index_pattern(kind, B, S, R, gen)
    return x, y, w, modulation, idx


def _segment_launches_rms_modulate(pkg, oracle, x, w, eps, sc, sh, idx, out):
    """The reference's pattern on the GPU: one non-indexed launch per segment
    on broadcast views (patches/InfiniLM.patch:1376-1381)."""
    k = pkg.make_rms_modulate()
    for b in range(x.shape[0]):
        for start, length, row in oracle.adaln_segments(idx[b].cpu()):
            part = x[b:b + 1, start:start + length]
            k(part, w, eps, sc[row].expand_as(part), sh[row].expand_as(part), out[b:b + 1, start:start + length])


@pytest.mark.gpu
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("B,S,W", CASES, ids=[f"{b}x{s}x{w}" for b, s, w in CASES])
def test_rms_modulate_indexed(pkg, oracle, device, B, S, W, kind):
    R = 3
    x, _, w, modulation, idx = _inputs(B, S, W, R, kind, 10 + W, device)
    cols = pkg.modulation_columns(modulation, W)
    ref = oracle.rms_modulate_indexed(x, w, 1e-6, cols["scale_msa"], cols["shift_msa"], idx)
    xd, wd, md, idd = x.to(device), w.to(device), modulation.to(device), idx.to(device)
    cd = pkg.modulation_columns(md, W)
    out = torch.full_like(xd, float("nan"))
    pkg.make_rms_modulate_indexed()(xd, wd, 1e-6, cd["scale_msa"], cd["shift_msa"], idd, out)
    torch.cuda.synchronize()
    assert_bitwise(out, ref, f"rms_modulate_indexed {B}x{S}x{W} {kind}")
    seg = torch.full_like(xd, float("nan"))
    _segment_launches_rms_modulate(pkg, oracle, xd, wd, 1e-6, cd["scale_msa"], cd["shift_msa"], idd, seg)
    torch.cuda.synchronize()
    assert_bitwise(out, seg, "indexed vs per-segment launches")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("B,S,W", CASES, ids=[f"{b}x{s}x{w}" for b, s, w in CASES])
def test_gated_residual_rms_modulate_indexed(pkg, oracle, device, B, S, W, kind):
    R = 4
    x, y, w, modulation, idx = _inputs(B, S, W, R, kind, 20 + W, device)
    cols = pkg.modulation_columns(modulation, W)
    res_ref, out_ref = oracle.gated_residual_rms_modulate_indexed(x, cols["gate_msa"], y, w, 1e-6,
                                                                  cols["scale_mlp"], cols["shift_mlp"], idx)
    xd, yd, wd, md, idd = x.to(device), y.to(device), w.to(device), modulation.to(device), idx.to(device)
    cd = pkg.modulation_columns(md, W)
    res, out = torch.full_like(xd, float("nan")), torch.full_like(xd, float("nan"))
    pkg.make_gated_residual_rms_modulate_indexed()(xd, cd["gate_msa"], yd, wd, 1e-6, cd["scale_mlp"],
                                                   cd["shift_mlp"], idd, res, out)
    torch.cuda.synchronize()
    assert_bitwise(res, res_ref, f"residual {B}x{S}x{W} {kind}")
    assert_bitwise(out, out_ref, f"out {B}x{S}x{W} {kind}")
    # The reference's per-segment launches (patches/InfiniLM.patch:1384-1390).
    k = pkg.make_gated_residual_rms_modulate()
    res2, out2 = torch.full_like(xd, float("nan")), torch.full_like(xd, float("nan"))
    for b in range(B):
        for start, length, row in oracle.adaln_segments(idx[b]):
            sl = (slice(b, b + 1), slice(start, start + length))
            part = xd[sl]
            k(part, cd["gate_msa"][row].expand_as(part), yd[sl], wd, 1e-6, cd["scale_mlp"][row].expand_as(part),
              cd["shift_mlp"][row].expand_as(part), res2[sl], out2[sl])
    torch.cuda.synchronize()
    assert_bitwise(res, res2, "indexed vs per-segment residual")
    assert_bitwise(out, out2, "indexed vs per-segment out")


@pytest.mark.gpu
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("B,S,W", [(1, 300, 128), (1, 77, 12), (2, 150, 3072), (1, 1500, 5376), (1, 5, 16384)],
                         ids=["1x300x128", "1x77x12", "2x150x3072", "1x1500x5376", "1x5x16384"])
def test_gated_residual_indexed(pkg, oracle, device, B, S, W, kind):
    R = 3
    x, y, _, modulation, idx = _inputs(B, S, W, R, kind, 30 + W, device)
    cols = pkg.modulation_columns(modulation, W)
    ref = oracle.gated_residual_indexed(x, cols["gate_mlp"], y, idx)
    xd, yd, md, idd = x.to(device), y.to(device), modulation.to(device), idx.to(device)
    cd = pkg.modulation_columns(md, W)
    out = torch.full_like(xd, float("nan"))
    pkg.make_gated_residual_indexed()(xd, cd["gate_mlp"], yd, idd, out)
    torch.cuda.synchronize()
    assert_bitwise(out, ref, f"gated_residual_indexed {B}x{S}x{W} {kind}")
    k = pkg.make_gated_residual()
    seg = torch.full_like(xd, float("nan"))
    for b in range(B):
        for start, length, row in oracle.adaln_segments(idx[b]):
            sl = (slice(b, b + 1), slice(start, start + length))
            k(xd[sl], cd["gate_mlp"][row].expand_as(xd[sl]), yd[sl], seg[sl])
    torch.cuda.synchronize()
    assert_bitwise(out, seg, "indexed vs per-segment launches")


@pytest.mark.gpu
def test_indexed_strided_views_and_int32(pkg, oracle, device):
    """Non-contiguous x / y / out (element path), transposed index view, int32
    indices, and contiguous [R, W] tables (not column blocks)."""
    gen = torch.Generator().manual_seed(40)
    B, S, W, R = 2, 90, 520, 5
    xb, yb = randn(gen, B, S, 2 * W), randn(gen, B, S, 2 * W)
    x, y = xb[..., ::2], yb[..., 1::2]
    w = (randn(gen, W, scale=0.1) + 1).to(BF)
    g, sc, sh = (randn(gen, R, W, scale=0.5) for _ in range(3))
    idx = torch.randint(0, R, (S, B), generator=gen).t()  # [B, S] with strides (1, B)
    res_ref, out_ref = oracle.gated_residual_rms_modulate_indexed(x, g, y, w, 1e-6, sc, sh, idx)
    dev = lambda t: t.to(device)  # noqa: E731
    xd, yd = dev(xb)[..., ::2], dev(yb)[..., 1::2]
    idd = dev(idx.to(torch.int32).t().contiguous()).t()
    resb, outb = torch.full((B, S, 2 * W), float("nan"), dtype=BF, device=device), \
        torch.full((B, S, 2 * W), float("nan"), dtype=BF, device=device)
    res, out = resb[..., 1::2], outb[..., ::2]
    pkg.make_gated_residual_rms_modulate_indexed()(xd, dev(g), yd, dev(w), 1e-6, dev(sc), dev(sh), idd, res, out)
    torch.cuda.synchronize()
    assert_bitwise(res, res_ref, "strided residual")
    assert_bitwise(out, out_ref, "strided out")
    out2 = torch.full_like(xd, float("nan"))
    pkg.make_rms_modulate_indexed()(xd, dev(w), 1e-6, dev(sc), dev(sh), idd, out2)
    torch.cuda.synchronize()
    assert_bitwise(out2, oracle.rms_modulate_indexed(x, w, 1e-6, sc, sh, idx), "strided rms_modulate")
    out3 = torch.full_like(xd, float("nan"))
    pkg.make_gated_residual_indexed()(xd, dev(g), yd, idd, out3)
    torch.cuda.synchronize()
    assert_bitwise(out3, oracle.gated_residual_indexed(x, g, y, idx), "strided gated residual")


@pytest.mark.gpu
def test_indexed_out_of_range_is_checked_or_clamped(pkg, oracle, device):
    """With the host check (default) an out-of-range index raises before any
    launch; without it the kernels clamp the index into [0, R) and read only
    inside the tables."""
    gen = torch.Generator().manual_seed(50)
    S, W, R = 200, 5376, 3
    x, y = randn(gen, 1, S, W, scale=2.0), randn(gen, 1, S, W)
    w = (randn(gen, W, scale=0.1) + 1).to(BF)
    g, sc, sh = (randn(gen, R, W, scale=0.5) for _ in range(3))
    idx = torch.randint(-4, R + 4, (1, S), generator=gen)
    clamped = idx.clamp(0, R - 1)
    xd, yd, wd, gd, scd, shd, idd = (t.to(device) for t in (x, y, w, g, sc, sh, idx))
    out = torch.empty_like(xd)
    with pytest.raises(ValueError, match="out of range"):
        pkg.make_rms_modulate_indexed()(xd, wd, 1e-6, scd, shd, idd, out)
    pkg.make_rms_modulate_indexed(check_indices=False)(xd, wd, 1e-6, scd, shd, idd, out)
    res2, out2 = torch.empty_like(xd), torch.empty_like(xd)
    pkg.make_gated_residual_rms_modulate_indexed(check_indices=False)(xd, gd, yd, wd, 1e-6, scd, shd, idd, res2,
                                                                      out2)
    out3 = torch.empty_like(xd)
    pkg.make_gated_residual_indexed(check_indices=False)(xd, gd, yd, idd, out3)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.rms_modulate_indexed(x, w, 1e-6, sc, sh, clamped), "clamped rms_modulate")
    r_ref, o_ref = oracle.gated_residual_rms_modulate_indexed(x, g, y, w, 1e-6, sc, sh, clamped)
    assert_bitwise(res2, r_ref, "clamped residual")
    assert_bitwise(out2, o_ref, "clamped out")
    assert_bitwise(out3, oracle.gated_residual_indexed(x, g, y, clamped), "clamped gated residual")


@pytest.mark.gpu
def test_indexed_adaln_block_sites_at_production_shape(pkg, oracle, device):
    """The three AdaLN sites of one DiT block at the reference's per-rank shape
    [1, 5726, 5376] with two modality runs, chained as forward_segmented does
    (patches/InfiniLM.patch:1374-1396), the attention and MLP outputs stood in
    by random tensors."""
    gen = torch.Generator().manual_seed(60)
    T, C, R = 5726, 5376, 2
    hidden, attn, mlp = randn(gen, 1, T, C, scale=2.0), randn(gen, 1, T, C), randn(gen, 1, T, C)
    w1, w2 = ((randn(gen, C, scale=0.1) + 1).to(BF) for _ in range(2))
    modulation = randn(gen, R, 6 * C, scale=0.5)
    idx = torch.tensor([0] * 1000 + [1] * (T - 1000)).view(1, T)
    segs = oracle.adaln_segments(idx)
    cols = pkg.modulation_columns(modulation, C)
    norm_ref = oracle.rms_modulate_segments(hidden, w1, 1e-6, cols["scale_msa"], cols["shift_msa"], segs)
    res_ref, norm2_ref = oracle.gated_residual_rms_modulate_segments(hidden, cols["gate_msa"], attn, w2, 1e-6,
                                                                     cols["scale_mlp"], cols["shift_mlp"], segs)
    out_ref = oracle.gated_residual_segments(res_ref, cols["gate_mlp"], mlp, segs)
    hd, ad, md_, w1d, w2d, modd, idd = (t.to(device) for t in (hidden, attn, mlp, w1, w2, modulation, idx))
    cd = pkg.modulation_columns(modd, C)
    norm, res, norm2, out = (torch.empty_like(hd) for _ in range(4))
    pkg.make_rms_modulate_indexed()(hd, w1d, 1e-6, cd["scale_msa"], cd["shift_msa"], idd, norm)
    pkg.make_gated_residual_rms_modulate_indexed()(hd, cd["gate_msa"], ad, w2d, 1e-6, cd["scale_mlp"],
                                                   cd["shift_mlp"], idd, res, norm2)
    pkg.make_gated_residual_indexed()(res, cd["gate_mlp"], md_, idd, out)
    torch.cuda.synchronize()
    assert_bitwise(norm, norm_ref, "normalized")
    assert_bitwise(res, res_ref, "residual")
    assert_bitwise(norm2, norm2_ref, "normalized_mlp")
    assert_bitwise(out, out_ref, "output")

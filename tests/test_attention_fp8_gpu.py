"""GPU parity of the fp8 (OCP e4m3fn) path.

- Quantiser: bitwise equal to the oracle (same fp32 products, RNE to e4m3fn)
  in both output layouts, ragged S, B > 1, and S x H large enough that each
  amax block folds several chunks; an amax of 23 puts codes on exact ties.
- Attention, both variants: against the oracle's CPU emulation of the same
  algorithm (tight). The fp8 configuration's accuracy bar, relative RMS <=
  5e-2 against fp32 softmax attention, is asserted as it stands:
  - bf16 logits + fp8 P.V (fp8pv) meets it, at small shapes and at S = 73,984
    with 1% of key rows x8;
  - two-term e4m3 Q and K (fp8x2: hi + lo codes, three fp8 Q.K^T products on
    one accumulator) meets it too, at S = 73,984 with the outliers;
  - the all-fp8 recipe (e4m3 Q and K on the fp8 MFMA) does not: per-head e4m3
    Q and K err by up to 2^-5 per element, so the logits of the x8 keys (a
    median 36 log2 units per row's largest) err by a median 0.29 log2 units
    and the weights of those keys by ~22%. Its S = 73,984 case
    is an expected failure (measured relative RMS ~0.12), and its accuracy is
    not asserted elsewhere: the emulation match is its parity check.
- At S = 73,984, all three recipes keep two properties bitwise: V -> 2 V
  doubles the output, and permuting query rows and heads permutes it.
No reference fp8 implementation exists to compare with: parity partial.
"""
from __future__ import annotations

import pytest
import torch

from conftest import attention_error

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _inputs(S, H, seed, outliers):
    from oracle import h3_oracle
    q, k, v = h3_oracle.attention_inputs(S, H=H, seed=seed, outlier_fraction=outliers)
    return tuple(t.transpose(1, 2) for t in (q, k, v))  # [1, H, S, D] views


@pytest.mark.parametrize("S,H,transposed", [(200, 3, False), (200, 3, True), (4096, 2, True), (77, 1, False)])
def test_quantizer_bitwise(pkg, oracle, device, S, H, transposed):
    x, _, _ = _inputs(S, H, 1, 0.01)
    x8, d = pkg.quantize_fp8_per_head(x.to(device), transposed=transposed)
    torch.cuda.synchronize()
    ref8, refd = oracle.quantize_fp8_per_head(x)
    assert torch.equal(d.cpu(), refd)
    assert torch.equal(x8.cpu().view(torch.uint8), ref8.view(torch.uint8))
    if transposed:
        assert x8.stride(2) == 1


@pytest.mark.parametrize("B,S,H,transposed", [(3, 333, 2, False), (3, 333, 2, True), (1, 40000, 14, False),
                                               (1, 40000, 14, True)])
def test_quantizer_bitwise_batched_and_long(pkg, oracle, device, B, S, H, transposed):
    """B > 1 (rows split into (batch, token)) and S x H large enough that each
    amax block folds several 256-row chunks of its head; one outlier per head
    at a varying position sets that head's scale."""
    gen = torch.Generator("cpu").manual_seed(B * 7 + S + H)
    x = torch.randn(B, S, H, 128, generator=gen)
    for h in range(H):
        x[h % B, (h * 7919) % S, h, (h * 31) % 128] = 20.0 + h
    x = x.to(BF).transpose(1, 2)  # [B, H, S, D] view
    x8, d = pkg.quantize_fp8_per_head(x.to(device), transposed=transposed)
    torch.cuda.synchronize()
    ref8, refd = oracle.quantize_fp8_per_head(x)
    assert torch.equal(d.cpu(), refd)
    assert torch.equal(x8.cpu().view(torch.uint8), ref8.view(torch.uint8))


@pytest.mark.parametrize("B,S,H,transposed", [(1, 200, 3, True), (3, 333, 2, True), (2, 77, 5, False),
                                               (1, 73984, 2, True)])
def test_quantizer_from_slots_bitwise(pkg, oracle, device, B, S, H, transposed):
    """The quantiser fed with a producer's amax slots: each head's amax is put
    in one random slot and smaller values in others; codes and descales equal
    the oracle's per-head quantisation bitwise in both layouts (the V^T layout
    is one launch that also writes the descales)."""
    gen = torch.Generator("cpu").manual_seed(B * 31 + S + H)
    x = torch.randn(B, S, H, 128, generator=gen).to(BF).transpose(1, 2)  # [B, H, S, D] view
    amax = x.float().abs().amax(dim=(0, 2, 3))
    slots = torch.rand(H, pkg._lib.AMAX_SLOTS, generator=gen) * amax.view(H, 1) * 0.9
    slots[torch.arange(H), torch.randint(0, pkg._lib.AMAX_SLOTS, (H,), generator=gen)] = amax
    x8, d = pkg.quantize_fp8_per_head(x.to(device), transposed=transposed, amax_slots=slots.to(device))
    torch.cuda.synchronize()
    ref8, refd = oracle.quantize_fp8_per_head(x)
    assert torch.equal(d.cpu(), refd)
    assert torch.equal(x8.cpu().view(torch.uint8), ref8.view(torch.uint8))


@pytest.mark.parametrize("transposed", [False, True])
def test_quantizer_tiny_amax_bitwise(pkg, oracle, device, transposed):
    """Heads whose 448 / amax overflows fp32 (amax 1e-37, 1e-38 and 3e-40, bf16
    normals and subnormals) take the (x 2^64) * (448 / (amax 2^64)) form in
    kernel and oracle alike: bitwise equal codes and descales, zeros stay 0."""
    gen = torch.Generator("cpu").manual_seed(21)
    base = torch.randn(1, 4, 200, 128, generator=gen)
    x = torch.empty_like(base)
    for h, amax in enumerate((1e-37, 1e-38, 3e-40, 1.5)):
        x[0, h] = base[0, h] / base[0, h].abs().max() * amax
    x[0, :, 7] = 0.0
    x = x.to(BF)
    x8, d = pkg.quantize_fp8_per_head(x.to(device), transposed=transposed)
    torch.cuda.synchronize()
    ref8, refd = oracle.quantize_fp8_per_head(x)
    assert torch.equal(d.cpu(), refd)
    assert torch.equal(x8.cpu().view(torch.uint8), ref8.view(torch.uint8))
    assert int(x8.cpu()[0, :, 7].view(torch.uint8).max()) == 0


def test_quantizer_rejects_before_touching_descale(pkg, device):
    """An oversize call (2^31 row chunks) is rejected on the host before the
    quantiser's first launch, so the caller's descale keeps its contents. The
    x / codes views point at a small real buffer and are never read."""
    lib = pkg._lib
    descale = torch.full((16,), 7.0, device=device)
    buf = torch.empty(4096, dtype=BF, device=device)
    shape = [1, 16, 1 << 24, 128]
    strides = [16 * (1 << 24) * 128, (1 << 24) * 128, 128, 1]
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        status = lib.call("launch_h3_quantize_fp8_per_head", stream, lib.raw_tensor(buf.data_ptr(), shape, strides),
                          lib.raw_tensor(buf.data_ptr(), shape, strides), lib.tensor(descale))
    torch.cuda.synchronize()
    assert status == lib.HIP_ERROR_INVALID_VALUE
    assert torch.equal(descale.cpu(), torch.full((16,), 7.0))


@pytest.mark.parametrize("B,S,H", [(1, 200, 3), (3, 333, 2), (1, 40000, 14)])
def test_quantizer_two_term_bitwise(pkg, oracle, device, B, S, H):
    """The two-term split: hi codes, lo codes and the hi descale bitwise equal
    to the oracle's quantize_fp8_two_term (hi equal to the one-term codes),
    with an amax of 23 putting codes on ties and a head of subnormal codes."""
    gen = torch.Generator("cpu").manual_seed(B * 5 + S + H)
    x = torch.randn(B, S, H, 128, generator=gen)
    x[..., 0, :] = (23.0 / 64) * torch.randint(-64, 65, (B, S, 128), generator=gen)
    x[0, 0, 0, 0] = 23.0
    x[..., -1, :] *= 1e-3
    x = x.to(BF).transpose(1, 2)  # [B, H, S, D] view
    hi, lo, d = pkg.quantize_fp8_two_term(x.to(device))
    torch.cuda.synchronize()
    rh, rdh, rl, rdl = oracle.quantize_fp8_two_term(x)
    assert torch.equal(d.cpu(), rdh)
    assert torch.equal(hi.cpu().view(torch.uint8), rh.view(torch.uint8))
    assert torch.equal(lo.cpu().view(torch.uint8), rl.view(torch.uint8))


def test_quantizer_zero_head(pkg, device):
    x = torch.zeros(1, 2, 64, 128, dtype=BF, device=device)
    x[:, 1] = 1.0
    x8, d = pkg.quantize_fp8_per_head(x)
    torch.cuda.synchronize()
    assert torch.equal(d.cpu(), torch.tensor([1.0, 1.0 / 448.0], dtype=torch.float32))
    assert int(x8[:, 0].view(torch.uint8).max()) == 0


def _run(pkg, device, q, k, v, scale, mode):
    qd_, kd_, vd_ = (t.to(device) for t in (q, k, v))
    out = torch.empty(qd_.shape, dtype=BF, device=device)
    v8, vd = pkg.quantize_fp8_per_head(vd_, transposed=True)
    if mode == "fp8":
        q8, qd = pkg.quantize_fp8_per_head(qd_)
        k8, kd = pkg.quantize_fp8_per_head(kd_)
        pkg.make_attention_fp8()(q8, k8, v8, qd, kd, vd, scale, out)
    elif mode == "fp8x2":
        q8, ql, qd = pkg.quantize_fp8_two_term(qd_)
        k8, kl, kd = pkg.quantize_fp8_two_term(kd_)
        pkg.make_attention_fp8x2()(q8, ql, k8, kl, v8, qd, kd, vd, scale, out)
    else:
        pkg.make_attention_fp8pv()(qd_, kd_, v8, vd, scale, out)
    torch.cuda.synchronize()
    return out


# Kernel-to-emulation distance bars, about twice the largest measured on an
# MI355X over this file's cases (relative RMS: fp8 1.5e-3, fp8pv 3.4e-4, fp8x2
# 2.3e-3; max abs under 1e-2 for all). The kernel departs from the emulation
# only in fp32 summation order inside the MFMAs and in exp2's last bit, which
# can move a 448 P across an e4m3 rounding boundary.
EMU_REL = {"fp8": 3e-3, "fp8pv": 8e-4, "fp8x2": 5e-3}
EMU_MAX = 2e-2


def _emu_check(mode, q, k, scale, mx, rel):
    print(f"EMU {mode} {tuple(q.shape)} {tuple(k.shape)} scale {scale:+.3f}: rel {rel:.3e} max {mx:.3e}", flush=True)
    assert rel <= EMU_REL[mode] and mx <= EMU_MAX, (mode, mx, rel)


def _emulated(oracle, q, k, v, scale, mode):
    v8, vd = oracle.quantize_fp8_per_head(v)
    if mode == "fp8":
        q8, qd = oracle.quantize_fp8_per_head(q)
        k8, kd = oracle.quantize_fp8_per_head(k)
        return oracle.attention_fp8_emulated(q8, k8, v8, qd, kd, vd, scale)
    if mode == "fp8x2":
        qh, qdh, ql, qdl = oracle.quantize_fp8_two_term(q)
        kh, kdh, kl, kdl = oracle.quantize_fp8_two_term(k)
        return oracle.attention_fp8_emulated(qh, kh, v8, qdh, kdh, vd, scale, lo_terms=(ql, qdl, kl, kdl))
    return oracle.attention_fp8_emulated(q, k, v8, None, None, vd, scale)


@pytest.mark.parametrize("mode", ["fp8", "fp8pv", "fp8x2"])
@pytest.mark.parametrize("S,H", [(64, 1), (200, 3), (1000, 2), (2048, 2)])
def test_fp8_attention_matches_emulation(pkg, oracle, device, mode, S, H):
    q, k, v = _inputs(S, H, 2, 0.0)
    scale = 128 ** -0.5
    out = _run(pkg, device, q, k, v, scale, mode)
    emu = _emulated(oracle, q, k, v, scale, mode)
    mx, rel = attention_error(out.cpu(), emu)
    _emu_check(mode, q, k, scale, mx, rel)
    if mode in ("fp8pv", "fp8x2"):  # the fp8 configuration's bar; the one-term all-fp8 recipe misses it
        ref = oracle.attention(q, k, v, scale)
        _, rel_ref = attention_error(out.cpu(), ref)
        assert rel_ref <= 5e-2, (mode, rel_ref)


@pytest.mark.parametrize("mode", ["fp8", "fp8pv", "fp8x2"])
@pytest.mark.parametrize("S,H", [(200, 3), (1000, 2)])
def test_fp8_attention_negative_scale(pkg, oracle, device, mode, S, H):
    """A negative softmax scale (the kernels' minimum-logit instantiation: the
    largest c*s is c times the smallest raw logit) against the emulation of
    the same recipe, and a sign mistake there would pick the wrong keys: the
    output must also differ from the positive-scale one."""
    q, k, v = _inputs(S, H, 3, 0.0)
    scale = -(128 ** -0.5)
    out = _run(pkg, device, q, k, v, scale, mode)
    emu = _emulated(oracle, q, k, v, scale, mode)
    mx, rel = attention_error(out.cpu(), emu)
    _emu_check(mode, q, k, scale, mx, rel)
    pos = _run(pkg, device, q, k, v, -scale, mode)
    _, rel_pos = attention_error(out.cpu(), pos.cpu())
    assert rel_pos > 0.2, rel_pos
    if mode in ("fp8pv", "fp8x2"):
        _, rel_ref = attention_error(out.cpu(), oracle.attention(q, k, v, scale))
        assert rel_ref <= 5e-2, (mode, rel_ref)


ALL_FP8_MISSES_THE_BAR = pytest.mark.xfail(
    strict=True, reason="the all-fp8 recipe (per-head e4m3 Q and K) measures relative RMS ~0.12 on the fp8 "
                        "configuration's data against the 5e-2 bar: e4m3 logits of the x8 keys err by a median "
                        "0.29 log2 units")


@pytest.mark.parametrize("mode", [pytest.param("fp8", marks=ALL_FP8_MISSES_THE_BAR), "fp8pv", "fp8x2"])
def test_fp8_attention_config_s73984(pkg, oracle, device, mode):
    """The fp8 configuration: S = 73,984, H = 14, 1% of key rows x8, relative
    RMS <= 5e-2 against fp32 attention."""
    from test_attention_gpu import gpu_reference_fp32
    q, k, v = _inputs(73984, 14, 0, 0.01)
    scale = 128 ** -0.5
    out = _run(pkg, device, q, k, v, scale, mode)
    ref = gpu_reference_fp32(q.to(device), k.to(device), v.to(device), scale)
    mx, rel = attention_error(out, ref)
    print(f"fp8 config ({mode}): max abs {mx:.4f}, relative RMS {rel:.4f}")
    assert rel <= 5e-2, rel


@pytest.mark.parametrize("mode", ["fp8", "fp8pv", "fp8x2"])
@pytest.mark.parametrize("B,H,Sq,Sk", [(2, 2, 130, 333), (2, 1, 64, 65), (1, 3, 1, 100), (2, 2, 300, 64)])
def test_fp8_attention_ragged_batched(pkg, oracle, device, mode, B, H, Sq, Sk):
    """B > 1 and Sq != Sk (the operator contract of launch_h3_full_attention,
    patches/InfiniCore.patch:1366-1376) on both fp8 variants, including a
    partial last key tile, against the CPU emulation of the same algorithm."""
    gen = torch.Generator("cpu").manual_seed(B * 1000 + Sq + Sk)
    q = torch.randn(B, Sq, H, 128, generator=gen).to(BF).transpose(1, 2)
    k = torch.randn(B, Sk, H, 128, generator=gen).to(BF).transpose(1, 2)
    v = torch.randn(B, Sk, H, 128, generator=gen).to(BF).transpose(1, 2)
    scale = 128 ** -0.5
    out = _run(pkg, device, q, k, v, scale, mode)
    emu = _emulated(oracle, q, k, v, scale, mode)
    mx, rel = attention_error(out.cpu(), emu)
    _emu_check(mode, q, k, scale, mx, rel)


@pytest.mark.parametrize("mode", ["fp8x2", "fp8pv", "fp8"])
def test_fp8_attention_exact_invariants_s73984(pkg, device, mode):
    """Bitwise properties at the fp8 configuration's size (S = 73,984, H = 14,
    1% of key rows x8), quantisers included:
      - V -> 2 V doubles every output: V's per-head amax doubles, so its codes
        are the same and its descale doubles, which the epilogue applies as a
        product;
      - permuting the query rows and the heads permutes the output rows: the
        per-head scales move with their heads, and each query's running
        maximum is its own."""
    S, H = 73984, 14
    q, k, v = _inputs(S, H, 0, 0.01)
    scale = 128 ** -0.5
    out = _run(pkg, device, q, k, v, scale, mode)
    out2 = _run(pkg, device, q, k, v * 2, scale, mode)
    assert torch.equal(out2, out * 2), (mode, "V -> 2V")
    gen = torch.Generator("cpu").manual_seed(S)
    perm, hperm = torch.randperm(S, generator=gen), torch.randperm(H, generator=gen)
    qp = q[:, hperm][:, :, perm]  # [1, H, S, D] views: heads, then queries
    outp = _run(pkg, device, qp, k[:, hperm], v[:, hperm], scale, mode)
    assert torch.equal(outp, out[:, hperm][:, :, perm]), (mode, "query and head permutation")


def _codes_equal(got, ref):
    """e4m3fn codes equal bitwise, except that a NaN code matches any NaN code
    (the conversion keeps the NaN's sign bit)."""
    g, r = got.cpu().view(torch.uint8), ref.view(torch.uint8)
    g_nan, r_nan = (g & 0x7F) == 0x7F, (r & 0x7F) == 0x7F
    return torch.equal(g_nan, r_nan) and torch.equal(g[~g_nan], r[~r_nan])


@pytest.mark.parametrize("transposed", [False, True])
def test_quantizer_nan_and_inf(pkg, oracle, device, transposed):
    """A head holding a NaN, one holding +inf, one holding -inf, and a finite
    head: the amax of the first three is not finite, so their code scale is 0
    (finite elements code 0) and NaN and inf * 0 give the NaN code, in kernel
    and oracle alike -- the saturation keeps NaN rather than turning it into
    +-448. Descales bitwise (1 for a head whose amax is NaN), codes bitwise
    with NaN codes matched as NaN. The two-term split likewise."""
    gen = torch.Generator("cpu").manual_seed(33)
    x = torch.randn(1, 4, 200, 128, generator=gen)
    x[0, 0, 17, 5] = float("nan")
    x[0, 1, 3, 100] = float("inf")
    x[0, 2, 150, 0] = float("-inf")
    x = x.to(BF)
    x8, d = pkg.quantize_fp8_per_head(x.to(device), transposed=transposed)
    torch.cuda.synchronize()
    ref8, refd = oracle.quantize_fp8_per_head(x)
    assert torch.equal(d.cpu(), refd), (d.cpu(), refd)
    assert _codes_equal(x8, ref8)
    assert bool(((x8.cpu().view(torch.uint8) & 0x7F) == 0x7F).any())  # the NaN and inf elements are NaN codes
    if not transposed:
        hi, lo, dh = pkg.quantize_fp8_two_term(x.to(device))
        torch.cuda.synchronize()
        rh, rdh, rl, _ = oracle.quantize_fp8_two_term(x)
        assert torch.equal(dh.cpu(), rdh)
        assert _codes_equal(hi, rh) and _codes_equal(lo, rl)

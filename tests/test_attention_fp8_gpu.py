"""GPU parity of the fp8 (OCP e4m3fn) path.

- Quantiser: bitwise equal to the oracle (same fp32 products, RNE to e4m3fn)
  in both output layouts, ragged S, B > 1, and S x H large enough that each
  amax block folds several chunks; an amax of 23 puts codes on exact ties.
- Attention, both variants: against the oracle's CPU emulation of the same
  algorithm (tight), and against the fp32 softmax reference (the bar of the fp8
  configuration: relative RMS <= 5e-2).
- S = 73,984 with 1% of key rows x8: the bf16-logit variant meets 5e-2; the
  all-fp8 recipe's error on that data is measured and bounded (e4m3 logits err
  by ~5% of up to ~30 log2 units, which the CPU emulation reproduces).
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
    else:
        pkg.make_attention_fp8pv()(qd_, kd_, v8, vd, scale, out)
    torch.cuda.synchronize()
    return out


def _emulated(oracle, q, k, v, scale, mode):
    v8, vd = oracle.quantize_fp8_per_head(v)
    if mode == "fp8":
        q8, qd = oracle.quantize_fp8_per_head(q)
        k8, kd = oracle.quantize_fp8_per_head(k)
        return oracle.attention_fp8_emulated(q8, k8, v8, qd, kd, vd, scale)
    return oracle.attention_fp8_emulated(q, k, v8, None, None, vd, scale)


@pytest.mark.parametrize("mode", ["fp8", "fp8pv"])
@pytest.mark.parametrize("S,H", [(64, 1), (200, 3), (1000, 2), (2048, 2)])
def test_fp8_attention_matches_emulation(pkg, oracle, device, mode, S, H):
    q, k, v = _inputs(S, H, 2, 0.0)
    scale = 128 ** -0.5
    out = _run(pkg, device, q, k, v, scale, mode)
    emu = _emulated(oracle, q, k, v, scale, mode)
    mx, rel = attention_error(out.cpu(), emu)
    assert rel <= 1.5e-2 and mx <= 0.05, (mode, mx, rel)
    ref = oracle.attention(q, k, v, scale)
    _, rel_ref = attention_error(out.cpu(), ref)
    assert rel_ref <= 6e-2, (mode, rel_ref)


@pytest.mark.parametrize("mode", ["fp8", "fp8pv"])
def test_fp8_attention_config_s73984(pkg, oracle, device, mode):
    """The fp8 configuration: S = 73,984, H = 14, 1% of key rows x8."""
    from test_attention_gpu import gpu_reference_fp32
    q, k, v = _inputs(73984, 14, 0, 0.01)
    scale = 128 ** -0.5
    out = _run(pkg, device, q, k, v, scale, mode)
    ref = gpu_reference_fp32(q.to(device), k.to(device), v.to(device), scale)
    mx, rel = attention_error(out, ref)
    print(f"fp8 config ({mode}): max abs {mx:.4f}, relative RMS {rel:.4f}")
    if mode == "fp8pv":
        assert rel <= 5e-2, rel
    else:
        assert rel <= 0.2, rel  # measured ~0.12: the all-fp8 recipe misses 5e-2 on this data


@pytest.mark.parametrize("mode", ["fp8", "fp8pv"])
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
    assert rel <= 1.5e-2 and mx <= 0.05, (mode, mx, rel)

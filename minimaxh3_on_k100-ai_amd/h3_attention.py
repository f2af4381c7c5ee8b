"""Non-causal full attention forward on gfx950 MFMA.

Drop-in for tools/h3_attention.py: `make_attention` takes the same keywords and
returns kernel(q, k, v, scale, out) on [B, H, S, D] tensors (any strides on B,
H and S, unit stride on D), with Sq free to differ from Sk. The tile keywords
(block_m, block_n, num_warps, num_stages, backend_options) are accepted for
signature compatibility; the gfx950 kernel uses its own tiles (256 queries x
64 keys per step).

Numerics (tools/h3_attention.py:25-101):
  - "fp32_qk" (default), "fp32_qk_dotacc", "fp32_qk_split": fp32 logits
    scaled by scale*log2(e), exp2 online softmax, bf16 P for P.V, fp32
    denominator. On MFMA the P.V product always accumulates in place and only
    the last key tile is masked, so the three coincide.
Only head_dim 128 (the DiT's) is built; D = 72 (Qwen vision) is not.

fp8: `make_attention_fp8` / `quantize_fp8_per_head` add an OCP e4m3fn variant
with per-head descales (no counterpart in the reference).
"""
from __future__ import annotations

import torch

from . import _lib

__all__ = ["make_attention", "make_attention_fp8", "quantize_fp8_per_head", "NUMERICS"]

NUMERICS = ("fp32_qk", "fp32_qk_dotacc", "fp32_qk_split")


def _check_qkvo(q, k, v, out):
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out)):
        if t.dim() != 4:
            raise ValueError(f"{name} must be [B, H, S, D], got shape {tuple(t.shape)}")
    if q.shape != out.shape or k.shape != v.shape:
        raise ValueError("q/out and k/v must have matching shapes")
    if q.shape[0] != k.shape[0] or q.shape[1] != k.shape[1] or q.shape[3] != k.shape[3]:
        raise ValueError("q and k must agree on B, H and D")


def make_attention(block_m=128, block_n=32, num_warps=4, num_stages=1, caller="torch", output_dir=None,
                   archs=None, backend_options=None, kernel_name="h3_full_attention", numerics="fp32_qk",
                   head_dim=128, dtype=None):
    if head_dim <= 0:
        raise ValueError("head_dim must be positive")
    if head_dim != 128:
        raise ValueError(f"the gfx950 attention kernel is built for head_dim 128, got {head_dim}")
    if numerics not in NUMERICS:
        raise ValueError(f"Unknown attention numerics: {numerics}")
    if dtype is not None and str(getattr(dtype, "name", dtype)).lower() not in ("bfloat16", "torch.bfloat16", "bf16"):
        raise ValueError(f"only the bfloat16 attention kernel is built, got dtype={dtype!r}")

    def kernel(q, k, v, scale, out):
        _check_qkvo(q, k, v, out)
        device = _lib.check_cuda(q, k, v, out)
        _lib.check_dtype(torch.bfloat16, q, k, v, out)
        _lib.launch("launch_h3_full_attention", device, _lib.tensor(q), _lib.tensor(k), _lib.tensor(v),
                    _lib.scalar(scale), _lib.tensor(out))

    return kernel


def quantize_fp8_per_head(x: torch.Tensor, x8: torch.Tensor | None = None,
                          descale: torch.Tensor | None = None):
    """Per-head absmax e4m3fn quantisation of x [B, H, S, 128] (bf16).
    Returns (x8 as torch.float8_e4m3fn [B, H, S, 128], descale fp32 [H]) with
    x ~= x8 * descale[h]; descale = amax_h / 448."""
    if x.dim() != 4:
        raise ValueError("x must be [B, H, S, D]")
    device = _lib.check_cuda(x)
    _lib.check_dtype(torch.bfloat16, x)
    if x8 is None:
        x8 = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=device)
    if descale is None:
        descale = torch.empty(x.shape[1], dtype=torch.float32, device=device)
    _lib.check_dtype(torch.float8_e4m3fn, x8)
    _lib.check_dtype(torch.float32, descale)
    if x8.shape != x.shape or descale.shape != (x.shape[1],) or not descale.is_contiguous():
        raise ValueError("x8 must match x and descale must be a contiguous [H] tensor")
    _lib.launch("launch_h3_quantize_fp8_per_head", device, _lib.tensor(x), _lib.tensor(x8.view(torch.uint8)),
                _lib.tensor(descale))
    return x8, descale


def make_attention_fp8():
    """fp8 (e4m3fn) attention with per-head descales.
    Returns kernel(q8, k8, v8, q_descale, k_descale, v_descale, scale, out)."""

    def kernel(q8, k8, v8, q_descale, k_descale, v_descale, scale, out):
        _check_qkvo(q8, k8, v8, out)
        device = _lib.check_cuda(q8, k8, v8, q_descale, k_descale, v_descale, out)
        _lib.check_dtype(torch.float8_e4m3fn, q8, k8, v8)
        _lib.check_dtype(torch.float32, q_descale, k_descale, v_descale)
        _lib.check_dtype(torch.bfloat16, out)
        for d in (q_descale, k_descale, v_descale):
            if d.shape != (q8.shape[1],) or not d.is_contiguous():
                raise ValueError("descales must be contiguous [H] tensors")
        _lib.launch("launch_h3_full_attention_fp8", device, _lib.tensor(q8.view(torch.uint8)),
                    _lib.tensor(k8.view(torch.uint8)), _lib.tensor(v8.view(torch.uint8)),
                    _lib.tensor(q_descale), _lib.tensor(k_descale), _lib.tensor(v_descale),
                    _lib.scalar(scale), _lib.tensor(out))

    return kernel

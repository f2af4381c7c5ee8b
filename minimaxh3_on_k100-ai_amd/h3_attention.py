"""Non-causal full attention forward on gfx950 MFMA.

Drop-in for tools/h3_attention.py: `make_attention` takes the same keywords and
returns kernel(q, k, v, scale, out) on [B, H, S, D] tensors of any strides
(views without a unit head-dim stride or with rows that are not 16-byte
aligned run on an element-strided path, as the reference's generic stride
variant does), with Sq free to differ from Sk. The tile keywords
(block_m, block_n, num_warps, num_stages, backend_options) are accepted for
signature compatibility; the gfx950 kernel uses its own tiles (256 queries x
64 keys per step).

Numerics (tools/h3_attention.py:25-101):
  - "fp32_qk" (default), "fp32_qk_dotacc", "fp32_qk_split": fp32 logits
    scaled by scale*log2(e), exp2 softmax, bf16 P for P.V. On MFMA the P.V
    product always accumulates in place and only the last key tile is
    masked, so the three coincide.
  - "bf16_prescale" (:87-101): q enters the product as bf16(fp32(scale log2 e) q)
    and the logits are used unscaled (launch_h3_full_attention_bf16_prescale).
  At head_dim 128 the softmax's stabilising maximum is the first key tile's,
  kept for the rest of a 256-query unit (the unit is recomputed with the
  running maximum if anything overflows against it), and the denominator
  sums the same bf16-rounded P that multiplies V. The reference rescales at
  every new running maximum and sums P in fp32; the results agree within the
  operator's tolerance. head_dim 72 keeps the reference's order.
head_dim 128 (the DiT's) and 72 (the Qwen vision tower's, launcher
launch_h3_vision_attention_72 as in scripts/build_h3_attention.py:23-24) are
built; as in the reference, a factory runs only tensors of its own head_dim.

fp8 (no counterpart in the reference): `quantize_fp8_per_head` (per-head
absmax e4m3fn codes), `make_attention_fp8` (Q K^T and P.V on the fp8 MFMA)
and `make_attention_fp8pv` (bf16 logits, fp8 P.V).
"""
from __future__ import annotations

import torch

from . import _lib

__all__ = ["make_attention", "make_attention_fp8", "make_attention_fp8pv", "make_attention_fp8x2",
           "quantize_fp8_per_head", "quantize_fp8_two_term", "NUMERICS"]

NUMERICS = ("fp32_qk", "fp32_qk_dotacc", "fp32_qk_split", "bf16_prescale")


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
                   head_dim=128, dtype=None, *, split_last_round=True):
    """The reference's factory (tools/h3_attention.py:104-121). split_last_round
    (fp32_qk numerics, head_dim 128; no counterpart in the reference): when the
    launch's last round of 256-query workgroups is only partly filled, its
    units are split along the keys (launch_h3_full_attention_ws) with a
    workspace from torch's caching allocator; False always runs the unsplit
    launch_h3_full_attention."""
    if head_dim <= 0:
        raise ValueError("head_dim must be positive")
    if head_dim not in (128, 72):
        raise ValueError(f"the gfx950 attention kernel is built for head_dim 128 and 72, got {head_dim}")
    if head_dim == 72 and numerics == "bf16_prescale":
        raise ValueError("bf16_prescale is built for head_dim 128 only")
    if numerics not in NUMERICS:
        raise ValueError(f"Unknown attention numerics: {numerics}")
    if dtype is not None and str(getattr(dtype, "name", dtype)).lower() not in ("bfloat16", "torch.bfloat16", "bf16"):
        raise ValueError(f"only the bfloat16 attention kernel is built, got dtype={dtype!r}")

    if head_dim == 72:
        entry = "launch_h3_vision_attention_72"
    else:
        entry = "launch_h3_full_attention_bf16_prescale" if numerics == "bf16_prescale" else "launch_h3_full_attention"

    split = split_last_round and entry == "launch_h3_full_attention"
    plans: dict = {}  # (device, B, H, Sq, Sk) -> workspace bytes

    def kernel(q, k, v, scale, out):
        _check_qkvo(q, k, v, out)
        if q.shape[3] != head_dim:
            raise ValueError(f"this kernel is built for head_dim {head_dim}, got tensors of head dim {q.shape[3]}")
        device = _lib.check_cuda(q, k, v, out)
        _lib.check_dtype(torch.bfloat16, q, k, v, out)
        if split:
            key = (device, q.shape[0], q.shape[1], q.shape[2], k.shape[2])
            nbytes = plans.get(key)
            if nbytes is None:
                with torch.cuda.device(device):
                    nbytes = plans[key] = _lib.attention_workspace_bytes(*key[1:])
            if nbytes > 0:
                ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
                _lib.launch("launch_h3_full_attention_ws", device, _lib.tensor(q), _lib.tensor(k), _lib.tensor(v),
                            _lib.scalar(scale), _lib.tensor(out), _lib.tensor(ws))
                return
        _lib.launch(entry, device, _lib.tensor(q), _lib.tensor(k), _lib.tensor(v), _lib.scalar(scale),
                    _lib.tensor(out))

    return kernel


def quantize_fp8_per_head(x: torch.Tensor, transposed: bool = False, x8: torch.Tensor | None = None,
                          descale: torch.Tensor | None = None, amax_slots: torch.Tensor | None = None):
    """Per-head absmax e4m3fn quantisation of x [B, H, S, 128] (bf16).
    Returns (x8, descale): x8 a torch.float8_e4m3fn [B, H, S, 128] view and
    descale fp32 [H] with x ~= x8 * descale[h], descale = amax_h / 448.
    transposed=True stores x8 S-contiguous (physically [B, H, 128, S'] with S'
    rounded up to 16), the layout the fp8 attention kernels read V in.
    amax_slots: fp32 [H, 64] per-head maxima of |x| already folded by the
    producer (make_qkv_norm_rope_pack_fp8_vamax); then only the code pass
    reads x."""
    if x.dim() != 4:
        raise ValueError("x must be [B, H, S, D]")
    device = _lib.check_cuda(x)
    _lib.check_dtype(torch.bfloat16, x)
    B, H, S, D = x.shape
    if x8 is None:
        if transposed:
            s_pad = -(-S // 16) * 16
            store = torch.empty(B, H, D, s_pad, dtype=torch.float8_e4m3fn, device=device)
            x8 = store[..., :S].transpose(2, 3)
        else:
            x8 = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=device)
    if descale is None:
        descale = torch.empty(H, dtype=torch.float32, device=device)
    _lib.check_dtype(torch.float8_e4m3fn, x8)
    _lib.check_dtype(torch.float32, descale)
    if x8.shape != x.shape or descale.shape != (H,) or not descale.is_contiguous():
        raise ValueError("x8 must match x and descale must be a contiguous [H] tensor")
    if amax_slots is not None:
        _lib.check_cuda(x, amax_slots)
        _lib.check_dtype(torch.float32, amax_slots)
        if amax_slots.shape != (H, _lib.AMAX_SLOTS) or not amax_slots.is_contiguous():
            raise ValueError(f"amax_slots must be a contiguous fp32 [H, {_lib.AMAX_SLOTS}] tensor")
        _lib.launch("launch_h3_quantize_fp8_per_head_slots", device, _lib.tensor(x), _lib.tensor(amax_slots),
                    _lib.tensor(x8.view(torch.uint8)), _lib.tensor(descale))
        return x8, descale
    _lib.launch("launch_h3_quantize_fp8_per_head", device, _lib.tensor(x), _lib.tensor(x8.view(torch.uint8)),
                _lib.tensor(descale))
    return x8, descale


def _check_descales(h, *ds):
    for d in ds:
        _lib.check_dtype(torch.float32, d)
        if d.shape != (h,) or not d.is_contiguous():
            raise ValueError("descales must be contiguous fp32 [H] tensors")


def make_attention_fp8():
    """All-fp8 attention (e4m3fn Q, K, V, per-head descales, P requantised to
    e4m3 per 64-key tile). v8 must be S-contiguous (quantize_fp8_per_head(v,
    transposed=True)). Returns kernel(q8, k8, v8, q_descale, k_descale,
    v_descale, scale, out) with out bf16 [B, H, Sq, 128]."""

    def kernel(q8, k8, v8, q_descale, k_descale, v_descale, scale, out):
        _check_qkvo(q8, k8, v8, out)
        device = _lib.check_cuda(q8, k8, v8, q_descale, k_descale, v_descale, out)
        _lib.check_dtype(torch.float8_e4m3fn, q8, k8, v8)
        _lib.check_dtype(torch.bfloat16, out)
        _check_descales(q8.shape[1], q_descale, k_descale, v_descale)
        _lib.launch("launch_h3_full_attention_fp8", device, _lib.tensor(q8.view(torch.uint8)),
                    _lib.tensor(k8.view(torch.uint8)), _lib.tensor(v8.view(torch.uint8)),
                    _lib.tensor(q_descale), _lib.tensor(k_descale), _lib.tensor(v_descale),
                    _lib.scalar(scale), _lib.tensor(out))

    return kernel


def quantize_fp8_two_term(x: torch.Tensor, x8: torch.Tensor | None = None, x8_lo: torch.Tensor | None = None,
                          descale: torch.Tensor | None = None):
    """Two-term per-head e4m3fn split of x [B, H, S, 128] (bf16), D-contiguous:
    x ~= (x8 + x8_lo / 16) * descale[h] with x8 the codes of
    quantize_fp8_per_head and x8_lo = e4m3(16 (y - x8)) for y = x * 448 /
    amax_h (about 8 significant bits). Returns (x8, x8_lo, descale); the lo
    term's descale is descale / 16."""
    if x.dim() != 4:
        raise ValueError("x must be [B, H, S, D]")
    device = _lib.check_cuda(x)
    _lib.check_dtype(torch.bfloat16, x)
    if x8 is None:
        x8 = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=device)
    if x8_lo is None:
        x8_lo = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=device)
    if descale is None:
        descale = torch.empty(x.shape[1], dtype=torch.float32, device=device)
    _lib.check_dtype(torch.float8_e4m3fn, x8, x8_lo)
    _lib.check_dtype(torch.float32, descale)
    _lib.launch("launch_h3_quantize_fp8_two_term", device, _lib.tensor(x), _lib.tensor(x8.view(torch.uint8)),
                _lib.tensor(x8_lo.view(torch.uint8)), _lib.tensor(descale))
    return x8, x8_lo, descale


def make_attention_fp8x2():
    """fp8 attention with two-term Q and K (quantize_fp8_two_term) and
    single-term e4m3 V (S-contiguous, quantize_fp8_per_head(v,
    transposed=True)): the logits are (q8.k8 + (q8.k8_lo + q8_lo.k8) / 16) *
    q_descale * k_descale * scale on the fp8 MFMA (the lo operands' 1/16 is the
    MFMA's block scale), P as in make_attention_fp8; the denominator is the
    fp32 sum of the unquantised P (make_attention_fp8 sums the quantised one).
    Returns kernel(q8, q8_lo, k8, k8_lo, v8, q_descale, k_descale, v_descale,
    scale, out). No counterpart in the reference."""

    def kernel(q8, q8_lo, k8, k8_lo, v8, q_descale, k_descale, v_descale, scale, out):
        _check_qkvo(q8, k8, v8, out)
        if q8_lo.shape != q8.shape or k8_lo.shape != k8.shape:
            raise ValueError("the lo codes must match the hi codes' shapes")
        device = _lib.check_cuda(q8, q8_lo, k8, k8_lo, v8, q_descale, k_descale, v_descale, out)
        _lib.check_dtype(torch.float8_e4m3fn, q8, q8_lo, k8, k8_lo, v8)
        _lib.check_dtype(torch.bfloat16, out)
        _check_descales(q8.shape[1], q_descale, k_descale, v_descale)
        _lib.launch("launch_h3_full_attention_fp8x2", device, *(_lib.tensor(t.view(torch.uint8))
                                                                for t in (q8, q8_lo, k8, k8_lo, v8)),
                    _lib.tensor(q_descale), _lib.tensor(k_descale), _lib.tensor(v_descale), _lib.scalar(scale),
                    _lib.tensor(out))

    return kernel


def make_attention_fp8pv():
    """bf16 logits with an fp8 P.V product: q, k bf16 as for make_attention;
    v8 e4m3fn S-contiguous with v_descale. Returns kernel(q, k, v8, v_descale,
    scale, out)."""

    def kernel(q, k, v8, v_descale, scale, out):
        _check_qkvo(q, k, v8, out)
        device = _lib.check_cuda(q, k, v8, v_descale, out)
        _lib.check_dtype(torch.bfloat16, q, k, out)
        _lib.check_dtype(torch.float8_e4m3fn, v8)
        _check_descales(q.shape[1], v_descale)
        _lib.launch("launch_h3_full_attention_fp8pv", device, _lib.tensor(q), _lib.tensor(k),
                    _lib.tensor(v8.view(torch.uint8)), _lib.tensor(v_descale), _lib.scalar(scale),
                    _lib.tensor(out))

    return kernel

"""Writes tests/golden/h3_golden.npz: small seeded inputs for every op of the
hot path and the oracle's outputs for them.

The reference ships no vectors for this path and its kernels cannot run here
(they need the ninetoothed package), so the fixtures are the oracle's own
outputs, frozen: tests/test_golden.py checks that the oracle still reproduces
them (CPU) and that the HIP kernels match them (GPU). bf16 tensors are stored
as their uint16 bit patterns, fp8 codes as uint8; the file holds plain arrays
only (numpy.load with allow_pickle=False reads it).

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import h3_oracle as O  # noqa: E402

BF = torch.bfloat16
OUT = Path(__file__).resolve().parent / "h3_golden.npz"


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 array of its bit patterns."""
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def randn(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(BF)


def special_values(n: int, gen) -> torch.Tensor:
    """n bf16 values: the special cases first (signed zeros, infinities, NaN,
    largest and smallest normals, subnormals), then N(0, 16)."""
    specials = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), float("nan"), 3.3895314e38, -3.3895314e38,
                             1.1754944e-38, -1.1754944e-38, 9.1835e-41, -9.1835e-41, 1.0, -1.0, 88.5, -88.5,
                             -100.0, 100.0, 64.0, -64.0, 63.75, -63.75], dtype=torch.float32).to(BF)
    rest = randn(gen, n - specials.numel(), scale=4.0)
    return torch.cat([specials, rest])


def build() -> dict:
    gen = torch.Generator("cpu").manual_seed(20261201)
    d = {}

    # RMSNorm at the two widths the reference specialises (W = 128, 5376).
    for W, S in ((128, 64), (5376, 12)):
        x = randn(gen, 1, S, W, scale=4.0)
        w = randn(gen, W, scale=0.1) + 1
        d[f"rms{W}_x"], d[f"rms{W}_w"] = bits(x), bits(w.to(BF))
        d[f"rms{W}_out"] = bits(O.rms_norm(x, w.to(BF), 1e-5))

    # AdaLN RMSNorm, modulation rows per batch entry broadcast over S.
    B, S, C = 2, 6, 7168
    x = randn(gen, B, S, C, scale=4.0)
    w = (randn(gen, C, scale=0.1) + 1).to(BF)
    sc, sh = randn(gen, B, 1, C, scale=0.5), randn(gen, B, 1, C, scale=0.5)
    d.update(mod_x=bits(x), mod_w=bits(w), mod_scale=bits(sc), mod_shift=bits(sh))
    d["mod_out"] = bits(O.rms_modulate(x, w, 1e-6, sc.expand(B, S, C), sh.expand(B, S, C)))

    # Gated residual with special values in x and y, broadcast gate.
    S, C = 8, 1024
    x = special_values(S * C, gen).view(1, S, C)
    y = special_values(S * C, gen)[torch.randperm(S * C, generator=gen)].view(1, S, C)
    g = randn(gen, 1, 1, C, scale=0.5)
    d.update(gres_x=bits(x), gres_gate=bits(g), gres_y=bits(y))
    d["gres_out"] = bits(O.gated_residual(x, g.expand(1, S, C), y))

    # Fused gated residual + AdaLN RMSNorm.
    S, C = 8, 5376
    x, y = randn(gen, 1, S, C, scale=4.0), randn(gen, 1, S, C)
    g, sc, sh = (randn(gen, 1, 1, C, scale=0.5) for _ in range(3))
    w = (randn(gen, C, scale=0.1) + 1).to(BF)
    res, out = O.gated_residual_rms_modulate(x, g.expand(1, S, C), y, w, 1e-6, sc.expand(1, S, C),
                                             sh.expand(1, S, C))
    d.update(fused_x=bits(x), fused_gate=bits(g), fused_y=bits(y), fused_w=bits(w), fused_scale=bits(sc),
             fused_shift=bits(sh), fused_residual=bits(res), fused_out=bits(out))

    # SwiGLU with special gate values (both sides of the |g| < 64 split).
    S, F = 16, 1024
    up = randn(gen, 1, S, F, scale=2.0)
    gate = special_values(S * F, gen).view(1, S, F)
    d.update(swiglu_up=bits(up), swiglu_gate=bits(gate))
    d["swiglu_out"] = bits(O.swiglu(up, gate))

    # Rotate-half RoPE on [S, H, 128] and the fused q/k RMSNorm + RoPE on
    # [T, P, Hs, 128], tables from the RoPE-cache op of the grid positions.
    pos = O.grid_positions(2, 4, 4)  # T = 32
    T = pos.shape[0]
    cache = O.rope_cache(pos, O.rope_powers())
    d.update(cache_pos=pos.numpy(), cache_power=O.rope_powers().numpy(), cache_out=bits(cache))
    x = randn(gen, T, 4, 128, scale=2.0)
    d.update(rope_x=bits(x))
    d["rope_out"] = bits(O.rope_rotate_half(x, cache[:, None, :48], cache[:, None, 48:]))
    x = randn(gen, T, 1, 4, 128, scale=2.0)
    w = (randn(gen, 128, scale=0.1) + 1).to(BF)
    d.update(qk_x=bits(x), qk_w=bits(w))
    d["qk_out"] = bits(O.qk_norm_rope(x, w, 1e-6, cache[:, :48], cache[:, 48:]))
    cos64, sin64 = O.rope_table_interleaved(pos)
    d.update(qki_cos=bits(cos64), qki_sin=bits(sin64))
    d["qki_out"] = bits(O.qk_norm_rope_interleaved(x, w, 1e-6, cos64, sin64))

    # Attention [1, H, S, D] with 1% outlier keys and a partial last tile, the
    # fp64 softmax(q k^T s) v stored in fp32; the fp8 quantiser and the
    # bf16-logit / fp8-P.V emulation on the same inputs.
    q, k, v = (t.transpose(1, 2).contiguous() for t in O.attention_inputs(200, H=2, seed=7, outlier_fraction=0.01))
    scale = 128 ** -0.5
    d.update(attn_q=bits(q), attn_k=bits(k), attn_v=bits(v), attn_scale=np.float64(scale))
    d["attn_out"] = O.attention(q, k, v, scale).to(torch.float32).numpy()
    v8, vd = O.quantize_fp8_per_head(v)
    d.update(fp8_v_codes=v8.view(torch.uint8).numpy(), fp8_v_descale=vd.numpy())
    d["fp8pv_out"] = bits(O.attention_fp8_emulated(q, k, v8, None, None, vd, scale))
    return d


if __name__ == "__main__":
    arrays = build()
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size / 1024:.0f} KiB, {len(arrays)} arrays)")

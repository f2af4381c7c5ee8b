"""Golden fixtures (tests/golden/h3_golden.npz, written by
tests/golden/make_golden.py): small seeded inputs of every hot-path op and the
oracle's outputs for them.

- CPU: the oracle still reproduces every stored output (bitwise for the
  pointwise ops and the fp8 quantiser; attention within 1e-6 of the stored
  fp64 result rounded to fp32; the fp8 emulation within 1 bf16 ulp, whose fp32
  matmuls may round differently on another CPU).
- GPU: the HIP kernels on the stored inputs match the stored outputs --
  bitwise for the pointwise ops and the quantiser, the RoPE table within 1
  bf16 ulp (device cosf/sinf vs the CPU's); attention
  within the bf16 tolerance (max abs <= 2e-2, relative RMS <= 1e-2); the fp8
  P.V variant within relative RMS 1e-3 of its emulation.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import assert_bitwise, attention_error

BF = torch.bfloat16
FIXTURES = Path(__file__).resolve().parent / "golden" / "h3_golden.npz"


@pytest.fixture(scope="module")
def g():
    with np.load(FIXTURES, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def bf(a: np.ndarray) -> torch.Tensor:
    """uint16 bit patterns -> bf16 tensor."""
    return torch.from_numpy(a.astype(np.uint16).view(np.int16).copy()).view(BF)


def test_fixture_file_is_plain_arrays():
    with np.load(FIXTURES, allow_pickle=False) as f:
        assert len(f.files) == 45
        assert all(f[k].dtype != object for k in f.files)


# ------------------------------------------------------------------ CPU: oracle


def test_oracle_reproduces_pointwise(g, oracle):
    for W in (128, 5376):
        assert_bitwise(oracle.rms_norm(bf(g[f"rms{W}_x"]), bf(g[f"rms{W}_w"]), 1e-5), bf(g[f"rms{W}_out"]), f"rms{W}")
    x, sc, sh = bf(g["mod_x"]), bf(g["mod_scale"]), bf(g["mod_shift"])
    assert_bitwise(oracle.rms_modulate(x, bf(g["mod_w"]), 1e-6, sc.expand_as(x), sh.expand_as(x)), bf(g["mod_out"]),
                   "rms_modulate")
    x = bf(g["gres_x"])
    assert_bitwise(oracle.gated_residual(x, bf(g["gres_gate"]).expand_as(x), bf(g["gres_y"])), bf(g["gres_out"]),
                   "gated_residual")
    x = bf(g["fused_x"])
    res, out = oracle.gated_residual_rms_modulate(x, bf(g["fused_gate"]).expand_as(x), bf(g["fused_y"]),
                                                  bf(g["fused_w"]), 1e-6, bf(g["fused_scale"]).expand_as(x),
                                                  bf(g["fused_shift"]).expand_as(x))
    assert_bitwise(res, bf(g["fused_residual"]), "fused residual")
    assert_bitwise(out, bf(g["fused_out"]), "fused out")
    assert_bitwise(oracle.swiglu(bf(g["swiglu_up"]), bf(g["swiglu_gate"])), bf(g["swiglu_out"]), "swiglu")


def test_oracle_reproduces_rope(g, oracle):
    pos, power = torch.from_numpy(g["cache_pos"]), torch.from_numpy(g["cache_power"])
    assert torch.equal(oracle.rope_powers(), power)
    cache = oracle.rope_cache(pos, power)
    assert_bitwise(cache, bf(g["cache_out"]), "rope cache")
    assert_bitwise(oracle.rope_rotate_half(bf(g["rope_x"]), cache[:, None, :48], cache[:, None, 48:]),
                   bf(g["rope_out"]), "rope")
    x, w = bf(g["qk_x"]), bf(g["qk_w"])
    assert_bitwise(oracle.qk_norm_rope(x, w, 1e-6, cache[:, :48], cache[:, 48:]), bf(g["qk_out"]), "qk_norm_rope")
    cos, sin = oracle.rope_table_interleaved(pos)
    assert_bitwise(cos, bf(g["qki_cos"]), "interleaved cos")
    assert_bitwise(sin, bf(g["qki_sin"]), "interleaved sin")
    assert_bitwise(oracle.qk_norm_rope_interleaved(x, w, 1e-6, cos, sin), bf(g["qki_out"]), "qk interleaved")


def test_oracle_reproduces_attention(g, oracle):
    q, k, v, scale = bf(g["attn_q"]), bf(g["attn_k"]), bf(g["attn_v"]), float(g["attn_scale"])
    ref = torch.from_numpy(g["attn_out"])
    assert (oracle.attention(q, k, v, scale).float() - ref).abs().max().item() <= 1e-6
    v8, vd = oracle.quantize_fp8_per_head(v)
    assert np.array_equal(v8.view(torch.uint8).numpy(), g["fp8_v_codes"])
    assert np.array_equal(vd.numpy(), g["fp8_v_descale"])
    emu = oracle.attention_fp8_emulated(q, k, v8, None, None, vd, scale)
    assert int(oracle.ulp_distance(emu, bf(g["fp8pv_out"])).max()) <= 1


# ------------------------------------------------------------------ GPU: kernels


@pytest.mark.gpu
def test_kernels_match_golden_pointwise(g, pkg, device):
    def dev(name):
        return bf(g[name]).to(device)

    for W in (128, 5376):
        x = dev(f"rms{W}_x")
        out = torch.empty_like(x)
        pkg.make_rms(width=W)(x, dev(f"rms{W}_w"), 1e-5, out)
        torch.cuda.synchronize()
        assert_bitwise(out, bf(g[f"rms{W}_out"]), f"rms{W}")
    x = dev("mod_x")
    out = torch.empty_like(x)
    pkg.make_rms_modulate()(x, dev("mod_w"), 1e-6, dev("mod_scale").expand_as(x), dev("mod_shift").expand_as(x), out)
    torch.cuda.synchronize()
    assert_bitwise(out, bf(g["mod_out"]), "rms_modulate")
    x = dev("gres_x")
    out = torch.empty_like(x)
    pkg.make_gated_residual()(x, dev("gres_gate").expand_as(x), dev("gres_y"), out)
    torch.cuda.synchronize()
    assert_bitwise(out, bf(g["gres_out"]), "gated_residual")
    x = dev("fused_x")
    res, out = torch.empty_like(x), torch.empty_like(x)
    pkg.make_gated_residual_rms_modulate()(x, dev("fused_gate").expand_as(x), dev("fused_y"), dev("fused_w"), 1e-6,
                                           dev("fused_scale").expand_as(x), dev("fused_shift").expand_as(x), res,
                                           out)
    torch.cuda.synchronize()
    assert_bitwise(res, bf(g["fused_residual"]), "fused residual")
    assert_bitwise(out, bf(g["fused_out"]), "fused out")
    up = dev("swiglu_up")
    out = torch.empty_like(up)
    pkg.make_swiglu()(up, dev("swiglu_gate"), out)
    torch.cuda.synchronize()
    assert_bitwise(out, bf(g["swiglu_out"]), "swiglu")


@pytest.mark.gpu
def test_kernels_match_golden_rope(g, pkg, oracle, device):
    pos = torch.from_numpy(g["cache_pos"]).to(device)
    power = torch.from_numpy(g["cache_power"]).to(device)
    T = pos.shape[0]
    cos = torch.empty(T, 48, dtype=BF, device=device)
    sin = torch.empty_like(cos)
    pkg.make_rope_cache()(pos, power, cos, sin)
    torch.cuda.synchronize()
    cache = bf(g["cache_out"])
    # cosf/sinf on the device vs torch's CPU cos/sin: within 1 bf16 ulp.
    assert int(oracle.ulp_distance(torch.cat([cos, sin], dim=1).cpu(), cache).max()) <= 1
    cos, sin = cache[:, :48].contiguous().to(device), cache[:, 48:].contiguous().to(device)
    x = bf(g["rope_x"]).to(device)
    out = torch.empty_like(x)
    pkg.make_rope()(x, cos, sin, out)
    torch.cuda.synchronize()
    assert_bitwise(out, bf(g["rope_out"]), "rope")
    x, w = bf(g["qk_x"]).to(device), bf(g["qk_w"]).to(device)
    out = torch.empty_like(x)
    pkg.make_qk_norm_rope()(x, w, 1e-6, cos, sin, out)
    torch.cuda.synchronize()
    assert_bitwise(out, bf(g["qk_out"]), "qk_norm_rope")
    out = torch.empty_like(x)
    pkg.make_qk_norm_rope_interleaved()(x, w, 1e-6, bf(g["qki_cos"]).to(device), bf(g["qki_sin"]).to(device), out)
    torch.cuda.synchronize()
    assert_bitwise(out, bf(g["qki_out"]), "qk interleaved")


@pytest.mark.gpu
def test_kernels_match_golden_attention(g, pkg, device):
    q, k, v = (bf(g[n]).to(device) for n in ("attn_q", "attn_k", "attn_v"))
    scale = float(g["attn_scale"])
    out = torch.empty_like(q)
    pkg.make_attention()(q, k, v, scale, out)
    torch.cuda.synchronize()
    mx, rel = attention_error(out.cpu(), torch.from_numpy(g["attn_out"]))
    assert mx <= 2e-2 and rel <= 1e-2, (mx, rel)
    v8, vd = pkg.quantize_fp8_per_head(v, transposed=True)
    torch.cuda.synchronize()
    assert np.array_equal(v8.cpu().contiguous().view(torch.uint8).numpy(), g["fp8_v_codes"])
    assert np.array_equal(vd.cpu().numpy(), g["fp8_v_descale"])
    out8 = torch.empty_like(q)
    pkg.make_attention_fp8pv()(q, k, v8, vd, scale, out8)
    torch.cuda.synchronize()
    _, rel8 = attention_error(out8.cpu(), bf(g["fp8pv_out"]))
    print(f"EMU golden fp8pv: rel {rel8:.3e}", flush=True)
    assert rel8 <= 1e-3, rel8  # the fp8pv kernel-to-emulation distance measures at most 3.4e-4

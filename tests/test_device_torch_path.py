"""The kernels against the reference's own torch compositions evaluated on the
GPU, as the reference checks them (tools/bench_h3_ops.py:74-78 compares each
kernel bitwise with its torch composition on device tensors; its RoPE table
probe, tools/probe_rope_cache.py:33-61, reports ALL_BITWISE against torch on
the device).

The compositions below restate tools/bench_h3_ops.py:81-113,251-254 and
tools/probe_rope_cache.py:11-23 and run on cuda tensors, so they use the
device's rsqrt, exp, cos and sin (ROCm's ocml) where the CPU oracle uses
exactly rounded mathematics. Each test counts the elements that differ and
their bf16 ulp distance and prints the counts. Measured on an MI355X every
count is zero, so the element-wise tests require bitwise equality; the row
reductions allow the rows where the device's own fp32 summation order could
round a mean differently (none occur on the configuration's inputs).
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
F32 = torch.float32


# --------------------------------------------- the reference's compositions

def rms_norm_reference(x, weight, eps):
    """tools/bench_h3_ops.py:81-88, on x's device."""
    squared = (x.float() * x.float()).to(x.dtype)
    mean = (squared.float().sum(-1, keepdim=True) / x.shape[-1]).to(x.dtype)
    variance = (mean.float() + torch.tensor(eps, dtype=F32, device=x.device)).to(x.dtype)
    reciprocal = torch.rsqrt(variance.float()).to(x.dtype)
    return ((x.float() * reciprocal.float()).to(x.dtype).float() * weight.float()).to(x.dtype)


def modulate_reference(normalized, scale, shift):
    """tools/bench_h3_ops.py:91-93."""
    factor = (scale.float() + 1.0).to(scale.dtype)
    return ((normalized.float() * factor.float()).to(normalized.dtype).float() + shift.float()).to(normalized.dtype)


def rope_reference(x, cos, sin):
    """tools/bench_h3_ops.py:96-106: rotate-half RoPE on the first 96 channels."""
    a, b, passthrough = x[..., :48], x[..., 48:96], x[..., 96:]
    c = cos.float().unsqueeze(-2)
    s = sin.float().unsqueeze(-2)
    ac = (a.float() * c).to(x.dtype)
    bs = (-b.float() * s).to(x.dtype)
    bc = (b.float() * c).to(x.dtype)
    a_s = (a.float() * s).to(x.dtype)
    return torch.cat([(ac.float() + bs.float()).to(x.dtype), (bc.float() + a_s.float()).to(x.dtype), passthrough],
                     dim=-1)


def rotary_cache_reference(position_ids, rope_freq_dim=16, rope_theta=10000.0):
    """tools/bench_h3_ops.py:109-113 (tools/probe_rope_cache.py:11-16)."""
    inverse = 1.0 / (rope_theta ** (torch.arange(0, 2 * rope_freq_dim, 2, dtype=F32, device=position_ids.device)
                                    / (2 * rope_freq_dim)))
    frequencies = (position_ids.float().unsqueeze(-1) * inverse.view(1, 1, -1)).flatten(1)
    return torch.cat((frequencies.cos(), frequencies.sin()), dim=-1).to(BF)


def device_power(device, rope_freq_dim=16, rope_theta=10000.0):
    """tools/probe_rope_cache.py:19-23: theta ** (2k / 32) with the device's powf."""
    exponent = torch.tensor([2 * k / (2 * rope_freq_dim) for k in range(rope_freq_dim)], dtype=F32, device=device)
    return torch.full_like(exponent, rope_theta) ** exponent


def swiglu_reference(up, gate):
    """tools/bench_h3_ops.py:251-254."""
    value = gate.float()
    activated = (value / (1.0 + torch.exp(-value))).to(up.dtype)
    return up * activated


def _ulps(oracle, a, b):
    return oracle.ulp_distance(a.cpu(), b.cpu())


def _report(oracle, what, got, want, bar=0):
    d = _ulps(oracle, got, want)
    n, worst = int((d > 0).sum()), int(d.max())
    print(f"{what}: {n} of {d.numel()} elements differ from the device torch path, max {worst} ulp", flush=True)
    assert worst <= bar, (what, n, worst)
    return n, worst


# --------------------------------------------- every variance through rsqrt

def _variance_rows():
    """One 128-wide row per non-negative bf16 variance V = 1.m 2^E, E in
    [-126, 120] (31,616 rows), plus a zero row: the row's elements are powers
    of two whose squares sum to exactly 128 V (each set bit 2^j of 128 V is one
    element 2^(j/2), or two elements 2^((j-1)/2) when j is odd), so every
    square, partial sum and mean is exact in any summation order, and with
    eps = 0 the variance is V itself. Each output element is then x_i times
    the bf16 reciprocal, exactly."""
    rows = []
    for e in range(-126, 121):
        for m in range(128):
            total = (128 + m) << (e + 7 + 126 - 7)  # 128 V in units of 2^-126, an integer
            row = []
            j = 0
            while total:
                if total & 1:
                    p = j - 126
                    if p % 2 == 0:
                        row.append(2.0 ** (p // 2))
                    else:
                        row += [2.0 ** ((p - 1) // 2)] * 2
                total >>= 1
                j += 1
            rows.append(row + [0.0] * (128 - len(row)))
    rows.append([0.0] * 128)
    return torch.tensor(rows, dtype=torch.float64).to(BF)


def test_rsqrt_over_every_variance(pkg, oracle, device):
    """bf16(rsqrt(V)) for every non-negative normal bf16 variance V from
    2^-126 to 2^121 and V = 0, through both reciprocal paths of the library --
    the RMS family's IEEE sqrt-then-divide (make_rms, W = 128) and the head-row
    kernels' table (make_qk_norm_rope with cos = 1, sin = 0, where RoPE is the
    identity) -- against rms_norm_reference (then rope_reference) on the device,
    which calls the device's torch.rsqrt. Every variance's row is checked
    element by element (x_i times the reciprocal). Measured on an MI355X:
    bitwise on all 31,617 rows for both paths."""
    x = _variance_rows()
    T = x.shape[0]
    xd = x.to(device)
    w = torch.ones(128, dtype=BF, device=device)
    # The variances the rows are built for are what the composition forms.
    var = (((xd.float() * xd.float()).to(BF).float().sum(-1) / 128).to(BF))
    assert int(torch.unique(var[:-1].view(torch.int16)).numel()) == T - 1
    want = rms_norm_reference(xd.view(1, T, 128), w, 0.0)
    out = torch.empty(1, T, 128, dtype=BF, device=device)
    pkg.make_rms(width=128)(xd.view(1, T, 128), w, 0.0, out)
    torch.cuda.synchronize()
    _report(oracle, "rms (IEEE reciprocal), every variance", out, want)
    cos = torch.ones(T, 48, dtype=BF, device=device)
    sin = torch.zeros(T, 48, dtype=BF, device=device)
    head = torch.empty(T, 1, 1, 128, dtype=BF, device=device)
    pkg.make_qk_norm_rope()(xd.view(T, 1, 1, 128), w, 0.0, cos, sin, head)
    torch.cuda.synchronize()
    want_head = rope_reference(rms_norm_reference(xd.view(T, 1, 1, 128), w, 0.0), cos.view(T, 1, 48),
                               sin.view(T, 1, 48))
    _report(oracle, "head rows (reciprocal table), every variance", head, want_head)


# --------------------------------------------- SwiGLU over every gate

def test_swiglu_every_gate_against_device_exp(pkg, oracle, device):
    """All 65,536 bf16 gate values with up = 1, -1, 0.125 and 3, against
    swiglu_reference on the device (its torch.exp is the device's). The kernel
    computes exp with its own short reduction and a correctly rounded division
    (exhaustively equal to the exactly rounded CPU oracle). Measured on an
    MI355X: bitwise for every gate and up value."""
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(BF).view(1, 256, 256).to(device)
    for up_value in (1.0, -1.0, 0.125, 3.0):
        up = torch.full_like(bits, up_value)
        out = torch.empty_like(bits)
        pkg.make_swiglu()(up, bits, out)
        torch.cuda.synchronize()
        _report(oracle, f"swiglu up={up_value}, every gate", out, swiglu_reference(up, bits))


# --------------------------------------------- the RoPE table

@pytest.mark.parametrize("kind", ["grid", "integer", "uniform", "fine", "fine64", "int64"])
def test_rope_cache_against_device_torch(pkg, oracle, device, kind):
    """The position sets of tools/probe_rope_cache.py:54-59 (same sizes, seed
    0) and the configuration's 8 x 32 x 32 grid, the power table from the
    device's powf as in the probe, against rotary_cache_reference on the
    device. The reference reports this comparison bitwise for its kernel
    (docs/技术报告-算子优化.md:87-89). Measured on an MI355X: bitwise on every
    set."""
    torch.manual_seed(0)
    if kind == "grid":
        pos = oracle.grid_positions(8, 32, 32).to(device)
    elif kind == "integer":
        pos = torch.randint(0, 4096, (50000, 3), device=device).float()
    elif kind == "uniform":
        pos = torch.rand(50000, 3, device=device) * 2000 - 100
    elif kind == "fine":
        pos = torch.arange(150000, device=device).float().view(-1, 3) / 37
    elif kind == "fine64":
        pos = torch.arange(150000, device=device).double().view(-1, 3) / 37
    else:
        pos = torch.randint(-5000, 5000, (50000, 3), device=device)
    want = rotary_cache_reference(pos)
    cache = torch.empty(pos.shape[0], 96, dtype=BF, device=device)
    pkg.make_rope_cache()(pos.double().contiguous(), device_power(device), cache[:, :48], cache[:, 48:])
    torch.cuda.synchronize()
    _report(oracle, f"rope table {kind}", cache, want)


# --------------------------------------------- the chain at configuration size

def test_chain_config_size_against_device_torch(pkg, oracle, device):
    """RMSNorm + AdaLN, gated residual and the fused gated residual + RMSNorm +
    AdaLN at [1, 8192, 7168] (seeded as the configuration), against the
    compositions on the device. The device's torch sum over a row runs in its
    own order, so a row whose two fp32 sums round to different bf16 means can
    differ (by at most a few ulp); every other element is bitwise. Measured on
    an MI355X: every row bitwise (0 of 8192 differ, for both fused ops)."""
    gen = torch.Generator(device=device).manual_seed(0)
    S, C = 8192, 7168

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=gen, device=device) * scale).to(BF)

    x = rnd(1, S, C)
    shift, scale, gate = (rnd(1, 1, C, scale=0.1) for _ in range(3))
    y = rnd(1, S, C)
    w = rnd(C, scale=0.1) + 1
    out = torch.empty_like(x)
    pkg.make_rms_modulate()(x, w, 1e-6, scale.expand(1, S, C), shift.expand(1, S, C), out)
    want = modulate_reference(rms_norm_reference(x, w, 1e-6), scale, shift)
    torch.cuda.synchronize()
    d = _ulps(oracle, out, want)
    rows = int((d.amax(-1) > 0).sum())
    print(f"rms_modulate: {rows} of {S} rows differ, {int((d > 0).sum())} elements, max {int(d.max())} ulp,"
          f" {int((d > 1).sum())} beyond 1 ulp", flush=True)
    assert rows <= S // 50 and float((d > 1).float().mean()) < 1e-3
    residual, fused = torch.empty_like(x), torch.empty_like(x)
    pkg.make_gated_residual()(x, gate.expand(1, S, C), y, residual)
    torch.cuda.synchronize()
    want_res = (x.float() + (gate.float() * y.float()).to(BF).float()).to(BF)  # tools/h3_pointwise.py:121-124
    _report(oracle, "gated_residual", residual, want_res)
    res2 = torch.empty_like(x)
    pkg.make_gated_residual_rms_modulate()(x, gate.expand(1, S, C), y, w, 1e-6, scale.expand(1, S, C),
                                           shift.expand(1, S, C), res2, fused)
    torch.cuda.synchronize()
    _report(oracle, "fused gated residual (residual output)", res2, want_res)
    d = _ulps(oracle, fused, modulate_reference(rms_norm_reference(want_res, w, 1e-6), scale, shift))
    rows = int((d.amax(-1) > 0).sum())
    print(f"gated_residual_rms_modulate: {rows} of {S} rows differ, max {int(d.max())} ulp,"
          f" {int((d > 1).sum())} elements beyond 1 ulp", flush=True)
    assert rows <= S // 50 and float((d > 1).float().mean()) < 1e-3

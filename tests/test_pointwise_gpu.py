"""GPU parity of the pointwise kernels against the CPU oracle.

Bar: bitwise equality with the oracle's fixed-order composition (the reduction
order the kernels use). Against the literal torch composition (torch's own
sum order) every row whose bf16 mean agrees is bitwise equal, and the rows where
the two fp32 sums round to different bf16 means ("tie rows") stay within 2 ulp;
the count of tie rows is reported. Layouts follow the reference's own checks:
packed / offset views (tools/verify_h3_pointwise_native.py:26-56), broadcast
modulation rows (patches/InfiniLM.patch:1360-1364), permuted send buffers
(tools/probe_qk_norm_rope.py:20-44, tools/bench_h3_ops.py:129-153).
"""
from __future__ import annotations

import pytest
import torch

from conftest import assert_bitwise

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _gen(seed):
    return torch.Generator("cpu").manual_seed(seed)


def _randn(gen, *shape, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(BF)


def _row_ties(oracle, x, eps):
    """Rows whose bf16 mean differs between the fixed and the torch sum order."""
    v = x.float()
    sq = oracle.rb(v * v)
    fixed = oracle.rb(oracle.fixed_order_sum(sq) / v.shape[-1])
    loose = oracle.rb(sq.sum(-1) / v.shape[-1])
    return fixed != loose


def _check_torch_order(oracle, out_gpu, ref_torch, ties, what):
    """Against the literal torch composition (torch's own sum order): rows whose
    fp32 sums round to the same bf16 mean are bitwise equal; the tie rows
    (the two orders round the mean differently) are counted and reported, may
    differ by up to 2 ulp, and must stay rare (under 2% of the rows)."""
    d = oracle.ulp_distance(out_gpu.cpu(), ref_torch)
    non_tie = ~ties
    assert int(d[non_tie].max()) == 0 if non_tie.any() else True, f"{what}: non-tie rows differ from torch order"
    n_ties, rows = int(ties.sum()), ties.numel()
    beyond_one = int((d > 1).sum())
    print(f"{what}: {n_ties} tie rows of {rows}; {beyond_one} of {d.numel()} elements beyond 1 ulp of the torch order")
    if ties.any():
        assert int(d[ties].max()) <= 2, f"{what}: tie rows {n_ties} max ulp {int(d[ties].max())}"
        assert n_ties <= max(1, rows // 50), f"{what}: {n_ties} tie rows of {rows}"


# ------------------------------------------------------------------ RMS family

RMS_CASES = [
    # (B, S, W, layout)
    (1, 257, 128, "contiguous"),
    (2, 129, 5376, "contiguous"),
    (1, 300, 7168, "contiguous"),
    (2, 129, 5376, "packed_offset"),      # inner stride 1, rows not 16-byte aligned -> generic path
    (2, 129, 7168, "packed_aligned"),     # strided rows, 16-byte aligned -> vector path
    (1, 33, 72, "contiguous"),
    (1, 65, 200, "contiguous"),           # 25 groups -> 32-lane rows (lane fold from xor 16)
    (2, 33, 384, "contiguous"),           # 48 groups -> 64-lane rows (lane fold from xor 32)
    (1, 31, 256, "packed_aligned"),       # exactly 32 lanes of one group each
    (1, 33, 100, "contiguous"),           # W % 8 != 0 -> generic path
    (1, 17, 1000, "transposed"),          # non-unit inner stride
    (1, 5, 8, "contiguous"),
    (1, 3, 32768, "contiguous"),
    (2, 40, 520, "contiguous"),           # one row per wave, two groups per lane
    (1, 70, 3072, "contiguous"),
    (1, 50, 8192, "contiguous"),          # largest one-row-per-wave width
    (1, 9, 8200, "contiguous"),           # smallest one-row-per-block width
    (1, 7, 16384, "packed_aligned"),
]


def _layout(gen, B, S, W, layout, scale=1.0):
    if layout == "contiguous":
        return _randn(gen, B, S, W, scale=scale)
    if layout == "packed_offset":
        return _randn(gen, B, S, 2 * W + 1, scale=scale)[..., 1:W + 1]
    if layout == "packed_aligned":
        return _randn(gen, B, S, 2 * W + 8, scale=scale)[..., 8:W + 8]
    if layout == "transposed":
        return _randn(gen, B, W, S, scale=scale).transpose(1, 2)
    raise ValueError(layout)


@pytest.mark.parametrize("B,S,W,layout", RMS_CASES)
@pytest.mark.parametrize("scale", [0.01, 1.0, 100.0, 10000.0])  # tools/probe_rms_rounding.py:23
def test_rms(pkg, oracle, device, B, S, W, layout, scale):
    gen = _gen(W + S)
    x = _layout(gen, B, S, W, layout, scale)
    w = _randn(gen, 2 * W)[::2]  # strided weight (tools/verify_h3_pointwise_native.py:37)
    out = torch.empty(B, S, W, dtype=BF, device=device)
    pkg.make_rms(width=W)(x.to(device), w.to(device), 1e-5, out)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.rms_norm(x, w, 1e-5), f"rms W={W} {layout}")
    ties = _row_ties(oracle, x, 1e-5)
    _check_torch_order(oracle, out, oracle.rms_norm(x, w, 1e-5, order="torch"), ties, "rms torch-order")


@pytest.mark.parametrize("B,S,W,layout", [c for c in RMS_CASES if c[2] <= 8192])
@pytest.mark.parametrize("broadcast", [False, True])
def test_rms_modulate(pkg, oracle, device, B, S, W, layout, broadcast):
    gen = _gen(3 * W + S)
    x = _layout(gen, B, S, W, layout, 8.0)
    w = _randn(gen, W)
    if broadcast:  # one AdaLN row per batch entry, broadcast over S
        scale = _randn(gen, B, 1, W, scale=0.5).expand(B, S, W)
        shift = _randn(gen, B, 1, W, scale=0.5).expand(B, S, W)
    else:
        table = _randn(gen, B, S, 6 * W, scale=0.5)
        shift, scale = table[..., :W], table[..., W:2 * W]
        scale[:, :3] = -1.0  # modulation edge of tools/verify_h3_pointwise_native.py:118
    out = torch.empty(B, S, W, dtype=BF, device=device)
    pkg.make_rms_modulate()(x.to(device), w.to(device), 1e-6, scale.to(device), shift.to(device), out)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.rms_modulate(x, w, 1e-6, scale, shift), f"rms_modulate W={W} {layout}")


@pytest.mark.parametrize("B,S,W", [(1, 257, 5376), (2, 65, 7168), (1, 33, 100), (1, 64, 128)])
@pytest.mark.parametrize("broadcast_gate", [False, True])
def test_gated_residual(pkg, oracle, device, B, S, W, broadcast_gate):
    gen = _gen(5 * W + S)
    x = _randn(gen, B, S, W, scale=8.0)
    y = _randn(gen, B, S, W)
    gate = (_randn(gen, 1, 1, W, scale=0.5).expand(B, S, W) if broadcast_gate
            else _randn(gen, B, S, W, scale=0.5))
    out = torch.empty(B, S, W, dtype=BF, device=device)
    pkg.make_gated_residual()(x.to(device), gate.to(device), y.to(device), out)
    torch.cuda.synchronize()
    ref = oracle.gated_residual(x, gate, y)
    assert_bitwise(out, ref, f"gated_residual W={W}")
    # The reference's eager form: torch.add(x, torch.mul(gate, y)) in bf16 (tools/bench_h3_ops.py:215).
    assert_bitwise(out, torch.add(x, torch.mul(gate, y)), "gated_residual vs torch bf16 ops")


@pytest.mark.parametrize("B,S,W", [(1, 257, 5376), (2, 65, 7168), (1, 33, 100), (1, 64, 128), (3, 19, 2048),
                                   (1, 65, 200), (2, 33, 384)])
@pytest.mark.parametrize("broadcast", [False, True])
def test_gated_residual_rms_modulate(pkg, oracle, device, B, S, W, broadcast):
    gen = _gen(7 * W + S)
    x = _randn(gen, B, S, W, scale=8.0)
    y = _randn(gen, B, S, W)
    if broadcast:  # AdaLN rows per batch entry, broadcast over S
        table = _randn(gen, B, 1, 6 * W, scale=0.5).expand(B, S, 6 * W)
    else:
        table = _randn(gen, B, S, 6 * W, scale=0.5)
    shift, scale, gate = table[..., :W], table[..., W:2 * W], table[..., 2 * W:3 * W]
    w = _randn(gen, W)
    residual = torch.empty(B, S, W, dtype=BF, device=device)
    out = torch.empty_like(residual)
    pkg.make_gated_residual_rms_modulate()(x.to(device), gate.to(device), y.to(device), w.to(device), 1e-6,
                                           scale.to(device), shift.to(device), residual, out)
    torch.cuda.synchronize()
    ref_res, ref_out = oracle.gated_residual_rms_modulate(x, gate, y, w, 1e-6, scale, shift)
    assert_bitwise(residual, ref_res, "fused residual")
    assert_bitwise(out, ref_out, "fused modulated")
    # Fused == unfused on the device (tools/probe_gated_residual.py:36-60).
    res2 = torch.empty_like(residual)
    out2 = torch.empty_like(residual)
    pkg.make_gated_residual()(x.to(device), gate.to(device), y.to(device), res2)
    pkg.make_rms_modulate()(res2, w.to(device), 1e-6, scale.to(device), shift.to(device), out2)
    torch.cuda.synchronize()
    assert_bitwise(residual, res2, "fused vs unfused residual")
    assert_bitwise(out, out2, "fused vs unfused modulated")


# ------------------------------------------------------------------ SwiGLU

def test_swiglu_exhaustive_gate(pkg, oracle, device):
    """Every bf16 gate value, with up = 1, -1, 2^-3 and 3 (tools/probe_swiglu.py)."""
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(BF).view(1, 256, 256)
    for up_value in (1.0, -1.0, 0.125, 3.0):
        up = torch.full_like(bits, up_value)
        out = torch.empty(1, 256, 256, dtype=BF, device=device)
        pkg.make_swiglu()(up.to(device), bits.to(device), out)
        torch.cuda.synchronize()
        assert_bitwise(out, oracle.swiglu(up, bits), f"swiglu exhaustive up={up_value}")


@pytest.mark.parametrize("S,F", [(129, 14336), (65, 18432), (33, 100)])
@pytest.mark.parametrize("scale", [1.0, 4.0, 16.0])
def test_swiglu_packed(pkg, oracle, device, S, F, scale):
    gen = _gen(F + S)
    packed = _randn(gen, 1, S, 2 * F, scale=scale)  # up, gate = halves (tools/bench_h3_ops.py:246-247)
    up, gate = packed[..., :F], packed[..., F:]
    out = torch.empty(1, S, F, dtype=BF, device=device)
    pd = packed.to(device)
    pkg.make_swiglu()(pd[..., :F], pd[..., F:], out)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.swiglu(up, gate), f"swiglu F={F}")


# ------------------------------------------------------------------ RoPE

@pytest.mark.parametrize("S,H", [(17, 28), (257, 56), (64, 14)])
def test_rope(pkg, oracle, device, S, H):
    gen = _gen(S * H)
    x = _randn(gen, S, H, 385)[..., 1:129]   # offset view -> generic path (tools/verify_h3_pointwise_native.py:53)
    angles = _randn(gen, S, 96)
    cos, sin = angles[:, :48], angles[:, 48:]
    out = torch.empty(S, H, 128, dtype=BF, device=device)
    pkg.make_rope()(x.to(device), cos.to(device), sin.to(device), out)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.rope_rotate_half(x, cos[:, None, :], sin[:, None, :]), "rope offset")
    xc = x.contiguous()
    pkg.make_rope()(xc.to(device), cos.to(device), sin.to(device), out)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.rope_rotate_half(xc, cos[:, None, :], sin[:, None, :]), "rope contiguous")


@pytest.mark.parametrize("tokens,ranks,heads", [(5725, 4, 7), (257, 1, 14), (33, 2, 3)])
def test_qk_norm_rope_send_buffer(pkg, oracle, device, tokens, ranks, heads):
    """Strided [T, P, Hs, 128] view of a fused QKV projection written into a
    permuted [P, T, Hs, 128] send buffer (tools/probe_qk_norm_rope.py:20-44)."""
    gen = _gen(tokens + ranks)
    n = ranks * heads
    projected = _randn(gen, tokens, 3, n, 128, scale=3.0)
    weight = _randn(gen, 128)
    table = _randn(gen, tokens, 96)
    cos, sin = table[:, :48], table[:, 48:]
    pd = projected.to(device)
    x4 = pd[:, 0].view(tokens, ranks, heads, 128)
    send = torch.zeros(ranks, tokens, heads, 128, dtype=BF, device=device)
    td = table.to(device)
    pkg.make_qk_norm_rope()(x4, weight.to(device), 1e-5, td[:, :48], td[:, 48:], send.permute(1, 0, 2, 3))
    torch.cuda.synchronize()
    ref = oracle.qk_norm_rope(projected[:, 0].view(tokens, ranks, heads, 128), weight, 1e-5, cos, sin)
    assert_bitwise(send.permute(1, 0, 2, 3), ref, "qk_norm_rope send buffer")
    # The raw 12-argument form (caller != "torch").
    raw = pkg.make_qk_norm_rope(caller="hip")
    send2 = torch.zeros_like(send)
    o = send2.permute(1, 0, 2, 3)
    wd = weight.to(device)
    raw(x4, x4, x4, wd, wd, wd, 1e-5, td[:, :48], td[:, 48:], o, o, o)
    torch.cuda.synchronize()
    assert_bitwise(send2, send, "raw 12-argument form")


def test_qk_norm_rope_matches_rms_then_rope(pkg, device):
    """Fused == h3_rms_exact(128) then h3_rope_exact on the device
    (tools/probe_qk_norm_rope.py:38-44)."""
    gen = _gen(11)
    T, H = 300, 14
    x = _randn(gen, T, H, 128, scale=3.0).to(device)
    w = _randn(gen, 128).to(device)
    table = _randn(gen, T, 96).to(device)
    normed = torch.empty_like(x)
    pkg.make_rms(width=128)(x, w, 1e-6, normed)
    rotated = torch.empty_like(x)
    pkg.make_rope()(normed, table[:, :48], table[:, 48:], rotated)
    fused = torch.empty(T, 1, H, 128, dtype=BF, device=device)
    pkg.make_qk_norm_rope()(x.view(T, 1, H, 128), w, 1e-6, table[:, :48], table[:, 48:], fused)
    torch.cuda.synchronize()
    assert_bitwise(fused.view(T, H, 128), rotated, "fused vs unfused")


@pytest.mark.parametrize("eps", [1e-6, 0.0])
def test_head_rows_across_magnitudes(pkg, oracle, device, eps):
    """Head rows scaled by 2^-70 .. 2^60 (var over every exponent parity,
    subnormal var at the small end, infinite squares at the large end) and zero
    rows (var = eps; 0 with eps = 0, so 0 * inf = NaN as in the reference), for
    the three head-row kernels: rotate-half, interleaved and the q/k/v pack."""
    gen = _gen(21)
    T, H = 139, 4
    x = torch.randn(T, 1, H, 128, generator=gen)
    scales = 2.0 ** torch.arange(-70, 61, dtype=torch.float32)
    x = x * scales[torch.arange(T * H) % scales.numel()].view(T, 1, H, 1)
    x[::17, :, 1] = 0.0
    x = x.to(BF)
    w = _randn(gen, 128)
    table48, table64 = _randn(gen, T, 96), _randn(gen, T, 128)
    xd, wd = x.to(device), w.to(device)
    out = torch.empty_like(xd)
    pkg.make_qk_norm_rope()(xd, wd, eps, table48[:, :48].to(device), table48[:, 48:].to(device), out)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.qk_norm_rope(x, w, eps, table48[:, :48], table48[:, 48:]), "rotate-half")
    out = torch.empty_like(xd)
    pkg.make_qk_norm_rope_interleaved()(xd, wd, eps, table64[:, :64].to(device), table64[:, 64:].to(device), out)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.qk_norm_rope_interleaved(x, w, eps, table64[:, :64], table64[:, 64:]), "interleaved")
    outs = [torch.empty_like(xd) for _ in range(3)]
    positions = torch.arange(T)
    pkg.make_qkv_norm_rope_pack()(xd, xd, xd, wd, wd, eps, table48.to(device), positions.to(device), *outs)
    torch.cuda.synchronize()
    q_ref, _, _ = oracle.qkv_norm_rope_pack(x, x, x, w, w, eps, table48, positions)
    assert_bitwise(outs[0], q_ref, "q/k/v pack")
    assert_bitwise(outs[1], q_ref, "q/k/v pack (k)")


def test_head_rows_special_values(pkg, oracle, device):
    """Head rows holding +inf, -inf or NaN (the whole row's sum, and so every
    channel, follows IEEE: inf * 0 = NaN), rows of bf16 subnormals, rows whose
    squares overflow (2^70) and zero rows, through rotate-half, interleaved, q
    and k in one launch (different rows in each) and the q/k/v pack, bitwise
    against the oracle (NaN == NaN)."""
    gen = _gen(57)
    T, H = 64, 4
    x = torch.randn(T, 1, H, 128, generator=gen)
    x[1, 0, 0, 5] = float("inf")
    x[2, 0, 1, 77] = float("-inf")
    x[3, 0, 2, 100] = float("nan")
    x[4, 0, 3] = torch.randn(128, generator=gen) * 2.0 ** -130  # bf16 subnormals
    x[5, 0, 0] = torch.randn(128, generator=gen) * 2.0 ** 70  # squares overflow
    x[6, 0, 1] = 0.0
    x[7, 0, 2, 64:] = float("inf")  # the pass-through and rotated halves of one row
    x = x.to(BF)
    k = torch.flip(x, dims=(0,)).contiguous()  # the special rows at other tokens for k
    w = _randn(gen, 128)
    w2 = _randn(gen, 128)
    table48, table64 = _randn(gen, T, 96), _randn(gen, T, 128)
    xd, kd, wd, w2d = x.to(device), k.to(device), w.to(device), w2.to(device)
    out = torch.empty_like(xd)
    pkg.make_qk_norm_rope()(xd, wd, 1e-6, table48[:, :48].to(device), table48[:, 48:].to(device), out)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.qk_norm_rope(x, w, 1e-6, table48[:, :48], table48[:, 48:]), "rotate-half")
    c64, s64 = table64[:, :64], table64[:, 64:]
    ref_q = oracle.qk_norm_rope_interleaved(x, w, 1e-6, c64, s64)
    ref_k = oracle.qk_norm_rope_interleaved(k, w2, 1e-6, c64, s64)
    out = torch.empty_like(xd)
    pkg.make_qk_norm_rope_interleaved()(xd, wd, 1e-6, c64.to(device), s64.to(device), out)
    torch.cuda.synchronize()
    assert_bitwise(out, ref_q, "interleaved")
    qo, ko = torch.empty_like(xd), torch.empty_like(kd)
    pkg.make_qk_norm_rope_interleaved_qk()(xd, kd, wd, w2d, 1e-6, c64.to(device), s64.to(device), qo, ko)
    torch.cuda.synchronize()
    assert_bitwise(qo, ref_q, "q of q + k")
    assert_bitwise(ko, ref_k, "k of q + k")
    outs = [torch.empty_like(xd) for _ in range(3)]
    positions = torch.arange(T)
    pkg.make_qkv_norm_rope_pack()(xd, kd, xd, wd, w2d, 1e-6, table48.to(device), positions.to(device), *outs)
    torch.cuda.synchronize()
    q_ref, k_ref, v_ref = oracle.qkv_norm_rope_pack(x, k, x, w, w2, 1e-6, table48, positions)
    assert_bitwise(outs[0], q_ref, "q/k/v pack (q)")
    assert_bitwise(outs[1], k_ref, "q/k/v pack (k)")
    assert_bitwise(outs[2], v_ref, "q/k/v pack (v)")


def test_qk_norm_rope_interleaved(pkg, oracle, device):
    q, k, w_q, w_k, pos = oracle.qk_norm_rope_inputs(T=2048, H=14, seed=3)
    cos, sin = oracle.rope_table_interleaved(pos)
    kern = pkg.make_qk_norm_rope_interleaved()
    for x, w in ((q, w_q), (k, w_k)):
        x4 = x[0].view(2048, 1, 14, 128)
        out = torch.empty(2048, 1, 14, 128, dtype=BF, device=device)
        kern(x4.to(device), w.to(device), 1e-6, cos.to(device), sin.to(device), out)
        torch.cuda.synchronize()
        assert_bitwise(out, oracle.qk_norm_rope_interleaved(x4, w, 1e-6, cos, sin), "interleaved")


@pytest.mark.parametrize("stride", [(1 << 24) - 128, (1 << 24) + 128])
def test_head_rows_token_stride_near_2_24(pkg, oracle, device, stride):
    """Token strides on both sides of the head-row kernels' 32-bit offset
    limit (strides below 2^24, offsets below 2^31: 24-bit multiplies): just
    below it the largest offset is 127 x (2^24 - 128) + 1791, about 2^31 -
    1.7e7; just above it the launch takes the 64-bit offset path. One tensor
    and q + k in one launch, bitwise against the oracle."""
    T, H = 128, 14
    q, k, w_q, w_k, pos = oracle.qk_norm_rope_inputs(T=T, H=H, seed=11)
    cos, sin = oracle.rope_table_interleaved(pos)
    cd, sd = cos.to(device), sin.to(device)
    refs = (oracle.qk_norm_rope_interleaved(q[0].view(T, 1, H, 128), w_q, 1e-6, cos, sin),
            oracle.qk_norm_rope_interleaved(k[0].view(T, 1, H, 128), w_k, 1e-6, cos, sin))

    def strided(src):
        buf = torch.empty(T, stride, dtype=BF, device=device)
        if src is not None:
            buf[:, :H * 128] = src.reshape(T, H * 128).to(device)
        return buf, buf[:, :H * 128].view(T, 1, H, 128)

    qbuf, qv = strided(q)
    obuf, ov = strided(None)
    pkg.make_qk_norm_rope_interleaved()(qv, w_q.to(device), 1e-6, cd, sd, ov)
    torch.cuda.synchronize()
    assert_bitwise(ov.cpu(), refs[0], f"q, token stride {stride}")
    kbuf, kv = strided(k)
    o2buf, o2v = strided(None)
    pkg.make_qk_norm_rope_interleaved_qk()(qv, kv, w_q.to(device), w_k.to(device), 1e-6, cd, sd, ov, o2v)
    torch.cuda.synchronize()
    assert_bitwise(ov.cpu(), refs[0], f"q of q + k, token stride {stride}")
    assert_bitwise(o2v.cpu(), refs[1], f"k of q + k, token stride {stride}")
    del qbuf, obuf, kbuf, o2buf


def test_qk_norm_rope_interleaved_qk_one_pass(pkg, oracle, device):
    """q and k in one launch: bitwise against the oracle per tensor, on the
    one-pass path (aligned rows) and on the two-launch fallback (head dim with
    element stride 2), with different q / k weights and P = 2 rank-split views."""
    q, k, w_q, w_k, pos = oracle.qk_norm_rope_inputs(T=1024, H=14, seed=4)
    cos, sin = oracle.rope_table_interleaved(pos)
    kern = pkg.make_qk_norm_rope_interleaved_qk()
    q4, k4 = q[0].view(1024, 2, 7, 128), k[0].view(1024, 2, 7, 128)
    qd, kd = q4.to(device), k4.to(device)
    cd, sd, wqd, wkd = cos.to(device), sin.to(device), w_q.to(device), w_k.to(device)
    refs = (oracle.qk_norm_rope_interleaved(q4, w_q, 1e-6, cos, sin),
            oracle.qk_norm_rope_interleaved(k4, w_k, 1e-6, cos, sin))
    qo, ko = torch.empty_like(qd), torch.empty_like(kd)
    kern(qd, kd, wqd, wkd, 1e-6, cd, sd, qo, ko)
    torch.cuda.synchronize()
    assert_bitwise(qo, refs[0], "q (one pass)")
    assert_bitwise(ko, refs[1], "k (one pass)")
    qs = torch.zeros(1024, 2, 7, 256, dtype=BF, device=device)
    ks = torch.zeros_like(qs)
    qs[..., ::2] = qd
    ks[..., ::2] = kd
    qo2, ko2 = torch.empty_like(qd), torch.empty_like(kd)
    kern(qs[..., ::2], ks[..., ::2], wqd, wkd, 1e-6, cd, sd, qo2, ko2)
    torch.cuda.synchronize()
    assert_bitwise(qo2, refs[0], "q (strided fallback)")
    assert_bitwise(ko2, refs[1], "k (strided fallback)")


# ------------------------------------------------------------------ RoPE table

@pytest.mark.parametrize("kind", ["grid", "integer", "uniform", "fine", "fine64", "int64"])
def test_rope_cache(pkg, oracle, device, kind):
    """Position sets of tools/probe_rope_cache.py:37-55; within 1 bf16 ulp of
    the oracle (device ocml vs host libm cos/sin)."""
    gen = _gen(0)
    if kind == "grid":
        pos = oracle.grid_positions(8, 32, 32)
    elif kind == "integer":
        pos = torch.randint(0, 4096, (5000, 3), generator=gen).double()
    elif kind == "uniform":
        pos = (torch.rand(5000, 3, generator=gen) * 2000 - 100).double()
    elif kind == "fine":  # fp32 positions, widened to fp64 at the call (tools/probe_rope_cache.py:56)
        pos = (torch.arange(15000).float().view(-1, 3) / 37).double()
    elif kind == "fine64":
        pos = torch.arange(15000).double().view(-1, 3) / 37
    else:
        pos = torch.randint(-5000, 5000, (5000, 3), generator=gen).double()
    power = oracle.rope_powers()
    cache = torch.empty(pos.shape[0], 96, dtype=BF, device=device)
    pkg.make_rope_cache()(pos.to(device), power.to(device), cache[:, :48], cache[:, 48:])
    torch.cuda.synchronize()
    ref = oracle.rope_cache(pos, power)
    d = oracle.ulp_distance(cache.cpu(), ref)
    assert int(d.max()) <= 1, f"{kind}: max ulp {int(d.max())}"
    assert float((d == 0).float().mean()) > 0.999


# ------------------------------------------------------------------ full-size configurations

def test_qk_norm_rope_config_size(pkg, oracle, device):
    """q, k [1, 8192, 14, 128], weights N(1, 0.1), eps 1e-6, 8x32x32 grid:
    both RoPE layouts, bitwise against the oracle."""
    q, k, w_q, w_k, pos = oracle.qk_norm_rope_inputs()
    cos_i, sin_i = oracle.rope_table_interleaved(pos)
    cache = oracle.rope_cache(pos, oracle.rope_powers())
    for x, w in ((q, w_q), (k, w_k)):
        x4 = x[0].view(8192, 1, 14, 128)
        out = torch.empty(8192, 1, 14, 128, dtype=BF, device=device)
        pkg.make_qk_norm_rope_interleaved()(x4.to(device), w.to(device), 1e-6, cos_i.to(device),
                                            sin_i.to(device), out)
        torch.cuda.synchronize()
        assert_bitwise(out, oracle.qk_norm_rope_interleaved(x4, w, 1e-6, cos_i, sin_i), "cfg interleaved")
        cd = cache.to(device)
        pkg.make_qk_norm_rope()(x4.to(device), w.to(device), 1e-6, cd[:, :48], cd[:, 48:], out)
        torch.cuda.synchronize()
        assert_bitwise(out, oracle.qk_norm_rope(x4, w, 1e-6, cache[:, :48], cache[:, 48:]), "cfg rotate-half")
    # q and k in one pass.
    q4, k4 = q[0].view(8192, 1, 14, 128), k[0].view(8192, 1, 14, 128)
    qo = torch.empty(8192, 1, 14, 128, dtype=BF, device=device)
    ko = torch.empty_like(qo)
    pkg.make_qk_norm_rope_interleaved_qk()(q4.to(device), k4.to(device), w_q.to(device), w_k.to(device), 1e-6,
                                           cos_i.to(device), sin_i.to(device), qo, ko)
    torch.cuda.synchronize()
    assert_bitwise(qo, oracle.qk_norm_rope_interleaved(q4, w_q, 1e-6, cos_i, sin_i), "cfg q+k (q)")
    assert_bitwise(ko, oracle.qk_norm_rope_interleaved(k4, w_k, 1e-6, cos_i, sin_i), "cfg q+k (k)")


def test_chain_config_size(pkg, oracle, device):
    """AdaLN RMSNorm, SwiGLU, gated residual and the fused residual+norm at
    S = 8192, C = 7168, F = 18432 with broadcast [1, C] modulation vectors."""
    t = oracle.chain_inputs()
    S, C = t["x"].shape
    d = {k: v.to(device) for k, v in t.items()}
    bc = lambda v: v.view(1, 1, C).expand(1, S, C)  # noqa: E731
    out = torch.empty(1, S, C, dtype=BF, device=device)
    pkg.make_rms_modulate()(d["x"].view(1, S, C), d["w"], 1e-6, bc(d["scale"]), bc(d["shift"]), out)
    torch.cuda.synchronize()
    ref = oracle.rms_modulate(t["x"].view(1, S, C), t["w"], 1e-6, bc(t["scale"]), bc(t["shift"]))
    assert_bitwise(out, ref, "cfg rms_modulate")
    ties = _row_ties(oracle, t["x"].view(1, S, C), 1e-6)
    ref_t = oracle.rms_modulate(t["x"].view(1, S, C), t["w"], 1e-6, bc(t["scale"]), bc(t["shift"]), order="torch")
    _check_torch_order(oracle, out, ref_t, ties, "cfg rms_modulate torch-order")

    F = t["up"].shape[1]
    sw = torch.empty(1, S, F, dtype=BF, device=device)
    pkg.make_swiglu()(d["up"].view(1, S, F), d["gate_act"].view(1, S, F), sw)
    torch.cuda.synchronize()
    assert_bitwise(sw, oracle.swiglu(t["up"].view(1, S, F), t["gate_act"].view(1, S, F)), "cfg swiglu")

    gr = torch.empty(1, S, C, dtype=BF, device=device)
    pkg.make_gated_residual()(d["residual"].view(1, S, C), bc(d["gate"]), d["y"].view(1, S, C), gr)
    torch.cuda.synchronize()
    assert_bitwise(gr, oracle.gated_residual(t["residual"].view(1, S, C), bc(t["gate"]), t["y"].view(1, S, C)),
                   "cfg gated_residual")

    res = torch.empty(1, S, C, dtype=BF, device=device)
    fused = torch.empty_like(res)
    pkg.make_gated_residual_rms_modulate()(d["residual"].view(1, S, C), bc(d["gate"]), d["y"].view(1, S, C),
                                           d["w"], 1e-6, bc(d["scale"]), bc(d["shift"]), res, fused)
    torch.cuda.synchronize()
    r_ref, o_ref = oracle.gated_residual_rms_modulate(t["residual"].view(1, S, C), bc(t["gate"]),
                                                      t["y"].view(1, S, C), t["w"], 1e-6, bc(t["scale"]),
                                                      bc(t["shift"]))
    assert_bitwise(res, r_ref, "cfg fused residual")
    assert_bitwise(fused, o_ref, "cfg fused out")


@pytest.mark.parametrize("W", [7168, 5376])
def test_rms_family_special_values(pkg, oracle, device, W):
    """The wide RMS kernels (broadcast modulation: the staged row-per-wave
    kernel and the streamed gated kernel) and the gated residual on rows that
    reach every edge of the bf16 chain, bitwise against the oracle (NaN ==
    NaN): rows scaled by 2^-70 .. 2^60 (subnormal means at the small end,
    infinite squares at the large end), zero and negative-zero rows (var = eps),
    a row of bf16 subnormals, rows holding +inf, -inf or NaN, and modulation
    rows with scale = -1, gate = 0 and an infinite y under a zero gate
    (0 * inf = NaN, as in the reference); then the per-token (indexed)
    kernels on the same rows with three-row tables holding such entries and
    an infinite shift."""
    gen = _gen(W + 77)
    S = 70
    x = torch.randn(1, S, W, generator=gen)
    exps = torch.linspace(-70, 60, S).round()
    x = x * (2.0 ** exps).view(1, S, 1)
    x[0, 3] = 0.0
    x[0, 4] = -0.0
    x[0, 5] = torch.randn(W, generator=gen) * 2.0 ** -130  # bf16 subnormals
    x[0, 6, 17] = float("inf")
    x[0, 7, 100] = float("-inf")
    x[0, 8, 5] = float("nan")
    x = x.to(BF)
    y = _randn(gen, 1, S, W)
    y[0, 9, 33] = float("inf")
    w = _randn(gen, W)
    scale = _randn(gen, 1, 1, W, scale=0.5)
    shift = _randn(gen, 1, 1, W, scale=0.5)
    gate = _randn(gen, 1, 1, W, scale=0.5)
    scale[..., :64] = -1.0
    gate[..., 33] = 0.0
    scale, shift, gate = (t.expand(1, S, W) for t in (scale, shift, gate))
    xd, yd, wd = x.to(device), y.to(device), w.to(device)
    sd, hd, gd = scale.to(device), shift.to(device), gate.to(device)
    out = torch.empty(1, S, W, dtype=BF, device=device)
    pkg.make_rms_modulate()(xd, wd, 1e-6, sd, hd, out)
    torch.cuda.synchronize()
    assert_bitwise(out, oracle.rms_modulate(x, w, 1e-6, scale, shift), f"rms_modulate W={W}")
    res = torch.empty_like(out)
    pkg.make_gated_residual()(xd, gd, yd, res)
    torch.cuda.synchronize()
    assert_bitwise(res, oracle.gated_residual(x, gate, y), f"gated_residual W={W}")
    res2, out2 = torch.empty_like(out), torch.empty_like(out)
    pkg.make_gated_residual_rms_modulate()(xd, gd, yd, wd, 1e-6, sd, hd, res2, out2)
    torch.cuda.synchronize()
    ref_res, ref_out = oracle.gated_residual_rms_modulate(x, gate, y, w, 1e-6, scale, shift)
    assert_bitwise(res2, ref_res, f"fused residual W={W}")
    assert_bitwise(out2, ref_out, f"fused modulated W={W}")
    # The per-token (indexed) kernels on the same rows: three-row tables with
    # special entries, tokens cycling through the rows.
    tables = _randn(gen, 3, 3, W, scale=0.5)  # gate, scale, shift
    tables[:, 1, :64] = -1.0
    tables[0, 0, 33] = 0.0
    tables[2, 2, 7] = float("inf")
    g_t, s_t, h_t = tables[:, 0], tables[:, 1], tables[:, 2]
    index = (torch.arange(S) % 3).view(1, S)
    gtd, std_, htd, idd = g_t.to(device), s_t.to(device), h_t.to(device), index.to(device)
    out3 = torch.empty_like(out)
    pkg.make_rms_modulate_indexed()(xd, wd, 1e-6, std_, htd, idd, out3)
    res3 = torch.empty_like(out)
    pkg.make_gated_residual_indexed()(xd, gtd, yd, idd, res3)
    res4, out4 = torch.empty_like(out), torch.empty_like(out)
    pkg.make_gated_residual_rms_modulate_indexed()(xd, gtd, yd, wd, 1e-6, std_, htd, idd, res4, out4)
    torch.cuda.synchronize()
    assert_bitwise(out3, oracle.rms_modulate_indexed(x, w, 1e-6, s_t, h_t, index), f"indexed rms_modulate W={W}")
    assert_bitwise(res3, oracle.gated_residual_indexed(x, g_t, y, index), f"indexed gated_residual W={W}")
    ref_res, ref_out = oracle.gated_residual_rms_modulate_indexed(x, g_t, y, w, 1e-6, s_t, h_t, index)
    assert_bitwise(res4, ref_res, f"indexed fused residual W={W}")
    assert_bitwise(out4, ref_out, f"indexed fused modulated W={W}")

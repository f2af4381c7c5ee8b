"""GPU parity of the bf16 attention kernel.

Bar (the operator's tolerance): max |err| <= 2e-2 and relative RMS <= 1e-2 against an fp32
(or fp64) softmax(q k^T s) v reference. Small and ragged shapes are checked
against the fp64 CPU oracle; the S = 8192 and S = 73,984 configurations
against a chunked fp32 reference computed on the GPU with torch (fp32 matmul)
plus fp64 oracle rows sampled as in tools/verify_attention.py:62-65.
"""
from __future__ import annotations

import math

import pytest
import torch

from conftest import attention_error

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
MAX_ABS, REL_RMS = 2e-2, 1e-2


def _bhsd(x):
    """[B, S, H, D] -> the kernel's [B, H, S, D] view (strides swapped, as the
    reference's MHA operator passes it, patches/InfiniCore.patch:1403-1411)."""
    return x.transpose(1, 2)


def gpu_reference_fp32(q, k, v, scale, chunk=512):
    """softmax(q k^T scale) v in fp32 on the GPU, chunked over queries."""
    B, H, Sq, D = q.shape
    out = torch.empty(B, H, Sq, D, dtype=torch.float32, device=q.device)
    kt = k.float().transpose(-2, -1).contiguous()
    vf = v.float().contiguous()
    for s0 in range(0, Sq, chunk):
        logits = torch.matmul(q[:, :, s0:s0 + chunk].float().contiguous(), kt) * scale
        out[:, :, s0:s0 + chunk] = torch.matmul(torch.softmax(logits, dim=-1), vf)
    return out


@pytest.mark.parametrize("B,H,Sq,Sk", [
    (1, 1, 1, 1), (1, 2, 64, 64), (2, 3, 65, 63), (1, 2, 200, 129), (1, 1, 300, 1000),
    (2, 2, 257, 257), (1, 1, 513, 64),
])
def test_attention_small_vs_fp64(pkg, oracle, device, B, H, Sq, Sk):
    gen = torch.Generator("cpu").manual_seed(Sq * 7 + Sk)
    q = torch.randn(B, Sq, H, 128, generator=gen).to(BF)
    k = torch.randn(B, Sk, H, 128, generator=gen).to(BF)
    v = torch.randn(B, Sk, H, 128, generator=gen).to(BF)
    scale = 128 ** -0.5
    qd, kd, vd = (t.to(device) for t in (q, k, v))
    out = torch.empty(B, Sq, H, 128, dtype=BF, device=device)
    pkg.make_attention()(_bhsd(qd), _bhsd(kd), _bhsd(vd), scale, _bhsd(out))
    torch.cuda.synchronize()
    ref = oracle.attention(_bhsd(q), _bhsd(k), _bhsd(v), scale)
    mx, rel = attention_error(_bhsd(out).cpu(), ref)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)


def test_attention_packed_qkv(pkg, oracle, device):
    """q, k, v as strided slices of one packed [1, S, 3, H, D] tensor
    (tools/verify_attention.py:42-43)."""
    gen = torch.Generator("cpu").manual_seed(2026)
    S, H = 1024, 14
    packed = torch.randn(1, S, 3, H, 128, generator=gen).to(BF)
    pd = packed.to(device)
    q, k, v = (pd[:, :, i].transpose(1, 2) for i in range(3))
    out = torch.empty(1, H, S, 128, dtype=BF, device=device)
    pkg.make_attention()(q, k, v, 128 ** -0.5, out)
    torch.cuda.synchronize()
    ref = oracle.attention(*(packed[:, :, i].transpose(1, 2) for i in range(3)), 128 ** -0.5)
    mx, rel = attention_error(out.cpu(), ref)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)
    # Repeat determinism (tools/verify_attention.py:54-59).
    first = out.clone()
    pkg.make_attention()(q, k, v, 128 ** -0.5, out)
    torch.cuda.synchronize()
    assert torch.equal(first, out)


def test_attention_broadcast_keys_take_the_pointer_path(pkg, oracle, device):
    """K and V broadcast along S (stride 0: every key the same row), which the
    buffer-load path does not take (its rows must not overlap): softmax is
    uniform, so every output row equals the V row; also Sk not a multiple of 64
    and a second head with its own row."""
    gen = torch.Generator("cpu").manual_seed(9)
    Sq, Sk, H = 150, 333, 2
    q = torch.randn(1, H, Sq, 128, generator=gen).to(BF)
    krow = torch.randn(1, H, 1, 128, generator=gen).to(BF)
    vrow = torch.randn(1, H, 1, 128, generator=gen).to(BF)
    k, v = krow.expand(1, H, Sk, 128), vrow.expand(1, H, Sk, 128)
    kd, vd = krow.to(device).expand(1, H, Sk, 128), vrow.to(device).expand(1, H, Sk, 128)
    assert kd.stride(2) == 0 and vd.stride(2) == 0
    out = torch.empty(1, H, Sq, 128, dtype=BF, device=device)
    pkg.make_attention()(q.to(device), kd, vd, 128 ** -0.5, out)
    torch.cuda.synchronize()
    ref = oracle.attention(q, k.contiguous(), v.contiguous(), 128 ** -0.5)
    mx, rel = attention_error(out.cpu(), ref)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)
    assert (out.cpu().float() - vrow.float()).abs().max().item() <= 2 ** -7 * vrow.float().abs().max().item()


def _strided(x, device, case, gen):
    """x [B, H, S, D] on `device` as the view `case` names, sentinels around:
    "dstride2": every other element of a [.., 2D] buffer (head-dim stride 2);
    "offset1": rows starting one element into their buffer (2-byte aligned,
    not 16); "odd_rows": an S stride of D + 3 elements; "dense": the
    contiguous view. Returns (view, its buffer or None)."""
    B, H, S, D = x.shape
    if case == "dense":
        return x.to(device).contiguous(), None
    if case == "dstride2":
        buf = torch.randn(B, H, S, 2 * D, generator=gen).to(BF)
        buf[..., ::2] = x
        return buf.to(device)[..., ::2], buf.to(device)
    if case == "offset1":
        buf = torch.randn(B, H, S, D + 1, generator=gen).to(BF)
        buf[..., 1:] = x
        return buf.to(device)[..., 1:], buf.to(device)
    if case == "odd_rows":
        buf = torch.randn(B, H, S, D + 3, generator=gen).to(BF)
        buf[..., :D] = x
        return buf.to(device)[..., :D], buf.to(device)
    raise ValueError(case)


@pytest.mark.parametrize("dim", [128, 72])
@pytest.mark.parametrize("cases", [
    ("dstride2", "dense", "dense", "dense"),
    ("dense", "offset1", "dstride2", "dense"),
    ("offset1", "odd_rows", "odd_rows", "dstride2"),
    ("dense", "dense", "dense", "offset1"),
])
def test_attention_element_strided_views(pkg, oracle, device, dim, cases):
    """Views the 16-byte accesses cannot take -- a head-dim stride other than
    1, rows that are 2- but not 16-byte aligned, S strides
    that are not multiples of 8 -- run on the element-strided path, as the
    reference's generic stride variant does (patches/ninetoothed.patch:131-169):
    within the operator's bar of the fp64 oracle, Sq not a multiple of 256 and
    Sk not of 64, and the out buffer's elements outside the view untouched."""
    gen = torch.Generator("cpu").manual_seed(dim + len("".join(cases)))
    B, H, Sq, Sk = 2, 2, 300, 129
    q = torch.randn(B, H, Sq, dim, generator=gen).to(BF)
    k = torch.randn(B, H, Sk, dim, generator=gen).to(BF)
    v = torch.randn(B, H, Sk, dim, generator=gen).to(BF)
    qd, _ = _strided(q, device, cases[0], gen)
    kd, _ = _strided(k, device, cases[1], gen)
    vd, _ = _strided(v, device, cases[2], gen)
    out, out_buf = _strided(torch.full((B, H, Sq, dim), float("nan")).to(BF), device, cases[3], gen)
    before = out_buf.clone() if out_buf is not None else None
    scale = dim ** -0.5
    print(f"strided attention dim={dim} cases={cases}", flush=True)
    pkg.make_attention(head_dim=dim)(qd, kd, vd, scale, out)
    torch.cuda.synchronize()
    ref = oracle.attention(q, k, v, scale)
    mx, rel = attention_error(out.cpu(), ref)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)
    if out_buf is not None:
        inside = torch.zeros(out_buf.shape, dtype=torch.bool, device=device)
        if cases[3] == "dstride2":
            inside[..., ::2] = True
        elif cases[3] == "offset1":
            inside[..., 1:] = True
        else:
            inside[..., :dim] = True
        assert torch.equal(out_buf[~inside].view(torch.int16), before[~inside].view(torch.int16)), "wrote outside the view"


def test_attention_negative_head_dim_stride_through_the_abi(pkg, oracle, device):
    """A view torch cannot express, handed to launch_h3_full_attention as the
    C ABI allows: q, k, v and o with head-dim stride -1 (data points at each
    row's last element). Same bar against the fp64 oracle of the reversed
    rows."""
    L = pkg._lib
    gen = torch.Generator("cpu").manual_seed(77)
    B, H, Sq, Sk, D = 1, 2, 200, 100, 128
    q, k, v = (torch.randn(B, H, s, D, generator=gen).to(BF) for s in (Sq, Sk, Sk))
    stores = [t.flip(-1).contiguous().to(device) for t in (q, k, v)]
    o_store = torch.full((B, H, Sq, D), float("nan"), dtype=BF, device=device)

    def rev(t):  # element (b, h, s, d) of the view is t_store[b, h, s, D - 1 - d]
        sb, sh, ss, _ = t.stride()
        return L.raw_tensor(t.data_ptr() + 2 * (D - 1), list(t.shape), [sb, sh, ss, -1])

    stream = torch.cuda.current_stream(device).cuda_stream
    rc = L.call("launch_h3_full_attention", stream, rev(stores[0]), rev(stores[1]), rev(stores[2]),
                L.scalar(128 ** -0.5), rev(o_store))
    assert rc == 0, rc
    torch.cuda.synchronize()
    ref = oracle.attention(q, k, v, 128 ** -0.5)
    mx, rel = attention_error(o_store.flip(-1).cpu(), ref)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)


@pytest.mark.parametrize("scale", [128 ** -0.5, -0.07])
def test_attention_bf16_prescale(pkg, oracle, device, scale):
    """numerics="bf16_prescale" (tools/h3_attention.py:87-101) against its own
    fp64 oracle, ragged Sq / Sk, positive and negative scale."""
    gen = torch.Generator("cpu").manual_seed(17)
    q = torch.randn(2, 3, 197, 128, generator=gen).to(BF)
    k = torch.randn(2, 3, 333, 128, generator=gen).to(BF)
    v = torch.randn(2, 3, 333, 128, generator=gen).to(BF)
    out = torch.empty_like(q, device=device)
    pkg.make_attention(numerics="bf16_prescale")(q.to(device), k.to(device), v.to(device), scale, out)
    torch.cuda.synchronize()
    mx, rel = attention_error(out.cpu(), oracle.attention_bf16_prescale(q, k, v, scale))
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)


def test_attention_scale_edge_cases(pkg, oracle, device):
    gen = torch.Generator("cpu").manual_seed(5)
    q = torch.randn(1, 2, 130, 128, generator=gen).to(BF)
    k = torch.randn(1, 2, 190, 128, generator=gen).to(BF)
    v = torch.randn(1, 2, 190, 128, generator=gen).to(BF)
    for scale in (0.0, -0.05, 0.5):
        out = torch.empty_like(q, device=device)
        pkg.make_attention()(q.to(device), k.to(device), v.to(device), scale, out)
        torch.cuda.synchronize()
        ref = oracle.attention(q, k, v, scale)
        mx, rel = attention_error(out.cpu(), ref)
        assert mx <= MAX_ABS and rel <= REL_RMS, (scale, mx, rel)


@pytest.mark.parametrize("B,H,Sq,Sk", [(1, 1, 1, 1), (2, 3, 65, 63), (1, 2, 200, 129), (2, 2, 257, 1000)])
def test_vision_attention_72_small_vs_fp64(pkg, oracle, device, B, H, Sq, Sk):
    """Head dim 72 (launch_h3_vision_attention_72, scripts/build_h3_attention.py:23-24)
    in the [B, S, H, 72] layout of the reference's MHA operator."""
    gen = torch.Generator("cpu").manual_seed(Sq * 11 + Sk)
    q = torch.randn(B, Sq, H, 72, generator=gen).to(BF)
    k = torch.randn(B, Sk, H, 72, generator=gen).to(BF)
    v = torch.randn(B, Sk, H, 72, generator=gen).to(BF)
    scale = 72 ** -0.5
    # A sentinel past dim 72 of every output row: the kernel stores dims 0..71 only.
    outbuf = torch.full((B, Sq, H, 80), 7.0, dtype=BF, device=device)
    out = outbuf[..., :72]
    pkg.make_attention(head_dim=72)(*(_bhsd(t.to(device)) for t in (q, k, v)), scale, _bhsd(out))
    torch.cuda.synchronize()
    ref = oracle.attention(_bhsd(q), _bhsd(k), _bhsd(v), scale)
    mx, rel = attention_error(_bhsd(out).cpu(), ref)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)
    assert bool((outbuf[..., 72:] == 7.0).all())


def test_vision_attention_72_packed_and_broadcast(pkg, oracle, device):
    """Head dim 72: q, k, v as slices of one packed [1, S, 3, H, 72] tensor
    (buffer-load path), then K / V broadcast along S (pointer path)."""
    gen = torch.Generator("cpu").manual_seed(72)
    S, H = 1000, 16
    packed = torch.randn(1, S, 3, H, 72, generator=gen).to(BF)
    pd = packed.to(device)
    attn = pkg.make_attention(head_dim=72)
    out = torch.empty(1, H, S, 72, dtype=BF, device=device)
    attn(*(pd[:, :, i].transpose(1, 2) for i in range(3)), 72 ** -0.5, out)
    torch.cuda.synchronize()
    ref = oracle.attention(*(packed[:, :, i].transpose(1, 2) for i in range(3)), 72 ** -0.5)
    mx, rel = attention_error(out.cpu(), ref)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)

    q = packed[:, :200, 0].transpose(1, 2)
    krow = torch.randn(1, H, 1, 72, generator=gen).to(BF)
    vrow = torch.randn(1, H, 1, 72, generator=gen).to(BF)
    kd, vd = krow.to(device).expand(1, H, 333, 72), vrow.to(device).expand(1, H, 333, 72)
    out = torch.empty(1, H, 200, 72, dtype=BF, device=device)
    attn(q.to(device), kd, vd, 72 ** -0.5, out)
    torch.cuda.synchronize()
    ref = oracle.attention(q, krow.expand(1, H, 333, 72).contiguous(), vrow.expand(1, H, 333, 72).contiguous(),
                           72 ** -0.5)
    mx, rel = attention_error(out.cpu(), ref)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)


def test_vision_attention_72_s4096_vs_fp32(pkg, device):
    """A vision-tower sized call (16 heads of 72 over 4096 patches) against the
    chunked fp32 reference."""
    gen = torch.Generator("cpu").manual_seed(4096)
    q, k, v = (torch.randn(1, 4096, 16, 72, generator=gen).to(BF).to(device) for _ in range(3))
    out = torch.empty_like(q)
    pkg.make_attention(head_dim=72)(_bhsd(q), _bhsd(k), _bhsd(v), 72 ** -0.5, _bhsd(out))
    torch.cuda.synchronize()
    ref = gpu_reference_fp32(_bhsd(q), _bhsd(k), _bhsd(v), 72 ** -0.5)
    mx, rel = attention_error(_bhsd(out), ref)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)


def _config_check(pkg, oracle, device, S, outlier_fraction):
    q, k, v = oracle.attention_inputs(S, outlier_fraction=outlier_fraction)
    scale = 128 ** -0.5
    qd, kd, vd = (t.to(device) for t in (q, k, v))
    out = torch.empty_like(qd)
    pkg.make_attention()(_bhsd(qd), _bhsd(kd), _bhsd(vd), scale, _bhsd(out))
    torch.cuda.synchronize()
    ref = gpu_reference_fp32(_bhsd(qd), _bhsd(kd), _bhsd(vd), scale)
    mx, rel = attention_error(_bhsd(out), ref)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)
    rows = torch.linspace(0, S - 1, 16).long()
    ref_rows = oracle.attention_rows(_bhsd(q), _bhsd(k), _bhsd(v), scale, rows)
    mx, rel = attention_error(_bhsd(out)[:, :, rows].cpu(), ref_rows)
    assert mx <= MAX_ABS and rel <= REL_RMS, ("fp64 rows", mx, rel)
    return out


def test_attention_config_s8192(pkg, oracle, device):
    _config_check(pkg, oracle, device, 8192, 0.0)


def test_attention_config_s73984_peaky(pkg, oracle, device):
    """S = 73,984 (32x48x48 video + 256 text tokens), H = 14, 1% of key rows x8."""
    _config_check(pkg, oracle, device, 73984, 0.01)


@pytest.mark.parametrize("B,H,Sq,Sk,sign", [
    (2, 3, 5000, 4500, 1.0),    # B > 1, Sq != Sk, ragged keys (partial last tile)
    (2, 3, 5000, 4500, -1.0),   # the same with a negative scale (the loop's min path)
    (1, 5, 16384, 4097, 1.0),   # one key past a whole tile
    (1, 14, 8192, 8192, 1.0),   # the S = 8192 configuration
])
def test_attention_large_ragged(pkg, device, B, H, Sq, Sk, sign):
    """Large launches in the [B, S, H, D] layout: batched, Sq != Sk, a partial
    last key tile and a negative scale, against the chunked fp32 reference over
    every row; two launches bitwise equal."""
    gen = torch.Generator("cpu").manual_seed(Sq + Sk + H)
    q = torch.randn(B, Sq, H, 128, generator=gen).to(BF).to(device)
    k = torch.randn(B, Sk, H, 128, generator=gen).to(BF).to(device)
    v = torch.randn(B, Sk, H, 128, generator=gen).to(BF).to(device)
    scale = sign * 128 ** -0.5
    out = torch.full((B, Sq, H, 128), float("nan"), dtype=BF, device=device)
    kernel = pkg.make_attention()
    kernel(_bhsd(q), _bhsd(k), _bhsd(v), scale, _bhsd(out))
    torch.cuda.synchronize()
    first = out.clone()
    kernel(_bhsd(q), _bhsd(k), _bhsd(v), scale, _bhsd(out))
    torch.cuda.synchronize()
    assert torch.equal(first, out), "two launches differ"
    ref = gpu_reference_fp32(_bhsd(q), _bhsd(k), _bhsd(v), scale)
    mx, rel = attention_error(_bhsd(out), ref)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)


@pytest.mark.parametrize("seq", [1024, 8192, 40000])
@pytest.mark.parametrize("heads", [14, 28, 56])
def test_attention_reference_acceptance_grid(pkg, device, seq, heads):
    """The reference's own acceptance run for this operator
    (tools/verify_attention.py:39-77): q, k, v strided slices of one packed
    [1, S, 3, H, 128] bf16 tensor, scale 1/sqrt(128), two launches bitwise
    equal, and max |err| <= 2e-3 with mean |err| <= 2e-4 (:73-74). The
    reference compares against torch SDPA and against fp32 on 16 sampled rows;
    here every row is compared against the chunked fp32 GPU reference (bf16
    SDPA is not called on the device). Inputs are drawn from a CPU generator
    seeded 2026 (the reference seeds its device generator with 2026, whose
    values depend on the device RNG)."""
    gen = torch.Generator("cpu").manual_seed(2026)
    packed = torch.randn(1, seq, 3, heads, 128, generator=gen).to(BF).to(device)
    q, k, v = (packed[:, :, i].transpose(1, 2) for i in range(3))
    out = torch.empty_like(q)
    kernel = pkg.make_attention()
    kernel(q, k, v, 128 ** -0.5, out)
    torch.cuda.synchronize()
    first = out.clone()
    kernel(q, k, v, 128 ** -0.5, out)
    torch.cuda.synchronize()
    assert torch.equal(first, out), "two launches differ"
    ref = gpu_reference_fp32(q, k, v, 128 ** -0.5, chunk=256)
    delta = (out.float() - ref).abs()
    mx, mean = delta.max().item(), delta.mean().item()
    assert mx <= 2e-3 and mean <= 2e-4, (seq, heads, mx, mean)


# ------------------------------------------------------------ reference maximum and its fallback


@pytest.mark.parametrize("case", ["late_logit_overflows_p", "huge_values_overflow_o"])
def test_attention_reference_max_overflow_falls_back_to_exact(pkg, oracle, device, case):
    """The D = 128 kernel keeps each unit's first-tile maximum as the softmax
    reference. Inputs that overflow against it make the workgroup recompute
    the unit with the exact online rescale, so the result is the reference
    order's: a key whose logit lies ~200 log2 units above the first tile's
    (p = exp2 of that is +inf), and values near 1e33 whose sum overflows fp32
    once p grows by 2^20. Checked against the fp64 oracle."""
    B, H, Sq, Sk = 1, 2, 300, 700
    gen = torch.Generator("cpu").manual_seed(11)
    q = torch.randn(B, H, Sq, 128, generator=gen)
    k = torch.randn(B, H, Sk, 128, generator=gen) * 0.1
    v = torch.randn(B, H, Sk, 128, generator=gen)
    if case == "late_logit_overflows_p":
        q[..., 0] = 16.0
        k[:, :, 500, 0] = 100.0  # logit ~ 16 * 100 / sqrt(128) * log2 e ~ 204 in log2 units, tile 7
    else:
        q[..., 0] = 4.0
        k[:, :, 300:, 0] = 40.0  # later logits ~ 20 log2 units above the first tiles'
        v = v.sign() * 1e33 + v * 1e31
    q, k, v = (t.to(BF) for t in (q, k, v))
    want = oracle.attention(q.double(), k.double(), v.double(), 128 ** -0.5)
    out = torch.full((B, H, Sq, 128), float("nan"), dtype=BF, device=device)
    pkg.make_attention(split_last_round=False)(q.to(device), k.to(device), v.to(device), 128 ** -0.5, out)
    torch.cuda.synchronize()
    got = out.double().cpu()
    assert torch.isfinite(got).all()
    rel = float((got - want).norm() / want.norm())
    assert rel <= 1e-2, (case, rel)


def _dominant_keys(Sk, keys, logit_log2, v_value):
    """q = 16 e0 for every query, k = 0 except k[key, 0] = x at `keys`, so
    every logit is 0 except those keys', which sit `logit_log2` log2 units
    above (x = logit / (16 scale log2 e), exact in bf16 for the values used
    here); v = v_value at those keys, N(0, 1) elsewhere. The fp64 reference
    output of every query is about v_value."""
    gen = torch.Generator("cpu").manual_seed(Sk)
    q = torch.zeros(1, 1, 256, 128)
    q[..., 0] = 16.0
    k = torch.zeros(1, 1, Sk, 128)
    k[0, 0, keys, 0] = logit_log2 / (16 * 128 ** -0.5 * math.log2(math.e))
    v = torch.randn(1, 1, Sk, 128, generator=gen)
    v[0, 0, keys] = v_value
    return q.to(BF), k.to(BF), v.to(BF)


def test_attention_dominated_rows_are_exact(pkg, oracle, device):
    """One key of a later tile dominates every query (about 50 log2 units
    above the first tile's logits, which set the reference maximum), and its
    V row is 1.96875 in every dim. The weight p of that key is a power of two
    far from 1, so bf16(p) differs from p by a quarter of a percent or more
    (the key value is chosen so): a denominator that summed the fp32 p would
    leave o = 1.96875 (1 + delta), which rounds to the next bf16 value. The
    kernel's denominator sums the same bf16 weights that multiply V, so o is
    the V row exactly, in every query and dim, as the fp64 reference's is."""
    c = torch.tensor(128 ** -0.5 * math.log2(math.e), dtype=torch.float32)
    pick = None
    for kval in torch.arange(20.0, 30.0, 0.125):  # bf16-exact key values
        p = torch.exp2(c * (16.0 * kval.to(torch.float32)))
        delta = float((p.to(BF).float() - p).abs() / p)
        if delta >= 2.5e-3:
            pick = float(kval)
            break
    assert pick is not None
    key, v_dom = 333, 1.96875
    q, k, v = _dominant_keys(700, [key], 1.0, v_dom)
    k[0, 0, key, 0] = pick
    assert float(k[0, 0, key, 0]) == pick and float(v[0, 0, key, 5]) == v_dom
    out = torch.full(q.shape, float("nan"), dtype=BF, device=device)
    pkg.make_attention(split_last_round=False)(q.to(device), k.to(device), v.to(device), 128 ** -0.5, out)
    torch.cuda.synchronize()
    want = oracle.attention(q.double(), k.double(), v.double(), 128 ** -0.5)
    assert torch.equal(want.to(BF), torch.full_like(want, v_dom).to(BF))
    assert torch.equal(out.cpu(), torch.full(q.shape, v_dom, dtype=BF)), int((out.cpu() != v_dom).sum())


def test_attention_folded_denominator_overflow_falls_back(pkg, oracle, device):
    """Four keys of one later tile, one in each 16-lane group of the lanes
    that hold a query's keys (tile offsets 0, 4, 8, 12), each 127 log2 units
    above the first tile's maximum: every weight (2^127) and every
    accumulator (4 * 2^127 * 0.25) stays finite, but their sum, the
    denominator (2^129), overflows. The unit must take the exact fallback and
    give about 0.25 everywhere, not o = 0."""
    keys = [320, 324, 328, 332]
    q, k, v = _dominant_keys(700, keys, 127.0, 0.25)
    assert torch.equal(k[0, 0, keys, 0].float(), torch.full((4,), 62.25))
    want = oracle.attention(q.double(), k.double(), v.double(), 128 ** -0.5)
    out = torch.full(q.shape, float("nan"), dtype=BF, device=device)
    pkg.make_attention(split_last_round=False)(q.to(device), k.to(device), v.to(device), 128 ** -0.5, out)
    torch.cuda.synchronize()
    mx, rel = attention_error(out.cpu(), want)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)


def test_attention_split_pieces_near_overflow_fall_back(pkg, oracle, device):
    """A single unit split along the keys, with two keys 126.5 log2 units
    above their piece's first tile in each of the first two pieces: each
    piece's own denominator (about 2^127.5) is finite, but the merge's sum
    over the pieces would overflow. A piece whose denominator or accumulators
    exceed FLT_MAX / 8 takes the exact pass, so the merged result is finite
    and matches the fp64 reference."""
    Sk = 6400
    nbytes = pkg._lib.attention_workspace_bytes(1, 1, 256, Sk)
    split = nbytes // WS_SLOT_BYTES
    assert split >= 2, nbytes
    tiles = -(-Sk // 64)
    keys = []
    for p in range(2):
        t = p * tiles // split + 1  # the piece's second tile
        keys += [64 * t, 64 * t + 4]
    q, k, v = _dominant_keys(Sk, keys, 126.5, 0.25)
    want = oracle.attention(q.double(), k.double(), v.double(), 128 ** -0.5)
    out = torch.full(q.shape, float("nan"), dtype=BF, device=device)
    pkg.make_attention(split_last_round=True)(q.to(device), k.to(device), v.to(device), 128 ** -0.5, out)
    torch.cuda.synchronize()
    mx, rel = attention_error(out.cpu(), want)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)


# ------------------------------------------------------------ key split of the last round

WS_SLOT_BYTES = (256 * 128 + 256 * 2) * 4  # per piece: O of its 256 queries + (m, l) per query


@pytest.mark.parametrize("B,H,Sq,Sk,sign,outliers", [
    (1, 28, 8192, 8192, 1.0, 0.01),   # 896 units: 3 full rounds and a half-full one, split in 2
    (2, 3, 5000, 4500, -1.0, 0.0),    # one partial round, ragged keys, negative scale
    (1, 2, 700, 3000, 1.0, 0.01),     # Sq not a multiple of 256, Sk % 64 != 0
    (1, 1, 256, 6400, 1.0, 0.0),      # a single unit split up to 8 ways
])
def test_attention_split_last_round(pkg, device, B, H, Sq, Sk, sign, outliers):
    """make_attention splits these launches' last round along the keys
    (launch_h3_full_attention_ws): deterministic, within the operator's bar of
    the fp32 reference, no further from it than the unsplit kernel (relative
    RMS within 5e-4), and within relative RMS 5e-3 of it: they differ where P
    is rounded to bf16 against a piece's reference maximum instead of the
    unit's, and then by the output's bf16 rounding (2^-9 relative each)."""
    nbytes = pkg._lib.attention_workspace_bytes(B, H, Sq, Sk)
    assert nbytes > 0 and nbytes % WS_SLOT_BYTES == 0, nbytes
    if (B, H, Sq, Sk) == (1, 28, 8192, 8192) and torch.cuda.get_device_properties(device).multi_processor_count == 256:
        assert nbytes == 128 * 2 * WS_SLOT_BYTES  # 128 tail units, 2 key halves each
    gen = torch.Generator("cpu").manual_seed(B * Sq + Sk)
    q = torch.randn(B, Sq, H, 128, generator=gen).to(BF)
    k = torch.randn(B, Sk, H, 128, generator=gen).to(BF)
    v = torch.randn(B, Sk, H, 128, generator=gen).to(BF)
    if outliers:
        rows = torch.randperm(Sk, generator=gen)[: max(1, int(Sk * outliers))]
        k[:, rows] *= 8
    q, k, v = (t.to(device) for t in (q, k, v))
    scale = sign * 128 ** -0.5
    outs = []
    for split in (True, True, False):
        out = torch.full((B, Sq, H, 128), float("nan"), dtype=BF, device=device)
        pkg.make_attention(split_last_round=split)(_bhsd(q), _bhsd(k), _bhsd(v), scale, _bhsd(out))
        torch.cuda.synchronize()
        outs.append(out)
    assert torch.equal(outs[0], outs[1]), "two split launches differ"
    ref = gpu_reference_fp32(_bhsd(q), _bhsd(k), _bhsd(v), scale)
    mx, rel = attention_error(_bhsd(outs[0]), ref)
    assert mx <= MAX_ABS and rel <= REL_RMS, (mx, rel)
    _, rel_unsplit = attention_error(_bhsd(outs[2]), ref)
    assert rel <= rel_unsplit + 5e-4, ("split vs unsplit against fp32", rel, rel_unsplit)
    mx, rel = attention_error(_bhsd(outs[0]), _bhsd(outs[2]).float())
    assert rel <= 5e-3, ("split vs unsplit", mx, rel)


def test_attention_split_plan_leaves_a_three_quarter_round(pkg, device):
    """At S = 8192, H = 14 (448 units on 256 CUs) the last round is 3/4 full:
    it runs as a round of 192-query units, which needs no workspace; the
    configuration at S = 73,984 (a 4/5-full last round of 16) is not split
    either. At S = 12,288 (672 units: a 5/8-full last
    round) it splits, which measured 3.4% faster (848.5 against 877.8 us)."""
    if torch.cuda.get_device_properties(device).multi_processor_count != 256:
        pytest.skip("the plan is stated for 256 CUs")
    assert pkg._lib.attention_workspace_bytes(1, 14, 8192, 8192) == 0
    assert pkg._lib.attention_workspace_bytes(1, 14, 73984, 73984) == 0
    assert pkg._lib.attention_workspace_bytes(1, 14, 12288, 12288) > 0


def test_attention_ws_small_workspace_runs_unsplit(pkg, device):
    """launch_h3_full_attention_ws with a workspace smaller than the plan's
    (empty, one byte short) runs the unsplit kernel: bitwise equal to
    launch_h3_full_attention."""
    L = pkg._lib
    B, H, S = 1, 3, 2000
    gen = torch.Generator("cpu").manual_seed(5)
    q, k, v = (torch.randn(B, H, S, 128, generator=gen).to(BF).to(device) for _ in range(3))
    nbytes = L.attention_workspace_bytes(B, H, S, S)
    assert nbytes > 0
    stream = torch.cuda.current_stream(device).cuda_stream
    args = [L.tensor(q), L.tensor(k), L.tensor(v), L.scalar(0.09)]
    ref = torch.empty_like(q)
    assert L.call("launch_h3_full_attention", stream, *args, L.tensor(ref)) == 0
    for size in (0, nbytes - 1):
        ws = torch.empty(max(size, 1), dtype=torch.uint8, device=device)[:size]
        out = torch.full_like(q, float("nan"))
        assert L.call("launch_h3_full_attention_ws", stream, *args, L.tensor(out), L.tensor(ws)) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, ref), size
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    out = torch.full_like(q, float("nan"))
    assert L.call("launch_h3_full_attention_ws", stream, *args, L.tensor(out), L.tensor(ws)) == 0
    torch.cuda.synchronize()
    assert not torch.equal(out, ref) and not torch.isnan(out).any()
    assert attention_error(out, ref.float())[1] <= 5e-3


# ------------------------------------------------------------ 192-query last round

def _attention16_launched(fn):
    """The D = 128 attention kernels `fn` launches, as name<template args>."""
    from torch.profiler import ProfilerActivity, profile
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        fn()
        torch.cuda.synchronize()
    return sorted({"attention16" + e.name.split("attention16")[1].split(">")[0] + ">"
                   for e in prof.events() if "attention16" in e.name})


@pytest.mark.parametrize("B,H,Sq,Sk,scale,entry,case", [
    (1, 14, 8192, 8192, 128 ** -0.5, "launch_h3_full_attention", "config"),
    (1, 14, 8192, 5000, -0.07, "launch_h3_full_attention", "partial key tile, negative scale"),
    (2, 14, 4096, 4096, 128 ** -0.5, "launch_h3_full_attention", "B = 2"),
    (20, 16, 768, 700, 0.09, "launch_h3_full_attention", "64 heads all 192-query, one all 256"),
    (1, 14, 8192, 8192, 128 ** -0.5, "launch_h3_full_attention_bf16_prescale", "prescale"),
    (1, 14, 8192, 8192, 128 ** -0.5, "launch_h3_full_attention", "overflow in 192-query units"),
])
def test_attention_192_query_last_round(pkg, device, B, H, Sq, Sk, scale, entry, case):
    """A launch whose last round of 256-query units would leave a quarter of
    the CUs idle (448 units on 256 CUs at S = 8192, H = 14) runs that round as
    256 units of 192 queries instead (waves 0-3 with 32 queries, waves 4-7 with
    16). Each query's arithmetic is that of the ordinary launch, so one launch
    over all heads equals launches of one head each (which are too small for
    the plan) bitwise, whatever unit a query lands in. The 'overflow' case
    puts a key ~200 log2 units above the first tile's maximum for every query
    of head 0, most of whose queries lie in 192-query units: every workgroup
    of that head takes the exact fallback, in both launches."""
    if torch.cuda.get_device_properties(device).multi_processor_count != 256:
        pytest.skip("the plan is stated for 256 CUs")
    L = pkg._lib
    gen = torch.Generator("cpu").manual_seed(Sq + Sk + B * H)
    q = torch.randn(B, H, Sq, 128, generator=gen)
    k = torch.randn(B, H, Sk, 128, generator=gen)
    v = torch.randn(B, H, Sk, 128, generator=gen)
    if case.startswith("overflow"):
        q[0, 0, :, 0] = 16.0
        k[0, 0, :, 0] *= 0.1
        k[0, 0, 4000, 0] = 100.0  # a logit ~204 log2 units up, in tile 62
    q, k, v = (t.to(BF).to(device) for t in (q, k, v))
    stream = torch.cuda.current_stream(device).cuda_stream
    print(f"192-query round: {case} B={B} H={H} Sq={Sq} Sk={Sk} {entry}", flush=True)
    out = torch.full_like(q, float("nan"))
    launched = _attention16_launched(
        lambda: L.call(entry, stream, L.tensor(q), L.tensor(k), L.tensor(v), L.scalar(scale), L.tensor(out)))
    neg = "true" if scale < 0 and "prescale" not in entry else "false"
    assert launched == [f"attention16_small_kernel<{neg}>"], launched
    ref = torch.full_like(q, float("nan"))
    for b in range(B):
        for h in range(H):
            sl = (slice(b, b + 1), slice(h, h + 1))
            assert L.call(entry, stream, L.tensor(q[sl]), L.tensor(k[sl]), L.tensor(v[sl]), L.scalar(scale),
                          L.tensor(ref[sl])) == 0
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    assert torch.equal(out, ref), int((out != ref).sum())
    if case.startswith("overflow"):
        head0 = out[0, 0].float()
        assert torch.isfinite(head0).all()
        assert float((head0 - v[0, 0, 4000].float()).abs().max()) <= 2e-2


@pytest.mark.parametrize("S,outliers", [(73984, 0.01), (16384, 0.0)])
def test_attention_exact_invariants_at_full_size(pkg, oracle, device, S, outliers):
    """Size-independent properties that hold bitwise, at the configuration
    size (S = 73,984, 1% of key rows x8) and at S = 16,384, where the plan
    splits the last round along the keys:
      - V -> 2 V doubles every output exactly (the weights do not depend on V,
        and doubling commutes with the fp32 sums and the bf16 rounding);
      - where the plan leaves the launch unsplit (S = 73,984), permuting the
        query rows (and heads) permutes the output rows: each query keeps its
        own reference maximum and is computed independently of the unit,
        wave and lane it lands in (these inputs take no overflow fallback).
        Split launches are excluded: a query moved into a split unit rounds P
        against its piece's reference maximum."""
    H = 14
    q, k, v = oracle.attention_inputs(S, outlier_fraction=outliers)
    qd, kd, vd = (t.to(device) for t in (q, k, v))
    scale = 128 ** -0.5
    f = pkg.make_attention()
    out = torch.empty_like(qd)
    f(_bhsd(qd), _bhsd(kd), _bhsd(vd), scale, _bhsd(out))
    out2 = torch.empty_like(qd)
    f(_bhsd(qd), _bhsd(kd), _bhsd(vd * 2), scale, _bhsd(out2))
    torch.cuda.synchronize()
    assert torch.equal(out2, out * 2), "V -> 2V"
    if pkg._lib.attention_workspace_bytes(1, H, S, S) != 0:
        return
    gen = torch.Generator(device=device).manual_seed(S)
    perm = torch.randperm(S, generator=gen, device=device)
    hperm = torch.randperm(H, generator=gen, device=device)
    qp = qd[:, perm][:, :, hperm].contiguous()
    outp = torch.empty_like(qd)
    f(_bhsd(qp), _bhsd(kd[:, :, hperm].contiguous()), _bhsd(vd[:, :, hperm].contiguous()), scale, _bhsd(outp))
    torch.cuda.synchronize()
    assert torch.equal(outp, out[:, perm][:, :, hperm]), "query and head permutation"


@pytest.mark.gpu
def test_head_groups_with_copies_on_a_second_stream_match_one_launch(pkg, device):
    """Head-grouped attention (each group's q, k, v copied on a second stream
    while the previous group computes, bench.py's head_group_calls) writes
    bitwise the output of one launch over all heads: units are independent per
    head, so the grouping and the overlap change nothing."""
    import bench
    gen = torch.Generator(device=device).manual_seed(21)
    S, H = 3000, 6
    q, k, v = (torch.randn(1, S, H, 128, generator=gen, device=device).to(torch.bfloat16) for _ in range(3))
    out_full, out_grp = torch.zeros_like(q), torch.zeros_like(q)
    pkg.make_attention(split_last_round=False)(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), 0.09,
                                               out_full.transpose(1, 2))
    grouped, _ = bench.head_group_calls(pkg, q, k, v, out_grp, 0.09, 3)
    for _ in range(2):
        grouped()
        torch.cuda.synchronize()
        assert torch.equal(out_grp, out_full)
        out_grp.zero_()

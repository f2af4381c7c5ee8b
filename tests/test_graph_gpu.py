"""The launchers under HIP graph capture.

Every entry point runs on the caller's stream, allocates nothing and clears
its own accumulators with a fill kernel (the fp8 quantiser's amax), so a chain
of them can be captured once and replayed. This test captures a DiT-block
shaped chain -- RMSNorm + AdaLN, q + k norm + RoPE, attention, the fused
gated residual + RMSNorm + AdaLN, SwiGLU, the gated residual, and the fp8
quantiser with the fp8 P.V attention -- in one graph, then replays it three
times. Before each replay the inputs are rewritten by eager work on the same
stream. Every replay is checked bitwise against the same chain run eagerly on
those inputs into separate outputs.
"""
from __future__ import annotations

import pytest
import torch

from conftest import assert_bitwise

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def test_block_chain_graph_replays_match_eager(pkg, oracle, device):
    T, H, C, F = 512, 4, 1024, 2048
    gen = torch.Generator(device=device).manual_seed(5)

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=gen, device=device) * scale).to(BF)

    # Inputs rewritten before every replay (the graph reads them in place).
    x, y, up, gact = rnd(1, T, C), rnd(1, T, C), rnd(1, T, F), rnd(1, T, F)
    q, k, v = rnd(T, 1, H, 128), rnd(T, 1, H, 128), rnd(T, 1, H, 128)
    w = rnd(C, scale=0.1) + 1
    wq, wk = rnd(128, scale=0.1) + 1, rnd(128, scale=0.1) + 1
    scale, shift, gate = (rnd(1, 1, C, scale=0.1).expand(1, T, C) for _ in range(3))
    cos, sin = (t.to(device) for t in oracle.rope_table_interleaved(oracle.grid_positions(2, 16, 16)))

    mod, qk = pkg.make_rms_modulate(), pkg.make_qk_norm_rope_interleaved_qk()
    attn, grm = pkg.make_attention(), pkg.make_gated_residual_rms_modulate()
    swiglu, gres = pkg.make_swiglu(), pkg.make_gated_residual()
    fp8pv = pkg.make_attention_fp8pv()

    def chain(o):
        mod(x, w, 1e-6, scale, shift, o["mod"])
        qk(q, k, wq, wk, 1e-6, cos, sin, o["q"], o["k"])
        attn(o["q"].permute(1, 2, 0, 3), o["k"].permute(1, 2, 0, 3), v.permute(1, 2, 0, 3), 128 ** -0.5,
             o["attn"].permute(1, 2, 0, 3))
        grm(x, gate, y, w, 1e-6, scale, shift, o["res"], o["norm"])
        swiglu(up, gact, o["act"])
        gres(o["res"], gate, o["norm"], o["out"])
        v8, vd = o["v8"]
        pkg.quantize_fp8_per_head(v.permute(1, 2, 0, 3), transposed=True, x8=v8, descale=vd)
        fp8pv(o["q"].permute(1, 2, 0, 3), o["k"].permute(1, 2, 0, 3), v8, vd, 128 ** -0.5,
              o["attn8"].permute(1, 2, 0, 3))

    def outputs():
        o = {name: torch.empty(1, T, C, dtype=BF, device=device) for name in ("mod", "res", "norm", "out")}
        o.update({name: torch.empty(T, 1, H, 128, dtype=BF, device=device) for name in ("q", "k", "attn", "attn8")})
        o["act"] = torch.empty(1, T, F, dtype=BF, device=device)
        o["v8"] = pkg.quantize_fp8_per_head(v.permute(1, 2, 0, 3), transposed=True)
        return o

    graph_out, eager_out = outputs(), outputs()
    torch.cuda.synchronize()
    chain(graph_out)  # warm-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            chain(graph_out)
    torch.cuda.synchronize()

    for replay in range(3):
        for t in (x, y, up, gact, q, k, v):
            t.copy_(rnd(*t.shape))  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        chain(eager_out)
        torch.cuda.synchronize()
        for name in ("mod", "q", "k", "attn", "res", "norm", "act", "out", "attn8"):
            assert_bitwise(graph_out[name], eager_out[name], f"replay {replay}: {name}")
        assert torch.equal(graph_out["v8"][0].view(torch.uint8), eager_out["v8"][0].view(torch.uint8))
        assert torch.equal(graph_out["v8"][1], eager_out["v8"][1]), f"replay {replay}: v descale"


@pytest.mark.parametrize("B,H,Sq,Sk,plan", [(1, 2, 700, 3000, "key split"), (20, 16, 768, 700, "192-query round")])
def test_attention_key_split_graph_replays_match_eager(pkg, device, B, H, Sq, Sk, plan):
    """The key-split attention (two kernels and a workspace from torch's
    caching allocator, taken inside the capture), and a launch whose last
    round runs as 192-query units, replay bitwise like the eager launch, with
    the inputs rewritten between replays."""
    if plan == "key split":
        assert pkg._lib.attention_workspace_bytes(B, H, Sq, Sk) > 0
    elif torch.cuda.get_device_properties(device).multi_processor_count != 256:
        pytest.skip("the 192-query plan of this shape is stated for 256 CUs")
    gen = torch.Generator(device=device).manual_seed(11)
    q = torch.randn(B, H, Sq, 128, generator=gen, device=device).to(BF)
    k = torch.randn(B, H, Sk, 128, generator=gen, device=device).to(BF)
    v = torch.randn(B, H, Sk, 128, generator=gen, device=device).to(BF)
    attn = pkg.make_attention()
    graph_out, eager_out = torch.empty_like(q), torch.empty_like(q)
    attn(q, k, v, 0.09, graph_out)  # warm-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            attn(q, k, v, 0.09, graph_out)
    torch.cuda.synchronize()
    for replay in range(3):
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, generator=gen, device=device).to(BF))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        attn(q, k, v, 0.09, eager_out)
        torch.cuda.synchronize()
        assert_bitwise(graph_out, eager_out, f"replay {replay}")


def test_fp8_configuration_pipeline_graph_replays_match_eager(pkg, device):
    """The fp8 configuration's pipeline -- the two-term q/k/v pack that folds
    V's amax into slots (cleared by a fill kernel inside the launcher), V^T
    quantised from those slots, and the two-term fp8 attention -- captured
    once and replayed three times with the projected rows rewritten between
    replays. Each replay is bitwise equal to the same chain run eagerly into
    separate outputs, so the slots start from zero on every replay."""
    from test_qkv_pack import _case
    T, P, Hs = 1024, 1, 4
    projected, wq, wk, cache, positions = _case(T, P, Hs, 7, device)
    projected, wq, wk, cache, positions = (t.to(device) for t in (projected, wq, wk, cache, positions))
    q, k, v = pkg.qkv_by_rank(projected, P)
    pack, attn = pkg.make_qkv_norm_rope_pack_fp8x2_vamax(), pkg.make_attention_fp8x2()
    bhsd = lambda t: t[:, 0].unsqueeze(0).transpose(1, 2)  # noqa: E731  [T, 1, Hs, 128] -> [1, Hs, T, 128]

    def outputs():
        o = {n: torch.empty(T, P, Hs, 128, dtype=torch.float8_e4m3fn, device=device) for n in ("q8", "ql", "k8", "kl")}
        o["v"] = torch.zeros(T, P, Hs, 128, dtype=BF, device=device)
        o.update({n: torch.empty(Hs, device=device) for n in ("qd", "kd")})
        o["slots"] = torch.empty(Hs, pkg._lib.AMAX_SLOTS, device=device)
        o["v8"], o["vd"] = pkg.quantize_fp8_per_head(bhsd(o["v"]).contiguous(), transposed=True)
        o["out"] = torch.empty(1, Hs, T, 128, dtype=BF, device=device)
        return o

    def chain(o):
        pack(q, k, v, wq, wk, 1e-6, cache, positions, o["q8"], o["ql"], o["k8"], o["kl"], o["v"], o["qd"], o["kd"],
             o["slots"])
        pkg.quantize_fp8_per_head(bhsd(o["v"]), transposed=True, x8=o["v8"], descale=o["vd"], amax_slots=o["slots"])
        attn(bhsd(o["q8"]), bhsd(o["ql"]), bhsd(o["k8"]), bhsd(o["kl"]), o["v8"], o["qd"], o["kd"], o["vd"],
             128 ** -0.5, o["out"])

    graph_out, eager_out = outputs(), outputs()
    torch.cuda.synchronize()
    chain(graph_out)  # warm-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            chain(graph_out)
    torch.cuda.synchronize()
    gen = torch.Generator(device=device).manual_seed(13)
    for replay in range(3):
        # Smaller rows on each later replay: slots left from an earlier
        # replay would exceed the new maxima, so a missed clear changes V's
        # descale and codes.
        projected.copy_((torch.randn(projected.shape, generator=gen, device=device) * (3 - replay)).to(BF))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        chain(eager_out)
        torch.cuda.synchronize()
        assert_bitwise(graph_out["out"], eager_out["out"], f"replay {replay}: attention")
        assert_bitwise(graph_out["v"], eager_out["v"], f"replay {replay}: v")
        for n in ("q8", "ql", "k8", "kl", "v8"):
            assert torch.equal(graph_out[n].view(torch.uint8), eager_out[n].view(torch.uint8)), (replay, n)
        for n in ("qd", "kd", "vd", "slots"):
            assert torch.equal(graph_out[n], eager_out[n]), (replay, n)

"""launch_h3_qkv_norm_rope_pack_fp8_noalloc, the allocation-free pack: V's
amax slots live in the library's static device array instead of a caller's
buffer. Through the C ABI, against the two calls it stands for
(launch_h3_qkv_norm_rope_pack_fp8_vamax with a caller's slot buffer, then
launch_h3_quantize_fp8_per_head_slots): bitwise on every output, over calls in
a row whose inputs shrink and grow (the array keeps the previous call's
contents), up to the array's 1024 heads."""
from __future__ import annotations

import pytest
import torch

from conftest import assert_bitwise
from test_qkv_pack import _case

BF = torch.bfloat16


def _v8_view(T, Hs, device, fill):
    """A [1, Hs, T, 128] uint8 view stored S-contiguous (S padded to 16), the
    layout the fp8 attention reads V in, filled with `fill`."""
    store = torch.full((1, Hs, 128, -(-T // 16) * 16), fill, dtype=torch.uint8, device=device)
    return store[..., :T].transpose(2, 3)


def _pack_args(L, q, k, v, wq, wk, cache, positions, q8, k8, v_out, q_descale, k_descale):
    return [L.tensor(q), L.tensor(k), L.tensor(v), L.tensor(wq), L.tensor(wk), L.scalar(1e-6),
            L.tensor(cache[:, :48]), L.tensor(cache[:, 48:]), L.tensor(positions), L.tensor(q8), L.tensor(k8),
            L.tensor(v_out), L.tensor(q_descale), L.tensor(k_descale)]


@pytest.mark.gpu
def test_noalloc_pack_equals_the_two_calls(pkg, device):
    L = pkg._lib
    stream = torch.cuda.current_stream(device).cuda_stream
    # Second call smaller than the first; then the most heads the array holds;
    # then one head.
    for T, Hs, seed in ((3000, 14, 1), (700, 6, 2), (33, L.NOALLOC_MAX_HEADS, 3), (5, 1, 4)):
        print(f"noalloc pack T={T} Hs={Hs}", flush=True)
        projected, wq, wk, cache, positions = _case(T, 1, Hs, seed, device)
        projected[T // 3, 2, Hs - 1, 5] = -29.0  # one head's amax is a single element
        q, k, v = pkg.qkv_by_rank(projected.to(device), 1)
        wq, wk, cache, positions = wq.to(device), wk.to(device), cache.to(device), positions.to(device)
        outs = {}
        for route in ("two_calls", "noalloc"):
            q8 = torch.full((T, 1, Hs, 128), 0x7F, dtype=torch.uint8, device=device)
            k8 = torch.full_like(q8, 0x7F)
            v_out = torch.full((T, 1, Hs, 128), float("nan"), dtype=BF, device=device)
            q_descale, k_descale, v_descale = (torch.full((Hs,), float("nan"), device=device) for _ in range(3))
            v8 = _v8_view(T, Hs, device, 0x7F)
            args = _pack_args(L, q, k, v, wq, wk, cache, positions, q8, k8, v_out, q_descale, k_descale)
            v_rows = v_out[:, 0].unsqueeze(0).transpose(1, 2)  # [1, Hs, T, 128]
            if route == "two_calls":
                slots = torch.full((Hs, L.AMAX_SLOTS), float("nan"), device=device)
                assert L.call("launch_h3_qkv_norm_rope_pack_fp8_vamax", stream, *args, L.tensor(slots)) == 0
                assert L.call("launch_h3_quantize_fp8_per_head_slots", stream, L.tensor(v_rows), L.tensor(slots),
                              L.tensor(v8), L.tensor(v_descale)) == 0
            else:
                assert L.call("launch_h3_qkv_norm_rope_pack_fp8_noalloc", stream, *args, L.tensor(v8),
                              L.tensor(v_descale)) == 0
            torch.cuda.synchronize()
            outs[route] = (q8.cpu(), k8.cpu(), v_out.cpu(), q_descale.cpu(), k_descale.cpu(), v8.cpu(),
                           v_descale.cpu())
        ref, got = outs["two_calls"], outs["noalloc"]
        for name, a, b in zip(("q8", "k8", "v_out", "q_descale", "k_descale", "v8", "v_descale"), got, ref):
            if a.dtype == BF:
                assert_bitwise(a, b, name)
            else:
                assert torch.equal(a, b), (T, Hs, name)
        assert float(ref[6].max()) * 448 == pytest.approx(29.0, rel=1e-6)
        assert not torch.isnan(ref[6]).any() and not (ref[5] == 0x7F).all()


@pytest.mark.gpu
def test_noalloc_pack_python_face(pkg, device):
    """The Python face of the same entry point equals the C ABI call."""
    T, Hs = 257, 5
    projected, wq, wk, cache, positions = _case(T, 1, Hs, 9, device)
    q, k, v = pkg.qkv_by_rank(projected.to(device), 1)
    wq, wk, cache, positions = wq.to(device), wk.to(device), cache.to(device), positions.to(device)
    res = []
    for _ in range(2):
        q8 = torch.zeros(T, 1, Hs, 128, dtype=torch.float8_e4m3fn, device=device)
        k8 = torch.zeros_like(q8)
        v_out = torch.empty(T, 1, Hs, 128, dtype=BF, device=device)
        q_descale, k_descale, v_descale = (torch.zeros(Hs, device=device) for _ in range(3))
        v8 = _v8_view(T, Hs, device, 0).view(torch.float8_e4m3fn)
        pkg.make_qkv_norm_rope_pack_fp8_noalloc()(q, k, v, wq, wk, 1e-6, cache, positions, q8, k8, v_out,
                                                  q_descale, k_descale, v8, v_descale)
        torch.cuda.synchronize()
        res.append([t.cpu().view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t.cpu()
                    for t in (q8, k8, v_out, q_descale, k_descale, v8, v_descale)])
    for a, b in zip(*res):
        if a.dtype == BF:
            assert_bitwise(a, b)
        else:
            assert torch.equal(a, b)
    ref8, refd = pkg.quantize_fp8_per_head(res[0][2].to(device)[:, 0].unsqueeze(0).transpose(1, 2),
                                           transposed=True)
    assert torch.equal(refd.cpu(), res[0][6])
    assert torch.equal(ref8.cpu().view(torch.uint8), res[0][5])


_CAPTURE_SCRIPT = r'''
import sys
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
import importlib
import torch
from test_qkv_pack import _case
from test_zz_no_alloc import _v8_view, _pack_args

pkg = importlib.import_module("minimaxh3_on_k100-ai_amd")
L = pkg._lib
device = torch.device("cuda:0")
BF = torch.bfloat16
T, Hs = 1000, 6
projected, wq, wk, cache, positions = _case(T, 1, Hs, 13, device)
projected = projected.to(device)
q, k, v = pkg.qkv_by_rank(projected, 1)
wq, wk, cache, positions = wq.to(device), wk.to(device), cache.to(device), positions.to(device)


def buffers():
    q8 = torch.zeros(T, 1, Hs, 128, dtype=torch.uint8, device=device)
    return dict(q8=q8, k8=torch.zeros_like(q8), v_out=torch.zeros(T, 1, Hs, 128, dtype=BF, device=device),
                qd=torch.zeros(Hs, device=device), kd=torch.zeros(Hs, device=device),
                v8=_v8_view(T, Hs, device, 0), vd=torch.zeros(Hs, device=device))


def args(b):
    return _pack_args(L, q, k, v, wq, wk, cache, positions, b["q8"], b["k8"], b["v_out"], b["qd"], b["kd"])


graph_b, eager_b = buffers(), buffers()
side = torch.cuda.Stream()
graph = torch.cuda.CUDAGraph()
torch.cuda.synchronize()
print("capturing the first allocation-free call of this process", flush=True)
with torch.cuda.stream(side):
    with torch.cuda.graph(graph, stream=side):
        rc = L.call("launch_h3_qkv_norm_rope_pack_fp8_noalloc", side.cuda_stream, *args(graph_b),
                    L.tensor(graph_b["v8"]), L.tensor(graph_b["vd"]))
assert rc == 0, rc
torch.cuda.synchronize()
gen = torch.Generator(device=device).manual_seed(3)
stream = torch.cuda.current_stream(device).cuda_stream
for replay in range(3):
    projected.copy_((torch.randn(projected.shape, generator=gen, device=device) * (1 + replay)).to(BF))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    slots = torch.full((Hs, L.AMAX_SLOTS), float("nan"), device=device)
    assert L.call("launch_h3_qkv_norm_rope_pack_fp8_vamax", stream, *args(eager_b), L.tensor(slots)) == 0
    v_rows = eager_b["v_out"][:, 0].unsqueeze(0).transpose(1, 2)
    assert L.call("launch_h3_quantize_fp8_per_head_slots", stream, L.tensor(v_rows), L.tensor(slots),
                  L.tensor(eager_b["v8"]), L.tensor(eager_b["vd"])) == 0
    torch.cuda.synchronize()
    for name in graph_b:
        a, b = graph_b[name], eager_b[name]
        same = torch.equal(a.view(torch.int16), b.view(torch.int16)) if a.dtype == BF else torch.equal(a, b)
        assert same, (replay, name)
    print(f"replay {replay} bitwise", flush=True)
print("CAPTURE_OK", flush=True)
'''


@pytest.mark.gpu
def test_noalloc_pack_first_call_inside_graph_capture(device):
    """In a fresh process (so the device's slot address is not yet looked up),
    the first call of launch_h3_qkv_norm_rope_pack_fp8_noalloc is made inside
    a HIP graph capture; the graph is replayed three times, the projection
    rewritten by eager work before each replay, and every output of every
    replay equals the two-call sequence (caller's slots) run eagerly on the
    same inputs, bitwise."""
    import subprocess
    import sys
    from pathlib import Path
    root = str(Path(__file__).resolve().parents[1])
    proc = subprocess.run([sys.executable, "-u", "-c", _CAPTURE_SCRIPT, root], capture_output=True, text=True,
                          timeout=240)
    print(proc.stdout[-2000:], proc.stderr[-2000:])
    assert proc.returncode == 0 and "CAPTURE_OK" in proc.stdout, proc.returncode

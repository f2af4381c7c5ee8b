#!/usr/bin/env python3
"""Benchmark of the H3 DiT hot path on one MI355X.

Headline (one JSON line on stdout): non-causal bf16 attention forward at
S = 73,984 (32x48x48 video latents + 256 text tokens), H = 14, D = 128, B = 1,
q/k/v ~ N(0, 1) with 1% of key rows x8, in the [B, S, H, D] layout the
reference's MHA operator receives. One step = one attention forward over the
whole sequence; value = 4*B*H*S^2*D flops / seconds per step (the reference's
formula, tools/bench_h3_ops.py:125).

Extra fields on the same line:
  roofline      the attention kernel against the bf16 dense MFMA peak
  cpu_baseline  the CPU oracle's fp32 attention on a bounded sample of the same
                workload, on this host's cores
  pointwise     GB/s of each fused pointwise op at its configuration size
                (q/k [1, 8192, 14, 128]; [8192, 7168] / [8192, 18432]), timed
                as back-to-back launches in a HIP graph over rotating buffers
                larger than the 256 MB last-level cache; beside the
                configuration ops, the reference's torch CPU path (cpu_us)
  attention_s8192, fp8   further attention configurations; the fp8 entry's
                config5 is the Q/K/V-in-e4m3 variant that meets the fp8
                configuration's accuracy bar (relative RMS <= 5e-2, measured here
                on sampled rows), beside the bf16-logit variant and the one-term
                recipe that misses the bar, each with the fp8 MFMA work it
                executes against the part's sustained fp8 rate
  vendor_sdpa   torch's own fused SDPA kernel on the same inputs (the
                reference's production route, patches/InfiniCore.patch:1293-1332),
                timed beside the hand kernel at S = 73,984 and S = 8192
  attention_key_split   the key split of a partly filled last round of
                workgroups against the unsplit launch, on two shapes it splits
  attention_head_groups   two head groups of 7, each group's q, k, v copied on
                a second stream while the previous group computes (the
                all-to-all overlap of patches/InfiniLM.patch:960-1018 with a
                device copy in its place), against one 14-head launch
  mfma_peak_measured    the bf16 (per product shape) and fp8 MFMA rates the
                part sustains with random and with zero operands, and the
                headline's fraction of the bf16 random-operand rates
"""
from __future__ import annotations

import argparse
import hashlib
import re
import importlib
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
METRIC = "attn TFLOP/s (% MFMA peak) at S=73,984 H=14 D=128; fused-op HBM GB/s"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def attention_inputs_gpu(S: int, H: int, seed: int, outlier_fraction: float, device):
    """q, k, v [1, S, H, 128] bf16 ~ N(0, 1) from a seeded device generator;
    `outlier_fraction` of key rows scaled x8 (exact in bf16)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    q, k, v = (torch.randn(1, S, H, 128, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
               for _ in range(3))
    if outlier_fraction > 0:
        rows = torch.randperm(S, generator=gen, device=device)[: int(round(S * outlier_fraction))]
        k[:, rows] *= 8
    return q, k, v


def kernel_source_digest() -> str:
    """sha256 (16 hex digits) of the bf16 attention kernel's sources with their
    comments removed and whitespace collapsed: a profile records it, and its
    HBM-traffic figure is used only while the code still matches (an edit to a
    comment or to layout leaves it)."""
    h = hashlib.sha256()
    for name in ("h3_attention.hip", "h3_common.hpp"):
        text = (ROOT / "minimaxh3_on_k100-ai_amd" / "csrc" / name).read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        h.update(" ".join(text.split()).encode())
    return h.hexdigest()[:16]


def profiled_traffic() -> dict:
    """HBM bytes per launch of the headline kernel from its FETCH_SIZE /
    WRITE_SIZE profile, with the digest of the sources that profile measured;
    traffic is null when the sources changed since."""
    profile = ROOT / "profiles" / "attention_bf16_s73984_traffic.md"
    fields = {}
    if profile.exists():
        for text_line in profile.read_text().splitlines():
            key, sep, value = text_line.partition(":")
            if sep and key in ("hbm_bytes_per_launch", "csrc_digest"):
                fields[key] = value.strip()
    digest = kernel_source_digest()
    fresh = "hbm_bytes_per_launch" in fields and fields.get("csrc_digest") == digest
    return {"traffic": int(fields["hbm_bytes_per_launch"]) if fresh else None,
            "traffic_source": {"profile": "profiles/attention_bf16_s73984_traffic.md",
                               "profile_csrc_digest": fields.get("csrc_digest"), "csrc_digest": digest,
                               "stale": not fresh}}


def sampled_rel_rms(out, q, k, v, scale: float, rows) -> float:
    """Relative RMS of out[:, :, rows] (bf16 [B, H, S, D] views) against fp32
    softmax(q k^T scale) v of those rows, computed on the GPU in fp32."""
    kt = k.float().transpose(-2, -1).contiguous()
    vf = v.float().contiguous()
    num, den = 0.0, 0.0
    for r0 in range(0, rows.numel(), 512):
        sel = rows[r0:r0 + 512]
        logits = torch.matmul(q[:, :, sel].float().contiguous(), kt) * scale
        ref = torch.matmul(torch.softmax(logits, dim=-1), vf)
        num += float((out[:, :, sel].float() - ref).double().pow(2).sum())
        den += float(ref.double().pow(2).sum())
        del logits, ref
    return math.sqrt(num / den)


def vendor_sdpa(q, k, v, scale: float, ours, steps: int, warmup: int = 1) -> dict:
    """torch's fused SDPA on [B, H, S, D] views of the [B, S, H, D] inputs, the
    reference's vendor route (patches/InfiniCore.patch:1301-1313;
    tools/bench_vendor_attention.py:19-33). Only the fused backends are
    allowed, in torch's priority order (flash, then memory-efficient): the
    first that accepts the inputs is the one torch's default picks. The math
    backend is never run (it would materialise the S x S scores). Returns its
    ms, TFLOP/s and the relative RMS of its output against the hand kernel's."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    import torch.nn.functional as F
    B, H, S, D = q.shape
    flops = 4.0 * B * H * S * S * D
    for backend in (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION):
        try:
            with sdpa_kernel([backend]):
                out = F.scaled_dot_product_attention(q, k, v, scale=scale)
                ms = time_launches(lambda: F.scaled_dot_product_attention(q, k, v, scale=scale), steps, warmup)
        except RuntimeError as exc:
            log(f"  vendor SDPA {backend.name}: not available ({str(exc)[:80]})")
            continue
        d = (out.float() - ours.float()).double()
        rel = float(d.norm() / ours.double().norm())
        return {"backend": backend.name, "ms": round(ms, 4), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2),
                "rel_rms_vs_hand_kernel": round(rel, 6), "torch": torch.__version__}
    return {"backend": None, "note": "no fused SDPA backend accepted the inputs"}


def time_launches(fn, steps: int, warmup: int) -> float:
    """Mean milliseconds per call: `warmup` untimed calls, then `steps` calls
    bracketed by synchronize + HIP events on the launch stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def graph_kernel_time(calls, replays: int = 10) -> float | None:
    """Milliseconds of device kernel time per call of `calls` (the library's
    kernels only), from torch's profiler over `replays` replays of one HIP
    graph of them: the kernels' own durations, without the gaps between
    graph nodes that time_graph's per-launch figure includes. None unless the
    profiler records at least one kernel per call and replay (under an outside
    tracer such as rocprofv3 it sees only some of them)."""
    from torch.profiler import ProfilerActivity, profile
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for c in calls:
                c()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        for _ in range(replays):
            graph.replay()
        torch.cuda.synchronize()
    total_us = 0.0
    found = 0
    for e in prof.events():
        if "h3::" in e.name:
            total_us += getattr(e, "device_time_total", None) or e.cuda_time_total
            found += 1
    if found < replays * len(calls):
        return None
    return total_us / 1e3 / (replays * len(calls))


def time_graph(calls, repeats: int = 20, rounds: int = 5) -> float:
    """Milliseconds per launch of `calls` (a list of zero-argument launches)
    captured back to back in one HIP graph: the median over `rounds` rounds of
    the mean over `repeats` replays (a round of the shortest ops lasts about
    3 ms, which a passing clock transient can move by several percent)."""
    for c in calls:
        c()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for c in calls:
                c()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    per_round = []
    for _ in range(rounds):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(repeats):
            graph.replay()
        end.record(stream)
        torch.cuda.synchronize()
        per_round.append(start.elapsed_time(end) / (repeats * len(calls)))
    return statistics.median(per_round)


def pattern_ceilings(pkg, device, read_bytes: int, n_in: int, n_out: int, row_bytes: int | None) -> dict:
    """Times the measurement copies with an op's bytes: n_in inputs and n_out
    outputs of read_bytes each, as one flat non-temporal stream and (row_bytes
    given) as whole rows with one wave per row -- the pattern's practical
    ceiling on this part. Buffers rotate past the 256 MB last-level cache."""
    cal = pkg.h3_calibration
    rot = max(2, -(-512 * 2 ** 20 // (read_bytes * (n_in + n_out))))
    sets = [([torch.empty(read_bytes, dtype=torch.uint8, device=device) for _ in range(n_in)],
             [torch.empty(read_bytes, dtype=torch.uint8, device=device) for _ in range(n_out)]) for _ in range(rot)]
    for ins, _ in sets:
        for t in ins:
            t.random_(0, 256)
    total = read_bytes * (n_in + n_out)
    out = {}

    def entry(calls):
        ms = time_graph(calls)
        gbs = total / (ms * 1e-3) / 1e9
        e = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        kms = graph_kernel_time(calls)
        if kms is not None:
            e["kernel_us"] = round(kms * 1e3, 2)
            e["kernel_frac"] = round(total / (kms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        return e

    out["stream"] = entry([lambda i=i, o=o: cal.stream(i[0], o[0], *(i[1:] + o[1:2] if n_in > 1 else ()))
                           for i, o in sets])
    if row_bytes:
        out["row_copy"] = entry([lambda i=i, o=o: cal.row_copy(
            i[0], o[0], row_bytes, *(i[1:] + o[1:2] if n_in > 1 else ())) for i, o in sets])
    del sets
    return out


def bench_pointwise(pkg, device) -> dict:
    """GB/s per op; bytes = compulsory bf16 reads + writes (broadcast vectors
    counted once). `us` / `frac`: per launch of a captured HIP graph of
    back-to-back launches (the gaps between graph nodes included);
    `kernel_us` / `kernel_frac`: the kernels' own device durations in the same
    graph, from torch's profiler (the figure a kernel trace gives). Beside each
    configuration op, `ceiling`: the same bytes moved by a plain stream and
    (for the row-complete RMS family) by whole-row copies, timed the same two
    ways, and `frac_of_ceiling` / `kernel_frac_of_ceiling`, the op's time
    against the best of them."""
    results = {}
    gen = torch.Generator(device=device).manual_seed(0)
    bf = torch.bfloat16

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=gen, device=device) * scale).to(bf)

    last_calls: list = []

    def timed(calls):
        last_calls[:] = calls
        return time_graph(calls)

    def record(name, ms, nbytes, shape):
        gbs = nbytes / (ms * 1e-3) / 1e9
        results[name] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "bytes": nbytes, "shape": shape}
        kms = graph_kernel_time(last_calls)
        extra = ""
        if kms is not None:
            kgbs = nbytes / (kms * 1e-3) / 1e9
            results[name].update({"kernel_us": round(kms * 1e3, 2), "kernel_GB/s": round(kgbs, 1),
                                  "kernel_frac": round(kgbs / HBM_PEAK_GBS, 4)})
            extra = f"; kernel alone {kms * 1e3:.2f} us ({kgbs / HBM_PEAK_GBS:.1%})"
        log(f"  {name:34s} {ms * 1e3:8.2f} us  {gbs:8.1f} GB/s  ({gbs / HBM_PEAK_GBS:.1%} of HBM peak){extra}")

    def ceiling(name, read_bytes, n_in, n_out, row_bytes):
        entry = results[name]
        entry["ceiling"] = pattern_ceilings(pkg, device, read_bytes, n_in, n_out, row_bytes)
        best = min(c["us"] for c in entry["ceiling"].values())
        entry["frac_of_ceiling"] = round(best / entry["us"], 4)
        kbest = [c["kernel_us"] for c in entry["ceiling"].values() if "kernel_us" in c]
        if kbest and "kernel_us" in entry:
            entry["kernel_frac_of_ceiling"] = round(min(kbest) / entry["kernel_us"], 4)
        log(f"  {'':34s} same bytes: " + ", ".join(
            f"{k} {c['us']:.2f} us ({c['frac']:.1%}; kernel alone {c.get('kernel_us', float('nan')):.2f} us)"
            for k, c in entry["ceiling"].items()) + f"; op at {entry['frac_of_ceiling']:.1%} of the best")

    # q/k RMSNorm + RoPE, [1, 8192, 14, 128] per tensor, both layouts.
    T, H = 8192, 14
    rot = 12  # 12 x 2 x 29 MB > 512 MB
    xs = [rnd(T, 1, H, 128) for _ in range(rot)]
    outs = [torch.empty_like(x) for x in xs]
    w = rnd(128, scale=0.1) + 1
    table64 = rnd(T, 128)
    table48 = rnd(T, 96)
    k_int = pkg.make_qk_norm_rope_interleaved()
    k_rh = pkg.make_qk_norm_rope()
    nbytes = 2 * T * H * 128 * 2 + T * 64 * 2 * 2 + 128 * 2
    ms = timed([lambda x=x, o=o: k_int(x, w, 1e-6, table64[:, :64], table64[:, 64:], o) for x, o in zip(xs, outs)])
    record("qk_norm_rope_interleaved", ms, nbytes, [T, 1, H, 128])
    nbytes = 2 * T * H * 128 * 2 + T * 48 * 2 * 2 + 128 * 2
    ms = timed([lambda x=x, o=o: k_rh(x, w, 1e-6, table48[:, :48], table48[:, 48:], o) for x, o in zip(xs, outs)])
    record("qk_norm_rope", ms, nbytes, [T, 1, H, 128])
    # q and k in one pass (the fused QK-RMSNorm + 3D RoPE workload: 2 x 58.7 MB
    # of head rows + the [8192, 64] x 2 table + two weights).
    k_qk = pkg.make_qk_norm_rope_interleaved_qk()
    w2 = rnd(128, scale=0.1) + 1
    nbytes = 4 * T * H * 128 * 2 + T * 64 * 2 * 2 + 2 * 128 * 2
    ms = timed([lambda i=i: k_qk(xs[2 * i], xs[2 * i + 1], w, w2, 1e-6, table64[:, :64], table64[:, 64:],
                                      outs[2 * i], outs[2 * i + 1]) for i in range(rot // 2)])
    record("qk_norm_rope_interleaved_qk", ms, nbytes, [2, T, 1, H, 128])
    ceiling("qk_norm_rope_interleaved_qk", 2 * T * H * 128 * 2, 1, 1, None)
    del xs, outs
    # q, k and v of one head group in one launch: by-rank views of the fused
    # [T, 3, H, 128] projection in, [1, T, H, 128] send buffers out, RoPE cache
    # rows gathered by a permutation of the positions.
    projs = [rnd(T, 3, H, 128) for _ in range(3)]
    sends = [torch.empty(3, 1, T, H, 128, dtype=bf, device=device) for _ in range(3)]
    views = [(pkg.qkv_by_rank(p, 1), [s[i].permute(1, 0, 2, 3) for i in range(3)]) for p, s in zip(projs, sends)]
    positions = torch.randperm(T, device=device)
    k_pack = pkg.make_qkv_norm_rope_pack()
    nbytes = 6 * T * H * 128 * 2 + T * 8 + T * 96 * 2 + 2 * 128 * 2
    ms = timed([lambda i=i, o=o: k_pack(*i, w, w, 1e-6, table48, positions, *o) for i, o in views])
    record("qkv_norm_rope_pack", ms, nbytes, [T, 1, H, 128])
    # The same with the fp8 epilogue: q and k leave as e4m3 codes.
    codes = [torch.empty(2, 1, T, H, 128, dtype=torch.float8_e4m3fn, device=device) for _ in range(3)]
    descales = torch.empty(2, H, device=device)
    views8 = [(i, [c[0].permute(1, 0, 2, 3), c[1].permute(1, 0, 2, 3), o[2]]) for (i, o), c in zip(views, codes)]
    k_pack8 = pkg.make_qkv_norm_rope_pack_fp8()
    nbytes = 3 * T * H * 128 * 2 + 2 * T * H * 128 + T * H * 128 * 2 + T * 8 + T * 96 * 2 + 2 * 128 * 2
    ms = timed([lambda i=i, o=o: k_pack8(*i, w, w, 1e-6, table48, positions, *o, descales[0], descales[1])
                     for i, o in views8])
    record("qkv_norm_rope_pack_fp8", ms, nbytes, [T, 1, H, 128])
    # The same with V's per-head amax folded into slots while v is copied.
    k_pack8v = pkg.make_qkv_norm_rope_pack_fp8_vamax()
    v_amax = torch.empty(H, 64, device=device)
    ms = timed([lambda i=i, o=o: k_pack8v(*i, w, w, 1e-6, table48, positions, *o, descales[0], descales[1],
                                                v_amax) for i, o in views8])
    record("qkv_norm_rope_pack_fp8_vamax", ms, nbytes, [T, 1, H, 128])
    # The same with two-term q and k codes (the fp8 configuration's recipe): lo codes beside the hi ones.
    codes_lo = [torch.empty(2, 1, T, H, 128, dtype=torch.float8_e4m3fn, device=device) for _ in range(3)]
    k_pack8x2 = pkg.make_qkv_norm_rope_pack_fp8x2_vamax()
    nbytes2 = nbytes + 2 * T * H * 128
    ms = timed([lambda i=i, o=o, c=c: k_pack8x2(*i, w, w, 1e-6, table48, positions, o[0],
                                                      c[0].permute(1, 0, 2, 3), o[1], c[1].permute(1, 0, 2, 3), o[2],
                                                      descales[0], descales[1], v_amax)
                     for (i, o), c in zip(views8, codes_lo)])
    record("qkv_norm_rope_pack_fp8x2_vamax", ms, nbytes2, [T, 1, H, 128])
    del projs, sends, views, codes, views8, codes_lo

    S, C, F = 8192, 7168, 18432
    rot = 3
    xs = [rnd(1, S, C) for _ in range(rot)]
    ys = [rnd(1, S, C) for _ in range(rot)]
    outs = [torch.empty_like(x) for x in xs]
    res = [torch.empty_like(x) for x in xs]
    wC = rnd(C, scale=0.1) + 1
    scale = rnd(1, 1, C, scale=0.1).expand(1, S, C)
    shift = rnd(1, 1, C, scale=0.1).expand(1, S, C)
    gate = rnd(1, 1, C, scale=0.1).expand(1, S, C)
    k_mod = pkg.make_rms_modulate()
    ms = timed([lambda x=x, o=o: k_mod(x, wC, 1e-6, scale, shift, o) for x, o in zip(xs, outs)])
    record("rms_modulate", ms, 2 * S * C * 2 + 3 * C * 2, [1, S, C])
    ceiling("rms_modulate", S * C * 2, 1, 1, C * 2)
    k_gr = pkg.make_gated_residual()
    ms = timed([lambda x=x, y=y, o=o: k_gr(x, gate, y, o) for x, y, o in zip(xs, ys, outs)])
    record("gated_residual", ms, 3 * S * C * 2 + C * 2, [1, S, C])
    ceiling("gated_residual", S * C * 2, 2, 1, None)
    k_grm = pkg.make_gated_residual_rms_modulate()
    ms = timed([lambda x=x, y=y, o=o, r=r: k_grm(x, gate, y, wC, 1e-6, scale, shift, r, o)
                     for x, y, o, r in zip(xs, ys, outs, res)])
    record("gated_residual_rms_modulate", ms, 4 * S * C * 2 + 4 * C * 2, [1, S, C])
    ceiling("gated_residual_rms_modulate", S * C * 2, 2, 2, C * 2)
    # The same three ops with per-token AdaLN rows: two runs of tokens (1/8 and
    # 7/8 of S) taking rows 0 and 1 of the [2, 6C] modulation matrix.
    R = 2
    cols = pkg.modulation_columns(rnd(R, 6 * C, scale=0.1), C)
    index = torch.cat([torch.zeros(S // 8, dtype=torch.int64), torch.ones(S - S // 8, dtype=torch.int64)])
    index = index.to(device).view(1, S)
    tables = R * C * 2
    k_mod_i = pkg.make_rms_modulate_indexed(check_indices=False)
    ms = timed([lambda x=x, o=o: k_mod_i(x, wC, 1e-6, cols["scale_msa"], cols["shift_msa"], index, o)
                     for x, o in zip(xs, outs)])
    record("rms_modulate_indexed", ms, 2 * S * C * 2 + C * 2 + 2 * tables + S * 8, [1, S, C])
    k_gr_i = pkg.make_gated_residual_indexed(check_indices=False)
    ms = timed([lambda x=x, y=y, o=o: k_gr_i(x, cols["gate_mlp"], y, index, o) for x, y, o in zip(xs, ys, outs)])
    record("gated_residual_indexed", ms, 3 * S * C * 2 + tables + S * 8, [1, S, C])
    k_grm_i = pkg.make_gated_residual_rms_modulate_indexed(check_indices=False)
    ms = timed([lambda x=x, y=y, o=o, r=r: k_grm_i(x, cols["gate_msa"], y, wC, 1e-6, cols["scale_mlp"],
                                                        cols["shift_mlp"], index, r, o)
                     for x, y, o, r in zip(xs, ys, outs, res)])
    record("gated_residual_rms_modulate_indexed", ms, 4 * S * C * 2 + C * 2 + 3 * tables + S * 8, [1, S, C])
    del xs, ys, outs, res
    ups = [rnd(1, S, F) for _ in range(2)]
    gates = [rnd(1, S, F) for _ in range(2)]
    outs = [torch.empty_like(u) for u in ups]
    k_sw = pkg.make_swiglu()
    ms = timed([lambda u=u, g=g, o=o: k_sw(u, g, o) for u, g, o in zip(ups, gates, outs)])
    record("swiglu", ms, 3 * S * F * 2, [1, S, F])
    del ups, gates, outs
    ceiling("swiglu", S * F * 2, 2, 1, None)
    return results


def cpu_host() -> dict:
    """The host CPU the CPU figures run on: its model, the CPUs the OS reports
    and the ones this process may run on, and torch's thread count (the
    threads every CPU figure uses: a host that grants a job a share of its
    CPUs sets OMP_NUM_THREADS to it, which torch follows)."""
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"cpu_model": model, "host_cpus": os.cpu_count(), "usable_cpus": usable,
            "threads": torch.get_num_threads()}


def median_time(fn, warmup: int = 3, runs: int = 5) -> float:
    """Median seconds of `runs` calls after `warmup` untimed ones."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_reference_path(device, pointwise: dict | None, attention_s8192: dict | None) -> None:
    """The reference's torch CPU path beside each measured op: the oracle's
    restatement of the torch compositions (order="torch", the literal eager
    sums; tools/bench_h3_ops.py:81-113,145-149,215,232-234,251-254) at the
    configuration sizes, the median of 5 runs after 3 warm-ups each, on this
    host's threads; and the fp32 attention at S = 8192, H = 14 (the median of 3
    runs after one warm-up). Adds "cpu_us" /
    "cpu_GB/s" (same algorithmic bytes as the GPU figure) to the pointwise
    entries and "cpu_TFLOP/s" to the S = 8192 line. Inputs are drawn on the
    GPU from a seeded generator and copied to the host (same shapes and
    distributions as the GPU runs)."""
    from oracle import h3_oracle
    gen = torch.Generator(device=device).manual_seed(1)
    bf = torch.bfloat16

    def rnd(*shape, scale=1.0, offset=0.0):
        return (torch.randn(*shape, generator=gen, device=device) * scale + offset).to(bf).cpu()

    timed = median_time
    threads = torch.get_num_threads()

    def note(name, seconds):
        if pointwise is None or name not in pointwise:
            return
        entry = pointwise[name]
        entry["cpu_us"] = round(seconds * 1e6, 1)
        entry["cpu_GB/s"] = round(entry["bytes"] / seconds / 1e9, 2)
        log(f"  cpu {name:30s} {seconds * 1e3:9.1f} ms  {entry['cpu_GB/s']:7.2f} GB/s  ({threads} threads)")

    if pointwise is not None:
        T, H = 8192, 14
        q, k = rnd(T, 1, H, 128), rnd(T, 1, H, 128)
        wq, wk = rnd(128, scale=0.1, offset=1.0), rnd(128, scale=0.1, offset=1.0)
        cos, sin = h3_oracle.rope_table_interleaved(h3_oracle.grid_positions(8, 32, 32))
        note("qk_norm_rope_interleaved_qk", timed(lambda: [h3_oracle.qk_norm_rope_interleaved(
            x, w, 1e-6, cos, sin, order="torch") for x, w in ((q, wq), (k, wk))]))
        del q, k
        S, C, F = 8192, 7168, 18432
        x, y = rnd(1, S, C), rnd(1, S, C)
        w = rnd(C, scale=0.1, offset=1.0)
        scale, shift, gate = (rnd(1, 1, C, scale=0.1) for _ in range(3))
        note("rms_modulate", timed(lambda: h3_oracle.rms_modulate(x, w, 1e-6, scale, shift, order="torch")))
        note("gated_residual", timed(lambda: h3_oracle.gated_residual(x, gate, y)))
        note("gated_residual_rms_modulate", timed(lambda: h3_oracle.gated_residual_rms_modulate(
            x, gate, y, w, 1e-6, scale, shift, order="torch")))
        del x, y
        up, gact = rnd(1, S, F), rnd(1, S, F)
        note("swiglu", timed(lambda: h3_oracle.swiglu(up, gact)))
        del up, gact
    if attention_s8192 is not None:
        S2, H = 8192, 14
        q, k, v = (rnd(1, H, S2, 128) for _ in range(3))
        seconds = median_time(lambda: h3_oracle.attention(q, k, v, 128 ** -0.5, dtype=torch.float32, chunk=2048),
                              warmup=1, runs=3)
        attention_s8192["cpu_TFLOP/s"] = round(4.0 * H * S2 * S2 * 128 / seconds / 1e12, 4)
        attention_s8192["cpu_threads"] = threads
        log(f"  cpu attention S={S2}: {seconds:.2f} s, {attention_s8192['cpu_TFLOP/s']} TFLOP/s ({threads} threads)")


def cpu_baseline(budget_s: float = 12.0) -> dict:
    """The CPU oracle's fp32 attention (softmax(q k^T s) v, chunked 2048 query
    rows) on heads of the S = 73,984, H = 14 workload, head after head until
    `budget_s` seconds have elapsed (at least one head)."""
    from oracle import h3_oracle
    S, H = 73984, 14
    gen = torch.Generator("cpu").manual_seed(0)
    threads = torch.get_num_threads()
    flops = 0.0
    heads = 0
    elapsed = 0.0
    while heads < H and elapsed < budget_s:
        q, k, v = (torch.randn(1, 1, S, 128, generator=gen).to(torch.bfloat16) for _ in range(3))
        t_head = time.perf_counter()
        h3_oracle.attention(q, k, v, 128 ** -0.5, dtype=torch.float32, chunk=2048)
        elapsed += time.perf_counter() - t_head
        flops += 4.0 * S * S * 128
        heads += 1
    host = cpu_host()
    return {"value": round(flops / elapsed / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"{heads} of 14 heads of the S=73,984 D=128 attention, fp32 on the host CPU "
                      f"(oracle softmax(q k^T s) v, 2048-query chunks), {elapsed:.1f} s",
            "cpu_model": host["cpu_model"], "host_cpus": host["host_cpus"], "usable_cpus": host["usable_cpus"]}


def mfma_peak_measured(pkg, device, headline_tflops: float | None) -> dict:
    """The bf16 MFMA rate the part sustains (launch_h3_calibration_mfma:
    v_mfma_f32_32x32x16_bf16 only, 8 workgroups of 512 threads per CU, four
    chains per wave, operands rotating through four A and four B fragments;
    launch_h3_calibration_mfma_16x16x32: the same flops as 16x16x32 products
    over eight chains), with random N(0, 1) operands (the clock the power
    allows under MFMA load) and with zero operands; each launch ~35 ms like the
    headline's. Reports the headline attention (16x16x32 products) against the
    32x32x16 random-operand rate and against the best shape's. The same for the
    fp8 kernels' product (launch_h3_calibration_mfma_fp8:
    v_mfma_scale_f32_32x32x64_f8f6f4 on e4m3 operands), which the fp8 lines'
    executed work is set against."""
    cal = pkg.h3_calibration
    blocks = 8 * torch.cuda.get_device_properties(device).multi_processor_count
    iters = 8000
    flop = blocks * 512 * iters * cal.MFMA_FLOP_PER_THREAD_ITERATION
    gen = torch.Generator(device=device).manual_seed(7)
    out = torch.empty(blocks, 512, device=device)
    res = {"kernel": "v_mfma_f32_32x32x16_bf16, 4 chains per wave", "flop_per_launch": flop}
    rand = torch.randn(512, 64, generator=gen, device=device).to(torch.bfloat16)
    zero = torch.zeros(512, 64, dtype=torch.bfloat16, device=device)
    for shape, prefix in (("32x32x16", ""), ("16x16x32", "mfma_16x16x32_")):
        for name, ops in (("random", rand), ("zero", zero)):
            ms = time_launches(lambda: cal.mfma(ops, out, iters, shape=shape), 5, 2)
            res[f"{prefix}{name}_operands_TFLOP/s"] = round(flop / (ms * 1e-3) / 1e12, 1)
        log(f"measured bf16 MFMA rate, {shape}: random operands {res[prefix + 'random_operands_TFLOP/s']} TFLOP/s, "
            f"zero operands {res[prefix + 'zero_operands_TFLOP/s']} TFLOP/s")
    # The fp8 kernels' product, v_mfma_scale_f32_32x32x64_f8f6f4 on e4m3 operands
    # (4000 rounds: ~35 ms per launch, like the bf16 ones).
    fp8_iters = 4000
    fp8_flop = blocks * 512 * fp8_iters * cal.MFMA_FP8_FLOP_PER_THREAD_ITERATION
    rand8 = torch.randn(512, 256, generator=gen, device=device).to(torch.float8_e4m3fn)
    for name, ops in (("random", rand8), ("zero", torch.zeros_like(rand8))):
        ms = time_launches(lambda: cal.mfma_fp8(ops, out, fp8_iters), 5, 2)
        res[f"fp8_32x32x64_{name}_operands_TFLOP/s"] = round(fp8_flop / (ms * 1e-3) / 1e12, 1)
    log(f"measured fp8 MFMA rate, 32x32x64: random operands {res['fp8_32x32x64_random_operands_TFLOP/s']} TFLOP/s, "
        f"zero operands {res['fp8_32x32x64_zero_operands_TFLOP/s']} TFLOP/s")
    if headline_tflops is not None:
        best = max(res["random_operands_TFLOP/s"], res["mfma_16x16x32_random_operands_TFLOP/s"])
        res["headline_frac_of_random"] = round(headline_tflops / res["random_operands_TFLOP/s"], 4)
        res["headline_frac_of_best_random"] = round(headline_tflops / best, 4)
        log(f"  the headline attention is {res['headline_frac_of_random']:.1%} of the 32x32x16 random-operand rate, "
            f"{res['headline_frac_of_best_random']:.1%} of the best shape's")
    return res


def bench_key_split(pkg, device) -> dict:
    """The key split of a partly filled last round of workgroups
    (make_attention's default, launch_h3_full_attention_ws) against the
    unsplit launch, on shapes where the plan splits: S = 16,384, H = 14 (896
    units on 256 CUs: 3 full rounds and a half one, split in 2) and a short
    query block over long keys (2 units, split in 8). Inputs N(0, 1), scale
    1/sqrt(128); each variant warmed, then timed over ~70 ms of launches."""
    out = {}
    gen = torch.Generator(device=device).manual_seed(3)
    for name, (B, H, Sq, Sk) in (("s16384_h14", (1, 14, 16384, 16384)), ("q700_k9000_h2", (1, 2, 700, 9000))):
        q = torch.randn(B, H, Sq, 128, generator=gen, device=device).to(torch.bfloat16)
        k = torch.randn(B, H, Sk, 128, generator=gen, device=device).to(torch.bfloat16)
        v = torch.randn(B, H, Sk, 128, generator=gen, device=device).to(torch.bfloat16)
        o = torch.empty_like(q)
        flops = 4.0 * B * H * Sq * Sk * 128
        entry = {"shape": [B, H, Sq, Sk], "workspace_bytes": pkg._lib.attention_workspace_bytes(B, H, Sq, Sk)}
        for variant, split in (("split", True), ("unsplit", False)):
            attn = pkg.make_attention(split_last_round=split)
            call = lambda: attn(q, k, v, 128 ** -0.5, o)  # noqa: E731
            n = max(20, min(2000, int(70.0 / time_launches(call, 5, 2))))
            ms = time_launches(call, n, n)
            entry[f"{variant}_ms"] = round(ms, 4)
            entry[f"{variant}_TFLOP/s"] = round(flops / (ms * 1e-3) / 1e12, 2)
        entry["speedup"] = round(entry["unsplit_ms"] / entry["split_ms"], 3)
        out[name] = entry
        log(f"  key split {name}: {entry['split_ms']:.4f} ms against {entry['unsplit_ms']:.4f} ms unsplit "
            f"({entry['speedup']:.2f}x)")
        del q, k, v, o
    return out


def bench_s8192(pkg, device) -> dict:
    """bf16 attention at S = 8192, H = 14 (the launch whose last round runs as
    192-query units): 100 timed launches after 100 warm-up ones (~45 ms: the
    first tens of launches on fresh inputs run up to 19% slower, 0.52 against
    0.44 ms, until the clock settles)."""
    S, H, D = 8192, 14, 128
    q, k, v = attention_inputs_gpu(S, H, 0, 0.0, device)
    out = torch.empty_like(q)
    attn = pkg.make_attention()
    ms = time_launches(lambda: attn(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), D ** -0.5,
                                    out.transpose(1, 2)), 100, 100)
    t = 4.0 * S * S * D * H / (ms * 1e-3) / 1e12
    log(f"attention S={S} H={H}: {ms:.3f} ms, {t:.1f} TFLOP/s")
    return {"ms": round(ms, 4), "TFLOP/s": round(t, 2), "frac": round(t / BF16_PEAK_TFLOPS, 4)}


def head_group_calls(pkg, q, k, v, out, scale: float, groups: int):
    """Head-grouped attention on one GPU: the heads of [1, S, H, 128] q, k, v
    in `groups` equal groups, each an attention launch on its head slice. Group
    g + 1's q, k, v are copied into staging buffers on a second stream (default
    priority) while group g computes -- the bytes a sequence-parallel rank's
    all-to-all would deliver for that group, and the overlap the reference runs
    on its head groups (patches/InfiniLM.patch:960-1018). Returns (grouped
    call, staging buffers); each group's output lands in its slice of out."""
    attn = pkg.make_attention(split_last_round=False)
    H = q.shape[2]
    gs = H // groups
    sl = [slice(g * gs, (g + 1) * gs) for g in range(groups)]
    stage = [[torch.empty(q.shape[0], q.shape[1], gs, q.shape[3], dtype=q.dtype, device=q.device)
              for _ in range(3)] for _ in range(groups)]
    side = torch.cuda.Stream()
    bhsd = lambda t: t.transpose(1, 2)  # noqa: E731

    def call():
        main = torch.cuda.current_stream()
        side.wait_stream(main)
        done = []
        for g in range(groups):
            with torch.cuda.stream(side):
                for dst, src in zip(stage[g], (q, k, v)):
                    dst.copy_(src[:, :, sl[g]])
                ev = torch.cuda.Event()
                ev.record(side)
            done.append(ev)
        for g in range(groups):
            main.wait_event(done[g])
            sq, sk, sv = stage[g]
            attn(bhsd(sq), bhsd(sk), bhsd(sv), scale, bhsd(out[:, :, sl[g]]))
        main.wait_stream(side)

    return call, stage


def bench_head_groups(pkg, device) -> dict:
    """S = 73,984, H = 14 as two head groups of 7 whose q, k, v arrive by a
    copy on a second stream while the previous group computes, against the one
    14-head launch; the first group's copy is exposed, as a rank's first
    all-to-all is."""
    S, H = 73984, 14
    q, k, v = attention_inputs_gpu(S, H, 1, 0.0, device)
    out_full, out_grp = torch.empty_like(q), torch.empty_like(q)
    full = pkg.make_attention(split_last_round=False)
    scale = 128 ** -0.5
    grouped, _ = head_group_calls(pkg, q, k, v, out_grp, scale, 2)
    ms_full = time_launches(lambda: full(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), scale,
                                         out_full.transpose(1, 2)), 3, 1)
    ms_grp = time_launches(grouped, 3, 1)
    copy_bytes = 3 * q.numel() * 2
    res = {"heads": H, "groups": 2, "copied_MB": round(copy_bytes / 1e6, 1), "one_launch_ms": round(ms_full, 3),
           "grouped_with_copies_ms": round(ms_grp, 3), "overhead": round(ms_grp / ms_full - 1, 4),
           "outputs_bitwise_equal": bool(torch.equal(out_full, out_grp))}
    log(f"  head groups: 2 x 7 heads with q/k/v copies on a second stream {ms_grp:.3f} ms against one "
        f"14-head launch {ms_full:.3f} ms ({res['overhead']:+.1%}); outputs equal {res['outputs_bitwise_equal']}")
    return res


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=10)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-pointwise", action="store_true")
    parser.add_argument("--no-extra", action="store_true", help="skip the S=8192 and fp8 attention lines")
    parser.add_argument("--pointwise-only", action="store_true",
                        help="time only the pointwise ops (for per-kernel profiles)")
    parser.add_argument("--mfma-only", action="store_true", help="measure only the sustained bf16 and fp8 MFMA rates")
    parser.add_argument("--s8192-only", action="store_true",
                        help="time only the bf16 attention at S = 8192, H = 14 (for its kernel profile)")
    parser.add_argument("--key-split-only", action="store_true",
                        help="time only the attention key split against the unsplit launch")
    parser.add_argument("--copy-calibration", type=int, metavar="MIB",
                        help="run a plain device copy of MIB MiB five times (PMC byte-counter calibration)")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU's share (14 heads at full sequence length) on one GPU; it has no "
              "multi-GPU mode (the path would shard by heads across GPUs, with an all-to-all either side)",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    pkg = importlib.import_module("minimaxh3_on_k100-ai_amd")
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    props = torch.cuda.get_device_properties(device)
    log(f"device {props.name} ({props.gcnArchName}), torch {torch.__version__}")
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device=device).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": n, "launches": 5}))
        return 0
    if args.pointwise_only:
        print(json.dumps({"pointwise": bench_pointwise(pkg, device)}))
        return 0
    if args.mfma_only:
        print(json.dumps({"mfma_peak_measured": mfma_peak_measured(pkg, device, None)}))
        return 0
    if args.key_split_only:
        print(json.dumps({"attention_key_split": bench_key_split(pkg, device)}))
        return 0
    if args.s8192_only:
        print(json.dumps({"attention_s8192": bench_s8192(pkg, device)}))
        return 0

    S, H, D = 73984, 14, 128
    q, k, v = attention_inputs_gpu(S, H, 0, 0.01, device)
    out = torch.empty_like(q)
    attn = pkg.make_attention()
    scale = D ** -0.5

    def step():
        attn(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), scale, out.transpose(1, 2))

    ms = time_launches(step, args.steps, args.warmup)
    flops = 4.0 * S * S * D * H
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"attention S={S} H={H}: {ms:.3f} ms/step, {tflops:.1f} TFLOP/s ({tflops / BF16_PEAK_TFLOPS:.1%} of bf16 peak)")

    line = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1), 1% key rows x8)",
        "config": {"workload": "non-causal bf16 attention forward, B=1 H=14 S=73984 D=128 "
                               "(73,728 video + 256 text tokens), [B,S,H,D] layout, scale 1/sqrt(128)",
                   "global_batch": 1, "seq_len": S, "heads": H, "head_dim": D, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "traffic": None},
    }
    # HBM bytes per launch of this kernel, measured with FETCH_SIZE / WRITE_SIZE
    # counters (calibrated on a plain copy) and recorded in the profile summary
    # together with the digest of the sources it measured.
    traffic = profiled_traffic()
    line["roofline"]["traffic"] = traffic["traffic"]
    line["roofline"]["traffic_source"] = traffic["traffic_source"]
    if not args.no_extra:
        line["mfma_peak_measured"] = mfma_peak_measured(pkg, device, tflops)
        log("vendor SDPA (torch's fused kernel) on the same inputs...")
        line["vendor_sdpa"] = {"s73984": vendor_sdpa(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), scale,
                                                     out.transpose(1, 2), 3)}
        log(f"  S={S}: {line['vendor_sdpa']['s73984']}")
    del q, k, v, out

    if not args.no_extra:
        S2 = 8192
        line["attention_s8192"] = bench_s8192(pkg, device)
        q, k, v = attention_inputs_gpu(S2, H, 0, 0.0, device)
        out = torch.empty_like(q)
        attn(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), scale, out.transpose(1, 2))  # the hand kernel's output, compared below
        line["vendor_sdpa"]["s8192"] = vendor_sdpa(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), scale,
                                                   out.transpose(1, 2), 100, 100)
        log(f"  vendor S={S2}: {line['vendor_sdpa']['s8192']}")
        del q, k, v, out
        line["attention_key_split"] = bench_key_split(pkg, device)
        line["attention_head_groups"] = bench_head_groups(pkg, device)

    if not args.no_extra:
        # fp8 configuration: the same S = 73,984 tensors, per-head e4m3fn.
        q, k, v = attention_inputs_gpu(S, H, 0, 0.01, device)
        qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        out = torch.empty_like(q)
        quant = lambda: (pkg.quantize_fp8_per_head(qt), pkg.quantize_fp8_per_head(kt),  # noqa: E731
                         pkg.quantize_fp8_per_head(vt, transposed=True))
        ms_q = time_launches(quant, 5, 1)
        (q8, qd), (k8, kd), (v8, vd) = quant()
        # V alone: the two-pass quantiser against the code pass from a
        # producer's amax slots (the q/k/v pack folds them while it copies v).
        ms_v = time_launches(lambda: pkg.quantize_fp8_per_head(vt, transposed=True), 10, 2)
        slots = torch.zeros(H, 64, device=device)
        slots[:, 0] = vt.float().abs().amax(dim=(0, 2, 3))
        ms_v_slots = time_launches(lambda: pkg.quantize_fp8_per_head(vt, transposed=True, amax_slots=slots), 10, 2)
        f8 = pkg.make_attention_fp8()
        f8pv = pkg.make_attention_fp8pv()
        f8x2 = pkg.make_attention_fp8x2()
        out8 = torch.empty_like(q)
        ms_f8 = time_launches(lambda: f8(q8, k8, v8, qd, kd, vd, scale, out8.transpose(1, 2)), args.steps, 2)
        ms_pv = time_launches(lambda: f8pv(qt, kt, v8, vd, scale, out.transpose(1, 2)), args.steps, 2)
        t8, tpv = flops / (ms_f8 * 1e-3) / 1e12, flops / (ms_pv * 1e-3) / 1e12
        # Two-term Q and K (hi + lo e4m3 codes), V one-term: Q, K and V all on the fp8 MFMA.
        quant2 = lambda: (pkg.quantize_fp8_two_term(qt), pkg.quantize_fp8_two_term(kt))  # noqa: E731
        ms_q2 = time_launches(quant2, 5, 1)
        (q8h, q8l, qd2), (k8h, k8l, kd2) = quant2()
        out82 = torch.empty_like(q)
        ms_x2 = time_launches(lambda: f8x2(q8h, q8l, k8h, k8l, v8, qd2, kd2, vd, scale, out82.transpose(1, 2)),
                              args.steps, 2)
        tx2 = flops / (ms_x2 * 1e-3) / 1e12
        # Accuracy against fp32 attention on every 37th query row (2000 rows x 14 heads).
        rows = torch.arange(0, S, 37, device=device)
        rel_pv = sampled_rel_rms(out.transpose(1, 2), qt, kt, vt, scale, rows)
        rel_f8 = sampled_rel_rms(out8.transpose(1, 2), qt, kt, vt, scale, rows)
        rel_x2 = sampled_rel_rms(out82.transpose(1, 2), qt, kt, vt, scale, rows)
        bar = 5e-2
        # The fp8 MFMA rate the part sustains with these kernels' product
        # (mfma_peak_measured: v_mfma_scale_f32_32x32x64_f8f6f4, random e4m3).
        fp8_random = line["mfma_peak_measured"]["fp8_32x32x64_random_operands_TFLOP/s"]
        # MFMA work each recipe executes, per algorithmic flop (4 B H S^2 D):
        # two-term Q.K^T is three products and sums its denominator on the
        # VALU; the one-term recipe adds a ones x P product per 64-key tile
        # and 32 queries (a quarter of P.V's) for its denominator.
        exec_x2, exec_f8 = (3 + 1) / 2, (1 + 1 + 0.25) / 2
        line["fp8"] = {
            "config5": {
                "variant": "fp8x2: per-head e4m3 Q and K as two terms (hi + lo / 16, three fp8 Q.K^T MFMAs on one "
                           "accumulator), per-head e4m3 V and e4m3 P, all on the fp8 MFMA",
                "ms": round(ms_x2, 4), "TFLOP/s": round(tx2, 2), "frac_fp8_peak": round(tx2 / FP8_PEAK_TFLOPS, 4),
                "executed_fp8_TFLOP/s": round(tx2 * exec_x2, 1),
                "executed_frac_fp8_peak": round(tx2 * exec_x2 / FP8_PEAK_TFLOPS, 4),
                "executed_frac_fp8_random_rate": round(tx2 * exec_x2 / fp8_random, 4),
                "rel_rms": round(rel_x2, 5), "meets_rel_rms_5e-2": rel_x2 <= bar,
                "quantize_qk_two_term_ms": round(ms_q2, 4)},
            "fp8pv_bf16_logits": {"variant": "fp8pv: bf16 Q.K^T logits, e4m3 P and per-head e4m3 V on the fp8 MFMA",
                                  "ms": round(ms_pv, 4), "TFLOP/s": round(tpv, 2), "rel_rms": round(rel_pv, 5),
                                  "meets_rel_rms_5e-2": rel_pv <= bar},
            "all_fp8_misses_accuracy_bar": {
                "variant": "all-fp8: per-head e4m3 Q, K, V and e4m3 P on the fp8 MFMA",
                "ms": round(ms_f8, 4), "TFLOP/s": round(t8, 2), "frac_fp8_peak": round(t8 / FP8_PEAK_TFLOPS, 4),
                "executed_fp8_TFLOP/s": round(t8 * exec_f8, 1),
                "executed_frac_fp8_random_rate": round(t8 * exec_f8 / fp8_random, 4),
                "rel_rms": round(rel_f8, 5), "meets_rel_rms_5e-2": rel_f8 <= bar},
            "executed_work_per_algorithmic_flop": {
                "config5": exec_x2, "all_fp8": exec_f8,
                "note": "two-term Q.K^T is three fp8 products (hi.hi, lo.hi, hi.lo) and its denominator is an fp32 "
                        "VALU sum; the one-term recipe adds a ones x P product per 64-key tile for the denominator"},
            "fp8_mfma_random_operands_TFLOP/s": fp8_random,
            "accuracy_sample": f"{rows.numel()} query rows x {H} heads (every 37th row) vs fp32 attention",
            "quantize_qkv_ms": round(ms_q, 4),
            "quantize_v_ms": {"two_pass": round(ms_v, 4), "code_pass_from_pack_slots": round(ms_v_slots, 4)},
        }
        log(f"measured fp8 MFMA rate (32x32x64, random e4m3 operands): {fp8_random:.1f} TFLOP/s; config 5 executes "
            f"{tx2 * exec_x2:.1f} TFLOP/s of fp8 products, {tx2 * exec_x2 / fp8_random:.1%} of it")
        log(f"fp8 attention S={S}: config 5 (two-term e4m3 Q/K, e4m3 V) {ms_x2:.3f} ms ({tx2:.1f} TFLOP/s), "
            f"rel RMS {rel_x2:.4f}; bf16 logits + fp8 P.V {ms_pv:.3f} ms ({tpv:.1f} TFLOP/s), rel RMS {rel_pv:.4f}; "
            f"one-term all-fp8 {ms_f8:.3f} ms ({t8:.1f} TFLOP/s), rel RMS {rel_f8:.4f} "
            f"({'meets' if rel_f8 <= bar else 'misses'} 5e-2); quantise q,k,v {ms_q:.3f} ms, two-term q,k "
            f"{ms_q2:.3f} ms; "
            f"v alone {ms_v:.3f} ms, from the pack's amax slots {ms_v_slots:.3f} ms")
        del q, k, v, out, out8, out82, q8, k8, v8, q8h, q8l, k8h, k8l

    if not args.no_pointwise:
        log("pointwise ops:")
        line["pointwise"] = bench_pointwise(pkg, device)

    if not args.no_cpu_baseline:
        log("cpu baseline (oracle fp32 attention on the host)...")
        line["cpu_baseline"] = cpu_baseline()
        log(f"  {line['cpu_baseline']}")
        log("reference torch CPU path beside each op...")
        cpu_reference_path(device, line.get("pointwise"), line.get("attention_s8192"))

    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

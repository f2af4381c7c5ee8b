"""The C ABI of libh3mi355x.so on the CPU: the library loads, exports exactly
the entry points include/h3mi355x.h declares, and every launcher rejects
malformed arguments with hipErrorInvalidValue (1) on the host, before any HIP
call -- so these run without a GPU. Empty launches return 0 without touching
the device (patches/ninetoothed.patch:304-307)."""
from __future__ import annotations

import ctypes
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "h3mi355x.h"
INVALID = 1


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg._lib


def declared_entry_points():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"NineToothedResult\s+(launch_\w+)\s*\(", text)))


def declared_arity():
    text = HEADER.read_text()
    out = {}
    for name, args in re.findall(r"NineToothedResult\s+(launch_\w+)\s*\(([^;]*)\);", text, re.S):
        out[name] = args.count("NineToothedTensor")
    return out


def test_header_declares_the_binding_table(lib):
    assert declared_entry_points() == sorted(lib.ENTRY_POINTS)
    assert declared_arity() == lib.ENTRY_POINTS


def test_library_exports_every_declared_symbol(lib):
    so = lib.library()
    for name in declared_entry_points():
        assert hasattr(so, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", str(lib.LIBRARY_PATH)], capture_output=True, text=True)
    exported = set(re.findall(r" T (launch_\w+)", nm.stdout))
    assert exported == set(declared_entry_points())


def test_attention_workspace_query_is_exported(lib):
    """h3_full_attention_workspace_bytes, the size query beside
    launch_h3_full_attention_ws: exported, declared, and 0 for an empty
    launch without any HIP call."""
    assert "h3_full_attention_workspace_bytes" in HEADER.read_text()
    for shape in ((0, 1, 1, 1), (1, 0, 5, 5), (1, 1, 0, 9), (1, 1, 9, 0), (1, 1, 9, LONG_S), (1, 1, LONG_S, 9)):
        assert lib.attention_workspace_bytes(*shape) == 0


def test_library_is_built_for_gfx950(lib):
    data = lib.LIBRARY_PATH.read_bytes()
    assert b"gfx950" in data


# ------------------------------------------------------------------ argument validation

BUF = ctypes.create_string_buffer(1 << 16)
ADDR = (ctypes.addressof(BUF) + 255) & ~255  # 256-byte aligned host memory, never dereferenced


def t(shape, strides=None, data=ADDR):
    if strides is None:
        strides = []
        acc = 1
        for s in reversed(shape):
            strides.insert(0, acc)
            acc *= s
    return lambda L: L.raw_tensor(data, shape, strides)


def scal(v=1e-6):
    return lambda L: L.scalar(v)


def vt(B, H, S, data=ADDR):
    """A [B, H, S, 128] e4m3 V^T view: S-contiguous, S padded to 16 bytes."""
    sp = -(-S // 16) * 16
    return t([B, H, S, 128], [H * 128 * sp, 128 * sp, 1, sp], data)


LONG_S = (1 << 31) - 1000  # above the launchers' sequence limit, 2^31 - 1 - 1024
NULLSHAPE = lambda L: L._Arg(ADDR, (), None)  # noqa: E731  (tensor with NULL shape/strides)
NULLSCALAR = lambda L: L._Arg(0, (), None)  # noqa: E731  (scalar with NULL data)

CASES = [
    # (entry point, args, why)
    ("launch_h3_rms_exact_128", [t([1, 4, 64]), t([64]), scal(), t([1, 4, 64])], "width 64 on the 128 kernel"),
    ("launch_h3_rms_exact_5376", [t([1, 4, 128]), t([128]), scal(), t([1, 4, 128])], "width 128 on the 5376 kernel"),
    ("launch_h3_rms_exact", [t([1, 4, 128]), t([64]), scal(), t([1, 4, 128])], "weight length"),
    ("launch_h3_rms_exact", [t([1, 4, 128]), t([128]), scal(), t([1, 5, 128])], "out shape"),
    ("launch_h3_rms_exact", [t([1, 4, 128]), t([128]), NULLSCALAR, t([1, 4, 128])], "eps without data"),
    ("launch_h3_rms_exact", [NULLSHAPE, t([128]), scal(), t([1, 4, 128])], "x without shape"),
    ("launch_h3_rms_exact", [t([1, 2, 40000]), t([40000]), scal(), t([1, 2, 40000])], "width above 32768"),
    ("launch_h3_rms_exact", [t([1, 4, 128], data=0), t([128]), scal(), t([1, 4, 128])], "null data"),
    ("launch_h3_rms_modulate_exact", [t([1, 4, 128]), t([128]), scal(), t([1, 4, 64]), t([1, 4, 128]),
                                      t([1, 4, 128])], "scale shape"),
    ("launch_h3_gated_residual_exact", [t([1, 4, 128]), t([1, 4, 128]), t([1, 3, 128]), t([1, 4, 128])], "y shape"),
    ("launch_h3_gated_residual_rms_modulate_exact",
     [t([1, 4, 128]), t([1, 4, 128]), t([1, 4, 128]), t([128]), scal(), t([1, 4, 128]), t([1, 4, 128]),
      t([1, 4, 127]), t([1, 4, 128])], "residual shape"),
    ("launch_h3_swiglu_exact", [t([1, 4, 128]), t([1, 4, 256]), t([1, 4, 128])], "gate shape"),
    ("launch_h3_rms_modulate_indexed", [t([1, 4, 128]), t([128]), scal(), t([3, 128]), t([3, 128]), t([1, 5]),
                                        t([1, 4, 128])], "index shape"),
    ("launch_h3_rms_modulate_indexed", [t([1, 4, 128]), t([128]), scal(), t([3, 64]), t([3, 64]), t([1, 4]),
                                        t([1, 4, 128])], "table width"),
    ("launch_h3_rms_modulate_indexed", [t([1, 4, 128]), t([128]), scal(), t([3, 128]), t([2, 128]), t([1, 4]),
                                        t([1, 4, 128])], "tables of different row counts"),
    ("launch_h3_rms_modulate_indexed", [t([1, 4, 128]), t([128]), scal(), t([0, 128]), t([0, 128]), t([1, 4]),
                                        t([1, 4, 128])], "empty tables"),
    ("launch_h3_rms_modulate_indexed", [t([1, 4, 128]), t([128]), scal(), t([3, 128]), t([3, 128]), NULLSHAPE,
                                        t([1, 4, 128])], "index without shape"),
    ("launch_h3_gated_residual_rms_modulate_indexed",
     [t([1, 4, 128]), t([2, 128]), t([1, 4, 128]), t([128]), scal(), t([3, 128]), t([3, 128]), t([1, 4]),
      t([1, 4, 128]), t([1, 4, 128])], "gate table rows"),
    ("launch_h3_gated_residual_rms_modulate_indexed",
     [t([1, 4, 128]), t([3, 128]), t([1, 4, 128]), t([128]), scal(), t([3, 128]), t([3, 128]), t([4, 1]),
      t([1, 4, 128]), t([1, 4, 128])], "index transposed"),
    ("launch_h3_gated_residual_indexed", [t([1, 4, 128]), t([1, 4, 128]), t([1, 4, 128]), t([1, 4]),
                                          t([1, 4, 128])], "3-D gate on the indexed kernel"),
    ("launch_h3_gated_residual_indexed", [t([1, 4, 128]), t([0, 128]), t([1, 4, 128]), t([1, 4]),
                                          t([1, 4, 128])], "empty gate table"),
    ("launch_h3_rope_exact", [t([4, 2, 128]), t([4, 2, 128], data=ADDR + 256), t([4, 2, 128]), t([4, 48]),
                              t([4, 48]), t([4, 2, 128]), t([4, 2, 128]), t([4, 2, 128])], "unaliased x views"),
    ("launch_h3_rope_exact", [t([4, 2, 128])] * 3 + [t([4, 64]), t([4, 64])] + [t([4, 2, 128])] * 3, "table 64"),
    ("launch_h3_rope_exact", [t([4, 2, 64])] * 3 + [t([4, 48]), t([4, 48])] + [t([4, 2, 64])] * 3, "head dim 64"),
    ("launch_h3_qk_norm_rope", [t([4, 1, 2, 128])] * 3 + [t([128])] * 3 + [scal(), t([5, 48]), t([5, 48])]
     + [t([4, 1, 2, 128])] * 3, "table rows != tokens"),
    ("launch_h3_qk_norm_rope", [t([4, 1, 2, 128])] * 3 + [t([64])] * 3 + [scal(), t([4, 48]), t([4, 48])]
     + [t([4, 1, 2, 128])] * 3, "weight 64"),
    ("launch_h3_qk_norm_rope_interleaved", [t([4, 1, 2, 128]), t([128]), scal(), t([4, 48]), t([4, 48]),
                                            t([4, 1, 2, 128])], "interleaved needs a 64-wide table"),
    ("launch_h3_qkv_norm_rope_pack", [t([4, 2, 3, 128])] * 3 + [t([128]), t([128]), scal(), t([9, 48]),
                                      t([9, 48]), t([5])] + [t([4, 2, 3, 128])] * 3, "positions length"),
    ("launch_h3_qkv_norm_rope_pack", [t([4, 2, 3, 128])] * 3 + [t([128]), t([128]), scal(), t([9, 64]),
                                      t([9, 64]), t([4])] + [t([4, 2, 3, 128])] * 3, "table width 64"),
    ("launch_h3_qkv_norm_rope_pack", [t([4, 2, 3, 128]), t([4, 2, 3, 128]), t([4, 3, 2, 128]), t([128]),
                                      t([128]), scal(), t([9, 48]), t([9, 48]), t([4])]
     + [t([4, 2, 3, 128])] * 3, "v shape"),
    ("launch_h3_qkv_norm_rope_pack", [t([4, 2, 3, 128])] * 3 + [t([128]), t([128]), scal(), t([0, 48]),
                                      t([0, 48]), t([4])] + [t([4, 2, 3, 128])] * 3, "empty cache"),
    ("launch_h3_qkv_norm_rope_pack_fp8", [t([4, 2, 3, 128])] * 3 + [t([128]), t([128]), scal(), t([9, 48]),
                                          t([9, 48]), t([4])] + [t([4, 2, 3, 128])] * 3 + [t([5]), t([6])],
     "descale length"),
    ("launch_h3_qkv_norm_rope_pack_fp8", [t([4, 2, 3, 128])] * 3 + [t([128]), t([128]), scal(), t([9, 48]),
                                          t([9, 48]), t([4]), t([4, 2, 3, 64]), t([4, 2, 3, 128]),
                                          t([4, 2, 3, 128]), t([6]), t([6])], "q8 width"),
    ("launch_h3_qk_norm_rope_interleaved_qk", [t([4, 1, 2, 128]), t([4, 1, 3, 128]), t([128]), t([128]), scal(),
                                               t([4, 64]), t([4, 64]), t([4, 1, 2, 128]), t([4, 1, 3, 128])],
     "q/k head counts differ"),
    ("launch_h3_qk_norm_rope_interleaved_qk", [t([4, 1, 2, 128])] * 2 + [t([128]), t([64]), scal(), t([4, 64]),
                                               t([4, 64])] + [t([4, 1, 2, 128])] * 2, "k weight length"),
    ("launch_h3_qk_norm_rope_interleaved_qk", [t([4, 1, 2, 128])] * 2 + [t([128]), t([128]), scal(), t([4, 48]),
                                               t([4, 48])] + [t([4, 1, 2, 128])] * 2, "table width 48"),
    ("launch_h3_rope_cache", [t([4, 3]), t([15]), t([4, 48]), t([4, 48])], "15 powers"),
    ("launch_h3_rope_cache", [t([4, 2]), t([16]), t([4, 48]), t([4, 48])], "2 position axes"),
    ("launch_h3_full_attention", [t([1, 2, 8, 64]), t([1, 2, 8, 64]), t([1, 2, 8, 64]), scal(0.1),
                                  t([1, 2, 8, 64])], "head dim 64"),
    ("launch_h3_full_attention", [t([1, 2, 8, 128]), t([1, 3, 8, 128]), t([1, 3, 8, 128]), scal(0.1),
                                  t([1, 2, 8, 128])], "head count mismatch"),
    ("launch_h3_full_attention", [t([1, 2, 8, 128]), t([1, 2, 9, 128]), t([1, 2, 8, 128]), scal(0.1),
                                  t([1, 2, 8, 128])], "k/v length mismatch"),
    # Views with any strides and 2-byte aligned rows run (element-strided
    # path); a bf16 element at an odd address does not.
    ("launch_h3_full_attention", [t([1, 2, 8, 128], data=ADDR + 1), t([1, 2, 8, 128]), t([1, 2, 8, 128]),
                                  scal(0.1), t([1, 2, 8, 128])], "odd address q"),
    ("launch_h3_full_attention", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), t([1, 2, 8, 128]),
                                  scal(0.1), t([1, 2, 8, 128], data=ADDR + 3)], "odd address o"),
    ("launch_h3_full_attention", [t([1, 2, 8, 128]), t([1, 2, 0, 128]), t([1, 2, 0, 128]), scal(0.1),
                                  t([1, 2, 8, 128])], "no keys"),
    ("launch_h3_full_attention", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), t([1, 2, 8, 128]), NULLSCALAR,
                                  t([1, 2, 8, 128])], "scale without data"),
    ("launch_h3_full_attention", [t([1 << 16, 1 << 12, 1 << 20, 128]), t([1 << 16, 1 << 12, 8, 128]),
                                  t([1 << 16, 1 << 12, 8, 128]), scal(0.1), t([1 << 16, 1 << 12, 1 << 20, 128])],
     "grid above 2^31"),
    ("launch_h3_full_attention", [t([1, 2, 8, 72])] * 3 + [scal(0.1), t([1, 2, 8, 72])], "head dim 72 on the 128 launcher"),
    ("launch_h3_vision_attention_72", [t([1, 2, 8, 128])] * 3 + [scal(0.1), t([1, 2, 8, 128])],
     "head dim 128 on the 72 launcher"),
    ("launch_h3_vision_attention_72", [t([1, 2, 8, 72]), t([1, 2, 9, 72]), t([1, 2, 8, 72]), scal(0.1),
                                       t([1, 2, 8, 72])], "vision k/v length mismatch"),
    ("launch_h3_vision_attention_72", [t([1, 2, 8, 72])] * 2 + [t([1, 2, 8, 72], data=ADDR + 1)]
     + [scal(0.1), t([1, 2, 8, 72])], "vision odd address v"),
    ("launch_h3_vision_attention_72", [t([1, 2, 8, 72]), t([1, 2, 0, 72]), t([1, 2, 0, 72]), scal(0.1),
                                       t([1, 2, 8, 72])], "vision no keys"),
    # fp8 quantiser: x [B, H, S, 128] bf16, codes u8, descale [H] fp32; every
    # check comes before its first launch (descale is also its amax scratch).
    ("launch_h3_quantize_fp8_per_head", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), t([3])], "quantiser descale length"),
    ("launch_h3_quantize_fp8_per_head", [t([1, 2, 8, 128]), t([1, 2, 9, 128]), t([2])], "quantiser codes shape"),
    ("launch_h3_quantize_fp8_per_head", [t([1, 2, 8, 64]), t([1, 2, 8, 64]), t([2])], "quantiser head dim 64"),
    ("launch_h3_quantize_fp8_per_head", [t([1, 2, 8, 128], [2048, 1024, 128, 2]), t([1, 2, 8, 128]), t([2])],
     "quantiser non-unit head-dim stride"),
    ("launch_h3_quantize_fp8_per_head", [t([1, 2, 8, 128]), t([1, 2, 8, 128], [2048, 1024, 128, 1], ADDR + 4),
                                         t([2])], "quantiser misaligned codes"),
    ("launch_h3_quantize_fp8_per_head", [t([1, 16, 1 << 24, 128]), t([1, 16, 1 << 24, 128]), t([16])],
     "quantiser 2^31 chunks"),
    ("launch_h3_quantize_fp8_per_head_slots", [t([1, 2, 8, 128]), t([2, 32]), t([1, 2, 8, 128]), t([2])],
     "quantiser slots per head"),
    ("launch_h3_quantize_fp8_per_head_slots", [t([1, 2, 8, 128]), t([3, 64]), t([1, 2, 8, 128]), t([2])],
     "quantiser slot heads"),
    ("launch_h3_quantize_fp8_per_head_slots", [t([1, 2, 8, 128]), t([2, 64], [1, 2]), t([1, 2, 8, 128]), t([2])],
     "quantiser slots transposed"),
    ("launch_h3_quantize_fp8_per_head_slots", [t([1, 2, 8, 128]), t([2, 64], [0, 1]), t([1, 2, 8, 128]), t([2])],
     "quantiser slots of one head broadcast"),
    ("launch_h3_quantize_fp8_per_head_slots", [t([1, 2, 8, 128]), t([2, 64], [128, 1]), t([1, 2, 8, 128]), t([2])],
     "quantiser slots padded between heads"),
    ("launch_h3_quantize_fp8_per_head_slots", [t([1, 16, 1 << 24, 128]), t([16, 64]), t([1, 16, 1 << 24, 128]),
                                               t([16])], "quantiser slots 2^31 chunks"),
    ("launch_h3_qkv_norm_rope_pack_fp8_vamax", [t([4, 2, 3, 128])] * 3 + [t([128]), t([128]), scal(), t([9, 48]),
                                                t([9, 48]), t([4])] + [t([4, 2, 3, 128])] * 3
     + [t([6]), t([6]), t([6, 32])], "vamax slots per head"),
    ("launch_h3_qkv_norm_rope_pack_fp8_vamax", [t([4, 2, 3, 128])] * 3 + [t([128]), t([128]), scal(), t([9, 48]),
                                                t([9, 48]), t([4])] + [t([4, 2, 3, 128])] * 3
     + [t([6]), t([6]), t([5, 64])], "vamax slot heads"),
    ("launch_h3_qkv_norm_rope_pack_fp8_vamax", [t([4, 8, 130, 128])] * 3 + [t([128]), t([128]), scal(),
                                                t([9, 48]), t([9, 48]), t([4])] + [t([4, 8, 130, 128])] * 3
     + [t([1040]), t([1040]), t([1040, 64])], "vamax above 1024 heads"),
    # attention with a workspace: q, k, v, scale, o, workspace (1-D bytes).
    ("launch_h3_full_attention_ws", [t([1, 2, 8, 128])] * 3 + [scal(0.1), t([1, 2, 8, 128]), t([4096], [2])],
     "workspace not contiguous"),
    ("launch_h3_full_attention_ws", [t([1, 2, 8, 128])] * 3 + [scal(0.1), t([1, 2, 8, 128]), t([4096], data=ADDR + 16)],
     "workspace not 256-byte aligned"),
    ("launch_h3_full_attention_ws", [t([1, 2, 8, 128])] * 3 + [scal(0.1), t([1, 2, 8, 128]), NULLSHAPE],
     "workspace without shape"),
    ("launch_h3_full_attention_ws", [t([1, 2, 8, 128]), t([1, 2, 8, 64]), t([1, 2, 8, 128]), scal(0.1),
                                     t([1, 2, 8, 128]), t([4096])], "ws k head dim"),
    # two-term pack: 9 inputs, q8, q8_lo, k8, k8_lo, v_out, 2 descales, v_amax.
    ("launch_h3_qkv_norm_rope_pack_fp8x2_vamax", [t([4, 1, 3, 128])] * 3 + [t([128]), t([128]), scal(), t([9, 48]),
                                                  t([9, 48]), t([4])] + [t([4, 1, 3, 128]), t([4, 1, 2, 128])] +
     [t([4, 1, 3, 128])] * 3 + [t([3]), t([3]), t([3, 64])], "fp8x2 pack q lo shape"),
    ("launch_h3_qkv_norm_rope_pack_fp8x2_vamax", [t([4, 1, 3, 128])] * 3 + [t([128]), t([128]), scal(), t([9, 48]),
                                                  t([9, 48]), t([4])] + [t([4, 1, 3, 128])] * 3 +
     [t([4, 1, 3, 128], [768, 384, 256, 1]), t([4, 1, 3, 128]), t([3]), t([3]), t([3, 64])], "fp8x2 pack k lo strides"),
    ("launch_h3_qkv_norm_rope_pack_fp8x2_vamax", [t([4, 1, 3, 128])] * 3 + [t([128]), t([128]), scal(), t([9, 48]),
                                                  t([9, 48]), t([4])] + [t([4, 1, 3, 128])] * 5 +
     [t([3]), t([3]), t([3, 32])], "fp8x2 pack slots"),
    # allocation-free pack + V quantisation: 9 pack inputs, q8, k8, v_out, 2 descales, v8, v_descale.
    ("launch_h3_qkv_norm_rope_pack_fp8_noalloc", [t([4, 2, 3, 128])] * 3 + [t([128]), t([128]), scal(),
                                                  t([9, 48]), t([9, 48]), t([4])] + [t([4, 2, 3, 128])] * 3
     + [t([6]), t([6]), vt(1, 6, 4), t([6])], "noalloc more than one rank"),
    ("launch_h3_qkv_norm_rope_pack_fp8_noalloc", [t([4, 1, 1040, 128])] * 3 + [t([128]), t([128]), scal(),
                                                  t([9, 48]), t([9, 48]), t([4])] + [t([4, 1, 1040, 128])] * 3
     + [t([1040]), t([1040]), vt(1, 1040, 4), t([1040])], "noalloc above the slot array's heads"),
    ("launch_h3_qkv_norm_rope_pack_fp8_noalloc", [t([4, 1, 3, 128])] * 3 + [t([128]), t([128]), scal(),
                                                  t([9, 48]), t([9, 48]), t([4])] + [t([4, 1, 3, 128])] * 3
     + [t([3]), t([3]), vt(1, 3, 5), t([3])], "noalloc v8 tokens"),
    ("launch_h3_qkv_norm_rope_pack_fp8_noalloc", [t([4, 1, 3, 128])] * 3 + [t([128]), t([128]), scal(),
                                                  t([9, 48]), t([9, 48]), t([4])] + [t([4, 1, 3, 128])] * 3
     + [t([3]), t([3]), vt(1, 3, 4), t([2])], "noalloc v descale length"),
    ("launch_h3_qkv_norm_rope_pack_fp8_noalloc", [t([4, 1, 3, 128])] * 3 + [t([64]), t([128]), scal(),
                                                  t([9, 48]), t([9, 48]), t([4])] + [t([4, 1, 3, 128])] * 3
     + [t([3]), t([3]), vt(1, 3, 4), t([3])], "noalloc q weight length"),
    ("launch_h3_qkv_norm_rope_pack_fp8_noalloc", [t([4, 1, 3, 128])] * 3 + [t([128]), t([128]), scal(),
                                                  t([9, 48]), t([9, 48]), t([4])] + [t([4, 1, 3, 128])] * 3
     + [t([3]), t([3]), vt(1, 3, 4, ADDR + 8), t([3])], "noalloc misaligned v8"),
    # two-term quantiser: x, x8, x8_lo (D-contiguous, x8's strides), descale.
    ("launch_h3_quantize_fp8_two_term", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), t([1, 2, 7, 128]), t([2])],
     "two-term lo shape"),
    ("launch_h3_quantize_fp8_two_term", [t([1, 2, 8, 128]), t([1, 2, 8, 128]),
                                         t([1, 2, 8, 128], [4096, 2048, 256, 1]), t([2])], "two-term lo strides"),
    ("launch_h3_quantize_fp8_two_term", [t([1, 2, 8, 128]), vt(1, 2, 8), vt(1, 2, 8), t([2])],
     "two-term S-contiguous codes"),
    ("launch_h3_quantize_fp8_two_term", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), t([1, 2, 8, 128]), t([3])],
     "two-term descale length"),
    # two-term attention: q8, q8_lo, k8, k8_lo, v8 (V^T), 3 descales, scale, o.
    ("launch_h3_full_attention_fp8x2", [t([1, 2, 8, 128]), t([1, 2, 9, 128]), t([1, 2, 8, 128]), t([1, 2, 8, 128]),
                                        vt(1, 2, 8), t([2]), t([2]), t([2]), scal(0.1), t([1, 2, 8, 128])],
     "fp8x2 q lo shape"),
    ("launch_h3_full_attention_fp8x2", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), t([1, 2, 8, 128]),
                                        t([1, 2, 8, 128], [4096, 2048, 256, 1]), vt(1, 2, 8), t([2]), t([2]), t([2]),
                                        scal(0.1), t([1, 2, 8, 128])], "fp8x2 k lo strides"),
    ("launch_h3_full_attention_fp8x2", [t([1, 2, 8, 128])] * 4 + [t([1, 2, 8, 128]), t([2]), t([2]), t([2]),
                                                                  scal(0.1), t([1, 2, 8, 128])],
     "fp8x2 v8 not S-contiguous"),
    ("launch_h3_full_attention_fp8x2", [t([1, 2, 8, 128])] * 4 + [vt(1, 2, 8), t([2]), t([3]), t([2]), scal(0.1),
                                                                  t([1, 2, 8, 128])], "fp8x2 k descale length"),
    ("launch_h3_full_attention_fp8x2", [t([1, 2, 8, 128])] * 2 + [t([1, 2, 0, 128])] * 2 +
     [vt(1, 2, 0), t([2]), t([2]), t([2]), scal(0.1), t([1, 2, 8, 128])], "fp8x2 no keys"),
    # all-fp8 attention: q8, k8 [B, H, S, 128] u8; v8 as V^T; descales [H].
    ("launch_h3_full_attention_fp8", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), t([1, 2, 8, 128]), t([2]), t([2]),
                                      t([2]), scal(0.1), t([1, 2, 8, 128])], "fp8 v8 not S-contiguous"),
    ("launch_h3_full_attention_fp8", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), vt(1, 2, 8, ADDR + 8), t([2]), t([2]),
                                      t([2]), scal(0.1), t([1, 2, 8, 128])], "fp8 misaligned v8"),
    ("launch_h3_full_attention_fp8", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), vt(1, 2, 8), t([3]), t([2]), t([2]),
                                      scal(0.1), t([1, 2, 8, 128])], "fp8 q descale length"),
    ("launch_h3_full_attention_fp8", [t([1, 2, 8, 128]), t([1, 2, 0, 128]), vt(1, 2, 0), t([2]), t([2]), t([2]),
                                      scal(0.1), t([1, 2, 8, 128])], "fp8 no keys"),
    ("launch_h3_full_attention_fp8", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), vt(1, 2, 8), t([2]), t([2]), t([2]),
                                      NULLSCALAR, t([1, 2, 8, 128])], "fp8 scale without data"),
    ("launch_h3_full_attention_fp8", [t([1 << 16, 1 << 12, 1 << 20, 128]), t([1 << 16, 1 << 12, 8, 128]),
                                      vt(1 << 16, 1 << 12, 8), t([1 << 12]), t([1 << 12]), t([1 << 12]), scal(0.1),
                                      t([1 << 16, 1 << 12, 1 << 20, 128])], "fp8 grid above 2^31"),
    # bf16 logits + fp8 P.V: q, k bf16; v8 as V^T; v_descale [H].
    ("launch_h3_full_attention_fp8pv", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), t([1, 2, 8, 128]), t([2]), scal(0.1),
                                        t([1, 2, 8, 128])], "fp8pv v8 not S-contiguous"),
    ("launch_h3_full_attention_fp8pv", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), vt(1, 2, 8, ADDR + 8), t([2]),
                                        scal(0.1), t([1, 2, 8, 128])], "fp8pv misaligned v8"),
    ("launch_h3_full_attention_fp8pv", [t([1, 2, 8, 128]), t([1, 2, 8, 128]), vt(1, 2, 8), t([1]), scal(0.1),
                                        t([1, 2, 8, 128])], "fp8pv v descale length"),
    ("launch_h3_full_attention_fp8pv", [t([1, 2, 8, 128]), t([1, 2, 0, 128]), vt(1, 2, 0), t([2]), scal(0.1),
                                        t([1, 2, 8, 128])], "fp8pv no keys"),
    ("launch_h3_full_attention_fp8pv", [t([1, 2, 8, 128], data=ADDR + 2), t([1, 2, 8, 128]), vt(1, 2, 8), t([2]),
                                        scal(0.1), t([1, 2, 8, 128])], "fp8pv misaligned q"),
    # Sequences within 1024 of 2^31 (stride-0 keys: no memory behind them):
    # rounding them up to whole tiles would overflow the kernels' 32-bit counts.
    ("launch_h3_full_attention", [t([1, 1, 8, 128]), t([1, 1, LONG_S, 128], [0, 0, 0, 1]),
                                  t([1, 1, LONG_S, 128], [0, 0, 0, 1]), scal(0.1), t([1, 1, 8, 128])],
     "keys within 1024 of 2^31"),
    ("launch_h3_full_attention", [t([1, 1, LONG_S, 128], [0, 0, 0, 1]), t([1, 1, 8, 128]), t([1, 1, 8, 128]),
                                  scal(0.1), t([1, 1, LONG_S, 128], [0, 0, 0, 1])], "queries within 1024 of 2^31"),
    ("launch_h3_full_attention_fp8pv", [t([1, 1, 8, 128]), t([1, 1, LONG_S, 128], [0, 0, 0, 1]), vt(1, 1, LONG_S),
                                        t([1]), scal(0.1), t([1, 1, 8, 128])], "fp8pv keys within 1024 of 2^31"),
]


@pytest.mark.parametrize("name,args,why", CASES, ids=[c[2] for c in CASES])
def test_invalid_arguments_rejected_on_host(lib, name, args, why):
    status = lib.call(name, 0, *(a(lib) for a in args))
    assert status == INVALID, f"{name}: {why}: status {status}"


EMPTY = [
    ("launch_h3_rms_exact", [t([1, 0, 128]), t([128]), scal(), t([1, 0, 128])]),
    ("launch_h3_rms_modulate_exact", [t([0, 4, 128]), t([128]), scal(), t([0, 4, 128]), t([0, 4, 128]),
                                      t([0, 4, 128])]),
    ("launch_h3_gated_residual_exact", [t([1, 0, 64])] * 4),
    ("launch_h3_swiglu_exact", [t([1, 4, 0])] * 3),
    ("launch_h3_rms_modulate_indexed", [t([1, 0, 128]), t([128]), scal(), t([0, 128]), t([0, 128]), t([1, 0]),
                                        t([1, 0, 128])]),
    ("launch_h3_gated_residual_rms_modulate_indexed",
     [t([1, 0, 128]), t([2, 128]), t([1, 0, 128]), t([128]), scal(), t([2, 128]), t([2, 128]), t([1, 0]),
      t([1, 0, 128]), t([1, 0, 128])]),
    ("launch_h3_gated_residual_indexed", [t([1, 0, 64]), t([2, 64]), t([1, 0, 64]), t([1, 0]), t([1, 0, 64])]),
    ("launch_h3_qk_norm_rope", [t([0, 1, 2, 128])] * 3 + [t([128])] * 3 + [scal(), t([0, 48]), t([0, 48])]
     + [t([0, 1, 2, 128])] * 3),
    ("launch_h3_rope_cache", [t([0, 3]), t([16]), t([0, 48]), t([0, 48])]),
    ("launch_h3_qkv_norm_rope_pack", [t([0, 2, 3, 128])] * 3 + [t([128]), t([128]), scal(), t([0, 48]),
                                      t([0, 48]), t([0])] + [t([0, 2, 3, 128])] * 3),
    ("launch_h3_full_attention", [t([1, 2, 0, 128]), t([1, 2, 8, 128]), t([1, 2, 8, 128]), scal(0.1),
                                  t([1, 2, 0, 128])]),
    ("launch_h3_vision_attention_72", [t([1, 2, 0, 72]), t([1, 2, 8, 72]), t([1, 2, 8, 72]), scal(0.1),
                                       t([1, 2, 0, 72])]),
    ("launch_h3_full_attention_fp8", [t([1, 2, 0, 128]), t([1, 2, 8, 128]), vt(1, 2, 8), t([2]), t([2]), t([2]),
                                      scal(0.1), t([1, 2, 0, 128])]),
    ("launch_h3_full_attention_fp8pv", [t([1, 2, 0, 128]), t([1, 2, 8, 128]), vt(1, 2, 8), t([2]), scal(0.1),
                                        t([1, 2, 0, 128])]),
    ("launch_h3_quantize_fp8_per_head", [t([1, 0, 8, 128]), t([1, 0, 8, 128]), t([0])]),
    ("launch_h3_quantize_fp8_two_term", [t([1, 0, 8, 128]), t([1, 0, 8, 128]), t([1, 0, 8, 128]), t([0])]),
    ("launch_h3_full_attention_fp8x2", [t([1, 2, 0, 128])] * 2 + [t([1, 2, 8, 128])] * 2 +
     [vt(1, 2, 8), t([2]), t([2]), t([2]), scal(0.1), t([1, 2, 0, 128])]),
    ("launch_h3_full_attention_ws", [t([1, 2, 0, 128]), t([1, 2, 8, 128]), t([1, 2, 8, 128]), scal(0.1),
                                     t([1, 2, 0, 128]), t([4096])]),
]


@pytest.mark.parametrize("name,args", EMPTY, ids=[e[0] for e in EMPTY])
def test_empty_launch_is_a_no_op(lib, name, args):
    assert lib.call(name, 0, *(a(lib) for a in args)) == 0


# ------------------------------------------------------------------ Python faces

def test_python_factories_validate(pkg):
    with pytest.raises(ValueError):
        pkg.make_attention(head_dim=64)
    with pytest.raises(ValueError):
        pkg.make_attention(head_dim=0)
    with pytest.raises(ValueError):
        pkg.make_attention(head_dim=72, numerics="bf16_prescale")
    pkg.make_attention(head_dim=72)
    with pytest.raises(ValueError):
        pkg.make_attention(numerics="tf32")
    with pytest.raises(ValueError):
        pkg.make_attention(dtype=torch.float16)
    with pytest.raises(ValueError):
        pkg.make_qk_norm_rope(block_tokens=2, ranks=2)
    with pytest.raises(ValueError):
        pkg.make_swiglu(dtype="float16")
    for numerics in ("fp32_qk", "fp32_qk_dotacc", "fp32_qk_split", "bf16_prescale"):
        assert callable(pkg.make_attention(numerics=numerics))


def test_python_faces_reject_host_tensors(pkg):
    x = torch.zeros(1, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="cuda"):
        pkg.make_rms(width=128)(x, torch.zeros(128, dtype=torch.bfloat16), 1e-6, x)
    q = torch.zeros(1, 2, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pkg.make_attention()(q, q, q, 0.1, q)
    with pytest.raises(ValueError):
        pkg.make_attention()(q[0], q, q, 0.1, q)


def test_noalloc_pack_face_rejects_what_it_cannot_take(pkg):
    """The allocation-free pack's Python face: one rank, at most the slot
    array's heads, int64 positions (converting would allocate); each raises
    before any device work."""
    kernel = pkg.make_qkv_norm_rope_pack_fp8_noalloc()
    bf = torch.bfloat16

    def call(T, P, Hs, positions_dtype=torch.int64):
        x = torch.zeros(T, P, Hs, 128, dtype=bf)
        w = torch.zeros(128, dtype=bf)
        u8 = torch.zeros(T, P, Hs, 128, dtype=torch.uint8)
        d = torch.zeros(P * Hs)
        kernel(x, x, x, w, w, 1e-6, torch.zeros(T, 96, dtype=bf), torch.zeros(T, dtype=positions_dtype),
               u8, u8, x, d, d, torch.zeros(1, Hs, T, 128, dtype=torch.uint8), torch.zeros(Hs))

    with pytest.raises(ValueError, match="one rank"):
        call(4, 2, 3)
    with pytest.raises(ValueError, match="static slot array holds 1024 heads"):
        call(2, 1, 1025)
    with pytest.raises(ValueError, match="int64 positions"):
        call(4, 1, 3, torch.int32)


def test_missing_library_raises_for_every_entry_point(tmp_path):
    """Without libh3mi355x.so every entry point raises ImportError (in a fresh
    interpreter, whose library path names a file that does not exist): the
    package has no non-HIP path to fall back to."""
    code = (
        "import importlib, sys\n"
        "from pathlib import Path\n"
        f"sys.path.insert(0, {str(ROOT)!r})\n"
        "L = importlib.import_module('minimaxh3_on_k100-ai_amd._lib')\n"
        f"L.LIBRARY_PATH = Path({str(tmp_path / 'absent.so')!r})\n"
        "names = sorted(L.ENTRY_POINTS)\n"
        "for name in names:\n"
        "    try:\n"
        "        L.entry(name)\n"
        "    except ImportError as e:\n"
        "        assert 'no non-HIP fallback' in str(e), e\n"
        "        continue\n"
        "    raise SystemExit('no error for ' + name)\n"
        "try:\n"
        "    L.attention_workspace_bytes(1, 1, 1, 1)\n"
        "    raise SystemExit('no error for the workspace query')\n"
        "except ImportError:\n"
        "    pass\n"
        "print('raised for', len(names))\n"
    )
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert f"raised for {len(declared_entry_points())}" in r.stdout, r.stdout


def test_raw_qk_norm_rope_form_is_twelve_arguments(pkg):
    raw = pkg.make_qk_norm_rope(caller="hip")
    assert raw.__code__.co_argcount == 12

"""The C ABI (CPU): the built library loads, exports every function include/*.h
declares, and rejects bad arguments before touching the device."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

import homelab_amd as hip
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"^[A-Za-z_][\w \*]*?\b(oom_\w+)\s*\(", text, flags=re.M))
    return names


def test_every_declared_symbol_is_exported_and_bound():
    names = declared_functions()
    assert len(names) >= 10
    out = subprocess.run(["nm", "-D", "--defined-only", hip.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r" T (oom_\w+)$", out.stdout, flags=re.M))
    assert names <= exported, names - exported
    assert names == set(hip.SIGNATURES), names ^ set(hip.SIGNATURES)
    lib = hip.lib()
    for n in names:
        assert getattr(lib, n) is not None


def test_library_has_no_oracle_dependency():
    out = subprocess.run(["ldd", hip.LIB_PATH], capture_output=True, text=True)
    assert "oracle" not in out.stdout
    syms = subprocess.run(["nm", "-D", hip.LIB_PATH], capture_output=True, text=True).stdout
    assert "oracle_" not in syms


def test_argument_errors_without_a_device():
    lib = hip.lib()
    null = ctypes.c_void_p(0)
    rc = lib.oom_router_topk(null, null, null, 1, 128, 33, null)
    assert rc == -1 and b"top-k > 32" in lib.oom_last_error()
    rc = lib.oom_gemv_fp8(null, 0, null, null, 0, null, 0, 1, 16, 130, null, 0, null)
    assert rc == -1 and b"multiple of 16" in lib.oom_last_error()
    geo = hip.record_geometry(4096, 1536)
    bad = hip.Fp8Record(4096, 1530, geo.gate_weight, geo.gate_scale, geo.up_weight, geo.up_scale, geo.down_weight,
                        geo.down_scale)
    rc = lib.oom_moe_gate_up_fp8(null, null, null, 1, null, 0, null, ctypes.byref(bad), null)
    assert rc == -1 and b"multiples of 16" in lib.oom_last_error()
    rc = lib.oom_moe_decode_fp8(null, null, 0, null, 1, 128, 8, ctypes.byref(geo), null, null, null, 0, null, 0, null)
    assert rc == -1 and b"null buffer" in lib.oom_last_error()
    rc = lib.oom_attn_decode_paged(null, 1, null, null, null, 1, 16, 10, 64, 8, 64, 0.1, null, 1, null, 0, null)
    assert rc == -1 and b"head_dim" in lib.oom_last_error()
    rc = lib.oom_attn_decode_paged(null, 1, null, null, null, 1, 16, 10, 64, 4, 128, 0.1, null, 1, null, 0, null)
    assert rc == -1 and b"at most 8" in lib.oom_last_error()
    rc = lib.oom_attn_decode_paged(null, 1, null, null, null, 1, 8, 10, 64, 8, 128, 0.1, null, 1, null, 0, null)
    assert rc == -1 and b"multiple of 16" in lib.oom_last_error()
    rc = lib.oom_attn_decode_paged(null, 1, null, null, null, 1, 16, 10, 64, 8, 128, 0.1, null, 1, null, 0, null)
    assert rc == -1 and b"null buffer" in lib.oom_last_error()
    g4 = hip.nvfp4_geometry(2560, 640)
    bad4 = hip.nvfp4_geometry(2560, 648)
    bad4.inter = 644
    rc = lib.oom_moe_gate_up_nvfp4(null, null, null, 1, null, 1, null, ctypes.byref(bad4), null)
    assert rc == -1 and b"multiples of 16" in lib.oom_last_error()
    wide = hip.nvfp4_geometry(8192, 640)
    rc = lib.oom_moe_down_nvfp4(null, null, 1, null, null, ctypes.byref(wide), null)
    assert rc == -1 and b"at most 4096" in lib.oom_last_error()
    rc = lib.oom_moe_decode_nvfp4(null, null, 1, null, 1, 512, 10, ctypes.byref(g4), null, null, null, 1, null, 0, null)
    assert rc == -1 and b"null buffer" in lib.oom_last_error()
    rc = lib.oom_moe_decode_nvfp4(null, null, 1, null, 1, 512, 40, ctypes.byref(g4), null, null, null, 1, null, 0, null)
    assert rc == -1 and b"top-k > 32" in lib.oom_last_error()


def test_workspace_sizes():
    geo = hip.record_geometry(4096, 1536)
    assert hip.gemv_fp8_workspace_size(1, 512, 2560) > 0  # split-K shape
    need = hip.moe_decode_fp8_workspace_size(16, 128, 8, geo)
    assert need >= 16 * 8 * (4096 + 1536) * 4
    assert hip.moe_plan_size(16, 128, 8) == 2 + 2 * 128 + 2 * 128


def test_nvfp4_geometry_agrees_with_oracle():
    for h, i in [(2560, 640), (4096, 1536), (1040, 432)]:
        a, b = hip.nvfp4_geometry(h, i), oracle.nvfp4_geometry(h, i)
        assert [getattr(a, f) for f, _ in a._fields_[:-1]] == [getattr(b, f) for f, _ in b._fields_[:-1]]
        assert list(a.scale2) == list(b.scale2)
        assert hip.nvfp4_stride(a) == oracle.nvfp4_stride(b)
    g = hip.nvfp4_geometry(2560, 640)
    assert hip.moe_decode_nvfp4_workspace_size(1, 512, 10, g) >= 10 * (2560 + 640) * 4


def test_geometry_agrees_with_oracle():
    for h, i in [(4096, 1536), (256, 128), (2560, 640)]:
        a, b = hip.record_geometry(h, i), oracle.record_geometry(h, i)
        assert [getattr(a, f) for f, _ in a._fields_] == [getattr(b, f) for f, _ in b._fields_]
        assert hip.record_stride(a) == oracle.record_stride(b)

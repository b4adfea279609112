"""The oracle: a CPU restatement of oom-inference's decode hot path (C, in this folder).

TEST INFRASTRUCTURE. Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline
leg of ``bench.py`` import this package, and only as the checker (or, for the CPU
baseline, as the timed restatement of the reference's CPU path). The product
library never loads it and has no fallback to it.

Every function here wraps one C function of ``oom_oracle.h``; the reference
file:line each restates is cited there.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboom_oracle.so")

F32, BF16 = 0, 1
SCALE_ROW, SCALE_1X128, SCALE_128X128 = 0, 1, 2

_lib = None


def build() -> str:
    """Compiles liboom_oracle.so with gcc (make)."""
    subprocess.run(["make", "-s", "-C", HERE, "-B", "liboom_oracle.so"], check=True)
    return LIB_PATH


class Fp8Record(ctypes.Structure):
    """OomFp8Record of include/oom_hip.h: byte offsets of an FP8 expert record's parts."""

    _fields_ = [(n, ctypes.c_int64) for n in (
        "hidden", "inter", "gate_weight", "gate_scale", "up_weight", "up_scale", "down_weight", "down_scale")]


def record_geometry(hidden: int, inter: int) -> Fp8Record:
    """The fp8-e4m3-b128 record layout: parts in the order gate.weight, gate.scale,
    up.weight, up.scale, down.weight, down.scale, each 256-byte aligned."""
    def al(v):
        return (v + 255) // 256 * 256
    nb = lambda n, k: ((n + 127) // 128) * ((k + 127) // 128) * 4  # noqa: E731
    o = 0
    gw = o; o = al(o + inter * hidden)
    gs = o; o = al(o + nb(inter, hidden))
    uw = o; o = al(o + inter * hidden)
    us = o; o = al(o + nb(inter, hidden))
    dw = o; o = al(o + hidden * inter)
    ds = o; o = al(o + nb(hidden, inter))
    return Fp8Record(hidden, inter, gw, gs, uw, us, dw, ds)


class Bf16Record(ctypes.Structure):
    """OomBf16Record of include/oom_hip.h: byte offsets of a bf16 expert record's parts."""

    _fields_ = [(n, ctypes.c_int64) for n in ("hidden", "inter", "gate_weight", "up_weight", "down_weight")]


def bf16_geometry(hidden: int, inter: int) -> Bf16Record:
    """The bf16 record layout (docs/dev/format.md:72-73): gate.weight, up.weight bf16
    [inter, hidden], down.weight bf16 [hidden, inter], each part 256-byte aligned."""
    def al(v):
        return (v + 255) // 256 * 256
    gw = 0
    uw = al(gw + inter * hidden * 2)
    dw = al(uw + inter * hidden * 2)
    return Bf16Record(hidden, inter, gw, uw, dw)


def bf16_stride(geo: Bf16Record) -> int:
    return (geo.down_weight + geo.hidden * geo.inter * 2 + 4095) // 4096 * 4096


class Nvfp4Record(ctypes.Structure):
    """OomNvfp4Record of include/oom_hip.h: byte offsets of an NVFP4 expert record's parts
    and the float indices of the three weight_scale_2 scalars."""

    _fields_ = [(n, ctypes.c_int64) for n in (
        "hidden", "inter", "gate_weight", "gate_scale", "up_weight", "up_scale", "down_weight", "down_scale")] + [
        ("scale2", ctypes.c_int64 * 3)]


def nvfp4_geometry(hidden: int, inter: int) -> Nvfp4Record:
    """The nvfp4-modelopt-g16 record of docs/dev/format.md:111-118: a 256-byte part of six
    f32 scalars (gate/up/down weight_scale_2 at floats 0, 2, 4, each followed by its
    input_scale), then gate.weight [inter, hidden / 2], gate.weight_scale [inter,
    hidden / 16], up.*, down.weight [hidden, inter / 2], down.weight_scale [hidden,
    inter / 16], each part 256-byte aligned."""
    def al(v):
        return (v + 255) // 256 * 256
    o = 256
    gw = o; o = al(o + inter * hidden // 2)
    gs = o; o = al(o + inter * hidden // 16)
    uw = o; o = al(o + inter * hidden // 2)
    us = o; o = al(o + inter * hidden // 16)
    dw = o; o = al(o + hidden * inter // 2)
    ds = o
    g = Nvfp4Record(hidden, inter, gw, gs, uw, us, dw, ds)
    g.scale2[0], g.scale2[1], g.scale2[2] = 0, 2, 4
    return g


def nvfp4_size(geo: Nvfp4Record) -> int:
    """Bytes of an NVFP4 record up to the end of its last part."""
    return geo.down_scale + geo.hidden * geo.inter // 16


def nvfp4_stride(geo: Nvfp4Record) -> int:
    """Record size rounded up to 4096 bytes (ALIGN, docs/dev/format.md:37)."""
    return (nvfp4_size(geo) + 4095) // 4096 * 4096


def record_stride(geo: Fp8Record) -> int:
    """Record size rounded up to 4096 bytes (ALIGN, docs/dev/format.md:37)."""
    end = geo.down_scale + ((geo.hidden + 127) // 128) * ((geo.inter + 127) // 128) * 4
    return (end + 4095) // 4096 * 4096


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        I64, I32, F = ctypes.c_int64, ctypes.c_int, ctypes.c_float
        sig = {
            "oracle_e4m3_from_f32": (ctypes.c_uint8, [F]),
            "oracle_e4m3_to_f32": (F, [ctypes.c_uint8]),
            "oracle_bf16_from_f32_n": (None, [P, P, ctypes.c_size_t]),
            "oracle_bf16_to_f32_n": (None, [P, P, ctypes.c_size_t]),
            "oracle_quantize": (I32, [P, I64, I64, I32, P, P]),
            "oracle_scale_count": (I64, [I64, I64, I32]),
            "oracle_quantize_act": (None, [P, I64, I64, I64, P, P]),
            "oracle_seed": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint64]),
            "oracle_gaussian": (None, [P, ctypes.c_size_t, ctypes.c_uint64, F]),
            "oracle_gaussian_bf16": (None, [P, ctypes.c_size_t, ctypes.c_uint64, F, ctypes.c_size_t, I32]),
            "oracle_zipf_bias": (None, [P, I32, ctypes.c_double, ctypes.c_uint64]),
            "oracle_permutation": (None, [P, I32, ctypes.c_uint64]),
            "oracle_router_topk": (None, [P, I32, I32, I32, P, P]),
            "oracle_router_probs": (None, [P, I32, I32, P]),
            "oracle_gemv_fp8": (None, [P, I32, P, P, I32, I64, I64, P]),
            "oracle_gemv_bf16": (None, [P, I32, P, I64, I64, P]),
            "oracle_moe_combine_shared": (None, [P, P, P, P, I32, I32]),
            "oracle_moe_layer_decode_fp8": (I32, [P, I32, P, P, I32, I32, P, P, P, P, P, P, P, P, P]),
            "oracle_moe_plan": (I32, [P, I32, I32, I32, P, P, P, P]),
            "oracle_moe_gate_up_fp8": (None, [P, P, P, I32, P, P, P]),
            "oracle_moe_down_fp8": (None, [P, P, I32, P, P, P]),
            "oracle_moe_combine_slots": (None, [P, P, P, P, I32, I32, I32]),
            "oracle_moe_decode_fp8": (I32, [P, P, P, I32, I32, I32, P, P, P, P]),
            "oracle_e2m1_to_f32": (F, [ctypes.c_uint8]),
            "oracle_nvfp4_rows": (None, [P, P, F, I64, I64, P, I32, P]),
            "oracle_moe_gate_up_nvfp4": (None, [P, P, P, I32, P, P, P]),
            "oracle_moe_gate_up_bf16": (None, [P, P, P, I32, P, P, P]),
            "oracle_moe_down_bf16": (None, [P, P, I32, P, P, P]),
            "oracle_moe_down_nvfp4": (None, [P, P, I32, P, P, P]),
            "oracle_moe_decode_nvfp4": (I32, [P, P, P, I32, I32, I32, P, P, P, P]),
            "oracle_grouped_gemm_fp8": (None, [P, P, P, I32, P, P, I32, P, I64, I64, I64, I64]),
            "oracle_moe_prefill_fp8": (I32, [P, P, P, I32, I32, I32, P, I32, P, P, P]),
            "oracle_attn_decode_paged": (None, [P, P, P, P, I32, I32, I32, I32, I32, F, P]),
            "oracle_host_experts": (I32, [P, P, P, P, I32, P, P, I32]),
            "oracle_f16_from_f32": (ctypes.c_uint16, [F]),
            "oracle_f16_to_f32": (F, [ctypes.c_uint16]),
            "oracle_kv_codebooks": (None, [P]),
            "oracle_kv_row_bytes": (ctypes.c_size_t, [I32, I32]),
            "oracle_kv_rotate": (None, [P, I32, I32, I32]),
            "oracle_kv_append": (None, [P, P, I64, I32, I32, I32, P]),
            "oracle_kv_read": (None, [P, P, I32, I32, I32, P]),
            "oracle_mask_compact": (I32, [P, P, I32]),
            "oracle_attn_decode_turbo": (None, [P, P, P, I32, I32, P, P, I32, I32, I32, F, P]),
            "oracle_moe_tiled_nvfp4": (None, [P, P, P, I32, P, P, I64, I64, I64, I64, I32, I32]),
            "oracle_host_has_avx512": (I32, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    # a pointer object that holds a reference to `a`: an array made inline for one call
    # (a dtype conversion, an address table) stays alive until the call returns
    return a.ctypes.data_as(ctypes.c_void_p)


def _ptrs(arrs) -> np.ndarray:
    """uint64 array of the data addresses of host arrays (a host `recs` table)."""
    return np.array([a.ctypes.data for a in arrs], dtype=np.uint64)


# ---- formats -------------------------------------------------------------------

def e4m3_from_f32(x: float) -> int:
    return int(lib().oracle_e4m3_from_f32(float(x)))


def e4m3_to_f32(b: int) -> float:
    return float(lib().oracle_e4m3_to_f32(int(b)))


def e4m3_decode(q: np.ndarray) -> np.ndarray:
    """Vectorised decode through the oracle's table of all 256 codes."""
    table = np.array([e4m3_to_f32(b) for b in range(256)], dtype=np.float32)
    return table[q]


def bf16_from_f32(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(v.shape, dtype=np.uint16)
    lib().oracle_bf16_from_f32_n(_p(v), _p(out), v.size)
    return out


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().oracle_bf16_to_f32_n(_p(b), _p(out), b.size)
    return out


def scale_count(n: int, k: int, layout: int) -> int:
    return int(lib().oracle_scale_count(n, k, layout))


def quantize(w_bf16: np.ndarray, layout: int):
    """(q uint8 [n, k], scale f32) of bf16 weights under a scale layout."""
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    n, k = w.shape
    q = np.empty((n, k), dtype=np.uint8)
    s = np.empty(scale_count(n, k, layout), dtype=np.float32)
    assert lib().oracle_quantize(_p(w), n, k, layout, _p(q), _p(s)) == 0
    return q, s


def quantize_act(x: np.ndarray, group: int = 0):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    ng = 1 if group == 0 else (cols + group - 1) // group
    q = np.empty((rows, cols), dtype=np.uint8)
    s = np.empty((rows, ng), dtype=np.float32)
    lib().oracle_quantize_act(_p(x), rows, cols, group, _p(q), _p(s))
    return q, (s[:, 0].copy() if group == 0 else s)


def dequantize(q: np.ndarray, scale: np.ndarray, layout: int) -> np.ndarray:
    n, k = q.shape
    w = e4m3_decode(q)
    if layout == SCALE_ROW:
        return w * scale.reshape(n, 1)
    nkb = (k + 127) // 128
    cols = np.arange(k) // 128
    if layout == SCALE_1X128:
        return w * scale.reshape(n, nkb)[:, cols]
    s = scale.reshape((n + 127) // 128, nkb)
    return w * s[np.arange(n) // 128][:, cols]


# ---- generators ----------------------------------------------------------------

def seed(base: int, stream: int) -> int:
    return int(lib().oracle_seed(base, stream))


def gaussian(n: int, seed_: int, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().oracle_gaussian(_p(out), n, seed_, std)
    return out


def gaussian_bf16(shape, seed_: int, std: float = 1.0, chunk: int = 1 << 16, threads: int | None = None) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16)
    lib().oracle_gaussian_bf16(_p(out), n, seed_, std, chunk, threads or min(16, os.cpu_count() or 1))
    return out.reshape(shape)


def zipf_bias(E: int, s: float, seed_: int) -> np.ndarray:
    out = np.empty(E, dtype=np.float32)
    lib().oracle_zipf_bias(_p(out), E, s, seed_)
    return out


def permutation(n: int, seed_: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().oracle_permutation(_p(out), n, seed_)
    return out


# ---- router / GEMV / experts ---------------------------------------------------

def router_topk(logits: np.ndarray, k: int):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    ids = np.empty((T, k), dtype=np.int32)
    w = np.empty((T, k), dtype=np.float32)
    lib().oracle_router_topk(_p(logits), T, E, k, _p(ids), _p(w))
    return ids, w


def router_probs(logits: np.ndarray) -> np.ndarray:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    p = np.empty((T, E), dtype=np.float32)
    lib().oracle_router_probs(_p(logits), T, E, _p(p))
    return p


def gemv_fp8(x: np.ndarray, q: np.ndarray, scale: np.ndarray, layout: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, K = x.shape
    N = q.shape[0]
    y = np.empty((T, N), dtype=np.float32)
    lib().oracle_gemv_fp8(_p(x), T, _p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(scale, dtype=np.float32)),
                          layout, N, K, _p(y))
    return y


def gemv_bf16(x: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    """y[t, n] = sum_k x[t, k] * bf16(w[n, k]) (w_bits uint16 [N, K])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, K = x.shape
    N = w_bits.shape[0]
    y = np.empty((T, N), dtype=np.float32)
    lib().oracle_gemv_bf16(_p(x), T, _p(np.ascontiguousarray(w_bits, dtype=np.uint16)), N, K, _p(y))
    return y


def moe_combine_shared(routed: np.ndarray, shared: np.ndarray, gate: np.ndarray) -> np.ndarray:
    routed = np.ascontiguousarray(routed, dtype=np.float32)
    T, H = routed.shape
    out = np.empty((T, H), dtype=np.float32)
    lib().oracle_moe_combine_shared(_p(routed), _p(np.ascontiguousarray(shared, dtype=np.float32)),
                                    _p(np.ascontiguousarray(gate, dtype=np.float32).reshape(-1)), _p(out), T, H)
    return out


def moe_layer_decode(x: np.ndarray, router_w_bits: np.ndarray, all_recs, k: int, geo: Fp8Record, shared_rec,
                     shared_geo: Fp8Record, gate_w_bits: np.ndarray):
    """(logits, gate, ids, weights, out f32) of one decode MoE layer (router GEMV, routed
    experts, shared expert gated by sigmoid(x . gate_w))."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    E = router_w_bits.shape[0]
    logits = np.empty((T, E), dtype=np.float32)
    gate = np.empty((T, 1), dtype=np.float32)
    ids = np.empty((T, k), dtype=np.int32)
    w = np.empty((T, k), dtype=np.float32)
    out = np.empty((T, geo.hidden), dtype=np.float32)
    table = _ptrs(all_recs)
    rc = lib().oracle_moe_layer_decode_fp8(_p(x), T, _p(np.ascontiguousarray(router_w_bits, dtype=np.uint16)),
                                           _p(table), E, k, ctypes.byref(geo), _p(np.ascontiguousarray(shared_rec)),
                                           ctypes.byref(shared_geo),
                                           _p(np.ascontiguousarray(gate_w_bits, dtype=np.uint16)), _p(logits),
                                           _p(gate), _p(ids), _p(w), _p(out))
    assert rc == 0
    return logits, gate, ids, w, out


def moe_plan(ids: np.ndarray, E: int):
    """(experts, off, assign_tok, slot_assign) of one step, all experts resident."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, k = ids.shape
    A = T * k
    experts = np.empty(A + 1, dtype=np.int32)
    off = np.empty(A + 2, dtype=np.int32)
    tok = np.empty(A, dtype=np.int32)
    slot = np.empty(A, dtype=np.int32)
    n_e = lib().oracle_moe_plan(_p(ids), T, k, E, _p(experts), _p(off), _p(tok), _p(slot))
    if n_e < 0:
        raise ValueError("router id out of range")
    return experts[:n_e].copy(), off[:n_e + 1].copy(), tok, slot


def moe_gate_up(recs, off, assign_tok, x: np.ndarray, geo: Fp8Record) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    A = int(off[-1])
    h = np.empty((A, geo.inter), dtype=np.float32)
    table = _ptrs(recs)
    lib().oracle_moe_gate_up_fp8(_p(table), _p(np.ascontiguousarray(off, dtype=np.int32)),
                                 _p(np.ascontiguousarray(assign_tok, dtype=np.int32)), len(recs), _p(x), _p(h),
                                 ctypes.byref(geo))
    return h


def moe_down(recs, off, h: np.ndarray, geo: Fp8Record) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.float32)
    A = int(off[-1])
    y = np.empty((A, geo.hidden), dtype=np.float32)
    table = _ptrs(recs)
    lib().oracle_moe_down_fp8(_p(table), _p(np.ascontiguousarray(off, dtype=np.int32)), len(recs), _p(h), _p(y),
                              ctypes.byref(geo))
    return y


def moe_combine_slots(y: np.ndarray, slot_assign: np.ndarray, w: np.ndarray) -> np.ndarray:
    T, k = w.shape
    H = y.shape[1]
    out = np.empty((T, H), dtype=np.float32)
    lib().oracle_moe_combine_slots(_p(np.ascontiguousarray(y, dtype=np.float32)),
                                   _p(np.ascontiguousarray(slot_assign, dtype=np.int32)),
                                   _p(np.ascontiguousarray(w, dtype=np.float32)), _p(out), T, H, k)
    return out


def moe_decode(logits: np.ndarray, x: np.ndarray, all_recs, k: int, geo: Fp8Record):
    """(ids, weights, out f32) of one decode MoE step; all_recs[e] is expert e's record (uint8 array)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, E = logits.shape
    ids = np.empty((T, k), dtype=np.int32)
    w = np.empty((T, k), dtype=np.float32)
    out = np.empty((T, geo.hidden), dtype=np.float32)
    table = _ptrs(all_recs)
    rc = lib().oracle_moe_decode_fp8(_p(logits), _p(x), _p(table), T, E, k, ctypes.byref(geo), _p(ids), _p(w), _p(out))
    assert rc == 0
    return ids, w, out


def e2m1_to_f32(code: int) -> float:
    return float(lib().oracle_e2m1_to_f32(code))


def nvfp4_rows(packed: np.ndarray, scales: np.ndarray, s2: float, x: np.ndarray) -> np.ndarray:
    """y [T, rows] of one NVFP4 matrix (packed [rows, cols / 2], scales [rows, cols / 16])."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, half = packed.shape
    T = x.shape[0]
    y = np.empty((T, rows), dtype=np.float32)
    lib().oracle_nvfp4_rows(_p(packed), _p(scales), s2, rows, 2 * half, _p(x), T, _p(y))
    return y


def moe_gate_up_bf16(recs, off, assign_tok, x: np.ndarray, geo: Bf16Record) -> np.ndarray:
    """h f32 [A, inter] over bf16 records (uint8 arrays), x f32 [*, hidden]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    h = np.empty((int(off[-1]), geo.inter), dtype=np.float32)
    lib().oracle_moe_gate_up_bf16(_p(_ptrs(recs)), _p(np.ascontiguousarray(off, dtype=np.int32)),
                                  _p(np.ascontiguousarray(assign_tok, dtype=np.int32)), len(recs), _p(x), _p(h),
                                  ctypes.byref(geo))
    return h


def moe_down_bf16(recs, off, h: np.ndarray, geo: Bf16Record) -> np.ndarray:
    """y f32 [A, hidden] over bf16 records, h f32 [A, inter]."""
    h = np.ascontiguousarray(h, dtype=np.float32)
    y = np.empty((int(off[-1]), geo.hidden), dtype=np.float32)
    lib().oracle_moe_down_bf16(_p(_ptrs(recs)), _p(np.ascontiguousarray(off, dtype=np.int32)), len(recs), _p(h), _p(y),
                               ctypes.byref(geo))
    return y


def moe_gate_up_nvfp4(recs, off, assign_tok, x: np.ndarray, geo: Nvfp4Record) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    h = np.empty((int(off[-1]), geo.inter), dtype=np.float32)
    table = _ptrs(recs)
    lib().oracle_moe_gate_up_nvfp4(_p(table), _p(np.ascontiguousarray(off, dtype=np.int32)),
                                   _p(np.ascontiguousarray(assign_tok, dtype=np.int32)), len(recs), _p(x), _p(h),
                                   ctypes.byref(geo))
    return h


def moe_tiled_nvfp4(recs, off, rows, x: np.ndarray, N: int, K: int, w_off: int, s_off: int, s2_idx: int,
                    terms: int) -> np.ndarray:
    """y f32 [A, N] of one NVFP4 projection over host records (uint8 arrays), x f32 [*, K]."""
    off = np.ascontiguousarray(off, dtype=np.int32)
    A = int(off[-1])
    y = np.zeros((A, N), dtype=np.float32)
    tab = _ptrs(recs) if len(recs) else np.zeros(1, dtype=np.uint64)
    lib().oracle_moe_tiled_nvfp4(_p(tab), _p(off), None if rows is None else _p(np.ascontiguousarray(rows, np.int32)),
                                 len(recs), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(y), N, K, w_off, s_off,
                                 s2_idx, terms)
    return y


def moe_down_nvfp4(recs, off, h: np.ndarray, geo: Nvfp4Record) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.float32)
    y = np.empty((int(off[-1]), geo.hidden), dtype=np.float32)
    table = _ptrs(recs)
    lib().oracle_moe_down_nvfp4(_p(table), _p(np.ascontiguousarray(off, dtype=np.int32)), len(recs), _p(h), _p(y),
                                ctypes.byref(geo))
    return y


def moe_decode_nvfp4(logits: np.ndarray, x: np.ndarray, all_recs, k: int, geo: Nvfp4Record):
    """(ids, weights, out f32) of one decode MoE step over NVFP4 records."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, E = logits.shape
    ids = np.empty((T, k), dtype=np.int32)
    w = np.empty((T, k), dtype=np.float32)
    out = np.empty((T, geo.hidden), dtype=np.float32)
    table = _ptrs(all_recs)  # held for the call: the C side reads it
    rc = lib().oracle_moe_decode_nvfp4(_p(logits), _p(x), _p(table), T, E, k, ctypes.byref(geo), _p(ids), _p(w),
                                       _p(out))
    assert rc == 0
    return ids, w, out


def grouped_gemm_fp8(recs, off, rows, xq, x_scale, x_group, N, K, w_off, s_off) -> np.ndarray:
    A = int(off[-1])
    y = np.empty((A, N), dtype=np.float32)
    table = _ptrs(recs)
    rows_arr = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    lib().oracle_grouped_gemm_fp8(_p(table), _p(np.ascontiguousarray(off, dtype=np.int32)), _p(rows_arr), len(recs),
                                  _p(np.ascontiguousarray(xq, dtype=np.uint8)),
                                  _p(np.ascontiguousarray(x_scale, dtype=np.float32)), x_group, _p(y), N, K, w_off, s_off)
    return y


def moe_prefill(logits: np.ndarray, x: np.ndarray, all_recs, k: int, geo: Fp8Record, h_bf16: bool = False):
    """The whole prefill step; h_bf16 rounds h to bf16 before the down projection (the
    reference's ExpertPrecision::Bf16), else h stays fp32 (ExpertPrecision::Exact)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, E = logits.shape
    ids = np.empty((T, k), dtype=np.int32)
    w = np.empty((T, k), dtype=np.float32)
    out = np.empty((T, geo.hidden), dtype=np.float32)
    table = _ptrs(all_recs)
    n_e = lib().oracle_moe_prefill_fp8(_p(logits), _p(x), _p(table), T, E, k, ctypes.byref(geo), int(h_bf16), _p(ids),
                                       _p(w), _p(out))
    assert n_e >= 0
    return ids, w, out


def attn_decode_paged(q_bf16, k_pages, v_pages, page_table, page_size, kv_len, H, Hkv, D, scale) -> np.ndarray:
    out = np.empty((H, D), dtype=np.float32)
    lib().oracle_attn_decode_paged(_p(np.ascontiguousarray(q_bf16, dtype=np.uint16)),
                                   _p(np.ascontiguousarray(k_pages, dtype=np.uint16)),
                                   _p(np.ascontiguousarray(v_pages, dtype=np.uint16)),
                                   _p(np.ascontiguousarray(page_table, dtype=np.int32)), page_size, kv_len, H, Hkv, D,
                                   scale, _p(out))
    return out


def host_experts(geo: Fp8Record, records, job_tokens, x: np.ndarray, threads: int) -> np.ndarray:
    """The reference CPU path: per job (record, token list), unweighted expert outputs by job then token."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    off = np.zeros(len(job_tokens) + 1, dtype=np.int32)
    for i, t in enumerate(job_tokens):
        off[i + 1] = off[i] + len(t)
    toks = np.ascontiguousarray(np.concatenate([np.asarray(t, dtype=np.int32) for t in job_tokens])
                                if job_tokens else np.zeros(0, np.int32))
    y = np.empty((int(off[-1]), geo.hidden), dtype=np.float32)
    table = _ptrs(records)
    lib().oracle_host_experts(ctypes.byref(geo), _p(table), _p(toks), _p(off), len(job_tokens), _p(x), _p(y), threads)
    return y


def host_has_avx512() -> bool:
    return bool(lib().oracle_host_has_avx512())


# ---- Turbo KV cache and the d = 256, G = 12 decode attention (turbo.c) ----

_codebooks = None


def kv_codebooks() -> np.ndarray:
    """KvFormat::codebooks: 508 levels (2..8 bits, ascending, concatenated); the levels for
    b bits start at 2^b - 4."""
    global _codebooks
    if _codebooks is None:
        t = np.empty(508, dtype=np.float32)
        lib().oracle_kv_codebooks(_p(t))
        _codebooks = t
    return _codebooks


def f16_from_f32(x: float) -> int:
    return int(lib().oracle_f16_from_f32(x))


def f16_to_f32(h: int) -> float:
    return float(lib().oracle_f16_to_f32(h))


def kv_row_bytes(d: int, bits: int) -> int:
    return int(lib().oracle_kv_row_bytes(d, bits))


def kv_rotate(x: np.ndarray, inverse: bool) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    d = y.shape[-1]
    lib().oracle_kv_rotate(_p(y), y.size // d, d, int(inverse))
    return y


def kv_append(src: np.ndarray, bits: int, cache: np.ndarray | None = None, row0: int = 0) -> np.ndarray:
    """Rows of src (..., d) appended at cache row row0 (a fresh zeroed cache when None)."""
    src = np.ascontiguousarray(src, dtype=np.float32)
    d = src.shape[-1]
    rows = src.size // d
    rb = kv_row_bytes(d, bits)
    if cache is None:
        cache = np.zeros((row0 + rows) * rb, dtype=np.uint8)
    lib().oracle_kv_append(_p(src), _p(cache), row0, rows, d, bits, _p(kv_codebooks()))
    return cache


def kv_read(cache: np.ndarray, rows: int, d: int, bits: int) -> np.ndarray:
    out = np.empty((rows, d), dtype=np.float32)
    lib().oracle_kv_read(_p(np.ascontiguousarray(cache, dtype=np.uint8)), _p(out), rows, d, bits, _p(kv_codebooks()))
    return out


def mask_compact(mask: np.ndarray) -> np.ndarray:
    mask = np.ascontiguousarray(mask, dtype=np.uint8)
    sel = np.zeros(mask.size + 1, dtype=np.int32)
    lib().oracle_mask_compact(_p(mask), _p(sel), mask.size)
    return sel


def attn_decode_turbo(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, kb: int, vb: int, mask: np.ndarray,
                      H: int, Hkv: int, kv_len: int, scale: float) -> np.ndarray:
    out = np.empty((H, 256), dtype=np.float32)
    lib().oracle_attn_decode_turbo(_p(np.ascontiguousarray(q, dtype=np.float32)),
                                   _p(np.ascontiguousarray(k_cache, dtype=np.uint8)),
                                   _p(np.ascontiguousarray(v_cache, dtype=np.uint8)), kb, vb, _p(kv_codebooks()),
                                   _p(np.ascontiguousarray(mask, dtype=np.uint8)), H, Hkv, kv_len, scale, _p(out))
    return out

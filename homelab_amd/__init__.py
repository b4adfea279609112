"""homelab_amd: MI355X (gfx950) kernels for oom-inference's decode hot path.

The product is liboom_hip.so, a C ABI (include/oom_hip.h) that an `oominf-rocm`
backend crate binds. This module loads that library with ctypes so tests and the
bench call exactly the entry points the engine would; torch provides device memory
and streams only. There is no fallback: without the built library every call raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboom_hip.so")

OK = 0
ERR_ARG, ERR_WORKSPACE, ERR_LAUNCH, ERR_KERNEL = -1, -2, -3, -4
F32, BF16 = 0, 1
SCALE_ROW, SCALE_1X128, SCALE_128X128 = 0, 1, 2
EXPERT_EXACT, EXPERT_BF16 = 0, 1  # the prefill down projection's activation precision

_lib = None


class OomError(RuntimeError):
    pass


class Fp8Record(ctypes.Structure):
    """OomFp8Record: byte offsets of an FP8 expert record's parts."""

    _fields_ = [(n, ctypes.c_int64) for n in (
        "hidden", "inter", "gate_weight", "gate_scale", "up_weight", "up_scale", "down_weight", "down_scale")]


# entry point -> (restype, argtypes); every symbol include/oom_hip.h declares
P, I32, I64, SZ, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float
U64 = ctypes.c_uint64
SIGNATURES = {
    "oom_last_error": (ctypes.c_char_p, []),
    "oom_workspace_init": (I32, [P, SZ, P]),
    "oom_status": (I32, [P]),
    "oom_set_wait_limit": (I32, [ctypes.c_uint32]),
    "oom_router_topk": (I32, [P, P, P, I32, I32, I32, P]),
    "oom_gemv_fp8_workspace_size": (SZ, [I32, I64, I64]),
    "oom_gemv_fp8": (I32, [P, I32, P, P, I32, P, I32, I32, I64, I64, P, SZ, P]),
    "oom_gemv_bf16_workspace_size": (SZ, [I32, I64, I64]),
    "oom_gemv_bf16": (I32, [P, I32, P, P, I32, I32, I64, I64, P, SZ, P]),
    "oom_moe_combine_shared": (I32, [P, P, P, P, I32, I32, I32, P]),
    "oom_moe_layer_decode_fp8_workspace_size": (SZ, [I32, I32, I32, P, P]),
    "oom_moe_layer_decode_fp8": (I32, [P, I32, P, P, I32, I32, I32, P, P, P, P, P, P, P, I32, P, SZ, P]),
    "oom_moe_gate_up_fp8": (I32, [P, P, P, I32, P, I32, P, P, P]),
    "oom_moe_down_fp8": (I32, [P, P, I32, P, P, P, P]),
    "oom_moe_gate_up_bf16": (I32, [P, P, P, I32, P, I32, P, P, P]),
    "oom_moe_down_bf16": (I32, [P, P, I32, P, P, P, P]),
    "oom_moe_combine_slots": (I32, [P, P, P, P, I32, I32, I32, I32, P]),
    "oom_moe_plan_size": (SZ, [I32, I32, I32]),
    "oom_moe_plan": (I32, [P, I32, I32, I32, P, P, P, P]),
    "oom_moe_decode_fp8_workspace_size": (SZ, [I32, I32, I32, P]),
    "oom_moe_decode_fp8": (I32, [P, P, I32, P, I32, I32, I32, P, P, P, P, I32, P, SZ, P]),
    "oom_moe_decode_fp8_noalloc_max_bytes": (SZ, []),
    "oom_moe_decode_fp8_noalloc": (I32, [P, P, I32, P, I32, I32, I32, P, P, P, P, I32, P]),
    "oom_moe_gate_up_nvfp4": (I32, [P, P, P, I32, P, I32, P, P, P]),
    "oom_moe_down_nvfp4": (I32, [P, P, I32, P, P, P, P]),
    "oom_moe_decode_nvfp4_workspace_size": (SZ, [I32, I32, I32, P]),
    "oom_moe_decode_nvfp4": (I32, [P, P, I32, P, I32, I32, I32, P, P, P, P, I32, P, SZ, P]),
    "oom_quantize_rows_fp8": (I32, [P, I32, I64, I64, P, P, P]),
    "oom_moe_grouped_gemm_fp8": (I32, [P, P, P, I32, I32, P, P, I32, P, I64, I64, I64, I64, P]),
    "oom_moe_prefill_fp8_workspace_size": (SZ, [I32, I32, I32, P]),
    "oom_moe_prefill_fp8": (I32, [P, P, I32, P, I32, I32, I32, P, I32, P, P, P, I32, P, SZ, P]),
    "oom_moe_tiled_nvfp4": (I32, [P, P, P, I32, I32, P, P, I32, I32, I64, I64, I32, I32, P]),
    "oom_moe_swiglu_range": (I32, [P, P, P, I64, I64, P]),
    "oom_attn_decode_workspace_size": (SZ, [I32, I32, I32, I32]),
    "oom_attn_decode_paged": (I32, [P, I32, P, P, P, I32, I32, I32, I32, I32, I32, F, P, I32, P, SZ, P]),
    "oom_kv_codebook_size": (SZ, []),
    "oom_kv_codebooks": (I32, [P, SZ]),
    "oom_kv_row_bytes": (SZ, [I32, I32]),
    "oom_kv_rotate": (I32, [P, I32, I32, I32, P]),
    "oom_kv_append": (I32, [P, P, I64, I32, I32, I32, I32, P, P]),
    "oom_kv_read": (I32, [P, P, I32, I32, I32, I32, P, P]),
    "oom_mask_compact": (I32, [P, P, I32, P]),
    "oom_attn_decode_turbo_workspace_size": (SZ, [I32, I32, I32, I32]),
    "oom_attn_decode_turbo": (I32, [P, P, P, I32, I32, P, P, I32, I32, I32, I32, F, P, P, SZ, P]),
    "oom_copy_queue_create": (I32, [P]),
    "oom_copy_queue_destroy": (I32, [P]),
    "oom_host_alloc": (I32, [P, SZ]),
    "oom_host_free": (I32, [P]),
    "oom_copy_to_device": (I32, [P, U64, P, SZ]),
    "oom_copy_on_device": (I32, [P, U64, U64, SZ]),
    "oom_copy_records_to_device": (I32, [P, P, P, SZ, I32]),
    "oom_download_async": (I32, [P, P, P, SZ]),
    "oom_event_create": (I32, [P]),
    "oom_event_destroy": (I32, [P]),
    "oom_event_record": (I32, [P, P]),
    "oom_stream_wait_event": (I32, [P, P]),
    "oom_event_done": (I32, [P]),
    "oom_event_wait": (I32, [P]),
    "oom_stream_sync": (I32, [P]),
}


def lib() -> ctypes.CDLL:
    """The loaded product library; raises if it was not built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OomError(f"{LIB_PATH} is missing: build it with `python -m homelab_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        raise OomError(f"status {rc}: {lib().oom_last_error().decode()}")


def status(stream=None) -> int:
    """oom_status: waits for `stream`, returns OK or ERR_KERNEL (a bounded wait inside an
    earlier kernel gave up; its outputs are invalid) and clears the device's status word."""
    return lib().oom_status(_stream(stream))


def set_wait_limit(spins: int) -> None:
    """oom_set_wait_limit: polls of each bounded wait of later launches (0: the default)."""
    check(lib().oom_set_wait_limit(spins))


def _ptr(t) -> ctypes.c_void_p | None:
    if t is None:
        return None
    if isinstance(t, int):
        return ctypes.c_void_p(t)
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream=None) -> ctypes.c_void_p:
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _dtype_code(t) -> int:
    import torch

    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.bfloat16:
        return BF16
    raise OomError(f"unsupported activation dtype {t.dtype}")


def record_geometry(hidden: int, inter: int) -> Fp8Record:
    """The fp8-e4m3-b128 record layout (gate.weight, gate.scale, up.weight, up.scale,
    down.weight, down.scale; parts 256-byte aligned)."""
    def al(v):
        return (v + 255) // 256 * 256

    def nb(n, k):
        return ((n + 127) // 128) * ((k + 127) // 128) * 4
    o = 0
    gw = o; o = al(o + inter * hidden)
    gs = o; o = al(o + nb(inter, hidden))
    uw = o; o = al(o + inter * hidden)
    us = o; o = al(o + nb(inter, hidden))
    dw = o; o = al(o + hidden * inter)
    ds = o
    return Fp8Record(hidden, inter, gw, gs, uw, us, dw, ds)


def record_stride(geo: Fp8Record) -> int:
    end = geo.down_scale + ((geo.hidden + 127) // 128) * ((geo.inter + 127) // 128) * 4
    return (end + 4095) // 4096 * 4096


class Bf16Record(ctypes.Structure):
    """OomBf16Record of include/oom_hip.h: part offsets of a bf16 expert record."""

    _fields_ = [(n, ctypes.c_int64) for n in ("hidden", "inter", "gate_weight", "up_weight", "down_weight")]


def bf16_geometry(hidden: int, inter: int) -> Bf16Record:
    """The bf16 record layout (gate.weight, up.weight, down.weight; parts 256-byte aligned)."""
    def al(v):
        return (v + 255) // 256 * 256
    gw = 0
    uw = al(gw + inter * hidden * 2)
    dw = al(uw + inter * hidden * 2)
    return Bf16Record(hidden, inter, gw, uw, dw)


class Nvfp4Record(ctypes.Structure):
    """OomNvfp4Record of include/oom_hip.h: part offsets of an NVFP4 expert record and the
    float indices of its three weight_scale_2 scalars."""

    _fields_ = [(n, ctypes.c_int64) for n in (
        "hidden", "inter", "gate_weight", "gate_scale", "up_weight", "up_scale", "down_weight", "down_scale")] + [
        ("scale2", ctypes.c_int64 * 3)]


def nvfp4_geometry(hidden: int, inter: int) -> Nvfp4Record:
    """The nvfp4-modelopt-g16 record as released (docs/dev/format.md:111-118): a 256-byte
    part of six f32 scalars (weight_scale_2 of gate, up, down at floats 0, 2, 4), then
    gate.weight, gate.weight_scale, up.weight, up.weight_scale, down.weight,
    down.weight_scale, each part 256-byte aligned."""
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


def nvfp4_stride(geo: Nvfp4Record) -> int:
    return (geo.down_scale + geo.hidden * geo.inter // 16 + 4095) // 4096 * 4096


# ---- entry points (torch tensors in, results in the given output tensors) ----------

def workspace_init(ws, stream=None) -> None:
    check(lib().oom_workspace_init(_ptr(ws), ws.numel() * ws.element_size(), _stream(stream)))


def router_topk(logits, ids, weights, k: int, stream=None) -> None:
    T, E = logits.shape
    check(lib().oom_router_topk(_ptr(logits), _ptr(ids), _ptr(weights), T, E, k, _stream(stream)))


def gemv_fp8_workspace_size(T: int, N: int, K: int) -> int:
    return int(lib().oom_gemv_fp8_workspace_size(T, N, K))


def gemv_fp8(x, q, scale, scale_layout: int, y, ws=None, stream=None) -> None:
    T, K = x.shape
    N = q.shape[0]
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().oom_gemv_fp8(_ptr(x), _dtype_code(x), _ptr(q), _ptr(scale), scale_layout, _ptr(y), _dtype_code(y),
                             T, N, K, _ptr(ws), ws_bytes, _stream(stream)))


def moe_gate_up_fp8(recs, off, assign_tok, n_experts: int, x, h, geo: Fp8Record, stream=None) -> None:
    check(lib().oom_moe_gate_up_fp8(_ptr(recs), _ptr(off), _ptr(assign_tok), n_experts, _ptr(x), _dtype_code(x),
                                    _ptr(h), ctypes.byref(geo), _stream(stream)))


def moe_down_fp8(recs, off, n_experts: int, h, y, geo: Fp8Record, stream=None) -> None:
    check(lib().oom_moe_down_fp8(_ptr(recs), _ptr(off), n_experts, _ptr(h), _ptr(y), ctypes.byref(geo),
                                 _stream(stream)))


def moe_gate_up_bf16(recs, off, assign_tok, n_experts: int, x, h, geo: Bf16Record, stream=None) -> None:
    check(lib().oom_moe_gate_up_bf16(_ptr(recs), _ptr(off), _ptr(assign_tok), n_experts, _ptr(x), _dtype_code(x),
                                     _ptr(h), ctypes.byref(geo), _stream(stream)))


def moe_down_bf16(recs, off, n_experts: int, h, y, geo: Bf16Record, stream=None) -> None:
    check(lib().oom_moe_down_bf16(_ptr(recs), _ptr(off), n_experts, _ptr(h), _ptr(y), ctypes.byref(geo),
                                  _stream(stream)))


def moe_combine_slots(y, slot_assign, w, out, stream=None) -> None:
    T, k = w.shape
    H = y.shape[1]
    check(lib().oom_moe_combine_slots(_ptr(y), _ptr(slot_assign), _ptr(w), _ptr(out), _dtype_code(out), T, H, k,
                                      _stream(stream)))


def moe_plan_size(T: int, E: int, k: int) -> int:
    return int(lib().oom_moe_plan_size(T, E, k))


def moe_plan(ids, E: int, all_recs, plan, recs, stream=None) -> None:
    T, k = ids.shape
    check(lib().oom_moe_plan(_ptr(ids), T, E, k, _ptr(all_recs), _ptr(plan), _ptr(recs), _stream(stream)))


def gemv_bf16_workspace_size(T: int, N: int, K: int) -> int:
    return int(lib().oom_gemv_bf16_workspace_size(T, N, K))


def gemv_bf16(x, w, y, ws=None, stream=None) -> None:
    """y[t, n] = sum_k x[t, k] * w[n, k]; w a bf16 tensor [N, K]."""
    T, K = x.shape
    N = w.shape[0]
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    check(lib().oom_gemv_bf16(_ptr(x), _dtype_code(x), _ptr(w), _ptr(y), _dtype_code(y), T, N, K, _ptr(ws), ws_bytes,
                              _stream(stream)))


def moe_combine_shared(routed, shared, gate_logit, out, stream=None) -> None:
    T, H = routed.shape
    check(lib().oom_moe_combine_shared(_ptr(routed), _ptr(shared), _ptr(gate_logit), _ptr(out), _dtype_code(out), T,
                                       H, _stream(stream)))


def moe_layer_decode_fp8_workspace_size(T: int, E: int, k: int, geo: Fp8Record, shared_geo: Fp8Record) -> int:
    return int(lib().oom_moe_layer_decode_fp8_workspace_size(T, E, k, ctypes.byref(geo), ctypes.byref(shared_geo)))


def moe_layer_decode_fp8(x, router_w, all_recs, k: int, geo: Fp8Record, shared_rec, shared_geo: Fp8Record,
                         shared_gate_w, ids, weights, out, ws, stream=None) -> None:
    """One decode MoE layer: router GEMV (bf16 router_w [E, H]), routed experts, shared
    expert (its record address in the device tensor shared_rec [1]) gated by
    sigmoid(x . shared_gate_w)."""
    T = x.shape[0]
    E = router_w.shape[0]
    check(lib().oom_moe_layer_decode_fp8(_ptr(x), _dtype_code(x), _ptr(router_w), _ptr(all_recs), T, E, k,
                                         ctypes.byref(geo), _ptr(shared_rec), ctypes.byref(shared_geo),
                                         _ptr(shared_gate_w), _ptr(ids), _ptr(weights), _ptr(out), _dtype_code(out),
                                         _ptr(ws), ws.numel() * ws.element_size(), _stream(stream)))


def moe_decode_fp8_workspace_size(T: int, E: int, k: int, geo: Fp8Record) -> int:
    return int(lib().oom_moe_decode_fp8_workspace_size(T, E, k, ctypes.byref(geo)))


def moe_decode_fp8(logits, x, all_recs, k: int, geo: Fp8Record, ids, weights, out, ws, stream=None) -> None:
    T, E = logits.shape
    check(lib().oom_moe_decode_fp8(_ptr(logits), _ptr(x), _dtype_code(x), _ptr(all_recs), T, E, k, ctypes.byref(geo),
                                   _ptr(ids), _ptr(weights), _ptr(out), _dtype_code(out), _ptr(ws),
                                   ws.numel() * ws.element_size(), _stream(stream)))


def moe_gate_up_nvfp4(recs, off, assign_tok, n_experts: int, x, h, geo: Nvfp4Record, stream=None) -> None:
    check(lib().oom_moe_gate_up_nvfp4(_ptr(recs), _ptr(off), _ptr(assign_tok), n_experts, _ptr(x), _dtype_code(x),
                                      _ptr(h), ctypes.byref(geo), _stream(stream)))


def moe_down_nvfp4(recs, off, n_experts: int, h, y, geo: Nvfp4Record, stream=None) -> None:
    check(lib().oom_moe_down_nvfp4(_ptr(recs), _ptr(off), n_experts, _ptr(h), _ptr(y), ctypes.byref(geo),
                                   _stream(stream)))


def moe_decode_nvfp4_workspace_size(T: int, E: int, k: int, geo: Nvfp4Record) -> int:
    return int(lib().oom_moe_decode_nvfp4_workspace_size(T, E, k, ctypes.byref(geo)))


def moe_decode_nvfp4(logits, x, all_recs, k: int, geo: Nvfp4Record, ids, weights, out, ws, stream=None) -> None:
    T, E = logits.shape
    check(lib().oom_moe_decode_nvfp4(_ptr(logits), _ptr(x), _dtype_code(x), _ptr(all_recs), T, E, k,
                                     ctypes.byref(geo), _ptr(ids), _ptr(weights), _ptr(out), _dtype_code(out),
                                     _ptr(ws), ws.numel() * ws.element_size(), _stream(stream)))


def attn_decode_workspace_size(kv_len: int, heads: int, kv_heads: int, d: int) -> int:
    return int(lib().oom_attn_decode_workspace_size(kv_len, heads, kv_heads, d))


def attn_decode_paged(q, k_pages, v_pages, page_table, kv_len: int, scale: float, out, ws, stream=None) -> None:
    """q [heads, d]; k_pages / v_pages bf16 [n_pages, kv_heads, page_size, d]; page_table i32."""
    heads, d = q.shape
    n_pages, kv_heads, page_size, _ = k_pages.shape
    check(lib().oom_attn_decode_paged(_ptr(q), _dtype_code(q), _ptr(k_pages), _ptr(v_pages), _ptr(page_table),
                                      n_pages, page_size, kv_len, heads, kv_heads, d, scale, _ptr(out),
                                      _dtype_code(out), _ptr(ws), ws.numel() * ws.element_size(), _stream(stream)))


# ---- Turbo KV cache and the d = 256, G = 12 decode attention ----

def kv_codebooks():
    """The codebook table (numpy f32, 508 levels) of oom_kv_codebooks."""
    import numpy as np

    n = int(lib().oom_kv_codebook_size())
    t = np.empty(n, dtype=np.float32)
    check(lib().oom_kv_codebooks(t.ctypes.data_as(ctypes.c_void_p), n))
    return t


def kv_row_bytes(d: int, bits: int) -> int:
    return int(lib().oom_kv_row_bytes(d, bits))


def kv_rotate(x, inverse: bool, stream=None) -> None:
    d = x.shape[-1]
    check(lib().oom_kv_rotate(_ptr(x), x.numel() // d, d, int(inverse), _stream(stream)))


def kv_append(src, cache, start: int, bits: int, levels, stream=None) -> None:
    """src f32 [t, kv_heads, d] at sequence position `start` of cache (u8 rows [len, kv_heads])."""
    t, kv_heads, d = src.shape
    check(lib().oom_kv_append(_ptr(src), _ptr(cache), start, t, kv_heads, d, bits, _ptr(levels), _stream(stream)))


def kv_read(cache, dst, bits: int, levels, stream=None) -> None:
    """dst f32 [len, kv_heads, d] from the first len * kv_heads rows of cache."""
    ln, kv_heads, d = dst.shape
    check(lib().oom_kv_read(_ptr(cache), _ptr(dst), ln, kv_heads, d, bits, _ptr(levels), _stream(stream)))


def mask_compact(mask, sel, stream=None) -> None:
    check(lib().oom_mask_compact(_ptr(mask), _ptr(sel), mask.numel(), _stream(stream)))


def attn_decode_turbo_workspace_size(heads: int, kv_heads: int, d: int, kv_len: int) -> int:
    return int(lib().oom_attn_decode_turbo_workspace_size(heads, kv_heads, d, kv_len))


def attn_decode_turbo(q, k, v, k_bits: int, v_bits: int, levels, mask, kv_heads: int, kv_len: int, scale: float, out,
                      ws, stream=None) -> None:
    """q f32 [heads, 256]; k / v u8 cache rows [kv_len, kv_heads]; mask u8 [kv_len]; out f32 [heads, 256]."""
    heads, d = q.shape
    check(lib().oom_attn_decode_turbo(_ptr(q), _ptr(k), _ptr(v), k_bits, v_bits, _ptr(levels), _ptr(mask), heads,
                                      kv_heads, d, kv_len, scale, _ptr(out), _ptr(ws), ws.numel() * ws.element_size(),
                                      _stream(stream)))


def quantize_rows_fp8(x, q, scale, stream=None) -> None:
    rows, cols = x.shape
    check(lib().oom_quantize_rows_fp8(_ptr(x), _dtype_code(x), rows, cols, _ptr(q), _ptr(scale), _stream(stream)))


def moe_grouped_gemm_fp8(recs, off, rows, n_experts: int, max_per_expert: int, xq, x_scale, x_group: int, y,
                         N: int, K: int, w_off: int, s_off: int, stream=None) -> None:
    check(lib().oom_moe_grouped_gemm_fp8(_ptr(recs), _ptr(off), _ptr(rows), n_experts, max_per_expert, _ptr(xq),
                                         _ptr(x_scale), x_group, _ptr(y), N, K, w_off, s_off, _stream(stream)))


def moe_prefill_fp8_workspace_size(T: int, E: int, k: int, geo: Fp8Record) -> int:
    return int(lib().oom_moe_prefill_fp8_workspace_size(T, E, k, ctypes.byref(geo)))


def moe_prefill_fp8(logits, x, all_recs, k: int, geo: Fp8Record, ids, weights, out, ws, stream=None,
                    precision: int = EXPERT_EXACT) -> None:
    T, E = logits.shape
    check(lib().oom_moe_prefill_fp8(_ptr(logits), _ptr(x), _dtype_code(x), _ptr(all_recs), T, E, k, ctypes.byref(geo),
                                    precision, _ptr(ids), _ptr(weights), _ptr(out), _dtype_code(out), _ptr(ws),
                                    ws.numel() * ws.element_size(), _stream(stream)))


def moe_tiled_nvfp4(recs, off, rows, n_experts: int, max_per_expert: int, x, y, n: int, k: int, w_off: int,
                    s_off: int, s2_idx: int, precision: int = EXPERT_EXACT, stream=None) -> None:
    """y f32 [A, n] = x[row(a)] . W_e^T for one NVFP4 projection (w_off, s_off, s2_idx)."""
    check(lib().oom_moe_tiled_nvfp4(_ptr(recs), _ptr(off), _ptr(rows), n_experts, max_per_expert, _ptr(x), _ptr(y), n,
                                    k, w_off, s_off, s2_idx, precision, _stream(stream)))


def moe_swiglu_range(g, u, h, start: int, end: int, stream=None) -> None:
    check(lib().oom_moe_swiglu_range(_ptr(g), _ptr(u), _ptr(h), start, end, _stream(stream)))


# ---- copies beside compute: the Transfer trait (crates/oominf-core/src/backend.rs:945-1018) ----

def _handle(x) -> ctypes.c_void_p:
    """A copy queue, a torch stream or None (torch's current stream) as a stream handle."""
    if isinstance(x, CopyQueue):
        return x.handle
    return _stream(x)


class CopyQueue:
    """Transfer::copy_queue: a HIP stream of its own (default priority) for copies."""

    def __init__(self):
        h = ctypes.c_void_p()
        check(lib().oom_copy_queue_create(ctypes.byref(h)))
        self.handle = h

    def copy_to_device(self, dst: int, src: int, nbytes: int) -> None:
        check(lib().oom_copy_to_device(self.handle, dst, ctypes.c_void_p(src), nbytes))

    def copy_on_device(self, dst: int, src: int, nbytes: int) -> None:
        check(lib().oom_copy_on_device(self.handle, dst, src, nbytes))

    def copy_records(self, dst: list[int], src: list[int], nbytes: int) -> None:
        """Records src[i] (pinned host) -> dst[i] (device), nbytes each, in order."""
        n = len(dst)
        d = (ctypes.c_uint64 * n)(*dst)
        s = (ctypes.c_void_p * n)(*src)
        check(lib().oom_copy_records_to_device(self.handle, d, s, nbytes, n))

    def sync(self) -> None:
        check(lib().oom_stream_sync(self.handle))

    def close(self) -> None:
        if self.handle:
            check(lib().oom_copy_queue_destroy(self.handle))
            self.handle = None


class Event:
    """A Transfer event: record on the compute stream or a copy queue, wait on either."""

    def __init__(self):
        h = ctypes.c_void_p()
        check(lib().oom_event_create(ctypes.byref(h)))
        self.handle = h

    def record(self, stream=None) -> None:
        check(lib().oom_event_record(self.handle, _handle(stream)))

    def wait_on(self, stream=None) -> None:
        """Work queued later on `stream` waits for this event (compute_wait / copies_wait)."""
        check(lib().oom_stream_wait_event(_handle(stream), self.handle))

    def done(self) -> bool:
        rc = lib().oom_event_done(self.handle)
        if rc < 0:
            check(rc)
        return rc == 1

    def wait(self) -> None:
        check(lib().oom_event_wait(self.handle))

    def close(self) -> None:
        if self.handle:
            check(lib().oom_event_destroy(self.handle))
            self.handle = None


class PinnedHost:
    """Pinned host memory from oom_host_alloc; `array()` is a numpy view of it."""

    def __init__(self, nbytes: int):
        h = ctypes.c_void_p()
        check(lib().oom_host_alloc(ctypes.byref(h), nbytes))
        self.ptr = int(h.value)
        self.nbytes = nbytes

    def array(self, dtype="uint8"):
        import numpy as np

        buf = (ctypes.c_uint8 * self.nbytes).from_address(self.ptr)
        return np.frombuffer(buf, dtype=np.uint8).view(dtype)

    def close(self) -> None:
        if self.ptr:
            check(lib().oom_host_free(ctypes.c_void_p(self.ptr)))
            self.ptr = 0


def download_async(dst_host: int, src, nbytes: int, stream=None) -> None:
    """Transfer::download_async: after the work queued on `stream`, device src -> pinned host."""
    check(lib().oom_download_async(_handle(stream), ctypes.c_void_p(dst_host), _ptr(src), nbytes))

"""Seeded synthetic inputs for the hot path's configurations (shared by tests and bench).

Weights are drawn from N(0, 0.02) (xorshift64* + Box-Muller, as the reference's
tests draw them: crates/oominf-cuda/tests/kv_cache.rs:10-24), rounded to bf16 and
quantised to e4m3 with fp32 block scales on the host, as the reference's loader
quantises dense FP8 weights (crates/oominf-core/src/fp8.rs:52-88).
Expert e's part p (0 gate, 1 up, 2 down) comes from stream oracle.seed(seed, 3 e + p).
"""
from __future__ import annotations

import numpy as np

import oracle

WEIGHT_STD = 0.02


def expert_record(geo: oracle.Fp8Record, seed: int, e: int, stride: int | None = None) -> np.ndarray:
    """One fp8-e4m3-b128 expert record (uint8, `stride` bytes) of expert e."""
    stride = stride or oracle.record_stride(geo)
    rec = np.zeros(stride, dtype=np.uint8)
    H, I = geo.hidden, geo.inter
    parts = [(geo.gate_weight, geo.gate_scale, I, H), (geo.up_weight, geo.up_scale, I, H),
             (geo.down_weight, geo.down_scale, H, I)]
    for p, (wo, so, n, k) in enumerate(parts):
        w = oracle.gaussian_bf16((n, k), oracle.seed(seed, 3 * e + p), WEIGHT_STD)
        q, s = oracle.quantize(w, oracle.SCALE_128X128)
        rec[wo:wo + n * k] = q.reshape(-1)
        rec[so:so + s.size * 4] = s.view(np.uint8)
    return rec


def expert_records(geo: oracle.Fp8Record, seed: int, E: int, only=None) -> list[np.ndarray]:
    """Records of E experts; experts outside `only` (when given) are left zero."""
    stride = oracle.record_stride(geo)
    return [expert_record(geo, seed, e, stride) if only is None or e in only else np.zeros(stride, np.uint8)
            for e in range(E)]


def constant_record(geo: oracle.Fp8Record, code: int = 0x38, scale: float = 1.0) -> np.ndarray:
    """A record whose every weight is e4m3 `code` and every scale `scale`."""
    rec = np.zeros(oracle.record_stride(geo), dtype=np.uint8)
    H, I = geo.hidden, geo.inter
    for wo, so, n, k in [(geo.gate_weight, geo.gate_scale, I, H), (geo.up_weight, geo.up_scale, I, H),
                         (geo.down_weight, geo.down_scale, H, I)]:
        rec[wo:wo + n * k] = code
        nb = ((n + 127) // 128) * ((k + 127) // 128)
        rec[so:so + nb * 4] = np.full(nb, scale, dtype=np.float32).view(np.uint8)
    return rec


def record_weights(rec: np.ndarray, geo: oracle.Fp8Record):
    """Dequantised (gate [I, H], up [I, H], down [H, I]) fp32 weights of a record,
    decoded with torch's float8_e4m3fn (a library decode independent of the oracle)."""
    import torch

    H, I = geo.hidden, geo.inter
    out = []
    for wo, so, n, k in [(geo.gate_weight, geo.gate_scale, I, H), (geo.up_weight, geo.up_scale, I, H),
                         (geo.down_weight, geo.down_scale, H, I)]:
        q = torch.from_numpy(rec[wo:wo + n * k].copy()).view(torch.float8_e4m3fn).float().numpy().reshape(n, k)
        nb = ((n + 127) // 128) * ((k + 127) // 128)
        s = rec[so:so + nb * 4].view(np.float32).reshape((n + 127) // 128, (k + 127) // 128)
        out.append(q * s[np.arange(n) // 128][:, np.arange(k) // 128])
    return out


def decode_logits(seed: int, T: int, E: int, zipf: float | None = None) -> np.ndarray:
    """Router logits [T, E] from N(0, 1), plus a Zipf(s) popularity bias when given."""
    logits = oracle.gaussian(T * E, oracle.seed(seed, 1 << 40)).reshape(T, E)
    if zipf is not None:
        logits = logits + oracle.zipf_bias(E, zipf, oracle.seed(seed, (1 << 40) + 1))[None, :]
    return np.ascontiguousarray(logits, dtype=np.float32)


def activations_bf16(seed: int, T: int, H: int) -> np.ndarray:
    """x [T, H] bf16 bits from N(0, 1)."""
    return oracle.gaussian_bf16((T, H), oracle.seed(seed, (1 << 40) + 2), 1.0)


def f64_moe(logits_ids_w, x: np.ndarray, recs, geo: oracle.Fp8Record) -> np.ndarray:
    """f64 evaluation of the routed MoE FFN over dequantised weights: per token,
    sum_s w_s down(silu(g) * u) with the given ids and weights."""
    ids, w = logits_ids_w
    T, k = ids.shape
    out = np.zeros((T, geo.hidden))
    cache = {}
    for t in range(T):
        xt = x[t].astype(np.float64)
        for s in range(k):
            e = int(ids[t, s])
            if e not in cache:
                cache[e] = [m.astype(np.float64) for m in record_weights(recs[e], geo)]
            g, u, d = cache[e]
            gv, uv = g @ xt, u @ xt
            h = gv / (1.0 + np.exp(-gv)) * uv
            out[t] += float(w[t, s]) * (d @ h)
    return out


# E2M1 values by code as the reference's tests list them (crates/oominf-cuda/tests/moe_tiled.rs:28-32,
# crates/oominf-metal/src/tests.rs:252-254): the f64 decode below uses this table, not the oracle.
E2M1_F64 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def nvfp4_parts(geo: oracle.Nvfp4Record):
    """(weight offset, scale offset, scale_2 float index, rows, cols) of gate, up, down."""
    H, I = geo.hidden, geo.inter
    return [(geo.gate_weight, geo.gate_scale, geo.scale2[0], I, H), (geo.up_weight, geo.up_scale, geo.scale2[1], I, H),
            (geo.down_weight, geo.down_scale, geo.scale2[2], H, I)]


def nvfp4_record(geo: oracle.Nvfp4Record, seed: int, e: int, stride: int | None = None) -> np.ndarray:
    """One NVFP4 record: random code bytes; scale bytes in [0x28, 0x50), positive and finite
    (about 2^-2 .. 2^2, as crates/oominf-cuda/tests/moe_tiled.rs:58-78 draws them);
    weight_scale_2 in [0.01, 0.03) and input_scale 1 in the scalars part."""
    stride = stride or oracle.nvfp4_stride(geo)
    rng = np.random.default_rng([seed, e, 4])
    rec = np.zeros(stride, dtype=np.uint8)
    scal = np.zeros(64, dtype=np.float32)
    scal[[1, 3, 5]] = 1.0
    for wo, so, s2i, n, k in nvfp4_parts(geo):
        scal[s2i] = 0.01 + 0.02 * rng.random()
        rec[wo:wo + n * k // 2] = rng.integers(0, 256, n * k // 2, dtype=np.uint8)
        rec[so:so + n * k // 16] = rng.integers(0x28, 0x50, n * k // 16, dtype=np.uint8)
    rec[:256] = scal.view(np.uint8)
    return rec


def nvfp4_records(geo: oracle.Nvfp4Record, seed: int, E: int, only=None) -> list[np.ndarray]:
    """Records of E experts; experts outside `only` (when given) are left zero."""
    stride = oracle.nvfp4_stride(geo)
    return [nvfp4_record(geo, seed, e, stride) if only is None or e in only else np.zeros(stride, np.uint8)
            for e in range(E)]


def nvfp4_weights(rec: np.ndarray, geo: oracle.Nvfp4Record):
    """(gate [I, H], up [I, H], down [H, I]) float64 weights of an NVFP4 record:
    e2m1(code) * e4m3(scale) * scale_2 exactly (the reference's f64 test decode,
    moe_tiled.rs:85-95), e4m3 through torch's float8_e4m3fn."""
    import torch

    out = []
    for wo, so, s2i, n, k in nvfp4_parts(geo):
        b = rec[wo:wo + n * k // 2].reshape(n, k // 2)
        codes = np.empty((n, k), dtype=np.uint8)
        codes[:, 0::2] = b & 15
        codes[:, 1::2] = b >> 4
        sc = torch.from_numpy(rec[so:so + n * k // 16].copy()).view(torch.float8_e4m3fn).double().numpy()
        s2 = float(rec[:256].view(np.float32)[s2i])
        out.append(E2M1_F64[codes] * np.repeat(sc.reshape(n, k // 16), 16, axis=1) * s2)
    return out


def f64_moe_nvfp4(ids_w, x: np.ndarray, recs, geo: oracle.Nvfp4Record) -> np.ndarray:
    """f64 evaluation of the routed MoE FFN over NVFP4 records with the given ids and weights."""
    ids, w = ids_w
    T, k = ids.shape
    out = np.zeros((T, geo.hidden))
    cache = {}
    for t in range(T):
        xt = x[t].astype(np.float64)
        for s in range(k):
            e = int(ids[t, s])
            if e not in cache:
                cache[e] = nvfp4_weights(recs[e], geo)
            g, u, d = cache[e]
            gv, uv = g @ xt, u @ xt
            out[t] += float(w[t, s]) * (d @ (gv / (1.0 + np.exp(-gv)) * uv))
    return out


def paged_attention_case(seed, H, Hkv, D, kv_len, page=16, spare_pages=3):
    """q bf16 [H, D]; K and V bf16 [n_pages, Hkv, page, D] with a few pages more than the
    sequence uses; the page table maps logical page i to a seeded random physical page."""
    n_used = (kv_len + page - 1) // page
    n_pages = n_used + spare_pages
    table = oracle.permutation(n_pages, seed)[:n_used].astype(np.int32)
    q = oracle.gaussian_bf16((H, D), oracle.seed(seed, 1))
    k = oracle.gaussian_bf16((n_pages, Hkv, page, D), oracle.seed(seed, 2))
    v = oracle.gaussian_bf16((n_pages, Hkv, page, D), oracle.seed(seed, 3))
    return q, k, v, table


def f64_attention(qf, k, v, table, page, kv_len, H, Hkv, D, scale):
    """softmax(q . k * scale) v in float64 over the kv_len visible keys (q as floats)."""
    G = H // Hkv
    kf = oracle.bf16_to_f32(k).astype(np.float64)
    vf = oracle.bf16_to_f32(v).astype(np.float64)
    j = np.arange(kv_len)
    phys = table[j // page]
    out = np.zeros((H, D))
    for h in range(H):
        K = kf[phys, h // G, j % page]
        V = vf[phys, h // G, j % page]
        s = K @ np.asarray(qf[h], dtype=np.float64) * scale
        p = np.exp(s - s.max())
        out[h] = p @ V / p.sum()
    return out

"""Pins of the oracle's Turbo KV cache, mask_compact and d = 256, G = 12 decode attention
(oracle/turbo.c) against what the reference's tests and the mathematics fix:

* codebooks: the reference's own known answers (Max 1960 levels for 3 and 4 bits,
  crates/oominf-core/src/backend.rs:720-760), ascending order, symmetry, and each level
  the conditional mean of its cell under the exact Gaussian (math.erfc);
* fp16: round to nearest even against numpy's binary16 conversion;
* rotation: the explicit Walsh-Hadamard matrix with the sign hash, in f64, and the inverse;
* rows: every code is the nearest level (brute force, ties to the lower) of the rotated
  coordinate over its block's fp16 RMS; round trips within the reference's distortion
  bounds (crates/oominf-cuda/tests/kv_cache.rs:47-80) on its heavy-tailed rows;
* mask_compact against np.nonzero;
* decode attention against f64 softmax attention over the decoded cache (the rotation
  preserves dot products), and a k8v8 cache against an fp32 one within the reference's
  1e-2 (kv_cache.rs:127-145).
"""
import math

import numpy as np
import pytest

import oracle


def ref_gaussian(n, state):
    """crates/oominf-cuda/tests/kv_cache.rs:10-24: xorshift64* and Box-Muller."""
    out = np.empty(n, dtype=np.float32)
    mask = (1 << 64) - 1
    for i in range(n):
        vals = []
        for _ in range(2):
            state ^= state >> 12
            state ^= (state << 25) & mask
            state ^= state >> 27
            vals.append((((state * 0x2545F4914F6CDD1D) & mask) >> 11) / float(1 << 53) + 0.5 / float(1 << 53))
        u, v = vals
        out[i] = math.sqrt(-2.0 * math.log(u)) * math.cos(2.0 * math.pi * v)
    return out


def heavy_rows(t, kvh, d, seed=11):
    x = np.random.default_rng(seed).standard_normal(t * kvh * d).astype(np.float32)
    x[::37] *= 8.0  # a few large coordinates, as real keys have (kv_cache.rs:52-58)
    return x.reshape(t, kvh, d)


def levels(bits):
    t = oracle.kv_codebooks()
    return t[(1 << bits) - 4:(1 << bits) - 4 + (1 << bits)]


def test_codebooks_known_answers():
    t = oracle.kv_codebooks()
    assert t.size == sum(1 << b for b in range(2, 9))
    known = {2: [0.4528, 1.5104], 3: [0.2451, 0.7560, 1.3440, 2.1520],
             4: [0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6181, 2.0690, 2.7326]}
    for bits, vals in known.items():
        lv, half = levels(bits), 1 << (bits - 1)
        for i, k in enumerate(vals):
            assert abs(lv[half + i] - k) < 2e-3 and abs(lv[half - 1 - i] + k) < 2e-3, (bits, i)
    for bits in range(2, 9):
        lv = levels(bits).astype(np.float64)
        assert np.all(np.diff(lv) > 0)
        np.testing.assert_allclose(lv, -lv[::-1], atol=1e-6)


@pytest.mark.parametrize("bits", [2, 5, 8])
def test_codebooks_are_cell_means(bits):
    # Lloyd-Max fixed point under the exact Gaussian: level i = E[X | X in cell i], the
    # cell edges halfway between levels. The reference iterates with the erfcc
    # approximation (fractional error < 1.2e-7), so the levels sit within ~1e-5 of it.
    lv = levels(bits).astype(np.float64)
    n = lv.size
    pdf = lambda x: math.exp(-0.5 * x * x) / math.sqrt(2 * math.pi) if math.isfinite(x) else 0.0
    tail = lambda x: 0.5 * math.erfc(x / math.sqrt(2))
    for i in range(n):
        a = -math.inf if i == 0 else 0.5 * (lv[i - 1] + lv[i])
        b = math.inf if i == n - 1 else 0.5 * (lv[i] + lv[i + 1])
        mean = (pdf(a) - pdf(b)) / (tail(a) - tail(b))
        assert abs(mean - lv[i]) < 2e-5 * max(1.0, abs(lv[i])), (bits, i, mean, lv[i])


def test_product_codebooks_match_the_oracle():
    import homelab_amd

    np.testing.assert_array_equal(homelab_amd.kv_codebooks(), oracle.kv_codebooks())


def test_f16_round_to_nearest_even():
    rng = np.random.default_rng(3)
    xs = np.concatenate([rng.standard_normal(4000).astype(np.float32) * s for s in (1e-7, 1e-5, 1e-2, 1, 300, 7e4)])
    halfway = np.array([1 + 2 ** -11, 1 + 3 * 2 ** -11, 2 ** -24 * 1.5, 2 ** -25, 65504 + 16, 65520], np.float32)
    for x in np.concatenate([xs, halfway, -halfway, np.array([0.0, -0.0, np.inf, -np.inf], np.float32)]):
        with np.errstate(over="ignore"):  # past 65504 numpy's cast overflows to inf, as RNE does
            h = np.float32(x).astype(np.float16)
        want = int(h.view(np.uint16))
        assert oracle.f16_from_f32(float(x)) == want, x
        assert oracle.f16_to_f32(want) == float(h), x


def sign_hash(d):
    i = np.arange(d, dtype=np.uint64)
    return np.where(((i * np.uint64(2654435761)) & np.uint64(0xFFFFFFFF)) >> np.uint64(31), -1.0, 1.0)


@pytest.mark.parametrize("d", [32, 64, 256])
def test_rotation_is_the_signed_hadamard(d):
    from scipy.linalg import hadamard

    x = np.random.default_rng(d).standard_normal((5, d)).astype(np.float32)
    H = hadamard(d).astype(np.float64)
    s = sign_hash(d)
    want = (x.astype(np.float64) * s) @ H.T / math.sqrt(d)
    y = oracle.kv_rotate(x, inverse=False)
    np.testing.assert_allclose(y, want, atol=1e-5)
    np.testing.assert_allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-5)
    np.testing.assert_allclose(oracle.kv_rotate(y, inverse=True), x, atol=1e-5)


@pytest.mark.parametrize("bits", [2, 3, 4, 6, 8])
@pytest.mark.parametrize("d", [64, 256])
def test_codes_are_nearest_levels(bits, d):
    x = heavy_rows(3, 2, d, seed=bits + d).reshape(-1, d)
    cache = oracle.kv_append(x, bits)
    rb = oracle.kv_row_bytes(d, bits)
    lv = levels(bits)
    y = oracle.kv_rotate(x, inverse=False)  # rotated coordinates (the append's own division is a
    # multiplication here; for d = 64 they may differ in the last bit, so codes are checked
    # against the append's own u with a one-ulp allowance on near-ties)
    sb = ((d // 32) * 2 + 15) & ~15
    for r in range(x.shape[0]):
        row = cache[r * rb:(r + 1) * rb]
        for b in range(d // 32):
            yy = y[r, 32 * b:32 * b + 32].astype(np.float64)
            hs = int(row[2 * b:2 * b + 2].view(np.uint16)[0])
            sc = oracle.f16_to_f32(hs)
            # the scale: fp16 of the block RMS
            rms = math.sqrt(float(np.sum(yy * yy)) / 32.0)
            assert abs(sc - rms) <= 2 ** -10 * rms * 1.01, (r, b)
            words = row[sb + 4 * b * bits:sb + 4 * (b + 1) * bits].view(np.uint32)
            idx = np.zeros(32, dtype=np.int64)
            for j in range(bits):
                idx |= ((words[j] >> np.arange(32, dtype=np.uint32)) & 1).astype(np.int64) << j
            u = yy / sc
            dist = np.abs(u[:, None] - lv[None, :].astype(np.float64))
            best = dist.min(1)
            assert np.all(dist[np.arange(32), idx] <= best + 1e-6 * np.maximum(1, np.abs(u))), (r, b)


@pytest.mark.parametrize("bits,bound", [(2, 0.14), (3, 0.045), (4, 0.013), (5, 0.0035), (6, 0.001), (8, 0.0001)])
def test_round_trip_distortion(bits, bound):
    # kv_cache.rs:47-80: Lloyd-Max distortion of a unit Gaussian 0.1175 (2 bits) ... 4e-5 (8)
    x = heavy_rows(64, 2, 256).reshape(-1, 256)
    back = oracle.kv_read(oracle.kv_append(x, bits), x.shape[0], 256, bits)
    e = float(np.sum((x.astype(np.float64) - back) ** 2) / np.sum(x.astype(np.float64) ** 2))
    assert e < bound, (bits, e)
    assert e > bound / 40, (bits, e)  # the codes do quantise (not a pass-through)


def test_fp32_rows_round_trip_exactly():
    x = heavy_rows(5, 2, 96).reshape(-1, 96)
    np.testing.assert_array_equal(oracle.kv_read(oracle.kv_append(x, 0), x.shape[0], 96, 0), x)


def test_mask_compact():
    rng = np.random.default_rng(1)
    for n in [1, 7, 1000, 65537]:
        m = (rng.random(n) < 0.3).astype(np.uint8)
        m[: min(n, 4)] = 1
        sel = oracle.mask_compact(m)
        pos = np.nonzero(m)[0]
        assert sel[0] == pos.size
        np.testing.assert_array_equal(sel[1:1 + pos.size], pos)


def f64_attention(q, kd, vd, mask, G, scale):
    H, D = q.shape
    out = np.zeros((H, D))
    vis = np.nonzero(mask)[0]
    for h in range(H):
        kk = kd[vis, h // G].astype(np.float64)
        s = kk @ q[h].astype(np.float64) * scale
        p = np.exp(s - s.max())
        out[h] = p @ vd[vis, h // G].astype(np.float64) / p.sum()
    return out


@pytest.mark.parametrize("kb,vb,kv_len,sparse", [(8, 6, 300, False), (0, 0, 200, False), (4, 3, 700, True),
                                                  (8, 6, 5000, True)])
def test_decode_turbo_matches_f64_over_the_decoded_cache(kb, vb, kv_len, sparse):
    H, Hkv, D = 24, 2, 256
    rng = np.random.default_rng(kv_len + kb)
    q = rng.standard_normal((H, D)).astype(np.float32)
    k = heavy_rows(kv_len, Hkv, D, seed=5)
    v = rng.standard_normal((kv_len, Hkv, D)).astype(np.float32)
    kc, vc = oracle.kv_append(k.reshape(-1, D), kb), oracle.kv_append(v.reshape(-1, D), vb)
    kd = oracle.kv_read(kc, kv_len * Hkv, D, kb).reshape(kv_len, Hkv, D)
    vd = oracle.kv_read(vc, kv_len * Hkv, D, vb).reshape(kv_len, Hkv, D)
    mask = np.ones(kv_len, dtype=np.uint8)
    if sparse:  # sinks, recent keys and scattered blocks, as a QSA selection
        mask[:] = 0
        mask[:4] = 1
        mask[-64:] = 1
        for b in rng.choice(kv_len // 16, size=kv_len // 160, replace=False):
            mask[16 * b:16 * b + 16] = 1
    scale = 1.0 / 16.0
    got = oracle.attn_decode_turbo(q, kc, vc, kb, vb, mask, H, Hkv, kv_len, scale)
    want = f64_attention(q, kd, vd, mask, H // Hkv, scale)
    assert np.abs(got - want).max() < 2e-5 * max(1.0, np.abs(want).max()), np.abs(got - want).max()


def test_k8v8_cache_against_fp32_cache():
    # kv_cache.rs:127-145: relative output error of a k8v8 cache below 1e-2
    H, Hkv, D, L = 24, 2, 256, 1024
    q = ref_gaussian(H * D, 3).reshape(H, D)
    k = np.random.default_rng(5).standard_normal((L, Hkv, D)).astype(np.float32)
    v = np.random.default_rng(7).standard_normal((L, Hkv, D)).astype(np.float32)
    mask = np.ones(L, dtype=np.uint8)
    outs = []
    for bits in (0, 8):
        kc, vc = oracle.kv_append(k.reshape(-1, D), bits), oracle.kv_append(v.reshape(-1, D), bits)
        outs.append(oracle.attn_decode_turbo(q, kc, vc, bits, bits, mask, H, Hkv, L, 1.0 / 16.0).astype(np.float64))
    e = math.sqrt(float(np.sum((outs[0] - outs[1]) ** 2) / np.sum(outs[0] ** 2)))
    assert e < 1e-2, e

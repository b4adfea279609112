"""GPU parity of the Turbo KV cache rows, mask_compact and the d = 256, G = 12 decode
attention through the C ABI, against the oracle (oracle/turbo.c, pinned in
tests/test_oracle_turbo.py).

Bars: rotation, appended cache bytes (codes and fp16 scales), decoded rows and the compacted
key list bit-exact; the decode attention within 2e-5 of scale of the oracle's (fp32 with the
oracle's operation order; exp may differ in the last place), and, at the real shape (24 query
heads over 2 KV heads, k8v6), within 2e-5 of f64 attention over the decoded cache.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import torch

    import homelab_amd

    homelab_amd.lib()  # raises if the library is missing: no fallback
    torch.cuda.init()
    return homelab_amd


@pytest.fixture(scope="module")
def levels(hip):
    import torch

    return torch.from_numpy(hip.kv_codebooks()).cuda()


def heavy_rows(t, kvh, d, seed=11):
    x = np.random.default_rng(seed).standard_normal(t * kvh * d).astype(np.float32)
    x[::37] *= 8.0
    return x.reshape(t, kvh, d)


@pytest.mark.parametrize("d", [32, 64, 128, 256])
def test_rotate_bit_exact(hip, d):
    import torch

    print(f"case: kv_rotate d={d}", flush=True)
    x = np.random.default_rng(d).standard_normal((37, d)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    hip.kv_rotate(xd, inverse=False)
    torch.cuda.synchronize()
    y = oracle.kv_rotate(x, inverse=False)
    np.testing.assert_array_equal(xd.cpu().numpy(), y)
    hip.kv_rotate(xd, inverse=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(xd.cpu().numpy(), oracle.kv_rotate(y, inverse=True))


@pytest.mark.parametrize("bits", [0, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("d", [32, 64, 128, 256])
def test_append_and_read_bit_exact(hip, levels, bits, d):
    import torch

    print(f"case: kv_append/kv_read d={d} bits={bits}", flush=True)
    t, kvh, start = 9, 2, 3
    x = heavy_rows(t, kvh, d, seed=bits * 7 + d)
    rb = hip.kv_row_bytes(d, bits)
    assert rb == oracle.kv_row_bytes(d, bits)
    rows = (start + t) * kvh
    cache = torch.zeros(rows * rb, dtype=torch.uint8, device="cuda")
    hip.kv_append(torch.from_numpy(x).cuda(), cache, start, bits, levels)
    torch.cuda.synchronize()
    want = oracle.kv_append(x.reshape(-1, d), bits, np.zeros(rows * rb, dtype=np.uint8), start * kvh)
    np.testing.assert_array_equal(cache.cpu().numpy(), want)
    back = torch.empty((start + t, kvh, d), dtype=torch.float32, device="cuda")
    hip.kv_read(cache, back, bits, levels)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(back.cpu().numpy().reshape(-1, d), oracle.kv_read(want, rows, d, bits))


def test_mask_compact_bit_exact(hip):
    import torch

    rng = np.random.default_rng(2)
    for n in [1, 5, 1023, 1024, 1025, 40000, 131072]:
        print(f"case: mask_compact n={n}", flush=True)
        m = (rng.random(n) < 0.1).astype(np.uint8)
        m[: min(4, n)] = 1
        m[-min(64, n):] = 1
        sel = torch.full((n + 1,), -7, dtype=torch.int32, device="cuda")
        hip.mask_compact(torch.from_numpy(m).cuda(), sel)
        torch.cuda.synchronize()
        want = oracle.mask_compact(m)
        got = sel.cpu().numpy()
        c = int(want[0])
        assert got[0] == c
        np.testing.assert_array_equal(got[1:1 + c], want[1:1 + c])


def qsa_mask(kv_len, rng):
    """Sinks, recent keys and scattered 16-key blocks, about 4096 keys: a QSA-like selection."""
    mask = np.zeros(kv_len, dtype=np.uint8)
    mask[:4] = 1
    mask[-256:] = 1
    nb = kv_len // 16
    for b in rng.choice(nb, size=min(nb, 240), replace=False):
        mask[16 * b:16 * b + 16] = 1
    return mask


CASES = [
    # H, Hkv, kv_len, kb, vb, mask
    (24, 2, 4096, 8, 6, "all"),     # the product's shape: 24 query heads over 2 KV heads, k8v6
    (24, 2, 32768, 8, 6, "qsa"),    # a long context, about 4k keys selected
    (24, 2, 1, 8, 6, "all"),
    (12, 1, 333, 4, 3, "qsa"),
    (12, 1, 65536, 4, 4, "qsa"),    # one KV head over 64k keys: 256 partials, the combine's second load batch
    (24, 2, 777, 0, 0, "all"),      # an fp32 cache
]


@pytest.mark.parametrize("H,Hkv,kv_len,kb,vb,mk", CASES)
def test_decode_turbo_parity(hip, levels, H, Hkv, kv_len, kb, vb, mk):
    import torch

    print(f"case: attn_decode_turbo H={H} Hkv={Hkv} kv_len={kv_len} k{kb}v{vb} mask={mk}", flush=True)
    D = 256
    rng = np.random.default_rng(kv_len + kb)
    q = rng.standard_normal((H, D)).astype(np.float32)
    k = heavy_rows(kv_len, Hkv, D, seed=5)
    v = rng.standard_normal((kv_len, Hkv, D)).astype(np.float32)
    mask = np.ones(kv_len, dtype=np.uint8) if mk == "all" else qsa_mask(kv_len, rng)
    kc = torch.zeros(kv_len * Hkv * hip.kv_row_bytes(D, kb), dtype=torch.uint8, device="cuda")
    vc = torch.zeros(kv_len * Hkv * hip.kv_row_bytes(D, vb), dtype=torch.uint8, device="cuda")
    hip.kv_append(torch.from_numpy(k).cuda(), kc, 0, kb, levels)
    hip.kv_append(torch.from_numpy(v).cuda(), vc, 0, vb, levels)
    out = torch.empty((H, D), dtype=torch.float32, device="cuda")
    ws = torch.zeros(hip.attn_decode_turbo_workspace_size(H, Hkv, D, kv_len), dtype=torch.uint8, device="cuda")
    scale = 1.0 / 16.0
    hip.attn_decode_turbo(torch.from_numpy(q).cuda(), kc, vc, kb, vb, levels, torch.from_numpy(mask).cuda(), Hkv,
                          kv_len, scale, out, ws)
    out2 = torch.empty_like(out)
    hip.attn_decode_turbo(torch.from_numpy(q).cuda(), kc, vc, kb, vb, levels, torch.from_numpy(mask).cuda(), Hkv,
                          kv_len, scale, out2, ws)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert torch.equal(out, out2), "a second call gives other bits"
    kch, vch = kc.cpu().numpy(), vc.cpu().numpy()
    want = oracle.attn_decode_turbo(q, kch, vch, kb, vb, mask, H, Hkv, kv_len, scale)
    mag = max(1.0, float(np.abs(want).max()))
    assert np.abs(got - want).max() < 2e-5 * mag, np.abs(got - want).max()
    if H == 24 and kv_len >= 4096:
        # f64 attention over the decoded cache (the rotation preserves dot products)
        kd = oracle.kv_read(kch, kv_len * Hkv, D, kb).reshape(kv_len, Hkv, D).astype(np.float64)
        vd = oracle.kv_read(vch, kv_len * Hkv, D, vb).reshape(kv_len, Hkv, D).astype(np.float64)
        vis = np.nonzero(mask)[0]
        f64 = np.zeros((H, D))
        for h in range(H):
            s = kd[vis, h // 12] @ q[h].astype(np.float64) * scale
            p = np.exp(s - s.max())
            f64[h] = p @ vd[vis, h // 12] / p.sum()
        assert np.abs(got - f64).max() < 2e-5 * mag, np.abs(got - f64).max()


def test_decode_turbo_rejects_bad_shapes(hip):
    import torch

    q = torch.zeros((16, 256), dtype=torch.float32, device="cuda")
    k = torch.zeros(1024, dtype=torch.uint8, device="cuda")
    m = torch.ones(4, dtype=torch.uint8, device="cuda")
    out = torch.zeros_like(q)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    lv = torch.zeros(508, dtype=torch.float32, device="cuda")
    with pytest.raises(hip.OomError, match="12 query heads"):
        hip.attn_decode_turbo(q, k, k, 8, 6, lv, m, 2, 4, 0.1, out, ws)
    q24 = torch.zeros((24, 256), dtype=torch.float32, device="cuda")
    with pytest.raises(hip.OomError, match="both 0"):
        hip.attn_decode_turbo(q24, k, k, 8, 0, lv, m, 2, 4, 0.1, torch.zeros_like(q24), ws)

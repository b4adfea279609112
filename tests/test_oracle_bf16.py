"""The bf16-record oracle (oracle/bf16rec.c) pinned without the reference: closed forms
with all weights 1.0 (the reference's own known answer for its host experts,
crates/oominf-cpu/src/lib.rs:446-494, restated for bf16 records) and f64 evaluation over
the exactly widened weights, at the bar of crates/oominf-cuda/tests/moe_tiled.rs:174-211
(worst error / sum |x w| < 2e-6). The record layout agrees with the format converter's
bf16 schema (docs/dev/format.md:72-73)."""
import numpy as np
import pytest

import oracle
from homelab_amd import fp8_format as ff


def bf16_records(geo, n, seed, scale=0.02):
    rng = np.random.default_rng(seed)
    stride = oracle.bf16_stride(geo)
    recs = []
    for _ in range(n):
        r = np.zeros(stride, dtype=np.uint8)
        for off, shape in [(geo.gate_weight, (geo.inter, geo.hidden)), (geo.up_weight, (geo.inter, geo.hidden)),
                           (geo.down_weight, (geo.hidden, geo.inter))]:
            w = oracle.bf16_from_f32((rng.standard_normal(shape) * scale).astype(np.float32))
            r[off:off + w.nbytes] = w.reshape(-1).view(np.uint8)
        recs.append(r)
    return recs


def widened(rec, off, shape):
    n = int(np.prod(shape))
    return oracle.bf16_to_f32(rec[off:off + 2 * n].view(np.uint16)).reshape(shape).astype(np.float64)


def test_geometry_matches_the_format_schema():
    for h, i in [(4096, 1536), (2560, 640), (64, 40)]:
        geo = oracle.bf16_geometry(h, i)
        schema = ff.record_schema(ff.LAYOUT_BF16, [("gate.weight", "BF16", [i, h]), ("up.weight", "BF16", [i, h]),
                                                   ("down.weight", "BF16", [h, i])])
        o = {p["name"]: p["offset"] for p in schema["parts"]}
        assert (geo.gate_weight, geo.up_weight, geo.down_weight) == (o["gate.weight"], o["up.weight"], o["down.weight"])
        assert oracle.bf16_stride(geo) == schema["stride"]


def test_all_ones_closed_form():
    H, I = 256, 64
    geo = oracle.bf16_geometry(H, I)
    rec = np.zeros(oracle.bf16_stride(geo), dtype=np.uint8)
    ones = np.full(H * I, 0x3F80, dtype=np.uint16).view(np.uint8)
    for off in (geo.gate_weight, geo.up_weight, geo.down_weight):
        rec[off:off + ones.size] = ones
    x = (np.arange(2 * H, dtype=np.float32).reshape(2, H) % 7 - 3) / 8  # exact sums
    off = np.array([0, 2], dtype=np.int32)
    tok = np.array([1, 0], dtype=np.int32)
    h = oracle.moe_gate_up_bf16([rec], off, tok, x, geo)
    for a, t in enumerate(tok):
        s = np.float32(x[t].astype(np.float64).sum())
        want = np.float32(s / (1 + np.exp(-np.float64(s)))) * s
        np.testing.assert_allclose(h[a], np.full(I, want, dtype=np.float32), rtol=2e-7)
    y = oracle.moe_down_bf16([rec], off, h, geo)
    np.testing.assert_allclose(y, np.repeat(h.astype(np.float64).sum(1, keepdims=True), H, 1), rtol=1e-6)


@pytest.mark.parametrize("H,I,E,A", [(512, 256, 3, 7), (4096, 1536, 1, 2), (104, 48, 2, 3)])
def test_matches_f64(H, I, E, A):
    geo = oracle.bf16_geometry(H, I)
    recs = bf16_records(geo, E, H + I)
    rng = np.random.default_rng(A)
    T = 4
    x = rng.standard_normal((T, H)).astype(np.float32)
    cuts = np.sort(rng.integers(0, A + 1, E - 1))
    off = np.concatenate([[0], cuts, [A]]).astype(np.int32)
    tok = rng.integers(0, T, A).astype(np.int32)
    h = oracle.moe_gate_up_bf16(recs, off, tok, x, geo)
    y = oracle.moe_down_bf16(recs, off, h, geo)
    for e in range(E):
        Wg = widened(recs[e], geo.gate_weight, (I, H))
        Wu = widened(recs[e], geo.up_weight, (I, H))
        Wd = widened(recs[e], geo.down_weight, (H, I))
        for a in range(off[e], off[e + 1]):
            xt = x[tok[a]].astype(np.float64)
            g, u = Wg @ xt, Wu @ xt
            assert np.abs(h[a] - (g / (1 + np.exp(-g))) * u).max() < 2e-6 * (np.abs(Wg) @ np.abs(xt)).max() * 4
            yd = Wd @ h[a].astype(np.float64)
            assert np.abs(y[a] - yd).max() <= 2e-6 * (np.abs(Wd) @ np.abs(h[a].astype(np.float64))).max()

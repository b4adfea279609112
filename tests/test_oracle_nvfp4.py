"""Pins of the oracle's NVFP4 (nvfp4-modelopt-g16) restatement, independently of itself:

* the E2M1 value of every code against the table the reference's tests list;
* the reference's own known-answer case (crates/oominf-metal/src/tests.rs:239-270, in
  tests/golden/known_answers.json) at its tolerance;
* the record geometry against the sizes docs/dev/format.md:120-121 states for the
  released model (hidden 2560, inter 640);
* the nibble order (low nibble = even column) and the scale-group index on records built by
  hand, with closed-form outputs;
* gate/up, down and the whole decode step against a float64 evaluation of the exact
  decode (the reference's f64 test oracle, crates/oominf-cuda/tests/moe_tiled.rs:85-95),
  within 1e-5 of sum |x . w| per output (fp32 serial summation against exact products).
"""
import json
import os

import numpy as np
import pytest

import oracle
import synth

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


def test_e2m1_values_match_the_reference_table():
    ka = GOLDEN["nvfp4_rows_known_answer"]
    got = [oracle.e2m1_to_f32(c) for c in range(16)]
    assert got == ka["e2m1"]
    # sign bit: code 8 is -0.0
    assert np.signbit(np.float32(oracle.e2m1_to_f32(8)))


def test_nvfp4_rows_known_answer():
    ka = GOLDEN["nvfp4_rows_known_answer"]
    T, R, C = ka["tokens"], ka["rows"], ka["cols"]
    x = np.array(ka["x"], dtype=np.float32).reshape(T, C)
    packed = np.array(ka["packed"], dtype=np.uint8).reshape(R, C // 2)
    scales = np.array(ka["scales"], dtype=np.uint8).reshape(R, C // 16)
    y = oracle.nvfp4_rows(packed, scales, ka["scale2"], x)
    want = np.array(ka["y"]).reshape(T, R)
    assert np.abs(y - want).max() < ka["tol"]
    # the scale bytes decode to the values the test states
    assert [oracle.e4m3_to_f32(b) for b in ka["scales"]] == ka["scale_values"]


def test_geometry_matches_the_released_record():
    g = oracle.nvfp4_geometry(2560, 640)
    assert oracle.nvfp4_size(g) == 256 + 3 * 819_200 + 3 * 102_400 == 2_765_056
    assert oracle.nvfp4_stride(g) == 2_768_896
    assert list(g.scale2) == [0, 2, 4]
    offs = [g.gate_weight, g.gate_scale, g.up_weight, g.up_scale, g.down_weight, g.down_scale]
    assert offs == sorted(offs) and all(o % 256 == 0 for o in offs)


def test_nibble_order_and_scale_groups_closed_form():
    """Byte 0x71 everywhere: even columns code 1 (0.5), odd columns code 7 (6.0); scale
    bytes 0x38 (1.0) for the first 16 columns and 0x40 (2.0) for the next 16; s2 = 0.5:
    y = 0.5 * (0.5 sum x_even[0:16] + 6 sum x_odd[0:16] + 2 (0.5 sum x_even[16:32] + 6 sum x_odd[16:32]))."""
    C = 32
    x = (np.arange(2 * C, dtype=np.float32).reshape(2, C) % 5) - 2.0
    packed = np.full((1, C // 2), 0x71, dtype=np.uint8)
    scales = np.array([[0x38, 0x40]], dtype=np.uint8)
    y = oracle.nvfp4_rows(packed, scales, 0.5, x)
    for t in range(2):
        a, b = x[t, :16], x[t, 16:]
        want = 0.5 * (0.5 * a[0::2].sum() + 6 * a[1::2].sum() + 2 * (0.5 * b[0::2].sum() + 6 * b[1::2].sum()))
        assert y[t, 0] == np.float32(want)


def _case(H, I, E, seed):
    geo = oracle.nvfp4_geometry(H, I)
    recs = synth.nvfp4_records(geo, seed, E)
    return geo, recs


@pytest.mark.parametrize("H,I,T", [(256, 128, 3), (1040, 432, 2), (2560, 640, 1)])
def test_gate_up_and_down_match_f64(H, I, T):
    geo, recs = _case(H, I, 2, 70 + H)
    x = oracle.bf16_to_f32(synth.activations_bf16(71, T, H))
    off = np.array([0, T, 2 * T], dtype=np.int32)
    tok = np.concatenate([np.arange(T), np.arange(T)[::-1]]).astype(np.int32)
    h = oracle.moe_gate_up_nvfp4(recs, off, tok, x, geo)
    y = oracle.moe_down_nvfp4(recs, off, h, geo)
    for i in range(2):
        g, u, d = synth.nvfp4_weights(recs[i], geo)
        for a in range(off[i], off[i + 1]):
            xt = x[tok[a]].astype(np.float64)
            gv, uv = g @ xt, u @ xt
            bound_g, bound_u = np.abs(g) @ np.abs(xt), np.abs(u) @ np.abs(xt)
            hv = gv / (1 + np.exp(-gv)) * uv
            # h's error bound carried through silu(g) * u (|d/dg| <= 1.1 |u|, |d/du| <= |g|)
            assert np.all(np.abs(h[a] - hv) <= 1e-5 * (1.1 * np.abs(uv) * bound_g + np.abs(gv) * bound_u) + 1e-12)
            hd = h[a].astype(np.float64)
            assert np.all(np.abs(y[a] - d @ hd) <= 1e-5 * (np.abs(d) @ np.abs(hd)) + 1e-12)


@pytest.mark.parametrize("T,E,k,H,I", [(1, 32, 10, 512, 128), (4, 16, 4, 1040, 432)])
def test_decode_matches_f64(T, E, k, H, I):
    geo, recs = _case(H, I, E, 80 + T)
    logits = synth.decode_logits(81 + T, T, E)
    x = oracle.bf16_to_f32(synth.activations_bf16(82, T, H))
    ids, w, out = oracle.moe_decode_nvfp4(logits, x, recs, k, geo)
    want_ids, want_w = oracle.router_topk(logits, k)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_array_equal(w, want_w)
    f64 = synth.f64_moe_nvfp4((ids, w), x, recs, geo)
    assert np.abs(out - f64).max() <= 2e-5 * np.abs(f64).max()

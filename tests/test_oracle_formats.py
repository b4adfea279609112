"""Pins the oracle's number formats and quantisers (CPU).

Each check is independent of the oracle's own code: the reference's known answers
(tests/golden/known_answers.json), torch's float8_e4m3fn / bfloat16 conversions,
and brute force over the 254 finite e4m3 values.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import oracle

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))

FINITE = [b for b in range(256) if b & 0x7F != 0x7F]


def torch_e4m3(codes):
    return torch.tensor(codes, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()


def test_encode_known_answers():
    for x, want in GOLD["e4m3_encode"]["cases"]:
        assert oracle.e4m3_from_f32(x) == want, (x, want)


def test_decode_known_answers():
    for b, want in GOLD["e4m3_decode"]["cases"]:
        got = oracle.e4m3_to_f32(b)
        if want is None:
            assert math.isnan(got)
        else:
            assert got == want


def test_decode_all_codes_match_torch_and_golden():
    ours = np.array([oracle.e4m3_to_f32(b) for b in range(256)], dtype=np.float32)
    theirs = torch_e4m3(list(range(256)))
    gold = np.array([np.nan if v is None else v for v in GOLD["e4m3_all_codes"]["values"]], dtype=np.float32)
    np.testing.assert_array_equal(ours, theirs)
    np.testing.assert_array_equal(ours, gold)


def test_every_finite_code_round_trips():
    # crates/oominf-core/src/fp8.rs:94-108
    for b in FINITE:
        v = oracle.e4m3_to_f32(b)
        back = oracle.e4m3_from_f32(v)
        assert back == b or (v == 0.0 and back & 0x7F == 0), (hex(b), v, hex(back))


def brute_force_e4m3(x: float) -> int:
    """Nearest finite e4m3 code by exhaustive search, ties to the even code,
    saturating at +-448 (fp8.rs:4-9)."""
    if math.isnan(x) or abs(x) >= 448.0:
        return (0x80 if math.copysign(1.0, x) < 0 else 0) | 0x7E
    sign = 0x80 if math.copysign(1.0, x) < 0 else 0
    a = abs(x)
    best, bd = None, None
    for b in range(0x7F):  # non-negative finite codes 0x00..0x7e
        d = abs(oracle.e4m3_to_f32(b) - a)
        if bd is None or d < bd or (d == bd and b % 2 == 0 and best % 2 == 1):
            best, bd = b, d
    return sign | best


def test_encode_matches_brute_force_and_torch():
    rng = np.random.default_rng(1)
    # every midpoint between neighbouring codes (the ties), their neighbours, and a sweep
    vals = [oracle.e4m3_to_f32(b) for b in range(0x7F)]
    mids = [(vals[i] + vals[i + 1]) / 2 for i in range(len(vals) - 1)]
    xs = list(mids) + [np.nextafter(np.float32(m), np.float32(0)) for m in mids] + \
        [np.nextafter(np.float32(m), np.float32(1e9)) for m in mids]
    xs += list(np.exp(rng.uniform(np.log(1e-4), np.log(500.0), 4000)).astype(np.float32))
    xs = np.array(xs, dtype=np.float32)
    xs = np.concatenate([xs, -xs])
    ours = np.array([oracle.e4m3_from_f32(float(v)) for v in xs], dtype=np.uint8)
    brute = np.array([brute_force_e4m3(float(v)) for v in xs], dtype=np.uint8)
    np.testing.assert_array_equal(ours, brute)
    # torch rounds to nearest even too; it does not saturate, so compare below 448
    inside = np.abs(xs) < 448.0
    theirs = torch.from_numpy(xs[inside]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    ours_in = ours[inside].copy()
    zero = (oracle_decode := np.array([oracle.e4m3_to_f32(b) for b in ours_in])) == 0.0
    np.testing.assert_array_equal(ours_in[~zero], theirs[~zero])
    assert np.all(torch_e4m3(list(theirs[zero])) == 0.0) and np.all(oracle_decode[zero] == 0.0)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(2)
    v = np.concatenate([rng.standard_normal(10000), rng.standard_normal(1000) * 1e-30]).astype(np.float32)
    ours = oracle.bf16_from_f32(v)
    theirs = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)
    np.testing.assert_array_equal(oracle.bf16_to_f32(ours), torch.from_numpy(v).to(torch.bfloat16).float().numpy())


def test_quantize_blocks_reference_example():
    g = GOLD["quantize_blocks"]
    w = np.zeros((g["n"], g["k"]), dtype=np.float32)
    for r, c, v in g["nonzero"]:
        w[r, c] = v
    q, s = oracle.quantize(oracle.bf16_from_f32(w), oracle.SCALE_1X128)
    np.testing.assert_array_equal(s, np.array(g["scales"], dtype=np.float32))
    for r, c, v in g["decoded"]:
        assert oracle.e4m3_to_f32(q[r, c]) * s[r * 2 + c // 128] == v
    assert np.all(q[1] == 0)


@pytest.mark.parametrize("layout", [oracle.SCALE_ROW, oracle.SCALE_1X128, oracle.SCALE_128X128])
def test_quantize_block_invariants(layout):
    n, k = 300, 520  # partial blocks on both axes
    w = oracle.gaussian_bf16((n, k), 7, 0.02)
    wf = oracle.bf16_to_f32(w)
    wf[5, :] = 0.0  # an all-zero row (scale 1 in the row layouts)
    w = oracle.bf16_from_f32(wf)
    q, s = oracle.quantize(w, layout)
    deq = oracle.dequantize(q, s, layout)
    # the block absmax lands exactly on +-448 * scale; every other weight rounds to its
    # nearest code: at most half a code step of w / scale (2^-4 relative for normals,
    # 2^-10 absolute for subnormals), times the scale
    scale_of = oracle.dequantize(np.full_like(q, 0x38), s, layout)  # code 0x38 is 1.0
    err = np.abs(deq - wf)
    bound = np.maximum(np.abs(wf) * 2.0 ** -4, 2.0 ** -10 * scale_of) * (1 + 1e-6)
    assert np.all(err <= bound)
    assert np.abs(oracle.e4m3_decode(q)).max() == 448.0
    if layout == oracle.SCALE_ROW:
        assert s[5] == 1.0
        assert np.all(np.abs(oracle.e4m3_decode(q[np.arange(n) != 5])).max(axis=1) == 448.0)
    # quantisation error of N(0, 0.02) weights: e4m3's few percent (gemv.rs:144-154 gate < 0.05)
    rel = np.sqrt(((deq - wf) ** 2).sum() / (wf ** 2).sum())
    assert rel < 0.05


def test_activation_quantiser_per_row():
    x = oracle.gaussian(8 * 512, 3).reshape(8, 512)
    q, s = oracle.quantize_act(x)
    np.testing.assert_array_equal(s, np.abs(x).max(axis=1) / np.float32(448.0))
    deq = oracle.e4m3_decode(q) * s[:, None]
    assert np.all(np.abs(deq - x) <= np.maximum(np.abs(x) * 2.0 ** -4, 2.0 ** -10 * s[:, None]))
    qg, sg = oracle.quantize_act(x, 128)
    assert sg.shape == (8, 4)
    np.testing.assert_array_equal(sg, np.abs(x.reshape(8, 4, 128)).max(axis=2) / np.float32(448.0))


def test_gaussian_stream_moments_and_determinism():
    a = oracle.gaussian(200000, 11)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    np.testing.assert_array_equal(a, oracle.gaussian(200000, 11))
    # chunked bf16 generation is independent of the thread count
    b1 = oracle.gaussian_bf16((1000, 700), 5, 0.02, chunk=4096, threads=1)
    b8 = oracle.gaussian_bf16((1000, 700), 5, 0.02, chunk=4096, threads=8)
    np.testing.assert_array_equal(b1, b8)
    assert abs(oracle.bf16_to_f32(b1).std() - 0.02) < 0.001


def test_zipf_bias_is_a_log_distribution():
    b = oracle.zipf_bias(128, 1.1, 9)
    p = np.exp(b.astype(np.float64))
    assert abs(p.sum() - 1.0) < 1e-5
    ranks = np.argsort(-p)
    r = np.arange(1, 129, dtype=np.float64)
    np.testing.assert_allclose(p[ranks], r ** -1.1 / (r ** -1.1).sum(), rtol=1e-5)

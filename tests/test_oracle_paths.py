"""Pins the oracle's router, GEMV, routed experts, grouped GEMM, attention and the
restated CPU path (CPU).

Checks are independent of the oracle's code: float64 numpy evaluations over weights
decoded by torch's float8_e4m3fn, brute force, closed forms from the reference's
tests and invariants (each cites its source).
"""
import json
import os

import numpy as np
import pytest

import oracle
import synth

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


# ---- router ------------------------------------------------------------------------

def f64_topk(logits: np.ndarray, k: int):
    """Brute force in float64: softmax, sort by (-p, id), renormalise over the picks."""
    l = logits.astype(np.float64)
    p = np.exp(l - l.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.array([sorted(range(l.shape[1]), key=lambda e: (-p[t, e], e))[:k] for t in range(l.shape[0])])
    w = np.take_along_axis(p, ids, 1)
    return ids, w / w.sum(axis=1, keepdims=True), p


def margin_ok(p, k):
    """No near-tie between the k-th and (k+1)-th probability (else ids are fragile)."""
    s = -np.sort(-p, axis=1)
    return np.all((s[:, k - 1] - s[:, k]) / s[:, k - 1] > 1e-5)


@pytest.mark.parametrize("T,E,k,zipf", [(1, 128, 8, None), (16, 128, 8, 1.1), (64, 128, 8, 1.1), (3, 300, 5, None),
                                        (2, 8192, 32, None)])
def test_router_matches_f64_brute_force(T, E, k, zipf):
    logits = synth.decode_logits(100 + T + E, T, E, zipf)
    ids, w = oracle.router_topk(logits, k)
    want_ids, want_w, p = f64_topk(logits, k)
    assert margin_ok(p, k)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_allclose(w, want_w, rtol=2e-6)
    pf = oracle.router_probs(logits)
    np.testing.assert_allclose(pf, p, rtol=2e-6, atol=1e-12)


def test_router_ties_go_to_the_lower_id():
    # equal logits give equal probabilities: picks in id order (ops.cu:262, backend.rs:814)
    logits = np.zeros((2, 64), dtype=np.float32)
    logits[1, [7, 3, 50, 20]] = 2.0
    ids, w = oracle.router_topk(logits, 6)
    assert ids[0].tolist() == [0, 1, 2, 3, 4, 5]
    assert ids[1].tolist() == [3, 7, 20, 50, 0, 1]
    np.testing.assert_allclose(w[0], np.full(6, 1 / 6), rtol=1e-6)


# ---- dense FP8 GEMV ---------------------------------------------------------------

def test_gemv_reference_partial_scale_blocks():
    g = GOLD["fp8_gemv_partial_blocks"]
    x = np.array([g["x"]], dtype=np.float32)
    q = np.array(g["q"], dtype=np.uint8).reshape(g["n"], g["k"])
    y = oracle.gemv_fp8(x, q, np.array(g["scale_1x128"], dtype=np.float32), oracle.SCALE_1X128)
    np.testing.assert_allclose(y[0], g["y"], atol=g["tol"], rtol=0)


def test_gemv_reads_every_code():
    vals = np.array([np.nan if v is None else v for v in GOLD["e4m3_all_codes"]["values"]], dtype=np.float32)
    y = oracle.gemv_fp8(np.ones((1, 1), np.float32), np.arange(256, dtype=np.uint8).reshape(256, 1),
                        np.ones(256, np.float32), oracle.SCALE_ROW)
    np.testing.assert_array_equal(y[0], vals)


@pytest.mark.parametrize("layout", [oracle.SCALE_ROW, oracle.SCALE_1X128, oracle.SCALE_128X128])
@pytest.mark.parametrize("T,N,K", [(1, 300, 1024), (4, 256, 2560), (16, 130, 640)])
def test_gemv_matches_f64(layout, T, N, K):
    # crates/oominf-cuda/tests/gemv.rs:126-186: f64 over the dequantised weights,
    # max |got - want| / sqrt(K) < 1e-5
    w = oracle.gaussian_bf16((N, K), 9, 0.02)
    q, s = oracle.quantize(w, layout)
    x = oracle.bf16_to_f32(synth.activations_bf16(T, T, K))
    y = oracle.gemv_fp8(x, q, s, layout)
    import torch
    deq = torch.from_numpy(q).view(torch.float8_e4m3fn).double().numpy()
    nkb = (K + 127) // 128
    if layout == oracle.SCALE_ROW:
        sc = np.repeat(s[:, None], K, 1)
    elif layout == oracle.SCALE_1X128:
        sc = s.reshape(N, nkb)[:, np.arange(K) // 128]
    else:
        sc = s.reshape((N + 127) // 128, nkb)[np.arange(N) // 128][:, np.arange(K) // 128]
    want = x.astype(np.float64) @ (deq * sc).T
    assert np.abs(y - want).max() / np.sqrt(K) < 1e-5


# ---- routed experts ---------------------------------------------------------------

def test_plan_groups_slots_by_expert():
    ids = np.array([[5, 2, 9], [2, 7, 5], [9, 5, 1]], dtype=np.int32)
    experts, off, tok, slot = oracle.moe_plan(ids, 10)
    assert experts.tolist() == [1, 2, 5, 7, 9]
    assert off.tolist() == [0, 1, 3, 6, 7, 9]
    assert tok.tolist() == [2, 0, 1, 0, 1, 2, 1, 0, 2]
    # slot_assign inverts the grouping: assignment a of slot s belongs to token s // k
    flat = ids.reshape(-1)
    for s_, a in enumerate(slot):
        assert tok[a] == s_ // 3
        e_idx = np.searchsorted(off, a, side="right") - 1
        assert experts[e_idx] == flat[s_]
    with pytest.raises(ValueError):
        oracle.moe_plan(np.array([[1, 10]], dtype=np.int32), 10)


def test_expert_known_record_closed_form():
    # crates/oominf-cpu/src/lib.rs:446-494 restated for e4m3: every weight code 0x38
    # (1.0) with scale 1: gate = up = sum(x), output = silu(s) * s * inter.
    g = GOLD["expert_known_record"]
    geo = oracle.record_geometry(g["hidden"], g["inter"])
    rec = synth.constant_record(geo)
    x = np.array(g["x"], dtype=np.float32).reshape(2, g["hidden"])
    off = np.array([0, 2], dtype=np.int32)
    tok = np.array(g["tokens"], dtype=np.int32)
    h = oracle.moe_gate_up([rec], off, tok, x, geo)
    y = oracle.moe_down([rec], off, h, geo)
    for i, want in enumerate(g["y_per_token"]):
        np.testing.assert_allclose(y[i], want, rtol=g["rtol"])
    yh = oracle.host_experts(geo, [rec], [g["tokens"]], x, threads=2)
    for i, want in enumerate(g["y_per_token"]):
        np.testing.assert_allclose(yh[i], want, rtol=g["rtol"])


def small_moe(seed=3, H=256, I=128, E=16):
    geo = oracle.record_geometry(H, I)
    return geo, synth.expert_records(geo, seed, E)


def test_decode_matches_f64():
    # moe_tiled.rs:174-211 gate: worst |got - want| / sum |terms| < 2e-6 per stage; here
    # on the whole FFN against the f64 evaluation, relative to the output scale.
    geo, recs = small_moe()
    T, E, k = 5, 16, 4
    logits = synth.decode_logits(7, T, E)
    x = oracle.bf16_to_f32(synth.activations_bf16(7, T, geo.hidden))
    ids, w, out = oracle.moe_decode(logits, x, recs, k, geo)
    want = synth.f64_moe((ids, w), x, recs, geo)
    assert np.abs(out - want).max() <= 1e-5 * np.abs(want).max()
    want_ids, _, _ = f64_topk(logits, k)
    np.testing.assert_array_equal(ids, want_ids)


def test_combine_slots_in_slot_order():
    y = oracle.gaussian(6 * 8, 5).reshape(6, 8)
    slot = np.array([4, 1, 0, 5, 3, 2], dtype=np.int32)
    w = np.array([[0.5, 0.25, 0.25], [0.1, 0.2, 0.7]], dtype=np.float32)
    out = oracle.moe_combine_slots(y, slot, w)
    want = np.stack([w[t] @ y[slot[t * 3:(t + 1) * 3]].astype(np.float64) for t in range(2)])
    np.testing.assert_allclose(out, want, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("nt", [1, 3, 4, 5, 16, 17, 37])
def test_host_experts_match_oracle(nt):
    # the CPU path equals the per-stage oracle to fp32 summation accuracy, on both its
    # vector (<= 4 tokens) and GEMM paths (lib.rs:496-561)
    geo, recs = small_moe(E=3)
    x = oracle.bf16_to_f32(synth.activations_bf16(11, 40, geo.hidden))
    jobs = [[(i * 31 + 7) % 40 for i in range(nt)], [3, 1], list(range(nt))]
    y = oracle.host_experts(geo, recs, jobs, x, threads=4)
    off = np.cumsum([0] + [len(j) for j in jobs]).astype(np.int32)
    tok = np.concatenate([np.array(j, np.int32) for j in jobs])
    h = oracle.moe_gate_up(recs, off, tok, x, geo)
    want = oracle.moe_down(recs, off, h, geo)
    scale = np.abs(want).max()
    assert np.abs(y - want).max() <= 1e-4 * scale


# ---- prefill grouped GEMM -----------------------------------------------------------

def test_grouped_gemm_matches_f64():
    # moe_tiled.rs:213-223: partial tiles, an empty expert, both projection shapes;
    # gate worst / sum |x w| < 2e-6 (products of two e4m3 are exact in fp32)
    import torch
    for (N, K, counts) in [(200, 256, [1, 0, 37, 70]), (384, 640, [3, 33, 64])]:
        geo_w = []
        recs = []
        for e, _ in enumerate(counts):
            w = oracle.gaussian_bf16((N, K), oracle.seed(5, e), 0.02)
            q, s = oracle.quantize(w, oracle.SCALE_128X128)
            rec = np.concatenate([q.reshape(-1), s.view(np.uint8)])
            recs.append(rec)
            geo_w.append((torch.from_numpy(q).view(torch.float8_e4m3fn).double().numpy(), s))
        off = np.cumsum([0] + counts).astype(np.int32)
        tokens = 64
        x = oracle.gaussian(tokens * K, 8).reshape(tokens, K) * 2
        xq, xs = oracle.quantize_act(x)
        rows = np.array([(a * 13 + 5) % tokens for a in range(off[-1])], dtype=np.int32)
        y = oracle.grouped_gemm_fp8(recs, off, rows, xq, xs, 0, N, K, 0, N * K)
        xd = torch.from_numpy(xq).view(torch.float8_e4m3fn).double().numpy() * xs[:, None].astype(np.float64)
        worst = 0.0
        for e in range(len(counts)):
            dq, s = geo_w[e]
            nkb = (K + 127) // 128
            W = dq * s.reshape((N + 127) // 128, nkb)[np.arange(N) // 128][:, np.arange(K) // 128]
            for a in range(off[e], off[e + 1]):
                terms = xd[rows[a]][None, :] * W
                want = terms.sum(1)
                worst = max(worst, (np.abs(y[a] - want) / np.abs(terms).sum(1)).max())
        assert worst < 2e-6


def test_prefill_matches_decode_semantics_within_quantisation():
    # the prefill pipeline quantises activations to e4m3; it must agree with the exact
    # decode path to e4m3 activation precision (a few percent of the output scale)
    geo, recs = small_moe()
    T, E, k = 12, 16, 4
    logits = synth.decode_logits(9, T, E)
    x = oracle.bf16_to_f32(synth.activations_bf16(9, T, geo.hidden))
    ids_p, w_p, out_p = oracle.moe_prefill(logits, x, recs, k, geo)
    ids_d, w_d, out_d = oracle.moe_decode(logits, x, recs, k, geo)
    np.testing.assert_array_equal(ids_p, ids_d)
    rel = np.linalg.norm(out_p - out_d) / np.linalg.norm(out_d)
    assert rel < 0.06


def test_prefill_is_decode_over_dequantised_activations():
    # with h kept in fp32, the prefill oracle is the decode oracle (pinned against f64 and
    # the closed-form record) applied to the per-token e4m3 activations xs * e4m3(xq): the
    # only difference is where xs multiplies (after each gate/up sum instead of into every
    # activation), a few fp32 roundings; a dropped term, a wrong scale or a quantised h
    # would move it by orders of magnitude more
    geo, recs = small_moe()
    T, E, k = 12, 16, 4
    logits = synth.decode_logits(19, T, E)
    x = oracle.bf16_to_f32(synth.activations_bf16(19, T, geo.hidden))
    xq, xs = oracle.quantize_act(x)
    xd = (oracle.e4m3_decode(xq).astype(np.float64) * xs[:, None]).astype(np.float32)
    ids_p, w_p, out_p = oracle.moe_prefill(logits, x, recs, k, geo)
    ids_d, w_d, out_d = oracle.moe_decode(logits, xd, recs, k, geo)
    np.testing.assert_array_equal(ids_p, ids_d)
    err = np.abs(out_p - out_d).max()
    assert err <= 2e-6 * np.abs(out_d).max(), err


# ---- paged decode attention -----------------------------------------------------------

def paged_case(seed, H, Hkv, D, kv_len, page=16):
    n_pages = (kv_len + page - 1) // page
    perm = oracle.permutation(n_pages, seed)
    q = oracle.gaussian_bf16((H, D), oracle.seed(seed, 1))
    k = oracle.gaussian_bf16((n_pages, Hkv, page, D), oracle.seed(seed, 2))
    v = oracle.gaussian_bf16((n_pages, Hkv, page, D), oracle.seed(seed, 3))
    return q, k, v, perm


def f64_attention(q, k, v, perm, page, kv_len, H, Hkv, D, scale):
    G = H // Hkv
    qf = oracle.bf16_to_f32(q).astype(np.float64)
    kf = oracle.bf16_to_f32(k).astype(np.float64)
    vf = oracle.bf16_to_f32(v).astype(np.float64)
    j = np.arange(kv_len)
    phys = perm[j // page]
    out = np.zeros((H, D))
    for h in range(H):
        K = kf[phys, h // G, j % page]
        V = vf[phys, h // G, j % page]
        s = K @ qf[h] * scale
        p = np.exp(s - s.max())
        out[h] = p @ V / p.sum()
    return out


@pytest.mark.parametrize("H,Hkv,D,kv_len", [(64, 8, 128, 1000), (8, 8, 64, 33), (16, 2, 128, 1)])
def test_attention_matches_f64(H, Hkv, D, kv_len):
    # kv_cache.rs:206-305: f64 softmax reference, max abs error < 1e-4 (fp32 path)
    q, k, v, perm = paged_case(4, H, Hkv, D, kv_len)
    scale = 1.0 / np.sqrt(D)
    out = oracle.attn_decode_paged(q, k, v, perm, 16, kv_len, H, Hkv, D, scale)
    want = f64_attention(q, k, v, perm, 16, kv_len, H, Hkv, D, scale)
    assert np.abs(out - want).max() < 1e-4


def test_attention_is_a_convex_combination_and_ignores_page_order():
    H, Hkv, D, kv_len = 8, 2, 64, 200
    q, k, v, perm = paged_case(6, H, Hkv, D, kv_len)
    out = oracle.attn_decode_paged(q, k, v, perm, 16, kv_len, H, Hkv, D, 0.125)
    vf = oracle.bf16_to_f32(v)
    # a convex combination of the visible V rows stays inside their range
    phys = perm[np.arange(kv_len) // 16]
    for h in range(H):
        rows = vf[phys, h // 4, np.arange(kv_len) % 16]
        assert np.all(out[h] <= rows.max(0) + 1e-5) and np.all(out[h] >= rows.min(0) - 1e-5)
    # the same logical cache stored in another page order reads identically
    perm2 = oracle.permutation(len(perm), 99)
    k2 = np.empty_like(k)
    v2 = np.empty_like(v)
    k2[perm2] = k[perm]
    v2[perm2] = v[perm]
    out2 = oracle.attn_decode_paged(q, k2, v2, perm2, 16, kv_len, H, Hkv, D, 0.125)
    np.testing.assert_array_equal(out, out2)
    # identical keys give uniform weights: the output is the mean of V
    k3 = np.broadcast_to(k[:1, :1, :1], k.shape).copy()
    out3 = oracle.attn_decode_paged(q, k3, v, perm, 16, kv_len, H, Hkv, D, 0.125)
    for h in range(H):
        rows = vf[phys, h // 4, np.arange(kv_len) % 16].astype(np.float64)
        np.testing.assert_allclose(out3[h], rows.mean(0), atol=2e-6)


# ---- the router GEMV (bf16 weights), the shared expert's gated add, the whole layer ----

@pytest.mark.parametrize("T,N,K", [(1, 128, 4096), (3, 17, 512), (16, 8, 1024)])
def test_gemv_bf16_matches_f64(T, N, K):
    """The reference's GEMV gate (crates/oominf-cuda/tests/gemv.rs:171-181): max |got - want| / sqrt(K) < 1e-5
    against f64 over the same bf16 weights."""
    w = oracle.gaussian_bf16((N, K), 31 + N, 0.02)
    x = oracle.gaussian(T * K, 32 + K).reshape(T, K).astype(np.float32)
    got = oracle.gemv_bf16(x, w)
    want = x.astype(np.float64) @ oracle.bf16_to_f32(w).astype(np.float64).T
    assert np.abs(got - want).max() / np.sqrt(K) < 1e-5


def test_gemv_bf16_closed_form():
    """w = bf16 1.0 (0x3f80) everywhere: y = sum_k x (exact for small integers); a row of
    bf16 -2.0 (0xc000) gives -2 sum_k x; bf16 2^-133 (0x0001, a subnormal) times 2^133 is 1."""
    T, K = 2, 256
    x = np.arange(T * K, dtype=np.float32).reshape(T, K) % 7 - 3
    w = np.full((3, K), 0x3F80, dtype=np.uint16)
    w[1, :] = 0xC000
    w[2, :] = 0
    w[2, 0] = 0x0001
    y = oracle.gemv_bf16(x, w)
    np.testing.assert_array_equal(y[:, 0], x.sum(axis=1))
    np.testing.assert_array_equal(y[:, 1], -2.0 * x.sum(axis=1))
    np.testing.assert_array_equal(y[:, 2], x[:, 0] * np.float32(2.0 ** -133))


def test_combine_shared_special_gates():
    """sigmoid(0) = 1/2 exactly, sigmoid(+inf) = 1, sigmoid(-inf) = 0: out = routed + s * shared."""
    rng = np.random.default_rng(3)
    routed = rng.standard_normal((3, 40)).astype(np.float32)
    shared = rng.standard_normal((3, 40)).astype(np.float32)
    gate = np.array([0.0, np.inf, -np.inf], dtype=np.float32)
    out = oracle.moe_combine_shared(routed, shared, gate)
    np.testing.assert_array_equal(out[0], routed[0] + np.float32(0.5) * shared[0])
    np.testing.assert_array_equal(out[1], routed[1] + shared[1])
    np.testing.assert_array_equal(out[2], routed[2])


def test_layer_composition_closed_form():
    """Zero router weights: every logit 0, so the picks are experts 0..k-1 (ties to the lower
    id) with weights 1/k; zero gate weights: gate 0, so out = routed + shared / 2, where routed
    is the decode step over experts 0..k-1 and shared the shared record's FFN at weight 1."""
    E, k, H, I, SI, T = 12, 4, 256, 128, 256, 3
    geo, sgeo = oracle.record_geometry(H, I), oracle.record_geometry(H, SI)
    recs = synth.expert_records(geo, 61, E)
    srec = synth.expert_records(sgeo, 62, 1)[0]
    x = oracle.bf16_to_f32(synth.activations_bf16(63, T, H))
    rw = np.zeros((E, H), dtype=np.uint16)
    gw = np.zeros((1, H), dtype=np.uint16)
    logits, gate, ids, w, out = oracle.moe_layer_decode(x, rw, recs, k, geo, srec, sgeo, gw)
    assert (logits == 0).all() and (gate == 0).all()
    np.testing.assert_array_equal(ids, np.tile(np.arange(k, dtype=np.int32), (T, 1)))
    np.testing.assert_array_equal(w, np.full((T, k), 1.0 / k, dtype=np.float32))
    _, _, routed = oracle.moe_decode(np.zeros((T, E), np.float32), x, recs, k, geo)
    sids, sw, shared = oracle.moe_decode(np.zeros((T, 1), np.float32), x, [srec], 1, sgeo)
    assert (sids == 0).all() and (sw == 1.0).all()
    np.testing.assert_array_equal(out, routed + np.float32(0.5) * shared)
    # the shared FFN against f64 over the dequantised record (weight 1, one token at a time)
    f64 = synth.f64_moe((np.zeros((T, 1), np.int32), np.ones((T, 1), np.float32)), x, [srec], sgeo)
    assert np.abs(shared - f64).max() <= 2e-5 * np.abs(f64).max()

"""GPU parity of the prefill path (per-token e4m3 quantiser, FP8 grouped GEMM on the
matrix cores, whole prefill MoE step) through the C ABI, against the oracle.

Bars: quantised codes and scales bit-exact; grouped GEMM worst |got - f64| / sum |x w|
< 3e-5 (the reference's own gate for its tiled path is 2e-6, crates/oominf-cuda/tests/moe_tiled.rs:174-223,
for a bf16-exact sum; the FP8 matrix core's block sum is coarser, see the test); prefill
outputs (bf16) end to end within rtol 2e-2 / atol 1e-3 of the oracle's whole prefill in the
same precision (exact: h in fp32, the reference's default path; bf16: h rounded to bf16),
router ids bit-exact.
"""
import numpy as np
import pytest

import oracle
import synth

pytestmark = pytest.mark.gpu
RTOL, ATOL = 2e-2, 1e-3


@pytest.fixture(scope="module")
def hip():
    import torch

    import homelab_amd

    homelab_amd.lib()  # raises if the library is missing: no fallback
    torch.cuda.init()
    return homelab_amd


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def upload_records(recs):
    import torch

    buf = torch.from_numpy(np.stack(recs)).cuda()
    stride = buf.shape[1]
    addrs = torch.tensor([buf.data_ptr() + e * stride for e in range(len(recs))], dtype=torch.int64, device="cuda")
    return buf, addrs


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_quantize_rows_bit_exact(hip, dtype):
    import torch

    rng = np.random.default_rng(3)
    x = (rng.standard_normal((37, 1000)) * np.exp(rng.uniform(-12, 6, (37, 1)))).astype(np.float32)
    x[5] = 0.0                                  # a zero row: scale 1
    x[6, :10] = [1e-30, -1e-30, 2e-3, 0, 448, -448, 1e6, -1e-6, 3.3, 7e-5]
    if dtype == "bf16":
        xb = oracle.bf16_from_f32(x)
        x = oracle.bf16_to_f32(xb)
        xd = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    else:
        xd = dev(x)
    want_q, want_s = oracle.quantize_act(x)
    q = torch.empty(x.shape, dtype=torch.uint8, device="cuda")
    s = torch.empty(x.shape[0], dtype=torch.float32, device="cuda")
    hip.quantize_rows_fp8(xd, q, s)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy(), want_s.reshape(-1))
    np.testing.assert_array_equal(q.cpu().numpy(), want_q)


@pytest.mark.parametrize("x_group", [0, 128])
@pytest.mark.parametrize("N,K,counts", [(256, 512, [1, 0, 37, 130, 200]), (128, 1536, [300, 5]),
                                        (384, 256, [64, 128, 129])])
def test_grouped_gemm_matches_oracle(hip, N, K, counts, x_group):
    import torch

    print(f"grouped gemm N={N} K={K} counts={counts} x_group={x_group}", flush=True)
    recs, dq = [], []
    for e, _ in enumerate(counts):
        w = oracle.gaussian_bf16((N, K), oracle.seed(21, e), 0.02)
        q, s = oracle.quantize(w, oracle.SCALE_128X128)
        recs.append(np.concatenate([q.reshape(-1), s.view(np.uint8)]))
        d = torch.from_numpy(q).view(torch.float8_e4m3fn).double().numpy()
        dq.append(d * s.reshape(N // 128, K // 128)[np.arange(N) // 128][:, np.arange(K) // 128])
    off = np.cumsum([0] + counts).astype(np.int32)
    tokens = 97
    x = oracle.gaussian(tokens * K, 8).reshape(tokens, K) * 3
    xq, xs = oracle.quantize_act(x, x_group)
    rows = np.array([(a * 13 + 5) % tokens for a in range(off[-1])], dtype=np.int32)
    want = oracle.grouped_gemm_fp8(recs, off, rows, xq, xs, x_group, N, K, 0, N * K)
    buf, addrs = upload_records(recs)
    y = torch.full((off[-1], N), float("nan"), dtype=torch.float32, device="cuda")
    hip.moe_grouped_gemm_fp8(addrs, dev(off), dev(rows), len(counts), max(counts), dev(xq), dev(xs), x_group, y,
                             N, K, 0, N * K)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    xd = torch.from_numpy(xq).view(torch.float8_e4m3fn).double().numpy()
    if x_group:
        xd = xd * np.repeat(xs.reshape(tokens, K // 128).astype(np.float64), 128, axis=1)
    else:
        xd = xd * xs.reshape(-1, 1).astype(np.float64)
    # Against the float64 sum. The FP8 matrix core (v_mfma_scale_f32_16x16x128_f8f6f4)
    # adds each group of 8 products at about 13 bits relative to the group's largest
    # product before its fp32 accumulation (one 448 with seven 2^-6 products in its group
    # sums to 448), so its block sums sit up to ~1e-5 of sum |x w| from the exact value
    # where the oracle's sequential fp32 sums sit ~3e-8. The bar is 3e-5 of sum |x w|
    # instead of the reference's 2e-6 for its bf16-exact path; both are far below bf16
    # output precision.
    worst64, worst_or, oracle64 = 0.0, 0.0, 0.0
    for e in range(len(counts)):
        for a in range(off[e], off[e + 1]):
            terms = xd[rows[a]][None, :] * dq[e]
            mag = np.abs(terms).sum(1)
            exact = terms.sum(1)
            worst64 = max(worst64, (np.abs(got[a] - exact) / mag).max())
            worst_or = max(worst_or, (np.abs(got[a] - want[a]) / mag).max())
            oracle64 = max(oracle64, (np.abs(want[a] - exact) / mag).max())
    print(f"worst / sum|x w|: gpu vs f64 {worst64:.2e}, gpu vs oracle {worst_or:.2e}, oracle vs f64 {oracle64:.2e}")
    assert worst64 < 3e-5, worst64
    assert worst_or < 3e-5, worst_or


def prefill_workspace(ws, T, E, k, H, I):
    """The intermediates oom_moe_prefill_fp8 leaves in its workspace (the layout of
    PrefillWs in homelab_amd/csrc/grouped.hip): plan, xq, xs, and h as its bf16 hi and lo
    planes (h = hi + lo)."""
    def al(v):
        return (v + 255) // 256 * 256
    A = T * k
    max_tiles = (A + 127) // 128 + min(E, A)     # 128-row tiles (down)
    max_tiles2 = (A + 255) // 256 + min(E, A)    # 256-row tiles (gate/up)
    o_recs = al((2 + 2 * E + 2 * A) * 4)
    o_xq = o_recs + al(min(E, A) * 8)
    o_xs = o_xq + al(T * H)
    o_tiles = o_xs + al(T * 4)
    o_tiles2 = o_tiles + al((2 * max_tiles + 1) * 4)
    o_hh = o_tiles2 + al((2 * max_tiles2 + 1) * 4)
    o_hl = o_hh + al(A * I * 2)
    W = ws.cpu().numpy()
    plan = W[:(2 + 2 * E + 2 * A) * 4].view(np.int32)
    hi = oracle.bf16_to_f32(W[o_hh:o_hh + A * I * 2].view(np.uint16)).reshape(A, I)
    lo = oracle.bf16_to_f32(W[o_hl:o_hl + A * I * 2].view(np.uint16)).reshape(A, I)
    return {"plan": plan, "xq": W[o_xq:o_xq + T * H].reshape(T, H), "xs": W[o_xs:o_xs + T * 4].view(np.float32),
            "h": (hi.astype(np.float64) + lo.astype(np.float64)).astype(np.float32), "hi": hi, "lo": lo}


MFMA_BAR = 3e-5  # |block sum - exact| / sum |x w| of the FP8 matrix core (test_grouped_gemm_matches_oracle)


def check_h(h, hi, lo, g, u, gabs, uabs, exact=True):
    """The GPU's h against the oracle's g, u: hi is bf16(h) and (exact) lo bf16(h - hi) of
    one fp32 h, and h sits within what the FP8 matrix core's block sums allow (g and u each
    within MFMA_BAR * sum |x w| of the oracle's, carried through silu(g) * u) plus the
    terms' rounding (2^-16 of |h| with two terms, 2^-8 with hi alone)."""
    assert np.array_equal(oracle.bf16_to_f32(oracle.bf16_from_f32(hi)), hi)
    if exact:
        assert np.all(np.abs(lo) <= np.abs(hi) * 2.0 ** -8 * 1.01 + 1e-38), "lo is not the residual of hi"
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-g64))
    h64 = g64 * sig * u64
    dh = MFMA_BAR * (np.abs(sig * (1 + g64 * (1 - sig)) * u64) * gabs + np.abs(g64 * sig) * uabs)
    err = np.abs(h.astype(np.float64) - h64)
    ok = err <= dh + (2.0 ** -16 if exact else 2.0 ** -8) * np.abs(h64) + 1e-30
    assert np.all(ok), f"{(~ok).sum()} of {h.size} h values outside the matrix-core bound; worst excess " \
                       f"{(err - dh)[~ok].max():.3e}"
    return float((err / np.maximum(dh, 1e-30)).max())


def prefill_check(hip, geo, recs, logits, xb, k, sample=None, precision=None):
    """GPU prefill against the oracle: router ids exact and weights to fp32 rounding; x
    codes and scales exact; h within the FP8 matrix core's bound of the oracle's fp32 h;
    the down projection and slot-order combine from the GPU's h within 2e-5 of scale of the
    oracle's (bf16 terms, exact products); and the output end to end within rtol 2e-2 /
    atol 1e-3 of the oracle's whole prefill in the same precision (oracle.moe_prefill:
    h in fp32, the reference's default exact path, or rounded to bf16)."""
    import torch

    if precision is None:
        precision = hip.EXPERT_EXACT
    exact = precision == hip.EXPERT_EXACT

    T, E = logits.shape
    H, I = geo.hidden, geo.inter
    x = oracle.bf16_to_f32(xb)
    hgeo = hip.record_geometry(H, I)
    buf, addrs = upload_records(recs) if isinstance(recs, list) else recs
    ws = torch.zeros(hip.moe_prefill_fp8_workspace_size(T, E, k, hgeo), dtype=torch.uint8, device="cuda")
    ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    out32 = torch.empty((T, H), dtype=torch.float32, device="cuda")
    xd = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    hip.moe_prefill_fp8(dev(logits), xd, addrs, k, hgeo, ids, w, out32, ws, precision=precision)
    hip.moe_prefill_fp8(dev(logits), xd, addrs, k, hgeo, ids, w, out, ws, precision=precision)
    torch.cuda.synchronize()
    host = recs if isinstance(recs, list) else [r for r in buf.cpu().numpy()]
    rows = np.arange(T) if sample is None else np.asarray(sample)
    # router and plan
    want_ids, want_w = oracle.router_topk(logits[rows], k)
    np.testing.assert_array_equal(ids.cpu().numpy()[rows], want_ids)
    np.testing.assert_allclose(w.cpu().numpy()[rows], want_w, rtol=2e-6)
    st = prefill_workspace(ws, T, E, k, H, I)
    ids_all, _ = oracle.router_topk(logits, k)
    experts, off, tok, slot = oracle.moe_plan(ids_all, E)
    # the step's device plan (built over many blocks at large steps), entry for entry
    A, pl = T * k, st["plan"]
    n_e = int(pl[0])
    assert n_e == len(experts)
    np.testing.assert_array_equal(pl[1:1 + n_e], experts)
    assert np.all(pl[1 + n_e:1 + E] == -1)
    np.testing.assert_array_equal(pl[1 + E:2 + E + n_e], off)
    assert np.all(pl[2 + E + n_e:2 + 2 * E] == A)
    np.testing.assert_array_equal(pl[2 + 2 * E:2 + 2 * E + A], tok)
    np.testing.assert_array_equal(pl[2 + 2 * E + A:2 + 2 * E + 2 * A], slot)
    # x codes and scales of the sampled tokens
    xq_or, xs_or = oracle.quantize_act(x[rows])
    np.testing.assert_array_equal(st["xq"][rows], xq_or)
    np.testing.assert_array_equal(st["xs"][rows], xs_or)
    # the sampled tokens' assignments (plan positions) and their experts
    assigns = slot.reshape(T, k)[rows]
    pos_expert = np.searchsorted(off, np.arange(T * k), side="right") - 1
    sel = assigns.reshape(-1)
    e_of = pos_expert[sel]
    # gate/up for those assignments on the oracle (one single-assignment group each)
    recs_sel = [host[experts[e]] for e in e_of]
    off1 = np.arange(len(sel) + 1, dtype=np.int32)
    xq_all, xs_all = oracle.quantize_act(x)
    g = oracle.grouped_gemm_fp8(recs_sel, off1, tok[sel], xq_all, xs_all, 0, I, H, geo.gate_weight, geo.gate_scale)
    u = oracle.grouped_gemm_fp8(recs_sel, off1, tok[sel], xq_all, xs_all, 0, I, H, geo.up_weight, geo.up_scale)
    # sum |x w| of every gate and up output of the sampled assignments
    xabs = np.abs(oracle.e4m3_decode(xq_all).astype(np.float64) * xs_all[:, None])
    gabs, uabs = np.empty_like(g, dtype=np.float64), np.empty_like(u, dtype=np.float64)
    for n, a in enumerate(sel):
        wg, wu, _ = synth.record_weights(host[experts[e_of[n]]], geo)
        xa = xabs[tok[a]].astype(np.float32)
        gabs[n] = np.abs(wg) @ xa
        uabs[n] = np.abs(wu) @ xa
    h_gpu = st["h"][sel] if exact else st["hi"][sel]
    h_used = check_h(h_gpu, st["hi"][sel], st["lo"][sel], g, u, gabs, uabs, exact)
    # down + combine from the GPU's h: the oracle's down over the same h (the bf16 terms
    # carry 16 or 8 bits of h; the products are exact; only the summation order differs)
    y = oracle.moe_down(recs_sel, off1, h_gpu, geo)
    want_gh = oracle.moe_combine_slots(y, np.arange(len(sel), dtype=np.int32).reshape(len(rows), k), want_w)
    got32 = out32.cpu().numpy()[rows]
    err = np.abs(got32 - want_gh).max()
    assert err <= 2e-5 * np.abs(want_gh).max(), f"down + combine from the GPU's h: {err:.3e}"
    # end to end against the oracle's whole prefill in the same precision: the bar (for
    # the exact precision, h in fp32 as the reference's default path keeps it; for bf16,
    # h rounded to bf16 as the reference's ExpertPrecision::Bf16, which at the full shape is
    # itself a few 1e-3 from the fp32-h result, past atol 1e-3)
    _, _, pure = oracle.moe_prefill(logits[rows], x[rows], host, k, geo, h_bf16=not exact)
    got = out.float().cpu().numpy()[rows]
    bad = ~np.isclose(got, pure, rtol=RTOL, atol=ATOL)
    assert not bad.any(), f"end to end: {bad.sum()} of {bad.size} outside rtol {RTOL} / atol {ATOL}; " \
                          f"worst {np.abs(got - pure)[bad].max():.3e}"
    print(f"prefill ({'exact' if exact else 'bf16'}): h within {h_used:.2f} of the matrix-core bound; end to end "
          f"worst abs {np.abs(got - pure).max():.2e}, f32 worst abs {np.abs(got32 - pure).max():.2e}")


def prefill_all_tokens_fp32(hip, geo, buf, addrs, logits, xb, k):
    """Every token of an exact-precision step, the complement of prefill_check's sample:
    router ids of all tokens exact and weights to fp32 rounding, every token's e4m3 x codes
    and scale equal to the oracle's, and the whole f32 output within rtol 2e-2 / atol 1e-3
    of a float32 restatement in torch on the GPU. The restatement decodes the e4m3 codes with
    torch's float8_e4m3fn, applies the 128 x 128 block scales and the per-token activation
    scale, forms h = silu(g) u in fp32 (the reference's default path) and sums the slots in
    slot order."""
    import torch

    T, E = logits.shape
    H, I = geo.hidden, geo.inter
    hgeo = hip.record_geometry(H, I)
    ws = torch.zeros(hip.moe_prefill_fp8_workspace_size(T, E, k, hgeo), dtype=torch.uint8, device="cuda")
    ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    out32 = torch.empty((T, H), dtype=torch.float32, device="cuda")
    xd = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    hip.moe_prefill_fp8(dev(logits), xd, addrs, k, hgeo, ids, w, out32, ws, precision=hip.EXPERT_EXACT)
    torch.cuda.synchronize()
    want_ids, want_w = oracle.router_topk(logits, k)
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
    np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=2e-6)
    st = prefill_workspace(ws, T, E, k, H, I)
    xq, xs = oracle.quantize_act(oracle.bf16_to_f32(xb))
    np.testing.assert_array_equal(st["xq"], xq)
    np.testing.assert_array_equal(st["xs"], xs)
    experts, off, tok, slot = oracle.moe_plan(want_ids, E)

    def e4m3(codes):
        return codes.contiguous().view(torch.float8_e4m3fn).float()

    def weights(e, w_off, s_off, n, kk):
        q = e4m3(buf[e, w_off:w_off + n * kk]).reshape(n // 128, 128, kk // 128, 128)
        sc = buf[e, s_off:s_off + (n // 128) * (kk // 128) * 4].clone().view(torch.float32)
        return (q * sc.reshape(n // 128, 1, kk // 128, 1)).reshape(n, kk)

    tf32 = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        xr = e4m3(torch.from_numpy(xq).cuda()) * torch.from_numpy(xs).cuda()[:, None]
        y = torch.empty((T * k, H), dtype=torch.float32, device="cuda")
        for i, e in enumerate(int(v) for v in experts):
            a0, a1 = int(off[i]), int(off[i + 1])
            xe = xr[torch.from_numpy(tok[a0:a1].astype(np.int64)).cuda()]
            g = torch.mm(xe, weights(e, geo.gate_weight, geo.gate_scale, I, H).t().contiguous())
            u = torch.mm(xe, weights(e, geo.up_weight, geo.up_scale, I, H).t().contiguous())
            h = g / (1.0 + torch.exp(-g)) * u
            y[a0:a1] = torch.mm(h, weights(e, geo.down_weight, geo.down_scale, H, I).t().contiguous())
        wt = torch.from_numpy(want_w).cuda()
        sl = torch.from_numpy(slot.reshape(T, k).astype(np.int64)).cuda()
        ref = torch.zeros((T, H), dtype=torch.float32, device="cuda")
        for j in range(k):
            ref = ref + wt[:, j:j + 1] * y[sl[:, j]]
        torch.cuda.synchronize()
    finally:
        torch.backends.cuda.matmul.allow_tf32 = tf32
    got, ref = out32.cpu().numpy(), ref.cpu().numpy()
    bad = ~np.isclose(got, ref, rtol=RTOL, atol=ATOL)
    assert not bad.any(), f"all tokens: {bad.sum()} of {bad.size} outside rtol {RTOL} / atol {ATOL}; " \
                          f"worst {np.abs(got - ref)[bad].max():.3e}"
    print(f"prefill, all {T} tokens against the fp32 restatement: worst abs {np.abs(got - ref).max():.2e} "
          f"(scale {np.abs(ref).max():.2e})")


@pytest.mark.parametrize("prec", ["bf16", "exact"])
@pytest.mark.parametrize("T,E,k,H,I", [(64, 16, 4, 512, 256), (7, 8, 2, 256, 128), (300, 32, 8, 1024, 384),
                                       (40, 8, 4, 384, 256)])
def test_prefill_small(hip, T, E, k, H, I, prec):
    """Small steps against the oracle. Hidden 384 (three K steps, an odd count) keeps the
    gate/up pass's tiles of at most 32 assignments on single-step stages; the others take
    two K steps a stage for them."""
    print(f"prefill T={T} E={E} k={k} H={H} I={I} precision={prec}", flush=True)
    geo = oracle.record_geometry(H, I)
    logits = synth.decode_logits(77 + T, T, E, 1.1)
    recs = synth.expert_records(geo, 77 + T, E)
    xb = synth.activations_bf16(77 + T, T, H)
    prefill_check(hip, geo, recs, logits, xb, k, precision=hip.EXPERT_EXACT if prec == "exact" else hip.EXPERT_BF16)


@pytest.mark.parametrize("prec", ["bf16", "exact"])
def test_prefill_full_shape_sampled_tokens(hip, prec):
    """2048 tokens, 128 experts (all routed), top-8 with a Zipf(1.1) bias, hidden 4096,
    inter 1536. A token's output depends only on its own row, routing and the experts
    it picks, so the oracle checks a sample of the full step: 12 fixed tokens, the last
    two tokens of each of the two heaviest experts' runs (their last, partial 128-row
    M-tiles) and the tokens of the lightest experts' runs (one or two assignments). At the
    exact precision every token is then checked against a float32 restatement in torch
    (prefill_all_tokens_fp32)."""
    import torch

    T, E, k, H, I = 2048, 128, 8, 4096, 1536
    print(f"prefill full shape, precision {prec}", flush=True)
    geo = oracle.record_geometry(H, I)
    stride = oracle.record_stride(geo)
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    buf = torch.zeros((E, stride), dtype=torch.uint8, device="cuda")
    for e0 in range(0, E, 16):
        for wo, so, n, kk in [(geo.gate_weight, geo.gate_scale, I, H), (geo.up_weight, geo.up_scale, I, H),
                              (geo.down_weight, geo.down_scale, H, I)]:
            wt = (torch.randn((16 * n, kk), generator=g, device="cuda") * 0.02).to(torch.bfloat16).float()
            b = wt.reshape(16 * n // 128, 128, kk // 128, 128)
            amax = b.abs().amax(dim=(1, 3))
            sc = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
            q = (b / sc[:, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
            buf[e0:e0 + 16, wo:wo + n * kk] = q.reshape(16, n * kk)
            buf[e0:e0 + 16, so:so + (n // 128) * (kk // 128) * 4] = sc.reshape(16, -1).contiguous().view(torch.uint8)
    addrs = torch.tensor([buf.data_ptr() + e * stride for e in range(E)], dtype=torch.int64, device="cuda")
    logits = synth.decode_logits(31, T, E, 1.1)
    xb = synth.activations_bf16(31, T, H)
    fixed = [0, 1, 2, 100, 511, 777, 1024, 1500, 1800, 2045, 2046, 2047]
    ids, _ = oracle.router_topk(logits, k)
    experts, off, tok, _ = oracle.moe_plan(ids, E)
    count = np.diff(off)
    heavy = np.argsort(-count, kind="stable")[:2]
    tail = [int(t) for i in heavy for t in tok[off[i + 1] - 2:off[i + 1]]]
    assert all(count[i] % 128 for i in heavy), "the heaviest experts' last M-tiles are full: pick another seed"
    light = np.nonzero(count <= 2)[0]
    assert light.size, "no expert with one or two assignments: pick another seed"
    singles = [int(t) for i in light[:6] for t in tok[off[i]:off[i + 1]]]
    sample = np.array(sorted(set(fixed + tail + singles)))
    print(f"sample: {sample.size} tokens (heaviest experts {count[heavy].tolist()} assignments, "
          f"{light.size} experts with <= 2)", flush=True)
    prefill_check(hip, geo, (buf, addrs), logits, xb, k, sample,
                  precision=hip.EXPERT_EXACT if prec == "exact" else hip.EXPERT_BF16)
    if prec == "exact":
        prefill_all_tokens_fp32(hip, geo, buf, addrs, logits, xb, k)

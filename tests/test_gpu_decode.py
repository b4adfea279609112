"""GPU parity of the decode path (router, FP8 GEMV, routed experts, fused MoE step)
through the C ABI, against the oracle on the same seeded inputs.

Bars: router ids bit-exact; fp32 outputs to the reference's own GEMV gate
(max |got - want| / sqrt(K) < 1e-5, crates/oominf-cuda/tests/gemv.rs:171-181);
bf16 outputs within rtol 2e-2 / atol 1e-3 of the oracle's fp32 result.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle
import synth

pytestmark = pytest.mark.gpu

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))
RTOL, ATOL = 2e-2, 1e-3


@pytest.fixture(scope="module")
def hip():
    import torch

    import homelab_amd

    homelab_amd.lib()  # raises if the library is missing: no fallback
    torch.cuda.init()
    return homelab_amd


def dev(a, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def bf16_dev(bits: np.ndarray):
    import torch

    return dev(bits.view(np.int16), torch.bfloat16) if bits.dtype == np.uint16 else dev(bits)


def to_f32(t) -> np.ndarray:
    import torch

    return t.float().cpu().numpy() if t.dtype == torch.bfloat16 else t.cpu().numpy()


def assert_bf16_close(got: np.ndarray, want: np.ndarray, what: str):
    bad = ~np.isclose(got, want, rtol=RTOL, atol=ATOL)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside rtol {RTOL} / atol {ATOL}; " \
                          f"worst {np.abs(got - want)[bad].max():.3e}"


# ---- formats ---------------------------------------------------------------------

def test_e4m3_decode_every_code_on_device(hip):
    import torch

    print("case: e4m3 all codes via gemv", flush=True)
    q = np.zeros((256, 16), dtype=np.uint8)
    q[:, 0] = np.arange(256)
    x = np.zeros((1, 16), dtype=np.float32)
    x[0, 0] = 1.0
    y = torch.empty((1, 256), dtype=torch.float32, device="cuda")
    hip.gemv_fp8(dev(x), dev(q), dev(np.ones(256, np.float32)), hip.SCALE_ROW, y)
    torch.cuda.synchronize()
    gold = np.array([np.nan if v is None else v for v in GOLD["e4m3_all_codes"]["values"]], dtype=np.float32)
    np.testing.assert_array_equal(y.cpu().numpy()[0], gold)


# ---- router -------------------------------------------------------------------------

@pytest.mark.parametrize("T,E,k,zipf", [(1, 128, 8, None), (16, 128, 8, 1.1), (64, 128, 8, 1.1),
                                        (2048, 128, 8, 1.1), (3, 300, 5, None), (2, 8192, 32, None),
                                        (1, 512, 10, None), (7, 400, 8, 1.1), (2, 512, 32, None)])
def test_router_bit_exact(hip, T, E, k, zipf):
    import torch

    print(f"case: router T={T} E={E} k={k}", flush=True)
    logits = synth.decode_logits(100 + T + E, T, E, zipf)
    want_ids, want_w = oracle.router_topk(logits, k)
    ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    hip.router_topk(dev(logits), ids, w, k)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
    np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=2e-6)


def test_router_ties_and_errors(hip):
    import torch

    logits = np.zeros((2, 64), dtype=np.float32)
    logits[1, [7, 3, 50, 20]] = 2.0
    ids = torch.empty((2, 6), dtype=torch.int32, device="cuda")
    w = torch.empty((2, 6), dtype=torch.float32, device="cuda")
    hip.router_topk(dev(logits), ids, w, 6)
    torch.cuda.synchronize()
    assert ids.cpu().numpy().tolist() == [[0, 1, 2, 3, 4, 5], [3, 7, 20, 50, 0, 1]]
    with pytest.raises(hip.OomError, match="top-k > 32"):
        hip.router_topk(dev(logits), ids, w, 33)


# ---- dense FP8 GEMV ----------------------------------------------------------------

@pytest.mark.parametrize("layout", [0, 1, 2])
@pytest.mark.parametrize("T,N,K", [(1, 4096, 4096), (3, 4100, 1040), (1, 300, 10240), (2, 640, 2560),
                                   (3, 2560, 640), (4, 512, 2560), (8, 1000, 1536), (13, 320, 4096),
                                   (16, 640, 2560)])
def test_gemv_fp8_parity(hip, layout, T, N, K):
    import torch

    print(f"case: gemv layout={layout} T={T} N={N} K={K}", flush=True)
    w = oracle.gaussian_bf16((N, K), 9 + N, 0.02)
    q, s = oracle.quantize(w, layout)
    xb = synth.activations_bf16(T + K, T, K)
    x = oracle.bf16_to_f32(xb)
    want = oracle.gemv_fp8(x, q, s, layout)
    ws_bytes = hip.gemv_fp8_workspace_size(T, N, K)
    ws = torch.zeros(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")
    qd, sd = dev(q), dev(s)
    for xdt in ("f32", "bf16"):
        xd = dev(x) if xdt == "f32" else bf16_dev(xb)
        y32 = torch.empty((T, N), dtype=torch.float32, device="cuda")
        hip.gemv_fp8(xd, qd, sd, layout, y32, ws)
        y16 = torch.empty((T, N), dtype=torch.bfloat16, device="cuda")
        hip.gemv_fp8(xd, qd, sd, layout, y16, ws)
        torch.cuda.synchronize()
        got = y32.cpu().numpy()
        assert np.abs(got - want).max() / math.sqrt(K) < 1e-5, f"x {xdt}"
        assert_bf16_close(to_f32(y16), want, f"gemv bf16 out, x {xdt}")
        # deterministic: a second call gives the same bits (split-K order is fixed)
        y2 = torch.empty_like(y32)
        hip.gemv_fp8(xd, qd, sd, layout, y2, ws)
        torch.cuda.synchronize()
        assert torch.equal(y2, y32)


def test_gemv_rejects_bad_shapes(hip):
    import torch

    q = torch.zeros((2, 130), dtype=torch.uint8, device="cuda")
    x = torch.zeros((1, 130), dtype=torch.float32, device="cuda")
    y = torch.zeros((1, 2), dtype=torch.float32, device="cuda")
    s = torch.ones(4, dtype=torch.float32, device="cuda")
    with pytest.raises(hip.OomError, match="multiple of 16"):
        hip.gemv_fp8(x, q, s, 1, y)
    # split-K shapes need a workspace
    q2 = torch.zeros((16, 16384), dtype=torch.uint8, device="cuda")
    x2 = torch.zeros((1, 16384), dtype=torch.float32, device="cuda")
    y2 = torch.zeros((1, 16), dtype=torch.float32, device="cuda")
    assert hip.gemv_fp8_workspace_size(1, 16, 16384) > 0
    with pytest.raises(hip.OomError, match="workspace"):
        hip.gemv_fp8(x2, q2, torch.ones(16, device="cuda"), 0, y2)


# ---- routed experts ---------------------------------------------------------------------

def upload_records(recs):
    """[E, stride] uint8 on the device and the table of record addresses."""
    import torch

    buf = torch.from_numpy(np.stack(recs)).cuda()
    stride = buf.shape[1]
    base = buf.data_ptr()
    addrs = torch.tensor([base + e * stride for e in range(len(recs))], dtype=torch.int64, device="cuda")
    return buf, addrs


def test_geometry_matches_oracle(hip):
    for h, i in [(4096, 1536), (256, 128), (32, 16), (2560, 640)]:
        a, b = hip.record_geometry(h, i), oracle.record_geometry(h, i)
        assert [getattr(a, f) for f, _ in a._fields_] == [getattr(b, f) for f, _ in b._fields_]
        assert hip.record_stride(a) == oracle.record_stride(b)


@pytest.mark.parametrize("H,I,E,T,k", [(256, 128, 16, 5, 4), (4096, 1536, 12, 3, 8), (1024, 512, 8, 16, 8)])
def test_experts_stage_by_stage(hip, H, I, E, T, k):
    """moe_gate_up / moe_down / moe_combine_slots with a host-built plan, each against the oracle."""
    import torch

    print(f"case: experts stages H={H} I={I} E={E} T={T} k={k}", flush=True)
    geo = oracle.record_geometry(H, I)
    hgeo = hip.record_geometry(H, I)
    recs = synth.expert_records(geo, 21, E)
    logits = synth.decode_logits(21, T, E)
    ids, w = oracle.router_topk(logits, k)
    experts, off, tok, slot = oracle.moe_plan(ids, E)
    sel = [recs[e] for e in experts]
    xb = synth.activations_bf16(21, T, H)
    x = oracle.bf16_to_f32(xb)
    h_want = oracle.moe_gate_up(sel, off, tok, x, geo)
    buf, addrs = upload_records(recs)
    recs_dev = addrs[torch.from_numpy(experts.astype(np.int64)).cuda()].contiguous()
    A = T * k
    h = torch.empty((A, I), dtype=torch.float32, device="cuda")
    hip.moe_gate_up_fp8(recs_dev, dev(off), dev(tok), len(experts), bf16_dev(xb), h, hgeo)
    torch.cuda.synchronize()
    hg = h.cpu().numpy()
    scale = np.abs(h_want).max()
    assert np.abs(hg - h_want).max() <= 1e-5 * scale, "gate_up"
    y_want = oracle.moe_down(sel, off, h_want, geo)
    y = torch.empty((A, H), dtype=torch.float32, device="cuda")
    hip.moe_down_fp8(recs_dev, dev(off), len(experts), dev(h_want), y, hgeo)
    torch.cuda.synchronize()
    assert np.abs(y.cpu().numpy() - y_want).max() <= 1e-5 * np.abs(y_want).max(), "down"
    out_want = oracle.moe_combine_slots(y_want, slot, w)
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    hip.moe_combine_slots(dev(y_want), dev(slot), dev(w), out)
    torch.cuda.synchronize()
    assert_bf16_close(to_f32(out), out_want, "combine")


@pytest.mark.parametrize("T,E,k,zipf", [(1, 128, 8, None), (16, 128, 8, 1.1), (64, 128, 8, 1.1), (5, 16, 4, None),
                                        (64, 512, 10, 1.1),   # the released model's E, ballot ranks, one round
                                        (128, 512, 10, 1.1),  # ... past 1024 slots: two rounds
                                        (3, 8192, 32, None),  # the largest E and k: the counting fallback
                                        (40, 8192, 32, 1.1),  # ... over two rounds of 1024 slots
                                        (2048, 128, 8, 1.1)])  # the prefill's plan: 16,384 slots, 16 rounds
def test_device_plan_matches_host_plan(hip, T, E, k, zipf):
    import torch

    print(f"case: device plan T={T} E={E} k={k} zipf={zipf}", flush=True)
    logits = synth.decode_logits(5 + T, T, E, zipf)
    ids, _ = oracle.router_topk(logits, k)
    experts, off, tok, slot = oracle.moe_plan(ids, E)
    plan = torch.full((hip.moe_plan_size(T, E, k),), -7, dtype=torch.int32, device="cuda")
    all_recs = torch.arange(E, dtype=torch.int64, device="cuda") * 4096 + 1
    recs = torch.zeros(E, dtype=torch.int64, device="cuda")
    hip.moe_plan(dev(ids), E, all_recs, plan, recs)
    torch.cuda.synchronize()
    p = plan.cpu().numpy()
    n_e = len(experts)
    A = T * k
    assert p[0] == n_e
    np.testing.assert_array_equal(p[1:1 + n_e], experts)
    assert np.all(p[1 + n_e:1 + E] == -1)
    np.testing.assert_array_equal(p[1 + E:1 + E + n_e + 1], off)
    np.testing.assert_array_equal(p[2 + 2 * E:2 + 2 * E + A], tok)
    np.testing.assert_array_equal(p[2 + 2 * E + A:2 + 2 * E + 2 * A], slot)
    np.testing.assert_array_equal(recs.cpu().numpy()[:n_e], experts.astype(np.int64) * 4096 + 1)


def decode_case(T, E, k, zipf, seed, H=4096, I=1536):
    geo = oracle.record_geometry(H, I)
    logits = synth.decode_logits(seed, T, E, zipf)
    ids, _ = oracle.router_topk(logits, k)
    chosen = set(int(e) for e in np.unique(ids))
    recs = synth.expert_records(geo, seed, E, only=chosen)
    xb = synth.activations_bf16(seed, T, H)
    return geo, logits, recs, xb


@pytest.mark.parametrize("T,E,k,zipf,H,I", [(1, 128, 8, None, 4096, 1536), (16, 128, 8, 1.1, 4096, 1536),
                                            (4, 128, 8, None, 4096, 1536), (64, 128, 8, 1.1, 1024, 512),
                                            (3, 16, 4, None, 256, 128), (80, 64, 8, None, 1024, 512),
                                            # E > 256 takes the multi-launch path (router, device plan at
                                            # E = 512, gate/up, down, combine)
                                            (4, 512, 8, None, 1024, 512), (1, 512, 10, None, 2048, 512),
                                            pytest.param(2, 300, 6, None, 512, 256, marks=pytest.mark.skip(
                                                reason="left the GPU faulted once with the one-launch kernel's "
                                                       "E > 256 router (cause not found on the CPU); that path is "
                                                       "off and this case stays off the GPU until a cause is shown"))])
def test_fused_decode_full_size(hip, T, E, k, zipf, H, I):
    """The whole decode MoE step on the device with no host sync, against the oracle:
    the benchmark's shapes (hidden 4096, inter 1536, 128 experts, top-8) at batch 1,
    4 and 16, small shapes with masked lanes, and a step past the one-launch kernel's
    limit (T * k > 512) that takes the multi-launch path."""
    import torch

    print(f"case: fused decode T={T} E={E} k={k} zipf={zipf} H={H} I={I}", flush=True)
    geo, logits, recs, xb = decode_case(T, E, k, zipf, 1000 + T, H, I)
    x = oracle.bf16_to_f32(xb)
    want_ids, want_w, want = oracle.moe_decode(logits, x, recs, k, geo)
    hgeo = hip.record_geometry(geo.hidden, geo.inter)
    buf, addrs = upload_records(recs)
    ws = torch.zeros(hip.moe_decode_fp8_workspace_size(T, E, k, hgeo), dtype=torch.uint8, device="cuda")
    ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    out = torch.empty((T, geo.hidden), dtype=torch.bfloat16, device="cuda")
    ld, xd = dev(logits), bf16_dev(xb)
    for rep in range(3):  # repeated calls reuse the workspace
        hip.moe_decode_fp8(ld, xd, addrs, k, hgeo, ids, w, out, ws)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
        np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=2e-6)
        assert_bf16_close(to_f32(out), want, f"fused decode rep {rep}")
    # f32 output against the f64 evaluation of the same routing
    out32 = torch.empty((T, geo.hidden), dtype=torch.float32, device="cuda")
    hip.moe_decode_fp8(ld, xd, addrs, k, hgeo, ids, w, out32, ws)
    torch.cuda.synchronize()
    f64 = synth.f64_moe((want_ids, want_w), x, recs, geo)
    assert np.abs(out32.cpu().numpy() - f64).max() <= 2e-5 * np.abs(f64).max()

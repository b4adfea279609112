"""GPU parity of the NVFP4 routed experts (oom_moe_gate_up_nvfp4, oom_moe_down_nvfp4,
oom_moe_decode_nvfp4) through the C ABI.

* The reference's own known answer (crates/oominf-metal/src/tests.rs:239-270, in
  tests/golden/known_answers.json) through the down projection: a record whose first
  three down rows are the test's bytes and scales, scale_2 = 0.75; y must match at the
  test's tolerance 1e-4. This fixes the nibble order and the scale-group index on the
  device.
* gate/up and down stage by stage against a float64 evaluation of the exact decode,
  within 1e-5 of sum |x . w| per output (the GPU sums 16-term groups scaled once).
* The whole step: router ids bit-exact and weights to fp32 rounding; bf16 outputs within
  rtol 2e-2 / atol 1e-3 of the oracle; f32 outputs within 2e-5 of scale of the float64
  evaluation; repeated calls on one workspace.
"""
import json
import os

import numpy as np
import pytest

import oracle
import synth

pytestmark = pytest.mark.gpu
RTOL, ATOL = 2e-2, 1e-3
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


@pytest.fixture(scope="module")
def hip():
    import torch

    import homelab_amd

    homelab_amd.lib()
    torch.cuda.init()
    return homelab_amd


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bf16(bits):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def _upload(recs):
    import torch

    buf = torch.from_numpy(np.stack(recs)).cuda()
    addrs = torch.tensor([buf.data_ptr() + e * buf.shape[1] for e in range(len(recs))], dtype=torch.int64,
                         device="cuda")
    return buf, addrs


def test_known_answer_through_down(hip):
    import torch

    print("case: nvfp4 known answer", flush=True)
    ka = GOLDEN["nvfp4_rows_known_answer"]
    T, R, C = ka["tokens"], ka["rows"], ka["cols"]
    H, I = 16, C  # down: [hidden 16, inter 32]; rows 3..15 zero
    geo = oracle.nvfp4_geometry(H, I)
    rec = np.zeros(oracle.nvfp4_stride(geo), dtype=np.uint8)
    rec[geo.down_weight:geo.down_weight + R * C // 2] = np.array(ka["packed"], dtype=np.uint8)
    rec[geo.down_scale:geo.down_scale + R * C // 16] = np.array(ka["scales"], dtype=np.uint8)
    rec[geo.scale2[2] * 4:geo.scale2[2] * 4 + 4] = np.array([ka["scale2"]], dtype=np.float32).view(np.uint8)
    buf, addrs = _upload([rec])
    h = _dev(np.array(ka["x"], dtype=np.float32).reshape(T, C))
    y = torch.full((T, H), float("nan"), dtype=torch.float32, device="cuda")
    off = _dev(np.array([0, T], dtype=np.int32))
    hip.moe_down_nvfp4(addrs, off, 1, h, y, hip.nvfp4_geometry(H, I))
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = np.array(ka["y"]).reshape(T, R)
    assert np.abs(got[:, :R] - want).max() < ka["tol"]
    assert (got[:, R:] == 0).all()


@pytest.mark.parametrize("H,I,T,xf32", [(2560, 640, 1, False), (1040, 432, 3, False), (4096, 1536, 2, True)])
def test_gate_up_and_down_stage_by_stage(hip, H, I, T, xf32):
    import torch

    print(f"case: nvfp4 stages H={H} I={I} T={T} x={'f32' if xf32 else 'bf16'}", flush=True)
    geo = oracle.nvfp4_geometry(H, I)
    recs = synth.nvfp4_records(geo, 300 + H, 2)
    xb = synth.activations_bf16(301, T, H)
    x = oracle.bf16_to_f32(xb)
    off = np.array([0, T, 2 * T], dtype=np.int32)
    tok = np.concatenate([np.arange(T), np.arange(T)[::-1]]).astype(np.int32)
    buf, addrs = _upload(recs)
    hgeo = hip.nvfp4_geometry(H, I)
    h = torch.full((2 * T, I), float("nan"), dtype=torch.float32, device="cuda")
    hip.moe_gate_up_nvfp4(addrs, _dev(off), _dev(tok), 2, _dev(x) if xf32 else _bf16(xb), h, hgeo)
    torch.cuda.synchronize()
    h_got = h.cpu().numpy()
    # down from the oracle's h, so the two stages are checked apart
    h_or = oracle.moe_gate_up_nvfp4(recs, off, tok, x, geo)
    y = torch.full((2 * T, H), float("nan"), dtype=torch.float32, device="cuda")
    hip.moe_down_nvfp4(addrs, _dev(off), 2, _dev(h_or), y, hgeo)
    torch.cuda.synchronize()
    y_got = y.cpu().numpy()
    for i in range(2):
        g, u, d = synth.nvfp4_weights(recs[i], geo)
        for a in range(off[i], off[i + 1]):
            xt = x[tok[a]].astype(np.float64)
            gv, uv = g @ xt, u @ xt
            bg, bu = np.abs(g) @ np.abs(xt), np.abs(u) @ np.abs(xt)
            hv = gv / (1 + np.exp(-gv)) * uv
            err = np.abs(h_got[a] - hv)
            assert np.all(err <= 1e-5 * (1.1 * np.abs(uv) * bg + np.abs(gv) * bu) + 1e-12), f"h of assignment {a}"
            hd = h_or[a].astype(np.float64)
            assert np.all(np.abs(y_got[a] - d @ hd) <= 1e-5 * (np.abs(d) @ np.abs(hd)) + 1e-12), f"y of {a}"


@pytest.mark.parametrize("T,E,k,zipf,H,I,xf32", [
    (1, 512, 10, None, 2560, 640, False),   # the released model's routed experts, one token
    (4, 512, 10, None, 2560, 640, False),   # ... four tokens: router, device plan at E = 512, staged launches
    (4, 64, 8, None, 4096, 1536, False),    # the FP8 benchmark's widths in NVFP4
    (16, 128, 8, 1.1, 1040, 432, False),    # widths ending inside a 32-column piece, popular experts
    (9, 32, 6, None, 512, 256, False),      # experts with more tokens than a pass holds
    (3, 16, 4, None, 256, 128, True),       # f32 activations
])
def test_decode_nvfp4_matches_oracle(hip, T, E, k, zipf, H, I, xf32):
    import torch

    print(f"case: nvfp4 decode T={T} E={E} k={k} zipf={zipf} H={H} I={I} x={'f32' if xf32 else 'bf16'}",
          flush=True)
    seed = 400 + T + E + H
    geo = oracle.nvfp4_geometry(H, I)
    logits = synth.decode_logits(seed, T, E, zipf)
    ids0, _ = oracle.router_topk(logits, k)
    recs = synth.nvfp4_records(geo, seed, E, only=set(int(e) for e in np.unique(ids0)))
    xb = synth.activations_bf16(seed, T, H)
    x = oracle.bf16_to_f32(xb)
    want_ids, want_w, want = oracle.moe_decode_nvfp4(logits, x, recs, k, geo)
    hgeo = hip.nvfp4_geometry(H, I)
    buf, addrs = _upload(recs)
    ws = torch.zeros(hip.moe_decode_nvfp4_workspace_size(T, E, k, hgeo), dtype=torch.uint8, device="cuda")
    ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    xd = _dev(x) if xf32 else _bf16(xb)
    ld = _dev(logits)
    for rep in range(2):
        out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        hip.moe_decode_nvfp4(ld, xd, addrs, k, hgeo, ids, w, out, ws)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ids.cpu().numpy(), want_ids, err_msg=f"rep {rep}")
        np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=2e-6, err_msg=f"rep {rep}")
        got = out.float().cpu().numpy()
        bad = ~np.isclose(got, want, rtol=RTOL, atol=ATOL)
        assert not bad.any(), f"rep {rep}: {bad.sum()} of {bad.size} outside; worst {np.abs(got - want)[bad].max():.3e}"
    out32 = torch.empty((T, H), dtype=torch.float32, device="cuda")
    hip.moe_decode_nvfp4(ld, xd, addrs, k, hgeo, ids, w, out32, ws)
    torch.cuda.synchronize()
    f64 = synth.f64_moe_nvfp4((want_ids, want_w), x, recs, geo)
    err = np.abs(out32.cpu().numpy() - f64).max()
    assert err <= 2e-5 * np.abs(f64).max(), f"f32 out: max err {err:.3e} vs scale {np.abs(f64).max():.3e}"


@pytest.mark.parametrize("E,k,H,I,xf32", [
    (512, 10, 2560, 640, False),   # the released model's routed experts (8 logits a lane in the router)
    (64, 8, 4096, 1536, False),    # the FP8 benchmark's widths: 64 KiB of staged h rows
    (100, 16, 1040, 432, True),    # 16 slots, widths ending inside a piece, f32 activations
    (16, 1, 256, 128, False),      # one slot; fewer output tiles than blocks
    (32, 4, 3072, 128, False),     # more 10-row output tiles than resident blocks (the second loads late)
    (64, 12, 2048, 1024, False),   # 3072 gate/up items over 2048 waves: half the waves take a second item
    (300, 6, 1024, 256, True),     # past 256 experts: 8 logits a lane, the last 212 lanes of the 5th..8th absent
    (512, 16, 4096, 640, False),   # 16 picks of 512, hidden past 3072: the 4-wave kernel with 8 logits a lane
])
def test_decode_nvfp4_one_launch_matches_stages(hip, E, k, H, I, xf32):
    """One token takes the one-launch kernel; its f32 output equals, bit for bit, the staged
    launches (router, gate/up, down, slot-order combine) over the same routing, on three
    calls in a row on one workspace (the grid barrier's generations advance)."""
    print(f"case: nvfp4 one-launch E={E} k={k} H={H} I={I} x={'f32' if xf32 else 'bf16'}", flush=True)
    seed = 900 + E + H
    _one_launch_check(hip, E, k, H, I, xf32, seed, synth.decode_logits(seed, 1, E, None))


@pytest.mark.parametrize("E,k,levels", [(512, 10, 2.0), (512, 16, 0.0), (300, 8, 4.0)])
def test_decode_nvfp4_one_launch_router_ties(hip, E, k, levels):
    """Logits on a coarse grid (levels a unit; 0: all equal), so many experts tie in p at the
    k-th pick: the one-launch router's descent (gathered one key a lane once at most 64
    remain) picks the lower ids among equals, as the router kernel and the oracle do."""
    print(f"case: nvfp4 one-launch router ties E={E} k={k} levels={levels}", flush=True)
    seed = 77 + E + k
    z = np.random.default_rng(seed).standard_normal((1, E))
    logits = (np.round(z * levels) / levels if levels else np.zeros_like(z)).astype(np.float32)
    _one_launch_check(hip, E, k, 1024, 256, False, seed, logits)


def _one_launch_check(hip, E, k, H, I, xf32, seed, logits):
    import torch

    geo = oracle.nvfp4_geometry(H, I)
    hgeo = hip.nvfp4_geometry(H, I)
    ids0, _ = oracle.router_topk(logits, k)
    recs = synth.nvfp4_records(geo, seed, E, only=set(int(e) for e in np.unique(ids0)))
    xb = synth.activations_bf16(seed, 1, H)
    x = oracle.bf16_to_f32(xb)
    xd = _dev(x) if xf32 else _bf16(xb)
    buf, addrs = _upload(recs)
    ld = _dev(logits)
    # staged: the router kernel, the oracle's grouping, then gate/up, down and combine launches
    ids_s = torch.empty((1, k), dtype=torch.int32, device="cuda")
    w_s = torch.empty((1, k), dtype=torch.float32, device="cuda")
    hip.router_topk(ld, ids_s, w_s, k)
    torch.cuda.synchronize()
    experts, off, tok, slot = oracle.moe_plan(ids_s.cpu().numpy(), E)
    n_e = len(experts)
    recs_s = addrs[torch.from_numpy(np.asarray(experts, dtype=np.int64)).cuda()]
    h = torch.empty((k, I), dtype=torch.float32, device="cuda")
    y = torch.empty((k, H), dtype=torch.float32, device="cuda")
    hip.moe_gate_up_nvfp4(recs_s, _dev(np.asarray(off, dtype=np.int32)), _dev(np.asarray(tok, dtype=np.int32)), n_e,
                          xd, h, hgeo)
    hip.moe_down_nvfp4(recs_s, _dev(np.asarray(off, dtype=np.int32)), n_e, h, y, hgeo)
    want = torch.empty((1, H), dtype=torch.float32, device="cuda")
    hip.moe_combine_slots(y, _dev(np.asarray(slot, dtype=np.int32).reshape(1, k)), w_s, want)
    torch.cuda.synchronize()
    want = want.cpu().numpy()
    ws = torch.zeros(hip.moe_decode_nvfp4_workspace_size(1, E, k, hgeo), dtype=torch.uint8, device="cuda")
    ids = torch.empty((1, k), dtype=torch.int32, device="cuda")
    w = torch.empty((1, k), dtype=torch.float32, device="cuda")
    for rep in range(3):
        out = torch.full((1, H), float("nan"), dtype=torch.float32, device="cuda")
        hip.moe_decode_nvfp4(ld, xd, addrs, k, hgeo, ids, w, out, ws)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ids.cpu().numpy(), ids_s.cpu().numpy(), err_msg=f"rep {rep}")
        np.testing.assert_array_equal(w.cpu().numpy(), w_s.cpu().numpy(), err_msg=f"rep {rep}")
        got = out.cpu().numpy()
        diff = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
        assert diff.size == 0, f"rep {rep}: {diff.size} of {H} differ, first at {diff[:4]}"
    # and the oracle's tolerance on a bf16 output
    want_ids, want_w, want_or = oracle.moe_decode_nvfp4(logits, x, recs, k, geo)
    outb = torch.empty((1, H), dtype=torch.bfloat16, device="cuda")
    hip.moe_decode_nvfp4(ld, xd, addrs, k, hgeo, ids, w, outb, ws)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
    got = outb.float().cpu().numpy()
    bad = ~np.isclose(got, want_or, rtol=RTOL, atol=ATOL)
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside; worst {np.abs(got - want_or)[bad].max():.3e}"
    assert hip.status() == hip.OK, "a wait of the one-launch kernel gave up"

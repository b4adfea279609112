"""GPU parity of the one-token decode step (oom_moe_decode_fp8 at T = 1, the barrier-free
one-launch kernel) through the C ABI, against the oracle on the same seeded inputs.

Bars (as for the whole decode path): router ids bit-exact and weights to fp32 rounding;
bf16 outputs within rtol 2e-2 / atol 1e-3 of the oracle's fp32 result; f32 outputs within
2e-5 of scale of the f64 evaluation of the same routing. The cases cover the shapes'
edges (k below 8 and the slot-register reload past slot 4, inter below one 512-column
group and partial groups, hidden below the grid's rows, E up to 256), calls that reuse one
workspace with a fresh routing each call (the call epoch), and a workspace shared by one-
and many-token steps.
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


def _check(got_ids, got_w, got, want_ids, want_w, want, what):
    np.testing.assert_array_equal(got_ids, want_ids, err_msg=f"{what}: router ids")
    np.testing.assert_allclose(got_w, want_w, rtol=2e-6, err_msg=f"{what}: router weights")
    bad = ~np.isclose(got, want, rtol=RTOL, atol=ATOL)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} outside rtol {RTOL} / atol {ATOL}; " \
                          f"worst {np.abs(got - want)[bad].max():.3e}"


def _status(hip) -> int:
    """oom_status after the calls: OK unless a bounded wait inside a kernel gave up."""
    return hip.status()


@pytest.mark.parametrize("E,k,H,I,xf32", [
    (128, 8, 4096, 1536, False),  # the benchmark's shape
    (128, 8, 4096, 1536, True),   # f32 activations
    (256, 8, 2048, 1024, False),  # 4 logits per lane, two 512-column groups
    (16, 4, 256, 128, False),     # k <= 4 (no reload), inter inside one partial group, few output rows
    (64, 6, 1024, 768, False),    # reload with two upper slots, a half group
    (200, 8, 512, 1536, True),    # E between 128 and 256, hidden below 16 x blocks
    (8, 8, 1024, 512, False),     # every expert routed
])
def test_decode1_matches_oracle(hip, E, k, H, I, xf32):
    import torch

    print(f"case: one-token decode E={E} k={k} H={H} I={I} x={'f32' if xf32 else 'bf16'}", flush=True)
    seed = 4000 + E + k + I
    geo = oracle.record_geometry(H, I)
    logits = synth.decode_logits(seed, 1, E)
    ids, _ = oracle.router_topk(logits, k)
    recs = synth.expert_records(geo, seed, E, only=set(int(e) for e in ids[0]))
    xb = synth.activations_bf16(seed, 1, H)
    x = oracle.bf16_to_f32(xb)
    want_ids, want_w, want = oracle.moe_decode(logits, x, recs, k, geo)
    hgeo = hip.record_geometry(H, I)
    buf, addrs = _upload(recs)
    ws = torch.zeros(hip.moe_decode_fp8_workspace_size(1, E, k, hgeo), dtype=torch.uint8, device="cuda")
    gids = torch.empty((1, k), dtype=torch.int32, device="cuda")
    gw = torch.empty((1, k), dtype=torch.float32, device="cuda")
    out = torch.empty((1, H), dtype=torch.bfloat16, device="cuda")
    xd = _dev(x) if xf32 else _bf16(xb)
    ld = _dev(logits)
    for rep in range(3):
        hip.moe_decode_fp8(ld, xd, addrs, k, hgeo, gids, gw, out, ws)
        torch.cuda.synchronize()
        _check(gids.cpu().numpy(), gw.cpu().numpy(), out.float().cpu().numpy(), want_ids, want_w, want,
               f"rep {rep}")
    out32 = torch.empty((1, H), dtype=torch.float32, device="cuda")
    hip.moe_decode_fp8(ld, xd, addrs, k, hgeo, gids, gw, out32, ws)
    torch.cuda.synchronize()
    f64 = synth.f64_moe((want_ids, want_w), x, recs, geo)
    err = np.abs(out32.cpu().numpy() - f64).max()
    assert err <= 2e-5 * np.abs(f64).max(), f"f32 out: max err {err:.3e} vs scale {np.abs(f64).max():.3e}"
    assert _status(hip) == hip.OK, "a wait of the decode kernel gave up"


def test_decode1_fresh_routing_each_call(hip):
    """Ten calls on one workspace, each with new logits (a different expert set), with no
    synchronisation between them: every call's h carries its own epoch, so no call reads
    the previous call's h."""
    import torch

    E, k, H, I = 32, 8, 2048, 1024
    geo = oracle.record_geometry(H, I)
    recs = synth.expert_records(geo, 77, E)
    xb = synth.activations_bf16(77, 1, H)
    x = oracle.bf16_to_f32(xb)
    hgeo = hip.record_geometry(H, I)
    buf, addrs = _upload(recs)
    n = 10
    logits = np.stack([synth.decode_logits(500 + i, 1, E) for i in range(n)])
    ws = torch.zeros(hip.moe_decode_fp8_workspace_size(1, E, k, hgeo), dtype=torch.uint8, device="cuda")
    gids = torch.empty((n, 1, k), dtype=torch.int32, device="cuda")
    gw = torch.empty((n, 1, k), dtype=torch.float32, device="cuda")
    out = torch.empty((n, 1, H), dtype=torch.bfloat16, device="cuda")
    ld, xd = _dev(logits), _bf16(xb)
    for i in range(n):
        hip.moe_decode_fp8(ld[i], xd, addrs, k, hgeo, gids[i], gw[i], out[i], ws)
    torch.cuda.synchronize()
    for i in range(n):
        want_ids, want_w, want = oracle.moe_decode(logits[i], x, recs, k, geo)
        _check(gids[i].cpu().numpy(), gw[i].cpu().numpy(), out[i].float().cpu().numpy(), want_ids, want_w, want,
               f"call {i}")
    assert _status(hip) == hip.OK


def test_decode1_workspace_shared_with_batched_steps(hip):
    """One workspace serves one-token and 4-token steps in turn (the one-token kernel and
    the multi-token kernel keep their state in the workspace header)."""
    import torch

    E, k, H, I = 32, 8, 1024, 512
    geo = oracle.record_geometry(H, I)
    recs = synth.expert_records(geo, 91, E)
    hgeo = hip.record_geometry(H, I)
    buf, addrs = _upload(recs)
    size = max(hip.moe_decode_fp8_workspace_size(T, E, k, hgeo) for T in (1, 4))
    ws = torch.zeros(size, dtype=torch.uint8, device="cuda")
    for i, T in enumerate((1, 4, 1, 1, 4, 1)):
        logits = synth.decode_logits(700 + i, T, E)
        xb = synth.activations_bf16(700 + i, T, H)
        x = oracle.bf16_to_f32(xb)
        want_ids, want_w, want = oracle.moe_decode(logits, x, recs, k, geo)
        gids = torch.empty((T, k), dtype=torch.int32, device="cuda")
        gw = torch.empty((T, k), dtype=torch.float32, device="cuda")
        out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        hip.moe_decode_fp8(_dev(logits), _bf16(xb), addrs, k, hgeo, gids, gw, out, ws)
        torch.cuda.synchronize()
        _check(gids.cpu().numpy(), gw.cpu().numpy(), out.float().cpu().numpy(), want_ids, want_w, want,
               f"step {i} (T={T})")
    assert _status(hip) == hip.OK


def test_decode1_router_ties(hip):
    """Equal logits: the picks are the lowest ids among equals, in the reference's order."""
    import torch

    E, k, H, I = 64, 8, 512, 256
    geo = oracle.record_geometry(H, I)
    logits = np.zeros((1, E), dtype=np.float32)
    logits[0, [5, 9, 40, 41, 63]] = 1.5  # five equal leaders, then 59 equal others
    ids, _ = oracle.router_topk(logits, k)
    assert list(ids[0][:5]) == [5, 9, 40, 41, 63] and list(ids[0][5:]) == [0, 1, 2]
    recs = synth.expert_records(geo, 5, E, only=set(int(e) for e in ids[0]))
    xb = synth.activations_bf16(5, 1, H)
    want_ids, want_w, want = oracle.moe_decode(logits, oracle.bf16_to_f32(xb), recs, k, geo)
    hgeo = hip.record_geometry(H, I)
    buf, addrs = _upload(recs)
    ws = torch.zeros(hip.moe_decode_fp8_workspace_size(1, E, k, hgeo), dtype=torch.uint8, device="cuda")
    gids = torch.empty((1, k), dtype=torch.int32, device="cuda")
    gw = torch.empty((1, k), dtype=torch.float32, device="cuda")
    out = torch.empty((1, H), dtype=torch.bfloat16, device="cuda")
    hip.moe_decode_fp8(_dev(logits), _bf16(xb), addrs, k, hgeo, gids, gw, out, ws)
    torch.cuda.synchronize()
    _check(gids.cpu().numpy(), gw.cpu().numpy(), out.float().cpu().numpy(), want_ids, want_w, want, "ties")

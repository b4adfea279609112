"""GPU parity of the small-batch decode step (oom_moe_decode_fp8 at 2..16 tokens with bf16
activations, the one-launch bf16-MFMA kernel) through the C ABI, against the oracle on
the same seeded inputs.

Bars (as for the whole decode path): router ids bit-exact and weights to fp32 rounding;
bf16 outputs within rtol 2e-2 / atol 1e-3 of the oracle's fp32 result; f32 outputs within
2e-5 of scale of the f64 evaluation of the same routing. The cases cover the kernel's
edges: 2 and 16 tokens, an expert shared by all 16 tokens (a full MFMA column tile),
E = 256, the widest hidden and inter, hidden and inter that end inside a 128-column K step,
narrow widths, shapes this kernel leaves to the general one-launch kernel (more than 16
tokens, f32 activations), and calls of different batch sizes on one workspace with
no synchronisation between them.
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


def _case(T, E, k, zipf, seed, H, I):
    geo = oracle.record_geometry(H, I)
    logits = synth.decode_logits(seed, T, E, zipf)
    ids, _ = oracle.router_topk(logits, k)
    recs = synth.expert_records(geo, seed, E, only=set(int(e) for e in np.unique(ids)))
    xb = synth.activations_bf16(seed, T, H)
    return geo, logits, recs, xb


@pytest.mark.parametrize("T,E,k,zipf,H,I,xf32", [
    (2, 64, 8, None, 1024, 512, False),     # the smallest batch
    (16, 8, 8, None, 512, 256, False),      # every expert routed by all 16 tokens
    (7, 256, 6, None, 2048, 1024, False),   # E = 256, k = 6
    (16, 32, 8, None, 4096, 2048, False),   # the widest hidden and inter
    (9, 48, 5, None, 1040, 432, False),     # hidden and inter ending inside a K step
    (12, 128, 8, 1.1, 272, 144, False),     # narrow widths, popular experts
    (16, 128, 8, 1.1, 4096, 1536, False),   # the benchmark's shape
    (20, 64, 8, None, 512, 256, False),     # past 16 tokens: the general kernel
    (6, 64, 8, None, 1024, 512, True),      # f32 activations: the general kernel
])
def test_batch_decode_matches_oracle(hip, T, E, k, zipf, H, I, xf32):
    import torch

    print(f"case: batch decode T={T} E={E} k={k} zipf={zipf} H={H} I={I} x={'f32' if xf32 else 'bf16'}",
          flush=True)
    geo, logits, recs, xb = _case(T, E, k, zipf, 6000 + 7 * T + E + I, H, I)
    x = oracle.bf16_to_f32(xb)
    want_ids, want_w, want = oracle.moe_decode(logits, x, recs, k, geo)
    hgeo = hip.record_geometry(H, I)
    buf, addrs = _upload(recs)
    ws = torch.zeros(hip.moe_decode_fp8_workspace_size(T, E, k, hgeo), dtype=torch.uint8, device="cuda")
    gids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    gw = torch.empty((T, k), dtype=torch.float32, device="cuda")
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    xd = _dev(x) if xf32 else _bf16(xb)
    ld = _dev(logits)
    for rep in range(3):  # repeated calls reuse the workspace (barrier words, tickets)
        hip.moe_decode_fp8(ld, xd, addrs, k, hgeo, gids, gw, out, ws)
        torch.cuda.synchronize()
        _check(gids.cpu().numpy(), gw.cpu().numpy(), out.float().cpu().numpy(), want_ids, want_w, want,
               f"rep {rep}")
    out32 = torch.empty((T, H), dtype=torch.float32, device="cuda")
    hip.moe_decode_fp8(ld, xd, addrs, k, hgeo, gids, gw, out32, ws)
    torch.cuda.synchronize()
    f64 = synth.f64_moe((want_ids, want_w), x, recs, geo)
    err = np.abs(out32.cpu().numpy() - f64).max()
    assert err <= 2e-5 * np.abs(f64).max(), f"f32 out: max err {err:.3e} vs scale {np.abs(f64).max():.3e}"
    assert _status(hip) == hip.OK, "a wait of the decode kernel gave up"


def test_batch_sizes_in_turn_on_one_workspace(hip):
    """Steps of 16, 3, 1, 16, 2 and 1 tokens on one workspace with no synchronisation
    between them: the one-token, small-batch and general kernels share the header's
    barrier words and tickets, and each leaves them ready for the next."""
    import torch

    E, k, H, I = 32, 8, 1024, 512
    geo = oracle.record_geometry(H, I)
    recs = synth.expert_records(geo, 93, E)
    hgeo = hip.record_geometry(H, I)
    buf, addrs = _upload(recs)
    sizes = (16, 3, 1, 16, 2, 1)
    ws = torch.zeros(max(hip.moe_decode_fp8_workspace_size(T, E, k, hgeo) for T in sizes), dtype=torch.uint8,
                     device="cuda")
    runs = []
    for i, T in enumerate(sizes):
        logits = synth.decode_logits(800 + i, T, E)
        xb = synth.activations_bf16(800 + i, T, H)
        gids = torch.empty((T, k), dtype=torch.int32, device="cuda")
        gw = torch.empty((T, k), dtype=torch.float32, device="cuda")
        out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        ld, xd = _dev(logits), _bf16(xb)
        hip.moe_decode_fp8(ld, xd, addrs, k, hgeo, gids, gw, out, ws)
        runs.append((logits, xb, gids, gw, out, ld, xd))
    torch.cuda.synchronize()
    for i, (logits, xb, gids, gw, out, _, _) in enumerate(runs):
        want_ids, want_w, want = oracle.moe_decode(logits, oracle.bf16_to_f32(xb), recs, k, geo)
        _check(gids.cpu().numpy(), gw.cpu().numpy(), out.float().cpu().numpy(), want_ids, want_w, want,
               f"step {i} (T={sizes[i]})")
    assert _status(hip) == hip.OK

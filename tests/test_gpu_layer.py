"""GPU parity of the whole decode MoE layer and its new parts through the C ABI, against the
oracle on the same seeded inputs: the bf16-weight GEMV (the router), the shared expert's
gated add, and oom_moe_layer_decode_fp8 (router GEMV, routed experts, shared expert, gate).

Bars: GEMV outputs to the reference's own GEMV gate (max |got - want| / sqrt(K) < 1e-5,
crates/oominf-cuda/tests/gemv.rs:171-181) against the oracle; router ids bit-exact and
weights to fp32 rounding, both from the device's logits (the GEMV's summation order differs
from the oracle's, so a near tie could flip a pick: ids are pinned on the same logits);
bf16 outputs within rtol 2e-2 / atol 1e-3 of the oracle's fp32 layer on those logits; f32
outputs within 1e-4 of scale of it.
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


def _device_logits(hip, xd, rw, gw, T, E, H):
    """The router logits and the shared gate logit as the layer computes them (the same
    GEMV kernel on the same operands), each GEMV on a workspace of its own."""
    import torch

    dlog = torch.empty((T, E), dtype=torch.float32, device="cuda")
    dgate = torch.empty((T, 1), dtype=torch.float32, device="cuda")
    for y, wb, n in ((dlog, rw, E), (dgate, gw, 1)):
        gws = torch.zeros(max(1, hip.gemv_bf16_workspace_size(T, n, H)), dtype=torch.uint8, device="cuda")
        hip.gemv_bf16(xd, _bf16(wb), y, gws)
    torch.cuda.synchronize()
    return dlog.cpu().numpy(), dgate.cpu().numpy()


def _upload(recs):
    import torch

    buf = torch.from_numpy(np.stack(recs)).cuda()
    addrs = torch.tensor([buf.data_ptr() + e * buf.shape[1] for e in range(len(recs))], dtype=torch.int64,
                         device="cuda")
    return buf, addrs


@pytest.mark.parametrize("T,N,K,xbf,ybf", [(1, 128, 4096, True, False), (16, 128, 4096, True, False),
                                            (4, 1, 4096, False, False), (3, 1000, 2560, False, True),
                                            (8, 640, 1536, True, True), (2, 256, 8192, True, False)])
def test_gemv_bf16_parity(hip, T, N, K, xbf, ybf):
    import torch

    print(f"case: gemv bf16 T={T} N={N} K={K} x={'bf16' if xbf else 'f32'} y={'bf16' if ybf else 'f32'}", flush=True)
    w = oracle.gaussian_bf16((N, K), 90 + N, 0.02)
    xb = synth.activations_bf16(91 + K, T, K)
    x = oracle.bf16_to_f32(xb)
    want = oracle.gemv_bf16(x, w)
    y = torch.empty((T, N), dtype=torch.bfloat16 if ybf else torch.float32, device="cuda")
    ws = torch.zeros(max(1, hip.gemv_bf16_workspace_size(T, N, K)), dtype=torch.uint8, device="cuda")
    for rep in range(2):  # the split-K tickets are reset by their user
        hip.gemv_bf16(_bf16(xb) if xbf else _dev(x), _bf16(w), y, ws)
        torch.cuda.synchronize()
        got = y.float().cpu().numpy()
        if ybf:
            bad = ~np.isclose(got, want, rtol=RTOL, atol=ATOL)
            assert not bad.any(), f"rep {rep}: {bad.sum()} outside"
        else:
            assert np.abs(got - want).max() / np.sqrt(K) < 1e-5, f"rep {rep}"


def test_gemv_bf16_batch_sizes_share_a_workspace(hip):
    """GEMVs of 16, 1, 4, 16 and 2 tokens over one N on one workspace, with no
    synchronisation between them: the split tickets sit where every T looks."""
    import torch

    N, K = 128, 4096
    w = oracle.gaussian_bf16((N, K), 97, 0.02)
    sizes = (16, 1, 4, 16, 2)
    ws = torch.zeros(max(1, max(hip.gemv_bf16_workspace_size(T, N, K) for T in sizes)), dtype=torch.uint8,
                     device="cuda")
    runs = []
    for i, T in enumerate(sizes):
        xb = synth.activations_bf16(970 + i, T, K)
        y = torch.empty((T, N), dtype=torch.float32, device="cuda")
        xd = _bf16(xb)
        hip.gemv_bf16(xd, _bf16(w), y, ws)
        runs.append((xb, xd, y))
    torch.cuda.synchronize()
    for i, (xb, _, y) in enumerate(runs):
        want = oracle.gemv_bf16(oracle.bf16_to_f32(xb), w)
        assert np.abs(y.cpu().numpy() - want).max() / np.sqrt(K) < 1e-5, f"call {i} (T={sizes[i]})"


def test_combine_shared_parity(hip):
    import torch

    print("case: combine shared", flush=True)
    rng = np.random.default_rng(5)
    T, H = 5, 4096 + 4
    routed = rng.standard_normal((T, H)).astype(np.float32)
    shared = rng.standard_normal((T, H)).astype(np.float32)
    gate = np.array([0.0, 3.5, -2.0, 40.0, -40.0], dtype=np.float32)
    want = oracle.moe_combine_shared(routed, shared, gate)
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    hip.moe_combine_shared(_dev(routed), _dev(shared), _dev(gate), out)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("T,E,k,H,I,SI,xf32", [
    (1, 128, 8, 4096, 1536, 1536, False),   # the benchmark's layer shape, one token (shared expert in the kernel)
    (1, 200, 6, 1024, 512, 512, False),     # one token, E > 128, k < 8: waves with only the shared rows
    (1, 64, 8, 2048, 1024, 2048, False),    # one token, a wider shared expert: its own launch
    (16, 128, 8, 4096, 1536, 1536, False),  # 16 tokens: the batch kernel with the shared expert as a plan entry
    (5, 200, 6, 1024, 512, 512, False),     # the same with E > 128 and 5 tokens
    (4, 64, 6, 1024, 512, 768, False),      # a shared expert wider than the routed ones
    (3, 16, 4, 256, 128, 256, True),        # f32 activations (the general one-launch kernel)
])
def test_layer_decode_matches_oracle(hip, T, E, k, H, I, SI, xf32):
    import torch

    print(f"case: layer decode T={T} E={E} k={k} H={H} I={I} SI={SI} x={'f32' if xf32 else 'bf16'}", flush=True)
    seed = 7000 + T + E + SI
    geo, sgeo = oracle.record_geometry(H, I), oracle.record_geometry(H, SI)
    rw = oracle.gaussian_bf16((E, H), oracle.seed(seed, 1), 0.02)
    gw = oracle.gaussian_bf16((1, H), oracle.seed(seed, 2), 0.02)
    xb = synth.activations_bf16(seed, T, H)
    x = oracle.bf16_to_f32(xb)
    # only the experts the oracle's logits route to carry weights (the others stay zero)
    ologits = oracle.gemv_bf16(x, rw)
    oids, _ = oracle.router_topk(ologits, k)
    recs = synth.expert_records(geo, seed, E, only=set(int(e) for e in np.unique(oids)))
    srec = synth.expert_records(sgeo, seed + 1, 1)[0]
    buf, addrs = _upload(recs)
    sbuf, saddr = _upload([srec])
    hgeo, hsgeo = hip.record_geometry(H, I), hip.record_geometry(H, SI)
    ws = torch.zeros(hip.moe_layer_decode_fp8_workspace_size(T, E, k, hgeo, hsgeo), dtype=torch.uint8, device="cuda")
    ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    xd = _dev(x) if xf32 else _bf16(xb)
    for odt in (torch.bfloat16, torch.float32, torch.bfloat16):  # repeated calls reuse the workspace
        out = torch.empty((T, H), dtype=odt, device="cuda")
        hip.moe_layer_decode_fp8(xd, _bf16(rw), addrs, k, hgeo, saddr, hsgeo, _bf16(gw), ids, w, out, ws)
        torch.cuda.synchronize()
        # the device's logits and gate sit in the workspace: recompute them the same way to
        # pin routing on the device's own numbers
        dlog_n, dgate_n = _device_logits(hip, xd, rw, gw, T, E, H)
        assert np.abs(dlog_n - ologits).max() / np.sqrt(H) < 1e-5
        assert np.abs(dgate_n - oracle.gemv_bf16(x, gw)).max() / np.sqrt(H) < 1e-5
        # (an expert the oracle's logits did not pick has a zero record on both sides)
        want_ids, want_w, routed = oracle.moe_decode(dlog_n, x, recs, k, geo)
        np.testing.assert_array_equal(ids.cpu().numpy(), want_ids)
        np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=2e-6)
        _, _, shared = oracle.moe_decode(dgate_n, x, [srec], 1, sgeo)
        want = oracle.moe_combine_shared(routed, shared, dgate_n)
        got = out.float().cpu().numpy()
        if odt == torch.bfloat16:
            bad = ~np.isclose(got, want, rtol=RTOL, atol=ATOL)
            assert not bad.any(), f"{bad.sum()} of {bad.size} outside rtol {RTOL} / atol {ATOL}; " \
                                  f"worst {np.abs(got - want)[bad].max():.3e}"
        else:
            assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max()


@pytest.mark.parametrize("SI", [768, 512])
def test_layer_batch_sizes_share_a_workspace(hip, SI):
    """Layer steps of 16, 1, 5, 16 and 2 tokens on one workspace made for 16, with no
    synchronisation between them (a decode batch that shrinks and grows); with SI = inter
    every step carries the shared expert inside its decode kernel (the one-token or the
    batch kernel)."""
    import torch

    E, k, H, I = 64, 8, 1024, 512
    geo, sgeo = oracle.record_geometry(H, I), oracle.record_geometry(H, SI)
    rw = oracle.gaussian_bf16((E, H), 981, 0.02)
    gw = oracle.gaussian_bf16((1, H), 982, 0.02)
    recs = synth.expert_records(geo, 983, E)
    srec = synth.expert_records(sgeo, 984, 1)[0]
    buf, addrs = _upload(recs)
    sbuf, saddr = _upload([srec])
    hgeo, hsgeo = hip.record_geometry(H, I), hip.record_geometry(H, SI)
    sizes = (16, 1, 5, 16, 2)
    ws = torch.zeros(hip.moe_layer_decode_fp8_workspace_size(16, E, k, hgeo, hsgeo), dtype=torch.uint8,
                     device="cuda")
    runs = []
    for i, T in enumerate(sizes):
        xb = synth.activations_bf16(990 + i, T, H)
        xd = _bf16(xb)
        ids = torch.empty((T, k), dtype=torch.int32, device="cuda")
        w = torch.empty((T, k), dtype=torch.float32, device="cuda")
        out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        hip.moe_layer_decode_fp8(xd, _bf16(rw), addrs, k, hgeo, saddr, hsgeo, _bf16(gw), ids, w, out, ws)
        runs.append((xb, xd, ids, w, out))
    torch.cuda.synchronize()
    for i, (xb, xd, ids, w, out) in enumerate(runs):
        T = sizes[i]
        x = oracle.bf16_to_f32(xb)
        dlog, dgate = _device_logits(hip, xd, rw, gw, T, E, H)
        want_ids, want_w, routed = oracle.moe_decode(dlog, x, recs, k, geo)
        np.testing.assert_array_equal(ids.cpu().numpy(), want_ids, err_msg=f"step {i} (T={T})")
        np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=2e-6, err_msg=f"step {i} (T={T})")
        _, _, shared = oracle.moe_decode(dgate, x, [srec], 1, sgeo)
        want = oracle.moe_combine_shared(routed, shared, dgate)
        bad = ~np.isclose(out.float().cpu().numpy(), want, rtol=RTOL, atol=ATOL)
        assert not bad.any(), f"step {i} (T={T}): {bad.sum()} of {bad.size} outside"

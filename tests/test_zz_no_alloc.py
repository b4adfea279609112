"""oom_moe_decode_fp8_noalloc (scratch in a device array, no caller workspace) against
oom_moe_decode_fp8 with a workspace, through the C ABI: two calls in a row, the second
smaller (fewer tokens, narrower widths), each bit for bit equal to the workspace entry
point on the same inputs (same kernels, deterministic), and router ids equal. A step
larger than the array is refused with OOM_ERR_WORKSPACE before anything launches."""
import ctypes

import numpy as np
import pytest

import oracle
import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import torch

    import homelab_amd

    homelab_amd.lib()
    torch.cuda.init()
    return homelab_amd


def _noalloc(hip, logits, x, addrs, k, hgeo, ids, w, out):
    T, E = logits.shape
    return hip.lib().oom_moe_decode_fp8_noalloc(
        hip._ptr(logits), hip._ptr(x), hip._dtype_code(x), hip._ptr(addrs), T, E, k, ctypes.byref(hgeo),
        hip._ptr(ids), hip._ptr(w), hip._ptr(out), hip._dtype_code(out), hip._stream())


def _case(hip, T, E, k, H, I, seed, zipf):
    import torch

    geo = oracle.record_geometry(H, I)
    logits = synth.decode_logits(seed, T, E, zipf)
    ids, _ = oracle.router_topk(logits, k)
    recs = synth.expert_records(geo, seed, E, only=set(int(e) for e in np.unique(ids)))
    xb = synth.activations_bf16(seed, T, H)
    buf = torch.from_numpy(np.stack(recs)).cuda()
    addrs = torch.tensor([buf.data_ptr() + e * buf.shape[1] for e in range(E)], dtype=torch.int64, device="cuda")
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    return hip.record_geometry(H, I), torch.from_numpy(logits).cuda(), x, buf, addrs


def test_noalloc_matches_workspace_entry(hip):
    import torch

    cases = [(16, 128, 8, 4096, 1536, 1.1),  # the batch-16 benchmark shape (two grid meetings)
             (1, 64, 8, 1024, 512, None)]    # then a smaller one-token step on the same array
    for n, (T, E, k, H, I, zipf) in enumerate(cases):
        print(f"case: noalloc call {n} T={T} E={E} k={k} H={H} I={I}", flush=True)
        hgeo, ld, x, buf, addrs = _case(hip, T, E, k, H, I, 8800 + n, zipf)
        assert hip.moe_decode_fp8_workspace_size(T, E, k, hgeo) <= hip.lib().oom_moe_decode_fp8_noalloc_max_bytes()
        ids_a = torch.empty((T, k), dtype=torch.int32, device="cuda")
        w_a = torch.empty((T, k), dtype=torch.float32, device="cuda")
        out_a = torch.full((T, H), float("nan"), dtype=torch.float32, device="cuda")
        rc = _noalloc(hip, ld, x, addrs, k, hgeo, ids_a, w_a, out_a)
        assert rc == hip.OK, hip.lib().oom_last_error().decode()
        ws = torch.zeros(hip.moe_decode_fp8_workspace_size(T, E, k, hgeo), dtype=torch.uint8, device="cuda")
        ids_b = torch.empty_like(ids_a)
        w_b = torch.empty_like(w_a)
        out_b = torch.full((T, H), float("nan"), dtype=torch.float32, device="cuda")
        hip.moe_decode_fp8(ld, x, addrs, k, hgeo, ids_b, w_b, out_b, ws)
        torch.cuda.synchronize()
        assert hip.status() == hip.OK
        np.testing.assert_array_equal(ids_a.cpu().numpy(), ids_b.cpu().numpy(), err_msg=f"call {n}: ids")
        np.testing.assert_array_equal(w_a.cpu().numpy().view(np.uint32), w_b.cpu().numpy().view(np.uint32),
                                      err_msg=f"call {n}: weights")
        a, b = out_a.cpu().numpy(), out_b.cpu().numpy()
        assert np.isfinite(a).all(), f"call {n}: non-finite output"
        diff = np.flatnonzero(a.view(np.uint32) != b.view(np.uint32))
        assert diff.size == 0, f"call {n}: {diff.size} of {a.size} outputs differ"


def test_noalloc_refuses_a_step_past_its_array(hip):
    import torch

    T, E, k, H, I = 64, 128, 8, 4096, 2048
    hgeo = hip.record_geometry(H, I)
    assert hip.moe_decode_fp8_workspace_size(T, E, k, hgeo) > hip.lib().oom_moe_decode_fp8_noalloc_max_bytes()
    d = torch.zeros(16, dtype=torch.float32, device="cuda")
    rc = _noalloc(hip, torch.zeros((T, E), device="cuda"), torch.zeros((T, H), dtype=torch.bfloat16, device="cuda"),
                  torch.zeros(E, dtype=torch.int64, device="cuda"), k, hgeo, d, d, d)
    assert rc == hip.ERR_WORKSPACE, rc
    assert "scratch" in hip.lib().oom_last_error().decode()

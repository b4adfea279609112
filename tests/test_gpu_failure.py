"""Kernel-side failure is reported through the C ABI (oom_status, oom_stream_sync).

The persistent decode kernels meet across the grid through bounded waits. Here the host
sets the wait limit to one poll (oom_set_wait_limit), so the waits give up at once: every
kernel still ends normally (all its accesses stay inside its buffers whatever the
timing), its outputs are invalid, and the next sync point must say so. With the default
limit restored, the next call on the same workspace must match the oracle again (the
barrier words are consistent after a call whose waits gave up) and report OK.

Cases: the one-token FP8 kernel, the 2..16-token FP8 kernel (two grid meetings) and the
one-token NVFP4 kernel, each at its benchmark shape, where phase 1 lasts tens of
microseconds, so early blocks certainly poll before the last block arrives.
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
    yield homelab_amd
    homelab_amd.set_wait_limit(0)


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


def _fail_then_recover(hip, run, check):
    import torch

    assert hip.status() == hip.OK, "the device status word was set before the test"
    hip.set_wait_limit(1)
    try:
        run()
    finally:
        hip.set_wait_limit(0)
    rc = hip.status()
    assert rc == hip.ERR_KERNEL, f"oom_status returned {rc} after waits limited to one poll"
    assert hip.status() == hip.OK, "oom_status did not clear the word"
    # the sync point reports it too
    hip.set_wait_limit(1)
    try:
        run()
    finally:
        hip.set_wait_limit(0)
    with pytest.raises(hip.OomError, match="status -4"):
        hip.check(hip.lib().oom_stream_sync(hip._stream()))
    # default limit: the same workspace serves a correct call
    run()
    torch.cuda.synchronize()
    assert hip.status() == hip.OK
    check()


@pytest.mark.parametrize("T", [1, 16])
def test_fp8_decode_reports_a_wait_that_gave_up(hip, T):
    import torch

    print(f"case: fp8 decode failure path T={T}", flush=True)
    E, k, H, I = 128, 8, 4096, 1536
    geo = oracle.record_geometry(H, I)
    logits = synth.decode_logits(4100 + T, T, E, 1.1 if T > 1 else None)
    ids, _ = oracle.router_topk(logits, k)
    recs = synth.expert_records(geo, 4100 + T, E, only=set(int(e) for e in np.unique(ids)))
    xb = synth.activations_bf16(4100 + T, T, H)
    want_ids, want_w, want = oracle.moe_decode(logits, oracle.bf16_to_f32(xb), recs, k, geo)
    hgeo = hip.record_geometry(H, I)
    buf, addrs = _upload(recs)
    ws = torch.zeros(hip.moe_decode_fp8_workspace_size(T, E, k, hgeo), dtype=torch.uint8, device="cuda")
    gids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    gw = torch.empty((T, k), dtype=torch.float32, device="cuda")
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    x, ld = _bf16(xb), _dev(logits)

    def run():
        hip.moe_decode_fp8(ld, x, addrs, k, hgeo, gids, gw, out, ws)

    def check():
        np.testing.assert_array_equal(gids.cpu().numpy(), want_ids)
        got = out.float().cpu().numpy()
        assert np.allclose(got, want, rtol=RTOL, atol=ATOL), "output after recovery outside the bar"

    _fail_then_recover(hip, run, check)


def test_nvfp4_decode_reports_a_wait_that_gave_up(hip):
    import torch

    print("case: nvfp4 one-token decode failure path", flush=True)
    E, k, H, I = 512, 10, 2560, 640
    geo = oracle.nvfp4_geometry(H, I)
    logits = synth.decode_logits(4200, 1, E)
    ids, _ = oracle.router_topk(logits, k)
    recs = synth.nvfp4_records(geo, 4200, E, only=set(int(e) for e in np.unique(ids)))
    xb = synth.activations_bf16(4200, 1, H)
    want_ids, want_w, want = oracle.moe_decode_nvfp4(logits, oracle.bf16_to_f32(xb), recs, k, geo)
    hgeo = hip.nvfp4_geometry(H, I)
    buf, addrs = _upload(recs)
    ws = torch.zeros(hip.moe_decode_nvfp4_workspace_size(1, E, k, hgeo), dtype=torch.uint8, device="cuda")
    gids = torch.empty((1, k), dtype=torch.int32, device="cuda")
    gw = torch.empty((1, k), dtype=torch.float32, device="cuda")
    out = torch.empty((1, H), dtype=torch.bfloat16, device="cuda")
    x, ld = _bf16(xb), _dev(logits)

    def run():
        hip.moe_decode_nvfp4(ld, x, addrs, k, hgeo, gids, gw, out, ws)

    def check():
        np.testing.assert_array_equal(gids.cpu().numpy(), want_ids)
        got = out.float().cpu().numpy()
        assert np.allclose(got, want, rtol=RTOL, atol=ATOL), "output after recovery outside the bar"

    _fail_then_recover(hip, run, check)

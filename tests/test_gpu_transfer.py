"""Copies beside compute (the Transfer trait, crates/oominf-core/src/backend.rs:945-1018):
host-tier expert records staged into device slots on a copy queue, ordered against the
decode step with events. Checked: every slot holds its host record byte for byte; the
step over the slots gives the same output as resident records, bit for bit, and the
oracle's output (moe_decode on the host records) within 2e-5 of scale; downloads queued
after compute (the output, and the router ids as download_start_i32 / download_wait_i32
take them, backend.rs:984-993) land in pinned host memory when their event completes."""
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


@pytest.mark.parametrize("E,k,H,I", [(64, 8, 1024, 512), (16, 4, 256, 128)])
def test_staged_records_match_resident(hip, E, k, H, I):
    import torch

    print(f"case: transfer E={E} k={k} H={H} I={I}", flush=True)
    seed = 7100 + E + H
    geo = oracle.record_geometry(H, I)
    hgeo = hip.record_geometry(H, I)
    logits = synth.decode_logits(seed, 1, E)
    ids, _ = oracle.router_topk(logits, k)
    recs = synth.expert_records(geo, seed, E, only=set(int(e) for e in ids[0]))
    stride = recs[0].size
    # resident: every record in device memory
    buf = torch.from_numpy(np.stack(recs)).cuda()
    addrs = torch.tensor([buf.data_ptr() + e * stride for e in range(E)], dtype=torch.int64, device="cuda")
    ld = torch.from_numpy(logits).cuda()
    xb = synth.activations_bf16(seed, 1, H)
    xd = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    ws = torch.zeros(hip.moe_decode_fp8_workspace_size(1, E, k, hgeo), dtype=torch.uint8, device="cuda")
    gids = torch.empty((1, k), dtype=torch.int32, device="cuda")
    gw = torch.empty((1, k), dtype=torch.float32, device="cuda")
    want = torch.empty((1, H), dtype=torch.float32, device="cuda")
    hip.moe_decode_fp8(ld, xd, addrs, k, hgeo, gids, gw, want, ws)
    torch.cuda.synchronize()
    want = want.cpu().numpy()
    want_ids, _, want_or = oracle.moe_decode(logits, oracle.bf16_to_f32(xb), recs, k, geo)
    # host tier: all records in pinned host memory; k device slots
    host = hip.PinnedHost(E * stride)
    host.array()[:] = np.stack(recs).reshape(-1)
    slots = torch.zeros((k, stride), dtype=torch.uint8, device="cuda")
    q, copied, computed = hip.CopyQueue(), hip.Event(), hip.Event()
    try:
        for rep in range(2):
            # the routed experts' records to slots on the copy queue (after the previous
            # step's compute, which read the slots), then compute waits for the copies
            computed.record()
            computed.wait_on(q)
            routed = [int(e) for e in ids[0]]
            order = routed if rep == 0 else routed[::-1]
            dst = [slots.data_ptr() + i * stride for i in range(k)]
            q.copy_records(dst, [host.ptr + e * stride for e in order], stride)
            copied.record(q)
            copied.wait_on(None)
            # the slots hold the host records, byte for byte
            copied.wait()
            for i, e in enumerate(order):
                assert np.array_equal(slots[i].cpu().numpy(), recs[e]), f"rep {rep}: slot {i} != record {e}"
            table = np.full(E, dst[0], dtype=np.int64)
            for i, e in enumerate(order):
                table[e] = dst[i]
            out = torch.full((1, H), float("nan"), dtype=torch.float32, device="cuda")
            hip.moe_decode_fp8(ld, xd, torch.from_numpy(table).cuda(), k, hgeo, gids, gw, out, ws)
            # the output downloads after the step, into pinned host memory
            dl = hip.PinnedHost(H * 4)
            done = hip.Event()
            hip.download_async(dl.ptr, out, H * 4)
            done.record()
            done.wait()
            assert done.done()
            got = dl.array("float32").copy()
            dl.close()
            done.close()
            # the ids as download_start_i32 / download_wait_i32 take them: a download after
            # the compute issued so far into pinned memory, then a wait on its event
            dli = hip.PinnedHost(k * 4)
            done_i = hip.Event()
            hip.download_async(dli.ptr, gids, k * 4)
            done_i.record()
            done_i.wait()
            got_ids = dli.array("int32").copy()
            dli.close()
            done_i.close()
            np.testing.assert_array_equal(got_ids, want_ids.reshape(-1), err_msg=f"rep {rep}: downloaded ids")
            np.testing.assert_array_equal(gids.cpu().numpy(), ids, err_msg=f"rep {rep}")
            diff = np.flatnonzero(got.view(np.uint32) != want.reshape(-1).view(np.uint32))
            assert diff.size == 0, f"rep {rep}: {diff.size} of {H} differ"
            err = np.abs(got - want_or.reshape(-1)).max()
            assert err <= 2e-5 * np.abs(want_or).max(), f"rep {rep}: staged output vs oracle: {err:.3e}"
        # a device-to-device copy on the queue
        moved = torch.zeros(stride, dtype=torch.uint8, device="cuda")
        q.copy_on_device(moved.data_ptr(), slots.data_ptr(), stride)
        q.sync()
        assert torch.equal(moved, slots[0])
    finally:
        q.close()
        copied.close()
        computed.close()
        host.close()

"""GPU parity of paged GQA decode attention (oom_attn_decode_paged) through the C ABI.

Bars: the fp32 output is within max abs 1e-4 of a float64 softmax reference, the
reference's own gate for its fp32 attention path (crates/oominf-cuda/tests/kv_cache.rs:206-305),
and of the oracle (oracle/paths.c, the reference's attn_prefill arithmetic); the bf16
output is within rtol 2e-2 / atol 1e-3 of the oracle's fp32 result.
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


def run(hip, q, k, v, table, kv_len, scale, out_dtype):
    import torch

    H, D = q.shape
    Hkv = k.shape[2]
    qd = torch.from_numpy(q.view(np.int16)).view(torch.bfloat16).cuda() if q.dtype == np.uint16 else \
        torch.from_numpy(q).cuda()
    kd = torch.from_numpy(k.view(np.int16)).view(torch.bfloat16).cuda()
    vd = torch.from_numpy(v.view(np.int16)).view(torch.bfloat16).cuda()
    td = torch.from_numpy(table).cuda()
    out = torch.empty((H, D), dtype=out_dtype, device="cuda")
    ws = torch.zeros(hip.attn_decode_workspace_size(kv_len, H, Hkv, D), dtype=torch.uint8, device="cuda")
    hip.attn_decode_paged(qd, kd, vd, td, kv_len, scale, out, ws)
    # a second call on the same workspace (tickets reset by their users) gives the same bits
    out2 = torch.empty_like(out)
    hip.attn_decode_paged(qd, kd, vd, td, kv_len, scale, out2, ws)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    return out.float().cpu().numpy()


CASES = [
    # H, Hkv, D, kv_len, page, q dtype
    (64, 8, 128, 32768, 16, "bf16"),  # the decode shape: 64 heads, 8 KV heads, 32768 keys
    (64, 8, 128, 1000, 16, "bf16"),
    (8, 1, 128, 1, 16, "bf16"),
    (8, 1, 128, 17, 16, "f32"),
    (16, 4, 128, 513, 32, "bf16"),
    (4, 4, 128, 300, 16, "f32"),      # one query head per KV head
    (24, 4, 128, 2100, 16, "bf16"),   # six query heads per KV head
    (8, 2, 128, 4097, 64, "f32"),
    (8, 1, 128, 32769, 16, "f32"),    # 33 partials a KV head (1024 keys a block)
    (16, 2, 128, 70000, 16, "bf16"),  # 69 partials a KV head
    (8, 1, 128, 131073, 16, "f32"),   # 129 partials: the merge's loop past its one-round 128
    (8, 1, 128, 280000, 16, "bf16"),  # 274 partials, three rounds of the merge's loop
]


@pytest.mark.parametrize("H,Hkv,D,kv_len,page,qdt", CASES)
def test_attention_decode_parity(hip, H, Hkv, D, kv_len, page, qdt):
    import torch

    print(f"attention case H={H} Hkv={Hkv} D={D} kv_len={kv_len} page={page} q={qdt}", flush=True)
    q, k, v, table = synth.paged_attention_case(11 + kv_len, H, Hkv, D, kv_len, page)
    scale = 1.0 / np.sqrt(D)
    if qdt == "f32":
        qf = np.random.default_rng(kv_len).standard_normal((H, D)).astype(np.float32)
        qin = qf
    else:
        qf = oracle.bf16_to_f32(q)
        qin = q
    want64 = synth.f64_attention(qf, k, v, table, page, kv_len, H, Hkv, D, scale)
    got = run(hip, qin, k, v, table, kv_len, scale, torch.float32)
    assert np.abs(got - want64).max() < 1e-4, np.abs(got - want64).max()
    if qdt == "bf16":
        ref = oracle.attn_decode_paged(q, k, v, table, page, kv_len, H, Hkv, D, scale)
        assert np.abs(got - ref).max() < 1e-4
        got16 = run(hip, qin, k, v, table, kv_len, scale, torch.bfloat16)
        bad = ~np.isclose(got16, ref, rtol=RTOL, atol=ATOL)
        assert not bad.any(), f"{bad.sum()} bf16 outputs outside rtol {RTOL} / atol {ATOL}"


def test_attention_convex_and_page_order(hip):
    import torch

    H, Hkv, D, kv_len = 64, 8, 128, 5000
    q, k, v, table = synth.paged_attention_case(3, H, Hkv, D, kv_len)
    got = run(hip, q, k, v, table, kv_len, 0.2, torch.float32)
    vf = oracle.bf16_to_f32(v)
    j = np.arange(kv_len)
    for h in range(H):
        rows = vf[table[j // 16], h // 8, j % 16]
        assert np.all(got[h] <= rows.max(0) + 1e-5) and np.all(got[h] >= rows.min(0) - 1e-5)
    # the same logical cache under another physical page order reads the same bits
    perm = np.random.default_rng(5).permutation(k.shape[0]).astype(np.int32)
    k2, v2 = np.empty_like(k), np.empty_like(v)
    k2[perm] = k
    v2[perm] = v
    got2 = run(hip, q, k2, v2, perm[table].astype(np.int32), kv_len, 0.2, torch.float32)
    np.testing.assert_array_equal(got, got2)


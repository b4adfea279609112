"""GPU parity of the bf16-record routed experts (oom_moe_gate_up_bf16, oom_moe_down_bf16)
through the C ABI, against the oracle (oracle/bf16rec.c, pinned in tests/test_oracle_bf16.py).

Bar: h and y within 1e-5 of the oracle's largest magnitude (fp32 products and sums; only
the summation order differs), x in f32 and in bf16, at the decode shape (hidden 4096,
inter 1536, eight experts, 1 to 16 tokens) and at small, ragged widths (multiples of 8,
partial 512-column chunks), with an expert that has no assignment."""
import numpy as np
import pytest

import oracle
from test_oracle_bf16 import bf16_records

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import torch

    import homelab_amd

    homelab_amd.lib()
    torch.cuda.init()
    return homelab_amd


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("H,I,E,T,k,xbf", [(4096, 1536, 8, 1, 8, True), (4096, 1536, 8, 16, 8, False),
                                           (4096, 1536, 8, 4, 4, True), (520, 136, 5, 3, 2, False),
                                           (104, 40, 3, 2, 2, True), (2560, 640, 6, 7, 3, False)])
def test_bf16_experts_match_oracle(hip, H, I, E, T, k, xbf):
    import torch

    print(f"case: bf16 experts H={H} I={I} E={E} T={T} k={k} x={'bf16' if xbf else 'f32'}", flush=True)
    geo = oracle.bf16_geometry(H, I)
    hgeo = hip.bf16_geometry(H, I)
    assert [getattr(hgeo, f) for f, _ in hgeo._fields_] == [getattr(geo, f) for f, _ in geo._fields_]
    recs = bf16_records(geo, E, H * 3 + I)
    rng = np.random.default_rng(T * 7 + E)
    # every token picks k distinct experts; expert E - 1 is never picked (an empty run)
    picks = np.stack([rng.choice(E - 1, size=min(k, E - 1), replace=False) for _ in range(T)])
    A = picks.size
    order = np.argsort(picks.reshape(-1), kind="stable")
    tok = (order // picks.shape[1]).astype(np.int32)
    counts = np.bincount(picks.reshape(-1), minlength=E)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    xf = rng.standard_normal((T, H)).astype(np.float32)
    if xbf:
        xb = oracle.bf16_from_f32(xf)
        x_host = oracle.bf16_to_f32(xb)
        x_dev = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    else:
        x_host, x_dev = xf, dev(xf)
    h_want = oracle.moe_gate_up_bf16(recs, off, tok, x_host, geo)
    buf = dev(np.stack(recs))
    addrs = torch.tensor([buf.data_ptr() + e * buf.shape[1] for e in range(E)], dtype=torch.int64, device="cuda")
    h = torch.full((A, I), np.nan, dtype=torch.float32, device="cuda")
    hip.moe_gate_up_bf16(addrs, dev(off), dev(tok), E, x_dev, h, hgeo)
    torch.cuda.synchronize()
    hg = h.cpu().numpy()
    assert np.abs(hg - h_want).max() <= 1e-5 * np.abs(h_want).max(), np.abs(hg - h_want).max()
    y_want = oracle.moe_down_bf16(recs, off, h_want, geo)
    y = torch.full((A, H), np.nan, dtype=torch.float32, device="cuda")
    hip.moe_down_bf16(addrs, dev(off), E, dev(h_want), y, hgeo)
    torch.cuda.synchronize()
    yg = y.cpu().numpy()
    assert np.abs(yg - y_want).max() <= 1e-5 * np.abs(y_want).max(), np.abs(yg - y_want).max()


def test_bf16_experts_reject_bad_shapes(hip):
    import torch

    z = torch.zeros(16, dtype=torch.int64, device="cuda")
    f = torch.zeros((1, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(hip.OomError, match="multiples of 8"):
        hip.moe_gate_up_bf16(z, z, z, 1, f, f, hip.Bf16Record(60, 64, 0, 8192, 16384))
    with pytest.raises(hip.OomError, match="up to 4096"):
        hip.moe_down_bf16(z, z, 1, f, f, hip.bf16_geometry(8192, 64))

"""GPU parity of the tiled NVFP4 grouped GEMM (oom_moe_tiled_nvfp4) and the SwiGLU range
(oom_moe_swiglu_range) through the C ABI.

Bar, as the reference's own test (crates/oominf-cuda/tests/moe_tiled.rs:176-226): at its
three shapes (partial tiles both ways and an empty expert; gate 640 x 2560 and down
2560 x 640) and both precisions, worst |y - f64| / sum |x w| below 2e-6, where the f64
evaluation takes x exact (OOM_EXPERT_EXACT) or rounded to bf16 (OOM_EXPERT_BF16); and the
same bar against the oracle's restatement. SwiGLU against numpy in f64 within 2 ulp.
"""
import numpy as np
import pytest

import oracle
from tiled_cases import SHAPES, case, f64_eval

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import torch

    import homelab_amd

    homelab_amd.lib()  # raises if the library is missing: no fallback
    torch.cuda.init()
    return homelab_amd


def run_tiled(hip, recs, x, off, rows, precision):
    import torch

    buf = torch.from_numpy(np.stack(recs.recs)).cuda()
    addrs = torch.tensor([buf.data_ptr() + e * recs.stride for e in range(len(recs.recs))], dtype=torch.int64,
                         device="cuda")
    A = int(off[-1])
    y = torch.full((max(A, 1), recs.n), float("nan"), dtype=torch.float32, device="cuda")
    rd = None if rows is None else torch.from_numpy(rows).cuda()
    max_n = int(np.diff(off).max())
    hip.moe_tiled_nvfp4(addrs, torch.from_numpy(off).cuda(), rd, len(recs.recs), max_n, torch.from_numpy(x).cuda(), y,
                        recs.n, recs.k, recs.w_off, recs.s_off, 0, precision)
    torch.cuda.synchronize()
    return y.cpu().numpy()[:A]


@pytest.mark.parametrize("n,k,counts", SHAPES)
@pytest.mark.parametrize("exact", [True, False])
def test_tiled_matches_f64_and_oracle(hip, n, k, counts, exact):
    print(f"case: moe_tiled_nvfp4 n={n} k={k} counts={counts} exact={exact}", flush=True)
    recs, x, off, rows = case(n, k, counts, seed=n * 31 + k)
    prec = hip.EXPERT_EXACT if exact else hip.EXPERT_BF16
    got = run_tiled(hip, recs, x, off, rows, prec)
    ref, mag = f64_eval(recs, x, off, rows, exact)
    tiny = np.finfo(np.float64).tiny
    worst = (np.abs(got - ref) / np.maximum(mag, tiny)).max()
    assert worst < 2e-6, f"worst error / sum|x*w| = {worst:.3e}"
    want = oracle.moe_tiled_nvfp4(recs.recs, off, rows, x, n, k, recs.w_off, recs.s_off, 0, 3 if exact else 1)
    assert (np.abs(got - want) / np.maximum(mag, tiny)).max() < 2e-6
    # a second call gives the same bits
    np.testing.assert_array_equal(run_tiled(hip, recs, x, off, rows, prec), got)


def test_tiled_without_rows(hip):
    recs, x, off, _ = case(136, 64, [7, 0, 12], seed=3, tokens=19)
    got = run_tiled(hip, recs, x, off, None, hip.EXPERT_EXACT)
    ref, mag = f64_eval(recs, x, off, np.arange(19, dtype=np.int32), True)
    assert (np.abs(got - ref) / mag).max() < 2e-6


def test_tiled_rejects_bad_arguments(hip):
    import torch

    z = torch.zeros(64, dtype=torch.float32, device="cuda")
    i = torch.zeros(4, dtype=torch.int32, device="cuda")
    with pytest.raises(hip.OomError, match="multiple of 32"):
        hip.moe_tiled_nvfp4(i, i, None, 1, 4, z, z, 16, 48, 64, 0, 0)
    with pytest.raises(hip.OomError, match="precision"):
        hip.moe_tiled_nvfp4(i, i, None, 1, 4, z, z, 16, 64, 64, 0, 0, precision=7)


def test_swiglu_range(hip):
    import torch

    rng = np.random.default_rng(4)
    g = (rng.standard_normal(10007) * 6).astype(np.float32)
    u = rng.standard_normal(10007).astype(np.float32)
    h = torch.full((10007,), -9.0, dtype=torch.float32, device="cuda")
    hip.moe_swiglu_range(torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda(), h, 13, 9001)
    torch.cuda.synchronize()
    got = h.cpu().numpy()
    want = (g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))) * u
    assert np.all(got[:13] == -9.0) and np.all(got[9001:] == -9.0)
    np.testing.assert_allclose(got[13:9001], want[13:9001], rtol=4e-7, atol=1e-30)

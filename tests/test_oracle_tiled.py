"""The oracle's restatement of the tiled NVFP4 GEMM (oracle_moe_tiled_nvfp4) against the f64
evaluation the reference's own test holds it to (crates/oominf-cuda/tests/moe_tiled.rs:176-214):
worst |y - f64| / sum |x w| below 2e-6, x exact (three terms) or rounded to bf16 (one)."""
import numpy as np
import pytest

import oracle
from tiled_cases import case, f64_eval


@pytest.mark.parametrize("terms", [3, 1])
def test_oracle_tiled_matches_f64(terms):
    recs, x, off, rows = case(200, 96, [1, 0, 37, 70], seed=5)
    y = oracle.moe_tiled_nvfp4(recs.recs, off, rows, x, recs.n, recs.k, recs.w_off, recs.s_off, 0, terms)
    ref, mag = f64_eval(recs, x, off, rows, exact=terms == 3)
    worst = (np.abs(y - ref) / np.maximum(mag, np.finfo(np.float64).tiny)).max()
    assert worst < 2e-6, worst
    if terms == 1:
        # the bf16 arithmetic differs from the exact one by the activation rounding
        exact, _ = f64_eval(recs, x, off, rows, exact=True)
        assert np.abs(y - exact).max() > 1e-4 * np.abs(exact).max()


def test_oracle_tiled_rows_default_to_assignment():
    recs, x, off, _ = case(64, 64, [5, 3], seed=9, tokens=8)
    y = oracle.moe_tiled_nvfp4(recs.recs, off, None, x, recs.n, recs.k, recs.w_off, recs.s_off, 0, 3)
    ref, mag = f64_eval(recs, x, off, np.arange(8, dtype=np.int32), exact=True)
    assert (np.abs(y - ref) / mag).max() < 2e-6

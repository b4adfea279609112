"""Writes the golden fixtures of this folder.

known_answers.json holds the known-answer vectors the reference's own tests fix
for this path (inputs and expected outputs, with the test each comes from), plus
small seeded cases whose expected outputs are evaluated here in float64 from the
format definition (torch's float8_e4m3fn decode), independently of the oracle.

Run from the repository root: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))


def e4m3_values_torch(codes):
    import torch

    return torch.tensor(codes, dtype=torch.uint8).view(torch.float8_e4m3fn).float().tolist()


def main():
    out = {}
    # crates/oominf-core/src/fp8.rs:110-122 (rounds_to_nearest_even_and_saturates).
    out["e4m3_encode"] = {
        "source": "crates/oominf-core/src/fp8.rs:110-122",
        "cases": [[1.0625, 0x38], [1.07, 0x39], [1000.0, 0x7E], [-1000.0, 0xFE], [2.0 ** -9, 0x01],
                  [2.0 ** -10, 0x00], [float(np.float32(2.0 ** -6) * np.float32(0.99)), 0x08]],
    }
    # crates/oominf-cpu/src/kernel.rs:530-539 (e4m3_decodes_known_values); NaN as null.
    out["e4m3_decode"] = {
        "source": "crates/oominf-cpu/src/kernel.rs:530-539",
        "cases": [[0x00, 0.0], [0x38, 1.0], [0x7E, 448.0], [0x01, 2.0 ** -9], [0xB8, -1.0], [0x7F, None]],
    }
    # crates/oominf-metal/src/tests.rs:503-525: every code through an FP8 GEMV with x = 1,
    # scale 1, K = 1 reads back as its value (NaN for 0x7f and 0xff).
    vals = e4m3_values_torch(list(range(256)))
    out["e4m3_all_codes"] = {
        "source": "crates/oominf-metal/src/tests.rs:503-525",
        "values": [None if math.isnan(v) else v for v in vals],
    }
    # crates/oominf-core/src/fp8.rs:124-138 (blocks_scale_to_448): two rows of 130 with
    # 1.0, -2.0 at columns 0, 1 and 0.5 at column 128 of row 0.
    out["quantize_blocks"] = {
        "source": "crates/oominf-core/src/fp8.rs:124-138",
        "k": 130, "n": 2, "nonzero": [[0, 0, 1.0], [0, 1, -2.0], [0, 128, 0.5]],
        "scales": [2.0 / 448.0, 0.5 / 448.0, 1.0, 1.0],
        "decoded": [[0, 1, -2.0], [0, 128, 0.5]],
    }
    # crates/oominf-metal/src/tests.rs:183-212: k = 130 (partial second scale block),
    # codes i % 256 with 0x7f-class codes stepped down, scales [0.25, 2, 1, 0.5].
    k = 130
    x = [(i - 65.0) / 128.0 for i in range(k)]
    packed = [((i % 256) - 1) if (i % 256) & 0x7F == 0x7F else (i % 256) for i in range(2 * k)]
    scales = [0.25, 2.0, 1.0, 0.5]
    w = e4m3_values_torch(packed)
    want = [sum(x[c] * w[r * k + c] * scales[r * 2 + c // 128] for c in range(k)) for r in range(2)]
    out["fp8_gemv_partial_blocks"] = {
        "source": "crates/oominf-metal/src/tests.rs:183-212",
        "k": k, "n": 2, "x": x, "q": packed, "scale_1x128": scales, "y": want, "tol": 1e-4,
    }
    # crates/oominf-cpu/src/lib.rs:446-494 (swiglu_expert_on_a_known_record): hidden 32,
    # inter 16, every weight 1.0, x[i] = (i % 7) * 0.01 over two tokens, jobs' tokens
    # [1, 0]: every output of token t is silu(s) * s * inter with s = sum(x_t).
    hidden, inter = 32, 16
    xs = [(i % 7) * 0.01 for i in range(2 * hidden)]
    ys = []
    for t in [1, 0]:
        s = float(np.sum(np.array(xs[t * hidden:(t + 1) * hidden], dtype=np.float32)))
        ys.append(s / (1.0 + math.exp(-s)) * s * inter)
    out["expert_known_record"] = {
        "source": "crates/oominf-cpu/src/lib.rs:446-494",
        "hidden": hidden, "inter": inter, "x": xs, "tokens": [1, 0], "y_per_token": ys, "rtol": 1e-4,
    }
    # crates/oominf-metal/src/tests.rs:239-270 (nvfp4_gemm_matches_cpu_reference_with_signs_and_scales):
    # 2 tokens x 3 rows x 32 columns, x[i] = (i - 31) / 17, packed byte i = (13 i) % 256,
    # scale bytes [0x38, 0x30, 0x40, 0x38, 0x28, 0x40] whose values the test states as
    # [1, 0.5, 2, 1, 0.25, 2], scale_2 = 0.75, E2M1 values by code as listed there;
    # y = sum_c x * code * scale * 0.75 (tolerance 1e-4).
    e2m1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    vals = [(i - 31.0) / 17.0 for i in range(64)]
    packed4 = [(i * 13) % 256 for i in range(48)]
    sbytes = [0x38, 0x30, 0x40, 0x38, 0x28, 0x40]
    svals = [1.0, 0.5, 2.0, 1.0, 0.25, 2.0]
    y4 = []
    for token in range(2):
        for row in range(3):
            acc = 0.0
            for c in range(32):
                nib = (packed4[row * 16 + c // 2] >> ((c % 2) * 4)) & 15
                acc += float(np.float32(vals[token * 32 + c])) * e2m1[nib] * svals[row * 2 + c // 16] * 0.75
            y4.append(acc)
    out["nvfp4_rows_known_answer"] = {
        "source": "crates/oominf-metal/src/tests.rs:239-270",
        "tokens": 2, "rows": 3, "cols": 32, "x": vals, "packed": packed4, "scales": sbytes,
        "scale_values": svals, "scale2": 0.75, "e2m1": e2m1, "y": y4, "tol": 1e-4,
    }
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", os.path.join(HERE, "known_answers.json"))


if __name__ == "__main__":
    main()

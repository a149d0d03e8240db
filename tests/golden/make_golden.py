"""Regenerate tests/golden/w4a16_cases.npz from the pinned oracle.

    python tests/golden/make_golden.py

The reference ships no golden vectors (its tests are generative: seeded
randn plus its fp32 oracle). These fixtures are written by oracle/oracle.py
after it has been pinned by the known-answer and closed-form checks in
tests/test_oracle.py, and cross-checked here against the independent scalar C
restatement before anything is written. They freeze inputs, packed words,
scales and float64 outputs for small shapes, including the edge shapes the
kernels must handle (one group, ragged M, K not a power of two, B > 16).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import c_oracle, oracle  # noqa: E402

# (name, M, K, B, seed, w_std)
CASES = [
    ("one_group", 4, 128, 1, 11, 0.05),
    ("ragged_m", 37, 256, 2, 12, 0.02),
    ("k_not_pow2", 24, 384, 3, 13, 0.02),
    ("batch_17", 16, 256, 17, 14, 0.05),
    ("square_small", 64, 512, 4, 15, 0.02),
]


def main() -> None:
    out = {}
    for name, m, k, b, seed, std in CASES:
        w, x = oracle.make_case(m, k, b, seed, std)
        packed, scales = oracle.quantize_and_pack(w)
        cp, cs = c_oracle.quantize_and_pack(w)
        assert np.array_equal(packed, cp), name
        assert np.array_equal(scales.view(np.uint16), cs.view(np.uint16)), name
        y = oracle.linear_f64(x, packed, scales)
        assert np.allclose(y, c_oracle.gemv_f64(x, packed, scales), rtol=0, atol=1e-12), name
        out[f"{name}/w"] = w
        out[f"{name}/x"] = x
        out[f"{name}/packed"] = packed
        out[f"{name}/scales"] = scales
        out[f"{name}/y"] = y
    np.savez_compressed(HERE / "w4a16_cases.npz", **out)
    print(f"wrote {HERE / 'w4a16_cases.npz'} ({len(CASES)} cases)")


if __name__ == "__main__":
    main()

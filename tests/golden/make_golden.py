"""Writes tests/golden/sweep_oracle.json: the oracle's outputs on the reference's
GPU-parity sweep (crates/staleynet-cuda/tests/kernels_match_reference.rs:54-91).

For every case (sizes x batch {1, 3} x {NN, TN, NT, TT}, scale 0.7,
accumulate onto LCG values, inputs from the test's LCG with seeds 1/2/3) it
records the SHA-256 of the output's little-endian f32 bytes and its first
eight values. The reference is Rust and cannot be run here; these vectors
pin the oracle against regressions and let the GPU tests check that the
oracle they run on the box is the one that produced them.

Run: python tests/golden/make_golden.py  (after `make -C oracle`).
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle  # noqa: E402

SIZES = [(1, 1, 1), (17, 33, 9), (64, 48, 70), (5, 129, 31), (130, 197, 100)]
VARIANTS = [("NN", False, False), ("TN", True, False), ("NT", False, True), ("TT", True, True)]


def sweep_cases():
    for rows, cols, inner in SIZES:
        for batch in (1, 3):
            for name, lt, rt in VARIANTS:
                yield dict(rows=rows, cols=cols, inner=inner, batch=batch, variant=name, left_t=lt, right_t=rt)


def oracle_output(case):
    rows, cols, inner, batch = case["rows"], case["cols"], case["inner"], case["batch"]
    left = oracle.random_values(batch * rows * inner, 1)
    right = oracle.random_values(batch * inner * cols, 2)
    out = oracle.random_values(batch * rows * cols, 3)
    p = oracle.Product(rows, cols, inner, case["left_t"], case["right_t"], batch, rows * inner, inner * cols,
                       rows * cols, 0.7, True)
    oracle.matmul(p, left, right, out)
    return out


def main():
    records = []
    for case in sweep_cases():
        out = oracle_output(case)
        records.append({**case, "sha256": hashlib.sha256(out.astype("<f4").tobytes()).hexdigest(),
                        "first": [float(v) for v in out[:8]]})
    path = os.path.join(HERE, "sweep_oracle.json")
    with open(path, "w") as f:
        json.dump({"_source": __doc__.strip().splitlines()[0], "cases": records}, f, indent=1)
    print(f"wrote {len(records)} cases to {path}")


if __name__ == "__main__":
    main()

"""GPU tests of the decode kernel's split-K hand-off (few-row products whose K is split into slices:
every slice but the last writes its partial sums into zeroed slots, and the last slice polls them,
adds them in slice order and clears them).

- Back-to-back products of different shapes reuse the same slots, so each call's clearing is what
  the next call's polling relies on. Each result is checked against the oracle (the reference's
  loop, crates/staleynet-cuda/src/reference.rs:19-38) at the fp32 tolerance, and reruns must give
  the same bits.
- NaN operands: the slots encode a partial as the NOT of its bits, with NaNs made canonical, so that
  no written slot reads as empty. A row of x holding NaNs, including the one bit pattern
  (0xFFFFFFFF) that would encode to an empty slot without that step, gives NaN in that row only.
  The call returns promptly, and the next call on clean inputs is correct.
"""
import time

import numpy as np
import pytest

from oracle import oracle
from staleynet_amd import gemm
from staleynet_amd.gemm import BatchStrides, MatmulSpec, Shape

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-5  # kernels_match_reference.rs:12

SPLIT_PRODUCTS = [
    MatmulSpec.new(1, 768, 768),                      # out: 12 column blocks, 6 slices
    MatmulSpec.new(1, 2304, 768).scaled(0.5),         # qkv
    MatmulSpec.new(4, 3072, 768).accumulate(),        # up, four rows, accumulating
    MatmulSpec.new(16, 768, 3072),                    # down, sixteen rows (matrix cores)
    MatmulSpec.new(3, 200, 5000),                     # ragged columns, long K
    MatmulSpec.new(2, 64, 4000).batched(BatchStrides(3, 2 * 4000, 4000 * 64, 2 * 64)),  # batched
    MatmulSpec.new(9, 1000, 1000).accumulate(),       # nine rows
    MatmulSpec.new(1, 768, 768),                      # out again, after all of the above
]


def run(gpu, spec, seed, x=None):
    left_len, right_len, out_len = spec.lengths()
    left = oracle.random_values(left_len, seed) if x is None else x
    right = oracle.random_values(right_len, seed + 1) * np.float32(0.05)
    initial = oracle.random_values(out_len, seed + 2)
    L, R = gpu.upload(Shape.vector(left_len), left), gpu.upload(Shape.vector(right_len), right)
    out = gpu.upload(Shape.vector(out_len), initial)
    gpu.matmul(spec, L, R, out)
    got = gpu.download(out)
    for t in (L, R, out):
        t.free()
    return (left, right, initial), got


def expected_of(spec, inputs):
    left, right, initial = inputs
    b = spec.batch
    p = oracle.Product(spec.rows, spec.cols, spec.inner, False, False, b.count, b.left, b.right, b.output, spec.scale,
                       spec.write == gemm.WriteMode.Accumulate)
    out = initial.copy()
    oracle.matmul(p, left, right, out)
    return out


def test_back_to_back_split_products_reuse_cleared_slots(gpu):
    for spec in SPLIT_PRODUCTS:
        plan = gemm.plan(spec)
        assert plan.path == gemm.PATH_FEW_ROWS and plan.splits > 1, (spec, plan.path, plan.splits)
    first = []
    for i, spec in enumerate(SPLIT_PRODUCTS):
        print(f"split product {i}: {spec.rows}x{spec.cols}x{spec.inner} batch {spec.batch.count}, "
              f"{gemm.plan(spec).splits} slices", flush=True)
        inputs, got = run(gpu, spec, 50 + 3 * i)
        error = oracle.relative_error(expected_of(spec, inputs), got)
        assert error < TOLERANCE, f"product {i}: relative error {error}"
        first.append(got)
    for i, spec in enumerate(SPLIT_PRODUCTS):
        _, again = run(gpu, spec, 50 + 3 * i)
        assert np.array_equal(first[i], again), f"product {i}: rerun differs"


@pytest.mark.parametrize("nan_bits", [0x7FC00000, 0xFFFFFFFF, 0xFF800001], ids=["quiet", "all_ones", "signalling"])
def test_nan_rows_stay_in_their_row_and_do_not_stall(gpu, nan_bits):
    spec = MatmulSpec.new(4, 2304, 768)
    assert gemm.plan(spec).splits > 1
    left_len, _, _ = spec.lengths()
    x = oracle.random_values(left_len, 81)
    x.view(np.uint32)[2 * 768 + 100] = np.uint32(nan_bits)  # one NaN in row 2
    print(f"NaN 0x{nan_bits:08X} in row 2 of x", flush=True)
    gpu.synchronize()
    start = time.perf_counter()
    inputs, got = run(gpu, spec, 81, x=x)
    elapsed = time.perf_counter() - start
    rows = got.reshape(4, 2304)
    assert np.all(np.isnan(rows[2]))
    expected = expected_of(spec, inputs).reshape(4, 2304)
    clean = [0, 1, 3]
    assert oracle.relative_error(expected[clean].ravel(), rows[clean].ravel()) < TOLERANCE
    # The polling deadline (0.5 s) was not what ended the call.
    assert elapsed < 0.25, f"{elapsed:.3f} s"
    # The next call on clean operands reads no slot this one left behind.
    inputs, got = run(gpu, spec, 82)
    assert oracle.relative_error(expected_of(spec, inputs), got) < TOLERANCE

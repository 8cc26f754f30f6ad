"""GPU parity against the CPU oracle, through the C ABI.

The sweep mirrors the reference's own GPU test,
``matmul_matches_reference_for_every_storage_and_kernel``
(crates/staleynet-cuda/tests/kernels_match_reference.rs:54-91): ragged sizes
x batch {1, 3} x {NN, TN, NT, TT}, scale 0.7, accumulate onto LCG values,
relative error below the kernel's tolerance. The oracle's outputs are also
checked against the committed vectors (tests/golden/sweep_oracle.json).
Edge cases the reference leaves implicit are added: empty products,
undersized/aliased operands, unaligned operands (the scalar-load path),
split-K, broadcast batches and the causal-mask extension.
"""
import hashlib
import json
import os
import sys

import numpy as np
import pytest

from oracle import oracle
from staleynet_amd import gemm
from staleynet_amd.gemm import (BatchStrides, MatmulKernel, MatmulPanic, MatmulSpec, Precision, Shape, SN_ERR_ALIASING,
                                SN_ERR_EMPTY_BATCH, SN_ERR_LEFT_TOO_SMALL, SN_ERR_OUTPUT_TOO_SMALL)

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402

pytestmark = pytest.mark.gpu

KERNELS = [MatmulKernel.MfmaF32, MatmulKernel.MfmaBf16, MatmulKernel.Simple]
GOLDEN = {(c["rows"], c["cols"], c["inner"], c["batch"], c["variant"]): c
          for c in json.load(open(os.path.join(HERE, "golden", "sweep_oracle.json")))["cases"]}


def to_product(spec: MatmulSpec) -> oracle.Product:
    return oracle.Product(spec.rows, spec.cols, spec.inner, bool(spec.left), bool(spec.right), spec.batch.count,
                          spec.batch.left, spec.batch.right, spec.batch.output, spec.scale, bool(spec.write))


def run_gpu(gpu, spec, left, right, initial, kernel=MatmulKernel.MfmaF32):
    gpu.matmul_kernel = kernel
    try:
        lt = gpu.upload(Shape.vector(left.size), left)
        rt = gpu.upload(Shape.vector(right.size), right)
        out = gpu.upload(Shape.vector(initial.size), initial)
        gpu.matmul(spec, lt, rt, out)
        return gpu.download(out)
    finally:
        gpu.matmul_kernel = MatmulKernel.MfmaF32


def expected_for(spec, left, right, initial):
    out = initial.copy()
    oracle.matmul(to_product(spec), left, right, out)
    return out


def check(expected, actual, tolerance, what=""):
    assert np.all(np.isfinite(actual)), f"{what}: non-finite output"
    error = oracle.relative_error(expected, actual)
    assert error < tolerance, f"{what}: relative error {error}"
    return error


@pytest.mark.parametrize("case", list(make_golden.sweep_cases()),
                         ids=lambda c: f"{c['rows']}x{c['cols']}x{c['inner']}-b{c['batch']}-{c['variant']}")
def test_matmul_matches_reference_for_every_storage_and_kernel(gpu, case):
    rows, cols, inner, batch = case["rows"], case["cols"], case["inner"], case["batch"]
    spec = MatmulSpec.new(rows, cols, inner).batched(
        BatchStrides(count=batch, left=rows * inner, right=inner * cols, output=rows * cols)).scaled(0.7).accumulate()
    if case["left_t"]:
        spec = spec.left_transposed()
    if case["right_t"]:
        spec = spec.right_transposed()
    left = oracle.random_values(batch * rows * inner, 1)
    right = oracle.random_values(batch * inner * cols, 2)
    initial = oracle.random_values(batch * rows * cols, 3)
    expected = expected_for(spec, left, right, initial)
    golden = GOLDEN[(rows, cols, inner, batch, case["variant"])]
    assert hashlib.sha256(expected.astype("<f4").tobytes()).hexdigest() == golden["sha256"]
    for kernel in KERNELS:
        actual = run_gpu(gpu, spec, left, right, initial, kernel)
        check(expected, actual, kernel.tolerance(), f"{kernel.name} {spec}")
        if kernel == MatmulKernel.Simple:
            # Same order, same separately rounded operations as the reference loop.
            assert np.array_equal(expected, actual)


def test_empty_products_follow_the_reference_loops(gpu):
    initial = oracle.random_values(20, 3)
    # rows = 0: nothing is written.
    out = run_gpu(gpu, MatmulSpec.new(0, 5, 3), np.zeros(1, np.float32), oracle.random_values(15, 2), initial)
    assert np.array_equal(out, initial)
    # inner = 0: the sum is 0, so overwrite stores scale*0 and accumulate keeps the previous value.
    out = run_gpu(gpu, MatmulSpec.new(4, 5, 0).scaled(0.7), np.zeros(1, np.float32), np.zeros(1, np.float32), initial)
    assert np.array_equal(out, np.zeros(20, np.float32))
    out = run_gpu(gpu, MatmulSpec.new(4, 5, 0).accumulate(), np.zeros(1, np.float32), np.zeros(1, np.float32),
                  initial)
    assert np.array_equal(out, initial)


def test_invalid_specs_raise_the_reference_panics(gpu):
    left = gpu.upload(Shape.vector(6), np.ones(6))
    right = gpu.upload(Shape.vector(6), np.ones(6))
    out = gpu.zeros(Shape.vector(4))
    with pytest.raises(MatmulPanic, match="left operand too small") as info:
        gpu.matmul(MatmulSpec.new(2, 2, 4), left, right, out)
    assert info.value.status == SN_ERR_LEFT_TOO_SMALL
    with pytest.raises(MatmulPanic, match="output too small") as info:
        gpu.matmul(MatmulSpec.new(3, 2, 2), left, right, out)
    assert info.value.status == SN_ERR_OUTPUT_TOO_SMALL
    with pytest.raises(MatmulPanic) as info:
        gpu.matmul(MatmulSpec.new(2, 2, 2).batched(BatchStrides(0, 4, 4, 4)), left, right, out)
    assert info.value.status == SN_ERR_EMPTY_BATCH
    with pytest.raises(MatmulPanic) as info:
        gpu.matmul(MatmulSpec.new(2, 2, 2), left, right, left)
    assert info.value.status == SN_ERR_ALIASING
    gpu.synchronize()
    assert np.array_equal(gpu.download(out), np.zeros(4, np.float32))


@pytest.mark.parametrize("variant", ["NN", "TN", "NT", "TT"])
def test_unaligned_operands_take_the_scalar_path(gpu, variant):
    # Operands that start 1 float past an aligned address cannot use 128-bit loads.
    rows, cols, inner = 96, 80, 68
    spec = MatmulSpec.new(rows, cols, inner).scaled(1.5)
    if variant[0] == "T":
        spec = spec.left_transposed()
    if variant[1] == "T":
        spec = spec.right_transposed()
    left = oracle.random_values(rows * inner + 1, 4)
    right = oracle.random_values(inner * cols + 1, 5)
    initial = np.zeros(rows * cols + 1, np.float32)
    expected = expected_for(spec, left[1:].copy(), right[1:].copy(), initial[1:].copy())
    lt = gpu.upload(Shape.vector(left.size), left)
    rt = gpu.upload(Shape.vector(right.size), right)
    out = gpu.upload(Shape.vector(initial.size), initial)
    gpu.matmul_raw(spec, lt.pointer + 4, left.size - 1, rt.pointer + 4, right.size - 1, out.pointer + 4,
                   initial.size - 1)
    actual = gpu.download(out)
    assert actual[0] == 0.0
    check(expected, actual[1:], 1e-5, variant)


@pytest.mark.parametrize("variant", ["NN", "TN", "NT", "TT"])
@pytest.mark.parametrize("rows,cols,inner,batch", [(132, 196, 100, 3), (260, 132, 36, 1), (128, 128, 32, 2),
                                                   (36, 516, 4, 1), (520, 60, 292, 2), (24, 40, 1028, 1)])
def test_aligned_ragged_shapes_load_straight_into_lds(gpu, variant, rows, cols, inner, batch):
    # Sizes that are multiples of 4 but not of the 128x128x32 tile: 16-byte-aligned
    # operands take the direct-to-LDS kernel, whose edge tiles and last partial
    # K-step are padded by out-of-range loads that write zeros into LDS.
    spec = MatmulSpec.new(rows, cols, inner).batched(
        BatchStrides(batch, rows * inner, inner * cols, rows * cols)).scaled(0.7).accumulate()
    if variant[0] == "T":
        spec = spec.left_transposed()
    if variant[1] == "T":
        spec = spec.right_transposed()
    left = oracle.random_values(batch * rows * inner, 21)
    right = oracle.random_values(batch * inner * cols, 22)
    initial = oracle.random_values(batch * rows * cols, 23)
    expected = expected_for(spec, left, right, initial)
    check(expected, run_gpu(gpu, spec, left, right, initial), 1e-5, f"{variant} {spec}")


@pytest.mark.parametrize("variant", ["NN", "TN", "NT"])
def test_split_k_matches_for_long_inner_dimensions(gpu, variant):
    # Few output tiles and a long K: the dispatcher splits K and reduces in order.
    rows, cols, inner = 200, 300, 8192
    spec = MatmulSpec.new(rows, cols, inner).scaled(0.5).accumulate()
    if variant[0] == "T":
        spec = spec.left_transposed()
    if variant[1] == "T":
        spec = spec.right_transposed()
    left = oracle.random_values(rows * inner, 6)
    right = oracle.random_values(inner * cols, 7)
    initial = oracle.random_values(rows * cols, 8)
    expected = expected_for(spec, left, right, initial)
    check(expected, run_gpu(gpu, spec, left, right, initial), 1e-5, variant)


def test_broadcast_batches_and_the_narrow_tile(gpu):
    # N = 64 uses the 128x64 tile; the right operand is shared by every matrix.
    rows, cols, inner, count = 300, 64, 200, 3
    spec = MatmulSpec.new(rows, cols, inner).batched(BatchStrides(count, rows * inner, 0, rows * cols))
    left = oracle.random_values(count * rows * inner, 9)
    right = oracle.random_values(inner * cols, 10)
    initial = np.zeros(count * rows * cols, np.float32)
    expected = expected_for(spec, left, right, initial)
    actual = run_gpu(gpu, spec, left, right, initial)
    check(expected, actual, 1e-5)
    # Broadcasting the left operand instead.
    spec = MatmulSpec.new(rows, cols, inner).batched(BatchStrides(count, 0, inner * cols, rows * cols))
    right = oracle.random_values(count * inner * cols, 11)
    left = oracle.random_values(rows * inner, 12)
    check(expected_for(spec, left, right, initial), run_gpu(gpu, spec, left, right, initial), 1e-5)


def causal_visible(queries, keys, offset):
    q = np.arange(queries)[:, None]
    k = np.arange(keys)[None, :]
    return k <= q + offset


@pytest.mark.parametrize("offset", [0, 37])
@pytest.mark.parametrize("accumulate", [False, True])
def test_causal_output_mask(gpu, offset, accumulate):
    # S = Q·Kᵀ per head (attention.rs:206-209) with masked tiles skipped.
    t, h, count = 300, 64, 2
    spec = MatmulSpec.new(t, t, h).right_transposed().batched(BatchStrides(count, t * h, t * h, t * t))
    if accumulate:
        spec = spec.accumulate()
    q = oracle.random_values(count * t * h, 13)
    k = oracle.random_values(count * t * h, 14)
    initial = oracle.random_values(count * t * t, 15)
    dense = expected_for(spec, q, k, initial).reshape(count, t, t)
    actual = run_gpu(gpu, spec.causal_output(offset), q, k, initial).reshape(count, t, t)
    visible = np.broadcast_to(causal_visible(t, t, offset), dense.shape)
    check(dense[visible], actual[visible], 1e-5)
    masked = actual[~visible]
    if accumulate:
        assert np.array_equal(masked, initial.reshape(count, t, t)[~visible])
    else:
        assert np.all(masked == 0.0)


@pytest.mark.parametrize("h", [64, 100, 4])
@pytest.mark.parametrize("mask,accumulate", [(None, False), (0, False), (37, True)])
def test_short_inner_products_over_many_heads(gpu, h, mask, accumulate):
    # Q.K^T-shaped NT products with K in one to four 32-deep steps (h = 100: a
    # partial last step) over 160 heads of 260 x 260 (ragged edge tiles next
    # to the interior tiles' fast epilogue), dense or causal, overwrite or
    # accumulate.
    t, count = 260, 160
    spec = MatmulSpec.new(t, t, h).right_transposed().batched(BatchStrides(count, t * h, t * h, t * t)).scaled(0.7)
    if accumulate:
        spec = spec.accumulate()
    q = oracle.random_values(count * t * h, 31)
    k = oracle.random_values(count * t * h, 32)
    initial = oracle.random_values(count * t * t, 33)
    dense = initial.copy()
    oracle.matmul_parallel(to_product(spec), q, k, dense)
    if mask is None:
        check(dense, run_gpu(gpu, spec, q, k, initial), 1e-5, f"h={h}")
        return
    actual = run_gpu(gpu, spec.causal_output(mask), q, k, initial).reshape(count, t, t)
    dense = dense.reshape(count, t, t)
    visible = np.broadcast_to(causal_visible(t, t, mask), dense.shape)
    check(dense[visible], actual[visible], 1e-5, f"h={h} offset={mask}")
    masked = actual[~visible]
    if accumulate:
        assert np.array_equal(masked, initial.reshape(count, t, t)[~visible])
    else:
        assert np.all(masked == 0.0)


@pytest.mark.parametrize("offset", [0, 45])
@pytest.mark.parametrize("transposed", [False, True])
def test_causal_left_mask(gpu, offset, transposed):
    # O = P·V (NN) and dV = Pᵀ·dO (TN) with P causal (attention.rs:212-213, 244-247).
    # The masked part of P holds large garbage that must not reach the result.
    t, h, count = 280, 64, 2
    p = oracle.random_values(count * t * t, 16).reshape(count, t, t)
    visible = causal_visible(t, t, offset)
    p_clean = np.where(visible, p, 0).astype(np.float32)
    p_dirty = np.where(visible, p, 1e4).astype(np.float32)
    v = oracle.random_values(count * t * h, 17)
    spec = MatmulSpec.new(t, h, t).batched(BatchStrides(count, t * t, t * h, t * h)).scaled(0.125)
    if transposed:
        spec = spec.left_transposed()
    initial = np.zeros(count * t * h, np.float32)
    expected = expected_for(spec, p_clean.ravel(), v, initial)
    actual = run_gpu(gpu, spec.causal_left(offset), p_dirty.ravel(), v, initial)
    check(expected, actual, 1e-5)
    simple = run_gpu(gpu, spec.causal_left(offset), p_dirty.ravel(), v, initial, MatmulKernel.Simple)
    check(expected, simple, 1e-6)


@pytest.mark.parametrize("m,offset", [(1, 700), (4, 300), (16, 40)])
def test_causal_left_few_rows_skip_the_masked_part_and_the_unwritten_tail(gpu, m, offset):
    # The decode mix (attention.rs:314-316) on the few-row path: P [m, capacity] holds garbage past
    # row r's horizon r + offset, and V's rows past the last row's horizon are an unwritten cache
    # tail (NaN here): neither may reach the result.
    capacity, h, count = 1408, 64, 3
    p = oracle.random_values(count * m * capacity, 40).reshape(count, m, capacity)
    visible = causal_visible(m, capacity, offset)
    p_clean = np.where(visible, p, 0).astype(np.float32)
    p_dirty = np.where(visible, p, 1e4).astype(np.float32)
    v = oracle.random_values(count * capacity * h, 41).reshape(count, capacity, h)
    v_dirty = v.copy()
    v_dirty[:, m + offset:, :] = np.nan
    spec = MatmulSpec.new(m, h, capacity).batched(BatchStrides(count, m * capacity, capacity * h, m * h))
    initial = np.zeros(count * m * h, np.float32)
    expected = expected_for(spec, p_clean.ravel(), v.ravel(), initial)
    actual = run_gpu(gpu, spec.causal_left(offset), p_dirty.ravel(), v_dirty.ravel(), initial)
    assert np.all(np.isfinite(actual))
    check(expected, actual, 1e-5)


@pytest.mark.parametrize("m,k,offset,accumulate", [(1, 64, 700, False), (3, 200, 90, True), (4, 128, 0, False),
                                                    (2, 64, None, True), (3, 130, 50, False)])
def test_few_rows_against_a_transposed_right_operand(gpu, m, k, offset, accumulate):
    # The decode scores S = q K^T against the cache (attention.rs:307-310): at most 4 rows of x
    # against B stored [n][k]. K a multiple of 4 takes the few-row kernel (several 64-float chunks at
    # k = 128, 200); k = 130 takes the tiled kernels. With the causal output mask, rows of B past the
    # last row's horizon are an unwritten cache tail (NaN here) and are not read; masked outputs are
    # 0 (overwrite) or left as they were (accumulate).
    n, count = 1408, 3
    x = oracle.random_values(count * m * k, 50)
    b = oracle.random_values(count * n * k, 51).reshape(count, n, k)
    spec = MatmulSpec.new(m, n, k).right_transposed().batched(BatchStrides(count, m * k, n * k, m * n)).scaled(0.125)
    if accumulate:
        spec = spec.accumulate()
    initial = oracle.random_values(count * m * n, 52)
    expected = expected_for(spec, x, b.ravel(), initial).reshape(count, m, n)
    if offset is None:
        actual = run_gpu(gpu, spec, x, b.ravel(), initial).reshape(count, m, n)
        check(expected.ravel(), actual.ravel(), 1e-5)
        return
    b_dirty = b.copy()
    b_dirty[:, m + offset:, :] = np.nan
    actual = run_gpu(gpu, spec.causal_output(offset), x, b_dirty.ravel(), initial).reshape(count, m, n)
    visible = np.broadcast_to(causal_visible(m, n, offset), actual.shape)
    check(expected[visible], actual[visible], 1e-5)
    masked = actual[~visible]
    if accumulate:
        assert np.array_equal(masked, initial.reshape(count, m, n)[~visible])
    else:
        assert np.all(masked == 0.0)


# ---- bf16-input variant ---------------------------------------------------------

@pytest.mark.parametrize("variant", ["NN", "TN", "NT", "TT"])
def test_bf16_is_exact_on_bf16_representable_integers(gpu, variant):
    # Integers of magnitude <= 16 are exact in bf16, their products are exact,
    # and every partial sum stays below 2^24, so any summation order gives the
    # exact result: a wrong lane layout or a wrong k pairing cannot hide.
    rows, cols, inner = 96, 160, 200
    rng = np.random.default_rng(11)
    left = rng.integers(-16, 17, size=rows * inner).astype(np.float32)
    right = rng.integers(-16, 17, size=inner * cols).astype(np.float32)
    spec = MatmulSpec.new(rows, cols, inner)
    if variant[0] == "T":
        spec = spec.left_transposed()
    if variant[1] == "T":
        spec = spec.right_transposed()
    initial = np.zeros(rows * cols, np.float32)
    expected = expected_for(spec, left, right, initial)
    actual = run_gpu(gpu, spec, left, right, initial, MatmulKernel.MfmaBf16)
    assert np.array_equal(expected, actual)


# Rounding to nearest even, hand-derived (IEEE roundTiesToEven), where each path rounds: k = 16 the
# narrow tile and k = 128 the 64 x 64 tile, both rounding fp32 fragments as they are read; "staged",
# a right operand of 256 identity blocks side by side (fewer rows than a 256 x 256 tile, as many
# 128 x 128 tiles as CUs), whose operands are first rounded into the workspace by the staging kernels.
BF16_RNE_CASES = [
    (1.0, 1.0),
    (1 + 2.0 ** -8, 1.0),                      # halfway, 1.0 is even
    (1 + 3 * 2.0 ** -8, 1 + 2 * 2.0 ** -7),    # halfway between 1+u (odd) and 1+2u (even), u = 2^-7
    (1 + 2.0 ** -8 + 2.0 ** -20, 1 + 2.0 ** -7),  # just above halfway
    (1 + 2.0 ** -8 - 2.0 ** -20, 1.0),         # just below halfway
    (-(1 + 3 * 2.0 ** -8), -(1 + 2 * 2.0 ** -7)),
    (3.0, 3.0),
    (1.0 / 3.0, 0.333984375),                  # 0x3EAB: 0.01010101 01010101... rounds up
    (float(np.finfo(np.float32).max), float("inf")),
    (2.0 ** -100 * 1.5, 2.0 ** -100 * 1.5),    # exact, small exponent
    (0.0, 0.0),
]


@pytest.mark.parametrize("case", ["k16", "k128", "staged"])
def test_bf16_inputs_round_to_nearest_even(gpu, case):
    # A times the identity (or identity blocks) returns A rounded to bf16 (7 stored mantissa bits).
    k = 16 if case == "k16" else 128
    blocks = 256 if case == "staged" else 1
    rows = len(BF16_RNE_CASES)
    a = np.zeros((rows, k), np.float32)
    a[:, 0] = [c[0] for c in BF16_RNE_CASES]
    right = np.tile(np.eye(k, dtype=np.float32), (1, blocks))
    spec = MatmulSpec.new(rows, k * blocks, k)
    plan = gemm.plan(spec.with_precision(Precision.Bf16))
    assert plan.path == {"k16": gemm.PATH_BF16_DIRECT, "k128": gemm.PATH_BF16_DIRECT,
                         "staged": gemm.PATH_BF16_STAGED}[case], f"path {plan.path}"
    out = run_gpu(gpu, spec, a.ravel(), right.ravel(), np.zeros(rows * k * blocks, np.float32),
                  MatmulKernel.MfmaBf16).reshape(rows, k * blocks)
    expected = [np.float32(c[1]) for c in BF16_RNE_CASES]
    assert out[:, 0].tolist() == expected
    assert out[:, k * (blocks - 1)].tolist() == expected  # the last identity block


# Unmasked aligned bf16 products with more than 64 columns, too small for the 256 x 256 kernel but
# with at least as many 128 x 128 tiles as CUs, first round both operands to bf16, K-contiguous, in
# the context's workspace (zeros pad K to a multiple of 8), then multiply; exact integer inputs pin
# every layout, padding, batch and shared-operand case. Each case checks that the plan stages.
@pytest.mark.parametrize("variant,rows,cols,inner", [
    ("TN", 96, 32800, 203),   # both operands transposed while staged, K padded to 208
    ("TT", 68, 32900, 36),    # A transposed, B K-contiguous
    ("NT", 32800, 100, 1000), # both K-contiguous
    ("NN", 1030, 4100, 96),   # the 128x256 tile, partial tiles on both edges
])
def test_bf16_staged_operands_are_exact_on_integers(gpu, variant, rows, cols, inner):
    rng = np.random.default_rng(rows + cols + inner)
    left = rng.integers(-16, 17, size=rows * inner).astype(np.float32)
    right = rng.integers(-16, 17, size=inner * cols).astype(np.float32)
    spec = MatmulSpec.new(rows, cols, inner).scaled(0.5)
    if variant[0] == "T":
        spec = spec.left_transposed()
    if variant[1] == "T":
        spec = spec.right_transposed()
    spec = spec.accumulate()
    assert gemm.plan(spec.with_precision(Precision.Bf16)).path == gemm.PATH_BF16_STAGED
    initial = rng.integers(-8, 9, size=rows * cols).astype(np.float32)
    expected = initial.copy()
    oracle.matmul_parallel(to_product(spec), left, right, expected)
    actual = run_gpu(gpu, spec, left, right, initial, MatmulKernel.MfmaBf16)
    assert np.array_equal(expected, actual)


@pytest.mark.parametrize("shared", ["none", "left", "right"])
def test_bf16_staged_batches_and_shared_operands(gpu, shared):
    batches, rows, cols, inner = 3, 72, 11000, 64
    rng = np.random.default_rng(5)
    left_stride = 0 if shared == "left" else rows * inner
    right_stride = 0 if shared == "right" else inner * cols
    left = rng.integers(-16, 17, size=max(left_stride, rows * inner) * (1 if shared == "left" else batches))
    right = rng.integers(-16, 17, size=max(right_stride, inner * cols) * (1 if shared == "right" else batches))
    spec = MatmulSpec.new(rows, cols, inner).right_transposed().batched(
        BatchStrides(batches, left_stride, right_stride, rows * cols))
    assert gemm.plan(spec.with_precision(Precision.Bf16)).path == gemm.PATH_BF16_STAGED
    initial = np.zeros(batches * rows * cols, np.float32)
    expected = initial.copy()
    oracle.matmul_parallel(to_product(spec), left.astype(np.float32), right.astype(np.float32), expected)
    actual = run_gpu(gpu, spec, left.astype(np.float32), right.astype(np.float32), initial, MatmulKernel.MfmaBf16)
    assert np.array_equal(expected, actual)


def test_bf16_without_room_to_stage_takes_the_fp32_staged_kernel():
    # A context whose workspace cannot hold the staged operands multiplies from fp32 stages
    # (rounding each fragment): the same exact result.
    from staleynet_amd.gemm import Gpu
    small = Gpu(0, workspace_bytes=4096)
    try:
        rows, cols, inner = 128, 256, 512
        rng = np.random.default_rng(8)
        left = rng.integers(-16, 17, size=rows * inner).astype(np.float32)
        right = rng.integers(-16, 17, size=inner * cols).astype(np.float32)
        spec = MatmulSpec.new(rows, cols, inner)
        initial = np.zeros(rows * cols, np.float32)
        actual = run_gpu(small, spec, left, right, initial, MatmulKernel.MfmaBf16)
        assert np.array_equal(expected_for(spec, left, right, initial), actual)
    finally:
        small.close()


# bf16 under the causal masks (the attention products at bf16 precision: fp32 LDS stages rounded per
# fragment, with the masks applied in the stages). Integers of magnitude <= 8 are exact in bf16 and
# every partial sum stays far below 2^24, so the result is exact whatever the order: a masked value
# that leaks, a tile skipped wrongly or a wrong offset cannot hide.

@pytest.mark.parametrize("offset", [0, 45])
@pytest.mark.parametrize("accumulate", [False, True])
def test_bf16_causal_output_mask_is_exact_on_integers(gpu, offset, accumulate):
    # S = Q K^T per head (attention.rs:206-209) with masked tiles skipped.
    t, h, count = 300, 64, 2
    rng = np.random.default_rng(offset + 3 * accumulate)
    q = rng.integers(-8, 9, size=count * t * h).astype(np.float32)
    k = rng.integers(-8, 9, size=count * t * h).astype(np.float32)
    initial = rng.integers(-8, 9, size=count * t * t).astype(np.float32)
    spec = MatmulSpec.new(t, t, h).right_transposed().batched(BatchStrides(count, t * h, t * h, t * t)).scaled(0.5)
    if accumulate:
        spec = spec.accumulate()
    dense = expected_for(spec, q, k, initial).reshape(count, t, t)
    actual = run_gpu(gpu, spec.causal_output(offset).with_precision(Precision.Bf16), q, k,
                     initial).reshape(count, t, t)
    visible = np.broadcast_to(causal_visible(t, t, offset), dense.shape)
    assert np.array_equal(dense[visible], actual[visible])
    masked = actual[~visible]
    if accumulate:
        assert np.array_equal(masked, initial.reshape(count, t, t)[~visible])
    else:
        assert np.all(masked == 0.0)


@pytest.mark.parametrize("offset", [0, 45])
@pytest.mark.parametrize("transposed", [False, True])
@pytest.mark.parametrize("accumulate", [False, True])
def test_bf16_causal_left_mask_is_exact_on_integers(gpu, offset, transposed, accumulate):
    # O = P V (NN) and dV = P^T dO, dK = s dS^T Q (TN) with P causal (attention.rs:212-213,
    # 244-260); the masked part of P holds large garbage that must not reach the result.
    t, h, count = 280, 64, 2
    rng = np.random.default_rng(10 + offset + 2 * transposed + accumulate)
    p = rng.integers(-8, 9, size=(count, t, t)).astype(np.float32)
    visible = causal_visible(t, t, offset)
    p_clean = np.where(visible, p, 0).astype(np.float32)
    p_dirty = np.where(visible, p, 1e4).astype(np.float32)
    v = rng.integers(-8, 9, size=count * t * h).astype(np.float32)
    spec = MatmulSpec.new(t, h, t).batched(BatchStrides(count, t * t, t * h, t * h)).scaled(0.125)
    if transposed:
        spec = spec.left_transposed()
    initial = np.zeros(count * t * h, np.float32)
    if accumulate:
        spec = spec.accumulate()
        initial = rng.integers(-8, 9, size=count * t * h).astype(np.float32)
    expected = expected_for(spec, p_clean.ravel(), v, initial)
    actual = run_gpu(gpu, spec.causal_left(offset).with_precision(Precision.Bf16), p_dirty.ravel(), v, initial)
    assert np.array_equal(expected, actual)


@pytest.mark.parametrize("mask", ["output", "left"])
def test_bf16_causal_masks_within_the_stated_tolerance(gpu, mask):
    # N(0, 1)-like inputs at config 3's head shape (T = 2048, h = 64, two heads), against the fp32
    # oracle at the variant's 2e-2.
    t, h, count = 2048, 64, 2
    if mask == "output":
        spec = MatmulSpec.new(t, t, h).right_transposed().batched(BatchStrides(count, t * h, t * h, t * t))
        left = oracle.random_values(count * t * h, 61)
        right = oracle.random_values(count * t * h, 62)
        expected = expected_for(spec, left, right, np.zeros(count * t * t, np.float32)).reshape(count, t, t)
        actual = run_gpu(gpu, spec.causal_output().with_precision(Precision.Bf16), left, right,
                         np.zeros(count * t * t, np.float32)).reshape(count, t, t)
        visible = np.broadcast_to(causal_visible(t, t, 0), expected.shape)
        check(expected[visible], actual[visible], 2e-2)
        assert np.all(actual[~visible] == 0.0)
    else:
        p = np.where(causal_visible(t, t, 0), oracle.random_values(count * t * t, 63).reshape(count, t, t),
                     0).astype(np.float32).ravel()
        right = oracle.random_values(count * t * h, 64)
        spec = MatmulSpec.new(t, h, t).left_transposed().batched(BatchStrides(count, t * t, t * h, t * h))
        initial = np.zeros(count * t * h, np.float32)
        check(expected_for(spec, p, right, initial),
              run_gpu(gpu, spec.causal_left().with_precision(Precision.Bf16), p, right, initial), 2e-2)


# ---- decode-shaped products (few rows, row-major weight) ------------------------------

@pytest.mark.parametrize("rows,cols,inner", [(1, 8, 1), (3, 100, 37), (5, 772, 1000), (16, 260, 4100),
                                             (7, 2304, 768), (2, 12, 20000), (1, 516, 1000), (2, 300, 777),
                                             (16, 768, 784)])
@pytest.mark.parametrize("accumulate", [False, True])
def test_few_row_products_match_the_oracle(gpu, rows, cols, inner, accumulate):
    spec = MatmulSpec.new(rows, cols, inner).scaled(0.7)
    if accumulate:
        spec = spec.accumulate()
    left = oracle.random_values(rows * inner, 21)
    right = oracle.random_values(inner * cols, 22)
    initial = oracle.random_values(rows * cols, 23)
    expected = expected_for(spec, left, right, initial)
    check(expected, run_gpu(gpu, spec, left, right, initial), 1e-5, f"{rows}x{cols}x{inner}")


def test_batched_few_row_products(gpu):
    # One query row per head against per-head weights (batch stride on both operands).
    heads, cols, inner = 12, 64, 1408
    spec = MatmulSpec.new(1, cols, inner).batched(BatchStrides(heads, inner, inner * cols, cols))
    left = oracle.random_values(heads * inner, 24)
    right = oracle.random_values(heads * inner * cols, 25)
    initial = np.zeros(heads * cols, np.float32)
    check(expected_for(spec, left, right, initial), run_gpu(gpu, spec, left, right, initial), 1e-5)

"""GPU parity of the bf16 kernel that rounds fp32 operands to bf16 as it loads them
(csrc/gemm_bf16_wide.hip: the weight- and input-gradient layouts TN, NT and TT, 256 x 256 tiles),
in the role of the reference's TF32 kernel (crates/staleynet-cuda/src/kernels/matmul.rs:357-448),
against the oracle's restatement of reference::matmul (reference.rs:10-38).

Integers of magnitude <= 16 are exact in bf16, their products are exact and every partial sum here
stays below 2^24, so those cases must match bit for bit in any summation order: ragged tiles on both
output axes, a K tail that is not a whole 32-deep step, split K, batches with a shared operand,
accumulate with a scale; and the products where the smaller operand is first rounded into the
workspace (K-contiguous bf16, from either stored layout) while the other is rounded as it loads.
Rounding to nearest even is pinned by hand-derived cases, and random inputs are held to the bf16
tolerance (2e-2, device.rs:51-66). Each case first checks that the launch plan really takes this
kernel."""
import numpy as np
import pytest

from oracle import oracle
from staleynet_amd import gemm
from staleynet_amd.gemm import BatchStrides, MatmulKernel, MatmulSpec, Shape

pytestmark = pytest.mark.gpu

BF16_TOLERANCE = 2e-2  # device.rs:51-66


def product_of(spec: MatmulSpec) -> oracle.Product:
    return oracle.Product(spec.rows, spec.cols, spec.inner, bool(spec.left), bool(spec.right), spec.batch.count,
                          spec.batch.left, spec.batch.right, spec.batch.output, spec.scale, bool(spec.write))


def layout(spec: MatmulSpec, variant: str) -> MatmulSpec:
    if variant[0] == "T":
        spec = spec.left_transposed()
    if variant[1] == "T":
        spec = spec.right_transposed()
    return spec


def run_bf16(gpu, spec, left, right, initial):
    gpu.matmul_kernel = MatmulKernel.MfmaBf16
    try:
        lt = gpu.upload(Shape.vector(left.size), left)
        rt = gpu.upload(Shape.vector(right.size), right)
        out = gpu.upload(Shape.vector(initial.size), initial)
        gpu.matmul(spec, lt, rt, out)
        result = gpu.download(out)
        for t in (lt, rt, out):
            t.free()
        return result
    finally:
        gpu.matmul_kernel = MatmulKernel.MfmaF32


def expected(spec, left, right, initial):
    out = initial.copy()
    oracle.matmul_parallel(product_of(spec), left, right, out)
    return out


def wide_plan(spec):
    plan = gemm.plan(spec, int(MatmulKernel.MfmaBf16))
    assert plan.path == gemm.PATH_BF16_WIDE, f"path {plan.path}"
    return plan


@pytest.mark.parametrize("variant,rows,cols,inner", [
    ("TN", 300, 260, 100),    # partial tiles on both output edges; K = 3 steps + a 4-deep tail
    ("NT", 256, 512, 64),     # whole tiles, two steps
    ("TT", 260, 384, 96),     # A row-contiguous, B K-contiguous
    ("NT", 520, 300, 1000),   # K = 31 steps + 8; three tile rows, two tile columns
    ("TN", 132, 136, 36),     # one partial tile each way, a step and a tail
])
def test_wide_is_exact_on_integers(gpu, variant, rows, cols, inner):
    print(f"wide {variant} {rows}x{cols}x{inner}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols + inner)
    left = rng.integers(-16, 17, size=rows * inner).astype(np.float32)
    right = rng.integers(-16, 17, size=inner * cols).astype(np.float32)
    initial = rng.integers(-8, 9, size=rows * cols).astype(np.float32)
    spec = layout(MatmulSpec.new(rows, cols, inner), variant).scaled(0.5).accumulate()
    wide_plan(spec)
    assert np.array_equal(expected(spec, left, right, initial), run_bf16(gpu, spec, left, right, initial))


@pytest.mark.parametrize("variant,rows,cols,inner", [
    ("NN", 1024, 256, 100),   # right operand (row-contiguous) staged through the transposing kernel
    ("NT", 600, 260, 96),     # right operand (K-contiguous) staged row by row
    ("TN", 256, 640, 300),    # left operand (row-contiguous) staged, right rounded as loaded
    ("TT", 260, 600, 64),     # left staged, right K-contiguous
    ("NN", 2100, 300, 1000),  # ragged edges, K = 31 steps + 8, split K
])
def test_wide_with_one_operand_staged_is_exact_on_integers(gpu, variant, rows, cols, inner):
    print(f"wide staged {variant} {rows}x{cols}x{inner}", flush=True)
    rng = np.random.default_rng(rows + 5 * cols + inner)
    left = rng.integers(-16, 17, size=rows * inner).astype(np.float32)
    right = rng.integers(-16, 17, size=inner * cols).astype(np.float32)
    initial = rng.integers(-8, 9, size=rows * cols).astype(np.float32)
    spec = layout(MatmulSpec.new(rows, cols, inner), variant).scaled(0.5).accumulate()
    plan = wide_plan(spec)
    partials = plan.splits * rows * cols * 4 if plan.splits > 1 else 0
    assert plan.workspace_bytes > partials  # the staged operand sits in the workspace
    assert np.array_equal(expected(spec, left, right, initial), run_bf16(gpu, spec, left, right, initial))


def test_wide_split_k_is_exact_on_integers(gpu):
    # A weight-gradient shape whose 9 output tiles take K in slices, reduced in slice order.
    rows, cols, inner = 768, 640, 4096
    rng = np.random.default_rng(3)
    left = rng.integers(-4, 5, size=rows * inner).astype(np.float32)
    right = rng.integers(-4, 5, size=inner * cols).astype(np.float32)
    initial = rng.integers(-8, 9, size=rows * cols).astype(np.float32)
    spec = MatmulSpec.new(rows, cols, inner).left_transposed().accumulate()
    plan = wide_plan(spec)
    assert plan.splits > 1
    assert np.array_equal(expected(spec, left, right, initial), run_bf16(gpu, spec, left, right, initial))


# "left" and "right": the shared operand is the smaller one and is staged once for the batch.
@pytest.mark.parametrize("shared", ["none", "left", "right"])
def test_wide_batches_and_shared_operands(gpu, shared):
    batches, rows, cols, inner = 3, 256, 300, 64
    rng = np.random.default_rng(9)
    left_stride = 0 if shared == "left" else rows * inner
    right_stride = 0 if shared == "right" else inner * cols
    left = rng.integers(-16, 17, size=max(left_stride, rows * inner) * (1 if shared == "left" else batches))
    right = rng.integers(-16, 17, size=max(right_stride, inner * cols) * (1 if shared == "right" else batches))
    spec = MatmulSpec.new(rows, cols, inner).right_transposed().batched(
        BatchStrides(batches, left_stride, right_stride, rows * cols))
    wide_plan(spec)
    initial = np.zeros(batches * rows * cols, np.float32)
    left, right = left.astype(np.float32), right.astype(np.float32)
    assert np.array_equal(expected(spec, left, right, initial), run_bf16(gpu, spec, left, right, initial))


def test_wide_rounds_to_nearest_even(gpu):
    # C = A^T I returns A^T rounded to bf16: row 0 of the stored A (K = 128 rows of M = 128) holds the
    # cases, which come back in column 0 of C. Expected values follow IEEE roundTiesToEven by hand.
    u = 2.0 ** -7  # bf16 ulp in [1, 2)
    cases = [
        (1 + 2.0 ** -8, 1.0),                  # halfway, 1.0 is even
        (1 + 3 * 2.0 ** -8, 1 + 2 * u),        # halfway between 1+u (odd) and 1+2u (even)
        (1 + 2.0 ** -8 + 2.0 ** -20, 1 + u),   # just above halfway
        (1 + 2.0 ** -8 - 2.0 ** -20, 1.0),     # just below halfway
        (-(1 + 3 * 2.0 ** -8), -(1 + 2 * u)),
        (1.0 / 3.0, 0.333984375),
        (float(np.finfo(np.float32).max), float("inf")),
        (0.0, 0.0),
    ]
    n = 128
    a = np.zeros((n, n), np.float32)
    a[0, :len(cases)] = [c[0] for c in cases]
    eye = np.eye(n, dtype=np.float32)
    spec = MatmulSpec.new(n, n, n).left_transposed()
    wide_plan(spec)
    out = run_bf16(gpu, spec, a.ravel(), eye.ravel(), np.zeros(n * n, np.float32)).reshape(n, n)
    assert out[:len(cases), 0].tolist() == [np.float32(c[1]) for c in cases]


@pytest.mark.parametrize("variant,rows,cols,inner", [("TN", 768, 768, 2048), ("NT", 1024, 768, 768)])
def test_wide_random_within_bf16_tolerance(gpu, variant, rows, cols, inner):
    left = oracle.random_values(rows * inner, 21)
    right = oracle.random_values(inner * cols, 22)
    initial = oracle.random_values(rows * cols, 23)
    spec = layout(MatmulSpec.new(rows, cols, inner), variant).scaled(0.7).accumulate()
    wide_plan(spec)
    got = run_bf16(gpu, spec, left, right, initial)
    want = expected(spec, left, right, initial)
    assert np.all(np.isfinite(got))
    assert oracle.relative_error(want, got) < BF16_TOLERANCE


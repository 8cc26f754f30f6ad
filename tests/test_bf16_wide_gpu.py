"""GPU parity of the bf16 kernel that rounds fp32 operands to bf16 as it loads them
(csrc/gemm_bf16_wide.hip: 256 x 256 tiles, every layout), in the role of the reference's TF32 kernel
(crates/staleynet-cuda/src/kernels/matmul.rs:357-448), against reference::matmul (reference.rs:10-38).

The kernel serves products whose 256 x 256 plan keeps at least half the CUs busy, so the shapes here
are that large (a few thousand rows), ragged where the case calls for it.

Integers of magnitude <= 16 are exact in bf16, their products are exact and every partial sum here
stays below 2^24, so those cases must match bit for bit in any summation order: the whole output is
compared with the exact integer product (float64 arithmetic, exact at these magnitudes), and sampled
outputs with the oracle's reference-order elements. They cover ragged tiles on both output axes, a K
tail that is not a whole 32-deep step, split K, batches with a shared operand, accumulate with a scale;
and the products where the smaller operand is first rounded into the workspace (K-contiguous bf16,
from either stored layout) while the other is rounded as it loads. Rounding to nearest even is pinned
by hand-derived cases, and random inputs are held to the bf16 tolerance (2e-2, device.rs:51-66) on
sampled outputs. Each case first checks that the launch plan really takes this kernel."""
import numpy as np
import pytest

from oracle import oracle
from staleynet_amd import gemm
from staleynet_amd.gemm import BatchStrides, MatmulKernel, MatmulSpec, Shape

pytestmark = pytest.mark.gpu

BF16_TOLERANCE = 2e-2  # device.rs:51-66
SAMPLES = 4096


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


def logical(spec, left, right, b):
    """Matrix b's logical A [rows, inner] and B [inner, cols] as float64 views of the stored operands."""
    m, n, k = spec.rows, spec.cols, spec.inner
    a = left[b * spec.batch.left:][:m * k].astype(np.float64)
    a = a.reshape(k, m).T if spec.left else a.reshape(m, k)
    bm = right[b * spec.batch.right:][:k * n].astype(np.float64)
    bm = bm.reshape(n, k).T if spec.right else bm.reshape(k, n)
    return a, bm


def exact_expected(spec, left, right, initial):
    """The product of integer-valued operands, exact: float64 sums of exact products stay below 2^53,
    and with |sum| < 2^24 the scaled, accumulated result is the one every summation order gives."""
    out = initial.astype(np.float64).copy()
    m, n = spec.rows, spec.cols
    for b in range(spec.batch.count):
        a, bm = logical(spec, left, right, b)
        dst = out[b * spec.batch.output:][:m * n]
        product = (a @ bm).ravel() * float(spec.scale)
        dst[:] = (dst + product) if spec.write else product
    return out.astype(np.float32)


def sample(spec, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, spec.batch.count, SAMPLES)
    r = rng.integers(0, spec.rows, SAMPLES)
    c = rng.integers(0, spec.cols, SAMPLES)
    return b, r, c


def check_sampled_against_oracle(spec, left, right, initial, got, seed):
    b, r, c = sample(spec, seed)
    at = b * spec.batch.output + r * spec.cols + c
    want = oracle.matmul_elements_parallel(product_of(spec), left, right, b, r, c, initial[at] if spec.write else None)
    return want, got[at]


def wide_plan(spec):
    plan = gemm.plan(spec, int(MatmulKernel.MfmaBf16))
    assert plan.path == gemm.PATH_BF16_WIDE, f"path {plan.path}"
    return plan


def integers(rng, count, bound):
    return rng.integers(-bound, bound + 1, size=count).astype(np.float32)


@pytest.mark.parametrize("variant,rows,cols,inner", [
    ("TN", 4100, 2060, 100),   # partial tiles on both output edges; K = 3 steps + a 4-deep tail
    ("NT", 3840, 2304, 64),    # whole tiles, two steps
    ("TT", 2820, 3080, 96),    # A row-contiguous, B K-contiguous, ragged
    ("NT", 3080, 2600, 1000),  # K = 31 steps + 8
    ("TN", 2300, 4360, 36),    # partial tiles each way, a step and a tail
])
def test_wide_is_exact_on_integers(gpu, variant, rows, cols, inner):
    print(f"wide {variant} {rows}x{cols}x{inner}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols + inner)
    left, right = integers(rng, rows * inner, 16), integers(rng, inner * cols, 16)
    initial = integers(rng, rows * cols, 8)
    spec = layout(MatmulSpec.new(rows, cols, inner), variant).scaled(0.5).accumulate()
    plan = wide_plan(spec)
    assert plan.workspace_bytes == (plan.splits * rows * cols * 4 if plan.splits > 1 else 0)  # nothing staged
    got = run_bf16(gpu, spec, left, right, initial)
    assert np.array_equal(exact_expected(spec, left, right, initial), got)
    want, sampled = check_sampled_against_oracle(spec, left, right, initial, got, inner)
    assert np.array_equal(want, sampled)


@pytest.mark.parametrize("variant,rows,cols,inner", [
    ("NN", 32768, 256, 100),   # right operand (row-contiguous) staged through the transposing kernel
    ("NT", 16400, 260, 96),    # right operand (K-contiguous) staged row by row
    ("TN", 260, 32800, 300),   # left operand (row-contiguous) staged, right rounded as loaded
    ("TT", 260, 16400, 64),    # left staged, right K-contiguous
    ("NN", 16500, 300, 1000),  # ragged edges, K = 31 steps + 8
])
def test_wide_with_one_operand_staged_is_exact_on_integers(gpu, variant, rows, cols, inner):
    print(f"wide staged {variant} {rows}x{cols}x{inner}", flush=True)
    rng = np.random.default_rng(rows + 5 * cols + inner)
    left, right = integers(rng, rows * inner, 16), integers(rng, inner * cols, 16)
    initial = integers(rng, rows * cols, 8)
    spec = layout(MatmulSpec.new(rows, cols, inner), variant).scaled(0.5).accumulate()
    plan = wide_plan(spec)
    partials = plan.splits * rows * cols * 4 if plan.splits > 1 else 0
    assert plan.workspace_bytes > partials  # the staged operand sits in the workspace
    got = run_bf16(gpu, spec, left, right, initial)
    assert np.array_equal(exact_expected(spec, left, right, initial), got)
    want, sampled = check_sampled_against_oracle(spec, left, right, initial, got, inner + 1)
    assert np.array_equal(want, sampled)


def test_wide_split_k_is_exact_on_integers(gpu):
    # A weight-gradient shape whose 9 output tiles take K in slices, reduced in slice order.
    rows, cols, inner = 768, 640, 4096
    rng = np.random.default_rng(3)
    left, right = integers(rng, rows * inner, 4), integers(rng, inner * cols, 4)
    initial = integers(rng, rows * cols, 8)
    spec = MatmulSpec.new(rows, cols, inner).left_transposed().accumulate()
    plan = wide_plan(spec)
    assert plan.splits > 1
    got = run_bf16(gpu, spec, left, right, initial)
    assert np.array_equal(exact_expected(spec, left, right, initial), got)
    want, sampled = check_sampled_against_oracle(spec, left, right, initial, got, 5)
    assert np.array_equal(want, sampled)


# "left" and "right": the shared operand is the smaller one and is staged once for the batch (read by
# 3 x 12 tile columns or 3 x 11 tile rows, over the 32 tiles staging asks for).
@pytest.mark.parametrize("shared", ["none", "left", "right"])
def test_wide_batches_and_shared_operands(gpu, shared):
    batches, rows, cols, inner = 3, 2816, 3000, 64
    rng = np.random.default_rng(9)
    left_stride = 0 if shared == "left" else rows * inner
    right_stride = 0 if shared == "right" else inner * cols
    left = integers(rng, rows * inner * (1 if shared == "left" else batches), 16)
    right = integers(rng, inner * cols * (1 if shared == "right" else batches), 16)
    spec = MatmulSpec.new(rows, cols, inner).right_transposed().batched(
        BatchStrides(batches, left_stride, right_stride, rows * cols))
    plan = wide_plan(spec)
    assert (plan.workspace_bytes > 0) == (shared != "none")
    initial = np.zeros(batches * rows * cols, np.float32)
    got = run_bf16(gpu, spec, left, right, initial)
    assert np.array_equal(exact_expected(spec, left, right, initial), got)
    want, sampled = check_sampled_against_oracle(spec, left, right, initial, got, 7)
    assert np.array_equal(want, sampled)


def test_wide_rounds_to_nearest_even(gpu):
    # C = A^T I returns A^T rounded to bf16: row 0 of the stored A (K = n rows of M = n) holds the
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
    n = 4096  # 256 tiles: square, so neither operand is staged and the kernel rounds both as loaded
    a = np.zeros((n, n), np.float32)
    a[0, :len(cases)] = [c[0] for c in cases]
    eye = np.eye(n, dtype=np.float32)
    spec = MatmulSpec.new(n, n, n).left_transposed()
    plan = wide_plan(spec)
    assert plan.workspace_bytes == 0
    out = run_bf16(gpu, spec, a.ravel(), eye.ravel(), np.zeros(n * n, np.float32)).reshape(n, n)
    assert out[:len(cases), 0].tolist() == [np.float32(c[1]) for c in cases]


@pytest.mark.parametrize("variant,rows,cols,inner", [("TN", 1536, 1536, 4096), ("NT", 4096, 2304, 768)])
def test_wide_random_within_bf16_tolerance(gpu, variant, rows, cols, inner):
    left = oracle.random_values(rows * inner, 21)
    right = oracle.random_values(inner * cols, 22)
    initial = oracle.random_values(rows * cols, 23)
    spec = layout(MatmulSpec.new(rows, cols, inner), variant).scaled(0.7).accumulate()
    wide_plan(spec)
    got = run_bf16(gpu, spec, left, right, initial)
    assert np.all(np.isfinite(got))
    want, sampled = check_sampled_against_oracle(spec, left, right, initial, got, 11)
    assert oracle.relative_error(want, sampled) < BF16_TOLERANCE

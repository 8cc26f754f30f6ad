"""GPU parity of ``sn_matmul_column_sums``: Linear::backward's weight-gradient product and bias
gradient (layers/linear.rs:54-59, ``Gpu::matmul`` then ``Gpu::accumulate_column_sums`` of the same
output gradient) in one call, the column sums taken inside the fp32 direct-to-LDS kernel while the
right operand's tiles sit in LDS.

* The product must be bit-identical to ``sn_matmul`` on the same inputs (the same kernel and plan).
* Integers of magnitude <= 16 keep every column sum exact in any order, so there the sums must equal
  the oracle's row-order sums (oracle.accumulate_column_sums, kernels/elementwise.rs:78-93) bit for
  bit: ragged column tiles, a K tail that is not a whole 32-deep step, split K (the slices' sums are
  reduced after the product's partials), both stored layouts of the left operand, the 64-column tile.
* Random inputs: the sums within the reference's fp32 tolerance (1e-5,
  kernels_match_reference.rs:12) of the oracle's, no further from an f64 sum than the oracle is
  (plus 1e-6 of the largest sum), and the same bits on every run.
* bf16 products on the 256 x 256 kernel take the sums from dY's fp32 values before rounding: exact on
  integers, the product bit-identical to sn_matmul's, the sums within the fp32 tolerance on random data.
* Products no fused kernel serves (small bf16 products, bf16 with dY the staged operand, right operand
  columns not a multiple of 4) run as the two calls and must give their bits.
Each fused case first checks, through the host-only planner, that the fused path is the one taken.
"""
import numpy as np
import pytest

from oracle import oracle
from staleynet_amd import gemm
from staleynet_amd.gemm import MatmulKernel, MatmulPanic, MatmulSpec, Shape

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-5  # kernels_match_reference.rs:12


def product_of(spec: MatmulSpec) -> oracle.Product:
    return oracle.Product(spec.rows, spec.cols, spec.inner, bool(spec.left), bool(spec.right), spec.batch.count,
                          spec.batch.left, spec.batch.right, spec.batch.output, spec.scale, bool(spec.write))


def weight_grad_spec(inputs, outputs, rows, left_transposed=True):
    spec = MatmulSpec.new(inputs, outputs, rows)
    if left_transposed:
        spec = spec.left_transposed()
    return spec.accumulate()


def fused(gpu, spec, left, right, initial, sums0, kernel=MatmulKernel.MfmaF32):
    """(output, sums) of sn_matmul_column_sums."""
    gpu.matmul_kernel = kernel
    try:
        lt = gpu.upload(Shape.vector(left.size), left)
        rt = gpu.upload(Shape.vector(right.size), right)
        out = gpu.upload(Shape.vector(initial.size), initial)
        sums = gpu.upload(Shape.vector(sums0.size), sums0)
        gpu.matmul_column_sums(spec, lt, rt, out, sums)
        return gpu.download(out), gpu.download(sums)
    finally:
        gpu.matmul_kernel = MatmulKernel.MfmaF32


def separate(gpu, spec, left, right, initial, sums0, kernel=MatmulKernel.MfmaF32):
    """(output, sums) of sn_matmul followed by sn_accumulate_column_sums over the stored right operand."""
    gpu.matmul_kernel = kernel
    try:
        lt = gpu.upload(Shape.vector(left.size), left)
        rt = gpu.upload(Shape(spec.inner, spec.cols), right)
        out = gpu.upload(Shape.vector(initial.size), initial)
        sums = gpu.upload(Shape.vector(sums0.size), sums0)
        gpu.matmul(spec, lt, rt, out)
        gpu.accumulate_column_sums(rt, sums)
        return gpu.download(out), gpu.download(sums)
    finally:
        gpu.matmul_kernel = MatmulKernel.MfmaF32


def fused_plan(spec, kernel=MatmulKernel.MfmaF32):
    plan = gemm.plan_column_sums(spec, int(kernel))
    assert plan.path == gemm.PATH_F32_DIRECT_SUMS, f"path {plan.path}"
    return plan


@pytest.mark.parametrize("inputs,outputs,rows,left_transposed", [
    (300, 260, 100, True),     # ragged tiles both ways; K = 3 steps + a 4-deep tail
    (256, 512, 64, True),      # whole tiles, two steps
    (132, 136, 36, False),     # left stored row-major (K-contiguous), one step and a tail
    (200, 48, 1000, True),     # the 64-column tile; 31 steps + 8
    (768, 640, 4096, True),    # 30 tiles: K split into slices, reduced in slice order
    (96, 2304, 32768, True),   # the shape of a narrow weight gradient: 18 tiles, many slices
])
def test_fused_sums_are_exact_on_integers(gpu, inputs, outputs, rows, left_transposed):
    print(f"column sums {inputs}x{outputs}x{rows} left_transposed={left_transposed}", flush=True)
    rng = np.random.default_rng(inputs + 3 * outputs + rows)
    bound = 16 if rows <= 4096 else 2
    left = rng.integers(-bound, bound + 1, size=inputs * rows).astype(np.float32)
    right = rng.integers(-bound, bound + 1, size=rows * outputs).astype(np.float32)
    initial = rng.integers(-8, 9, size=inputs * outputs).astype(np.float32)
    sums0 = rng.integers(-8, 9, size=outputs).astype(np.float32)
    spec = weight_grad_spec(inputs, outputs, rows, left_transposed)
    plan = fused_plan(spec)
    if rows >= 4096:
        assert plan.splits > 1
    out, sums = fused(gpu, spec, left, right, initial, sums0)
    want_out = initial.copy()
    oracle.matmul_parallel(product_of(spec), left, right, want_out)
    want_sums = sums0.copy()
    oracle.accumulate_column_sums(right, outputs, want_sums)
    assert np.array_equal(sums, want_sums)
    assert np.array_equal(out, want_out)


@pytest.mark.parametrize("inputs,outputs,rows", [(256, 768, 2048), (768, 2304, 8192), (520, 300, 1000)])
def test_fused_product_is_sn_matmul_and_sums_within_tolerance(gpu, inputs, outputs, rows):
    print(f"column sums random {inputs}x{outputs}x{rows}", flush=True)
    left = oracle.random_values(inputs * rows, 41)
    right = oracle.random_values(rows * outputs, 42)
    initial = oracle.random_values(inputs * outputs, 43)
    sums0 = oracle.random_values(outputs, 44)
    spec = weight_grad_spec(inputs, outputs, rows)
    fused_plan(spec)
    out, sums = fused(gpu, spec, left, right, initial, sums0)
    out2, sums2 = fused(gpu, spec, left, right, initial, sums0)
    sep_out, _ = separate(gpu, spec, left, right, initial, sums0)
    assert np.array_equal(out, sep_out), "the product's bits differ from sn_matmul's"
    assert np.array_equal(out, out2) and np.array_equal(sums, sums2), "results differ between two runs"
    expected = sums0.copy()
    oracle.accumulate_column_sums(right, outputs, expected)
    assert oracle.relative_error(expected, sums) < TOLERANCE
    truth = oracle.column_sums_f64(right, outputs, sums0)
    assert np.max(np.abs(sums - truth)) <= np.max(np.abs(expected - truth)) + 1e-6 * np.max(np.abs(truth))


def test_weight_gradient_at_config_2_scale(gpu):
    # The qkv weight and bias gradients: X [32768, 768], dY [32768, 2304] ~N(0, 1).
    rows, inputs, outputs = 32768, 768, 2304
    spec = weight_grad_spec(inputs, outputs, rows)
    fused_plan(spec)
    x = gpu.zeros(Shape(rows, inputs))
    dy = gpu.zeros(Shape(rows, outputs))
    gpu.fill_normal(x, 11, 1)
    gpu.fill_normal(dy, 12, 2)
    initial = oracle.random_values(outputs, 13)
    dw_fused, dw_separate = gpu.zeros(Shape(inputs, outputs)), gpu.zeros(Shape(inputs, outputs))
    db_fused = gpu.upload(Shape.vector(outputs), initial)
    db_separate = gpu.upload(Shape.vector(outputs), initial)
    gpu.matmul_column_sums(spec, x, dy, dw_fused, db_fused)
    gpu.matmul(spec, x, dy, dw_separate)
    gpu.accumulate_column_sums(dy, db_separate)
    assert np.array_equal(gpu.download(dw_fused), gpu.download(dw_separate))
    values = gpu.download(dy)
    expected = initial.copy()
    oracle.accumulate_column_sums(values, outputs, expected)
    got = gpu.download(db_fused)
    error = oracle.relative_error(expected, got)
    print(f"fused bias gradient 32768x2304: vs oracle {error:.2e}, separate kernel vs oracle "
          f"{oracle.relative_error(expected, gpu.download(db_separate)):.2e}")
    assert error < TOLERANCE


# bf16 on the 256 x 256 kernel: dY's fp32 values are summed in the registers before they are rounded,
# or, where dY is the operand staged as bf16, by the staging pass as it reads them.
# Integers of magnitude <= 2 (exact in bf16; every product sum and column sum stays below 2^24) make the
# product exact in any order: it is compared in full with the exact integer product (float64
# arithmetic), and the sums with the oracle's row-order sums, bit for bit.
@pytest.mark.parametrize("inputs,outputs,rows", [
    (768, 2304, 32768),   # the qkv weight gradient: x^T rounded as loaded (9 tile columns read it), 9 K slices
    (768, 8192, 8192),    # x^T staged as bf16 (32 tile columns read it)
    (768, 768, 32768),    # the out projection's: nothing staged, 28 slices
    (772, 2312, 20010),   # ragged tiles both ways, a K tail
    (3072, 768, 32768),   # the down projection's: dY staged as bf16, the staging pass takes the sums
    (3080, 772, 20010),   # dY staged, ragged: a partial last 64-k tile and column block
])
def test_bf16_fused_sums_are_exact_on_integers(gpu, inputs, outputs, rows):
    print(f"bf16 column sums {inputs}x{outputs}x{rows}", flush=True)
    rng = np.random.default_rng(inputs + outputs + rows)
    left = rng.integers(-2, 3, size=inputs * rows).astype(np.float32)
    right = rng.integers(-2, 3, size=rows * outputs).astype(np.float32)
    initial = rng.integers(-8, 9, size=inputs * outputs).astype(np.float32)
    sums0 = rng.integers(-8, 9, size=outputs).astype(np.float32)
    spec = weight_grad_spec(inputs, outputs, rows)
    assert gemm.plan_column_sums(spec, int(MatmulKernel.MfmaBf16)).path == gemm.PATH_BF16_WIDE_SUMS
    out, sums = fused(gpu, spec, left, right, initial, sums0, MatmulKernel.MfmaBf16)
    x = left.reshape(rows, inputs).astype(np.float64)
    dy = right.reshape(rows, outputs).astype(np.float64)
    want_out = (initial.astype(np.float64) + (x.T @ dy).ravel()).astype(np.float32)
    want_sums = sums0.copy()
    oracle.accumulate_column_sums(right, outputs, want_sums)
    assert np.array_equal(sums, want_sums)
    assert np.array_equal(out, want_out)


@pytest.mark.parametrize("inputs,outputs", [(768, 2304), (3072, 768)])  # nothing staged; dY staged
def test_bf16_fused_product_is_sn_matmul_and_sums_within_tolerance(gpu, inputs, outputs):
    rows = 32768
    print(f"bf16 column sums random {inputs}x{outputs}x{rows}", flush=True)
    left = oracle.random_values(inputs * rows, 71)
    right = oracle.random_values(rows * outputs, 72)
    initial = oracle.random_values(inputs * outputs, 73)
    sums0 = oracle.random_values(outputs, 74)
    spec = weight_grad_spec(inputs, outputs, rows)
    assert gemm.plan_column_sums(spec, int(MatmulKernel.MfmaBf16)).path == gemm.PATH_BF16_WIDE_SUMS
    out, sums = fused(gpu, spec, left, right, initial, sums0, MatmulKernel.MfmaBf16)
    out2, sums2 = fused(gpu, spec, left, right, initial, sums0, MatmulKernel.MfmaBf16)
    sep_out, _ = separate(gpu, spec, left, right, initial, sums0, MatmulKernel.MfmaBf16)
    assert np.array_equal(out, sep_out), "the product's bits differ from sn_matmul's"
    assert np.array_equal(out, out2) and np.array_equal(sums, sums2), "results differ between two runs"
    expected = sums0.copy()
    oracle.accumulate_column_sums(right, outputs, expected)
    assert oracle.relative_error(expected, sums) < TOLERANCE
    truth = oracle.column_sums_f64(right, outputs, sums0)
    assert np.max(np.abs(sums - truth)) <= np.max(np.abs(expected - truth)) + 1e-6 * np.max(np.abs(truth))


@pytest.mark.parametrize("case", ["bf16", "columns_not_multiple_of_4", "empty_rows"])
def test_unfused_products_run_as_the_two_calls(gpu, case):
    inputs, outputs, rows = 96, 80, 300
    kernel = MatmulKernel.MfmaF32
    if case == "bf16":
        inputs, outputs, rows = 256, 512, 256
        kernel = MatmulKernel.MfmaBf16
    elif case == "columns_not_multiple_of_4":
        outputs = 50
    else:
        inputs = 0
    spec = weight_grad_spec(inputs, outputs, rows)
    assert gemm.plan_column_sums(spec, int(kernel)).path not in (gemm.PATH_F32_DIRECT_SUMS, gemm.PATH_BF16_WIDE_SUMS)
    left = oracle.random_values(max(inputs * rows, 1), 51)
    right = oracle.random_values(rows * outputs, 52)
    initial = oracle.random_values(max(inputs * outputs, 1), 53)
    sums0 = oracle.random_values(outputs, 54)
    out, sums = fused(gpu, spec, left, right, initial, sums0, kernel)
    sep_out, sep_sums = separate(gpu, spec, left, right, initial, sums0, kernel)
    assert np.array_equal(out, sep_out)
    assert np.array_equal(sums, sep_sums)


def test_rejected_calls_leave_everything_unchanged(gpu):
    inputs, outputs, rows = 8, 12, 16
    x = gpu.upload(Shape(rows, inputs), oracle.random_values(rows * inputs, 61))
    dy = gpu.upload(Shape(rows, outputs), oracle.random_values(rows * outputs, 62))
    dw = gpu.zeros(Shape(inputs, outputs))
    db = gpu.zeros(Shape.vector(outputs))
    spec = weight_grad_spec(inputs, outputs, rows)
    dw2 = gpu.zeros(Shape(2 * inputs, outputs))  # room for a batch of two outputs
    for bad in (spec.right_transposed(), spec.batched(gemm.BatchStrides(2, 0, 0, inputs * outputs))):
        with pytest.raises(MatmulPanic) as info:
            gpu.matmul_column_sums(bad, x, dy, dw2, db)
        assert info.value.status == gemm.SN_ERR_UNSUPPORTED
    with pytest.raises(MatmulPanic) as info:
        gpu.matmul_column_sums(spec, x, dy, dw, gpu.zeros(Shape.vector(outputs + 1)))
    assert info.value.status == gemm.SN_ERR_LENGTH_MISMATCH
    # Sums of the right length that overlap the right operand, then the output (views that own nothing).
    for target in (dy, dw):
        view = gemm.Tensor(gpu, target.pointer + 4 * 4, Shape.vector(outputs))
        try:
            with pytest.raises(MatmulPanic) as info:
                gpu.matmul_column_sums(spec, x, dy, dw, view)
            assert info.value.status == gemm.SN_ERR_ALIASING
        finally:
            view.pointer = 0
    gpu.synchronize()
    assert not gpu.download(dw).any() and not gpu.download(dw2).any() and not gpu.download(db).any()

"""GPU parity of Linear's bias kernels and the fused bias epilogue, through the C ABI.

* ``sn_add_row_bias`` (``Gpu::add_row_bias``, ops/elementwise.rs:30-41): one f32
  add per element, so bit-identical to the oracle (kernels/elementwise.rs:62-68).
* ``sn_accumulate_column_sums`` (``Gpu::accumulate_column_sums``,
  ops/elementwise.rs:43-58): a fixed-order parallel sum, checked against the
  oracle's row-order f32 sum at the reference's tolerance, against an f64 sum,
  and for run-to-run determinism.
* ``sn_matmul_bias`` (Linear::forward's matmul + add_row_bias, layers/linear.rs:
  46-47, in one pass): bit-identical to ``sn_matmul`` followed by
  ``sn_add_row_bias`` on every kernel path, and within tolerance of the oracle.
The reference's own elementwise test (tests/kernels_match_reference.rs:125-170)
is restated first, on its inputs.
"""
import numpy as np
import pytest

from oracle import oracle
from staleynet_amd.gemm import BatchStrides, MatmulKernel, MatmulPanic, MatmulSpec, Shape

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-5  # kernels_match_reference.rs:12


def test_reference_elementwise_test_bias_and_column_sums(gpu):
    rows, cols = 9, 50
    values = oracle.random_values(rows * cols, 7)
    bias = oracle.random_values(cols, 9)
    out = gpu.upload(Shape(rows, cols), values)
    gpu.add_row_bias(out, gpu.upload(Shape.vector(cols), bias))
    expected = values.copy()
    oracle.add_row_bias(expected, cols, bias)
    assert np.array_equal(gpu.download(out), expected)

    sums = gpu.upload(Shape.vector(cols), bias)
    gpu.accumulate_column_sums(gpu.upload(Shape(rows, cols), values), sums)
    expected = bias.copy()
    oracle.accumulate_column_sums(values, cols, expected)
    assert oracle.relative_error(expected, gpu.download(sums)) < TOLERANCE


@pytest.mark.parametrize("rows,cols", [(1, 1), (1, 4), (7, 13), (5, 3), (33, 2304), (2048, 768), (3, 16384)])
def test_add_row_bias_is_bit_identical(gpu, rows, cols):
    values = oracle.random_values(rows * cols, rows + 3)
    bias = oracle.random_values(cols, cols + 5)
    out = gpu.upload(Shape(rows, cols), values)
    gpu.add_row_bias(out, gpu.upload(Shape.vector(cols), bias))
    expected = values.copy()
    oracle.add_row_bias(expected, cols, bias)
    assert np.array_equal(gpu.download(out), expected)


def test_bias_length_must_equal_the_columns(gpu):
    out = gpu.zeros(Shape(4, 6))
    with pytest.raises(AssertionError, match="add_row_bias: bias length must equal output columns"):
        gpu.add_row_bias(out, gpu.zeros(Shape.vector(5)))
    with pytest.raises(AssertionError, match="accumulate_column_sums: sums length must equal input columns"):
        gpu.accumulate_column_sums(out, gpu.zeros(Shape.vector(7)))


@pytest.mark.parametrize("rows,cols", [(1, 1), (1, 5), (9, 50), (1000, 13), (4096, 7), (64, 256), (300, 1028),
                                       (2048, 768), (8192, 2048)])
def test_column_sums_match_the_row_order_sum(gpu, rows, cols):
    values = oracle.random_values(rows * cols, rows * 7 + cols)
    initial = oracle.random_values(cols, 11)
    sums = gpu.upload(Shape.vector(cols), initial)
    gpu.accumulate_column_sums(gpu.upload(Shape(rows, cols), values), sums)
    got = gpu.download(sums)
    expected = initial.copy()
    oracle.accumulate_column_sums(values, cols, expected)
    assert oracle.relative_error(expected, got) < TOLERANCE
    truth = oracle.column_sums_f64(values, cols, initial)
    assert np.max(np.abs(got - truth)) <= np.max(np.abs(expected - truth)) + 1e-6 * np.max(np.abs(truth))


def test_column_sums_at_config_2_scale_and_determinism(gpu):
    # The qkv bias gradient: dY is [32768, 2304] ~N(0, 1); sums start from LCG values.
    rows, cols = 32768, 2304
    dy = gpu.zeros(Shape(rows, cols))
    gpu.fill_normal(dy, 1234, 7)
    initial = oracle.random_values(cols, 13)
    first = gpu.upload(Shape.vector(cols), initial)
    second = gpu.upload(Shape.vector(cols), initial)
    gpu.accumulate_column_sums(dy, first)
    gpu.accumulate_column_sums(dy, second)
    a, b = gpu.download(first), gpu.download(second)
    assert np.array_equal(a, b), "column sums differ between two runs"
    values = gpu.download(dy)
    expected = initial.copy()
    oracle.accumulate_column_sums(values, cols, expected)
    truth = oracle.column_sums_f64(values, cols, initial)
    error = oracle.relative_error(expected, a)
    print(f"column sums 32768x2304: vs oracle {error:.2e}, GPU vs f64 "
          f"{np.max(np.abs(a - truth)) / np.max(np.abs(truth)):.2e}, oracle vs f64 "
          f"{np.max(np.abs(expected - truth)) / np.max(np.abs(truth)):.2e}")
    assert error < TOLERANCE


def fused_and_separate(gpu, spec, left, right, bias, initial, kernel=MatmulKernel.MfmaF32):
    """(sn_matmul_bias result, sn_matmul + sn_add_row_bias result) on the same inputs."""
    gpu.matmul_kernel = kernel
    try:
        lt = gpu.upload(Shape.vector(left.size), left)
        rt = gpu.upload(Shape.vector(right.size), right)
        bt = gpu.upload(Shape.vector(bias.size), bias)
        fused = gpu.upload(Shape.vector(initial.size), initial)
        gpu.matmul_bias(spec, lt, rt, bt, fused)
        separate = gpu.upload(Shape.vector(initial.size), initial)
        gpu.matmul(spec, lt, rt, separate)
        # The output matrices are contiguous here: add_row_bias over all their rows at once.
        assert initial.size == spec.batch.count * spec.rows * spec.cols
        rows_view = separate.reshaped(Shape(spec.batch.count * spec.rows, spec.cols))
        gpu.add_row_bias(rows_view, bt)
        return gpu.download(fused), gpu.download(rows_view)
    finally:
        gpu.matmul_kernel = MatmulKernel.MfmaF32


CASES = {
    # (spec, left size, right size, output size); every GEMM path of the library
    "NN direct-to-LDS (c0 qkv)": (MatmulSpec.new(2048, 768, 256), 2048 * 256, 256 * 768, 2048 * 768),
    "NN ragged, scalar loads": (MatmulSpec.new(130, 197, 101), 130 * 101, 101 * 197, 130 * 197),
    "NN scaled accumulate": (MatmulSpec.new(256, 384, 64).scaled(0.7).accumulate(), 256 * 64, 64 * 384, 256 * 384),
    "TN split-K accumulate": (MatmulSpec.new(256, 256, 16384).left_transposed().accumulate(), 16384 * 256,
                              16384 * 256, 256 * 256),
    "TN split-K ragged": (MatmulSpec.new(130, 66, 9000).left_transposed(), 9000 * 130, 9000 * 66, 130 * 66),
    "NT narrow": (MatmulSpec.new(512, 64, 96).right_transposed(), 512 * 96, 64 * 96, 512 * 64),
    "decode M=1": (MatmulSpec.new(1, 2304, 768), 768, 768 * 2304, 2304),
    "decode M=7 split": (MatmulSpec.new(7, 768, 3072), 7 * 3072, 3072 * 768, 7 * 768),
    "decode M=16 head": (MatmulSpec.new(16, 16384, 768), 16 * 768, 768 * 16384, 16 * 16384),
    "batched": (MatmulSpec.new(64, 96, 40).batched(BatchStrides(3, 64 * 40, 0, 64 * 96)), 3 * 64 * 40, 40 * 96,
                3 * 64 * 96),
    "masked causal output": (MatmulSpec.new(128, 128, 32).right_transposed().causal_output(), 128 * 32, 128 * 32,
                             128 * 128),
}


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("kernel", [MatmulKernel.MfmaF32, MatmulKernel.Simple, MatmulKernel.MfmaBf16])
def test_matmul_bias_equals_matmul_then_add_row_bias(gpu, name, kernel):
    spec, nl, nr, no = CASES[name]
    seed = sum(map(ord, name))
    left = oracle.random_values(nl, seed)
    right = oracle.random_values(nr, seed + 1)
    bias = oracle.random_values(spec.cols, seed + 2)
    initial = oracle.random_values(no, seed + 3)
    fused, separate = fused_and_separate(gpu, spec, left, right, bias, initial, kernel)
    assert np.array_equal(fused, separate), f"{name}: fused bias differs from matmul + add_row_bias"
    if kernel == MatmulKernel.MfmaBf16:
        return
    expected = initial.copy()
    p = oracle.Product(spec.rows, spec.cols, spec.inner, bool(spec.left), bool(spec.right), spec.batch.count,
                       spec.batch.left, spec.batch.right, spec.batch.output, spec.scale, bool(spec.write))
    oracle.matmul(p, left, right, expected)
    if spec.mask:
        # the causal extension zeroes (overwrite) the keys past each query before the bias
        e = expected.reshape(spec.rows, spec.cols)
        e[np.triu_indices(spec.rows, 1, spec.cols)] = 0.0
    for b in range(spec.batch.count):
        view = expected[b * spec.batch.output: b * spec.batch.output + spec.rows * spec.cols]
        oracle.add_row_bias(view, spec.cols, bias)
    assert oracle.relative_error(expected, fused) < TOLERANCE


def test_matmul_bias_validation(gpu):
    spec = MatmulSpec.new(4, 5, 3)
    x, w, y = gpu.zeros(Shape(4, 3)), gpu.zeros(Shape(3, 5)), gpu.zeros(Shape(4, 5))
    with pytest.raises(MatmulPanic):
        gpu.matmul_bias(spec, x, w, gpu.zeros(Shape.vector(4)), y)
    with pytest.raises(MatmulPanic):
        gpu.matmul_bias(spec, x, w, y, y)  # bias overlaps the output


def test_linear_layer_round_trip_at_config_0(gpu):
    """Linear::forward and ::backward (linear.rs:43-63) at config 0's QKV shape: the fused
    forward, the weight gradient (TN accumulate), the bias gradient and the input gradient,
    each against the oracle."""
    rows, inputs, outputs = 2048, 256, 768
    x = oracle.random_values(rows * inputs, 31)
    w = oracle.random_values(inputs * outputs, 32) * np.float32(0.02)
    b = oracle.random_values(outputs, 33)
    dy = oracle.random_values(rows * outputs, 34)
    dw0 = oracle.random_values(inputs * outputs, 35)
    db0 = oracle.random_values(outputs, 36)
    X, W, B, DY = (gpu.upload(Shape(rows, inputs), x), gpu.upload(Shape(inputs, outputs), w),
                   gpu.upload(Shape.vector(outputs), b), gpu.upload(Shape(rows, outputs), dy))
    Y, DX = gpu.zeros(Shape(rows, outputs)), gpu.zeros(Shape(rows, inputs))
    DW, DB = gpu.upload(Shape(inputs, outputs), dw0), gpu.upload(Shape.vector(outputs), db0)
    gpu.matmul_bias(MatmulSpec.new(rows, outputs, inputs), X, W, B, Y)
    gpu.matmul(MatmulSpec.new(inputs, outputs, rows).left_transposed().accumulate(), X, DY, DW)
    gpu.accumulate_column_sums(DY, DB)
    gpu.matmul(MatmulSpec.new(rows, inputs, outputs).right_transposed(), DY, W, DX)

    y = np.zeros(rows * outputs, np.float32)
    oracle.matmul(oracle.Product(rows, outputs, inputs), x, w, y)
    oracle.add_row_bias(y, outputs, b)
    dw = dw0.copy()
    oracle.matmul(oracle.Product(inputs, outputs, rows, left_transposed=True, accumulate=True), x, dy, dw)
    db = db0.copy()
    oracle.accumulate_column_sums(dy, outputs, db)
    dx = np.zeros(rows * inputs, np.float32)
    oracle.matmul(oracle.Product(rows, inputs, outputs, right_transposed=True), dy, w, dx)
    for name, expected, tensor in (("y", y, Y), ("dW", dw, DW), ("db", db, DB), ("dX", dx, DX)):
        assert oracle.relative_error(expected, gpu.download(tensor)) < TOLERANCE, name

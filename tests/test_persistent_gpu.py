"""The persistent kernels: fp32 128 x 128 tiles (SN_PATH_F32_PERSISTENT, gemm_dma.hip's dma_persistent) and
bf16 256 x 256 tiles (SN_PATH_BF16_WIDE with a persistent grid, gemm_bf16_wide_persistent_kernel).

Each of its workgroups loops over work items (matrix, K slice, tile) and loads the next item's first two
K-steps under the current tile's last two, so the tile's output stores go out behind those loads. Per tile it
runs the one-tile kernel's schedule (the same K-steps, chunks and MFMA order), so its output must be bit for
bit the one-tile kernel's. A product that runs persistent is therefore compared with the same outputs
computed by calls too small to run persistent (row blocks, or single matrices of a batch: each output
element's sum is the same one); split-K weight gradients run on integer operands, where every summation
order is exact, against the exact product; a sample of rows goes through the oracle (the reference's loop,
reference.rs:10-38) at the fp32 tolerance (2e-2 for bf16 inputs); and reruns must give the same bits. The
device is an MI355X (256 CUs), whose plans these are."""
import numpy as np
import pytest

from oracle import oracle
from staleynet_amd import gemm
from staleynet_amd.gemm import BatchStrides, MatmulSpec, Precision, Shape

pytestmark = pytest.mark.gpu

CUS = 256
TOLERANCE = 1e-5
BF16_TOLERANCE = 2e-2


def upload(gpu, values):
    return gpu.upload(Shape.vector(values.size), values.astype(np.float32))


def assert_persistent(spec, expected=True):
    plan = gemm.plan(spec, cu_count=CUS)
    if spec.precision == Precision.Bf16:
        assert plan.path == gemm.PATH_BF16_WIDE and (plan.persistent_grid > 0) == expected, (spec, plan.path)
    else:
        assert (plan.path == gemm.PATH_F32_PERSISTENT) == expected, (spec, plan.path)
    return plan


def sample_rows_against_oracle(spec, left, right, out, rows):
    """The oracle's full-precision loop on a few output rows (NN / NT storage, unbatched)."""
    m, n, k = spec.rows, spec.cols, spec.inner
    tolerance = BF16_TOLERANCE if spec.precision == Precision.Bf16 else TOLERANCE
    for row in rows:
        product = oracle.Product(1, n, k, False, bool(spec.right), 1, 0, 0, 0, spec.scale, False)
        expected = np.zeros(n, np.float32)
        oracle.matmul(product, left[row * k:(row + 1) * k], right, expected)
        error = oracle.relative_error(expected, out[row * n:(row + 1) * n])
        assert error < tolerance, f"row {row}: relative error {error}"


@pytest.mark.parametrize("layout,m,n,k,parts,precision", [
    ("NN", 4096, 4096, 768, 2, Precision.F32), ("NT", 8192, 2048, 512, 2, Precision.F32),
    ("NN", 4096, 16384, 256, 8, Precision.F32),
    # K not a whole number of 32-deep steps (six steps, the last 4 deep): the loads past K read zeros.
    ("NN", 4096, 4096, 164, 2, Precision.F32), ("NT", 4096, 4096, 164, 2, Precision.F32),
    # bf16, 256 x 256 tiles (the weight staged as bf16 in both): 512 work items against blocks of 128.
    ("NN", 32768, 1024, 768, 4, Precision.Bf16), ("NT", 32768, 1024, 768, 4, Precision.Bf16)])
def test_persistent_matches_the_one_tile_kernel_bit_for_bit(gpu, layout, m, n, k, parts, precision):
    print(f"persistent {layout} {m}x{n}x{k} {precision.name} against {parts} row blocks", flush=True)
    spec = MatmulSpec.new(m, n, k).with_precision(precision)
    if layout == "NT":
        spec = spec.right_transposed()
    assert_persistent(spec)
    block = MatmulSpec.new(m // parts, n, k).with_precision(precision)
    if layout == "NT":
        block = block.right_transposed()
    block_plan = assert_persistent(block, expected=False)
    tile = 256 if precision == Precision.Bf16 else 128
    assert (block_plan.tile_rows, block_plan.tile_cols, block_plan.splits) == (tile, tile, 1)
    left = oracle.random_values(m * k, 11)
    right = oracle.random_values(k * n, 12) * np.float32(0.02)
    lt, rt = upload(gpu, left), upload(gpu, right)
    out = gpu.zeros(Shape(m, n))
    gpu.matmul(spec, lt, rt, out)
    whole = gpu.download(out)
    # The same rows, one block of rows per call (the one-tile kernel).
    pieces = []
    for p in range(parts):
        rows = m // parts
        lp = upload(gpu, left[p * rows * k:(p + 1) * rows * k])
        op = gpu.zeros(Shape(rows, n))
        gpu.matmul(block, lp, rt, op)
        pieces.append(gpu.download(op))
        lp.free()
        op.free()
    blocks = np.concatenate(pieces)
    assert np.array_equal(whole.view(np.uint32), blocks.view(np.uint32)), \
        f"{int(np.count_nonzero(whole != blocks))} outputs differ from the one-tile kernel"
    sample_rows_against_oracle(spec, left, right, whole, [0, 1, m // 2 + 3, m - 1])
    # A rerun over a dirtied output gives the same bits.
    gpu.fill_normal(out, 7, 7)
    gpu.matmul(spec, lt, rt, out)
    assert np.array_equal(gpu.download(out).view(np.uint32), whole.view(np.uint32))
    for t in (lt, rt, out):
        t.free()


def test_persistent_batches_match_single_matrices(gpu):
    # Four 4096 x 2048 x 256 matrices (2048 work items; one alone is 512, too few to run persistent, and
    # takes the same 128 x 128 tiles), the left operand shared by the batch (stride 0).
    count, m, n, k = 4, 4096, 2048, 256
    spec = MatmulSpec.new(m, n, k).batched(BatchStrides(count, 0, k * n, m * n)).scaled(0.5)
    assert_persistent(spec)
    single = MatmulSpec.new(m, n, k).scaled(0.5)
    single_plan = assert_persistent(single, expected=False)
    assert (single_plan.tile_rows, single_plan.tile_cols, single_plan.splits) == (128, 128, 1)
    left = oracle.random_values(m * k, 21)
    right = oracle.random_values(count * k * n, 22)
    lt, rt = upload(gpu, left), upload(gpu, right)
    out = gpu.zeros(Shape(count * m, n))
    gpu.matmul(spec, lt, rt, out)
    whole = gpu.download(out)
    for b in range(count):
        rb = upload(gpu, right[b * k * n:(b + 1) * k * n])
        ob = gpu.zeros(Shape(m, n))
        gpu.matmul(single, lt, rb, ob)
        got = whole[b * m * n:(b + 1) * m * n]
        assert np.array_equal(got.view(np.uint32), gpu.download(ob).view(np.uint32)), f"matrix {b}"
        if b == count - 1:
            sample_rows_against_oracle(single, left, right[b * k * n:(b + 1) * k * n], got, [0, m - 1])
        rb.free()
        ob.free()
    for t in (lt, rt, out):
        t.free()


def test_persistent_forward_with_bias_matches_the_one_tile_kernel(gpu):
    # The fused Linear forward (sn_matmul_bias): the bias rides in the persistent kernel's epilogue.
    m, n, k = 4096, 4096, 768
    spec = MatmulSpec.new(m, n, k)
    assert_persistent(spec)
    left = oracle.random_values(m * k, 31)
    right = oracle.random_values(k * n, 32) * np.float32(0.02)
    bias = oracle.random_values(n, 33)
    lt, rt, bt = upload(gpu, left), upload(gpu, right), upload(gpu, bias)
    out = gpu.zeros(Shape(m, n))
    gpu.matmul_bias(spec, lt, rt, bt, out)
    whole = gpu.download(out)
    half = MatmulSpec.new(m // 2, n, k)
    half_plan = assert_persistent(half, expected=False)
    assert (half_plan.tile_rows, half_plan.tile_cols, half_plan.splits) == (128, 128, 1)
    for p in range(2):
        lp = upload(gpu, left[p * (m // 2) * k:(p + 1) * (m // 2) * k])
        op = gpu.zeros(Shape(m // 2, n))
        gpu.matmul_bias(half, lp, rt, bt, op)
        assert np.array_equal(gpu.download(op).view(np.uint32), whole[p * (m // 2) * n:(p + 1) * (m // 2) * n]
                              .view(np.uint32)), f"row half {p}"
        lp.free()
        op.free()
    # The reference's combine then add_row_bias (elementwise.rs:62-93), row by row.
    for row in (0, m - 1):
        product = oracle.Product(1, n, k, False, False, 1, 0, 0, 0, 1.0, False)
        expected = np.zeros(n, np.float32)
        oracle.matmul(product, left[row * k:(row + 1) * k], right, expected)
        oracle.add_row_bias(expected, n, bias)
        assert oracle.relative_error(expected, whole[row * n:(row + 1) * n]) < TOLERANCE
    for t in (lt, rt, bt, out):
        t.free()


@pytest.mark.parametrize("inputs,outputs,tokens,precision", [(768, 2304, 32768, Precision.F32),
                                                              (768, 4096, 32768, Precision.F32),
                                                              (768, 16384, 8192, Precision.Bf16)])
def test_persistent_split_weight_gradients_are_exact_on_integers(gpu, inputs, outputs, tokens, precision):
    # dW += x^T dY at config 2's qkv shape and wider ones (K split into even slices), on integer operands
    # of magnitude <= 2 (exact in bf16 too): every partial sum is an integer below 2^24, so any summation
    # order gives the exact result.
    spec = MatmulSpec.new(inputs, outputs, tokens).left_transposed().accumulate().with_precision(precision)
    plan = assert_persistent(spec)
    assert plan.splits > 1
    print(f"persistent TN {inputs}x{outputs}x{tokens}: {plan.splits} slices of {plan.k_per_split}", flush=True)
    rng = np.random.default_rng(outputs)
    x = rng.integers(-2, 3, size=(tokens, inputs)).astype(np.float32)
    dy = rng.integers(-2, 3, size=(tokens, outputs)).astype(np.float32)
    dw0 = rng.integers(-8, 9, size=(inputs, outputs)).astype(np.float32)
    xt, dyt, dwt = upload(gpu, x.ravel()), upload(gpu, dy.ravel()), upload(gpu, dw0.ravel())
    gpu.matmul(spec, xt, dyt, dwt)
    got = gpu.download(dwt).reshape(inputs, outputs)
    # float32 products of these integers are exact whatever the order (sums below 2^24).
    exact = dw0 + x.T @ dy
    assert np.array_equal(got, exact), f"{int(np.count_nonzero(got != exact))} outputs differ"
    for t in (xt, dyt, dwt):
        t.free()

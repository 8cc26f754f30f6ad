"""Seeded random sweeps of products across the planner's choices, against the exact product; then the
fused Linear entry points (product + bias, weight gradient + bias gradient) the same way.

Each case draws a layout (NN / NT / TN / TT), sizes from 1 to a few thousand (so that aligned, ragged,
unaligned, few-row, split-K, small-tile, 256 x 256 bf16 and staged bf16 plans all come up), a batch of 1 to 3
with a shared (stride 0) operand now and then, a scale, overwrite or accumulate, and fp32 or bf16
precision. The operands are integers of magnitude <= 4 (exact in bf16), K <= 4096, so every partial
sum is an integer below 2^24 and the scale a power of two: every kernel, in any summation order, must
return the exact product, which float64 computes here (the reference's loop, reference.rs:10-38, is
exact on these inputs too). Every output element is compared bit for bit, and the sweep checks that
it reached the plan paths it is meant to cover."""
import numpy as np
import pytest

from staleynet_amd import gemm
from staleynet_amd.gemm import BatchStrides, MatmulKernel, MatmulSpec, Precision, Shape

pytestmark = pytest.mark.gpu

CASES = 96


def draw(rng):
    def size(hi):
        return int(np.exp(rng.uniform(0.0, np.log(hi))))

    kind = rng.random()
    if kind < 0.2:  # large enough for the 256 x 256 bf16 tiles and the staged operands
        rows, cols, inner = (int(rng.integers(1024, 3073)), int(rng.integers(1024, 3073)),
                             int(rng.integers(128, 2049)))
    else:
        rows = 1 + size(2048) if kind < 0.85 else int(rng.integers(1, 17))
        cols, inner = 1 + size(2048), 1 + size(4096)
    if kind < 0.2 or rng.random() < 0.6:  # aligned sizes take the direct-to-LDS and wide kernels
        cols, inner = 4 * ((cols + 3) // 4), 4 * ((inner + 3) // 4)
    spec = MatmulSpec.new(rows, cols, inner)
    layout = ("NN", "NT", "TN", "TT")[int(rng.integers(0, 4))]
    if layout[0] == "T":
        spec = spec.left_transposed()
    if layout[1] == "T":
        spec = spec.right_transposed()
    count = int(rng.choice([1, 1, 1, 2, 3]))
    if count > 1:
        shared = rng.integers(0, 3)  # 0: none, 1: left shared, 2: right shared
        spec = spec.batched(BatchStrides(count, 0 if shared == 1 else rows * inner,
                                         0 if shared == 2 else inner * cols, rows * cols))
    spec = spec.scaled(float(rng.choice([1.0, 0.5, 2.0, 0.25])))
    if rng.random() < 0.5:
        spec = spec.accumulate()
    if rng.random() < 0.35:
        spec = spec.with_precision(Precision.Bf16)
    return layout, spec


def exact(spec, left, right, initial):
    m, n, k = spec.rows, spec.cols, spec.inner
    out = initial.astype(np.float64).copy()
    for b in range(spec.batch.count):
        a = left[b * spec.batch.left:][:m * k].astype(np.float64)
        a = a.reshape(k, m).T if spec.left else a.reshape(m, k)
        w = right[b * spec.batch.right:][:k * n].astype(np.float64)
        w = w.reshape(n, k).T if spec.right else w.reshape(k, n)
        dst = out[b * spec.batch.output:][:m * n]
        product = (a @ w).ravel() * spec.scale
        dst[:] = dst + product if spec.write else product
    return out.astype(np.float32)


def test_random_products_are_exact_across_the_planners_choices(gpu):
    rng = np.random.default_rng(20261202)
    paths = set()
    for case in range(CASES):
        layout, spec = draw(rng)
        kernel = MatmulKernel.MfmaBf16 if spec.precision == Precision.Bf16 else MatmulKernel.MfmaF32
        plan = gemm.plan(spec, int(kernel))
        paths.add(plan.path)
        print(f"case {case}: {layout} {spec.rows}x{spec.cols}x{spec.inner} batch {spec.batch.count} "
              f"strides ({spec.batch.left}, {spec.batch.right}) scale {spec.scale} accumulate {bool(spec.write)} "
              f"precision {int(spec.precision)} path {plan.path} splits {plan.splits}", flush=True)
        left_len = (spec.batch.count - 1) * spec.batch.left + spec.rows * spec.inner
        right_len = (spec.batch.count - 1) * spec.batch.right + spec.inner * spec.cols
        out_len = spec.batch.count * spec.rows * spec.cols
        left = rng.integers(-4, 5, size=left_len).astype(np.float32)
        right = rng.integers(-4, 5, size=right_len).astype(np.float32)
        initial = rng.integers(-8, 9, size=out_len).astype(np.float32)
        lt, rt = gpu.upload(Shape.vector(left_len), left), gpu.upload(Shape.vector(right_len), right)
        ot = gpu.upload(Shape.vector(out_len), initial)
        gpu.matmul(spec, lt, rt, ot)
        got = gpu.download(ot)
        for t in (lt, rt, ot):
            t.free()
        want = exact(spec, left, right, initial)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"case {case}: {bad.size} outputs differ, first at {bad[0]}: {got[bad[0]]} != {want[bad[0]]}"
    print("paths covered", sorted(paths), flush=True)
    wanted = {gemm.PATH_F32_DIRECT, gemm.PATH_F32_REGISTER, gemm.PATH_FEW_ROWS, gemm.PATH_BF16_WIDE,
              gemm.PATH_BF16_DIRECT, gemm.PATH_BF16_REGISTER, gemm.PATH_BF16_STAGED}
    assert wanted <= paths, f"the sweep reached {sorted(paths)}"


def upload_case(gpu, rng, spec):
    left_len = (spec.batch.count - 1) * spec.batch.left + spec.rows * spec.inner
    right_len = (spec.batch.count - 1) * spec.batch.right + spec.inner * spec.cols
    out_len = spec.batch.count * spec.rows * spec.cols
    left = rng.integers(-4, 5, size=left_len).astype(np.float32)
    right = rng.integers(-4, 5, size=right_len).astype(np.float32)
    initial = rng.integers(-8, 9, size=out_len).astype(np.float32)
    tensors = (gpu.upload(Shape.vector(left_len), left), gpu.upload(Shape.vector(right_len), right),
               gpu.upload(Shape.vector(out_len), initial))
    return (left, right, initial), tensors


def test_random_products_with_the_fused_bias_are_exact(gpu):
    # sn_matmul_bias: Linear::forward's matmul then add_row_bias (linear.rs:46-47), the bias added to
    # every output matrix of the batch after the combine, as its own rounded add.
    rng = np.random.default_rng(7)
    for case in range(48):
        layout, spec = draw(rng)
        print(f"bias case {case}: {layout} {spec.rows}x{spec.cols}x{spec.inner} batch {spec.batch.count} "
              f"accumulate {bool(spec.write)} precision {int(spec.precision)}", flush=True)
        (left, right, initial), (lt, rt, ot) = upload_case(gpu, rng, spec)
        bias = rng.integers(-8, 9, size=spec.cols).astype(np.float32)
        bt = gpu.upload(Shape.vector(spec.cols), bias)
        gpu.matmul_bias(spec, lt, rt, bt, ot)
        got = gpu.download(ot)
        for t in (lt, rt, ot, bt):
            t.free()
        want = exact(spec, left, right, initial) + np.tile(bias, spec.batch.count * spec.rows)
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"case {case}: {bad.size} outputs differ"


def test_random_weight_gradients_with_fused_column_sums_are_exact(gpu):
    # sn_matmul_column_sums: Linear::backward's weight gradient dW (+)= X^T dY and the bias gradient
    # accumulate_column_sums(dY) (linear.rs:54-59), over weight shapes from tiny to config 2's and
    # token counts up to 4096 (left stored as X, or already transposed).
    rng = np.random.default_rng(11)
    paths = set()
    for case in range(48):
        def size(hi):
            return int(np.exp(rng.uniform(0.0, np.log(hi))))

        big = rng.random() < 0.3
        inputs = int(rng.integers(512, 3073)) if big else 1 + size(1024)
        outputs = int(rng.integers(512, 3073)) if big else 1 + size(1024)
        tokens = int(rng.integers(2048, 4097)) if big else 1 + size(4096)
        if big or rng.random() < 0.5:
            inputs, outputs, tokens = (4 * ((v + 3) // 4) for v in (inputs, outputs, tokens))
        spec = MatmulSpec.new(inputs, outputs, tokens)
        if rng.random() < 0.8:
            spec = spec.left_transposed()
        spec = spec.scaled(float(rng.choice([1.0, 0.5]))).accumulate()
        if rng.random() < 0.4:
            spec = spec.with_precision(Precision.Bf16)
        kernel = MatmulKernel.MfmaBf16 if spec.precision == Precision.Bf16 else MatmulKernel.MfmaF32
        plan = gemm.plan_column_sums(spec, int(kernel))
        paths.add(plan.path)
        print(f"column sums case {case}: {inputs}x{outputs}x{tokens} left transposed {bool(spec.left)} "
              f"precision {int(spec.precision)} path {plan.path} splits {plan.splits}", flush=True)
        (left, right, initial), (lt, rt, ot) = upload_case(gpu, rng, spec)
        sums0 = rng.integers(-8, 9, size=outputs).astype(np.float32)
        st = gpu.upload(Shape.vector(outputs), sums0)
        gpu.matmul_column_sums(spec, lt, rt, ot, st)
        got, sums = gpu.download(ot), gpu.download(st)
        for t in (lt, rt, ot, st):
            t.free()
        assert np.array_equal(got, exact(spec, left, right, initial)), f"case {case}: product"
        want_sums = (sums0.astype(np.float64) + right.astype(np.float64).reshape(tokens, outputs).sum(axis=0))
        assert np.array_equal(sums, want_sums.astype(np.float32)), f"case {case}: column sums"
    assert {gemm.PATH_F32_DIRECT_SUMS, gemm.PATH_BF16_WIDE_SUMS} <= paths, f"the sweep reached {sorted(paths)}"

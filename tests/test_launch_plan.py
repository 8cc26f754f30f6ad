"""CPU tests of the launch geometry, the counterpart of the reference's launch.rs unit tests
(crates/staleynet-cuda/src/launch.rs:59-113): the grid ``sn_plan_matmul`` reports for a product
(the same describe functions the launchers take their grids from) and the workgroup -> (matrix,
K slice, tile) map the tiled kernels evaluate on the device (``sn_tile_map``, the same function).
For every product of configs 0-4 and the attention batches: each (matrix, slice, tile) is covered by
exactly one workgroup, the slices cover K, and the batch regrouping gives each XCD whole matrices.
No GPU is used."""
import numpy as np
import pytest

from staleynet_amd import gemm
from staleynet_amd.gemm import BatchStrides, MatmulKernel, MatmulSpec, Precision

XCDS = 8
MODELS = {  # (tokens, width, ffn) of configs 0, 1, 2
    "c0": (4 * 512, 256, 1024),
    "c1": (8 * 1024, 512, 2048),
    "c2": (16 * 2048, 768, 3072),
}


def linear_products(tokens, d, f):
    """Every product of one training step's Linears (linear.rs:43-63) and the 16-codebook head."""
    for i, o in ((d, 3 * d), (d, d), (d, f), (f, d), (d, 16 * 1024)):
        yield f"NN {tokens}x{o}x{i}", MatmulSpec.new(tokens, o, i)
        yield f"TN {i}x{o}x{tokens}", MatmulSpec.new(i, o, tokens).left_transposed().accumulate()
        yield f"NT {tokens}x{i}x{o}", MatmulSpec.new(tokens, i, o).right_transposed()


def attention_products(bh=192, t=2048, h=64):
    """Config 3's six products (attention.rs:206-260), dense and causal."""
    per = BatchStrides(bh, t * h, t * h, t * t)
    scores = MatmulSpec.new(t, t, h).right_transposed().batched(per)
    mix = MatmulSpec.new(t, h, t).batched(BatchStrides(bh, t * t, t * h, t * h))
    dv = MatmulSpec.new(t, h, t).left_transposed().batched(BatchStrides(bh, t * t, t * h, t * h))
    yield "S", scores
    yield "S causal", scores.causal_output()
    yield "O", mix
    yield "O causal", mix.causal_left()
    yield "dV causal", dv.causal_left()
    yield "dQ causal", mix.scaled(0.125).causal_left()


def decode_products():
    """Config 4: M in {1, 4, 16} against the 111.5M weights and the head (decode.rs:123-161)."""
    for m in (1, 4, 16):
        for k, n in ((768, 2304), (768, 768), (768, 3072), (3072, 768), (768, 16384)):
            yield f"decode M={m} {k}x{n}", MatmulSpec.new(m, n, k)
    # The decode scores and mix against a 1408-position cache, 12 heads.
    yield "decode scores", MatmulSpec.new(1, 1408, 64).right_transposed().batched(
        BatchStrides(12, 64, 1408 * 64, 1408)).causal_output(700)
    yield "decode mix", MatmulSpec.new(1, 64, 1408).batched(BatchStrides(12, 1408, 1408 * 64, 64)).causal_left(700)


def all_products():
    for name, (tokens, d, f) in MODELS.items():
        for label, spec in linear_products(tokens, d, f):
            yield f"{name} {label}", spec, MatmulKernel.MfmaF32
    for label, spec in linear_products(*MODELS["c2"]):
        yield f"c2 bf16 {label}", spec.with_precision(Precision.Bf16), MatmulKernel.MfmaF32
    for label, spec in attention_products():
        yield f"c3 {label}", spec, MatmulKernel.MfmaF32
    for label, spec in attention_products(bh=12 * 16, t=2048, h=64):
        if "causal" in label:
            yield f"c3 bf16 {label}", spec.with_precision(Precision.Bf16), MatmulKernel.MfmaF32
    for label, spec in decode_products():
        yield f"c4 {label}", spec, MatmulKernel.MfmaF32


CASES = list(all_products())


def check_tiled_cover(plan):
    """Every (matrix, slice, tile row, tile column) of one launch is produced exactly once."""
    matrix, split, tm, tn = gemm.tile_map(plan.workgroups, plan.tiles_m, plan.tiles_n, plan.splits)
    assert matrix.max() < plan.batches_per_launch and split.max() < plan.splits
    assert tm.max() < plan.tiles_m and tn.max() < plan.tiles_n
    key = ((matrix.astype(np.int64) * plan.splits + split) * plan.tiles_m + tm) * plan.tiles_n + tn
    assert len(np.unique(key)) == plan.workgroups == plan.batches_per_launch * plan.splits * plan.tiles_m * plan.tiles_n
    return matrix, split


@pytest.mark.parametrize("label,spec,kernel", CASES, ids=[c[0] for c in CASES])
def test_every_tile_and_slice_is_launched_once(label, spec, kernel):
    plan = gemm.plan(spec, int(kernel))
    k = spec.inner
    if spec.mask == gemm.Mask.CausalLeft and plan.path == gemm.PATH_FEW_ROWS:
        # The decode mix multiplies keys up to the last row's horizon only; the cache tail is not read.
        k = min(k, spec.rows + spec.query_offset)
    assert plan.splits >= 1 and plan.k_per_split >= 1
    # The slices cover K: the last one starts inside it.
    assert (plan.splits - 1) * plan.k_per_split < max(k, 1) <= plan.splits * plan.k_per_split
    if plan.path in gemm.TILED_PATHS:
        assert plan.tiles_m == -(-spec.rows // plan.tile_rows) and plan.tiles_n == -(-spec.cols // plan.tile_cols)
        assert plan.launches * plan.batches_per_launch >= spec.batch.count
        assert (plan.launches - 1) * plan.batches_per_launch < spec.batch.count
        if plan.splits > 1:  # slices are whole K-steps
            step = 64 if plan.path == gemm.PATH_BF16_STAGED else 32
            assert plan.k_per_split % step == 0
        check_tiled_cover(plan)
    elif plan.path == gemm.PATH_FEW_ROWS:
        width = few_row_slab_width(spec.rows, spec.cols, spec.batch.count)
        assert plan.tile_cols == width and plan.tiles_n == -(-spec.cols // width)
        assert spec.rows <= 16 and plan.k_per_split % 16 == 0
        assert plan.workgroups == plan.tiles_n * plan.splits * spec.batch.count
    else:
        assert plan.path == gemm.PATH_FEW_ROWS_NT and spec.rows <= 4 and plan.splits == 1


def test_weight_gradients_take_the_column_sums_into_the_product():
    # Linear::backward's dW += x^T dY with db += column sums of dY (linear.rs:54-59), at the
    # configurations' shapes: the fp32 product keeps its plan, and each K slice adds N floats of sums.
    for inputs, outputs in ((768, 2304), (768, 768), (768, 3072), (3072, 768), (256, 768), (96, 48)):
        spec = MatmulSpec.new(inputs, outputs, 32768).left_transposed().accumulate()
        product = gemm.plan(spec)
        fused = gemm.plan_column_sums(spec)
        assert product.path in (gemm.PATH_F32_DIRECT, gemm.PATH_F32_PERSISTENT)
        assert fused.path == gemm.PATH_F32_DIRECT_SUMS
        assert (fused.splits, fused.k_per_split, fused.tiles_m, fused.tiles_n) == \
            (product.splits, product.k_per_split, product.tiles_m, product.tiles_n)
        extra = fused.splits * outputs * 4 if fused.splits > 1 else 0
        assert fused.workspace_bytes == product.workspace_bytes + extra
        check_tiled_cover(fused)
    # A workspace that holds the product's partial sums but not the sums beside them: fewer slices.
    spec = MatmulSpec.new(768, 2304, 32768).left_transposed().accumulate()
    product = gemm.plan(spec)
    tight = gemm.plan_column_sums(spec, workspace_bytes=product.workspace_bytes)
    assert tight.path == gemm.PATH_F32_DIRECT_SUMS and tight.splits < product.splits
    assert tight.workspace_bytes <= product.workspace_bytes
    # bf16 on the 256 x 256 kernel: the sums ride in it where dY reaches it as fp32 (x^T staged, for
    # the head, or nothing staged), N floats more per slice; the down projection's dY is the operand
    # staged as bf16, and the staging pass takes the sums, one partial per 64 k and column.
    for inputs, outputs in ((768, 2304), (768, 768), (768, 3072), (768, 16384)):
        bf16 = MatmulSpec.new(inputs, outputs, 32768).left_transposed().accumulate().with_precision(Precision.Bf16)
        product, fused = gemm.plan(bf16), gemm.plan_column_sums(bf16)
        assert product.path == gemm.PATH_BF16_WIDE and fused.path == gemm.PATH_BF16_WIDE_SUMS
        assert (fused.splits, fused.tiles_m, fused.tiles_n) == (product.splits, product.tiles_m, product.tiles_n)
        extra = fused.splits * outputs * 4 if fused.splits > 1 else 0
        assert fused.workspace_bytes == product.workspace_bytes + extra
    # (The plain down product, read by 12 tile rows, rounds dY as it loads it; the fused one stages it
    # for the sums whatever the reuse.)
    down = MatmulSpec.new(3072, 768, 32768).left_transposed().accumulate().with_precision(Precision.Bf16)
    product, fused = gemm.plan(down), gemm.plan_column_sums(down)
    assert fused.path == gemm.PATH_BF16_WIDE_SUMS
    # The same slices (the same summation order, so sn_matmul's bits) with dY staged or not.
    assert (fused.splits, fused.k_per_split, fused.tiles_m, fused.tiles_n) == \
        (product.splits, product.k_per_split, product.tiles_m, product.tiles_n)
    assert product.workspace_bytes == product.splits * 3072 * 768 * 4 * (product.splits > 1)
    assert fused.workspace_bytes == (768 * 32768 * 2 + fused.splits * 3072 * 768 * 4 * (fused.splits > 1)
                                     + (32768 // 64) * 768 * 4)
    odd = MatmulSpec.new(96, 50, 300).left_transposed()
    assert gemm.plan_column_sums(odd).path == gemm.PATH_F32_REGISTER
    # The unsupported forms are rejected by the planner as by the call.
    for bad in (spec.right_transposed(), spec.batched(gemm.BatchStrides(2, 0, 0, 768 * 2304))):
        with pytest.raises(gemm.GpuError):
            gemm.plan_column_sums(bad)


def test_configs_take_the_expected_kernel_families():
    assert gemm.plan(MatmulSpec.new(32768, 2304, 768)).path == gemm.PATH_F32_PERSISTENT
    # Large bf16 products round their fp32 operands as they load them, 256 x 256 tiles; the forward
    # and input-gradient products first round the (smaller) weight into the workspace.
    forward = gemm.plan(MatmulSpec.new(32768, 2304, 768).with_precision(Precision.Bf16))
    assert forward.path == gemm.PATH_BF16_WIDE and (forward.tile_rows, forward.tile_cols) == (256, 256)
    assert forward.splits == 1 and forward.workspace_bytes == 2304 * 768 * 2  # the staged weight
    wgrad = gemm.plan(MatmulSpec.new(768, 2304, 32768).left_transposed().with_precision(Precision.Bf16))
    assert wgrad.path == gemm.PATH_BF16_WIDE and wgrad.splits > 1
    # x^T is staged only where at least 32 tiles read it: the head's weight gradient (64 tile columns),
    # not the qkv one's (9), whose workspace holds only the partial sums.
    assert wgrad.workspace_bytes == wgrad.splits * 768 * 2304 * 4
    head = gemm.plan(MatmulSpec.new(768, 16384, 32768).left_transposed().with_precision(Precision.Bf16))
    assert head.workspace_bytes == head.splits * 768 * 16384 * 4 * (head.splits > 1) + 768 * 32768 * 2
    dgrad = gemm.plan(MatmulSpec.new(32768, 768, 2304).right_transposed().with_precision(Precision.Bf16))
    assert dgrad.path == gemm.PATH_BF16_WIDE and dgrad.workspace_bytes == 768 * 2304 * 2
    # The staged operand is blocked by 32-deep steps (each step's tile rows one 16 KB run), so its
    # loads need no offsets across K: with K in the millions the weight gradient still stages x^T
    # (rows padded to 256, K to 32), beside the partial sums.
    huge = gemm.plan(MatmulSpec.new(256, 8192, 5_000_000).left_transposed().with_precision(Precision.Bf16),
                     workspace_bytes=1 << 40)
    assert huge.path == gemm.PATH_BF16_WIDE
    assert huge.workspace_bytes == huge.splits * 256 * 8192 * 4 * (huge.splits > 1) + 256 * 5_000_000 * 2
    long_k = gemm.plan(MatmulSpec.new(200, 8192, 500_001).left_transposed().with_precision(Precision.Bf16),
                       workspace_bytes=1 << 40)
    assert long_k.workspace_bytes == long_k.splits * 200 * 8192 * 4 * (long_k.splits > 1) + 256 * 500_032 * 2
    # Too small for the wide tiles, and fewer 128 x 128 tiles than CUs: no staging pass, 64 x 64 tiles
    # rounding fp32 fragments as they are read.
    tiny = gemm.plan(MatmulSpec.new(96, 2304, 768).with_precision(Precision.Bf16))
    assert tiny.path == gemm.PATH_BF16_DIRECT and (tiny.tile_rows, tiny.tile_cols) == (64, 64)
    # 256 x 256 tiles that would leave more than half the CUs idle (config 0's 2048 x 768 x 256: 24 of
    # them) also go to the 128-wide kernels; 128 tiles are enough.
    small = gemm.plan(MatmulSpec.new(2048, 768, 256).with_precision(Precision.Bf16))
    assert small.path == gemm.PATH_BF16_DIRECT and (small.tile_rows, small.tile_cols) == (64, 64)
    mid = gemm.plan(MatmulSpec.new(4096, 4096, 256).with_precision(Precision.Bf16), cu_count=1024)
    assert mid.path == gemm.PATH_BF16_STAGED and (mid.tile_rows, mid.tile_cols) == (128, 256)
    assert gemm.plan(MatmulSpec.new(2048, 4096, 256).with_precision(Precision.Bf16)).path == gemm.PATH_BF16_WIDE
    assert gemm.plan(MatmulSpec.new(2048, 768, 256).with_precision(Precision.Bf16), cu_count=32).path == \
        gemm.PATH_BF16_WIDE
    # fp32: 64 x 64 tiles when the 128 x 128 plan has fewer workgroups than CUs.
    f32_small = gemm.plan(MatmulSpec.new(2048, 768, 256))
    assert f32_small.path == gemm.PATH_F32_DIRECT and (f32_small.tile_rows, f32_small.tile_cols) == (64, 64)
    assert (gemm.plan(MatmulSpec.new(2048, 768, 256), cu_count=32).tile_rows,
            gemm.plan(MatmulSpec.new(2048, 4096, 256)).tile_rows) == (128, 128)
    # ... and when it has fewer than two per CU with under 24 K-steps each (one GPU's share of config 2
    # over 8 GPUs; the 42.9M model's 512-wide products), but not on longer slices.
    for spec in (MatmulSpec.new(4096, 768, 768), MatmulSpec.new(4096, 768, 768).right_transposed(),
                 MatmulSpec.new(768, 768, 4096).left_transposed().accumulate(), MatmulSpec.new(8192, 512, 512)):
        assert gemm.plan(spec).tile_rows == 64, spec
    for spec in (MatmulSpec.new(768, 768, 32768).left_transposed().accumulate(),
                 MatmulSpec.new(512, 1536, 8192).left_transposed().accumulate(), MatmulSpec.new(32768, 768, 768)):
        assert gemm.plan(spec).tile_rows == 128, spec
    # Too narrow for a quarter tile: the staged kernels keep it.
    assert gemm.plan(MatmulSpec.new(32768, 64, 768).right_transposed().with_precision(Precision.Bf16)).path != \
        gemm.PATH_BF16_WIDE
    assert gemm.plan(MatmulSpec.new(1, 2304, 768)).path == gemm.PATH_FEW_ROWS
    assert gemm.plan(MatmulSpec.new(1, 1408, 64).right_transposed()).path == gemm.PATH_FEW_ROWS_NT
    # Masked bf16 products keep their fp32 stages (rounded per fragment).
    assert gemm.plan(MatmulSpec.new(2048, 64, 2048).causal_left().with_precision(Precision.Bf16)).path == \
        gemm.PATH_BF16_DIRECT
    # Unaligned operands go through registers.
    assert gemm.plan(MatmulSpec.new(130, 197, 100)).path == gemm.PATH_F32_REGISTER
    assert gemm.plan(MatmulSpec.new(256, 256, 256), left=gemm.ALIGNED_ADDRESS + 4).path == gemm.PATH_F32_REGISTER
    assert gemm.plan(MatmulSpec.new(2, 3, 4), int(MatmulKernel.Simple)).path == gemm.PATH_REFERENCE_ORDER
    assert gemm.plan(MatmulSpec.new(0, 3, 4)).path == gemm.PATH_NONE


def check_persistent_rules(spec, plan, cus):
    """The persistent fp32 grid: two workgroups per CU, rounded down to whole XCDs, at least two work
    items each; whole 128 x 128 tiles that read nothing back; every slice an even number of 32-deep
    K-steps; one launch; no mask; K above the streaming-store range. The persistent bf16 256 x 256
    grid: one workgroup per CU, whole tiles that read nothing back, slices of an even number (at least
    4) of K-steps, more items than workgroups: two each, or tiles of at most 32 K-steps."""
    if plan.path in (gemm.PATH_BF16_WIDE, gemm.PATH_BF16_WIDE_SUMS) and plan.persistent_grid:
        grid = plan.persistent_grid
        assert grid == cus // 8 * 8 and plan.workgroups > grid and plan.launches == 1
        assert spec.rows % 256 == 0 and spec.cols % 256 == 0 and (plan.splits > 1 or not spec.write)
        steps = -(-plan.k_per_split // 32)
        last = -(-(spec.inner - (plan.splits - 1) * plan.k_per_split) // 32)
        assert steps % 2 == 0 and last % 2 == 0 and last >= 4
        assert plan.workgroups >= 2 * grid or steps <= 32
        return
    if plan.path != gemm.PATH_F32_PERSISTENT:
        assert plan.persistent_grid == 0
        return
    grid = plan.persistent_grid
    assert grid == 2 * cus // 8 * 8 and plan.workgroups >= 2 * grid
    assert (plan.tile_rows, plan.tile_cols) == (128, 128)
    assert spec.rows % 128 == 0 and spec.cols % 128 == 0 and spec.mask == gemm.Mask.None_
    assert plan.splits > 1 or not spec.write
    assert plan.launches == 1 and spec.inner > 128
    last = spec.inner - (plan.splits - 1) * plan.k_per_split
    assert -(-plan.k_per_split // 32) % 2 == 0 and -(-last // 32) % 2 == 0


def test_persistent_products():
    # Config 2's forward and input-gradient products, its qkv and head weight gradients (split K, even
    # slices) and one GPU's share of the head run persistent; so does an NT product with an odd step
    # count's neighbour ruled out: every one of these plans obeys the rules above.
    persistent = [MatmulSpec.new(32768, 2304, 768), MatmulSpec.new(32768, 768, 768),
                  MatmulSpec.new(32768, 768, 2304).right_transposed(), MatmulSpec.new(32768, 768, 16384).right_transposed(),
                  MatmulSpec.new(768, 2304, 32768).left_transposed().accumulate(),
                  MatmulSpec.new(768, 16384, 32768).left_transposed().accumulate(),
                  MatmulSpec.new(4096, 16384, 768)]
    for spec in persistent:
        plan = gemm.plan(spec)
        assert plan.path == gemm.PATH_F32_PERSISTENT, (spec, plan.path)
        check_persistent_rules(spec, plan, 256)
        check_tiled_cover(plan)
    # Not persistent fp32: masked, ragged, accumulating without a split, odd slices, one item per slot,
    # K in the streaming-store range; bf16 takes its own kernels.
    others = [MatmulSpec.new(2048, 2048, 64).right_transposed().batched(BatchStrides(192, 2048 * 64, 2048 * 64,
                                                                                   2048 * 2048)).causal_output(),
              MatmulSpec.new(32768, 2300, 768), MatmulSpec.new(32768, 2304, 768).accumulate(),
              MatmulSpec.new(768, 3072, 32768).left_transposed().accumulate(),
              MatmulSpec.new(8192, 1024, 768),
              MatmulSpec.new(2048, 2048, 64).right_transposed().batched(BatchStrides(192, 2048 * 64, 2048 * 64,
                                                                                   2048 * 2048)),
              MatmulSpec.new(32768, 2304, 768).with_precision(Precision.Bf16)]
    for spec in others:
        plan = gemm.plan(spec)
        assert plan.path != gemm.PATH_F32_PERSISTENT, (spec, plan.path)
        assert plan.persistent_grid == 0 or plan.path == gemm.PATH_BF16_WIDE, (spec, plan.path)
    # The grid follows the CU count.
    assert gemm.plan(MatmulSpec.new(32768, 2304, 768), cu_count=80).persistent_grid == 160
    # bf16 on the 256 x 256 kernel: config 2's forward products and the wide input gradient loop over
    # their tiles; the 768-wide products with long K keep the one-tile launch.
    bf16 = Precision.Bf16
    for spec in (MatmulSpec.new(32768, 2304, 768), MatmulSpec.new(32768, 768, 768), MatmulSpec.new(32768, 16384, 768),
                 MatmulSpec.new(32768, 3072, 768).right_transposed(),
                 MatmulSpec.new(768, 16384, 32768).left_transposed().accumulate()):
        plan = gemm.plan(spec.with_precision(bf16))
        assert plan.path == gemm.PATH_BF16_WIDE and plan.persistent_grid == 256, spec
        check_persistent_rules(spec, plan, 256)
        check_tiled_cover(plan)
    for spec in (MatmulSpec.new(32768, 768, 3072), MatmulSpec.new(32768, 768, 2304).right_transposed(),
                 MatmulSpec.new(768, 2304, 32768).left_transposed().accumulate(), MatmulSpec.new(8192, 1024, 768)):
        plan = gemm.plan(spec.with_precision(bf16))
        assert plan.path == gemm.PATH_BF16_WIDE and plan.persistent_grid == 0, spec


def test_tiles_round_up_and_keep_the_batch_axis():
    # launch.rs:88-99: a ragged edge adds a tile; the batch stays on the grid.
    spec = MatmulSpec.new(129, 257, 64).batched(BatchStrides(3, 129 * 64, 64 * 257, 129 * 257))
    plan = gemm.plan(spec)
    assert (plan.tile_rows, plan.tile_cols) == (128, 128)
    assert (plan.tiles_m, plan.tiles_n, plan.splits) == (2, 3, 1)
    assert plan.batches_per_launch == 3 and plan.launches == 1 and plan.workgroups == 18 and plan.threads == 256
    # An output 64 columns wide takes the narrow tile (three workgroups per CU).
    narrow = gemm.plan(MatmulSpec.new(2048, 64, 2048))
    assert (narrow.tile_rows, narrow.tile_cols) == (128, 64)
    # The reference-order kernel: 16x16 threads per 16x16 outputs (launch.rs:77-86's shape).
    simple = gemm.plan(spec, int(MatmulKernel.Simple))
    assert (simple.tile_rows, simple.tile_cols, simple.threads) == (16, 16, 256)
    assert (simple.tiles_m, simple.tiles_n, simple.batches_per_launch) == (9, 17, 3)


def test_split_k_only_for_few_tiles_and_within_the_workspace():
    # c2's weight gradients (K = 32768, 36-768 tiles) split K; the forward products do not.
    assert gemm.plan(MatmulSpec.new(32768, 2304, 768)).splits == 1
    dw = MatmulSpec.new(768, 768, 32768).left_transposed().accumulate()
    full = gemm.plan(dw)
    assert full.splits > 1 and full.workspace_bytes == full.splits * 768 * 768 * 4
    # A smaller workspace caps the slices; none leaves a single pass.
    capped = gemm.plan(dw, workspace_bytes=4 * 768 * 768 * 4)
    assert 1 < capped.splits <= 4
    assert gemm.plan(dw, workspace_bytes=0).splits == 1
    # Masked and batched products never split.
    assert all(p.splits == 1 for p in (gemm.plan(s) for _, s in attention_products()))


def test_batched_launches_give_each_xcd_whole_matrices():
    # 192 attention matrices of 256 tiles: every XCD receives 24 whole heads, so the causal mix of
    # full and skipped tiles is the same on every XCD.
    plan = gemm.plan(MatmulSpec.new(2048, 2048, 64).right_transposed().batched(
        BatchStrides(192, 2048 * 64, 2048 * 64, 2048 * 2048)).causal_output())
    matrix, _ = check_tiled_cover(plan)
    xcd = np.arange(plan.workgroups) % XCDS
    for x in range(XCDS):
        heads, counts = np.unique(matrix[xcd == x], return_counts=True)
        assert len(heads) == 192 // XCDS and np.all(counts == plan.tiles_m * plan.tiles_n)
        assert heads.max() - heads.min() == len(heads) - 1  # a contiguous run


def test_split_products_give_each_xcd_whole_slices():
    plan = gemm.plan(MatmulSpec.new(768, 768, 32768).left_transposed().accumulate())
    _, split = check_tiled_cover(plan)
    xcd = np.arange(plan.workgroups) % XCDS
    tiles = plan.tiles_m * plan.tiles_n
    for x in range(XCDS):
        slices, counts = np.unique(split[xcd == x], return_counts=True)
        # Whole slices, except where a slice straddles two XCDs' ranges.
        assert np.sum(counts == tiles) >= len(slices) - 2


def test_tile_map_rejects_bad_arguments():
    with pytest.raises(gemm.GpuError):
        gemm.tile_map(0, 1, 1, 1)
    with pytest.raises(gemm.GpuError):
        gemm.plan(MatmulSpec.new(2, 3, 4).batched(BatchStrides(0, 0, 0, 0)))


# ---- randomized plans ------------------------------------------------------------------

from hypothesis import HealthCheck, given, settings  # noqa: E402
from hypothesis import strategies as st  # noqa: E402

TILE_SIZES = {gemm.PATH_F32_DIRECT: {(128, 128), (128, 64), (64, 64)},
              gemm.PATH_F32_PERSISTENT: {(128, 128)},
              gemm.PATH_F32_DIRECT_SUMS: {(128, 128), (128, 64), (64, 64)},
              gemm.PATH_BF16_WIDE: {(256, 256)},
              gemm.PATH_BF16_STAGED: {(128, 128), (128, 256), (128, 64)},
              gemm.PATH_BF16_DIRECT: {(128, 128), (128, 256), (128, 64), (64, 64)}}


@settings(max_examples=300, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(m=st.integers(1, 5000), n=st.integers(1, 5000), k=st.integers(1, 40000),
       left_t=st.booleans(), right_t=st.booleans(), batch=st.sampled_from([1, 1, 1, 2, 3, 12]),
       bf16=st.booleans(), cus=st.sampled_from([32, 80, 256, 304]),
       workspace=st.sampled_from([0, 1 << 20, 64 << 20, 1536 << 20]), align4=st.booleans())
def test_random_plans_cover_the_product_once(m, n, k, left_t, right_t, batch, bf16, cus, workspace, align4):
    # Shapes with 16-byte rows take the direct-to-LDS kernels, the rest the register-staged ones; any CU
    # count and workspace. Whatever the plan, its slices cover K, its tiles cover the output, the
    # workspace it asks for holds its partial sums, and the workgroup map visits each tile once.
    if align4:
        m, n, k = (max(4, x // 4 * 4) for x in (m, n, k))
    spec = MatmulSpec.new(m, n, k)
    if left_t:
        spec = spec.left_transposed()
    if right_t:
        spec = spec.right_transposed()
    if batch > 1:
        spec = spec.batched(BatchStrides(batch, m * k, k * n, m * n))
    if bf16:
        spec = spec.with_precision(Precision.Bf16)
    try:
        plan = gemm.plan(spec, cu_count=cus, workspace_bytes=workspace)
    except gemm.GpuError as err:
        assert err.status == gemm.SN_ERR_WORKSPACE
        return
    assert (plan.splits - 1) * plan.k_per_split < k <= plan.splits * plan.k_per_split
    if plan.path in TILE_SIZES:
        assert (plan.tile_rows, plan.tile_cols) in TILE_SIZES[plan.path], plan.path
    if plan.path in gemm.TILED_PATHS:
        assert plan.tiles_m == -(-m // plan.tile_rows) and plan.tiles_n == -(-n // plan.tile_cols)
        if plan.splits > 1:
            assert plan.workspace_bytes >= plan.splits * m * n * 4
        if plan.workgroups <= 1 << 16:
            check_tiled_cover(plan)
    check_persistent_rules(spec, plan, cus)
    # The 256 x 256 bf16 tiles only where they keep half the CUs busy.
    if plan.path == gemm.PATH_BF16_WIDE:
        assert 2 * plan.tiles_m * plan.tiles_n * plan.splits * batch >= cus
    assert plan.workspace_bytes <= workspace


@settings(max_examples=200, deadline=None)
@given(inputs=st.integers(1, 4000), outputs=st.integers(1, 4000), rows=st.integers(1, 70000),
       cus=st.sampled_from([80, 256]), workspace=st.sampled_from([0, 1 << 20, 1536 << 20]), bf16=st.booleans())
def test_random_column_sum_plans_keep_the_product_plan(inputs, outputs, rows, cus, workspace, bf16):
    # The weight-gradient spec of linear.rs:54-56: fused or not, the product's tiles and slices are
    # sn_matmul's; fused, the workspace adds N floats per slice.
    spec = MatmulSpec.new(inputs, outputs, rows).left_transposed().accumulate()
    if bf16:
        spec = spec.with_precision(Precision.Bf16)
    try:
        product = gemm.plan(spec, cu_count=cus, workspace_bytes=workspace)
    except gemm.GpuError:
        product = None
    try:
        fused = gemm.plan_column_sums(spec, cu_count=cus, workspace_bytes=workspace)
    except gemm.GpuError as err:
        assert err.status == gemm.SN_ERR_WORKSPACE
        return
    assert fused.workspace_bytes <= workspace
    if fused.path in (gemm.PATH_F32_DIRECT_SUMS, gemm.PATH_BF16_WIDE_SUMS):
        assert bf16 == (fused.path == gemm.PATH_BF16_WIDE_SUMS) and outputs % 4 == 0 and inputs % 4 == 0
        if fused.splits > 1:
            assert fused.workspace_bytes >= fused.splits * (inputs * outputs + outputs) * 4
        if fused.workgroups <= 1 << 16:
            check_tiled_cover(fused)
    elif product is not None:
        assert (fused.path, fused.tiles_m, fused.tiles_n, fused.splits) == \
            (product.path, product.tiles_m, product.tiles_n, product.splits)


# The few-row kernel's split hand-off uses its own zeroed slots (4 Mi words per context and in the
# allocation-free scratch): (splits - 1) slices of rows x (slab width) words per column block and matrix.
HANDOFF_WORDS = 1 << 20


def few_row_slab_width(m, n, batch):
    """Columns per workgroup of the few-row kernel: 32 for one row of x against one weight narrower
    than 256 64-column slabs (a weight K is split for), else 64."""
    return 32 if m == 1 and batch == 1 and -(-n // 64) < 256 else 64


@settings(max_examples=300, deadline=None)
@given(m=st.integers(1, 16), n=st.integers(1, 20000), k=st.integers(1, 200000),
       batch=st.sampled_from([1, 1, 2, 3, 12, 200]), cus=st.sampled_from([80, 256, 304]))
def test_few_row_split_plans_fit_the_handoff_slots(m, n, k, batch, cus):
    n = max(4, n // 4 * 4)
    spec = MatmulSpec.new(m, n, k)
    if batch > 1:
        spec = spec.batched(BatchStrides(batch, m * k, k * n, m * n))
    plan = gemm.plan(spec, cu_count=cus)
    if plan.path != gemm.PATH_FEW_ROWS:
        return
    assert plan.workspace_bytes == 0  # the hand-off never touches the workspace
    width = few_row_slab_width(m, n, batch)
    assert plan.tile_cols == width and plan.tiles_n == -(-n // width)
    assert plan.workgroups == plan.tiles_n * plan.splits * batch
    assert batch * plan.tiles_n * (plan.splits - 1) * m * width <= HANDOFF_WORDS


def test_decode_products_keep_the_few_row_path():
    # Every config-4 product (M = 1, 4, 16 against the 111.5M model's weights and the head).
    for m in (1, 4, 16):
        for k, n in ((768, 2304), (768, 768), (768, 3072), (3072, 768), (768, 16384)):
            plan = gemm.plan(MatmulSpec.new(m, n, k))
            assert plan.path == gemm.PATH_FEW_ROWS, (m, k, n, plan.path)
            assert plan.splits == 1 or plan.splits * plan.tiles_n <= 448


def test_single_row_layer_products_take_the_measured_slabs_and_slices():
    # M = 1 against the config-4 weights: 32-column slabs for the layer products, in the slices that
    # measured fastest (qkv 3, out 6, up whole; down 8, as fast as 6), and 64-column slabs for the head
    # (256 of them).
    for k, n, width, splits in ((768, 2304, 32, 3), (768, 768, 32, 6), (768, 3072, 32, 1), (3072, 768, 32, 8),
                                (768, 16384, 64, 1)):
        plan = gemm.plan(MatmulSpec.new(1, n, k))
        assert (plan.tile_cols, plan.splits) == (width, splits), (k, n, plan.tile_cols, plan.splits)
    # Two rows, or a batch of matrices, keep the 64-column slabs.
    assert gemm.plan(MatmulSpec.new(2, 768, 768)).tile_cols == 64
    assert gemm.plan(MatmulSpec.new(1, 64, 1408).batched(BatchStrides(12, 1408, 1408 * 64, 64))).tile_cols == 64

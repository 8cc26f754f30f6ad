"""GPU parity of the training attention that keeps no probabilities in memory: the forward with row
statistics (``sn_causal_attention_with_stats``) and the backward that rebuilds P from them
(``sn_causal_attention_backward``), against the oracle's restatement of the reference's calls in
CausalSelfAttention::forward and ::backward (crates/staleynet-model/src/layers/attention.rs:206-260):
the scores product, causal_softmax (reference.rs:100-119), the dP and dV products, softmax_backward
(reference.rs:121-137) and the dQ and dK products (reference.rs:19-38), at the reference's fp32
tolerance. Cases: ragged blocks, query offsets, more or fewer keys than queries, head dims 32 / 64 /
128, config 3's whole 192-head launch (eight heads across it compared in full, statistics included),
reruns bit-identical, a workspace left holding NaN, and the entry point's checks. For head dims 32 and
64 dQ comes from the key kernel's partial sums per key block when the workspace holds them (all heads
at once or in runs of heads), else from the query kernel; both ways are checked, and dK and dV must
not depend on the way."""
import numpy as np
import pytest

from oracle import oracle
from staleynet_amd.gemm import Gpu, GpuError, Shape

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-5  # kernels_match_reference.rs:12


def product(rows, cols, inner, lt=False, rt=False, batch=(1, 0, 0, 0), scale=1.0):
    return oracle.Product(rows, cols, inner, lt, rt, batch[0], batch[1], batch[2], batch[3], scale, False)


def reference(q, k, v, d_out, heads, queries, keys, h, scale, offset):
    """The reference's forward and backward calls on the oracle: O, P's row maximum and sum, dQ, dK, dV."""
    qb, kb, sb = queries * h, keys * h, queries * keys
    scores = np.zeros(heads * sb, np.float32)
    oracle.matmul_parallel(product(queries, keys, h, rt=True, batch=(heads, qb, kb, sb)), q, k, scores)
    visible = np.minimum(np.arange(queries) + offset + 1, keys)
    scaled = scores.reshape(heads, queries, keys) * np.float32(scale)
    mask = np.arange(keys)[None, :] < visible[:, None]
    row_max = np.where(mask[None], scaled, -np.inf).max(axis=2)
    p = scores.copy()
    oracle.causal_softmax(p, queries, keys, scale, offset)
    out = np.zeros(heads * qb, np.float32)
    oracle.matmul_parallel(product(queries, h, keys, batch=(heads, sb, kb, qb)), p, v, out)
    dp = np.zeros(heads * sb, np.float32)
    oracle.matmul_parallel(product(queries, keys, h, rt=True, batch=(heads, qb, kb, sb)), d_out, v, dp)
    dv = np.zeros(heads * kb, np.float32)
    oracle.matmul_parallel(product(keys, h, queries, lt=True, batch=(heads, sb, qb, kb)), p, d_out, dv)
    oracle.softmax_backward(p, dp, keys)
    dq = np.zeros(heads * qb, np.float32)
    oracle.matmul_parallel(product(queries, h, keys, batch=(heads, sb, kb, qb), scale=scale), dp, k, dq)
    dk = np.zeros(heads * kb, np.float32)
    oracle.matmul_parallel(product(keys, h, queries, lt=True, batch=(heads, sb, qb, kb), scale=scale), dp, q, dk)
    return out, row_max, dq, dk, dv


def run(gpu, heads, queries, keys, h, scale, offset, seed):
    rng = np.random.default_rng(seed)
    q = rng.normal(0, 1, heads * queries * h).astype(np.float32)
    k = rng.normal(0, 1, heads * keys * h).astype(np.float32)
    v = rng.normal(0, 1, heads * keys * h).astype(np.float32)
    d_out = rng.normal(0, 1, heads * queries * h).astype(np.float32)
    Q, K, V, dO = (gpu.upload(Shape.vector(x.size), x) for x in (q, k, v, d_out))
    O = gpu.upload(Shape.vector(heads * queries * h), np.full(heads * queries * h, np.nan, np.float32))
    stats = gpu.zeros(Shape.vector(2 * heads * queries))
    gpu.causal_attention_with_stats(Q, K, V, O, stats, heads, queries, keys, h, scale, offset)
    dQ = gpu.upload(Shape.vector(heads * queries * h), np.full(heads * queries * h, np.nan, np.float32))
    dK, dV = (gpu.upload(Shape.vector(heads * keys * h), np.full(heads * keys * h, np.nan, np.float32))
              for _ in range(2))
    gpu.causal_attention_backward(Q, K, V, O, dO, stats, dQ, dK, dV, heads, queries, keys, h, scale, offset)
    got = {name: gpu.download(t) for name, t in (("out", O), ("stats", stats), ("dq", dQ), ("dk", dK), ("dv", dV))}
    for t in (Q, K, V, dO, O, stats, dQ, dK, dV):
        t.free()
    return (q, k, v, d_out), got


CASES = [
    (2, 128, 128, 64, 0, 0.125),     # one query block and one key block, square causal
    (3, 200, 200, 64, 0, 0.125),     # ragged second blocks
    (2, 100, 300, 64, 200, 0.125),   # a cached prefix: more keys than queries
    (2, 96, 96, 32, 0, 0.17),        # head dim 32 (config 0)
    (1, 64, 130, 128, 66, 0.09),     # head dim 128
    (2, 37, 37, 64, 0, 1.0),         # fewer queries than a wave's block
    (1, 300, 260, 64, 0, 0.125),     # keys run out before the diagonal
    (2, 512, 512, 32, 0, 0.17),      # head dim 32 over several blocks
    (2, 384, 448, 128, 64, 0.09),    # head dim 128 over several blocks, with an offset
    (2, 260, 700, 64, 300, 0.125),   # keys 560.. are seen by no query: their gradients are 0
]


@pytest.mark.parametrize("heads,queries,keys,h,offset,scale", CASES)
def test_backward_without_probabilities_matches_the_reference_calls(gpu, heads, queries, keys, h, offset, scale):
    print(f"backward heads={heads} queries={queries} keys={keys} h={h} offset={offset}", flush=True)
    inputs, got = run(gpu, heads, queries, keys, h, scale, offset, seed=queries + keys + h)
    out, row_max, dq, dk, dv = reference(*inputs, heads, queries, keys, h, scale, offset)
    for name, expected in (("out", out), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert np.all(np.isfinite(got[name])), name
        error = oracle.relative_error(expected, got[name])
        assert error < TOLERANCE, f"{name}: relative error {error}"
    # The statistics: m is exactly the largest scaled visible score (a maximum, order-free, of the
    # same products up to their rounding); l >= 1 (the maximum's own term).
    stats = got["stats"].reshape(heads, queries, 2)
    assert oracle.relative_error(row_max.ravel(), stats[..., 0].ravel()) < TOLERANCE
    assert np.all(stats[..., 1] >= 1.0)
    # Keys that no query sees get zero gradients.
    seen = min(keys, queries + offset)
    assert not np.any(got["dk"].reshape(heads, keys, h)[:, seen:])
    assert not np.any(got["dv"].reshape(heads, keys, h)[:, seen:])


def test_random_shapes_match_the_reference_calls(gpu):
    # A seeded sweep: 1-3 heads, 1-300 queries, 1-600 keys, head dims 32 / 64 / 128, offsets 0-300.
    rng = np.random.default_rng(23)
    for case in range(16):
        heads, queries, keys = int(rng.integers(1, 4)), int(rng.integers(1, 301)), int(rng.integers(1, 601))
        h = int(rng.choice([32, 64, 128]))
        offset, scale = int(rng.integers(0, 301)), float(rng.choice([0.125, 0.17, 0.09]))
        print(f"backward case {case}: {heads} heads, {queries} queries, {keys} keys, h {h}, offset {offset}",
              flush=True)
        inputs, got = run(gpu, heads, queries, keys, h, scale, offset, seed=100 + case)
        out, _, dq, dk, dv = reference(*inputs, heads, queries, keys, h, scale, offset)
        for name, expected in (("out", out), ("dq", dq), ("dk", dk), ("dv", dv)):
            assert np.all(np.isfinite(got[name])), (case, name)
            error = oracle.relative_error(expected, got[name])
            assert error < TOLERANCE, f"case {case} {name}: relative error {error}"


def test_forward_with_stats_gives_the_same_output(gpu):
    # The statistics are an extra output of the same kernel: O is bit for bit sn_causal_attention's.
    heads, t, h = 2, 300, 64
    rng = np.random.default_rng(9)
    q, k, v = (rng.normal(0, 1, heads * t * h).astype(np.float32) for _ in range(3))
    Q, K, V = (gpu.upload(Shape.vector(x.size), x) for x in (q, k, v))
    plain, with_stats = gpu.zeros(Shape.vector(heads * t * h)), gpu.zeros(Shape.vector(heads * t * h))
    stats = gpu.zeros(Shape.vector(2 * heads * t))
    gpu.causal_attention(Q, K, V, plain, heads, t, t, h, 0.125)
    gpu.causal_attention_with_stats(Q, K, V, with_stats, stats, heads, t, t, h, 0.125)
    assert np.array_equal(gpu.download(plain), gpu.download(with_stats))


def test_config_3_heads_at_full_size_and_determinism(gpu):
    # Two of config 3's 192 heads: T = 2048, h = 64, scale 1/8; reruns give the same bits.
    heads, t, h = 2, 2048, 64
    inputs, got = run(gpu, heads, t, t, h, 0.125, 0, seed=31)
    out, _, dq, dk, dv = reference(*inputs, heads, t, t, h, 0.125, 0)
    errors = {name: oracle.relative_error(e, got[name]) for name, e in (("dq", dq), ("dk", dk), ("dv", dv))}
    print(" ".join(f"{k} {e:.2e}" for k, e in errors.items()))
    assert all(e < TOLERANCE for e in errors.values()), errors
    _, again = run(gpu, heads, t, t, h, 0.125, 0, seed=31)
    for name in ("dq", "dk", "dv"):
        assert np.array_equal(got[name], again[name]), name


# Config 3's whole launch: 16 sequences x 12 heads = 192 head matrices of T = 2048, h = 64. A
# workgroup's head is its index mod 192 and workgroup i runs on XCD i mod 8, so head % 8 names the XCD
# group: these eight heads are the first, the last and one on every XCD.
CONFIG_3_HEADS, CONFIG_3_T, CONFIG_3_H = 192, 2048, 64
CHECKED_HEADS = [0, 25, 50, 75, 100, 125, 150, 191]


def test_config_3_full_launch_matches_the_reference_calls_on_heads_across_it(gpu):
    heads, t, h, scale = CONFIG_3_HEADS, CONFIG_3_T, CONFIG_3_H, 0.125
    assert sorted(x % 8 for x in CHECKED_HEADS) == list(range(8))
    print(f"config 3 full launch: {heads} heads, T {t}, h {h}", flush=True)
    inputs, got = run(gpu, heads, t, t, h, scale, 0, seed=3)
    # The reference's calls on the checked heads only (each head is independent).
    picked = [x.reshape(heads, t * h)[CHECKED_HEADS].ravel() for x in inputs]
    n = len(CHECKED_HEADS)
    out, row_max, dq, dk, dv = reference(*picked, n, t, t, h, scale, 0)
    errors = {}
    for name, expected in (("out", out), ("dq", dq), ("dk", dk), ("dv", dv)):
        mine = got[name].reshape(heads, t * h)[CHECKED_HEADS]
        assert np.all(np.isfinite(got[name])), name
        errors[name] = max(oracle.relative_error(e, a) for e, a in zip(expected.reshape(n, t * h), mine))
    # The statistics in full: m against the largest scaled visible score, l against the f64 sum of
    # e^(x - m) over the visible keys (both from the oracle's scores product).
    stats = got["stats"].reshape(heads, t, 2)[CHECKED_HEADS]
    errors["m"] = oracle.relative_error(row_max.ravel(), stats[..., 0].ravel())
    q, k = picked[0].reshape(n, t, h), picked[1].reshape(n, t, h)
    scores = np.zeros(n * t * t, np.float32)
    oracle.matmul_parallel(product(t, t, h, rt=True, batch=(n, t * h, t * h, t * t)), q.ravel(), k.ravel(), scores)
    scaled = scores.reshape(n, t, t).astype(np.float64) * scale
    visible = np.tril(np.ones((t, t), bool))
    l_expected = np.where(visible[None], np.exp(scaled - stats[..., 0:1].astype(np.float64)), 0.0).sum(axis=2)
    errors["l"] = float(np.max(np.abs(stats[..., 1] - l_expected) / l_expected))
    print(" ".join(f"{k} {e:.2e}" for k, e in errors.items()))
    assert all(e < TOLERANCE for e in errors.values()), errors
    # Every head's gradients are finite, and a rerun of the whole launch gives the same bits.
    _, again = run(gpu, heads, t, t, h, scale, 0, seed=3)
    for name in ("out", "stats", "dq", "dk", "dv"):
        assert np.array_equal(got[name], again[name]), name


def record_bytes(heads, queries):
    """The row records' share of the workspace: three planes of queries rounded up to 4 per head,
    rounded up to 256 bytes (the partial sums start there)."""
    return (heads * 3 * ((queries + 3) // 4 * 4) * 4 + 255) // 256 * 256


def partial_bytes(heads, queries, keys, h, offset):
    """dQ's partial sums: per head, h floats per query and 128-key block whose 64-query stages reach
    the query (from the first query that sees the block's first key, rounded down to a stage)."""
    rows = sum(max(0, queries - max(0, b * 128 - offset) // 64 * 64) for b in range((keys + 127) // 128))
    return heads * rows * h * 4


@pytest.mark.parametrize("heads,queries,keys,h,offset,scale", [CASES[1], CASES[2], CASES[3], CASES[9]])
def test_query_kernel_path_without_room_for_the_partial_sums(gpu, heads, queries, keys, h, offset, scale):
    # A workspace that holds the row records but not one head's partial sums: dQ comes from the query
    # kernel, which recomputes S and dP. The reference's results either way; dK, dV and O bit for bit
    # those of the partial-sum path (the shared context's large workspace).
    room = record_bytes(heads, queries) + partial_bytes(1, queries, keys, h, offset) - 4
    print(f"query path: heads={heads} queries={queries} keys={keys} h={h} workspace {room} bytes", flush=True)
    small = Gpu(0, workspace_bytes=room)
    try:
        inputs, got = run(small, heads, queries, keys, h, scale, offset, seed=queries + keys + h)
    finally:
        small.close()
    out, _, dq, dk, dv = reference(*inputs, heads, queries, keys, h, scale, offset)
    for name, expected in (("out", out), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert np.all(np.isfinite(got[name])), name
        error = oracle.relative_error(expected, got[name])
        assert error < TOLERANCE, f"{name}: relative error {error}"
    _, partial = run(gpu, heads, queries, keys, h, scale, offset, seed=queries + keys + h)
    for name in ("out", "stats", "dk", "dv"):
        assert np.array_equal(got[name], partial[name]), name
    assert oracle.relative_error(partial["dq"], got["dq"]) < TOLERANCE


def test_head_runs_give_the_bits_of_one_launch(gpu):
    # 24 heads of T = 4096 (32 key blocks each). A workspace for 17 heads' partial sums splits the
    # launch into runs of 17 and 7 heads (17 x 32 workgroups fill the device); every bit equals that
    # of the one-launch result, and the last head (second run) matches the reference's calls.
    heads, t, h, scale = 24, 4096, 64, 0.125
    room = record_bytes(heads, t) + 17 * partial_bytes(1, t, t, h, 0) + 4
    assert record_bytes(heads, t) + partial_bytes(heads, t, t, h, 0) <= 1536 << 20  # one launch by default
    print(f"head runs: {heads} heads, T {t}, workspace {room} bytes", flush=True)
    inputs, whole = run(gpu, heads, t, t, h, scale, 0, seed=77)
    small = Gpu(0, workspace_bytes=room)
    try:
        _, runs = run(small, heads, t, t, h, scale, 0, seed=77)
    finally:
        small.close()
    for name in ("out", "stats", "dq", "dk", "dv"):
        assert np.array_equal(whole[name], runs[name]), name
    picked = [x.reshape(heads, t * h)[heads - 1] for x in inputs]
    _, _, dq, dk, dv = reference(*picked, 1, t, t, h, scale, 0)
    for name, expected in (("dq", dq), ("dk", dk), ("dv", dv)):
        mine = runs[name].reshape(heads, t * h)[heads - 1]
        error = oracle.relative_error(expected, mine)
        assert error < TOLERANCE, f"{name}: relative error {error}"


def poison_workspace(gpu):
    """Leaves NaN in the context workspace's first bytes: a split-K weight-gradient product whose
    left operand is all Inf stores non-finite partial sums there (Inf times values of both signs)."""
    from staleynet_amd.gemm import MatmulSpec, plan

    m, n, k = 256, 256, 32768
    spec = MatmulSpec.new(m, n, k).left_transposed()
    assert plan(spec).splits > 1
    left = gpu.upload(Shape.vector(k * m), np.full(k * m, np.inf, np.float32))
    right = gpu.upload(Shape.vector(k * n), np.random.default_rng(5).normal(0, 1, k * n).astype(np.float32))
    out = gpu.zeros(Shape(m, n))
    gpu.matmul(spec, left, right, out)
    assert np.all(np.isnan(gpu.download(out)))
    for buf in (left, right, out):
        buf.free()


@pytest.mark.parametrize("queries,h", [(37, 64), (299, 64), (37, 128), (301, 32)])
def test_record_padding_never_reaches_the_gradients(gpu, queries, h):
    # The row records are planes of queries rounded up to 4; the key kernels load the last 16-byte
    # chunk whole, so a query count that is not a multiple of 4 reads padding slots. Whatever the
    # workspace held there before (here NaN), the gradients stay finite and equal the reference's.
    heads, keys, scale = 2, queries, 0.125
    print(f"padding: heads={heads} queries={queries} h={h} after a NaN workspace", flush=True)
    poison_workspace(gpu)
    inputs, got = run(gpu, heads, queries, keys, h, scale, 0, seed=queries + h)
    out, _, dq, dk, dv = reference(*inputs, heads, queries, keys, h, scale, 0)
    for name, expected in (("out", out), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert np.all(np.isfinite(got[name])), name
        error = oracle.relative_error(expected, got[name])
        assert error < TOLERANCE, f"{name}: relative error {error}"


def test_entry_point_checks(gpu):
    heads, t, h = 2, 64, 64
    bufs = [gpu.zeros(Shape.vector(heads * t * h)) for _ in range(8)]
    q, k, v, o, do, dq, dk, dv = bufs
    stats = gpu.zeros(Shape.vector(2 * heads * t))
    with pytest.raises(AssertionError, match="too small"):
        gpu.causal_attention_backward(q, k, v, o, do, gpu.zeros(Shape.vector(10)), dq, dk, dv, heads, t, t, h, 1.0)
    with pytest.raises(AssertionError, match="no keys"):
        gpu.causal_attention_backward(q, k, v, o, do, stats, dq, dk, dv, heads, t, 0, h, 1.0)
    with pytest.raises(GpuError):  # a gradient overlapping an input
        gpu.causal_attention_backward(q, k, v, o, do, stats, q, dk, dv, heads, t, t, h, 1.0)
    with pytest.raises(GpuError):  # two gradients in one buffer
        gpu.causal_attention_backward(q, k, v, o, do, stats, dq, dq, dv, heads, t, t, h, 1.0)
    with pytest.raises(GpuError):  # head dim 48
        gpu.causal_attention_backward(q, k, v, o, do, stats, dq, dk, dv, heads, t, t, 48, 1.0)
    for b in bufs + [stats]:
        b.free()

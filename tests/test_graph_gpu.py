"""Captured sequences replay to the same results as eager calls.

The decode bench replays a captured HIP graph of sn_matmul calls (and of
decode-step attention). This checks the library state a replay relies on: the
split-K workspace and the arrival counters a few-row product or a decode-form
attention resets itself. The graph is replayed
three times with eager work and synchronizations between the replays; each
replay must equal the eager result bit for bit (every kernel sums in a fixed
order)."""
import numpy as np
import pytest

from bench import HipGraph
from oracle import oracle
from staleynet_amd.gemm import MatmulSpec, Shape

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager_results(gpu):
    rng_seed = 40
    products = [
        MatmulSpec.new(4, 3072, 768),                                   # few rows: 12 K slices, counters
        MatmulSpec.new(1, 16384, 768).scaled(0.5),                       # few rows, 64 column blocks
        MatmulSpec.new(256, 256, 8192).left_transposed().accumulate(),   # split-K weight gradient
        MatmulSpec.new(512, 384, 256),                                   # plain tiles
    ]
    tensors = []
    for i, spec in enumerate(products):
        left_shape = Shape(spec.inner, spec.rows) if spec.left else Shape(spec.rows, spec.inner)
        left = gpu.upload(left_shape, oracle.random_values(spec.rows * spec.inner, rng_seed + 3 * i))
        right = gpu.upload(Shape(spec.inner, spec.cols), oracle.random_values(spec.inner * spec.cols, rng_seed + 3 * i + 1))
        initial = oracle.random_values(spec.rows * spec.cols, rng_seed + 3 * i + 2)
        out = gpu.upload(Shape(spec.rows, spec.cols), initial)
        tensors.append((spec, left, right, out, initial))

    def run_all():
        for spec, left, right, out, _ in tensors:
            gpu.matmul(spec, left, right, out)

    def reset():
        for _, _, _, out, initial in tensors:
            gpu.copy_from_host(out, initial)

    run_all()
    eager = [gpu.download(out) for _, _, _, out, _ in tensors]
    reset()
    graph = HipGraph(gpu.stream, run_all)
    try:
        other = gpu.zeros(Shape(64, 64))
        ones = gpu.upload(Shape(64, 64), np.ones(64 * 64, np.float32))
        for replay in range(3):
            graph.launch()
            gpu.synchronize()
            for (_, _, _, out, _), expected in zip(tensors, eager):
                assert np.array_equal(gpu.download(out), expected), f"replay {replay}"
            # Eager work between replays, on the same stream and workspace.
            gpu.matmul(MatmulSpec.new(64, 64, 64), ones, ones, other)
            gpu.matmul(MatmulSpec.new(2, 3072, 768), tensors[0][1], tensors[0][2], gpu.zeros(Shape(2, 3072)))
            reset()
            gpu.synchronize()
    finally:
        graph.close()


def test_graph_replays_of_a_decode_attention_step(gpu):
    # One decode step's attention for two layers, as the reference calls it (masked scores against the
    # cache, causal_softmax, masked mix: the few-row kernels) and through the fused decode form (key
    # chunks merged through the workspace and arrival counters), captured once and replayed three
    # times with eager work between the replays; each replay must equal the eager result bit for bit.
    from staleynet_amd.gemm import BatchStrides

    heads, capacity, h, cached = 12, 1408, 64, 900
    offset = cached - 1
    q = gpu.upload(Shape(heads, h), oracle.random_values(heads * h, 60))
    k = gpu.upload(Shape(heads * capacity, h), oracle.random_values(heads * capacity * h, 61))
    v = gpu.upload(Shape(heads * capacity, h), oracle.random_values(heads * capacity * h, 62))
    scores = gpu.zeros(Shape(heads, capacity))
    mixed, fused = gpu.zeros(Shape(heads, h)), gpu.zeros(Shape(heads, h))
    score_spec = MatmulSpec.new(1, capacity, h).right_transposed().batched(
        BatchStrides(heads, h, capacity * h, capacity)).causal_output(offset)
    mix_spec = MatmulSpec.new(1, h, capacity).batched(BatchStrides(heads, capacity, capacity * h, h)).causal_left(offset)

    def step():
        for _ in range(2):
            gpu.matmul(score_spec, q, k, scores)
            gpu.causal_softmax(scores, 1, 0.125, offset)
            gpu.matmul(mix_spec, scores, v, mixed)
            gpu.causal_attention(q, k, v, fused, heads, 1, capacity, h, 0.125, query_offset=offset, q_stride=h,
                                 kv_stride=capacity * h)

    step()
    eager = (gpu.download(mixed), gpu.download(fused))
    assert oracle.relative_error(eager[0], eager[1]) < 1e-5
    graph = HipGraph(gpu.stream, step)
    try:
        for replay in range(3):
            for t in (scores, mixed, fused):
                gpu.fill_zero(t)
            graph.launch()
            gpu.synchronize()
            assert np.array_equal(gpu.download(mixed), eager[0]), f"replay {replay}: three calls"
            assert np.array_equal(gpu.download(fused), eager[1]), f"replay {replay}: fused"
            # Eager work between replays on the same workspace and counters.
            gpu.causal_attention(q, k, v, gpu.zeros(Shape(heads, h)), heads, 1, capacity, h, 0.125, query_offset=100,
                                 q_stride=h, kv_stride=capacity * h)
            gpu.matmul(MatmulSpec.new(2, 3072, 768), gpu.zeros(Shape(2, 768)), gpu.zeros(Shape(768, 3072)),
                       gpu.zeros(Shape(2, 3072)))
            gpu.synchronize()
    finally:
        graph.close()

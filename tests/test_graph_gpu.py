"""Captured sequences replay to the same results as eager calls.

The decode bench replays a captured HIP graph of sn_matmul calls. This
checks the library state a replay relies on: the split-K workspace and the
arrival counters a few-row product resets itself. The graph is replayed
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

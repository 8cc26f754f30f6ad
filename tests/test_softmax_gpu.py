"""GPU parity of the row-wise kernels between the attention products, through the C ABI.

``sn_causal_softmax`` (``Gpu::causal_softmax``, ops/attention.rs:56-74) and
``sn_softmax_backward`` (``Gpu::softmax_backward``, :76-92) against the oracle's
restatement of ``reference::causal_softmax`` / ``softmax_backward``
(reference.rs:100-137), at the reference's tolerance. The reference's own GPU
test (tests/kernels_match_reference.rs:175-195) comes first, on its inputs; then
the register-resident and multi-pass paths, the cached-decode shape, config 3's
row length at scale, determinism and the shape checks.
"""
import numpy as np
import pytest

from oracle import oracle
from staleynet_amd.gemm import Shape

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-5  # kernels_match_reference.rs:12


def run(gpu, matrices, queries, keys, query_offset, scale, seed_scores, seed_upstream):
    shape = Shape(matrices * queries, keys)
    scores = oracle.random_values(len(shape), seed_scores)
    upstream = oracle.random_values(len(shape), seed_upstream)
    expected = scores.copy()
    oracle.causal_softmax(expected, queries, keys, scale, query_offset)
    expected_grad = upstream.copy()
    oracle.softmax_backward(expected, expected_grad, keys)
    probabilities = gpu.upload(shape, scores)
    gpu.causal_softmax(probabilities, queries, scale, query_offset)
    grad = gpu.upload(shape, upstream)
    gpu.softmax_backward(probabilities, grad)
    return expected, gpu.download(probabilities), expected_grad, gpu.download(grad)


def test_reference_causal_softmax_and_backward_test(gpu):
    # (matrices, queries, keys, query_offset, scale) = (3, 5, 70, 40, 0.5); LCG seeds 10, 11.
    expected, got, expected_grad, got_grad = run(gpu, 3, 5, 70, 40, 0.5, 10, 11)
    assert oracle.relative_error(expected, got) < TOLERANCE
    assert oracle.relative_error(expected_grad, got_grad) < TOLERANCE


@pytest.mark.parametrize("matrices,queries,keys,offset,scale", [
    (1, 1, 1, 0, 1.0),            # one key
    (2, 7, 7, 0, 0.125),          # square causal, unaligned (multi-pass path)
    (4, 64, 64, 0, 0.125),        # aligned, one float4 per lane
    (3, 33, 256, 200, 0.5),       # offset: most keys visible
    (2, 130, 1028, 0, 0.125),     # 5 float4 per lane (8-vector instantiation)
    (1, 48, 4096, 4000, 0.125),   # the longest register-resident row
    (1, 16, 5000, 4990, 0.125),   # past 4096: multi-pass
    (12, 1, 1408, 700, 0.125),    # cached decode: one query against a 1408-key cache, half written
])
def test_causal_softmax_and_backward_match_the_oracle(gpu, matrices, queries, keys, offset, scale):
    expected, got, expected_grad, got_grad = run(gpu, matrices, queries, keys, offset, scale,
                                                 keys + queries, keys + 7)
    assert oracle.relative_error(expected, got) < TOLERANCE
    assert oracle.relative_error(expected_grad, got_grad) < TOLERANCE
    # keys past each query's horizon are exactly 0, as in the reference
    p = got.reshape(matrices * queries, keys)
    for r in range(matrices * queries):
        visible = min(r % queries + offset + 1, keys)
        assert not np.any(p[r, visible:])


def test_config_3_rows_at_scale_and_determinism(gpu):
    # 8 heads' worth of config 3's scores: [8 * 2048, 2048], scale 1/8, scores ~N(0, 8^2).
    heads, t = 8, 2048
    shape = Shape(heads * t, t)
    scores = gpu.zeros(shape)
    gpu.fill_normal(scores, 1234, 21, 0.0, 8.0)
    host_scores = gpu.download(scores)
    upstream = gpu.zeros(shape)
    gpu.fill_normal(upstream, 1234, 22)
    host_upstream = gpu.download(upstream)
    gpu.causal_softmax(scores, t, 0.125, 0)
    first = gpu.download(scores)
    gpu.copy_from_host(scores, host_scores)
    gpu.causal_softmax(scores, t, 0.125, 0)
    assert np.array_equal(first, gpu.download(scores)), "causal_softmax differs between runs"
    gpu.softmax_backward(scores, upstream)
    got_grad = gpu.download(upstream)

    expected = host_scores.copy()
    oracle.causal_softmax(expected, t, t, 0.125, 0)
    assert oracle.relative_error(expected, first) < TOLERANCE
    expected_grad = host_upstream.copy()
    oracle.softmax_backward(expected, expected_grad, t)
    assert oracle.relative_error(expected_grad, got_grad) < TOLERANCE


def test_shape_checks_raise_the_reference_panics(gpu):
    scores = gpu.zeros(Shape(10, 8))
    with pytest.raises(AssertionError, match="causal_softmax: rows must be a multiple of queries"):
        gpu.causal_softmax(scores, 3, 1.0, 0)
    with pytest.raises(AssertionError, match="softmax_backward: shape mismatch"):
        gpu.softmax_backward(scores, gpu.zeros(Shape(10, 9)))

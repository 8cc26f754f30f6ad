"""GPU parity of the fused causal attention forward (``sn_causal_attention``) against the oracle's
restatement of the three calls it replaces in CausalSelfAttention::forward
(crates/staleynet-model/src/layers/attention.rs:206-213): the scores product
(``MatmulSpec::new(T, keys, h).right_transposed()`` batched over the heads, reference.rs:19-38),
``causal_softmax`` (reference.rs:100-119) and the mix product (``MatmulSpec::new(T, h, keys)``).
O and the probabilities are compared at the reference's fp32 tolerance. Cases: ragged query
blocks and key counts, query offsets (a cached prefix), one-query decode against a partly written
cache, head dims 32 / 64 / 128, K and V shared by every head, config 3's size, determinism, and the
entry point's checks. The same for the fused probability gradient (``sn_causal_attention_score_grad``)
against the dP product and ``softmax_backward`` of CausalSelfAttention::backward (attention.rs:238-248).
"""
import numpy as np
import pytest

from oracle import oracle
from staleynet_amd.gemm import Shape

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-5  # kernels_match_reference.rs:12


def reference(q, k, v, heads, queries, keys, h, scale, offset, q_stride, kv_stride):
    scores = np.zeros(heads * queries * keys, np.float32)
    oracle.matmul_parallel(oracle.Product(queries, keys, h, False, True, heads, q_stride, kv_stride, queries * keys,
                                          1.0, False), q, k, scores)
    oracle.causal_softmax(scores, queries, keys, scale, offset)
    out = np.zeros(heads * queries * h, np.float32)
    oracle.matmul_parallel(oracle.Product(queries, h, keys, False, False, heads, queries * keys, kv_stride,
                                          queries * h, 1.0, False), scores, v, out)
    return out, scores


def run(gpu, heads, queries, keys, h, scale, offset, q_stride=None, kv_stride=None, seed=0, with_p=True, spread=1.0):
    q_stride = queries * h if q_stride is None else q_stride
    kv_stride = keys * h if kv_stride is None else kv_stride
    q_len = (heads - 1) * q_stride + queries * h
    kv_len = (heads - 1) * kv_stride + keys * h
    rng = np.random.default_rng(seed)
    q = rng.normal(0, spread, q_len).astype(np.float32)
    k = rng.normal(0, spread, kv_len).astype(np.float32)
    v = rng.normal(0, 1, kv_len).astype(np.float32)
    Q, K, V = (gpu.upload(Shape.vector(len(x)), x) for x in (q, k, v))
    out = gpu.upload(Shape.vector(heads * queries * h), np.full(heads * queries * h, np.nan, np.float32))
    probabilities = None
    if with_p:
        probabilities = gpu.upload(Shape.vector(heads * queries * keys),
                                   np.full(heads * queries * keys, np.nan, np.float32))
    gpu.causal_attention(Q, K, V, out, heads, queries, keys, h, scale, offset, q_stride, kv_stride, probabilities)
    expected_o, expected_p = reference(q, k, v, heads, queries, keys, h, scale, offset, q_stride, kv_stride)
    got_p = gpu.download(probabilities) if with_p else None
    return expected_o, gpu.download(out), expected_p, got_p


@pytest.mark.parametrize("heads,queries,keys,h,offset,scale", [
    (2, 128, 128, 64, 0, 0.125),     # one query block, square causal
    (3, 200, 200, 64, 0, 0.125),     # a ragged second query block, keys not a multiple of 64
    (2, 100, 300, 64, 200, 0.125),   # a cached prefix: offset 200, more keys than queries
    (2, 96, 96, 32, 0, 0.17),        # head dim 32 (config 0)
    (1, 64, 130, 128, 66, 0.09),     # head dim 128
    (2, 37, 37, 64, 0, 1.0),         # fewer queries than a wave's block
    (1, 300, 260, 64, 0, 0.125),     # keys run out before the diagonal
    (2, 512, 512, 32, 0, 0.17),      # head dim 32 over several query blocks (three waves per SIMD)
    (2, 384, 448, 128, 64, 0.09),    # head dim 128 over several query blocks, with an offset
])
def test_fused_attention_matches_the_three_calls(gpu, heads, queries, keys, h, offset, scale):
    eo, go, ep, gp = run(gpu, heads, queries, keys, h, scale, offset, seed=queries + keys + h)
    assert np.all(np.isfinite(go)) and np.all(np.isfinite(gp))
    assert oracle.relative_error(eo, go) < TOLERANCE
    assert oracle.relative_error(ep, gp) < TOLERANCE
    # Keys past each query's horizon are exactly 0, as causal_softmax leaves them.
    p = gp.reshape(heads, queries, keys)
    for r in range(queries):
        visible = min(r + offset + 1, keys)
        assert not np.any(p[:, r, visible:])


def test_random_shapes_match_the_three_calls(gpu):
    # A seeded sweep: 1-4 heads, 1-300 queries, 1-600 keys (fewer, as many, or more than the queries'
    # horizon reaches), head dims 32 / 64 / 128, query offsets 0-300, with and without probabilities.
    rng = np.random.default_rng(17)
    for case in range(24):
        heads, queries, keys = int(rng.integers(1, 5)), int(rng.integers(1, 301)), int(rng.integers(1, 601))
        h = int(rng.choice([32, 64, 128]))
        offset, scale = int(rng.integers(0, 301)), float(rng.choice([0.125, 0.17, 0.09]))
        with_p = bool(rng.random() < 0.5)
        print(f"attention case {case}: {heads} heads, {queries} queries, {keys} keys, h {h}, offset {offset}, "
              f"probabilities {with_p}", flush=True)
        eo, go, ep, gp = run(gpu, heads, queries, keys, h, scale, offset, seed=case, with_p=with_p)
        assert np.all(np.isfinite(go)) and oracle.relative_error(eo, go) < TOLERANCE, f"case {case}"
        if with_p:
            assert oracle.relative_error(ep, gp) < TOLERANCE, f"case {case}"


def test_large_logits(gpu):
    # Q and K ~ N(0, 9): scaled scores with a spread of about 9 and row maxima near 30, so the
    # differences from the maximum reach -60 or so. The exponential of a rounded difference d is
    # taken as 2^(d log2 e); its error grows with |d| but stays within the tolerance, because the
    # probabilities it affects are tiny.
    eo, go, ep, gp = run(gpu, 2, 1024, 1024, 64, 0.125, 0, seed=11, spread=3.0)
    assert np.all(np.isfinite(go)) and np.all(np.isfinite(gp))
    assert oracle.relative_error(eo, go) < TOLERANCE
    assert oracle.relative_error(ep, gp) < TOLERANCE
    print(f"large logits: O {oracle.relative_error(eo, go):.2e}, P {oracle.relative_error(ep, gp):.2e}")


def test_decode_query_against_a_partly_written_cache(gpu):
    # attention.rs:274-320: one new position per head against a 1408-step cache holding 701.
    heads, capacity, h = 12, 1408, 64
    eo, go, ep, gp = run(gpu, heads, 1, capacity, h, 0.125, 700, q_stride=h, kv_stride=capacity * h, seed=3)
    assert oracle.relative_error(eo, go) < TOLERANCE
    assert oracle.relative_error(ep, gp) < TOLERANCE


@pytest.mark.parametrize("heads,queries,keys,h,offset,kv_stride", [
    (12, 1, 1408, 64, 700, None),    # a decode step: 701 of 1408 cached positions (6 key chunks)
    (12, 1, 1408, 64, 1407, None),   # a full cache (11 chunks)
    (12, 1, 1408, 64, 0, None),      # the first position: one key
    (3, 4, 300, 32, 100, None),      # four new positions, head dim 32 (one chunk)
    (3, 4, 700, 32, 600, None),      # four new positions over 5 chunks
    (2, 2, 900, 64, 800, None),      # two new positions over 7 chunks
    (2, 3, 2000, 128, 1990, None),   # head dim 128, keys run out before the last query's horizon
    (2, 2, 64, 64, 0, None),         # one chunk; the queries see 1 and 2 keys
    (4, 1, 500, 64, 499, 0),         # K and V shared by every head
])
def test_decode_form_matches_the_three_calls(gpu, heads, queries, keys, h, offset, kv_stride):
    # At most 4 queries per head and no probabilities: the keys are split into 128-key chunks
    # whose partial softmax sums and outputs the last chunk of each head merges.
    q_stride = queries * h
    kv_stride = keys * h if kv_stride is None else kv_stride
    eo, go, _, _ = run(gpu, heads, queries, keys, h, 0.125, offset, q_stride=q_stride, kv_stride=kv_stride,
                       seed=heads + queries + keys, with_p=False)
    assert np.all(np.isfinite(go))
    assert oracle.relative_error(eo, go) < TOLERANCE


@pytest.mark.parametrize("heads,queries,keys,h,offset", [
    (12, 1, 1408, 64, 700),     # 6 chunks, the last one partly past the horizon
    (3, 4, 700, 32, 300),       # four queries: the tail starts at 304
    (2, 2, 900, 128, 129),      # the tail starts inside the second chunk
])
def test_decode_form_never_reads_the_unwritten_cache_tail(gpu, heads, queries, keys, h, offset):
    # A decode step's cache holds queries + offset written positions; the rest (the tail) is never
    # written. The reference's cache is zero-initialised, so its three calls see zeros there; here
    # the tail holds NaN, which must not reach the result (0 * NaN would).
    rng = np.random.default_rng(heads * 7 + offset)
    q = rng.normal(0, 1, heads * queries * h).astype(np.float32)
    k = rng.normal(0, 1, heads * keys * h).astype(np.float32).reshape(heads, keys, h)
    v = rng.normal(0, 1, heads * keys * h).astype(np.float32).reshape(heads, keys, h)
    written = queries + offset
    k[:, written:, :] = 0.0
    v[:, written:, :] = 0.0
    expected, _ = reference(q, k.ravel(), v.ravel(), heads, queries, keys, h, 0.125, offset, queries * h, keys * h)
    k_dirty, v_dirty = k.copy(), v.copy()
    k_dirty[:, written:, :] = np.nan
    v_dirty[:, written:, :] = np.nan
    Q, K, V = (gpu.upload(Shape.vector(x.size), x.ravel()) for x in (q, k_dirty, v_dirty))
    out = gpu.zeros(Shape.vector(heads * queries * h))
    gpu.causal_attention(Q, K, V, out, heads, queries, keys, h, 0.125, offset)
    got = gpu.download(out)
    assert np.all(np.isfinite(got))
    assert oracle.relative_error(expected, got) < TOLERANCE


def test_decode_form_is_deterministic_and_reusable(gpu):
    # Repeated calls (the arrival counters are reset by each call's last chunk) give the same bits.
    first = run(gpu, 12, 1, 1408, 64, 0.125, 1000, q_stride=64, kv_stride=1408 * 64, seed=21, with_p=False)[1]
    for _ in range(3):
        again = run(gpu, 12, 1, 1408, 64, 0.125, 1000, q_stride=64, kv_stride=1408 * 64, seed=21, with_p=False)[1]
        assert np.array_equal(first, again)


def test_keys_and_values_shared_by_every_head(gpu):
    eo, go, ep, gp = run(gpu, 3, 64, 64, 64, 0.125, 0, kv_stride=0, seed=4)
    assert oracle.relative_error(eo, go) < TOLERANCE
    assert oracle.relative_error(ep, gp) < TOLERANCE


def test_without_probabilities_the_output_is_the_same(gpu):
    eo, go, _, _ = run(gpu, 2, 256, 256, 64, 0.125, 0, seed=5, with_p=False)
    assert oracle.relative_error(eo, go) < TOLERANCE


def test_config_3_heads_at_full_size_and_determinism(gpu):
    # Two of config 3's 192 heads: T = 2048, h = 64, scale 1/8, Q, K, V ~ N(0, 1).
    heads, t, h = 2, 2048, 64
    eo, go, ep, gp = run(gpu, heads, t, t, h, 0.125, 0, seed=6)
    assert oracle.relative_error(eo, go) < TOLERANCE
    assert oracle.relative_error(ep, gp) < TOLERANCE
    _, go2, _, gp2 = run(gpu, heads, t, t, h, 0.125, 0, seed=6)
    assert np.array_equal(go, go2) and np.array_equal(gp, gp2)


def test_entry_point_checks(gpu):
    from staleynet_amd.gemm import GpuError
    q, k, v = (gpu.zeros(Shape.vector(2 * 64 * 64)) for _ in range(3))
    out = gpu.zeros(Shape.vector(2 * 64 * 64))
    with pytest.raises(AssertionError, match="no keys"):
        gpu.causal_attention(q, k, v, out, 2, 64, 0, 64, 1.0)
    with pytest.raises(AssertionError, match="too small"):
        gpu.causal_attention(q, k, v, out, 2, 64, 65, 64, 1.0)
    with pytest.raises(AssertionError, match="too small"):
        gpu.causal_attention(q, k, v, out, 2, 64, 64, 64, 1.0, probabilities=gpu.zeros(Shape.vector(100)))
    with pytest.raises(GpuError):  # head dim 48: unsupported
        gpu.causal_attention(q, k, v, out, 2, 64, 64, 48, 1.0)
    with pytest.raises(GpuError):  # the output overlapping an input
        gpu.causal_attention(q, k, v, q, 2, 64, 64, 64, 1.0)


# ---- the fused probability gradient (sn_causal_attention_score_grad) ---------------------------
# Against the reference's two calls in CausalSelfAttention::backward (attention.rs:238-248): the dP
# product (MatmulSpec::new(T, keys, h).right_transposed(), reference.rs:19-38) and softmax_backward
# (reference.rs:121-137), on the probabilities and output the oracle's forward gives.

def run_score_grad(gpu, heads, queries, keys, h, scale, offset, q_stride=None, kv_stride=None, seed=0,
                   with_q=False):
    q_stride = queries * h if q_stride is None else q_stride
    kv_stride = keys * h if kv_stride is None else kv_stride
    q_len = (heads - 1) * q_stride + queries * h
    kv_len = (heads - 1) * kv_stride + keys * h
    rng = np.random.default_rng(seed)
    q = rng.normal(0, 1, q_len).astype(np.float32)
    k = rng.normal(0, 1, kv_len).astype(np.float32)
    v = rng.normal(0, 1, kv_len).astype(np.float32)
    d_out = rng.normal(0, 1, q_len).astype(np.float32)
    out, p = reference(q, k, v, heads, queries, keys, h, scale, offset, q_stride, kv_stride)
    expected = np.zeros(heads * queries * keys, np.float32)
    oracle.matmul_parallel(oracle.Product(queries, keys, h, False, True, heads, q_stride, kv_stride, queries * keys,
                                          1.0, False), d_out, v, expected)
    oracle.softmax_backward(p, expected, keys)
    D, V, O, P = (gpu.upload(Shape.vector(len(x)), x) for x in (d_out, v, out, p))
    grad = gpu.upload(Shape.vector(len(p)), np.full(len(p), np.nan, np.float32))
    if not with_q:
        gpu.causal_attention_score_grad(D, V, O, P, grad, heads, queries, keys, h, offset, q_stride, kv_stride)
        return expected, gpu.download(grad)
    # The backward's next call: dQ = scale dS K (attention.rs:250-253).
    expected_q = np.zeros(heads * queries * h, np.float32)
    oracle.matmul_parallel(oracle.Product(queries, h, keys, False, False, heads, queries * keys, kv_stride, queries * h,
                                          scale, False), expected, k, expected_q)
    K = gpu.upload(Shape.vector(len(k)), k)
    q_grad = gpu.upload(Shape.vector(len(expected_q)), np.full(len(expected_q), np.nan, np.float32))
    gpu.causal_attention_score_grad(D, V, O, P, grad, heads, queries, keys, h, offset, q_stride, kv_stride, k=K,
                                    q_grad=q_grad, scale=scale)
    return expected, gpu.download(grad), expected_q, gpu.download(q_grad)


@pytest.mark.parametrize("heads,queries,keys,h,offset", [
    (2, 128, 128, 64, 0),
    (3, 200, 200, 64, 0),
    (2, 100, 300, 64, 200),
    (2, 96, 96, 32, 0),
    (1, 64, 130, 128, 66),
    (2, 37, 37, 64, 0),
    (1, 300, 260, 64, 0),
])
def test_fused_score_grad_matches_dp_and_softmax_backward(gpu, heads, queries, keys, h, offset):
    expected, got = run_score_grad(gpu, heads, queries, keys, h, 0.125, offset, seed=queries + keys + h + 1)
    assert np.all(np.isfinite(got))
    assert oracle.relative_error(expected, got) < TOLERANCE
    g = got.reshape(heads, queries, keys)
    for r in range(queries):
        assert not np.any(g[:, r, min(r + offset + 1, keys):])


@pytest.mark.parametrize("heads,queries,keys,h,offset", [
    (2, 128, 128, 64, 0),
    (3, 200, 200, 64, 0),
    (2, 100, 300, 64, 200),
    (2, 96, 96, 32, 0),
    (1, 64, 130, 128, 66),
])
def test_fused_query_grad_matches_the_next_product(gpu, heads, queries, keys, h, offset):
    eg, gg, eq, gq = run_score_grad(gpu, heads, queries, keys, h, 0.125, offset, seed=queries + h + 2, with_q=True)
    assert np.all(np.isfinite(gq))
    assert oracle.relative_error(eg, gg) < TOLERANCE
    assert oracle.relative_error(eq, gq) < TOLERANCE


def test_fused_score_grad_decode_and_shared_values(gpu):
    expected, got = run_score_grad(gpu, 12, 1, 1408, 64, 0.125, 700, q_stride=64, kv_stride=1408 * 64, seed=7)
    assert oracle.relative_error(expected, got) < TOLERANCE
    expected, got = run_score_grad(gpu, 3, 64, 64, 64, 0.125, 0, kv_stride=0, seed=8)
    assert oracle.relative_error(expected, got) < TOLERANCE


def test_fused_score_grad_config_3_heads_and_determinism(gpu):
    expected, got = run_score_grad(gpu, 2, 2048, 2048, 64, 0.125, 0, seed=9)
    assert oracle.relative_error(expected, got) < TOLERANCE
    _, again = run_score_grad(gpu, 2, 2048, 2048, 64, 0.125, 0, seed=9)
    assert np.array_equal(got, again)
    eg, gg, eq, gq = run_score_grad(gpu, 2, 2048, 2048, 64, 0.125, 0, seed=9, with_q=True)
    assert np.array_equal(gg, got)
    assert oracle.relative_error(eq, gq) < TOLERANCE


def test_fused_score_grad_checks(gpu):
    from staleynet_amd.gemm import GpuError
    x = gpu.zeros(Shape.vector(2 * 64 * 64))
    p, g = gpu.zeros(Shape.vector(2 * 64 * 64)), gpu.zeros(Shape.vector(2 * 64 * 64))
    with pytest.raises(AssertionError, match="too small"):
        gpu.causal_attention_score_grad(x, x, x, p, g, 2, 64, 65, 64)
    with pytest.raises(GpuError):  # the gradient overlapping the probabilities
        gpu.causal_attention_score_grad(x, x, x, p, p, 2, 64, 64, 64)

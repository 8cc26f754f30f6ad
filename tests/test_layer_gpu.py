"""Chained-layer GPU parity: one causal self-attention layer, forward and backward, through this
build's kernels, against the oracle's composition of the reference's calls in
CausalSelfAttention::forward / backward (crates/staleynet-model/src/layers/attention.rs:188-267)
and Linear::forward / backward (layers/linear.rs:43-63); and one cached decode step
(forward_cached, attention.rs:274-320) against the last row of the full causal forward, the check
of the reference's model_is_trainable.rs:161-213.

Three call sequences run on the GPU:
* ``reference``: the reference's calls one for one (dense scores and mix products, causal_softmax,
  softmax_backward, four backward products, separate bias calls);
* ``fused``: what a caller of this library would issue instead (the bias in the product's
  epilogue, the fused attention forward with probabilities, the fused probability and query
  gradient, the causal-left value and key gradients);
* ``no_probabilities``: the same Linears around the training attention that keeps no [T, T]
  matrix (the forward with per-query statistics, then the backward that rebuilds P from them).
Every activation and gradient is compared, in the reference test's metric, at the fp32 tolerance.
Weights and inputs come from the reference test's LCG (kernels_match_reference.rs:26-38)."""
import math

import numpy as np
import pytest

from oracle import oracle
from staleynet_amd.gemm import BatchStrides, HeadLayout, MatmulSpec, Shape

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-5  # kernels_match_reference.rs:12


def values(count, seed, scale=1.0):
    return (oracle.random_values(count, seed) * np.float32(scale)).astype(np.float32)


class Layer:
    """Host copies of one layer's parameters and input (Linear weights [in, out], attention.rs:38-51)."""

    def __init__(self, batch, time, width, heads, seed):
        self.batch, self.time, self.width, self.heads = batch, time, width, heads
        self.head_dim = width // heads
        self.scale = np.float32(1.0 / math.sqrt(self.head_dim))  # score_scale, attention.rs:180-182
        rows = batch * time
        self.x = values(rows * width, seed)
        self.w_qkv = values(width * 3 * width, seed + 1, 0.05)
        self.b_qkv = values(3 * width, seed + 2, 0.05)
        self.w_out = values(width * width, seed + 3, 0.05)
        self.b_out = values(width, seed + 4, 0.05)
        self.dy = values(rows * width, seed + 5)

    def layout(self, packed_width, column_offset, time=None, batch=None):
        return oracle.HeadLayout(batch or self.batch, time or self.time, self.heads, self.head_dim, packed_width,
                                 column_offset, time or self.time, 0)

    def per_head(self, left, right, out, count=None):
        return (count or self.batch * self.heads, left, right, out)


def product(rows, cols, inner, lt=False, rt=False, batch=(1, 0, 0, 0), scale=1.0, acc=False):
    return oracle.Product(rows, cols, inner, lt, rt, batch[0], batch[1], batch[2], batch[3], scale, acc)


def linear_forward(x, w, b, rows, inputs, outputs):
    out = np.zeros(rows * outputs, np.float32)
    oracle.matmul_parallel(product(rows, outputs, inputs), x, w, out)
    oracle.add_row_bias(out, outputs, b)
    return out


def linear_backward(x, w, dy, rows, inputs, outputs):
    dw = np.zeros(inputs * outputs, np.float32)
    oracle.matmul_parallel(product(inputs, outputs, rows, lt=True, acc=True), x, dy, dw)
    db = np.zeros(outputs, np.float32)
    oracle.accumulate_column_sums(dy, outputs, db)
    dx = np.zeros(rows * inputs, np.float32)
    oracle.matmul_parallel(product(rows, inputs, outputs, rt=True), dy, w, dx)
    return dw, db, dx


def oracle_layer(L: Layer, backward=True):
    """The reference's forward (and backward) call sequence on the oracle (attention.rs:188-267)."""
    B, T, d, H, h = L.batch, L.time, L.width, L.heads, L.head_dim
    rows, BH = B * T, B * L.heads
    hb, sb = T * h, T * T
    r = {}
    qkv = linear_forward(L.x, L.w_qkv, L.b_qkv, rows, d, 3 * d)
    q, k, v = (np.zeros(BH * T * h, np.float32) for _ in range(3))
    for i, t in enumerate((q, k, v)):
        oracle.split_heads(qkv, t, L.layout(3 * d, i * d))
    p = np.zeros(BH * T * T, np.float32)
    oracle.matmul_parallel(product(T, T, h, rt=True, batch=L.per_head(hb, hb, sb)), q, k, p)
    oracle.causal_softmax(p, T, T, L.scale, 0)
    ctx_heads = np.zeros(BH * T * h, np.float32)
    oracle.matmul_parallel(product(T, h, T, batch=L.per_head(sb, hb, hb)), p, v, ctx_heads)
    ctx = np.zeros(rows * d, np.float32)
    oracle.merge_heads(ctx_heads, ctx, L.layout(d, 0))
    r["qkv"], r["p"], r["context_heads"] = qkv, p, ctx_heads
    r["y"] = linear_forward(ctx, L.w_out, L.b_out, rows, d, d)
    if not backward:
        return r
    r["dw_out"], r["db_out"], dctx = linear_backward(ctx, L.w_out, L.dy, rows, d, d)
    do = np.zeros(BH * T * h, np.float32)
    oracle.split_heads(dctx, do, L.layout(d, 0))
    dp = np.zeros(BH * T * T, np.float32)
    oracle.matmul_parallel(product(T, T, h, rt=True, batch=L.per_head(hb, hb, sb)), do, v, dp)
    dv = np.zeros(BH * T * h, np.float32)
    oracle.matmul_parallel(product(T, h, T, lt=True, batch=L.per_head(sb, hb, hb)), p, do, dv)
    oracle.softmax_backward(p, dp, T)
    dq = np.zeros(BH * T * h, np.float32)
    oracle.matmul_parallel(product(T, h, T, scale=L.scale, batch=L.per_head(sb, hb, hb)), dp, k, dq)
    dk = np.zeros(BH * T * h, np.float32)
    oracle.matmul_parallel(product(T, h, T, lt=True, scale=L.scale, batch=L.per_head(sb, hb, hb)), dp, q, dk)
    dqkv = np.zeros(rows * 3 * d, np.float32)
    for i, t in enumerate((dq, dk, dv)):
        oracle.merge_heads(t, dqkv, L.layout(3 * d, i * d))
    r["ds"], r["dq"], r["dk"], r["dv"] = dp, dq, dk, dv
    r["dw_qkv"], r["db_qkv"], r["dx"] = linear_backward(L.x, L.w_qkv, dqkv, rows, d, 3 * d)
    return r


def gpu_layer(gpu, L: Layer, mode: str):
    """The same layer through the library: the reference's calls one for one (``reference_calls``),
    fused with the probabilities kept (``fused``), or the training attention that keeps none
    (``no_probabilities``: the forward with row statistics and the backward that rebuilds P)."""
    fused = mode != "reference_calls"
    B, T, d, H, h = L.batch, L.time, L.width, L.heads, L.head_dim
    rows, BH = B * T, B * L.heads
    hb, sb = T * h, T * T
    up = lambda a, n=None: gpu.upload(Shape.vector(a.size), a)  # noqa: E731
    zeros = lambda n: gpu.zeros(Shape.vector(n))  # noqa: E731
    matrix = lambda r, c: gpu.zeros(Shape(r, c))  # noqa: E731  (row kernels read the shape)
    layout = lambda width, offset: HeadLayout.dense(B, T, H, h, width, offset)  # noqa: E731
    per_head = lambda left, right, out: BatchStrides(BH, left, right, out)  # noqa: E731
    x, w_qkv, b_qkv, w_out, b_out = (up(a) for a in (L.x, L.w_qkv, L.b_qkv, L.w_out, L.b_out))
    dy = gpu.upload(Shape(rows, d), L.dy)

    def linear_forward_gpu(inp, w, b, out, inputs, outputs):
        spec = MatmulSpec.new(rows, outputs, inputs)
        if fused:
            gpu.matmul_bias(spec, inp, w, b, out)
        else:
            gpu.matmul(spec, inp, w, out)
            gpu.add_row_bias(out, b)

    def linear_backward_gpu(inp, w, dout, dw, db, dinp, inputs, outputs):
        gpu.matmul(MatmulSpec.new(inputs, outputs, rows).left_transposed().accumulate(), inp, dout, dw)
        gpu.accumulate_column_sums(dout, db)
        gpu.matmul(MatmulSpec.new(rows, inputs, outputs).right_transposed(), dout, w, dinp)

    qkv = matrix(rows, 3 * d)
    linear_forward_gpu(x, w_qkv, b_qkv, qkv, d, 3 * d)
    q, k, v = zeros(BH * hb), zeros(BH * hb), zeros(BH * hb)
    for i, t in enumerate((q, k, v)):
        gpu.split_heads(qkv, t, layout(3 * d, i * d))
    p, ctx_heads = matrix(BH * T, T), zeros(BH * hb)
    stats = zeros(2 * BH * T)
    if mode == "no_probabilities":
        gpu.causal_attention_with_stats(q, k, v, ctx_heads, stats, BH, T, T, h, float(L.scale))
    elif fused:
        gpu.causal_attention(q, k, v, ctx_heads, BH, T, T, h, float(L.scale), probabilities=p)
    else:
        gpu.matmul(MatmulSpec.new(T, T, h).right_transposed().batched(per_head(hb, hb, sb)), q, k, p)
        gpu.causal_softmax(p, T, float(L.scale), 0)
        gpu.matmul(MatmulSpec.new(T, h, T).batched(per_head(sb, hb, hb)), p, v, ctx_heads)
    ctx = zeros(rows * d)
    gpu.merge_heads(ctx_heads, ctx, layout(d, 0))
    y = matrix(rows, d)
    linear_forward_gpu(ctx, w_out, b_out, y, d, d)
    # Backward.
    dw_out, db_out, dctx = zeros(d * d), zeros(d), zeros(rows * d)
    linear_backward_gpu(ctx, w_out, dy, dw_out, db_out, dctx, d, d)
    do = zeros(BH * hb)
    gpu.split_heads(dctx, do, layout(d, 0))
    ds, dq, dk, dv = matrix(BH * T, T), zeros(BH * hb), zeros(BH * hb), zeros(BH * hb)
    mix_t = MatmulSpec.new(T, h, T).left_transposed().batched(per_head(sb, hb, hb))
    if mode == "no_probabilities":
        gpu.causal_attention_backward(q, k, v, ctx_heads, do, stats, dq, dk, dv, BH, T, T, h, float(L.scale))
    elif fused:
        gpu.causal_attention_score_grad(do, v, ctx_heads, p, ds, BH, T, T, h, k=k, q_grad=dq, scale=float(L.scale))
        gpu.matmul(mix_t.causal_left(), p, do, dv)
        gpu.matmul(mix_t.scaled(float(L.scale)).causal_left(), ds, q, dk)
    else:
        gpu.matmul(MatmulSpec.new(T, T, h).right_transposed().batched(per_head(hb, hb, sb)), do, v, ds)
        gpu.matmul(mix_t, p, do, dv)
        gpu.softmax_backward(p, ds)
        gpu.matmul(MatmulSpec.new(T, h, T).scaled(float(L.scale)).batched(per_head(sb, hb, hb)), ds, k, dq)
        gpu.matmul(mix_t.scaled(float(L.scale)), ds, q, dk)
    dqkv = matrix(rows, 3 * d)
    for i, t in enumerate((dq, dk, dv)):
        gpu.merge_heads(t, dqkv, layout(3 * d, i * d))
    dw_qkv, db_qkv, dx = zeros(d * 3 * d), zeros(3 * d), zeros(rows * d)
    linear_backward_gpu(x, w_qkv, dqkv, dw_qkv, db_qkv, dx, d, 3 * d)
    out = {"qkv": qkv, "p": p, "context_heads": ctx_heads, "y": y, "dw_out": dw_out, "db_out": db_out, "ds": ds,
           "dq": dq, "dk": dk, "dv": dv, "dw_qkv": dw_qkv, "db_qkv": db_qkv, "dx": dx}
    if mode == "no_probabilities":  # P and dS never exist on this path
        del out["p"], out["ds"]
    return {name: gpu.download(t) for name, t in out.items()}


@pytest.mark.parametrize("mode", ["reference_calls", "fused", "no_probabilities"])
@pytest.mark.parametrize("batch,time,width,heads", [
    (2, 512, 256, 8),   # config 0's layer (d = 256, 8 heads of 32), two sequences of 512
    (2, 300, 256, 4),   # head dim 64 (configs 2 and 3), a ragged sequence length
    (1, 301, 128, 2),   # head dim 64, a sequence length that is not a multiple of 4
])
def test_attention_layer_forward_and_backward(gpu, batch, time, width, heads, mode):
    L = Layer(batch, time, width, heads, seed=time + heads)
    print(f"layer B={batch} T={time} d={width} heads={heads} mode={mode}", flush=True)
    expected = oracle_layer(L)
    got = gpu_layer(gpu, L, mode)
    errors = {}
    for name, a in got.items():
        e = expected[name]
        assert np.all(np.isfinite(a)), name
        errors[name] = oracle.relative_error(e, a)
    print(" ".join(f"{k} {v:.1e}" for k, v in errors.items()))
    bad = {k: v for k, v in errors.items() if not v < TOLERANCE}
    assert not bad, f"relative errors above {TOLERANCE}: {bad}"


@pytest.mark.parametrize("fused", [False, True], ids=["three_calls", "decode_form"])
@pytest.mark.parametrize("time,width,heads", [(301, 256, 8), (701, 768, 12)])
def test_cached_decode_step_equals_the_last_row_of_the_full_forward(gpu, time, width, heads, fused):
    # forward_cached (attention.rs:274-320): the prompt's keys and values are in the cache, the
    # last position is decoded against it, and its output must be the full forward's last row
    # (model_is_trainable.rs:161-213). The cache's capacity is 1408; its unwritten tail holds NaN.
    L = Layer(1, time, width, heads, seed=width + heads)
    print(f"decode step T={time} d={width} heads={heads} fused={fused}", flush=True)
    expected = oracle_layer(L, backward=False)["y"].reshape(time, width)[-1]
    d, h, cap, prefix = width, width // heads, 1408, time - 1
    up = lambda a: gpu.upload(Shape.vector(a.size), a)  # noqa: E731
    zeros = lambda n: gpu.zeros(Shape.vector(n))  # noqa: E731
    w_qkv, b_qkv, w_out, b_out = (up(a) for a in (L.w_qkv, L.b_qkv, L.w_out, L.b_out))
    x = L.x.reshape(time, width)
    keys = up(np.full(heads * cap * h, np.nan, np.float32))
    vals = up(np.full(heads * cap * h, np.nan, np.float32))
    # Prefill: the prompt's projections into the cache from position 0.
    prompt_qkv = zeros(prefix * 3 * d)
    gpu.matmul_bias(MatmulSpec.new(prefix, 3 * d, d), up(np.ascontiguousarray(x[:prefix])), w_qkv, b_qkv, prompt_qkv)
    for i, t in ((1, keys), (2, vals)):
        gpu.split_heads(prompt_qkv, t, HeadLayout.dense(1, prefix, heads, h, 3 * d, i * d).in_cache(cap, 0))
    # The decode step: one new position at offset `prefix`.
    qkv = zeros(3 * d)
    gpu.matmul_bias(MatmulSpec.new(1, 3 * d, d), up(np.ascontiguousarray(x[prefix:])), w_qkv, b_qkv, qkv)
    q = zeros(heads * h)
    gpu.split_heads(qkv, q, HeadLayout.dense(1, 1, heads, h, 3 * d, 0))
    for i, t in ((1, keys), (2, vals)):
        gpu.split_heads(qkv, t, HeadLayout.dense(1, 1, heads, h, 3 * d, i * d).in_cache(cap, prefix))
    ctx_heads = zeros(heads * h)
    if fused:
        gpu.causal_attention(q, keys, vals, ctx_heads, heads, 1, cap, h, float(L.scale), query_offset=prefix,
                             q_stride=h, kv_stride=cap * h)
    else:
        scores = gpu.zeros(Shape(heads, cap))
        gpu.matmul(MatmulSpec.new(1, cap, h).right_transposed().batched(BatchStrides(heads, h, cap * h, cap))
                   .causal_output(prefix), q, keys, scores)
        gpu.causal_softmax(scores, 1, float(L.scale), prefix)
        gpu.matmul(MatmulSpec.new(1, h, cap).batched(BatchStrides(heads, cap, cap * h, h)).causal_left(prefix),
                   scores, vals, ctx_heads)
    ctx = zeros(d)
    gpu.merge_heads(ctx_heads, ctx, HeadLayout.dense(1, 1, heads, h, d, 0))
    y = zeros(d)
    gpu.matmul_bias(MatmulSpec.new(1, d, d), ctx, w_out, b_out, y)
    got = gpu.download(y)
    assert np.all(np.isfinite(got))
    error = oracle.relative_error(expected, got)
    print(f"last row relative error {error:.2e}")
    assert error < TOLERANCE

"""GPU parity at the benchmark configurations' shapes (configs 0-4), through the C ABI.

Inputs are seeded synthetic data generated in device memory (the same bytes
are downloaded for the oracle): activations and gradients ~N(0,1), weights
~N(0,0.02). Each product is the one the reference's model issues:
``Linear::forward`` (NN), ``Linear::backward`` (TN dW with accumulate, NT dX)
in crates/staleynet-model/src/layers/linear.rs:43-63, the 16-codebook head
(gpt.rs:72), the attention products (layers/attention.rs:197-267) and the
cached decode products (attention.rs:274-320).

Comparison, in the reference test's metric max|Δ|/max|expected|
(kernels_match_reference.rs:41-52), bound 1e-5 for fp32:
* config 0 (7.1M, M = 2048): every output of every product;
* configs 1 and 2 (M = 8192, 32768): 65536 sampled outputs per product,
  each computed by the oracle in the reference's order; the error against
  an f64 sum is recorded beside it;
* config 3 (causal attention, T = 2048, h = 64): every output of every head
  of a 4-head batch (config 3's per-head shape; its 192 heads repeat it);
* config 4 (decode, M in {1, 4, 16}): every output.
"""
import numpy as np
import pytest

from oracle import oracle
from staleynet_amd.gemm import BatchStrides, MatmulSpec, Shape

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-5
SEED = 1234
SAMPLES = 65536
MODELS = {
    "c0": dict(tokens=4 * 512, width=256, ffn=1024),
    "c1": dict(tokens=8 * 1024, width=512, ffn=2048),
    "c2": dict(tokens=16 * 2048, width=768, ffn=3072),
}
HEAD = 16 * 1024


def linears(model):
    d, f = model["width"], model["ffn"]
    return {"qkv": (d, 3 * d), "out": (d, d), "up": (d, f), "down": (f, d), "head": (d, HEAD)}


def product_of(spec: MatmulSpec) -> oracle.Product:
    return oracle.Product(spec.rows, spec.cols, spec.inner, bool(spec.left), bool(spec.right), spec.batch.count,
                          spec.batch.left, spec.batch.right, spec.batch.output, spec.scale, bool(spec.write))


def normal(gpu, shape, stream, std=1.0):
    t = gpu.zeros(shape)
    gpu.fill_normal(t, SEED, stream, 0.0, std)
    return t


def compare(spec, left, right, previous, actual, full: bool, rng):
    """Relative error of `actual` against the oracle (all outputs or a sample)."""
    product = product_of(spec)
    if full:
        expected = previous.copy() if spec.write else np.zeros_like(actual)
        oracle.matmul_parallel(product, left, right, expected)
        assert np.all(np.isfinite(actual))
        return oracle.relative_error(expected, actual), None
    total = spec.batch.count * spec.rows * spec.cols
    picks = rng.choice(total, size=min(SAMPLES, total), replace=False)
    b, rest = np.divmod(picks, spec.rows * spec.cols)
    r, c = np.divmod(rest, spec.cols)
    flat = b * spec.batch.output + r * spec.cols + c
    prev = previous[flat] if spec.write else None
    expected = oracle.matmul_elements_parallel(product, left, right, b, r, c, prev)
    truth = oracle.matmul_elements_parallel(product, left, right, b, r, c, prev, f64=True)
    got = actual[flat]
    assert np.all(np.isfinite(got))
    f64_error = float(np.max(np.abs(got.astype(np.float64) - truth)) / np.max(np.abs(truth)))
    return oracle.relative_error(expected, got), f64_error


@pytest.mark.parametrize("config,layer", [(c, l) for c in MODELS for l in ("qkv", "out", "up", "down", "head")])
def test_linear_products_match_the_oracle(gpu, config, layer):
    model = MODELS[config]
    m = model["tokens"]
    inputs, outputs = linears(model)[layer]
    base = 10 * list(MODELS).index(config) + 3 * ["qkv", "out", "up", "down", "head"].index(layer)
    x = normal(gpu, Shape(m, inputs), base + 0)
    w = normal(gpu, Shape(inputs, outputs), base + 1, 0.02)
    dy = normal(gpu, Shape(m, outputs), base + 2)
    dw = normal(gpu, Shape(inputs, outputs), base + 3, 0.01)  # a gradient accumulated earlier
    y, dx = gpu.zeros(Shape(m, outputs)), gpu.zeros(Shape(m, inputs))
    dw_before = gpu.download(dw)

    forward = MatmulSpec.new(m, outputs, inputs)
    weight_grad = MatmulSpec.new(inputs, outputs, m).left_transposed().accumulate()
    input_grad = MatmulSpec.new(m, inputs, outputs).right_transposed()
    gpu.matmul(forward, x, w, y)
    gpu.matmul(weight_grad, x, dy, dw)
    gpu.matmul(input_grad, dy, w, dx)
    xh, wh, dyh = gpu.download(x), gpu.download(w), gpu.download(dy)

    full = config == "c0"
    rng = np.random.default_rng(base)
    results = {}
    for name, spec, left, right, prev, out in (("NN", forward, xh, wh, None, y),
                                                ("TN", weight_grad, xh, dyh, dw_before, dw),
                                                ("NT", input_grad, dyh, wh, None, dx)):
        error, f64_error = compare(spec, left, right, prev, gpu.download(out), full, rng)
        results[name] = (error, f64_error)
        assert error < TOLERANCE, f"{config} {layer} {name}: relative error {error} (f64 {f64_error})"
    print(f"{config} {layer}: " + ", ".join(f"{k} {e:.2e}" + (f" (f64 {f:.2e})" if f is not None else "")
                                            for k, (e, f) in results.items()))


# ---- config 3: causal attention -------------------------------------------------------------

T, H, HEADS = 2048, 64, 4


@pytest.fixture(scope="module")
def attention(gpu):
    """Q, K, V, dO ~ N(0,1); P = causal softmax of seeded scores at scale 1/8
    (reference.rs:101-119); dS = softmax backward of P and a seeded dP
    (reference.rs:122-137). Row-major [heads·T, ·] as attention.rs:56-95 lays them out."""
    q = normal(gpu, Shape(HEADS * T, H), 100)
    k = normal(gpu, Shape(HEADS * T, H), 101)
    v = normal(gpu, Shape(HEADS * T, H), 102)
    do = normal(gpu, Shape(HEADS * T, H), 103)
    scores = normal(gpu, Shape(HEADS * T, T), 104)
    upstream = normal(gpu, Shape(HEADS * T, T), 105)
    p = gpu.download(scores)
    oracle.causal_softmax(p, T, T, 0.125, 0)
    ds = gpu.download(upstream)
    oracle.softmax_backward(p, ds, T)
    host = {"q": gpu.download(q), "k": gpu.download(k), "v": gpu.download(v), "do": gpu.download(do), "p": p,
            "ds": ds}
    dev = {"q": q, "k": k, "v": v, "do": do, "p": gpu.upload(Shape(HEADS * T, T), p),
           "ds": gpu.upload(Shape(HEADS * T, T), ds)}
    return host, dev


def attention_specs():
    head, score = T * H, T * T
    per_head = lambda left, right, out: BatchStrides(HEADS, left, right, out)  # noqa: E731
    s = 0.125
    # (name, spec, left, right, output kind) following attention.rs:206-260.
    return [
        ("scores", MatmulSpec.new(T, T, H).right_transposed().batched(per_head(head, head, score)), "q", "k", "out"),
        ("mix", MatmulSpec.new(T, H, T).batched(per_head(score, head, head)), "p", "v", "left"),
        ("prob_grad", MatmulSpec.new(T, T, H).right_transposed().batched(per_head(head, head, score)), "do", "v",
         "out"),
        ("value_grad", MatmulSpec.new(T, H, T).left_transposed().batched(per_head(score, head, head)), "p", "do",
         "left"),
        ("query_grad", MatmulSpec.new(T, H, T).scaled(s).batched(per_head(score, head, head)), "ds", "k", "left"),
        ("key_grad", MatmulSpec.new(T, H, T).left_transposed().scaled(s).batched(per_head(score, head, head)), "ds",
         "q", "left"),
    ]


@pytest.mark.parametrize("masked", [False, True], ids=["dense", "causal"])
@pytest.mark.parametrize("index", range(6), ids=[a[0] for a in attention_specs()])
def test_attention_products_match_the_oracle(gpu, attention, index, masked):
    host, dev = attention
    name, spec, left, right, kind = attention_specs()[index]
    if masked:
        spec = spec.causal_output() if kind == "out" else spec.causal_left()
    out = gpu.zeros(Shape(HEADS * spec.rows, spec.cols))
    gpu.matmul(spec, dev[left], dev[right], out)
    actual = gpu.download(out)
    expected = np.zeros_like(actual)
    oracle.matmul_parallel(product_of(spec), host[left], host[right], expected)
    assert np.all(np.isfinite(actual))
    if masked and kind == "out":
        q = np.arange(T)[:, None]
        visible = np.broadcast_to(np.arange(T)[None, :] <= q, (HEADS, T, T)).ravel()
        error = oracle.relative_error(expected[visible], actual[visible])
        assert np.all(actual[~visible] == 0.0)
    else:
        error = oracle.relative_error(expected, actual)
    assert error < TOLERANCE, f"{name} masked={masked}: relative error {error}"


# ---- config 3 at its full batch: 192 heads, sampled -------------------------------------------
# The launches bench.py times: 16 x 12 = 192 heads of T = 2048, h = 64, whose batch the tiled
# kernels deal over the XCDs in whole heads. Each product is checked on 65536 sampled outputs,
# each computed by the oracle in the reference's order; the fused kernels on 1024 sampled
# (head, query) rows, each the oracle's three calls (or the backward's calls) on that row alone,
# which is the same arithmetic as the full calls give that row.

BH3, ROWS3 = 192, 1024


@pytest.fixture(scope="module")
def attention_full(gpu):
    """Q, K, V, dO ~ N(0, 1) in device memory; P and dS from the fused kernels (causal matrices with
    zeros past the diagonal, inputs of the products here), and the host copies."""
    q, k, v, do = (normal(gpu, Shape(BH3 * T, H), 500 + i) for i in range(4))
    o = gpu.zeros(Shape(BH3 * T, H))
    p = gpu.zeros(Shape(BH3 * T, T))
    gpu.causal_attention(q, k, v, o, BH3, T, T, H, 0.125, probabilities=p)
    ds = gpu.zeros(Shape(BH3 * T, T))
    dq = gpu.zeros(Shape(BH3 * T, H))
    gpu.causal_attention_score_grad(do, v, o, p, ds, BH3, T, T, H, k=k, q_grad=dq, scale=0.125)
    dev = {"q": q, "k": k, "v": v, "do": do, "o": o, "p": p, "ds": ds, "dq": dq}
    host = {name: gpu.download(t) for name, t in dev.items()}
    yield host, dev
    for t in dev.values():
        t.free()


def full_batch_specs():
    head, score = T * H, T * T
    per_head = lambda left, right, out: BatchStrides(BH3, left, right, out)  # noqa: E731
    return [
        ("scores", MatmulSpec.new(T, T, H).right_transposed().batched(per_head(head, head, score)), "q", "k", "out"),
        ("mix", MatmulSpec.new(T, H, T).batched(per_head(score, head, head)), "p", "v", "left"),
        ("prob_grad", MatmulSpec.new(T, T, H).right_transposed().batched(per_head(head, head, score)), "do", "v",
         "out"),
        ("value_grad", MatmulSpec.new(T, H, T).left_transposed().batched(per_head(score, head, head)), "p", "do",
         "left"),
        ("query_grad", MatmulSpec.new(T, H, T).scaled(0.125).batched(per_head(score, head, head)), "ds", "k",
         "left"),
        ("key_grad", MatmulSpec.new(T, H, T).left_transposed().scaled(0.125).batched(per_head(score, head, head)),
         "ds", "q", "left"),
    ]


@pytest.mark.parametrize("masked", [False, True], ids=["dense", "causal"])
@pytest.mark.parametrize("index", range(6), ids=[a[0] for a in full_batch_specs()])
def test_attention_products_over_all_192_heads(gpu, attention_full, index, masked):
    host, dev = attention_full
    name, spec, left, right, kind = full_batch_specs()[index]
    print(f"c3 192 heads: {name} masked={masked}", flush=True)
    if masked:
        spec = spec.causal_output() if kind == "out" else spec.causal_left()
    out = gpu.zeros(Shape(BH3 * spec.rows, spec.cols))
    gpu.matmul(spec, dev[left], dev[right], out)
    actual = gpu.download(out)
    out.free()
    rng = np.random.default_rng(index + 10 * masked)
    picks = rng.choice(actual.size, size=SAMPLES, replace=False)
    b, rest = np.divmod(picks, spec.rows * spec.cols)
    r, c = np.divmod(rest, spec.cols)
    got = actual[picks]
    assert np.all(np.isfinite(got))
    expected = oracle.matmul_elements_parallel(product_of(spec), host[left], host[right], b, r, c)
    if masked and kind == "out":
        visible = c <= r
        assert np.all(got[~visible] == 0.0)
        error = oracle.relative_error(expected[visible], got[visible])
    else:
        error = oracle.relative_error(expected, got)
    assert error < TOLERANCE, f"{name} masked={masked}: relative error {error}"
    # Every head is represented in the sample.
    assert len(np.unique(b)) == BH3


def sampled_rows(seed):
    rng = np.random.default_rng(seed)
    picks = rng.choice(BH3 * T, size=ROWS3, replace=False)
    return np.divmod(picks, T)


def one_row(rows, cols, inner, right_transposed=False, scale=1.0):
    return oracle.Product(rows, cols, inner, False, right_transposed, 1, 0, 0, 0, scale, False)


def test_fused_forward_over_all_192_heads(gpu, attention_full):
    # sn_causal_attention at config 3's full batch against the three calls of attention.rs:206-213.
    host, _ = attention_full
    heads, queries = sampled_rows(1)
    o_err, p_err = [], []
    expected_o, got_o, expected_p, got_p = [], [], [], []
    for b, r in zip(heads, queries):
        row = b * T + r
        k_head, v_head = host["k"][b * T * H:(b + 1) * T * H], host["v"][b * T * H:(b + 1) * T * H]
        s = np.zeros(T, np.float32)
        oracle.matmul(one_row(1, T, H, right_transposed=True), host["q"][row * H:(row + 1) * H], k_head, s)
        oracle.causal_softmax(s, 1, T, 0.125, int(r))  # query r of its head sees keys 0 ..= r
        o = np.zeros(H, np.float32)
        oracle.matmul(one_row(1, H, T), s, v_head, o)
        expected_o.append(o)
        got_o.append(host["o"][row * H:(row + 1) * H])
        expected_p.append(s)
        got_p.append(host["p"][row * T:(row + 1) * T])
    assert len(np.unique(heads)) > 150
    for name, e, g in (("O", expected_o, got_o), ("P", expected_p, got_p)):
        e, g = np.concatenate(e), np.concatenate(g)
        assert np.all(np.isfinite(g))
        error = oracle.relative_error(e, g)
        print(f"fused forward {name}: {error:.2e}")
        assert error < TOLERANCE


def test_fused_score_and_query_gradients_over_all_192_heads(gpu, attention_full):
    # sn_causal_attention_score_grad (with dQ) at config 3's full batch against the backward's dP
    # product, softmax_backward and dQ product (attention.rs:238-253), given the same P.
    host, _ = attention_full
    heads, queries = sampled_rows(2)
    expected_ds, got_ds, expected_dq, got_dq = [], [], [], []
    for b, r in zip(heads, queries):
        row = b * T + r
        k_head, v_head = host["k"][b * T * H:(b + 1) * T * H], host["v"][b * T * H:(b + 1) * T * H]
        dp = np.zeros(T, np.float32)
        oracle.matmul(one_row(1, T, H, right_transposed=True), host["do"][row * H:(row + 1) * H], v_head, dp)
        p = host["p"][row * T:(row + 1) * T].copy()
        oracle.softmax_backward(p, dp, T)
        dq = np.zeros(H, np.float32)
        oracle.matmul(one_row(1, H, T, scale=0.125), dp, k_head, dq)
        expected_ds.append(dp)
        got_ds.append(host["ds"][row * T:(row + 1) * T])
        expected_dq.append(dq)
        got_dq.append(host["dq"][row * H:(row + 1) * H])
    for name, e, g in (("dS", expected_ds, got_ds), ("dQ", expected_dq, got_dq)):
        e, g = np.concatenate(e), np.concatenate(g)
        assert np.all(np.isfinite(g))
        error = oracle.relative_error(e, g)
        print(f"fused score gradient {name}: {error:.2e}")
        assert error < TOLERANCE


# ---- config 4: decode shapes ----------------------------------------------------------------

@pytest.mark.parametrize("rows", [1, 4, 16])
@pytest.mark.parametrize("inputs,outputs", [(768, 2304), (768, 768), (768, 3072), (3072, 768), (768, HEAD)])
def test_decode_products_match_the_oracle(gpu, rows, inputs, outputs):
    x = normal(gpu, Shape(rows, inputs), 200 + rows)
    w = normal(gpu, Shape(inputs, outputs), 210, 0.02)
    y = gpu.zeros(Shape(rows, outputs))
    spec = MatmulSpec.new(rows, outputs, inputs)
    gpu.matmul(spec, x, w, y)
    error, _ = compare(spec, gpu.download(x), gpu.download(w), None, gpu.download(y), True, None)
    assert error < TOLERANCE


@pytest.mark.parametrize("cached", [0, 700, 1407])
def test_cached_decode_attention_matches_the_oracle(gpu, cached):
    # forward_cached (attention.rs:300-316): one new position against a cache
    # of capacity 1408 per head; scores masked at query_offset = cached.
    heads, capacity, n = 12, 1408, 1
    q = normal(gpu, Shape(heads * n, H), 300)
    keys = normal(gpu, Shape(heads * capacity, H), 301)
    values = normal(gpu, Shape(heads * capacity, H), 302)
    scores_spec = MatmulSpec.new(n, capacity, H).right_transposed().batched(
        BatchStrides(heads, n * H, capacity * H, n * capacity))
    scores = gpu.zeros(Shape(heads * n, capacity))
    gpu.matmul(scores_spec.causal_output(cached), q, keys, scores)
    s = gpu.download(scores)
    dense = np.zeros_like(s)
    qh, kh, vh = gpu.download(q), gpu.download(keys), gpu.download(values)
    oracle.matmul(product_of(scores_spec), qh, kh, dense)
    visible = np.broadcast_to(np.arange(capacity)[None, :] <= cached, (heads, capacity)).ravel()
    assert oracle.relative_error(dense[visible], s[visible]) < TOLERANCE
    assert np.all(s[~visible] == 0.0)
    p = s.copy()
    oracle.causal_softmax(p, n, capacity, 0.125, cached)
    mix_spec = MatmulSpec.new(n, H, capacity).batched(BatchStrides(heads, n * capacity, capacity * H, n * H))
    out = gpu.zeros(Shape(heads * n, H))
    gpu.matmul(mix_spec.causal_left(cached), gpu.upload(Shape(heads * n, capacity), p), values, out)
    expected = np.zeros(heads * n * H, np.float32)
    oracle.matmul(product_of(mix_spec), p, vh, expected)
    assert oracle.relative_error(expected, gpu.download(out)) < TOLERANCE


# ---- bf16-input variant at config 2 ----------------------------------------------------------

@pytest.mark.parametrize("layer", ["qkv", "out", "up", "down", "head"])
def test_bf16_products_within_the_stated_tolerance(gpu, layer):
    """bf16 inputs with fp32 accumulation against the fp32 oracle: max relative
    error below 2e-2 (the variant's stated tolerance)."""
    from staleynet_amd.gemm import Precision
    model = MODELS["c2"]
    m = model["tokens"]
    inputs, outputs = linears(model)[layer]
    x = normal(gpu, Shape(m, inputs), 400)
    w = normal(gpu, Shape(inputs, outputs), 401, 0.02)
    dy = normal(gpu, Shape(m, outputs), 402)
    y, dx, dw = gpu.zeros(Shape(m, outputs)), gpu.zeros(Shape(m, inputs)), gpu.zeros(Shape(inputs, outputs))
    specs = [(MatmulSpec.new(m, outputs, inputs), x, w, y),
             (MatmulSpec.new(inputs, outputs, m).left_transposed().accumulate(), x, dy, dw),
             (MatmulSpec.new(m, inputs, outputs).right_transposed(), dy, w, dx)]
    host = {id(x): gpu.download(x), id(w): gpu.download(w), id(dy): gpu.download(dy)}
    rng = np.random.default_rng(7)
    for spec, left, right, out in specs:
        gpu.matmul(spec.with_precision(Precision.Bf16), left, right, out)
        error, _ = compare(spec, host[id(left)], host[id(right)], np.zeros(len(out), np.float32),
                           gpu.download(out), False, rng)
        assert error < 2e-2, f"bf16 {layer} {spec}: relative error {error}"

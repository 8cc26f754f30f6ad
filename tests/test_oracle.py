"""Pins the CPU oracle (oracle/matmul_oracle.c) before anything is checked against it.

Each check is chosen so that a plausible mistake in the restatement of
``reference::matmul`` (crates/staleynet-cuda/src/reference.rs:19-38) fails:
the reference's own known-answer tests, an order-sensitive case, exact
integer arithmetic, transpose/broadcast/scale/accumulate identities and an
f64 error bound.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle
from oracle.oracle import Product

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


def run(product: Product, left, right, output):
    left = np.asarray(left, np.float32)
    right = np.asarray(right, np.float32)
    out = np.asarray(output, np.float32).copy()
    oracle.matmul(product, left, right, out)
    return out


# ---- the reference's known-answer tests (reference.rs:177-232) -------------

@pytest.mark.parametrize("case", [c["name"] for c in json.load(open(os.path.join(GOLDEN, "reference_kats.json")))["matmul"]])
def test_reference_known_answers(case):
    kat = next(c for c in kats()["matmul"] if c["name"] == case)
    s = kat["spec"]
    product = Product(s["rows"], s["cols"], s["inner"], s.get("left_transposed", False),
                      s.get("right_transposed", False), s.get("count", 1), s.get("batch_left", 0),
                      s.get("batch_right", 0), s.get("batch_output", 0), s.get("scale", 1.0),
                      s.get("accumulate", False))
    out = run(product, kat["left"], kat["right"], kat["initial"])
    assert out.tolist() == kat["expected"]  # exact: every value is an exact small integer/half


def test_softmax_known_answers():
    data = kats()
    for kat in data["causal_softmax"]:
        scores = np.asarray(kat["scores"], np.float32)
        oracle.causal_softmax(scores, kat["queries"], kat["keys"], kat["scale"], kat["query_offset"])
        for index, value in kat["expected"].items():
            assert abs(scores[int(index)] - value) <= 1e-6
        for row in range(scores.size // kat["keys"]):
            assert abs(scores[row * kat["keys"]:(row + 1) * kat["keys"]].sum() - 1.0) <= 1e-6
    kat = data["softmax_backward"]
    grad = np.asarray(kat["grad"], np.float32)
    oracle.softmax_backward(np.asarray(kat["probabilities"], np.float32), grad, kat["cols"])
    assert np.allclose(grad, kat["expected"], atol=1e-6, rtol=0)


def test_causal_softmax_with_offset_orders_and_masks():
    # reference.rs:283-293: scale 0.5, offset 1, rows of [1, 2, 3].
    scores = np.asarray([1, 2, 3, 1, 2, 3], np.float32)
    oracle.causal_softmax(scores, 2, 3, 0.5, 1)
    assert scores[0] < scores[1] and scores[2] == 0.0
    assert scores[3] < scores[4] < scores[5]
    assert abs(scores[:3].sum() - 1) <= 1e-6 and abs(scores[3:].sum() - 1) <= 1e-6


# ---- summation order ---------------------------------------------------------

def test_sum_is_sequential_in_k_with_f32_rounding():
    # 2^24 + 1 rounds to 2^24 in f32, so summing k in order gives 0, while
    # the exact value (or any order that adds -2^24 before +1) gives 1.
    out = run(Product(1, 1, 3), [2.0 ** 24, 1.0, -(2.0 ** 24)], [1.0, 1.0, 1.0], [7.0])
    assert out[0] == 0.0
    # Reversing k changes the result: the oracle does not reorder.
    out = run(Product(1, 1, 3), [-(2.0 ** 24), 1.0, 2.0 ** 24], [1.0, 1.0, 1.0], [7.0])
    assert out[0] == 1.0


def test_products_are_rounded_before_the_sum():
    # x = 1 + 2^-12: x·x = 1 + 2^-11 + 2^-24 exactly, which rounds (ties to
    # even) to 1 + 2^-11. Summing [1·c, x·x] with c = -(1 + 2^-11) gives 0 when
    # the product is rounded first; a fused multiply-add would keep 2^-24.
    x = np.float32(1 + 2.0 ** -12)
    c = np.float32(-(1 + 2.0 ** -11))
    out = run(Product(1, 1, 2), [1.0, x], [c, x], [5.0])
    assert out[0] == 0.0


def test_scaled_sum_is_rounded_before_it_is_added_to_previous():
    # s = 1 + 2^-23: scale·sum = s·s = 1 + 2^-22 + 2^-46 rounds to 1 + 2^-22,
    # so prev + scale·sum = 0 for prev = -(1 + 2^-22); fusing would give 2^-46.
    s = np.float32(1 + 2.0 ** -23)
    out = run(Product(1, 1, 1, scale=float(s), accumulate=True), [s], [1.0], [-(1 + 2.0 ** -22)])
    assert out[0] == 0.0


# ---- exact integer arithmetic --------------------------------------------------

@pytest.mark.parametrize("left_t", [False, True])
@pytest.mark.parametrize("right_t", [False, True])
def test_integer_inputs_match_exact_integer_products(left_t, right_t):
    rng = np.random.default_rng(7)
    rows, cols, inner, count = 13, 11, 17, 3
    a = rng.integers(-8, 9, size=(count, rows, inner))
    b = rng.integers(-8, 9, size=(count, inner, cols))
    prev = rng.integers(-50, 51, size=(count, rows, cols))
    stored_a = np.ascontiguousarray(np.swapaxes(a, 1, 2) if left_t else a).astype(np.float32).ravel()
    stored_b = np.ascontiguousarray(np.swapaxes(b, 1, 2) if right_t else b).astype(np.float32).ravel()
    product = Product(rows, cols, inner, left_t, right_t, count, rows * inner, inner * cols, rows * cols, 2.0, True)
    out = run(product, stored_a, stored_b, prev.astype(np.float32).ravel())
    expected = prev + 2 * np.einsum("bij,bjk->bik", a, b)
    assert np.array_equal(out, expected.astype(np.float32).ravel())


# ---- identities over random inputs ------------------------------------------

def _random(count, seed):
    return oracle.random_values(count, seed)


def test_transposed_storage_equals_explicit_transpose_bitwise():
    rows, cols, inner = 9, 14, 23
    a = _random(rows * inner, 1).reshape(rows, inner)
    b = _random(inner * cols, 2).reshape(inner, cols)
    base = run(Product(rows, cols, inner), a.ravel(), b.ravel(), np.zeros(rows * cols))
    both = run(Product(rows, cols, inner, True, True), np.ascontiguousarray(a.T).ravel(),
               np.ascontiguousarray(b.T).ravel(), np.zeros(rows * cols))
    assert np.array_equal(base, both)


def test_zero_batch_stride_broadcasts():
    rows, cols, inner, count = 5, 6, 7, 4
    a = _random(count * rows * inner, 3)
    b = _random(inner * cols, 4)
    out = run(Product(rows, cols, inner, count=count, batch_left=rows * inner, batch_right=0,
                      batch_output=rows * cols), a, b, np.zeros(count * rows * cols))
    for i in range(count):
        single = run(Product(rows, cols, inner), a[i * rows * inner:(i + 1) * rows * inner], b,
                     np.zeros(rows * cols))
        assert np.array_equal(out[i * rows * cols:(i + 1) * rows * cols], single)


def test_power_of_two_scale_is_exact_and_accumulate_adds_previous():
    rows, cols, inner = 8, 8, 33
    a, b, prev = _random(rows * inner, 5), _random(inner * cols, 6), _random(rows * cols, 7)
    plain = run(Product(rows, cols, inner), a, b, np.zeros(rows * cols))
    scaled = run(Product(rows, cols, inner, scale=0.25), a, b, np.zeros(rows * cols))
    assert np.array_equal(scaled, (plain * np.float32(0.25)).astype(np.float32))
    acc = run(Product(rows, cols, inner, scale=0.7, accumulate=True), a, b, prev)
    over = run(Product(rows, cols, inner, scale=0.7), a, b, np.zeros(rows * cols))
    assert np.array_equal(acc, (prev + over).astype(np.float32))


def test_error_against_f64_is_within_the_sequential_bound():
    # |fl(sum) - sum| <= (k-1)·u·Σ|a||b| + k·u·Σ|a||b| for sequential f32 sums, u = 2^-24.
    rows, cols, inner = 4, 5, 4096
    a, b = _random(rows * inner, 8), _random(inner * cols, 9)
    p = Product(rows, cols, inner)
    out = run(p, a, b, np.zeros(rows * cols))
    r, c = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    truth = oracle.matmul_elements_f64(p, a, b, np.zeros(r.size), r.ravel(), c.ravel())
    mags = np.abs(a.reshape(rows, inner).astype(np.float64)) @ np.abs(b.reshape(inner, cols).astype(np.float64))
    bound = 2 * inner * 2.0 ** -24 * mags.ravel()
    assert np.all(np.abs(out.astype(np.float64) - truth) <= bound)
    assert np.max(np.abs(out - truth)) > 0  # f32 rounding is visible at this size


def test_elements_and_rows_agree_with_the_full_product():
    rows, cols, inner, count = 7, 9, 31, 2
    a, b, prev = _random(count * rows * inner, 10), _random(count * inner * cols, 11), _random(count * rows * cols, 12)
    p = Product(rows, cols, inner, True, False, count, rows * inner, inner * cols, rows * cols, 0.7, True)
    full = run(p, a, b, prev)
    part = prev.copy()
    oracle.matmul_rows(p, a, b, part, 2, 5)
    rows_mask = np.zeros((count, rows, cols), bool)
    rows_mask[:, 2:5, :] = True
    assert np.array_equal(part.reshape(count, rows, cols)[rows_mask], full.reshape(count, rows, cols)[rows_mask])
    assert np.array_equal(part.reshape(count, rows, cols)[~rows_mask], prev.reshape(count, rows, cols)[~rows_mask])
    bi, ri, ci = np.meshgrid(np.arange(count), np.arange(rows), np.arange(cols), indexing="ij")
    got = oracle.matmul_elements(p, a, b, bi.ravel(), ri.ravel(), ci.ravel(), prev)
    assert np.array_equal(got, full)


# ---- the test harness pieces -------------------------------------------------

def test_random_values_follow_knuths_mmix_lcg():
    # kernels_match_reference.rs:26-38 with Python integers as the arbitrary-precision check.
    mult, inc, mask = 6364136223846793005, 1442695040888963407, (1 << 64) - 1
    for seed in (0, 1, 2, 3, 12345):
        state = (seed * mult + inc) & mask
        expected = []
        for _ in range(100):
            state = (state * mult + inc) & mask
            expected.append((state >> 40) / 2.0 ** 24 * 2.0 - 1.0)
        got = oracle.random_values(100, seed)
        assert got.tolist() == expected  # every step is exact in f32
    values = oracle.random_values(1 << 16, 1)
    assert values.min() >= -1.0 and values.max() < 1.0
    assert abs(values.mean()) < 0.01 and abs(values.var() - 1 / 3) < 0.01


def test_relative_error_follows_the_reference_metric():
    expected = np.asarray([1.0, -4.0, 2.0], np.float32)
    actual = np.asarray([1.5, -4.0, 1.0], np.float32)
    assert oracle.relative_error(expected, actual) == pytest.approx(1.0 / 4.0)
    # The magnitude floor is f32::EPSILON.
    assert oracle.relative_error(np.zeros(3, np.float32), np.full(3, 1e-7, np.float32)) == pytest.approx(
        1e-7 / np.finfo(np.float32).eps)
    # Like Rust's f32::max, a NaN difference is skipped by the fold.
    assert oracle.relative_error(expected, np.asarray([np.nan, -4.0, 2.0], np.float32)) == 0.0


def test_parallel_drivers_are_bit_identical_to_the_serial_loop():
    rows, cols, inner, count = 64, 50, 70, 2
    p = Product(rows, cols, inner, True, False, count, rows * inner, inner * cols, rows * cols, 0.7, True)
    a, b, c = _random(count * rows * inner, 1), _random(count * inner * cols, 2), _random(count * rows * cols, 3)
    serial = run(p, a, b, c)
    threaded = c.copy()
    oracle.matmul_parallel(p, a, b, threaded, workers=5)
    assert np.array_equal(serial, threaded)
    bi, ri, ci = np.meshgrid(np.arange(count), np.arange(rows), np.arange(cols), indexing="ij")
    picked = oracle.matmul_elements_parallel(p, a, b, bi.ravel(), ri.ravel(), ci.ravel(), c, workers=7)
    assert np.array_equal(serial, picked)


# ---- Linear's bias kernels (kernels/elementwise.rs:62-93) -------------------

def test_reference_elementwise_test_for_bias_and_column_sums():
    # kernels_match_reference.rs:125-170 on its own inputs: shape 9 x 50, LCG seeds 7 (input), 9 (bias).
    # The expected column sums there are bias[c] + the f32 sum of the column in row order
    # (`.sum::<f32>()` folds left from 0), written here as an explicit f32 loop.
    rows, cols = 9, 50
    values = oracle.random_values(rows * cols, 7)
    bias = oracle.random_values(cols, 9)
    expected = np.empty(cols, np.float32)
    for c in range(cols):
        total = np.float32(0.0)
        for r in range(rows):
            total = np.float32(total + values[r * cols + c])
        expected[c] = np.float32(bias[c] + total)
    sums = bias.copy()
    oracle.accumulate_column_sums(values, cols, sums)
    assert np.array_equal(sums, expected)
    # add_row_bias: output[i] + bias[i % cols], one f32 add per element.
    out = values.copy()
    oracle.add_row_bias(out, cols, bias)
    assert np.array_equal(out, (values + np.tile(bias, rows)).astype(np.float32))


def test_column_sums_are_sequential_in_rows_with_f32_rounding():
    # Column 0: 2^24, 1, 1, -2^24 -> sequential f32 gives 0 (each 2^24 + 1 rounds back to 2^24);
    # a pairwise or reversed sum would give 2. Column 1: 1, 2^24, -2^24, 1 -> sequential 1.
    big = 2.0 ** 24
    values = np.array([[big, 1.0], [1.0, big], [1.0, -big], [-big, 1.0]], np.float32).ravel()
    sums = np.array([0.5, 0.0], np.float32)
    oracle.accumulate_column_sums(values, 2, sums)
    assert sums.tolist() == [0.5, 1.0]


def test_bias_and_column_sums_are_exact_on_integers():
    rng = np.random.default_rng(3)
    rows, cols = 37, 19
    values = rng.integers(-50, 50, rows * cols).astype(np.float32)
    bias = rng.integers(-9, 9, cols).astype(np.float32)
    sums = rng.integers(-9, 9, cols).astype(np.float32)
    expected = sums.astype(np.int64) + values.reshape(rows, cols).astype(np.int64).sum(axis=0)
    oracle.accumulate_column_sums(values, cols, sums)
    assert np.array_equal(sums.astype(np.int64), expected)
    out = values.copy()
    oracle.add_row_bias(out, cols, bias)
    assert np.array_equal(out.reshape(rows, cols).astype(np.int64),
                          values.reshape(rows, cols).astype(np.int64) + bias.astype(np.int64))


def test_column_sums_error_against_f64_is_within_the_sequential_bound():
    rows, cols = 4096, 7
    values = oracle.random_values(rows * cols, 21)
    initial = np.zeros(cols, np.float32)
    sums = initial.copy()
    oracle.accumulate_column_sums(values, cols, sums)
    truth = oracle.column_sums_f64(values, cols, initial)
    bound = rows * 2.0 ** -24 * np.abs(values.reshape(rows, cols).astype(np.float64)).sum(axis=0)
    assert np.all(np.abs(sums - truth) <= bound)
    assert np.max(np.abs(sums - truth)) > 0


# ---- cross-entropy (reference.rs:139-166), its known-answer tests (:308-366) --

def _ce(logits, targets, cols, head, losses_init, grad_init):
    logits = np.asarray(logits, np.float32)
    losses = np.asarray(losses_init, np.float32).copy()
    grad = np.asarray(grad_init, np.float32).copy()
    oracle.cross_entropy(logits, np.asarray(targets, np.uint32), cols, head, losses, grad)
    return losses, grad


def test_cross_entropy_writes_losses_and_gradients_for_the_target_head():
    head = oracle.CrossEntropyHead(column_offset=0, classes=3, target_stride=1, target_offset=0, grad_scale=1.0)
    losses, grad = _ce([1, 2, 3, 0, 0, 0, 0, 0], [2, 0], 4, head, [0, 0], [7.0] * 8)
    assert losses == pytest.approx([0.407606, 1.098612], abs=1e-5)
    assert grad[:3] == pytest.approx([0.09003, 0.24473, -0.33476], abs=1e-4)
    assert grad[3] == 7.0 and grad[7] == 7.0
    assert grad[4:7] == pytest.approx([-0.666667, 0.333333, 0.333333], abs=1e-5)


def test_cross_entropy_skips_empty_targets():
    head = oracle.CrossEntropyHead(column_offset=0, classes=3, target_stride=1, target_offset=0, grad_scale=1.0)
    losses, grad = _ce([1, 2, 3, 0, 0, 0, 0, 0], [oracle.EMPTY_TOKEN, 0], 4, head, [9, 9], [7.0] * 8)
    assert losses[0] == 0.0 and grad[:3].tolist() == [0.0, 0.0, 0.0] and grad[3] == 7.0
    assert losses[1] > 0 and grad[4] < 0 < grad[5] and grad[6] > 0


def test_cross_entropy_honours_head_offsets_and_gradient_scale():
    head = oracle.CrossEntropyHead(column_offset=2, classes=2, target_stride=2, target_offset=1, grad_scale=0.5)
    losses, grad = _ce([1, 2, 3, 4, 5, 1, 2, 3, 4, 5], [0, 1, 0, 0], 5, head, [0, 0], [7.0] * 10)
    assert grad[0:2].tolist() == [7.0, 7.0] and grad[4] == 7.0 and grad[5:7].tolist() == [7.0, 7.0]
    assert grad[9] == 7.0 and np.all(losses > 0) and np.all(np.isfinite(grad[[2, 3, 7, 8]]))
    # beyond the reference's checks: row 0's target is class 1 (logits 3, 4), row 1's class 0 (3, 4)
    lp = 4 + np.log1p(np.exp(-1.0))
    assert losses == pytest.approx([lp - 4, lp - 3], rel=1e-6)
    assert grad[[2, 3]] == pytest.approx([0.5 * np.exp(3 - lp), 0.5 * (np.exp(4 - lp) - 1)], rel=1e-5)


def test_cross_entropy_gradient_rows_sum_to_zero_and_match_f64():
    rng = np.random.default_rng(5)
    rows, cols = 64, 48
    head = oracle.CrossEntropyHead(column_offset=8, classes=33, target_stride=3, target_offset=2, grad_scale=0.25)
    logits = rng.normal(0, 3, rows * cols).astype(np.float32)
    targets = rng.integers(0, 33, rows * 3).astype(np.uint32)
    losses, grad = _ce(logits, targets, cols, head, np.zeros(rows), np.zeros(rows * cols))
    z = logits.reshape(rows, cols)[:, 8:41].astype(np.float64)
    t = targets.reshape(rows, 3)[:, 2]
    lse = np.log(np.exp(z - z.max(1, keepdims=True)).sum(1)) + z.max(1)
    assert losses == pytest.approx(lse - z[np.arange(rows), t], abs=2e-5)
    g = grad.reshape(rows, cols)[:, 8:41]
    assert np.abs(g.sum(1)).max() < 1e-6
    expected = (np.exp(z - lse[:, None]) - np.eye(33)[t]) * 0.25
    assert np.abs(g - expected).max() < 1e-6


# ---- head permutes (kernels/attention.rs:77-138) ------------------------------

def test_split_and_merge_heads_follow_the_reference_layout_formula():
    # kernels_match_reference.rs:199-231: dense(2, 5, 3, 4, 3*12+2, 13).in_cache(9, 2), LCG seed 12.
    layout = oracle.HeadLayout(batch=2, time=5, heads=3, head_dim=4, width=3 * 12 + 2, column_offset=13,
                               time_capacity=9, time_offset=2)
    packed = oracle.random_values(layout.batch * layout.time * layout.width, 12)
    head_major = np.zeros(layout.batch * layout.heads * layout.time_capacity * layout.head_dim, np.float32)
    oracle.split_heads(packed, head_major, layout)
    for b in range(2):
        for h in range(3):
            for t in range(5):
                for d in range(4):
                    source = (b * 5 + t) * layout.width + 13 + h * 4 + d
                    target = ((b * 3 + h) * 9 + 2 + t) * 4 + d
                    assert head_major[target] == packed[source]
    merged = np.zeros_like(packed)
    oracle.merge_heads(head_major, merged, layout)
    columns = np.arange(packed.size) % layout.width
    inside = (columns >= 13) & (columns < 13 + 3 * 4)
    assert np.array_equal(merged, np.where(inside, packed, 0.0).astype(np.float32))


def test_split_heads_is_numpys_reshape_and_transpose():
    batch, time, heads, head_dim = 3, 7, 4, 8
    width = 3 * heads * head_dim
    packed = np.arange(batch * time * width, dtype=np.float32)
    for offset in (0, heads * head_dim, 2 * heads * head_dim):
        layout = oracle.HeadLayout(batch, time, heads, head_dim, width, offset, time, 0)
        head_major = np.zeros(batch * heads * time * head_dim, np.float32)
        oracle.split_heads(packed, head_major, layout)
        expected = packed.reshape(batch, time, 3, heads, head_dim)[:, :, offset // (heads * head_dim)]
        assert np.array_equal(head_major.reshape(batch, heads, time, head_dim), expected.transpose(0, 2, 1, 3))

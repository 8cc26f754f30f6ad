/*
 * CPU ORACLE — test infrastructure only.
 *
 * This file restates, in plain C, the CPU arithmetic the reference uses as
 * the ground truth for its GEMM path, so that the HIP kernels can be checked
 * against it. Only tests, the smoke check and the bench's cpu_baseline leg
 * may load it; the product library never links or calls it.
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 * The reference is Rust, and Rust never contracts `a * b + c` into a fused
 * multiply-add, so neither may this file: every product and every sum is
 * rounded to f32 separately, in the same order as the reference.
 *
 * Functions and the reference code each one follows:
 *   oracle_matmul            crates/staleynet-cuda/src/reference.rs:10-38
 *                            (storage handling :11-16, loop order
 *                            batch → row → col → k, f32 accumulator,
 *                            overwrite `scale*sum` / accumulate
 *                            `prev + scale*sum`), sizes/strides as built by
 *                            crates/staleynet-cuda/src/ops/matmul.rs:24-32,125-136
 *   oracle_matmul_rows       the same loops restricted to a row range
 *   oracle_matmul_elements   the same per-element computation for a list of
 *                            (batch, row, col) positions
 *   oracle_matmul_f64        the same product in f64 (error reporting only;
 *                            no reference counterpart)
 *   oracle_random_values     crates/staleynet-cuda/tests/kernels_match_reference.rs:26-38
 *   oracle_relative_error    crates/staleynet-cuda/tests/kernels_match_reference.rs:41-52
 *   oracle_causal_softmax    crates/staleynet-cuda/src/reference.rs:100-119
 *   oracle_softmax_backward  crates/staleynet-cuda/src/reference.rs:121-137
 *   oracle_add_row_bias      crates/staleynet-cuda/src/kernels/elementwise.rs:62-68
 *                            (output[r, c] += bias[c], one f32 add each)
 *   oracle_accumulate_column_sums
 *                            crates/staleynet-cuda/src/kernels/elementwise.rs:78-93
 *                            (per column: f32 sum from 0 over the rows in
 *                            order, then sums[c] += sum)
 *   oracle_column_sums_f64   the same sums in f64 (error reporting only)
 *   oracle_split_heads, oracle_merge_heads
 *                            crates/staleynet-cuda/src/kernels/attention.rs:
 *                            77-138 (HeadLayout::element, packed_index,
 *                            head_major_index; one copy per moved element)
 *   oracle_cross_entropy     crates/staleynet-cuda/src/reference.rs:139-166
 *                            (per row of one head: max, log-partition from
 *                            the f32 sum of exp(logit - max) in class order,
 *                            loss = log_partition - logit[target], gradient
 *                            (exp(logit - log_partition) - onehot) * scale;
 *                            empty targets (0xFFFFFFFF) give 0 and 0)
 *
 * Parity pins (tests/test_oracle.py): the reference's known-answer tests
 * (reference.rs:177-232, 267-306), an order-sensitive case whose f32 result
 * differs from the exact one, integer-valued inputs whose products are exact,
 * transpose/broadcast/scale/accumulate invariants, and an f64 error bound;
 * for the bias functions, the reference's own elementwise test
 * (tests/kernels_match_reference.rs:125-170) restated, exact integer cases,
 * an order-sensitive column and an f64 bound; for cross-entropy, the
 * reference's three known-answer tests (reference.rs:308-366).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

/* Element (row, col) of the logical [rows, cols] matrix op(X) stored from
 * `base` either row-major or transposed (reference.rs:11-16). */
static inline float logical(const float *values, size_t base, size_t row, size_t col, size_t rows, size_t cols,
                            int transposed) {
    return transposed ? values[base + col * rows + row] : values[base + row * cols + col];
}

/* One output element, exactly as the reference's innermost loop computes it. */
static inline float dot_in_reference_order(size_t rows, size_t cols, size_t inner, int left_t, int right_t,
                                           size_t left_base, size_t right_base, const float *left,
                                           const float *right, size_t row, size_t col) {
    float sum = 0.0f;
    for (size_t step = 0; step < inner; ++step) {
        float left_value = logical(left, left_base, row, step, rows, inner, left_t);
        float right_value = logical(right, right_base, step, col, inner, cols, right_t);
        float product = left_value * right_value;
        sum = sum + product;
    }
    return sum;
}

static inline float combine(float previous, float sum, float scale, int accumulate) {
    float scaled = scale * sum;
    return accumulate ? previous + scaled : scaled;
}

void oracle_matmul_rows(size_t rows, size_t cols, size_t inner, int left_t, int right_t, size_t count,
                        size_t batch_left, size_t batch_right, size_t batch_output, float scale, int accumulate,
                        const float *left, const float *right, float *output, size_t row_begin, size_t row_end) {
    if (row_end > rows) row_end = rows;
    for (size_t batch = 0; batch < count; ++batch) {
        for (size_t row = row_begin; row < row_end; ++row) {
            for (size_t col = 0; col < cols; ++col) {
                float sum = dot_in_reference_order(rows, cols, inner, left_t, right_t, batch * batch_left,
                                                   batch * batch_right, left, right, row, col);
                float *slot = &output[batch * batch_output + row * cols + col];
                *slot = combine(*slot, sum, scale, accumulate);
            }
        }
    }
}

void oracle_matmul(size_t rows, size_t cols, size_t inner, int left_t, int right_t, size_t count, size_t batch_left,
                   size_t batch_right, size_t batch_output, float scale, int accumulate, const float *left,
                   const float *right, float *output) {
    oracle_matmul_rows(rows, cols, inner, left_t, right_t, count, batch_left, batch_right, batch_output, scale,
                       accumulate, left, right, output, 0, rows);
}

/* Output values at `n` positions. `previous[i]` is the value the output held
 * at that position before the product (read only when accumulating). */
void oracle_matmul_elements(size_t rows, size_t cols, size_t inner, int left_t, int right_t, size_t batch_left,
                            size_t batch_right, float scale, int accumulate, const float *left, const float *right,
                            size_t n, const uint64_t *batch, const uint64_t *row, const uint64_t *col,
                            const float *previous, float *result) {
    for (size_t i = 0; i < n; ++i) {
        float sum = dot_in_reference_order(rows, cols, inner, left_t, right_t, batch[i] * batch_left,
                                           batch[i] * batch_right, left, right, row[i], col[i]);
        result[i] = combine(accumulate ? previous[i] : 0.0f, sum, scale, accumulate);
    }
}

/* The same product accumulated in f64 (the "truth" beside the f32 oracle). */
void oracle_matmul_f64(size_t rows, size_t cols, size_t inner, int left_t, int right_t, size_t batch_left,
                       size_t batch_right, double scale, int accumulate, const float *left, const float *right,
                       size_t n, const uint64_t *batch, const uint64_t *row, const uint64_t *col,
                       const float *previous, double *result) {
    for (size_t i = 0; i < n; ++i) {
        double sum = 0.0;
        for (size_t step = 0; step < inner; ++step) {
            double l = logical(left, batch[i] * batch_left, row[i], step, rows, inner, left_t);
            double r = logical(right, batch[i] * batch_right, step, col[i], inner, cols, right_t);
            sum += l * r;
        }
        result[i] = (accumulate ? (double)previous[i] : 0.0) + scale * sum;
    }
}

/* Knuth's MMIX LCG, one draw per value, mapped to [-1, 1) in steps of 2^-23. */
void oracle_random_values(size_t count, uint64_t seed, float *out) {
    const uint64_t multiplier = 6364136223846793005ull;
    const uint64_t increment = 1442695040888963407ull;
    uint64_t state = seed * multiplier + increment;
    for (size_t i = 0; i < count; ++i) {
        state = state * multiplier + increment;
        float unit = (float)(state >> 40) / (float)(1ull << 24);
        out[i] = unit * 2.0f - 1.0f;
    }
}

/* max|expected - actual| / max(|expected|, FLT_EPSILON). Like Rust's
 * f32::max, fmaxf returns the other operand when one is NaN. */
float oracle_relative_error(const float *expected, const float *actual, size_t n) {
    float magnitude = 1.1920929e-7f; /* f32::EPSILON */
    float worst = 0.0f;
    for (size_t i = 0; i < n; ++i) magnitude = fmaxf(magnitude, fabsf(expected[i]));
    for (size_t i = 0; i < n; ++i) worst = fmaxf(worst, fabsf(expected[i] - actual[i]));
    return worst / magnitude;
}

/* Causal softmax over [total_rows, keys] in place: row r of each block of
 * `queries` rows sees keys 0 ..= (r mod queries) + query_offset. */
void oracle_causal_softmax(float *scores, size_t total_rows, size_t queries, size_t keys, float scale,
                           size_t query_offset) {
    for (size_t row = 0; row < total_rows; ++row) {
        float *values = scores + row * keys;
        size_t visible = row % queries + query_offset + 1;
        if (visible > keys) visible = keys;
        float maximum = -INFINITY;
        for (size_t k = 0; k < visible; ++k) maximum = fmaxf(maximum, values[k] * scale);
        for (size_t k = 0; k < visible; ++k) values[k] = expf(values[k] * scale - maximum);
        float total = 0.0f;
        for (size_t k = 0; k < visible; ++k) total = total + values[k];
        for (size_t k = 0; k < visible; ++k) values[k] = values[k] / total;
        for (size_t k = visible; k < keys; ++k) values[k] = 0.0f;
    }
}

/* grad <- p * (grad - sum(grad * p)) per row, in place. */
void oracle_softmax_backward(const float *probabilities, float *grad, size_t rows, size_t cols) {
    for (size_t row = 0; row < rows; ++row) {
        float *g = grad + row * cols;
        const float *p = probabilities + row * cols;
        float projection = 0.0f;
        for (size_t c = 0; c < cols; ++c) projection = projection + g[c] * p[c];
        for (size_t c = 0; c < cols; ++c) g[c] = p[c] * (g[c] - projection);
    }
}

/* output[r, c] += bias[c] over a [rows, cols] row-major matrix. */
void oracle_add_row_bias(float *output, size_t rows, size_t cols, const float *bias) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) output[r * cols + c] = output[r * cols + c] + bias[c];
}

/* sums[c] += (f32 sum of input[0, c], input[1, c], ... in row order). The
 * reference runs one thread per column; walking the rows in memory order and
 * keeping one running sum per column performs the same additions in the same
 * order. `scratch` holds `cols` floats. */
void oracle_accumulate_column_sums(const float *input, size_t rows, size_t cols, float *sums, float *scratch) {
    for (size_t c = 0; c < cols; ++c) scratch[c] = 0.0f;
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) scratch[c] = scratch[c] + input[r * cols + c];
    for (size_t c = 0; c < cols; ++c) sums[c] = sums[c] + scratch[c];
}

/* The column sums (plus the initial sums) in f64. */
void oracle_column_sums_f64(const float *input, size_t rows, size_t cols, const float *initial, double *out) {
    for (size_t c = 0; c < cols; ++c) out[c] = 0.0;
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) out[c] += (double)input[r * cols + c];
    for (size_t c = 0; c < cols; ++c) out[c] += (double)initial[c];
}

/* Cross-entropy of one classifier head over `rows` rows of [rows, cols]
 * logits: its classes are columns column_offset .. +classes, its target is
 * targets[row * target_stride + target_offset]. Writes losses[row] and the
 * head's columns of grad; other columns of grad are left alone. */
void oracle_cross_entropy(const float *logits, const uint32_t *targets, size_t rows, size_t cols,
                          size_t column_offset, size_t classes, size_t target_stride, size_t target_offset,
                          float grad_scale, float *losses, float *grad) {
    for (size_t row = 0; row < rows; ++row) {
        const float *z = logits + row * cols + column_offset;
        float *g = grad + row * cols + column_offset;
        const uint32_t target = targets[row * target_stride + target_offset];
        if (target == 0xFFFFFFFFu) {
            losses[row] = 0.0f;
            for (size_t c = 0; c < classes; ++c) g[c] = 0.0f;
            continue;
        }
        float maximum = -INFINITY;
        for (size_t c = 0; c < classes; ++c) maximum = fmaxf(maximum, z[c]);
        float total = 0.0f;
        for (size_t c = 0; c < classes; ++c) total = total + expf(z[c] - maximum);
        const float log_partition = maximum + logf(total);
        losses[row] = log_partition - z[target];
        for (size_t c = 0; c < classes; ++c) {
            const float one_hot = c == target ? 1.0f : 0.0f;
            const float probability = expf(z[c] - log_partition);
            g[c] = (probability - one_hot) * grad_scale;
        }
    }
}

/* HeadLayout (kernels/attention.rs:19-43): batch, time, heads, head_dim,
 * width, column_offset, time_capacity, time_offset. Element (b, h, t, d) is
 * packed[(b * time + t) * width + column_offset + h * head_dim + d] and
 * head_major[((b * heads + h) * time_capacity + time_offset + t) * head_dim + d]. */
static inline void head_indices(const size_t *layout, size_t b, size_t h, size_t t, size_t d, size_t *packed,
                                size_t *head_major) {
    const size_t time = layout[1], heads = layout[2], head_dim = layout[3], width = layout[4];
    const size_t column_offset = layout[5], capacity = layout[6], offset = layout[7];
    *packed = (b * time + t) * width + column_offset + h * head_dim + d;
    *head_major = ((b * heads + h) * capacity + offset + t) * head_dim + d;
}

void oracle_split_heads(const float *packed, float *head_major, const size_t *layout) {
    for (size_t b = 0; b < layout[0]; ++b)
        for (size_t h = 0; h < layout[2]; ++h)
            for (size_t t = 0; t < layout[1]; ++t)
                for (size_t d = 0; d < layout[3]; ++d) {
                    size_t p, m;
                    head_indices(layout, b, h, t, d, &p, &m);
                    head_major[m] = packed[p];
                }
}

void oracle_merge_heads(const float *head_major, float *packed, const size_t *layout) {
    for (size_t b = 0; b < layout[0]; ++b)
        for (size_t h = 0; h < layout[2]; ++h)
            for (size_t t = 0; t < layout[1]; ++t)
                for (size_t d = 0; d < layout[3]; ++d) {
                    size_t p, m;
                    head_indices(layout, b, h, t, d, &p, &m);
                    packed[p] = head_major[m];
                }
}

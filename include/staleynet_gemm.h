/*
 * staleynet_gemm.h — C ABI of the MI355X (gfx950) GEMM library that stands in
 * for StaleyNET's `staleynet-cuda` GEMM entry point.
 *
 * Every product the reference's model issues goes through one call,
 *   Gpu::matmul(&self, spec: &MatmulSpec, left: &Tensor, right: &Tensor,
 *               output: &mut Tensor) -> GpuResult
 * (reference: crates/staleynet-cuda/src/ops/matmul.rs:144-171), on a `Gpu`
 * that owns one device context and one stream (crates/staleynet-cuda/src/device.rs:129-208).
 * This header exports exactly that surface with plain pointers and sizes so a
 * Rust `-sys` crate (or any C FFI) can bind it; no GPU-runtime or framework
 * types appear in any signature.
 *
 * Semantics kept from the reference:
 *   output[b] = scale * op(left[b]) * op(right[b])            (overwrite)
 *   output[b] = output[b] + scale * op(left[b]) * op(right[b]) (accumulate)
 * op(X) is X or X^T per the operand's storage; element (r, c) of logical
 * matrix b of an operand with `Transposed` storage lives at
 * b*batch_stride + c*rows + r, otherwise at b*batch_stride + r*cols + c
 * (ops/matmul.rs:24-32). The output is always row-major with row stride
 * `cols` (kernels/matmul.rs:161-163). A batch stride of 0 broadcasts one
 * matrix. Calls are asynchronous on the context's stream; errors in a kernel
 * surface at the next synchronising call.
 *
 * Status convention: 0 is success; negative values are this library's own
 * validation errors (SN_ERR_*); positive values are HIP runtime error codes
 * passed through unchanged. No function aborts the process.
 *
 * Threading: a context is not internally locked, like the reference's `Gpu`
 * (tests share it behind a mutex, tests/kernels_match_reference.rs:14-23).
 */
#ifndef STALEYNET_GEMM_H
#define STALEYNET_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------- */
#define SN_OK 0
/* A required pointer argument was null (a null operand is allowed only when
 * the spec needs zero elements of it). */
#define SN_ERR_NULL_ARGUMENT (-1)
/* "matmul: left operand too small" (ops/matmul.rs:147). */
#define SN_ERR_LEFT_TOO_SMALL (-2)
/* "matmul: right operand too small" (ops/matmul.rs:148). */
#define SN_ERR_RIGHT_TOO_SMALL (-3)
/* "matmul: output too small" (ops/matmul.rs:149). */
#define SN_ERR_OUTPUT_TOO_SMALL (-4)
/* batch_count == 0: the reference's `required_len` underflows
 * (ops/matmul.rs:139-141) and panics; here it is reported instead. */
#define SN_ERR_EMPTY_BATCH (-5)
/* A size or index computation does not fit in 64 bits, or a dimension is too
 * large for the kernels' 32-bit tile counters. */
#define SN_ERR_OVERFLOW (-6)
/* An enum field holds an unknown value, or the combination is not supported
 * (for example a causal mask on a non-square-compatible product). */
#define SN_ERR_UNSUPPORTED (-7)
/* The output overlaps an input. The reference's borrow rules make this
 * impossible (`&mut Tensor` vs `&Tensor`); a C caller must be told. */
#define SN_ERR_ALIASING (-8)
/* No usable GPU at the requested ordinal. */
#define SN_ERR_NO_DEVICE (-9)
/* The context's split-K workspace cannot hold the partial sums this product
 * needs (only possible with a workspace smaller than the default). */
#define SN_ERR_WORKSPACE (-10)
/* A bias or column-sum vector whose length is not the matrix's column count:
 * "add_row_bias: bias length must equal output columns" and
 * "accumulate_column_sums: sums length must equal input columns"
 * (ops/elementwise.rs:33, :46). */
#define SN_ERR_LENGTH_MISMATCH (-11)
/* A row-wise kernel's shapes disagree: "causal_softmax: rows must be a
 * multiple of queries" (ops/attention.rs:59) or "softmax_backward: shape
 * mismatch" (ops/attention.rs:79). */
#define SN_ERR_SHAPE (-12)

/* ---- enums (carried as uint32_t in structs) ------------------------------ */
/* Storage (ops/matmul.rs:15-22). */
#define SN_ROW_MAJOR 0u
#define SN_TRANSPOSED 1u
/* WriteMode and its kernel flag (ops/mod.rs:253-269). */
#define SN_OVERWRITE 0u
#define SN_ACCUMULATE 1u
/* Causal masks: an extension with no reference counterpart; 0 keeps the
 * reference's dense behaviour. A causal [query, key] matrix has its element
 * (q, k) visible iff k <= q + query_offset, the rule of the reference's
 * causal_softmax (kernels/attention.rs:160), with q counted within each
 * matrix of the batch.
 *   SN_MASK_CAUSAL_OUTPUT: the output is such a matrix (scores S = Q K^T and
 *     dP = dO V^T, attention.rs:206-209, 239-242). Masked outputs are not
 *     computed; they are written as 0 when overwriting and left unchanged
 *     when accumulating (the product is treated as 0 there).
 *   SN_MASK_CAUSAL_LEFT: the left operand, as stored, is such a matrix
 *     (P or dS, attention.rs:212-213, 244-260) and is treated as 0 where
 *     masked; whole masked tiles of the inner dimension are skipped. With
 *     Transposed storage op(left) = P^T, so the mask applies to (k, r). */
#define SN_MASK_NONE 0u
#define SN_MASK_CAUSAL_OUTPUT 1u
#define SN_MASK_CAUSAL_LEFT 2u
/* Per-call precision override; DEFAULT uses the context's kernel choice. */
#define SN_PRECISION_DEFAULT 0u
#define SN_PRECISION_F32 1u
#define SN_PRECISION_BF16 2u
/* Kernel selection, the role of the reference's MatmulKernel
 * (device.rs:38-67; public field Gpu::matmul_kernel, device.rs:144):
 *   SN_KERNEL_MFMA_F32  fp32 matrix-core GEMM (default; the role of Blocked)
 *   SN_KERNEL_MFMA_BF16 inputs rounded to bf16 (nearest-even), fp32
 *                       accumulation (the role of TensorCore's TF32)
 *   SN_KERNEL_SIMPLE    one thread per output, k summed in order with
 *                       separately rounded products (the role of Naive);
 *                       a slow cross-check, bit-identical to the reference's
 *                       CPU loop. */
#define SN_KERNEL_MFMA_F32 0u
#define SN_KERNEL_MFMA_BF16 1u
#define SN_KERNEL_SIMPLE 2u

/* MatmulSpec (ops/matmul.rs:56-82) field for field, plus the extensions
 * `mask`, `query_offset` and `precision` (zero = reference behaviour).
 * Fill it with sn_matmul_spec_new() and adjust fields, as the reference's
 * builders do (MatmulSpec::new + left_transposed/right_transposed/
 * accumulate/scaled/batched, ops/matmul.rs:84-122). */
typedef struct sn_matmul_spec {
    size_t rows;          /* rows of op(left) and of the output */
    size_t cols;          /* columns of op(right) and of the output */
    size_t inner;         /* columns of op(left) = rows of op(right) */
    uint32_t left_storage;  /* SN_ROW_MAJOR or SN_TRANSPOSED */
    uint32_t right_storage; /* SN_ROW_MAJOR or SN_TRANSPOSED */
    size_t batch_count;   /* BatchStrides::count */
    size_t batch_left;    /* elements between consecutive left matrices (0 broadcasts) */
    size_t batch_right;   /* elements between consecutive right matrices (0 broadcasts) */
    size_t batch_output;  /* elements between consecutive outputs */
    float scale;          /* multiplier applied to the product */
    uint32_t write;       /* SN_OVERWRITE or SN_ACCUMULATE */
    uint32_t mask;        /* SN_MASK_* (extension) */
    uint32_t precision;   /* SN_PRECISION_* (extension) */
    size_t query_offset;  /* positions cached before query 0 (extension, masks only) */
} sn_matmul_spec;

typedef struct sn_context sn_context;

/* `MatmulSpec::new(rows, cols, inner)`: row-major operands, unbatched
 * (BatchStrides::SINGLE), overwrite, scale 1 (ops/matmul.rs:86-97). */
sn_matmul_spec sn_matmul_spec_new(size_t rows, size_t cols, size_t inner);

/* `Gpu::new(ordinal)` (device.rs:148-155): selects the device, creates one
 * stream and a workspace of the default size (1.5 GiB: split-K partial
 * sums, and the bf16 products' operands staged as bf16; every product of
 * the reference's model configurations fits in it). */
int sn_context_create(int ordinal, sn_context **out);
/* The same with an explicit workspace size in bytes (0 disables split-K and
 * bf16 staging; a product that does not fit takes a path that needs less). */
int sn_context_create_with_workspace(int ordinal, size_t workspace_bytes, sn_context **out);
int sn_context_destroy(sn_context *context);
/* `Gpu::bind_to_current_thread` (device.rs:157-161): makes the context's
 * device current on the calling thread. */
int sn_context_bind(sn_context *context);
/* `gpu.matmul_kernel = kernel` / read it back (device.rs:144). */
int sn_context_set_kernel(sn_context *context, uint32_t kernel);
int sn_context_get_kernel(const sn_context *context, uint32_t *kernel);
/* The context's stream as an opaque handle (a hipStream_t), for callers
 * that time work with events on the stream it runs on. */
void *sn_context_stream(sn_context *context);
/* `MatmulKernel::tolerance` (device.rs:56-66): the largest relative error,
 * in the reference test's metric, that the kernel's arithmetic allows
 * against the reference's f32 product (1e-5 f32, 2e-2 bf16 inputs);
 * NaN for an unknown kernel. */
float sn_kernel_tolerance(uint32_t kernel);

/* ---- buffers (device.rs:163-192) ----------------------------------------- */
/* `Gpu::synchronize`: blocks until all queued work has finished. */
int sn_synchronize(sn_context *context);
/* `Gpu::zeros`: a zero-filled device buffer of `count` floats. */
int sn_alloc_zeroed(sn_context *context, size_t count, float **out);
/* Releases a buffer from sn_alloc_zeroed / sn_upload. */
int sn_free(sn_context *context, float *buffer);
/* `Gpu::upload`: a new device buffer holding `count` host floats. */
int sn_upload(sn_context *context, const float *host, size_t count, float **out);
/* `Gpu::download`: copies `count` floats back to the host (synchronising). */
int sn_download(sn_context *context, const float *device, size_t count, float *host);
/* `Gpu::copy_from_host`: overwrites an existing buffer (synchronising). */
int sn_copy_from_host(sn_context *context, float *device, const float *host, size_t count);
/* `Gpu::fill_zero`: zeroes `count` floats in stream order. */
int sn_fill_zero(sn_context *context, float *device, size_t count);

/* ---- the GEMM ------------------------------------------------------------ */
/* The host-side checks of `Gpu::matmul` (ops/matmul.rs:147-149) as a pure
 * function: returns SN_OK or the SN_ERR_* code the call would return. The
 * lengths are element counts of the buffers passed for each operand. */
int sn_matmul_validate(const sn_matmul_spec *spec, size_t left_len, size_t right_len, size_t output_len);

/* `Gpu::matmul` (ops/matmul.rs:146-171): validates, then enqueues the
 * product on the context's stream and returns without waiting. Nothing is
 * allocated. A spec with rows or cols of 0 writes nothing; inner = 0 writes
 * scale*0 (overwrite) or leaves the output (accumulate), as the reference's
 * loops do. */
int sn_matmul(sn_context *context, const sn_matmul_spec *spec, const float *left, size_t left_len,
              const float *right, size_t right_len, float *output, size_t output_len);

/* ---- the Linear layer's bias kernels on either side of the GEMM ----------- */
/* `Gpu::add_row_bias` (ops/elementwise.rs:30-41; kernel kernels/elementwise.rs:
 * 62-68), called by Linear::forward after its product (layers/linear.rs:47):
 * output[r, c] += bias[c] over the [rows, cols] row-major output, one f32 add
 * per element (bit-identical to the reference). bias_len must equal cols
 * (SN_ERR_LENGTH_MISMATCH); bias must not overlap the output
 * (SN_ERR_ALIASING). Asynchronous on the context's stream. */
int sn_add_row_bias(sn_context *context, float *output, size_t rows, size_t cols, const float *bias,
                    size_t bias_len);

/* `Gpu::accumulate_column_sums` (ops/elementwise.rs:43-58; kernel
 * kernels/elementwise.rs:78-93), called by Linear::backward for the bias
 * gradient (layers/linear.rs:59): sums[c] += sum over r of input[r, c] for
 * the [rows, cols] row-major input. The reference sums each column in row
 * order with one thread per column; here a workgroup owns 64 columns and a
 * slice of rows, slices are added in a fixed order and the result is the same
 * on every run (not bit-identical to the row-order sum; within the fp32
 * tolerance of it). sums_len must equal cols (SN_ERR_LENGTH_MISMATCH).
 * Uses the context's split-K workspace for the per-slice sums. */
int sn_accumulate_column_sums(sn_context *context, const float *input, size_t rows, size_t cols, float *sums,
                              size_t sums_len);

/* Linear::forward's two calls (layers/linear.rs:46-47), `Gpu::matmul`
 * followed by `Gpu::add_row_bias` on its output, in one pass: the bias is
 * added in the product's epilogue, after the reference's combine and rounded
 * separately, so the result is the same as the two calls'. For a batched spec
 * the bias is added to every output matrix, which must not share memory
 * (batch_output >= rows * cols, else SN_ERR_UNSUPPORTED). bias_len must equal
 * spec->cols (SN_ERR_LENGTH_MISMATCH).
 * Saves the separate read and write of the output; a masked spec is run as
 * the two calls. */
int sn_matmul_bias(sn_context *context, const sn_matmul_spec *spec, const float *left, size_t left_len,
                   const float *right, size_t right_len, const float *bias, size_t bias_len, float *output,
                   size_t output_len);

/* Linear::backward's weight and bias gradients (layers/linear.rs:54-59),
 * `Gpu::matmul` with the weight-gradient spec followed by
 * `Gpu::accumulate_column_sums` on the same output gradient, in one call:
 * the product as sn_matmul computes it, and sums[c] += the sum over k of
 * right[k, c]. No single reference call corresponds; it replaces those two.
 * The right operand must be stored row-major ([inner, cols], spec->right ==
 * SN_ROW_MAJOR) and the spec unbatched (SN_ERR_UNSUPPORTED otherwise);
 * sums_len must equal spec->cols (SN_ERR_LENGTH_MISMATCH); sums must not
 * overlap the output or the operands (SN_ERR_ALIASING). fp32 products the
 * direct-to-LDS kernel serves add the column sums while the right operand's
 * tiles pass through LDS, and bf16 products the 256 x 256 kernel serves while
 * its fp32 values pass through the registers before rounding: the first tile
 * row of each K slice sums them (or, where the right operand is the one
 * staged as bf16, the staging pass sums each 64 k as it reads them), in a
 * fixed order, the same on every run, within the fp32 tolerance of the
 * row-order sum. That saves a second read of the right operand; other
 * products run as the two calls. The product's bits are sn_matmul's either
 * way. */
int sn_matmul_column_sums(sn_context *context, const sn_matmul_spec *spec, const float *left, size_t left_len,
                          const float *right, size_t right_len, float *output, size_t output_len, float *sums,
                          size_t sums_len);

/* ---- the row-wise kernels between the attention products ------------------ */
/* `Gpu::causal_softmax` (ops/attention.rs:56-74; kernel kernels/attention.rs:
 * 140-183), in place on the [rows, keys] scores, called between S = Q K^T and
 * O = P V (layers/attention.rs:210): row r of each block of `queries` rows
 * sees keys 0 ..= (r mod queries) + query_offset, which become
 * exp(s * scale - max) / sum over the visible keys; the other keys become 0.
 * rows must be a multiple of queries (SN_ERR_SHAPE). Summation order differs
 * from the reference's, so results are within the fp32 tolerance. */
int sn_causal_softmax(sn_context *context, float *scores, size_t rows, size_t keys, size_t queries, float scale,
                      size_t query_offset);

/* `Gpu::softmax_backward` (ops/attention.rs:76-92; kernel kernels/attention.rs:
 * 185-207), in place on the gradient (layers/attention.rs:249):
 * grad <- p * (grad - sum(grad * p)) per row. The two shapes must be equal
 * (SN_ERR_SHAPE); grad must not overlap probabilities (SN_ERR_ALIASING). */
int sn_softmax_backward(sn_context *context, const float *probabilities, size_t probability_rows,
                        size_t probability_cols, float *grad, size_t grad_rows, size_t grad_cols);

/* `HeadLayout` (kernels/attention.rs:19-43): where a group of attention heads
 * lives in the packed [batch * time, width] layout (head h of a row at columns
 * column_offset + h * head_dim ..) and in the head-major [batch, heads,
 * time_capacity, head_dim] layout (time steps written or read from
 * time_offset on, which appends to a key/value cache). */
typedef struct sn_head_layout {
    size_t batch;
    size_t time;
    size_t heads;
    size_t head_dim;
    size_t width;
    size_t column_offset;
    size_t time_capacity;
    size_t time_offset;
} sn_head_layout;

/* `Gpu::split_heads` / `Gpu::merge_heads` (ops/attention.rs:20-52; kernels
 * at kernels/attention.rs:113-138): packed columns -> head-major, and back (the
 * other packed columns are left alone). Bit-exact copies. The reference's
 * checks (ops/attention.rs:11-18) become SN_ERR_SHAPE ("HeadLayout: time range
 * exceeds capacity"; here also heads that run past a packed row) and
 * SN_ERR_LENGTH_MISMATCH ("HeadLayout: packed tensor too small", "HeadLayout:
 * head-major tensor too small"). */
int sn_split_heads(sn_context *context, const float *packed, size_t packed_len, float *head_major,
                   size_t head_major_len, const sn_head_layout *layout);
int sn_merge_heads(sn_context *context, const float *head_major, size_t head_major_len, float *packed,
                   size_t packed_len, const sn_head_layout *layout);

/* ---- fused causal attention forward --------------------------------------- */
/* Where the attention matrices are: `heads` (batch x heads) matrices; Q
 * [heads][queries][head_dim] with q_stride floats between heads, K and V
 * [heads][keys][head_dim] with kv_stride between heads (a key/value cache
 * of capacity `keys`), rows head_dim floats apart; query q of a head sees
 * keys 0 ..= q + query_offset. */
typedef struct sn_attention_shape {
    size_t heads;
    size_t queries;
    size_t keys;
    size_t head_dim;
    size_t q_stride;
    size_t kv_stride;
    size_t query_offset;
    float scale;
} sn_attention_shape;

/* Fused causal attention forward. It has no counterpart in the reference's
 * Gpu API: it computes in one launch what CausalSelfAttention::forward
 * (crates/staleynet-model/src/layers/attention.rs:206-213) computes with
 * three calls, the scores product (MatmulSpec::new(queries, keys, h)
 * .right_transposed(), batched over the heads), Gpu::causal_softmax(scores,
 * queries, scale, query_offset) and the mix product (MatmulSpec::new(
 * queries, h, keys)), without writing the scores. out: O [heads][queries]
 * [head_dim]. probabilities (may be null): the [heads][queries][keys]
 * matrix causal_softmax leaves, 0 past the diagonal, for the backward.
 * head_dim 32, 64 or 128 and 16-byte aligned buffers and strides
 * (SN_ERR_UNSUPPORTED; strides may overlap heads, 0 shares one K and V);
 * keys >= 1 (SN_ERR_SHAPE); buffers too small for the shape
 * (SN_ERR_LENGTH_MISMATCH);
 * out or probabilities overlapping an input or each other (SN_ERR_ALIASING).
 * Within the fp32 tolerance of the three calls. With at most 4 queries per
 * head and no probabilities (a decode step against the cache,
 * attention.rs:274-320), the keys are split over workgroups whose partial
 * results are merged in a fixed order through the context's workspace and
 * arrival counters, so calls on one context must not overlap (as for
 * sn_matmul's split products); deterministic. */
int sn_causal_attention(sn_context *context, const sn_attention_shape *shape, const float *q, size_t q_len,
                        const float *k, size_t k_len, const float *v, size_t v_len, float *out, size_t out_len,
                        float *probabilities, size_t probabilities_len);

/* The probability gradient of that attention, fused. It has no counterpart in
 * the reference's Gpu API: it computes in one launch what
 * CausalSelfAttention::backward (crates/staleynet-model/src/layers/
 * attention.rs:238-248) computes with the dP product (MatmulSpec::new(
 * queries, keys, h).right_transposed(): dP = dO V^T, batched over the heads)
 * and Gpu::softmax_backward(probabilities, dP), without writing dP: grad =
 * P * (dP - D) with D per query = sum over h of dO * O (equal to the
 * softmax's projection sum over keys of dP * P, since O = P V). d_out: dO
 * [heads][queries][head_dim], q_stride apart per head; v as in
 * sn_causal_attention; out: the forward's O, dense; probabilities: P as
 * causal_softmax leaves it (0 past the diagonal); grad: dS, same layout as
 * P, 0 past the diagonal. q_grad (may be null; then k may be null too): the
 * backward's next call as well, dQ = shape->scale * dS K (attention.rs:
 * 250-253, MatmulSpec::new(queries, h, keys).scaled(scale)), [heads]
 * [queries][head_dim], with k laid out as v. The same checks and codes as
 * sn_causal_attention; grad and q_grad must not overlap an input or each
 * other. Within the fp32 tolerance of the calls it replaces. */
int sn_causal_attention_score_grad(sn_context *context, const sn_attention_shape *shape, const float *d_out,
                                   size_t d_out_len, const float *v, size_t v_len, const float *out, size_t out_len,
                                   const float *probabilities, size_t probabilities_len, float *grad,
                                   size_t grad_len, const float *k, size_t k_len, float *q_grad, size_t q_grad_len);

/* ---- training attention without the probabilities in memory -------------- */
/* sn_causal_attention's forward for training without P: O, and per query
 * the softmax statistics the backward below rebuilds P from: stats[head]
 * [query] = {m, l}, m the largest of the query's scaled visible scores and l
 * the sum of e^(x - m) over them (2 floats per query, 8-byte aligned). No
 * counterpart in the reference, whose forward keeps P (attention.rs:
 * 206-213). The same checks and codes as sn_causal_attention; stats must not
 * overlap another buffer. */
int sn_causal_attention_with_stats(sn_context *context, const sn_attention_shape *shape, const float *q,
                                   size_t q_len, const float *k, size_t k_len, const float *v, size_t v_len,
                                   float *out, size_t out_len, float *stats, size_t stats_len);

/* The attention backward from the forward's output and statistics instead
 * of its probabilities: what CausalSelfAttention::backward (crates/
 * staleynet-model/src/layers/attention.rs:238-260) computes with the dP and
 * dV products, softmax_backward and the dQ and dK products, without any
 * [queries, keys] matrix in memory. q, k, v as for sn_causal_attention;
 * out: the forward's O [heads][queries][head_dim], dense; d_out: dO, laid
 * out as q (q_stride apart per head); stats: the forward's
 * sn_causal_attention_with_stats statistics. Writes q_grad = scale * dS K
 * [heads][queries][head_dim], k_grad = scale * dS^T Q and v_grad = P^T dO
 * [heads][keys][head_dim], all dense, with dS = P * (dO V^T - D) and D per
 * query = sum over h of dO * O (softmax_backward's projection, since O =
 * P V). Within the fp32 tolerance of the reference's calls; deterministic
 * (no atomics). Needs 12 bytes of the context's workspace per query
 * (SN_ERR_WORKSPACE). For head dims 32 and 64 it also keeps dQ's partial
 * sums per 128-key block there when they fit (256 or 128 bytes per query
 * and block whose keys the query's 64-query stage reaches: 855 MB at 192
 * heads of 2048), for all heads or in runs of heads, and then skips the
 * second recomputation of S and dP; the two ways sum dQ in different orders,
 * so its bits depend on the workspace size (dK and dV's do not). The same
 * shape codes as sn_causal_attention; an output overlapping an input or
 * another output is SN_ERR_ALIASING. */
int sn_causal_attention_backward(sn_context *context, const sn_attention_shape *shape, const float *q, size_t q_len,
                                 const float *k, size_t k_len, const float *v, size_t v_len, const float *out,
                                 size_t out_len, const float *d_out, size_t d_out_len, const float *stats,
                                 size_t stats_len, float *q_grad, size_t q_grad_len, float *k_grad,
                                 size_t k_grad_len, float *v_grad, size_t v_grad_len);

/* ---- the head's consumer: per-codebook softmax cross-entropy ------------- */
/* An empty target slot (crates/staleynet-cuda/src/kernels/mod.rs:46). */
#define SN_EMPTY_TOKEN 0xFFFFFFFFu

/* `CrossEntropyHead` (crates/staleynet-cuda/src/ops/loss.rs:14-30): which
 * columns of a logits row and which target of a target row one classifier
 * owns. */
typedef struct sn_cross_entropy_head {
    size_t column_offset;
    size_t classes;
    size_t target_stride;
    size_t target_offset;
    float grad_scale;
} sn_cross_entropy_head;

/* `Gpu::cross_entropy` (ops/loss.rs:34-71; kernel kernels/loss.rs:54-97),
 * called once per codebook on the head's logits (training.rs:208-239): for
 * each row, loss = log_partition - logit[target] and, in the head's columns
 * of logits_grad, (softmax - onehot) * grad_scale; an empty target gives 0
 * and 0, a target outside the head a NaN loss. The reference's asserts
 * become SN_ERR_SHAPE (gradient shape differs from the logits' "cross_entropy:
 * gradient shape"; head past the row "cross_entropy: head exceeds logits") and
 * SN_ERR_LENGTH_MISMATCH ("cross_entropy: losses too small", "cross_entropy:
 * too few targets"). targets are device memory (sn_upload_tokens). */
int sn_cross_entropy(sn_context *context, const float *logits, size_t rows, size_t cols, const uint32_t *targets,
                     size_t targets_len, const sn_cross_entropy_head *head, float *losses, size_t losses_len,
                     float *logits_grad, size_t grad_rows, size_t grad_cols);

/* Token id buffers in device memory (`Gpu::upload_tokens`, `download_tokens`,
 * device.rs:194-208). */
int sn_upload_tokens(sn_context *context, const uint32_t *host, size_t count, uint32_t **out);
int sn_download_tokens(sn_context *context, const uint32_t *device, size_t count, uint32_t *host);
int sn_free_tokens(sn_context *context, uint32_t *buffer);

/* ---- the allocation-free variant ------------------------------------------ */
/* The most scratch sn_matmul_noalloc's kernels use for split-K partial sums
 * (and bf16 staged operands); 64 KiB of arrival counters and 4 MiB of
 * few-row hand-off slots come on top. */
#define SN_NOALLOC_WORKSPACE_BYTES ((size_t)64 << 20)

/* sn_matmul without a context and without allocating anything. It has no
 * counterpart in the reference; it is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc. The product runs on the calling thread's
 * current device, on `stream` (a hipStream_t; null is the default stream),
 * with the kernel the spec's precision names (default and F32: fp32 matrix
 * cores; BF16: bf16 inputs). Its scratch is a device array of the
 * library's, one per device, held from the library's load until the process
 * ends: 64 KiB of arrival counters and 4 MiB of hand-off slots (zero from
 * the load; each kernel resets what it touched) and
 * SN_NOALLOC_WORKSPACE_BYTES for partial sums. The first
 * call on a device only looks up that array's address and enqueues nothing
 * else, so it may itself be under stream capture. A product that would need
 * more partial sums than that splits K into fewer slices (within the fp32
 * tolerance of sn_matmul's result; bit-identical when both plans agree);
 * one that cannot fit returns SN_ERR_WORKSPACE. The same checks and codes as
 * sn_matmul. Calls that overlap on one device (other streams or threads)
 * share the array and race. */
int sn_matmul_noalloc(const sn_matmul_spec *spec, const float *left, size_t left_len, const float *right,
                      size_t right_len, float *output, size_t output_len, void *stream);

/* ---- launch geometry (host only) ------------------------------------------ */
/* The kernel family a product runs on, as sn_plan_matmul reports it. */
#define SN_PATH_NONE 0u            /* rows or cols of 0: nothing is launched */
#define SN_PATH_REFERENCE_ORDER 1u /* SN_KERNEL_SIMPLE: one thread per output */
#define SN_PATH_FEW_ROWS 2u        /* decode GEMV: at most 16 rows, right operand row-major */
#define SN_PATH_FEW_ROWS_NT 3u     /* at most 4 rows against a right operand stored [cols][inner] */
#define SN_PATH_F32_DIRECT 4u      /* fp32 tiles, operands loaded straight into LDS */
#define SN_PATH_F32_REGISTER 5u    /* fp32 tiles, operands staged through registers (unaligned) */
#define SN_PATH_BF16_STAGED 6u     /* bf16: both operands first rounded into the workspace */
#define SN_PATH_BF16_DIRECT 7u     /* bf16: fp32 LDS stages rounded per fragment */
#define SN_PATH_BF16_REGISTER 8u   /* bf16: register-staged (unaligned) operands */
#define SN_PATH_BF16_WIDE 9u       /* bf16: 256x256 tiles rounding fp32 operands as they load */
#define SN_PATH_F32_DIRECT_SUMS 10u /* SN_PATH_F32_DIRECT adding the right operand's column sums */
#define SN_PATH_BF16_WIDE_SUMS 11u  /* SN_PATH_BF16_WIDE adding the right operand's column sums */
#define SN_PATH_F32_PERSISTENT 12u  /* SN_PATH_F32_DIRECT's 128x128 tiles, looped over by persistent_grid workgroups */

/* How one product is launched: the role of the reference's launch geometry
 * (`launch::matmul_tiles` / `matmul_blocks`, crates/staleynet-cuda/src/
 * launch.rs:28-48), for this library's kernels. A launch holds
 * `batches_per_launch` matrices of the batch; each matrix is split into
 * `splits` slices of `k_per_split` inner elements and tiles_m x tiles_n
 * output tiles of tile_rows x tile_cols (for the few-row paths: tiles_n
 * column blocks, or blocks of rows of the right operand, and tiles_m = 1).
 * A tiled launch's workgroup w covers the (matrix, slice, tile) that
 * sn_tile_map gives for it. */
typedef struct sn_launch_plan {
    uint32_t path;                /* SN_PATH_* */
    uint32_t threads;             /* threads per workgroup */
    uint32_t tile_rows, tile_cols;
    uint32_t tiles_m, tiles_n;
    uint32_t splits;
    uint32_t persistent_grid;     /* nonzero for a persistent launch (SN_PATH_F32_PERSISTENT always,
                                   * SN_PATH_BF16_WIDE(_SUMS) when its tiles allow): the workgroups
                                   * launched, workgroup g taking work items g, g + persistent_grid, ...
                                   * of the `workgroups`; otherwise 0 */
    uint64_t k_per_split;
    uint64_t batches_per_launch;
    uint64_t workgroups;          /* of one launch holding batches_per_launch matrices (persistent
                                   * path: its work items, one per workgroup of the other paths) */
    uint64_t launches;            /* kernel launches of the product (split-K reduce not counted) */
    uint64_t workspace_bytes;     /* split-K partial sums and staged operands */
} sn_launch_plan;

/* The plan sn_matmul would follow for `spec` with context kernel `kernel`
 * (SN_KERNEL_*) on a device of `cu_count` compute units whose context has a
 * workspace of `workspace_bytes`: pure host code, no device needed. The
 * operand addresses are only inspected for alignment (a path may need
 * 16-byte aligned operands); they are never dereferenced. Returns the
 * status sn_matmul_validate would, with every operand length taken as
 * sufficient; SN_ERR_WORKSPACE when the product would not fit. */
int sn_plan_matmul(const sn_matmul_spec *spec, uint32_t kernel, const float *left, const float *right,
                   const float *output, uint32_t cu_count, size_t workspace_bytes, sn_launch_plan *plan);
/* The same for sn_matmul_column_sums: path SN_PATH_F32_DIRECT_SUMS or
 * SN_PATH_BF16_WIDE_SUMS when the column sums are fused into the product (the
 * workspace then holds N more floats per K slice), else the product's plan
 * with the workspace the larger of the product's and
 * sn_accumulate_column_sums'. SN_ERR_UNSUPPORTED for what
 * sn_matmul_column_sums rejects as unsupported. */
int sn_plan_matmul_column_sums(const sn_matmul_spec *spec, uint32_t kernel, const float *left, const float *right,
                               const float *output, uint32_t cu_count, size_t workspace_bytes,
                               sn_launch_plan *plan);

/* The tiled kernels' map from workgroup id to (matrix of the launch, K
 * slice, tile row, tile column), for workgroups 0 .. workgroups - 1 of a
 * launch of `workgroups` over tiles_m x tiles_n tiles and `splits` slices
 * per matrix: the same function the kernels evaluate on the device. Ids are
 * regrouped so that each of the 8 XCDs (which receive workgroups
 * round-robin) holds a contiguous range. Each output array holds
 * `workgroups` entries. SN_ERR_NULL_ARGUMENT or SN_ERR_OVERFLOW (more than
 * 2^31 workgroups, or a zero count). */
int sn_tile_map(uint32_t workgroups, uint32_t tiles_m, uint32_t tiles_n, uint32_t splits, uint32_t *matrix,
                uint32_t *slice, uint32_t *tile_row, uint32_t *tile_col);

/* A short English description of a status code (never null). */
const char *sn_status_string(int status);

#ifdef __cplusplus
}
#endif

#endif /* STALEYNET_GEMM_H */

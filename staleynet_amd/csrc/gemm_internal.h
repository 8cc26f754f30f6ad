// Internal interface between the C-ABI layer (context.cpp) and the kernels.
// Not installed; the public surface is include/staleynet_gemm.h.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

#include "staleynet_gemm.h"

namespace sn {

// One (batched) product in the kernels' terms. "K-contiguous" means element
// (row, k) of the operand is at base[row * ld + k]; otherwise it is at
// base[k * ld + row]. For the left operand "row" is an output row (M), for
// the right operand an output column (N).
struct Problem {
    const float* a = nullptr;
    const float* b = nullptr;
    float* c = nullptr;
    int64_t m = 0, n = 0, k = 0;
    bool a_k_contiguous = true;  // left stored row-major
    bool b_k_contiguous = false; // right stored transposed
    int64_t lda = 0, ldb = 0;    // stride of the non-contiguous index
    int64_t batch = 1;
    int64_t stride_a = 0, stride_b = 0, stride_c = 0;
    float scale = 1.0f;
    bool accumulate = false;
    uint32_t mask = 0;           // SN_MASK_*
    int64_t query_offset = 0;
    // Linear's bias, fused: output[.., r, c] += bias[c] after the combine,
    // rounded separately. Only for unmasked products (the C entry point runs
    // a masked one as the product and then the bias kernel).
    const float* bias = nullptr;
    // Linear's bias gradient, fused into the weight-gradient product: sums
    // [c] += the sum over K of the right operand's column c (stored row-major
    // [K][N]). Only for the fp32 direct-to-LDS kernel, batch 1, unmasked.
    float* column_sums = nullptr;
};

// What a launch may use beyond its operands: the context's split-K scratch,
// its arrival counters (zero between calls; a kernel that increments one
// resets it before it ends), the decode kernel's hand-off slots (zero
// between calls; the kernel that fills a slot clears it before it ends) and
// the device's compute-unit count.
struct Env {
    float* workspace = nullptr;
    size_t workspace_bytes = 0;
    uint32_t* counters = nullptr;
    size_t counter_count = 0;
    uint32_t* handoff = nullptr;
    size_t handoff_words = 0;
    int cu_count = 256;
};

// Words of hand-off slots a context (and the allocation-free scratch)
// holds: 4 MiB, above the most any few-row plan needs (its slices number at
// most about 448 over all column blocks, each M x 64 words, M <= 16).
constexpr size_t kHandoffWords = size_t(1) << 20;

// How a product is launched (sn_launch_plan's fields): the kernel family,
// its tiles, K slices and grid. Each launcher below computes its grid with
// the describe_* function of its family, so the two cannot disagree.
struct LaunchShape {
    uint32_t path = 0;  // SN_PATH_*
    uint32_t threads = 0;
    int32_t tile_m = 0, tile_n = 0;
    int32_t tiles_m = 0, tiles_n = 0, splits = 1;
    int64_t k_per_split = 0;
    int64_t batches_per_launch = 0;
    int64_t workgroups = 0;
    int64_t launches = 0;
    size_t workspace_bytes = 0;
    int64_t persistent_grid = 0;  // SN_PATH_F32_PERSISTENT: workgroups launched, looping over `workgroups` items
};
LaunchShape describe_gemm_f32(const Problem& p, const Env& env);
LaunchShape describe_gemm_bf16(const Problem& p, const Env& env);
LaunchShape describe_gemm_simple(const Problem& p);
LaunchShape describe_gemv(const Problem& p);
LaunchShape describe_gemv_nt(const Problem& p);

// sn_matmul's host side (context.cpp): the checks of a call (the reference's
// asserts, null operands, an output overlapping an input), the kernels'
// description of a checked spec with `bias` (null: none) fused unless the
// product is masked, and the kernel a call runs (the context's choice,
// overridden by the spec's precision).
int check_matmul_call(const sn_matmul_spec* spec, const float* left, size_t left_len, const float* right,
                      size_t right_len, const float* bias, size_t bias_len, const float* output, size_t output_len);
Problem problem_of(const sn_matmul_spec* spec, const float* left, const float* right, float* output,
                   const float* bias);
uint32_t kernel_for(uint32_t context_kernel, uint32_t precision);

// The routing of sn_matmul: which family serves `p` under context kernel
// `kernel` (SN_KERNEL_*), and that family's launch.
LaunchShape describe_matmul(const Problem& p, uint32_t kernel, const Env& env);
hipError_t launch_matmul(const Problem& p, uint32_t kernel, const Env& env, hipStream_t stream);

// Launchers; each returns hipSuccess or the launch error.
hipError_t launch_gemm_f32(const Problem& p, const Env& env, hipStream_t stream);
hipError_t launch_gemm_bf16(const Problem& p, const Env& env, hipStream_t stream);
hipError_t launch_gemm_simple(const Problem& p, hipStream_t stream);
// Decode-shaped products (few rows, right operand N-contiguous); returns
// hipErrorNotSupported when the shape is not one it handles.
hipError_t launch_gemv(const Problem& p, const Env& env, hipStream_t stream);
bool gemv_applies(const Problem& p, const Env& env);
// Products of at most 4 rows against a right operand stored [n][k] (the
// decode step's scores against the cache); hipErrorNotSupported otherwise.
hipError_t launch_gemv_nt(const Problem& p, hipStream_t stream);
bool gemv_nt_applies(const Problem& p);

// Fused causal attention forward (attention.hip): O = causal_softmax(scale *
// Q K^T) V per head, and optionally the probabilities P. Q [heads][queries]
// [head_dim] rows q_stride floats apart per head, K and V [heads][keys]
// [head_dim] kv_stride apart; O [heads][queries][head_dim] and P [heads]
// [queries][keys] dense. Query q sees keys 0 ..= q + query_offset.
struct CausalAttentionArgs {
    const float* q = nullptr;
    const float* k = nullptr;
    const float* v = nullptr;
    float* o = nullptr;
    float* p = nullptr;
    // Null, or per query {m, l} [heads][queries][2]: the maximum of its scaled
    // visible scores and the sum of e^(x - m) (for the recomputing backward).
    float* stats = nullptr;
    int64_t heads = 0, queries = 0, keys = 0, head_dim = 0;
    int64_t q_stride = 0, kv_stride = 0;
    int64_t query_offset = 0;
    float scale = 1.f;
    // The context's workspace and arrival counters: the decode form (at most
    // 4 queries per head, no probabilities) keeps per-chunk records there.
    float* workspace = nullptr;
    size_t workspace_bytes = 0;
    uint32_t* counters = nullptr;
    size_t counter_count = 0;
};
hipError_t launch_causal_attention(const CausalAttentionArgs& args, hipStream_t stream);
// Head dims 32, 64, 128; 16-byte aligned pointers and strides; per-head
// offsets within 31 bits.
bool causal_attention_supported(const CausalAttentionArgs& args);

// The fused probability gradient of that attention (attention.hip): grad =
// softmax_backward(P, dO V^T) per head, with the softmax projection taken
// as sum over h of dO * O; 0 past each query's horizon. dO and O
// [heads][queries][head_dim] (dO rows q_stride apart per head, O dense),
// V [heads][keys][head_dim] kv_stride apart, P and grad [heads][queries][keys].
struct AttentionScoreGradArgs {
    const float* d_out = nullptr;
    const float* v = nullptr;
    const float* out = nullptr;
    const float* p = nullptr;
    float* grad = nullptr;
    const float* k = nullptr;   // with q_grad: K, kv_stride apart like V
    float* q_grad = nullptr;    // null, or dQ = scale grad K, [heads][queries][head_dim]
    float scale = 1.f;
    int64_t heads = 0, queries = 0, keys = 0, head_dim = 0;
    int64_t q_stride = 0, kv_stride = 0;
    int64_t query_offset = 0;
};
hipError_t launch_attention_score_grad(const AttentionScoreGradArgs& args, hipStream_t stream);
bool attention_score_grad_supported(const AttentionScoreGradArgs& args);

// The attention backward that recomputes the probabilities instead of
// reading them (attention_backward.hip): from Q, K, V, the forward's O and
// row statistics, and dO, the three gradients CausalSelfAttention::backward
// leaves (layers/attention.rs:238-260): dV = P^T dO, dQ = scale dS K,
// dK = scale dS^T Q with dS = P * (dO V^T - D), D = sum over h of dO * O.
// Q and dO [heads][queries][h] (q_stride apart per head), K and V
// [heads][keys][h] (kv_stride apart), O and dQ [heads][queries][h] dense,
// dK and dV [heads][keys][h] dense, stats [heads][queries][2]. The workspace
// holds 12 bytes per query (m, 1/l, D; queries rounded up to 4).
struct AttentionBackwardArgs {
    const float* q = nullptr;
    const float* k = nullptr;
    const float* v = nullptr;
    const float* out = nullptr;
    const float* d_out = nullptr;
    const float* stats = nullptr;
    float* q_grad = nullptr;
    float* k_grad = nullptr;
    float* v_grad = nullptr;
    float* workspace = nullptr;
    size_t workspace_bytes = 0;
    int64_t heads = 0, queries = 0, keys = 0, head_dim = 0;
    int64_t q_stride = 0, kv_stride = 0;
    int64_t query_offset = 0;
    float scale = 1.f;
};
hipError_t launch_attention_backward(const AttentionBackwardArgs& args, hipStream_t stream);
bool attention_backward_supported(const AttentionBackwardArgs& args);

// Rounds an fp32 operand to bf16 (nearest-even) into dst[batch][rows][kp],
// K-contiguous, zeros for k in [k, kp) (bf16_stage.hip). Element (r, k) of
// the source is src[r * ld + k] when k_contiguous, else src[k * ld + r];
// batches are src_stride floats apart. kp must be a multiple of 8 and >= k.
// row_sums (a row-contiguous source, one batch): also the fp32 sums of each
// row over K, left as stage_sum_tiles(kp) partials, row_sums[tile][row],
// each over 64 consecutive k in order, for launch_column_sums_finish.
hipError_t launch_stage_bf16(const float* src, bool k_contiguous, int64_t ld, int64_t rows, int64_t k, int64_t kp,
                             int64_t batch, int64_t src_stride, uint16_t* dst, hipStream_t stream,
                             float* row_sums = nullptr);
int64_t stage_sum_tiles(int64_t kp);

// The 256 x 256 bf16 kernel's right-operand rows in quad order: position p
// of each 128-row group holds row quad_row(p), so that the rows a lane's four
// adjacent outputs come from sit 32 positions apart (gemm_bf16_wide.hip);
// quad_position is the inverse.
__host__ __device__ constexpr int64_t quad_row(int64_t p) { return (p / 128) * 128 + 4 * (p % 32) + (p % 128) / 32; }
__host__ __device__ constexpr int64_t quad_position(int64_t r) {
    return (r / 128) * 128 + 32 * (r % 4) + (r % 128) / 4;
}

// The same rounding into the layout the 256 x 256 bf16 kernel loads: per
// batch, per 32-deep step of K, the operand's rows_pad rows of 32 k,
// dst[batch][k / 32][slot][k % 32] with slot = row (or quad_position(row)
// when quad), so that a step's rows of one tile are one contiguous run of
// 64-byte rows. rows_pad (a multiple of 256, >= rows) and kp (a multiple of
// 32, >= k) are filled with zeros past rows and K. row_sums as above.
hipError_t launch_stage_bf16_blocks(const float* src, bool k_contiguous, int64_t ld, int64_t rows, int64_t k,
                                    int64_t kp, int64_t rows_pad, bool quad, int64_t batch, int64_t src_stride,
                                    uint16_t* dst, hipStream_t stream, float* row_sums = nullptr);

// Bytes of workspace launch_gemm_* would use for `p` (0 = none): split-K
// partial sums, and for bf16 the staged operands.
size_t gemm_workspace_bytes(const Problem& p, bool bf16, const Env& env);

// Linear's bias kernels (bias.hip). add_row_bias: out[b][r][c] += bias[c]
// for `batch` [rows, cols] matrices `stride` floats apart. column_sums:
// sums[c] += column c's sum over the [rows, cols] input, per-slice sums in
// the workspace (column_sums_workspace_bytes of it).
hipError_t launch_add_row_bias(float* out, int64_t rows, int64_t cols, int64_t batch, int64_t stride,
                               const float* bias, hipStream_t stream);
hipError_t launch_column_sums(const float* in, int64_t rows, int64_t cols, float* sums, const Env& env,
                              hipStream_t stream);
size_t column_sums_workspace_bytes(int64_t rows, int64_t cols, const Env& env);
// sums[c] += the sum of partial[s * cols + c] over s = 0 .. slices - 1,
// eight accumulators taken in slice order, then added together in order.
hipError_t launch_column_sums_finish(const float* partial, int64_t slices, int64_t cols, float* sums,
                                     hipStream_t stream);

// The weight-gradient product with the bias gradient (sn_matmul_column_sums):
// p.column_sums[c] += the sum over K of the right operand's column c, beside
// the product. Fused into the fp32 direct-to-LDS kernel or the bf16 wide
// kernel where that serves `p` (column_sums_fusion), else the product and
// then launch_column_sums; the workspace bytes are then the larger of the
// two steps'.
enum class ColumnSumsFusion { None, F32Direct, Bf16Wide };
ColumnSumsFusion column_sums_fusion(const Problem& p, uint32_t kernel, const Env& env);
LaunchShape describe_matmul_column_sums(const Problem& p, uint32_t kernel, const Env& env);
hipError_t launch_matmul_column_sums(const Problem& p, uint32_t kernel, const Env& env, hipStream_t stream);

// The row-wise kernels between the attention products (softmax.hip).
hipError_t launch_causal_softmax(float* scores, int64_t rows, int64_t queries, int64_t keys, float scale,
                                 int64_t query_offset, hipStream_t stream);
hipError_t launch_softmax_backward(const float* probabilities, float* grad, int64_t rows, int64_t cols,
                                   hipStream_t stream);

// The attention head permutes (heads.hip): split = packed -> head-major.
struct HeadLayoutArgs {
    int64_t batch, time, heads, head_dim, width, column_offset, time_capacity, time_offset;
};
hipError_t launch_permute_heads(bool split, const float* src, float* dst, const HeadLayoutArgs& layout,
                                hipStream_t stream);

// One classifier head's softmax cross-entropy and gradient (loss.hip).
struct CrossEntropyArgs {
    const float* logits;
    const uint32_t* targets;
    float* losses;
    float* grad;
    int64_t rows, cols;
    int64_t column_offset, classes, target_stride, target_offset;
    float grad_scale;
};
hipError_t launch_cross_entropy(const CrossEntropyArgs& args, hipStream_t stream);

}  // namespace sn

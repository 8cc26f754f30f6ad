// staleynet_cuda.hpp — C++ host mirror of the reference's `staleynet-cuda` GEMM
// API, built on the C ABI in include/staleynet_gemm.h.
//
// Names, argument meaning and failure behaviour follow the Rust originals:
//   Storage, BatchStrides, MatmulSpec + builders   crates/staleynet-cuda/src/ops/matmul.rs:14-142
//   WriteMode                                      crates/staleynet-cuda/src/ops/mod.rs:251-269
//   MatmulKernel + tolerance                       crates/staleynet-cuda/src/device.rs:38-67
//   Gpu (new, bind, synchronize, zeros, upload,
//        download, copy_from_host, fill_zero)      crates/staleynet-cuda/src/device.rs:129-208
//   Gpu::matmul                                    crates/staleynet-cuda/src/ops/matmul.rs:144-171
//   Gpu::add_row_bias, Gpu::accumulate_column_sums crates/staleynet-cuda/src/ops/elementwise.rs:30-58
//   Gpu::matmul_bias (matmul + add_row_bias fused; no reference counterpart: the two calls of
//                     Linear::forward, crates/staleynet-model/src/layers/linear.rs:46-47)
//   Gpu::matmul_column_sums (matmul + accumulate_column_sums of the right operand fused; no
//                     reference counterpart: the two calls of Linear::backward,
//                     crates/staleynet-model/src/layers/linear.rs:54-59)
//   Shape, Tensor                                  crates/staleynet-cuda/src/device.rs:210-275
//   TokenBuffer, Gpu::upload_tokens                crates/staleynet-cuda/src/device.rs:35-36, :194-197
//   Gpu::causal_softmax, Gpu::softmax_backward     crates/staleynet-cuda/src/ops/attention.rs:54-92
//   HeadLayout, Gpu::split_heads / merge_heads     crates/staleynet-cuda/src/kernels/attention.rs:19-75,
//                                                  crates/staleynet-cuda/src/ops/attention.rs:10-52
//   CrossEntropyHead, Gpu::cross_entropy           crates/staleynet-cuda/src/ops/loss.rs:14-71
//   Gpu::causal_attention (scores, causal_softmax and mix in one launch; no reference counterpart:
//                     the three calls of crates/staleynet-model/src/layers/attention.rs:206-213)
//   Gpu::causal_attention_score_grad (the dP product and softmax_backward in one launch; no
//                     reference counterpart: crates/staleynet-model/src/layers/attention.rs:238-248)
//   Gpu::causal_attention_with_stats, Gpu::causal_attention_backward (the forward keeping per-query
//                     statistics instead of the probabilities, and the backward that recomputes
//                     them; no reference counterpart: layers/attention.rs:206-213 and :238-260)
// The reference panics on undersized operands; here that is a thrown
// staleynet_cuda::Panic carrying the same message. Driver errors (the
// reference's Err(DriverError)) are thrown as staleynet_cuda::GpuError.
// `new` is a C++ keyword, so constructors named `new` in Rust are `new_`.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "staleynet_gemm.h"

namespace staleynet_cuda {

// An `assert!` of the reference, reported instead of aborting.
struct Panic : std::logic_error {
    int status;
    Panic(int code, const char* message) : std::logic_error(message), status(code) {}
};

// A runtime failure (`Err(DriverError)` in the reference).
struct GpuError : std::runtime_error {
    int status;
    explicit GpuError(int code) : std::runtime_error(sn_status_string(code)), status(code) {}
};

inline void check(int status) {
    if (status == SN_OK) return;
    if (status > 0 || status == SN_ERR_NO_DEVICE) throw GpuError(status);
    throw Panic(status, sn_status_string(status));
}

enum class Storage { RowMajor, Transposed };
enum class WriteMode { Overwrite, Accumulate };

// The reference's kernel choice. Naive and Tiled map to the reference-order
// kernel, Blocked to the fp32 matrix-core kernel (the default), TensorCore
// to the bf16-input matrix-core kernel that takes TF32's role on MI355X.
enum class MatmulKernel { Naive, Tiled, Blocked, TensorCore };

inline uint32_t abi_kernel(MatmulKernel kernel) {
    switch (kernel) {
        case MatmulKernel::Naive:
        case MatmulKernel::Tiled:
            return SN_KERNEL_SIMPLE;
        case MatmulKernel::Blocked:
            return SN_KERNEL_MFMA_F32;
        case MatmulKernel::TensorCore:
            return SN_KERNEL_MFMA_BF16;
    }
    return SN_KERNEL_MFMA_F32;
}

// `MatmulKernel::tolerance`: the largest relative error the kernel's arithmetic allows.
inline float tolerance(MatmulKernel kernel) { return sn_kernel_tolerance(abi_kernel(kernel)); }

inline const char* name(MatmulKernel kernel) {
    switch (kernel) {
        case MatmulKernel::Naive:
            return "Naive";
        case MatmulKernel::Tiled:
            return "Tiled";
        case MatmulKernel::Blocked:
            return "Blocked";
        case MatmulKernel::TensorCore:
            return "TensorCore";
    }
    return "?";
}

struct BatchStrides {
    size_t count;
    size_t left;
    size_t right;
    size_t output;
    static constexpr BatchStrides single() { return BatchStrides{1, 0, 0, 0}; }
};

struct MatmulSpec {
    size_t rows = 0;
    size_t cols = 0;
    size_t inner = 0;
    Storage left = Storage::RowMajor;
    Storage right = Storage::RowMajor;
    BatchStrides batch = BatchStrides::single();
    float scale = 1.0f;
    WriteMode write = WriteMode::Overwrite;
    // Extensions (no reference counterpart; zero keeps the reference's behaviour).
    uint32_t mask = SN_MASK_NONE;
    size_t query_offset = 0;

    static MatmulSpec new_(size_t rows, size_t cols, size_t inner) {
        MatmulSpec spec;
        spec.rows = rows;
        spec.cols = cols;
        spec.inner = inner;
        return spec;
    }
    MatmulSpec left_transposed() const { MatmulSpec s = *this; s.left = Storage::Transposed; return s; }
    MatmulSpec right_transposed() const { MatmulSpec s = *this; s.right = Storage::Transposed; return s; }
    MatmulSpec accumulate() const { MatmulSpec s = *this; s.write = WriteMode::Accumulate; return s; }
    MatmulSpec scaled(float factor) const { MatmulSpec s = *this; s.scale = factor; return s; }
    MatmulSpec batched(BatchStrides strides) const { MatmulSpec s = *this; s.batch = strides; return s; }
    MatmulSpec causal_output(size_t offset) const {
        MatmulSpec s = *this;
        s.mask = SN_MASK_CAUSAL_OUTPUT;
        s.query_offset = offset;
        return s;
    }
    MatmulSpec causal_left(size_t offset) const {
        MatmulSpec s = *this;
        s.mask = SN_MASK_CAUSAL_LEFT;
        s.query_offset = offset;
        return s;
    }

    // Elements an operand of `per_matrix` elements must hold (ops/matmul.rs:139-141).
    size_t required_len(size_t stride, size_t per_matrix) const { return (batch.count - 1) * stride + per_matrix; }

    sn_matmul_spec to_ffi() const {
        sn_matmul_spec c = sn_matmul_spec_new(rows, cols, inner);
        c.left_storage = left == Storage::Transposed ? SN_TRANSPOSED : SN_ROW_MAJOR;
        c.right_storage = right == Storage::Transposed ? SN_TRANSPOSED : SN_ROW_MAJOR;
        c.batch_count = batch.count;
        c.batch_left = batch.left;
        c.batch_right = batch.right;
        c.batch_output = batch.output;
        c.scale = scale;
        c.write = write == WriteMode::Accumulate ? SN_ACCUMULATE : SN_OVERWRITE;
        c.mask = mask;
        c.query_offset = query_offset;
        return c;
    }
};

struct Shape {
    size_t rows;
    size_t cols;
    static constexpr Shape new_(size_t rows, size_t cols) { return Shape{rows, cols}; }
    static constexpr Shape vector(size_t cols) { return Shape{1, cols}; }
    constexpr size_t len() const { return rows * cols; }
    constexpr bool is_empty() const { return len() == 0; }
};

// A row-major f32 matrix in device memory; owns its buffer (move-only).
class Tensor {
   public:
    Tensor() = default;
    Tensor(sn_context* context, float* buffer, Shape shape) : context_(context), buffer_(buffer), shape_(shape) {}
    Tensor(const Tensor&) = delete;
    Tensor& operator=(const Tensor&) = delete;
    Tensor(Tensor&& other) noexcept { *this = std::move(other); }
    Tensor& operator=(Tensor&& other) noexcept {
        if (this != &other) {
            release();
            context_ = std::exchange(other.context_, nullptr);
            buffer_ = std::exchange(other.buffer_, nullptr);
            shape_ = other.shape_;
        }
        return *this;
    }
    ~Tensor() { release(); }

    Shape shape() const { return shape_; }
    size_t len() const { return shape_.len(); }
    bool is_empty() const { return shape_.is_empty(); }
    const float* data() const { return buffer_; }
    float* data() { return buffer_; }

   private:
    void release() {
        if (buffer_ != nullptr) sn_free(context_, buffer_);
        buffer_ = nullptr;
    }
    sn_context* context_ = nullptr;
    float* buffer_ = nullptr;
    Shape shape_{0, 0};
};

// Token ids (u32) in device memory; owns its buffer (move-only).
class TokenBuffer {
   public:
    TokenBuffer() = default;
    TokenBuffer(sn_context* context, uint32_t* buffer, size_t count) : context_(context), buffer_(buffer), count_(count) {}
    TokenBuffer(const TokenBuffer&) = delete;
    TokenBuffer& operator=(const TokenBuffer&) = delete;
    TokenBuffer(TokenBuffer&& other) noexcept { *this = std::move(other); }
    TokenBuffer& operator=(TokenBuffer&& other) noexcept {
        if (this != &other) {
            release();
            context_ = std::exchange(other.context_, nullptr);
            buffer_ = std::exchange(other.buffer_, nullptr);
            count_ = std::exchange(other.count_, 0);
        }
        return *this;
    }
    ~TokenBuffer() { release(); }

    size_t len() const { return count_; }
    const uint32_t* data() const { return buffer_; }

   private:
    void release() {
        if (buffer_ != nullptr) sn_free_tokens(context_, buffer_);
        buffer_ = nullptr;
    }
    sn_context* context_ = nullptr;
    uint32_t* buffer_ = nullptr;
    size_t count_ = 0;
};

// Where a group of attention heads sits in the packed activations and in the
// head-major tensor (HeadLayout, kernels/attention.rs:19-75).
struct HeadLayout {
    size_t batch, time, heads, head_dim, width, column_offset, time_capacity, time_offset;

    static HeadLayout dense(size_t batch, size_t time, size_t heads, size_t head_dim, size_t width,
                            size_t column_offset) {
        return HeadLayout{batch, time, heads, head_dim, width, column_offset, time, 0};
    }
    HeadLayout in_cache(size_t capacity, size_t offset) const {
        HeadLayout l = *this;
        l.time_capacity = capacity;
        l.time_offset = offset;
        return l;
    }
    size_t element_count() const { return batch * heads * time * head_dim; }
    sn_head_layout to_ffi() const {
        return sn_head_layout{batch, time, heads, head_dim, width, column_offset, time_capacity, time_offset};
    }
};

// Which columns of a logits row and which target of a target row one
// classifier owns (CrossEntropyHead, ops/loss.rs:14-30).
struct CrossEntropyHead {
    size_t column_offset, classes, target_stride, target_offset;
    float grad_scale;
};

// One device, one stream, and the kernel choice (device.rs:129-155).
class Gpu {
   public:
    // Public like the reference's field (device.rs:144); read on every matmul.
    MatmulKernel matmul_kernel = MatmulKernel::Blocked;

    static Gpu new_(int ordinal) {
        sn_context* context = nullptr;
        check(sn_context_create(ordinal, &context));
        return Gpu(context);
    }
    Gpu(Gpu&& other) noexcept : matmul_kernel(other.matmul_kernel), context_(std::exchange(other.context_, nullptr)) {}
    Gpu(const Gpu&) = delete;
    Gpu& operator=(const Gpu&) = delete;
    ~Gpu() {
        if (context_ != nullptr) sn_context_destroy(context_);
    }

    void bind_to_current_thread() const { check(sn_context_bind(context_)); }
    void synchronize() const { check(sn_synchronize(context_)); }

    Tensor zeros(Shape shape) const {
        float* buffer = nullptr;
        check(sn_alloc_zeroed(context_, shape.len(), &buffer));
        return Tensor(context_, buffer, shape);
    }

    Tensor upload(Shape shape, const std::vector<float>& values) const {
        if (values.size() != shape.len()) throw Panic(SN_ERR_UNSUPPORTED, "upload: value count does not match the shape");
        float* buffer = nullptr;
        check(sn_upload(context_, values.data(), values.size(), &buffer));
        return Tensor(context_, buffer, shape);
    }

    std::vector<float> download(const Tensor& tensor) const {
        std::vector<float> host(tensor.len());
        check(sn_download(context_, tensor.data(), host.size(), host.data()));
        return host;
    }

    void copy_from_host(Tensor& tensor, const std::vector<float>& values) const {
        if (values.size() != tensor.len()) throw Panic(SN_ERR_UNSUPPORTED, "copy_from_host: length mismatch");
        check(sn_copy_from_host(context_, tensor.data(), values.data(), values.size()));
    }

    void fill_zero(Tensor& tensor) const { check(sn_fill_zero(context_, tensor.data(), tensor.len())); }

    // `Gpu::matmul`: enqueue output = scale·op(left)·op(right) (+ output).
    void matmul(const MatmulSpec& spec, const Tensor& left, const Tensor& right, Tensor& output) const {
        check(sn_context_set_kernel(context_, abi_kernel(matmul_kernel)));
        const sn_matmul_spec c = spec.to_ffi();
        check(sn_matmul(context_, &c, left.data(), left.len(), right.data(), right.len(), output.data(),
                        output.len()));
    }

    // `Gpu::add_row_bias`: output[r, c] += bias[c].
    void add_row_bias(Tensor& output, const Tensor& bias) const {
        const int rc = sn_add_row_bias(context_, output.data(), output.shape().rows, output.shape().cols, bias.data(),
                                       bias.len());
        if (rc == SN_ERR_LENGTH_MISMATCH) throw Panic(rc, "add_row_bias: bias length must equal output columns");
        check(rc);
    }

    // `Gpu::accumulate_column_sums`: sums += the column sums of input.
    void accumulate_column_sums(const Tensor& input, Tensor& sums) const {
        const int rc = sn_accumulate_column_sums(context_, input.data(), input.shape().rows, input.shape().cols,
                                                 sums.data(), sums.len());
        if (rc == SN_ERR_LENGTH_MISMATCH)
            throw Panic(rc, "accumulate_column_sums: sums length must equal input columns");
        check(rc);
    }

    // `matmul` then `add_row_bias` on its output, in one pass (sn_matmul_bias).
    void matmul_bias(const MatmulSpec& spec, const Tensor& left, const Tensor& right, const Tensor& bias,
                     Tensor& output) const {
        check(sn_context_set_kernel(context_, abi_kernel(matmul_kernel)));
        const sn_matmul_spec c = spec.to_ffi();
        check(sn_matmul_bias(context_, &c, left.data(), left.len(), right.data(), right.len(), bias.data(),
                             bias.len(), output.data(), output.len()));
    }

    // `matmul` then `accumulate_column_sums(right, sums)`, in one call (sn_matmul_column_sums; the
    // right operand row-major, the spec unbatched).
    void matmul_column_sums(const MatmulSpec& spec, const Tensor& left, const Tensor& right, Tensor& output,
                            Tensor& sums) const {
        check(sn_context_set_kernel(context_, abi_kernel(matmul_kernel)));
        const sn_matmul_spec c = spec.to_ffi();
        check(sn_matmul_column_sums(context_, &c, left.data(), left.len(), right.data(), right.len(), output.data(),
                                    output.len(), sums.data(), sums.len()));
    }

    TokenBuffer upload_tokens(const std::vector<uint32_t>& tokens) const {
        uint32_t* buffer = nullptr;
        check(sn_upload_tokens(context_, tokens.data(), tokens.size(), &buffer));
        return TokenBuffer(context_, buffer, tokens.size());
    }

    std::vector<uint32_t> download_tokens(const TokenBuffer& tokens) const {
        std::vector<uint32_t> host(tokens.len());
        check(sn_download_tokens(context_, tokens.data(), host.size(), host.data()));
        return host;
    }

    // `Gpu::causal_softmax`: in place on [matrices · queries, keys] scores.
    void causal_softmax(Tensor& scores, size_t queries, float scale, size_t query_offset) const {
        const int rc = sn_causal_softmax(context_, scores.data(), scores.shape().rows, scores.shape().cols, queries,
                                         scale, query_offset);
        if (rc == SN_ERR_SHAPE) throw Panic(rc, "causal_softmax: rows must be a multiple of queries");
        check(rc);
    }

    // `Gpu::softmax_backward`: grad <- p * (grad - sum(grad * p)) per row.
    void softmax_backward(const Tensor& probabilities, Tensor& grad) const {
        const int rc = sn_softmax_backward(context_, probabilities.data(), probabilities.shape().rows,
                                           probabilities.shape().cols, grad.data(), grad.shape().rows,
                                           grad.shape().cols);
        if (rc == SN_ERR_SHAPE) throw Panic(rc, "softmax_backward: shape mismatch");
        check(rc);
    }

    // `Gpu::split_heads`: packed columns -> head-major tensor.
    void split_heads(const Tensor& packed, Tensor& head_major, const HeadLayout& layout) const {
        check_layout(layout, packed, head_major);
        const sn_head_layout l = layout.to_ffi();
        check(sn_split_heads(context_, packed.data(), packed.len(), head_major.data(), head_major.len(), &l));
    }

    // `Gpu::merge_heads`: head-major tensor -> packed columns (the others left alone).
    void merge_heads(const Tensor& head_major, Tensor& packed, const HeadLayout& layout) const {
        check_layout(layout, packed, head_major);
        const sn_head_layout l = layout.to_ffi();
        check(sn_merge_heads(context_, head_major.data(), head_major.len(), packed.data(), packed.len(), &l));
    }

    // `Gpu::cross_entropy`: one codebook's losses and its columns of the gradient.
    void cross_entropy(const Tensor& logits, const TokenBuffer& targets, const CrossEntropyHead& head, Tensor& losses,
                       Tensor& logits_grad) const {
        const Shape shape = logits.shape();
        if (logits_grad.shape().rows != shape.rows || logits_grad.shape().cols != shape.cols)
            throw Panic(SN_ERR_SHAPE, "cross_entropy: gradient shape");
        if (head.column_offset + head.classes > shape.cols) throw Panic(SN_ERR_SHAPE, "cross_entropy: head exceeds logits");
        if (losses.len() < shape.rows) throw Panic(SN_ERR_LENGTH_MISMATCH, "cross_entropy: losses too small");
        if (targets.len() < shape.rows * head.target_stride)
            throw Panic(SN_ERR_LENGTH_MISMATCH, "cross_entropy: too few targets");
        const sn_cross_entropy_head h{head.column_offset, head.classes, head.target_stride, head.target_offset,
                                      head.grad_scale};
        check(sn_cross_entropy(context_, logits.data(), shape.rows, shape.cols, targets.data(), targets.len(), &h,
                               losses.data(), losses.len(), logits_grad.data(), logits_grad.shape().rows,
                               logits_grad.shape().cols));
    }

    // The scores product, causal_softmax and the mix product in one launch
    // (sn_causal_attention); `probabilities` may be null.
    void causal_attention(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& out, const sn_attention_shape& shape,
                          Tensor* probabilities = nullptr) const {
        check(sn_causal_attention(context_, &shape, q.data(), q.len(), k.data(), k.len(), v.data(), v.len(),
                                  out.data(), out.len(), probabilities ? probabilities->data() : nullptr,
                                  probabilities ? probabilities->len() : 0));
    }

    // The dP product and softmax_backward of the attention backward in one launch
    // (sn_causal_attention_score_grad): grad = P * (dO V^T - rowsum(dO * O)).
    // With k and q_grad, also the query gradient q_grad = shape.scale * grad K.
    void causal_attention_score_grad(const Tensor& d_out, const Tensor& v, const Tensor& out, const Tensor& probabilities,
                                     Tensor& grad, const sn_attention_shape& shape, const Tensor* k = nullptr,
                                     Tensor* q_grad = nullptr) const {
        check(sn_causal_attention_score_grad(context_, &shape, d_out.data(), d_out.len(), v.data(), v.len(),
                                             out.data(), out.len(), probabilities.data(), probabilities.len(),
                                             grad.data(), grad.len(), k ? k->data() : nullptr, k ? k->len() : 0,
                                             q_grad ? q_grad->data() : nullptr, q_grad ? q_grad->len() : 0));
    }

    // The fused forward keeping, per query, the maximum m of its scaled visible scores and the sum
    // l of e^(x - m) (2 floats, in `stats`) instead of the probabilities
    // (sn_causal_attention_with_stats); `out` is causal_attention's O.
    void causal_attention_with_stats(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& out, Tensor& stats,
                                     const sn_attention_shape& shape) const {
        check(sn_causal_attention_with_stats(context_, &shape, q.data(), q.len(), k.data(), k.len(), v.data(), v.len(),
                                             out.data(), out.len(), stats.data(), stats.len()));
    }

    // The attention backward from O, dO and those statistics (sn_causal_attention_backward): the
    // query, key and value gradients CausalSelfAttention::backward leaves, with no P or dS in memory.
    void causal_attention_backward(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& out,
                                   const Tensor& d_out, const Tensor& stats, Tensor& q_grad, Tensor& k_grad,
                                   Tensor& v_grad, const sn_attention_shape& shape) const {
        check(sn_causal_attention_backward(context_, &shape, q.data(), q.len(), k.data(), k.len(), v.data(), v.len(),
                                           out.data(), out.len(), d_out.data(), d_out.len(), stats.data(), stats.len(),
                                           q_grad.data(), q_grad.len(), k_grad.data(), k_grad.len(), v_grad.data(),
                                           v_grad.len()));
    }

    sn_context* raw() const { return context_; }

   private:
    // check_layout (ops/attention.rs:11-18).
    static void check_layout(const HeadLayout& layout, const Tensor& packed, const Tensor& head_major) {
        if (layout.time_offset + layout.time > layout.time_capacity)
            throw Panic(SN_ERR_SHAPE, "HeadLayout: time range exceeds capacity");
        if (packed.len() < layout.batch * layout.time * layout.width)
            throw Panic(SN_ERR_LENGTH_MISMATCH, "HeadLayout: packed tensor too small");
        if (head_major.len() < layout.batch * layout.heads * layout.time_capacity * layout.head_dim)
            throw Panic(SN_ERR_LENGTH_MISMATCH, "HeadLayout: head-major tensor too small");
    }

    explicit Gpu(sn_context* context) : context_(context) {}
    sn_context* context_ = nullptr;
};

}  // namespace staleynet_cuda

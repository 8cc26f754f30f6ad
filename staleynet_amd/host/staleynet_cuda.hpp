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
//   Shape, Tensor                                  crates/staleynet-cuda/src/device.rs:210-275
// The reference panics on undersized operands; here that is a thrown
// staleynet_cuda::Panic carrying the same message. Driver errors (the
// reference's Err(DriverError)) are thrown as staleynet_cuda::GpuError.
// `new` is a C++ keyword, so constructors named `new` in Rust are `new_`.
#pragma once

#include <cstddef>
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

    sn_context* raw() const { return context_; }

   private:
    explicit Gpu(sn_context* context) : context_(context) {}
    sn_context* context_ = nullptr;
};

}  // namespace staleynet_cuda

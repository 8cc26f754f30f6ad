// The C ABI (include/staleynet_gemm.h): device context, buffers, validation
// and the GEMM dispatcher. Mirrors the reference's `Gpu` handle
// (crates/staleynet-cuda/src/device.rs:129-208) and `Gpu::matmul`
// (crates/staleynet-cuda/src/ops/matmul.rs:144-171).
#include "staleynet_gemm.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <new>

#include "gemm_internal.h"

struct sn_context {
    int device = 0;
    hipStream_t stream = nullptr;
    uint32_t kernel = SN_KERNEL_MFMA_F32;
    sn::Env env;
};

// The C structs' layouts are part of the ABI a Rust #[repr(C)] binding
// mirrors (x86-64 / aarch64 LP64): sizes and field offsets pinned here.
static_assert(sizeof(sn_matmul_spec) == 88 && offsetof(sn_matmul_spec, left_storage) == 24 &&
                  offsetof(sn_matmul_spec, batch_count) == 32 && offsetof(sn_matmul_spec, scale) == 64 &&
                  offsetof(sn_matmul_spec, write) == 68 && offsetof(sn_matmul_spec, mask) == 72 &&
                  offsetof(sn_matmul_spec, precision) == 76 && offsetof(sn_matmul_spec, query_offset) == 80,
              "sn_matmul_spec layout");
static_assert(sizeof(sn_attention_shape) == 64 && offsetof(sn_attention_shape, query_offset) == 48 &&
                  offsetof(sn_attention_shape, scale) == 56,
              "sn_attention_shape layout");
static_assert(sizeof(sn_head_layout) == 64 && offsetof(sn_head_layout, time_offset) == 56, "sn_head_layout layout");
static_assert(sizeof(sn_cross_entropy_head) == 40 && offsetof(sn_cross_entropy_head, grad_scale) == 32,
              "sn_cross_entropy_head layout");
static_assert(sizeof(sn_launch_plan) == 72 && offsetof(sn_launch_plan, k_per_split) == 32 &&
                  offsetof(sn_launch_plan, workspace_bytes) == 64,
              "sn_launch_plan layout");

namespace {

constexpr size_t kDefaultWorkspaceBytes = size_t(1536) << 20;
constexpr size_t kCounterCount = 16384;
// Dimensions above this would overflow the kernels' 32-bit tile counters.
constexpr size_t kMaxDimension = size_t(1) << 31;

int status(hipError_t err) { return err == hipSuccess ? SN_OK : int(err); }

bool mul_overflows(size_t a, size_t b, size_t* out) { return __builtin_mul_overflow(a, b, out); }

// `(count - 1) * stride + per_matrix` (ops/matmul.rs:139-141), or false on
// overflow. `count` is at least 1 here.
bool required_len(size_t count, size_t stride, size_t per_matrix, size_t* out) {
    size_t span;
    if (mul_overflows(count - 1, stride, &span)) return false;
    return !__builtin_add_overflow(span, per_matrix, out);
}

struct Lengths {
    size_t left, right, output;
};

int check_spec(const sn_matmul_spec* spec, Lengths* need) {
    if (spec == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (spec->batch_count == 0) return SN_ERR_EMPTY_BATCH;
    if (spec->left_storage > SN_TRANSPOSED || spec->right_storage > SN_TRANSPOSED) return SN_ERR_UNSUPPORTED;
    if (spec->write > SN_ACCUMULATE || spec->mask > SN_MASK_CAUSAL_LEFT) return SN_ERR_UNSUPPORTED;
    if (spec->precision > SN_PRECISION_BF16) return SN_ERR_UNSUPPORTED;
    if (spec->rows >= kMaxDimension || spec->cols >= kMaxDimension || spec->inner >= kMaxDimension ||
        spec->batch_count >= kMaxDimension)
        return SN_ERR_OVERFLOW;
    if (spec->query_offset >= (size_t(1) << 62)) return SN_ERR_OVERFLOW;
    size_t left_per, right_per, out_per;
    if (mul_overflows(spec->rows, spec->inner, &left_per) || mul_overflows(spec->inner, spec->cols, &right_per) ||
        mul_overflows(spec->rows, spec->cols, &out_per))
        return SN_ERR_OVERFLOW;
    if (!required_len(spec->batch_count, spec->batch_left, left_per, &need->left) ||
        !required_len(spec->batch_count, spec->batch_right, right_per, &need->right) ||
        !required_len(spec->batch_count, spec->batch_output, out_per, &need->output))
        return SN_ERR_OVERFLOW;
    // Byte offsets must stay below 2^63 for the kernels' signed arithmetic.
    const size_t limit = size_t(1) << 60;
    if (need->left >= limit || need->right >= limit || need->output >= limit) return SN_ERR_OVERFLOW;
    return SN_OK;
}

bool overlaps(const float* a, size_t a_len, const float* b, size_t b_len) {
    if (a_len == 0 || b_len == 0) return false;
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
    return a0 < b0 + b_len * sizeof(float) && b0 < a0 + a_len * sizeof(float);
}

}  // namespace

extern "C" {

sn_matmul_spec sn_matmul_spec_new(size_t rows, size_t cols, size_t inner) {
    sn_matmul_spec spec;
    std::memset(&spec, 0, sizeof(spec));
    spec.rows = rows;
    spec.cols = cols;
    spec.inner = inner;
    spec.left_storage = SN_ROW_MAJOR;
    spec.right_storage = SN_ROW_MAJOR;
    spec.batch_count = 1;
    spec.scale = 1.0f;
    spec.write = SN_OVERWRITE;
    spec.mask = SN_MASK_NONE;
    spec.precision = SN_PRECISION_DEFAULT;
    return spec;
}

int sn_context_create_with_workspace(int ordinal, size_t workspace_bytes, sn_context** out) {
    if (out == nullptr) return SN_ERR_NULL_ARGUMENT;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || ordinal < 0 || ordinal >= count) return SN_ERR_NO_DEVICE;
    hipError_t err = hipSetDevice(ordinal);
    if (err != hipSuccess) return status(err);
    sn_context* ctx = new (std::nothrow) sn_context();
    if (ctx == nullptr) return SN_ERR_OVERFLOW;
    ctx->device = ordinal;
    hipDeviceProp_t prop;
    err = hipGetDeviceProperties(&prop, ordinal);
    if (err == hipSuccess && prop.multiProcessorCount > 0) ctx->env.cu_count = prop.multiProcessorCount;
    if (err == hipSuccess) err = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (err == hipSuccess) {
        // The arrival counters and the hand-off slots: one allocation, zeroed once.
        void* counters = nullptr;
        const size_t words = kCounterCount + sn::kHandoffWords;
        err = hipMalloc(&counters, words * sizeof(uint32_t));
        if (err == hipSuccess) {
            ctx->env.counters = static_cast<uint32_t*>(counters);
            ctx->env.counter_count = kCounterCount;
            ctx->env.handoff = ctx->env.counters + kCounterCount;
            ctx->env.handoff_words = sn::kHandoffWords;
            err = hipMemsetAsync(counters, 0, words * sizeof(uint32_t), ctx->stream);
            if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
        }
    }
    if (err == hipSuccess && workspace_bytes > 0) {
        void* ws = nullptr;
        err = hipMalloc(&ws, workspace_bytes);
        if (err == hipSuccess) {
            ctx->env.workspace = static_cast<float*>(ws);
            ctx->env.workspace_bytes = workspace_bytes;
        }
    }
    if (err != hipSuccess) {
        sn_context_destroy(ctx);
        return status(err);
    }
    *out = ctx;
    return SN_OK;
}

int sn_context_create(int ordinal, sn_context** out) {
    return sn_context_create_with_workspace(ordinal, kDefaultWorkspaceBytes, out);
}

int sn_context_destroy(sn_context* ctx) {
    if (ctx == nullptr) return SN_OK;
    hipError_t first = hipSetDevice(ctx->device);
    if (ctx->stream != nullptr) {
        hipError_t err = hipStreamSynchronize(ctx->stream);
        if (first == hipSuccess) first = err;
        err = hipStreamDestroy(ctx->stream);
        if (first == hipSuccess) first = err;
    }
    if (ctx->env.workspace != nullptr) {
        hipError_t err = hipFree(ctx->env.workspace);
        if (first == hipSuccess) first = err;
    }
    if (ctx->env.counters != nullptr) {
        hipError_t err = hipFree(ctx->env.counters);
        if (first == hipSuccess) first = err;
    }
    delete ctx;
    return status(first);
}

int sn_context_bind(sn_context* ctx) {
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    return status(hipSetDevice(ctx->device));
}

int sn_context_set_kernel(sn_context* ctx, uint32_t kernel) {
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (kernel > SN_KERNEL_SIMPLE) return SN_ERR_UNSUPPORTED;
    ctx->kernel = kernel;
    return SN_OK;
}

int sn_context_get_kernel(const sn_context* ctx, uint32_t* kernel) {
    if (ctx == nullptr || kernel == nullptr) return SN_ERR_NULL_ARGUMENT;
    *kernel = ctx->kernel;
    return SN_OK;
}

void* sn_context_stream(sn_context* ctx) { return ctx == nullptr ? nullptr : static_cast<void*>(ctx->stream); }

float sn_kernel_tolerance(uint32_t kernel) {
    switch (kernel) {
        case SN_KERNEL_MFMA_F32:
        case SN_KERNEL_SIMPLE:
            return 1e-5f;
        case SN_KERNEL_MFMA_BF16:
            return 2e-2f;
        default:
            return NAN;
    }
}

int sn_synchronize(sn_context* ctx) {
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    return status(err);
}

int sn_alloc_zeroed(sn_context* ctx, size_t count, float** out) {
    if (ctx == nullptr || out == nullptr) return SN_ERR_NULL_ARGUMENT;
    *out = nullptr;
    size_t bytes;
    if (mul_overflows(count, sizeof(float), &bytes)) return SN_ERR_OVERFLOW;
    if (bytes == 0) return SN_OK;
    hipError_t err = hipSetDevice(ctx->device);
    void* p = nullptr;
    if (err == hipSuccess) err = hipMalloc(&p, bytes);
    if (err == hipSuccess) err = hipMemsetAsync(p, 0, bytes, ctx->stream);
    if (err != hipSuccess) {
        if (p != nullptr) (void)hipFree(p);
        return status(err);
    }
    *out = static_cast<float*>(p);
    return SN_OK;
}

int sn_free(sn_context* ctx, float* buffer) {
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (buffer == nullptr) return SN_OK;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess) err = hipFree(buffer);
    return status(err);
}

int sn_upload(sn_context* ctx, const float* host, size_t count, float** out) {
    if (ctx == nullptr || out == nullptr || (host == nullptr && count > 0)) return SN_ERR_NULL_ARGUMENT;
    *out = nullptr;
    size_t bytes;
    if (mul_overflows(count, sizeof(float), &bytes)) return SN_ERR_OVERFLOW;
    if (bytes == 0) return SN_OK;
    hipError_t err = hipSetDevice(ctx->device);
    void* p = nullptr;
    if (err == hipSuccess) err = hipMalloc(&p, bytes);
    if (err == hipSuccess) err = hipMemcpyAsync(p, host, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    if (err != hipSuccess) {
        if (p != nullptr) (void)hipFree(p);
        return status(err);
    }
    *out = static_cast<float*>(p);
    return SN_OK;
}

int sn_download(sn_context* ctx, const float* device, size_t count, float* host) {
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (count == 0) return SN_OK;
    if (device == nullptr || host == nullptr) return SN_ERR_NULL_ARGUMENT;
    size_t bytes;
    if (mul_overflows(count, sizeof(float), &bytes)) return SN_ERR_OVERFLOW;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess) err = hipMemcpyAsync(host, device, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    return status(err);
}

int sn_copy_from_host(sn_context* ctx, float* device, const float* host, size_t count) {
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (count == 0) return SN_OK;
    if (device == nullptr || host == nullptr) return SN_ERR_NULL_ARGUMENT;
    size_t bytes;
    if (mul_overflows(count, sizeof(float), &bytes)) return SN_ERR_OVERFLOW;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess) err = hipMemcpyAsync(device, host, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    return status(err);
}

int sn_fill_zero(sn_context* ctx, float* device, size_t count) {
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (count == 0) return SN_OK;
    if (device == nullptr) return SN_ERR_NULL_ARGUMENT;
    size_t bytes;
    if (mul_overflows(count, sizeof(float), &bytes)) return SN_ERR_OVERFLOW;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess) err = hipMemsetAsync(device, 0, bytes, ctx->stream);
    return status(err);
}

int sn_matmul_validate(const sn_matmul_spec* spec, size_t left_len, size_t right_len, size_t output_len) {
    Lengths need;
    const int rc = check_spec(spec, &need);
    if (rc != SN_OK) return rc;
    if (left_len < need.left) return SN_ERR_LEFT_TOO_SMALL;
    if (right_len < need.right) return SN_ERR_RIGHT_TOO_SMALL;
    if (output_len < need.output) return SN_ERR_OUTPUT_TOO_SMALL;
    return SN_OK;
}

}  // extern "C"

namespace sn {

// The kernels' description of a validated spec (ops/matmul.rs:24-32 for
// the storage conventions), with `bias` (null: none) fused into the
// epilogue unless the product is masked.
Problem problem_of(const sn_matmul_spec* spec, const float* left, const float* right, float* output,
                       const float* bias) {
    Problem p;
    p.a = left;
    p.b = right;
    p.c = output;
    p.m = int64_t(spec->rows);
    p.n = int64_t(spec->cols);
    p.k = int64_t(spec->inner);
    // Left [rows, inner]: row-major is K-contiguous (ld = inner); transposed
    // storage keeps it as [inner, rows] (ld = rows). Right [inner, cols]:
    // row-major is N-contiguous (ld = cols); transposed is [cols, inner],
    // K-contiguous (ld = inner).
    p.a_k_contiguous = spec->left_storage == SN_ROW_MAJOR;
    p.lda = p.a_k_contiguous ? p.k : p.m;
    p.b_k_contiguous = spec->right_storage == SN_TRANSPOSED;
    p.ldb = p.b_k_contiguous ? p.k : p.n;
    p.batch = int64_t(spec->batch_count);
    p.stride_a = int64_t(spec->batch_left);
    p.stride_b = int64_t(spec->batch_right);
    p.stride_c = int64_t(spec->batch_output);
    p.scale = spec->scale;
    p.accumulate = spec->write == SN_ACCUMULATE;
    p.mask = spec->mask;
    p.query_offset = int64_t(spec->query_offset);
    // A masked product takes its bias afterwards (the kernels fuse it only
    // into unmasked epilogues).
    p.bias = p.mask != SN_MASK_NONE ? nullptr : bias;
    return p;
}

// The kernel a call runs: the context's choice, overridden by the spec's
// precision.
uint32_t kernel_for(uint32_t context_kernel, uint32_t precision) {
    if (precision == SN_PRECISION_F32 && context_kernel == SN_KERNEL_MFMA_BF16) return SN_KERNEL_MFMA_F32;
    if (precision == SN_PRECISION_BF16) return SN_KERNEL_MFMA_BF16;
    return context_kernel;
}

int check_matmul_call(const sn_matmul_spec* spec, const float* left, size_t left_len, const float* right,
                      size_t right_len, const float* bias, size_t bias_len, const float* output, size_t output_len) {
    int rc = sn_matmul_validate(spec, left_len, right_len, output_len);
    if (rc != SN_OK) return rc;
    Lengths need;
    check_spec(spec, &need);
    if ((need.left > 0 && left == nullptr) || (need.right > 0 && right == nullptr) ||
        (need.output > 0 && output == nullptr))
        return SN_ERR_NULL_ARGUMENT;
    if (overlaps(output, need.output, left, need.left) || overlaps(output, need.output, right, need.right))
        return SN_ERR_ALIASING;
    if (bias != nullptr && overlaps(output, need.output, bias, bias_len)) return SN_ERR_ALIASING;
    return SN_OK;
}

}  // namespace sn

namespace {

// sn_plan_matmul and sn_plan_matmul_column_sums: the launch the call would
// make, from host code only.
int plan_of(const sn_matmul_spec* spec, uint32_t kernel, const float* left, const float* right, const float* output,
            uint32_t cu_count, size_t workspace_bytes, bool column_sums, sn_launch_plan* plan) {
    if (plan == nullptr) return SN_ERR_NULL_ARGUMENT;
    std::memset(plan, 0, sizeof(*plan));
    Lengths need;
    const int rc = check_spec(spec, &need);
    if (rc != SN_OK) return rc;
    if (kernel > SN_KERNEL_SIMPLE) return SN_ERR_UNSUPPORTED;
    if (column_sums && (spec->right_storage != SN_ROW_MAJOR || spec->batch_count != 1)) return SN_ERR_UNSUPPORTED;
    sn::Problem p = sn::problem_of(spec, left, right, const_cast<float*>(output), nullptr);
    // A context's environment as sn_context_create would set it up; the
    // workspace and counters are never touched, only their sizes and the
    // workspace's alignment matter (a device allocation is 2 MiB aligned).
    sn::Env env;
    env.cu_count = cu_count > 0 ? int(cu_count) : 256;
    env.workspace_bytes = workspace_bytes;
    env.workspace = workspace_bytes > 0 ? reinterpret_cast<float*>(uintptr_t(1) << 44) : nullptr;
    env.counters = reinterpret_cast<uint32_t*>(uintptr_t(1) << 45);
    env.counter_count = kCounterCount;
    env.handoff = env.counters + kCounterCount;
    env.handoff_words = sn::kHandoffWords;
    const uint32_t k = sn::kernel_for(kernel, spec->precision);
    sn::LaunchShape s;
    if (column_sums) {
        // Only the sums' address matters to the plan, and only its being
        // non-null: any aligned stand-in will do.
        p.column_sums = reinterpret_cast<float*>(uintptr_t(1) << 46);
        s = sn::describe_matmul_column_sums(p, k, env);
        switch (sn::column_sums_fusion(p, k, env)) {
            case sn::ColumnSumsFusion::F32Direct: s.path = SN_PATH_F32_DIRECT_SUMS; break;
            case sn::ColumnSumsFusion::Bf16Wide: s.path = SN_PATH_BF16_WIDE_SUMS; break;
            case sn::ColumnSumsFusion::None: break;
        }
    } else {
        s = sn::describe_matmul(p, k, env);
    }
    plan->path = s.path;
    plan->threads = s.threads;
    plan->tile_rows = uint32_t(s.tile_m);
    plan->tile_cols = uint32_t(s.tile_n);
    plan->tiles_m = uint32_t(s.tiles_m);
    plan->tiles_n = uint32_t(s.tiles_n);
    plan->splits = uint32_t(s.splits);
    plan->persistent_grid = uint32_t(s.persistent_grid);
    plan->k_per_split = uint64_t(s.k_per_split);
    plan->batches_per_launch = uint64_t(s.batches_per_launch);
    plan->workgroups = uint64_t(s.workgroups);
    plan->launches = uint64_t(s.launches);
    plan->workspace_bytes = uint64_t(s.workspace_bytes);
    return s.workspace_bytes > workspace_bytes ? SN_ERR_WORKSPACE : SN_OK;
}

// sn_matmul and sn_matmul_bias: validation, then the product with `bias`
// (null: none) added in its epilogue, or, for a masked spec, after it by the
// bias kernel.
int matmul_with_bias(sn_context* ctx, const sn_matmul_spec* spec, const float* left, size_t left_len,
                     const float* right, size_t right_len, const float* bias, size_t bias_len, float* output,
                     size_t output_len) {
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    const int rc = sn::check_matmul_call(spec, left, left_len, right, right_len, bias, bias_len, output, output_len);
    if (rc != SN_OK) return rc;
    if (spec->rows == 0 || spec->cols == 0) return SN_OK;

    const sn::Problem p = sn::problem_of(spec, left, right, output, bias);
    const bool bias_after = bias != nullptr && p.bias == nullptr;
    const uint32_t kernel = sn::kernel_for(ctx->kernel, spec->precision);
    if (sn::describe_matmul(p, kernel, ctx->env).workspace_bytes > ctx->env.workspace_bytes) return SN_ERR_WORKSPACE;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess) err = sn::launch_matmul(p, kernel, ctx->env, ctx->stream);
    if (err == hipSuccess && bias_after)
        err = sn::launch_add_row_bias(output, p.m, p.n, p.batch, p.stride_c, bias, ctx->stream);
    return status(err);
}

}  // namespace

extern "C" {

int sn_matmul(sn_context* ctx, const sn_matmul_spec* spec, const float* left, size_t left_len, const float* right,
              size_t right_len, float* output, size_t output_len) {
    return matmul_with_bias(ctx, spec, left, left_len, right, right_len, nullptr, 0, output, output_len);
}

int sn_matmul_bias(sn_context* ctx, const sn_matmul_spec* spec, const float* left, size_t left_len,
                   const float* right, size_t right_len, const float* bias, size_t bias_len, float* output,
                   size_t output_len) {
    const int rc = sn_matmul_validate(spec, left_len, right_len, output_len);
    if (rc != SN_OK) return rc;
    if (bias_len != spec->cols) return SN_ERR_LENGTH_MISMATCH;
    // Output matrices that share memory (a batch stride below one matrix)
    // would take the bias more than once.
    if (spec->batch_count > 1 && spec->batch_output < spec->rows * spec->cols) return SN_ERR_UNSUPPORTED;
    if (ctx == nullptr || (bias == nullptr && bias_len > 0)) return SN_ERR_NULL_ARGUMENT;
    return matmul_with_bias(ctx, spec, left, left_len, right, right_len, bias, bias_len, output, output_len);
}

int sn_plan_matmul(const sn_matmul_spec* spec, uint32_t kernel, const float* left, const float* right,
                   const float* output, uint32_t cu_count, size_t workspace_bytes, sn_launch_plan* plan) {
    return plan_of(spec, kernel, left, right, output, cu_count, workspace_bytes, false, plan);
}

int sn_plan_matmul_column_sums(const sn_matmul_spec* spec, uint32_t kernel, const float* left, const float* right,
                               const float* output, uint32_t cu_count, size_t workspace_bytes, sn_launch_plan* plan) {
    return plan_of(spec, kernel, left, right, output, cu_count, workspace_bytes, true, plan);
}

int sn_add_row_bias(sn_context* ctx, float* output, size_t rows, size_t cols, const float* bias, size_t bias_len) {
    if (bias_len != cols) return SN_ERR_LENGTH_MISMATCH;
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    size_t elements;
    if (mul_overflows(rows, cols, &elements) || elements >= (size_t(1) << 60)) return SN_ERR_OVERFLOW;
    if (elements == 0) return SN_OK;
    if (output == nullptr || bias == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (overlaps(output, elements, bias, bias_len)) return SN_ERR_ALIASING;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess)
        err = sn::launch_add_row_bias(output, int64_t(rows), int64_t(cols), 1, int64_t(elements), bias, ctx->stream);
    return status(err);
}

}  // extern "C"

namespace {

// sn_split_heads / sn_merge_heads: the reference's checks, then the copy.
int permute_heads(sn_context* ctx, bool split, const float* src, size_t src_len, float* dst, size_t dst_len,
                  const sn_head_layout* layout) {
    if (layout == nullptr) return SN_ERR_NULL_ARGUMENT;
    const sn_head_layout& l = *layout;
    const size_t limit = size_t(1) << 40;
    if (l.batch >= limit || l.time >= limit || l.heads >= limit || l.head_dim >= limit || l.width >= limit ||
        l.column_offset >= limit || l.time_capacity >= limit || l.time_offset >= limit)
        return SN_ERR_OVERFLOW;
    if (l.time_offset + l.time > l.time_capacity) return SN_ERR_SHAPE;
    size_t head_columns;
    if (mul_overflows(l.heads, l.head_dim, &head_columns)) return SN_ERR_OVERFLOW;
    if (l.column_offset + head_columns > l.width) return SN_ERR_SHAPE;
    // batch * time * width, batch * heads * time_capacity * head_dim and the moved count.
    size_t rows, packed_need, matrices, per_matrix, major_need, per_moved, moved;
    if (mul_overflows(l.batch, l.time, &rows) || mul_overflows(rows, l.width, &packed_need) ||
        mul_overflows(l.batch, l.heads, &matrices) || mul_overflows(l.time_capacity, l.head_dim, &per_matrix) ||
        mul_overflows(matrices, per_matrix, &major_need) || mul_overflows(l.time, l.head_dim, &per_moved) ||
        mul_overflows(matrices, per_moved, &moved))
        return SN_ERR_OVERFLOW;
    if (packed_need >= (size_t(1) << 60) || major_need >= (size_t(1) << 60)) return SN_ERR_OVERFLOW;
    const size_t packed_len = split ? src_len : dst_len;
    const size_t major_len = split ? dst_len : src_len;
    if (packed_len < packed_need || major_len < major_need) return SN_ERR_LENGTH_MISMATCH;
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (moved == 0) return SN_OK;
    if (src == nullptr || dst == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (overlaps(dst, split ? major_need : packed_need, src, split ? packed_need : major_need)) return SN_ERR_ALIASING;
    const sn::HeadLayoutArgs args{int64_t(l.batch),     int64_t(l.time),  int64_t(l.heads),
                                  int64_t(l.head_dim),  int64_t(l.width), int64_t(l.column_offset),
                                  int64_t(l.time_capacity), int64_t(l.time_offset)};
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess) err = sn::launch_permute_heads(split, src, dst, args, ctx->stream);
    return status(err);
}

}  // namespace

extern "C" {

int sn_split_heads(sn_context* ctx, const float* packed, size_t packed_len, float* head_major, size_t head_major_len,
                   const sn_head_layout* layout) {
    return permute_heads(ctx, true, packed, packed_len, head_major, head_major_len, layout);
}

int sn_merge_heads(sn_context* ctx, const float* head_major, size_t head_major_len, float* packed, size_t packed_len,
                   const sn_head_layout* layout) {
    return permute_heads(ctx, false, head_major, head_major_len, packed, packed_len, layout);
}

int sn_cross_entropy(sn_context* ctx, const float* logits, size_t rows, size_t cols, const uint32_t* targets,
                     size_t targets_len, const sn_cross_entropy_head* head, float* losses, size_t losses_len,
                     float* logits_grad, size_t grad_rows, size_t grad_cols) {
    if (head == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (grad_rows != rows || grad_cols != cols) return SN_ERR_SHAPE;
    if (head->column_offset > cols || head->classes > cols - head->column_offset) return SN_ERR_SHAPE;
    if (losses_len < rows) return SN_ERR_LENGTH_MISMATCH;
    size_t elements, target_span;
    if (mul_overflows(rows, cols, &elements) || elements >= (size_t(1) << 60) || rows >= (size_t(1) << 33) ||
        mul_overflows(rows, head->target_stride, &target_span))
        return SN_ERR_OVERFLOW;
    // Every row's target slot must exist: (rows - 1) * stride + offset < len.
    if (rows > 0 && (targets_len < target_span || head->target_offset >= targets_len ||
                     (rows - 1) * head->target_stride > targets_len - 1 - head->target_offset))
        return SN_ERR_LENGTH_MISMATCH;
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (rows == 0) return SN_OK;
    if (logits == nullptr || targets == nullptr || losses == nullptr || logits_grad == nullptr)
        return SN_ERR_NULL_ARGUMENT;
    if (overlaps(logits_grad, elements, logits, elements) || overlaps(losses, rows, logits, elements) ||
        overlaps(losses, rows, logits_grad, elements))
        return SN_ERR_ALIASING;
    sn::CrossEntropyArgs args;
    args.logits = logits;
    args.targets = targets;
    args.losses = losses;
    args.grad = logits_grad;
    args.rows = int64_t(rows);
    args.cols = int64_t(cols);
    args.column_offset = int64_t(head->column_offset);
    args.classes = int64_t(head->classes);
    args.target_stride = int64_t(head->target_stride);
    args.target_offset = int64_t(head->target_offset);
    args.grad_scale = head->grad_scale;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess) err = sn::launch_cross_entropy(args, ctx->stream);
    return status(err);
}

int sn_upload_tokens(sn_context* ctx, const uint32_t* host, size_t count, uint32_t** out) {
    static_assert(sizeof(uint32_t) == sizeof(float), "token ids travel as 4-byte words");
    return sn_upload(ctx, reinterpret_cast<const float*>(host), count, reinterpret_cast<float**>(out));
}

int sn_download_tokens(sn_context* ctx, const uint32_t* device, size_t count, uint32_t* host) {
    return sn_download(ctx, reinterpret_cast<const float*>(device), count, reinterpret_cast<float*>(host));
}

int sn_free_tokens(sn_context* ctx, uint32_t* buffer) { return sn_free(ctx, reinterpret_cast<float*>(buffer)); }

int sn_causal_softmax(sn_context* ctx, float* scores, size_t rows, size_t keys, size_t queries, float scale,
                      size_t query_offset) {
    if (queries == 0 || rows % queries != 0) return SN_ERR_SHAPE;
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    size_t elements;
    if (mul_overflows(rows, keys, &elements) || elements >= (size_t(1) << 60) || rows >= (size_t(1) << 33) ||
        query_offset >= (size_t(1) << 62))
        return SN_ERR_OVERFLOW;
    if (elements == 0) return SN_OK;
    if (scores == nullptr) return SN_ERR_NULL_ARGUMENT;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess)
        err = sn::launch_causal_softmax(scores, int64_t(rows), int64_t(queries), int64_t(keys), scale,
                                        int64_t(query_offset), ctx->stream);
    return status(err);
}

}  // extern "C"

namespace {

// Element counts an attention call's buffers must hold (SN_OK or the code).
struct AttentionNeed {
    size_t q = 0, kv = 0, o = 0, p = 0, kv_dense = 0;
};

int attention_need(const sn_attention_shape& a, AttentionNeed* need) {
    if (a.keys == 0) return SN_ERR_SHAPE;
    if (a.head_dim != 32 && a.head_dim != 64 && a.head_dim != 128) return SN_ERR_UNSUPPORTED;
    const size_t limit = size_t(1) << 60;
    size_t q_rows, kv_rows, q_last, kv_last, o_need, head_rows, p_rows, kv_dense;
    if (mul_overflows(a.queries, a.head_dim, &q_rows) || mul_overflows(a.keys, a.head_dim, &kv_rows) ||
        mul_overflows(a.heads - 1, a.q_stride, &q_last) || mul_overflows(a.heads - 1, a.kv_stride, &kv_last) ||
        mul_overflows(a.heads, q_rows, &o_need) || mul_overflows(a.heads, a.queries, &head_rows) ||
        mul_overflows(head_rows, a.keys, &p_rows) || mul_overflows(a.heads, kv_rows, &kv_dense) ||
        a.heads >= limit || a.queries >= limit || q_rows >= limit || kv_rows >= limit || q_last >= limit ||
        kv_last >= limit || o_need >= limit || p_rows >= limit || kv_dense >= limit ||
        a.query_offset >= (size_t(1) << 62))
        return SN_ERR_OVERFLOW;
    need->q = q_last + q_rows;
    need->kv = kv_last + kv_rows;
    need->o = o_need;
    need->p = p_rows;
    need->kv_dense = kv_dense;
    return SN_OK;
}

// sn_causal_attention and its variant with the row statistics.
int causal_attention_call(sn_context* ctx, const sn_attention_shape* shape, const float* q, size_t q_len,
                          const float* k, size_t k_len, const float* v, size_t v_len, float* out, size_t out_len,
                          float* probabilities, size_t probabilities_len, float* stats, size_t stats_len) {
    if (ctx == nullptr || shape == nullptr) return SN_ERR_NULL_ARGUMENT;
    const sn_attention_shape& a = *shape;
    if (a.heads == 0 || a.queries == 0) return SN_OK;
    AttentionNeed need;
    const int rc = attention_need(a, &need);
    if (rc != SN_OK) return rc;
    const size_t p_need = probabilities != nullptr ? need.p : 0;
    const size_t s_need = stats != nullptr ? 2 * need.o / a.head_dim : 0;
    if (q_len < need.q || k_len < need.kv || v_len < need.kv || out_len < need.o ||
        (probabilities != nullptr && probabilities_len < p_need) || (stats != nullptr && stats_len < s_need))
        return SN_ERR_LENGTH_MISMATCH;
    if (q == nullptr || k == nullptr || v == nullptr || out == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (overlaps(out, need.o, q, need.q) || overlaps(out, need.o, k, need.kv) || overlaps(out, need.o, v, need.kv))
        return SN_ERR_ALIASING;
    if (probabilities != nullptr &&
        (overlaps(probabilities, p_need, q, need.q) || overlaps(probabilities, p_need, k, need.kv) ||
         overlaps(probabilities, p_need, v, need.kv) || overlaps(probabilities, p_need, out, need.o)))
        return SN_ERR_ALIASING;
    if (stats != nullptr &&
        (overlaps(stats, s_need, q, need.q) || overlaps(stats, s_need, k, need.kv) ||
         overlaps(stats, s_need, v, need.kv) || overlaps(stats, s_need, out, need.o) ||
         overlaps(stats, s_need, probabilities, p_need)))
        return SN_ERR_ALIASING;
    const size_t q_rows = a.queries * a.head_dim, kv_rows = a.keys * a.head_dim;
    sn::CausalAttentionArgs args;
    args.q = q;
    args.k = k;
    args.v = v;
    args.o = out;
    args.p = probabilities;
    args.stats = stats;
    args.heads = int64_t(a.heads);
    args.queries = int64_t(a.queries);
    args.keys = int64_t(a.keys);
    args.head_dim = int64_t(a.head_dim);
    args.q_stride = int64_t(a.heads > 1 ? a.q_stride : q_rows);
    args.kv_stride = int64_t(a.heads > 1 ? a.kv_stride : kv_rows);
    args.query_offset = int64_t(a.query_offset);
    args.scale = a.scale;
    args.workspace = ctx->env.workspace;
    args.workspace_bytes = ctx->env.workspace_bytes;
    args.counters = ctx->env.counters;
    args.counter_count = ctx->env.counter_count;
    if (!sn::causal_attention_supported(args)) return SN_ERR_UNSUPPORTED;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess) err = sn::launch_causal_attention(args, ctx->stream);
    return status(err);
}

}  // namespace

extern "C" {

int sn_causal_attention(sn_context* ctx, const sn_attention_shape* shape, const float* q, size_t q_len,
                        const float* k, size_t k_len, const float* v, size_t v_len, float* out, size_t out_len,
                        float* probabilities, size_t probabilities_len) {
    return causal_attention_call(ctx, shape, q, q_len, k, k_len, v, v_len, out, out_len, probabilities,
                                 probabilities_len, nullptr, 0);
}

int sn_causal_attention_with_stats(sn_context* ctx, const sn_attention_shape* shape, const float* q, size_t q_len,
                                   const float* k, size_t k_len, const float* v, size_t v_len, float* out,
                                   size_t out_len, float* stats, size_t stats_len) {
    if (stats == nullptr) return SN_ERR_NULL_ARGUMENT;
    return causal_attention_call(ctx, shape, q, q_len, k, k_len, v, v_len, out, out_len, nullptr, 0, stats,
                                 stats_len);
}

int sn_causal_attention_backward(sn_context* ctx, const sn_attention_shape* shape, const float* q, size_t q_len,
                                 const float* k, size_t k_len, const float* v, size_t v_len, const float* out,
                                 size_t out_len, const float* d_out, size_t d_out_len, const float* stats,
                                 size_t stats_len, float* q_grad, size_t q_grad_len, float* k_grad,
                                 size_t k_grad_len, float* v_grad, size_t v_grad_len) {
    if (ctx == nullptr || shape == nullptr) return SN_ERR_NULL_ARGUMENT;
    const sn_attention_shape& a = *shape;
    if (a.heads == 0 || a.queries == 0) return SN_OK;
    AttentionNeed need;
    const int rc = attention_need(a, &need);
    if (rc != SN_OK) return rc;
    const size_t s_need = 2 * need.o / a.head_dim;
    if (q_len < need.q || k_len < need.kv || v_len < need.kv || out_len < need.o || d_out_len < need.q ||
        stats_len < s_need || q_grad_len < need.o || k_grad_len < need.kv_dense || v_grad_len < need.kv_dense)
        return SN_ERR_LENGTH_MISMATCH;
    if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || d_out == nullptr || stats == nullptr ||
        q_grad == nullptr || k_grad == nullptr || v_grad == nullptr)
        return SN_ERR_NULL_ARGUMENT;
    const float* inputs[6] = {q, k, v, out, d_out, stats};
    const size_t input_lens[6] = {need.q, need.kv, need.kv, need.o, need.q, s_need};
    float* outputs[3] = {q_grad, k_grad, v_grad};
    const size_t output_lens[3] = {need.o, need.kv_dense, need.kv_dense};
    for (int o = 0; o < 3; ++o) {
        for (int i = 0; i < 6; ++i)
            if (overlaps(outputs[o], output_lens[o], inputs[i], input_lens[i])) return SN_ERR_ALIASING;
        for (int p = o + 1; p < 3; ++p)
            if (overlaps(outputs[o], output_lens[o], outputs[p], output_lens[p])) return SN_ERR_ALIASING;
    }
    sn::AttentionBackwardArgs args;
    args.q = q;
    args.k = k;
    args.v = v;
    args.out = out;
    args.d_out = d_out;
    args.stats = stats;
    args.q_grad = q_grad;
    args.k_grad = k_grad;
    args.v_grad = v_grad;
    args.workspace = ctx->env.workspace;
    args.workspace_bytes = ctx->env.workspace_bytes;
    args.heads = int64_t(a.heads);
    args.queries = int64_t(a.queries);
    args.keys = int64_t(a.keys);
    args.head_dim = int64_t(a.head_dim);
    args.q_stride = int64_t(a.heads > 1 ? a.q_stride : a.queries * a.head_dim);
    args.kv_stride = int64_t(a.heads > 1 ? a.kv_stride : a.keys * a.head_dim);
    args.query_offset = int64_t(a.query_offset);
    args.scale = a.scale;
    if (size_t(a.heads) * 3 * ((a.queries + 3) / 4 * 4) * sizeof(float) > ctx->env.workspace_bytes)
        return SN_ERR_WORKSPACE;
    if (!sn::attention_backward_supported(args)) return SN_ERR_UNSUPPORTED;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess) err = sn::launch_attention_backward(args, ctx->stream);
    return status(err);
}

int sn_causal_attention_score_grad(sn_context* ctx, const sn_attention_shape* shape, const float* d_out,
                                   size_t d_out_len, const float* v, size_t v_len, const float* out, size_t out_len,
                                   const float* probabilities, size_t probabilities_len, float* grad,
                                   size_t grad_len, const float* k, size_t k_len, float* q_grad, size_t q_grad_len) {
    if (ctx == nullptr || shape == nullptr) return SN_ERR_NULL_ARGUMENT;
    const sn_attention_shape& a = *shape;
    if (a.heads == 0 || a.queries == 0) return SN_OK;
    if (a.keys == 0) return SN_ERR_SHAPE;
    if (a.head_dim != 32 && a.head_dim != 64 && a.head_dim != 128) return SN_ERR_UNSUPPORTED;
    const size_t limit = size_t(1) << 60;
    size_t q_rows, kv_rows, q_last, kv_last, o_need, head_rows, p_rows;
    if (mul_overflows(a.queries, a.head_dim, &q_rows) || mul_overflows(a.keys, a.head_dim, &kv_rows) ||
        mul_overflows(a.heads - 1, a.q_stride, &q_last) || mul_overflows(a.heads - 1, a.kv_stride, &kv_last) ||
        mul_overflows(a.heads, q_rows, &o_need) || mul_overflows(a.heads, a.queries, &head_rows) ||
        mul_overflows(head_rows, a.keys, &p_rows) || a.heads >= limit || a.queries >= limit || q_rows >= limit ||
        kv_rows >= limit || q_last >= limit || kv_last >= limit || o_need >= limit || p_rows >= limit ||
        a.query_offset >= (size_t(1) << 62))
        return SN_ERR_OVERFLOW;
    const size_t d_need = q_last + q_rows, kv_need = kv_last + kv_rows;
    if (d_out_len < d_need || v_len < kv_need || out_len < o_need || probabilities_len < p_rows || grad_len < p_rows ||
        (q_grad != nullptr && (k_len < kv_need || q_grad_len < o_need)))
        return SN_ERR_LENGTH_MISMATCH;
    if (d_out == nullptr || v == nullptr || out == nullptr || probabilities == nullptr || grad == nullptr ||
        (q_grad != nullptr && k == nullptr))
        return SN_ERR_NULL_ARGUMENT;
    if (overlaps(grad, p_rows, d_out, d_need) || overlaps(grad, p_rows, v, kv_need) ||
        overlaps(grad, p_rows, out, o_need) || overlaps(grad, p_rows, probabilities, p_rows))
        return SN_ERR_ALIASING;
    if (q_grad != nullptr &&
        (overlaps(q_grad, o_need, d_out, d_need) || overlaps(q_grad, o_need, v, kv_need) ||
         overlaps(q_grad, o_need, out, o_need) || overlaps(q_grad, o_need, probabilities, p_rows) ||
         overlaps(q_grad, o_need, grad, p_rows) || overlaps(q_grad, o_need, k, kv_need) ||
         overlaps(grad, p_rows, k, kv_need)))
        return SN_ERR_ALIASING;
    sn::AttentionScoreGradArgs args;
    args.d_out = d_out;
    args.v = v;
    args.out = out;
    args.p = probabilities;
    args.grad = grad;
    args.k = k;
    args.q_grad = q_grad;
    args.scale = a.scale;
    args.heads = int64_t(a.heads);
    args.queries = int64_t(a.queries);
    args.keys = int64_t(a.keys);
    args.head_dim = int64_t(a.head_dim);
    args.q_stride = int64_t(a.heads > 1 ? a.q_stride : q_rows);
    args.kv_stride = int64_t(a.heads > 1 ? a.kv_stride : kv_rows);
    args.query_offset = int64_t(a.query_offset);
    if (!sn::attention_score_grad_supported(args)) return SN_ERR_UNSUPPORTED;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess) err = sn::launch_attention_score_grad(args, ctx->stream);
    return status(err);
}

int sn_matmul_column_sums(sn_context* ctx, const sn_matmul_spec* spec, const float* left, size_t left_len,
                          const float* right, size_t right_len, float* output, size_t output_len, float* sums,
                          size_t sums_len) {
    int rc = sn_matmul_validate(spec, left_len, right_len, output_len);
    if (rc != SN_OK) return rc;
    if (spec->right_storage != SN_ROW_MAJOR || spec->batch_count != 1) return SN_ERR_UNSUPPORTED;
    if (sums_len != spec->cols) return SN_ERR_LENGTH_MISMATCH;
    if (ctx == nullptr || (sums == nullptr && sums_len > 0)) return SN_ERR_NULL_ARGUMENT;
    rc = sn::check_matmul_call(spec, left, left_len, right, right_len, nullptr, 0, output, output_len);
    if (rc != SN_OK) return rc;
    if (spec->cols == 0) return SN_OK;
    const size_t right_used = spec->inner * spec->cols;
    if (overlaps(sums, sums_len, output, spec->rows * spec->cols) || overlaps(sums, sums_len, right, right_used) ||
        overlaps(sums, sums_len, left, spec->rows * spec->inner))
        return SN_ERR_ALIASING;

    sn::Problem p = sn::problem_of(spec, left, right, output, nullptr);
    p.column_sums = sums;
    const uint32_t kernel = sn::kernel_for(ctx->kernel, spec->precision);
    if (sn::describe_matmul_column_sums(p, kernel, ctx->env).workspace_bytes > ctx->env.workspace_bytes)
        return SN_ERR_WORKSPACE;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess) err = sn::launch_matmul_column_sums(p, kernel, ctx->env, ctx->stream);
    return status(err);
}

int sn_softmax_backward(sn_context* ctx, const float* probabilities, size_t probability_rows,
                        size_t probability_cols, float* grad, size_t grad_rows, size_t grad_cols) {
    if (probability_rows != grad_rows || probability_cols != grad_cols) return SN_ERR_SHAPE;
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    size_t elements;
    if (mul_overflows(grad_rows, grad_cols, &elements) || elements >= (size_t(1) << 60) ||
        grad_rows >= (size_t(1) << 33))
        return SN_ERR_OVERFLOW;
    if (elements == 0) return SN_OK;
    if (probabilities == nullptr || grad == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (overlaps(grad, elements, probabilities, elements)) return SN_ERR_ALIASING;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess)
        err = sn::launch_softmax_backward(probabilities, grad, int64_t(grad_rows), int64_t(grad_cols), ctx->stream);
    return status(err);
}

int sn_accumulate_column_sums(sn_context* ctx, const float* input, size_t rows, size_t cols, float* sums,
                              size_t sums_len) {
    if (sums_len != cols) return SN_ERR_LENGTH_MISMATCH;
    if (ctx == nullptr) return SN_ERR_NULL_ARGUMENT;
    size_t elements;
    if (mul_overflows(rows, cols, &elements) || elements >= (size_t(1) << 60) || cols >= kMaxDimension ||
        rows >= kMaxDimension)
        return SN_ERR_OVERFLOW;
    if (cols == 0) return SN_OK;
    if (sums == nullptr || (elements > 0 && input == nullptr)) return SN_ERR_NULL_ARGUMENT;
    if (elements == 0) return SN_OK;  // every column sums to 0: sums unchanged
    if (overlaps(sums, sums_len, input, elements)) return SN_ERR_ALIASING;
    if (sn::column_sums_workspace_bytes(int64_t(rows), int64_t(cols), ctx->env) > ctx->env.workspace_bytes)
        return SN_ERR_WORKSPACE;
    hipError_t err = hipSetDevice(ctx->device);
    if (err == hipSuccess)
        err = sn::launch_column_sums(input, int64_t(rows), int64_t(cols), sums, ctx->env, ctx->stream);
    return status(err);
}

const char* sn_status_string(int code) {
    switch (code) {
        case SN_OK:
            return "success";
        case SN_ERR_NULL_ARGUMENT:
            return "a required pointer argument is null";
        case SN_ERR_LEFT_TOO_SMALL:
            return "matmul: left operand too small";
        case SN_ERR_RIGHT_TOO_SMALL:
            return "matmul: right operand too small";
        case SN_ERR_OUTPUT_TOO_SMALL:
            return "matmul: output too small";
        case SN_ERR_EMPTY_BATCH:
            return "matmul: batch count is zero";
        case SN_ERR_OVERFLOW:
            return "matmul: a size or offset overflows";
        case SN_ERR_UNSUPPORTED:
            return "matmul: unsupported spec field value";
        case SN_ERR_ALIASING:
            return "matmul: output overlaps an input";
        case SN_ERR_NO_DEVICE:
            return "no GPU at the requested ordinal";
        case SN_ERR_WORKSPACE:
            return "matmul: split-K workspace too small";
        case SN_ERR_LENGTH_MISMATCH:
            return "bias or sums length must equal the matrix's columns";
        case SN_ERR_SHAPE:
            return "row-wise kernel: rows must be a multiple of queries, or the shapes differ";
        default:
            break;
    }
    if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
    return "unknown status";
}

}  // extern "C"

// Linear's bias kernels, the steps on either side of its products
// (crates/staleynet-model/src/layers/linear.rs:43-63):
//
//  * add_row_bias (kernels/elementwise.rs:62-68): output[r, c] += bias[c]
//    after the forward product. One f32 add per element, as the reference
//    does it, so the result is bit-identical. HBM-bound: 8 bytes per
//    element (read and write the output); 16-byte accesses when the column
//    count and the pointers allow, the bias values of a lane's 4 columns
//    read once per pass through L2.
//  * accumulate_column_sums (kernels/elementwise.rs:78-93): sums[c] += the
//    sum of column c, the bias gradient beside the weight-gradient product.
//    The reference gives each column one thread that walks all rows in
//    order (at M = 32768: 2304 threads reading one float each per step, a
//    small fraction of the machine). Here the work is split two ways: a
//    workgroup owns 64 columns (a lane 4, one 16-byte load per row) and a
//    slice of rows, which its 4 row lanes x 4 waves take in turn; the lanes'
//    and then the waves' sums are added in a fixed order, and a second
//    kernel adds the slices' sums (eight accumulators, in slice order) and
//    adds the result to `sums`. The order is fixed, so every run gives the
//    same bits; it differs from the reference's row-order sum only in
//    rounding (the tests bound the gap).
//    HBM-bound: 4 bytes per element read once.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "gemm_internal.h"

namespace sn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

// Four consecutive elements of one row per thread (cols % 4 == 0, 16-byte
// aligned output and bias): a grid-stride loop over the batch's vectors.
__global__ __launch_bounds__(kThreads) void add_row_bias4_kernel(f32x4* __restrict__ out, int64_t vectors_per_matrix,
                                                                 int64_t batch, int64_t stride4, int64_t cols4,
                                                                 const f32x4* __restrict__ bias) {
    const int64_t total = vectors_per_matrix * batch;
    for (int64_t i = blockIdx.x * int64_t(kThreads) + threadIdx.x; i < total; i += int64_t(gridDim.x) * kThreads) {
        const int64_t b = i / vectors_per_matrix;
        const int64_t v = i % vectors_per_matrix;
        f32x4* dst = out + b * stride4 + v;
        *dst = *dst + bias[v % cols4];
    }
}

__global__ __launch_bounds__(kThreads) void add_row_bias_kernel(float* __restrict__ out, int64_t per_matrix,
                                                                int64_t batch, int64_t stride, int64_t cols,
                                                                const float* __restrict__ bias) {
    const int64_t total = per_matrix * batch;
    for (int64_t i = blockIdx.x * int64_t(kThreads) + threadIdx.x; i < total; i += int64_t(gridDim.x) * kThreads) {
        const int64_t b = i / per_matrix;
        const int64_t e = i % per_matrix;
        float* dst = out + b * stride + e;
        *dst = *dst + bias[e % cols];
    }
}

// Column sums: a workgroup owns 64 columns and a slice of rows. A lane owns 4
// columns (16 lanes cover a 256-byte row piece) and one of 4 row lanes, so a
// wave load covers 4 rows x 64 columns and the workgroup's 4 waves take 16
// consecutive rows per round; kUnroll rounds of loads are in flight before
// they are added.
constexpr int kColumns = 64;
constexpr int kUnroll = 8;

// Sum of columns [c0, c0 + 64) over rows [r0, r1): each lane sums its rows in
// order, the 4 row lanes of a wave are added (xor 16, then 32), then the 4
// waves in wave order through LDS. Writes partial[slice][c] (columns past
// `cols` are not written).
template <bool VECTOR>
__global__ __launch_bounds__(kThreads) void column_slice_sums_kernel(const float* __restrict__ in, int64_t rows,
                                                                     int64_t cols, int64_t rows_per_slice,
                                                                     float* __restrict__ partial) {
    __shared__ f32x4 wave_sums[kThreads / 64][16];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col_lane = lane & 15;
    const int row_lane = lane >> 4;
    const int64_t c = int64_t(blockIdx.x) * kColumns + 4 * col_lane;
    const int64_t slice = blockIdx.y;
    const int64_t r0 = slice * rows_per_slice;
    const int64_t r1 = std::min<int64_t>(rows, r0 + rows_per_slice);
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
    auto load = [&](int64_t r) -> f32x4 {
        const float* src = in + r * cols + c;
        if constexpr (VECTOR) {
            if (c < cols) return *reinterpret_cast<const f32x4*>(src);
            return f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (c + j < cols) v[j] = src[j];
            return v;
        }
    };
    int64_t r = r0 + 4 * wave + row_lane;
    for (; r + 16 * (kUnroll - 1) < r1; r += 16 * kUnroll) {
        f32x4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = load(r + 16 * u);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) sum = sum + v[u];
    }
    for (; r < r1; r += 16) sum = sum + load(r);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        sum[j] = sum[j] + __shfl_xor(sum[j], 16);
        sum[j] = sum[j] + __shfl_xor(sum[j], 32);
    }
    if (row_lane == 0) wave_sums[wave][col_lane] = sum;
    __syncthreads();
    if (threadIdx.x < 16) {
        f32x4 total = wave_sums[0][threadIdx.x];
#pragma unroll
        for (int w = 1; w < kThreads / 64; ++w) total = total + wave_sums[w][threadIdx.x];
        float* dst = partial + slice * cols + c;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (c + j < cols) dst[j] = total[j];
    }
}

// sums[c] += the slices' sums. A workgroup takes 32 columns; its 8 groups
// of 32 threads take slices g, g + 8, g + 16, ... of them (up to 16 loads in
// flight a thread, added in slice order), and the 8 group sums are then
// added in group order: a fixed order. Split-K leaves 2-32 slices; the bf16
// staging pass of a 32768-deep dY, 512.
constexpr int kFinishCols = 32;
constexpr int kFinishGroups = kThreads / kFinishCols;
__global__ __launch_bounds__(kThreads) void column_sums_finish_kernel(const float* __restrict__ partial,
                                                                      int64_t slices, int64_t cols,
                                                                      float* __restrict__ sums) {
    __shared__ float group_sums[kFinishGroups][kFinishCols];
    const int lane_col = threadIdx.x % kFinishCols;
    const int group = threadIdx.x / kFinishCols;
    const int64_t c = blockIdx.x * int64_t(kFinishCols) + lane_col;
    float acc = 0.f;
    if (c < cols) {
        constexpr int kInFlight = 16;
        int64_t s = group;
        for (; s + (kInFlight - 1) * kFinishGroups < slices; s += kInFlight * kFinishGroups) {
            float v[kInFlight];
#pragma unroll
            for (int j = 0; j < kInFlight; ++j) v[j] = partial[(s + j * kFinishGroups) * cols + c];
#pragma unroll
            for (int j = 0; j < kInFlight; ++j) acc = acc + v[j];
        }
        for (; s < slices; s += kFinishGroups) acc = acc + partial[s * cols + c];
    }
    group_sums[group][lane_col] = acc;
    __syncthreads();
    if (group == 0 && c < cols) {
        float total = group_sums[0][lane_col];
#pragma unroll
        for (int q = 1; q < kFinishGroups; ++q) total = total + group_sums[q][lane_col];
        sums[c] = sums[c] + total;
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Slices of rows for about 2 workgroups per CU, each at least 256 rows,
// capped by the workspace.
int64_t slices_for(int64_t rows, int64_t cols, const Env& env) {
    const int64_t column_blocks = (cols + kColumns - 1) / kColumns;
    int64_t slices = std::max<int64_t>(1, (int64_t(env.cu_count) * 2 + column_blocks - 1) / column_blocks);
    slices = std::min<int64_t>(slices, std::max<int64_t>(1, rows / 256));
    const int64_t fit = int64_t(env.workspace_bytes / (sizeof(float) * size_t(std::max<int64_t>(cols, 1))));
    return std::max<int64_t>(1, std::min<int64_t>({slices, fit, 65535}));
}

}  // namespace

hipError_t launch_add_row_bias(float* out, int64_t rows, int64_t cols, int64_t batch, int64_t stride,
                               const float* bias, hipStream_t stream) {
    const int64_t per_matrix = rows * cols;
    if (per_matrix == 0 || batch == 0) return hipSuccess;
    const int64_t total = per_matrix * batch;
    if (cols % 4 == 0 && stride % 4 == 0 && aligned16(out) && aligned16(bias)) {
        const int64_t grid = std::min<int64_t>((total / 4 + kThreads - 1) / kThreads, 8192);
        hipLaunchKernelGGL(add_row_bias4_kernel, dim3(unsigned(grid)), dim3(kThreads), 0, stream,
                           reinterpret_cast<f32x4*>(out), per_matrix / 4, batch, stride / 4, cols / 4,
                           reinterpret_cast<const f32x4*>(bias));
    } else {
        const int64_t grid = std::min<int64_t>((total + kThreads - 1) / kThreads, 8192);
        hipLaunchKernelGGL(add_row_bias_kernel, dim3(unsigned(grid)), dim3(kThreads), 0, stream, out, per_matrix,
                           batch, stride, cols, bias);
    }
    return hipGetLastError();
}

size_t column_sums_workspace_bytes(int64_t rows, int64_t cols, const Env& env) {
    if (rows == 0 || cols == 0) return 0;
    return size_t(slices_for(rows, cols, env)) * size_t(cols) * sizeof(float);
}

hipError_t launch_column_sums(const float* in, int64_t rows, int64_t cols, float* sums, const Env& env,
                              hipStream_t stream) {
    if (rows == 0 || cols == 0) return hipSuccess;
    const int64_t slices = slices_for(rows, cols, env);
    const int64_t rows_per_slice = (rows + slices - 1) / slices;
    const dim3 grid(unsigned((cols + kColumns - 1) / kColumns), unsigned(slices));
    if (cols % 4 == 0 && aligned16(in))
        hipLaunchKernelGGL((column_slice_sums_kernel<true>), grid, dim3(kThreads), 0, stream, in, rows, cols,
                           rows_per_slice, env.workspace);
    else
        hipLaunchKernelGGL((column_slice_sums_kernel<false>), grid, dim3(kThreads), 0, stream, in, rows, cols,
                           rows_per_slice, env.workspace);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_column_sums_finish(env.workspace, slices, cols, sums, stream);
}

hipError_t launch_column_sums_finish(const float* partial, int64_t slices, int64_t cols, float* sums,
                                     hipStream_t stream) {
    hipLaunchKernelGGL(column_sums_finish_kernel, dim3(unsigned((cols + kFinishCols - 1) / kFinishCols)),
                       dim3(kThreads), 0, stream, partial, slices, cols, sums);
    return hipGetLastError();
}

}  // namespace sn

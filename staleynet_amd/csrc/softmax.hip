// The row-wise kernels between the attention products
// (crates/staleynet-model/src/layers/attention.rs:210, :249):
//
//  * causal_softmax (kernels/attention.rs:140-183; CPU form reference.rs:
//    100-119), in place on the scores S = Q K^T: row r of each block of
//    `queries` rows sees keys 0 ..= (r mod queries) + query_offset; those get
//    exp(s * scale - max) / sum, the rest 0. Products, differences and
//    quotients are rounded separately (no contraction), as the reference
//    rounds them; exp is the device's expf.
//  * softmax_backward (kernels/attention.rs:185-207; reference.rs:121-137),
//    in place on the gradient: g <- p * (g - sum(g * p)) per row.
//
// One wave per row. Rows of up to 4096 aligned columns are held in
// registers (16-byte loads, VECTORS float4 per lane: one read and one write
// of each element; causal_softmax reads only the visible keys). The row's
// max and sums are reduced across the wave by a butterfly (xor 32, 16, .., 1):
// a fixed order, so every run gives the same bits; the order differs from
// the reference's sequential CPU loop, so parity is to the fp32 tolerance.
// Longer or unaligned rows take a multi-pass loop, one element per lane.
// HBM-bound: causal_softmax moves 4 bytes per visible element read plus 4 per
// element written; softmax_backward 12 bytes per element.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "gemm_internal.h"

namespace sn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Rows (one wave each) per workgroup. Two measured 3-5 % faster than four on
// 192 x 2048 x 2048 scores: causal softmax 0.92-0.94 ms against 0.95-0.97,
// its backward 1.72-1.75 against 1.80-1.84.
constexpr int kWaves = 2;
constexpr int kMaxVectors = 16;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int step = 32; step > 0; step >>= 1) v = fmaxf(v, __shfl_xor(v, step));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int step = 32; step > 0; step >>= 1) v = v + __shfl_xor(v, step);
    return v;
}

// Register-resident rows: float4 q = lane + 64 i (i < VECTORS) of the row.
template <int VECTORS>
__global__ __launch_bounds__(64 * kWaves) void causal_softmax_vector_kernel(float* __restrict__ scores, int64_t rows,
                                                                            int64_t queries, int64_t keys,
                                                                            float scale, int64_t query_offset) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t visible = std::min<int64_t>(row % queries + query_offset + 1, keys);
    f32x4* row4 = reinterpret_cast<f32x4*>(scores + row * keys);
    f32x4 v[VECTORS];
    float maximum = -INFINITY;
#pragma unroll
    for (int i = 0; i < VECTORS; ++i) {
        const int64_t k = 4 * (lane + 64 * i);
        v[i] = k < visible ? row4[lane + 64 * i] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (k + j < visible) maximum = fmaxf(maximum, v[i][j] * scale);
    }
    maximum = wave_max(maximum);
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < VECTORS; ++i) {
        const int64_t k = 4 * (lane + 64 * i);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float shifted = v[i][j] * scale - maximum;
            v[i][j] = k + j < visible ? expf(shifted) : 0.f;
            total = total + v[i][j];
        }
    }
    total = wave_sum(total);
#pragma unroll
    for (int i = 0; i < VECTORS; ++i) {
        const int64_t k = 4 * (lane + 64 * i);
        if (k < keys) {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[i][j] = v[i][j] / total;
            row4[lane + 64 * i] = v[i];
        }
    }
}

// Any row length or alignment: three passes over the row (max, exponentials
// stored in place with their sum, normalisation), one element per lane.
__global__ __launch_bounds__(64 * kWaves) void causal_softmax_loop_kernel(float* __restrict__ scores, int64_t rows,
                                                                          int64_t queries, int64_t keys, float scale,
                                                                          int64_t query_offset) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t visible = std::min<int64_t>(row % queries + query_offset + 1, keys);
    float* values = scores + row * keys;
    float maximum = -INFINITY;
    for (int64_t k = lane; k < visible; k += 64) maximum = fmaxf(maximum, values[k] * scale);
    maximum = wave_max(maximum);
    float total = 0.f;
    for (int64_t k = lane; k < visible; k += 64) {
        const float shifted = values[k] * scale - maximum;
        const float e = expf(shifted);
        values[k] = e;
        total = total + e;
    }
    total = wave_sum(total);
    for (int64_t k = lane; k < keys; k += 64) values[k] = k < visible ? values[k] / total : 0.f;
}

template <int VECTORS>
__global__ __launch_bounds__(64 * kWaves) void softmax_backward_vector_kernel(const float* __restrict__ probabilities,
                                                                              float* __restrict__ grad, int64_t rows,
                                                                              int64_t cols) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    const f32x4* p4 = reinterpret_cast<const f32x4*>(probabilities + row * cols);
    f32x4* g4 = reinterpret_cast<f32x4*>(grad + row * cols);
    f32x4 p[VECTORS], g[VECTORS];
    float projection = 0.f;
#pragma unroll
    for (int i = 0; i < VECTORS; ++i) {
        const int64_t c = 4 * (lane + 64 * i);
        const bool ok = c < cols;
        p[i] = ok ? p4[lane + 64 * i] : f32x4{0.f, 0.f, 0.f, 0.f};
        g[i] = ok ? g4[lane + 64 * i] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < VECTORS; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float product = g[i][j] * p[i][j];
            projection = projection + product;
        }
    projection = wave_sum(projection);
#pragma unroll
    for (int i = 0; i < VECTORS; ++i) {
        if (4 * (lane + 64 * i) < cols) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float difference = g[i][j] - projection;
                g[i][j] = p[i][j] * difference;
            }
            g4[lane + 64 * i] = g[i];
        }
    }
}

__global__ __launch_bounds__(64 * kWaves) void softmax_backward_loop_kernel(const float* __restrict__ probabilities,
                                                                            float* __restrict__ grad, int64_t rows,
                                                                            int64_t cols) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* p = probabilities + row * cols;
    float* g = grad + row * cols;
    float projection = 0.f;
    for (int64_t c = lane; c < cols; c += 64) {
        const float product = g[c] * p[c];
        projection = projection + product;
    }
    projection = wave_sum(projection);
    for (int64_t c = lane; c < cols; c += 64) {
        const float difference = g[c] - projection;
        g[c] = p[c] * difference;
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// float4 per lane a register-resident row of `cols` needs (0: too long).
int vectors_for(int64_t cols) {
    const int64_t vectors = (cols + 255) / 256;
    for (int v : {1, 2, 4, 8, 16})
        if (vectors <= v) return v;
    return 0;
}

template <class Launch>
hipError_t dispatch_vectors(int vectors, Launch&& launch) {
    switch (vectors) {
        case 1: launch(std::integral_constant<int, 1>{}); break;
        case 2: launch(std::integral_constant<int, 2>{}); break;
        case 4: launch(std::integral_constant<int, 4>{}); break;
        case 8: launch(std::integral_constant<int, 8>{}); break;
        default: launch(std::integral_constant<int, kMaxVectors>{}); break;
    }
    return hipGetLastError();
}

dim3 grid_for(int64_t rows) { return dim3(unsigned((rows + kWaves - 1) / kWaves)); }

}  // namespace

hipError_t launch_causal_softmax(float* scores, int64_t rows, int64_t queries, int64_t keys, float scale,
                                 int64_t query_offset, hipStream_t stream) {
    if (rows == 0 || keys == 0) return hipSuccess;
    const int vectors = vectors_for(keys);
    if (vectors > 0 && keys % 4 == 0 && aligned16(scores)) {
        return dispatch_vectors(vectors, [&](auto v) {
            hipLaunchKernelGGL((causal_softmax_vector_kernel<decltype(v)::value>), grid_for(rows), dim3(64 * kWaves),
                               0, stream, scores, rows, queries, keys, scale, query_offset);
        });
    }
    hipLaunchKernelGGL(causal_softmax_loop_kernel, grid_for(rows), dim3(64 * kWaves), 0, stream, scores, rows,
                       queries, keys, scale, query_offset);
    return hipGetLastError();
}

hipError_t launch_softmax_backward(const float* probabilities, float* grad, int64_t rows, int64_t cols,
                                   hipStream_t stream) {
    if (rows == 0 || cols == 0) return hipSuccess;
    const int vectors = vectors_for(cols);
    if (vectors > 0 && cols % 4 == 0 && aligned16(probabilities) && aligned16(grad)) {
        return dispatch_vectors(vectors, [&](auto v) {
            hipLaunchKernelGGL((softmax_backward_vector_kernel<decltype(v)::value>), grid_for(rows),
                               dim3(64 * kWaves), 0, stream, probabilities, grad, rows, cols);
        });
    }
    hipLaunchKernelGGL(softmax_backward_loop_kernel, grid_for(rows), dim3(64 * kWaves), 0, stream, probabilities,
                       grad, rows, cols);
    return hipGetLastError();
}

}  // namespace sn

// Softmax cross-entropy of one classifier head with its gradient: the head
// product's consumer (crates/staleynet-model/src/training.rs:208-239 calls it
// once per codebook; kernel kernels/loss.rs:54-97, CPU form reference.rs:
// 139-166). For the head's `classes` columns of each logits row and target y:
//   loss = log_partition - z_y,  log_partition = max + log(sum exp(z - max)),
//   grad = (exp(z - log_partition) - onehot(y)) * grad_scale,
// written into the head's columns of the gradient (other columns are left
// alone); an empty target (0xFFFFFFFF) gives loss 0 and gradient 0.
//
// One wave per row, as the softmax kernels: the head's logits held in
// registers (16-byte loads) when they are at most 4096 aligned columns,
// else three passes; the row's max and sum are reduced by a butterfly (a
// fixed order). Differences and products are rounded separately, as the
// reference rounds them; e^d of a rounded difference d is 2^(d log2 e) on the
// transcendental unit (v_exp_f32, about 1 ulp): rounding d log2 e adds at
// most |d| 2^-24 to the exponent, a relative error under 2e-6 for every term
// above e^-20 (the library expf took about 12 instructions, and two per
// element made the kernel compute-bound); the log is logf. A target
// outside the head (neither a class nor empty) gives a NaN loss and no
// onehot term. HBM-bound: 8 bytes per head element (read the logits, write
// the gradient).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "gemm_internal.h"

namespace sn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Two one-row waves per workgroup: over the head's 16 calls 0.92-0.95 ms
// against 0.94-0.98 with four, 0.94-1.03 with one and 1.03 with eight.
constexpr int kWaves = 2;
constexpr uint32_t kEmptyToken = 0xFFFFFFFFu;

constexpr float kLog2e = 1.44269504088896340736f;
__device__ __forceinline__ float exp_of(float d) { return __builtin_amdgcn_exp2f(d * kLog2e); }

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

template <int VECTORS>
__global__ __launch_bounds__(64 * kWaves) void cross_entropy_vector_kernel(CrossEntropyArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const float* z = a.logits + row * a.cols + a.column_offset;
    float* g = a.grad + row * a.cols + a.column_offset;
    const f32x4* z4 = reinterpret_cast<const f32x4*>(z);
    f32x4* g4 = reinterpret_cast<f32x4*>(g);
    const uint32_t target = a.targets[row * a.target_stride + a.target_offset];
    if (target == kEmptyToken) {
#pragma unroll
        for (int i = 0; i < VECTORS; ++i)
            if (4 * (lane + 64 * i) < a.classes) g4[lane + 64 * i] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (lane == 0) a.losses[row] = 0.f;
        return;
    }
    f32x4 v[VECTORS];
    float maximum = -INFINITY;
#pragma unroll
    for (int i = 0; i < VECTORS; ++i) {
        const bool ok = 4 * (lane + 64 * i) < a.classes;
        v[i] = ok ? z4[lane + 64 * i] : f32x4{0.f, 0.f, 0.f, 0.f};
        if (ok) maximum = fmaxf(fmaxf(maximum, fmaxf(v[i][0], v[i][1])), fmaxf(v[i][2], v[i][3]));
    }
    maximum = wave_max(maximum);
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < VECTORS; ++i)
        if (4 * (lane + 64 * i) < a.classes) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float shifted = v[i][j] - maximum;
                total = total + exp_of(shifted);
            }
        }
    total = wave_sum(total);
    const float log_partition = maximum + logf(total);
    if (lane == 0) a.losses[row] = target < uint32_t(a.classes) ? log_partition - z[target] : NAN;
#pragma unroll
    for (int i = 0; i < VECTORS; ++i) {
        const int64_t c = 4 * (lane + 64 * i);
        if (c < a.classes) {
            f32x4 out;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float shifted = v[i][j] - log_partition;
                const float one_hot = c + j == int64_t(target) ? 1.f : 0.f;
                const float difference = exp_of(shifted) - one_hot;
                out[j] = difference * a.grad_scale;
            }
            g4[lane + 64 * i] = out;
        }
    }
}

__global__ __launch_bounds__(64 * kWaves) void cross_entropy_loop_kernel(CrossEntropyArgs a) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const float* z = a.logits + row * a.cols + a.column_offset;
    float* g = a.grad + row * a.cols + a.column_offset;
    const uint32_t target = a.targets[row * a.target_stride + a.target_offset];
    if (target == kEmptyToken) {
        for (int64_t c = lane; c < a.classes; c += 64) g[c] = 0.f;
        if (lane == 0) a.losses[row] = 0.f;
        return;
    }
    float maximum = -INFINITY;
    for (int64_t c = lane; c < a.classes; c += 64) maximum = fmaxf(maximum, z[c]);
    maximum = wave_max(maximum);
    float total = 0.f;
    for (int64_t c = lane; c < a.classes; c += 64) {
        const float shifted = z[c] - maximum;
        total = total + exp_of(shifted);
    }
    total = wave_sum(total);
    const float log_partition = maximum + logf(total);
    if (lane == 0) a.losses[row] = target < uint32_t(a.classes) ? log_partition - z[target] : NAN;
    for (int64_t c = lane; c < a.classes; c += 64) {
        const float shifted = z[c] - log_partition;
        const float one_hot = c == int64_t(target) ? 1.f : 0.f;
        const float difference = exp_of(shifted) - one_hot;
        g[c] = difference * a.grad_scale;
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

hipError_t launch_cross_entropy(const CrossEntropyArgs& a, hipStream_t stream) {
    if (a.rows == 0) return hipSuccess;
    const dim3 grid(unsigned((a.rows + kWaves - 1) / kWaves));
    const int64_t vectors = (a.classes + 255) / 256;
    const bool vector_ok = a.classes % 4 == 0 && a.cols % 4 == 0 && a.column_offset % 4 == 0 &&
                           aligned16(a.logits) && aligned16(a.grad) && vectors <= 16;
    if (vector_ok) {
        if (vectors <= 1)
            hipLaunchKernelGGL(cross_entropy_vector_kernel<1>, grid, dim3(64 * kWaves), 0, stream, a);
        else if (vectors <= 2)
            hipLaunchKernelGGL(cross_entropy_vector_kernel<2>, grid, dim3(64 * kWaves), 0, stream, a);
        else if (vectors <= 4)
            hipLaunchKernelGGL(cross_entropy_vector_kernel<4>, grid, dim3(64 * kWaves), 0, stream, a);
        else if (vectors <= 8)
            hipLaunchKernelGGL(cross_entropy_vector_kernel<8>, grid, dim3(64 * kWaves), 0, stream, a);
        else
            hipLaunchKernelGGL(cross_entropy_vector_kernel<16>, grid, dim3(64 * kWaves), 0, stream, a);
    } else {
        hipLaunchKernelGGL(cross_entropy_loop_kernel, grid, dim3(64 * kWaves), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace sn

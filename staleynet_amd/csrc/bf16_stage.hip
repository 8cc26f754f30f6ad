// Operand staging for the bf16 products: an fp32 operand rounded to bf16
// (v_cvt_pk_bf16_f32, nearest-even: the rounding the bf16 kernels apply as
// they read their fp32 stages) and laid out K-contiguous,
// dst[batch][row][0 .. kp) with kp = K rounded up to 8 and zeros past K, so
// that the product's matrix cores read 8 consecutive k of a row as one
// 16-byte slot whatever the operand's stored layout.
//
//  * K-contiguous source (element (r, k) at src[r * ld + k]): a thread
//    converts 8 consecutive k of a row (two 16-byte loads, one 16-byte
//    store).
//  * Row-contiguous source (element (r, k) at src[k * ld + r]): 64 x 64
//    tiles transposed through LDS. Loads read 64 consecutive rows of each k
//    (16 bytes a lane); 8 consecutive lanes then write one row's 64 k (128
//    bytes). The LDS pitch of 65 floats keeps both sides conflict-free.
//    Optionally (SUMS) each tile also leaves its 64 rows' fp32 sums over its
//    64 k, in k order (Linear's bias gradient of a dY staged for the weight
//    gradient: the rows here are dY's columns).
//
// The same rounding can also write the 256 x 256 bf16 kernel's blocked layout
// (launch_stage_bf16_blocks): per 32-deep step of K, the operand's rows of 32
// k one after another, rows padded to a multiple of 256 and, for the right
// operand, in that kernel's quad order; a step's rows of one tile are then
// one contiguous 16 KB run, which its loads read 1 KB per wave instruction.
//
// HBM-bound: 4 bytes read and 2 written per element.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "gemm_internal.h"

namespace sn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;
constexpr int kTile = 64;
constexpr int kPitch = kTile + 1;

// Where a staged group of 8 k goes: the plain layout (rows_pad 0),
// [batch][rows][kp], or the blocked one, [batch][kp / 32][slot][32] over
// rows_pad rows, slot = row or quad_position(row).
struct StageDst {
    uint16_t* base;
    int64_t rows, kp, rows_pad;
    bool quad;
    __device__ __forceinline__ int64_t rows_out() const { return rows_pad > 0 ? rows_pad : rows; }
    __device__ __forceinline__ uint16_t* at(int64_t batch, int64_t r, int64_t k0) const {
        if (rows_pad == 0) return base + (batch * rows + r) * kp + k0;
        const int64_t slot = quad ? quad_position(r) : r;
        return base + batch * rows_pad * kp + (k0 / 32) * (rows_pad * 32) + slot * 32 + k0 % 32;
    }
};

__device__ __forceinline__ bf16x8 round8(const float (&v)[8]) {
    const f32x8 x = {v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
    return __builtin_convertvector(x, bf16x8);
}

// VECTOR: rows start 16-byte aligned (ld % 4 == 0, aligned base), so whole
// groups inside K load as two float4.
template <bool VECTOR>
__global__ __launch_bounds__(kThreads) void stage_rows_kernel(const float* __restrict__ src, int64_t ld,
                                                              int64_t rows, int64_t k, int64_t kp,
                                                              int64_t src_stride, StageDst dst) {
    const int64_t groups = kp / 8;
    const int64_t g = int64_t(blockIdx.x) * kThreads + threadIdx.x;
    if (g >= dst.rows_out() * groups) return;
    const int64_t batch = blockIdx.y;
    const int64_t r = g / groups;
    const int64_t k0 = (g - r * groups) * 8;
    const float* row = src + batch * src_stride + r * ld;
    float v[8];
    if (r >= rows) {  // the blocked layout's padding rows
#pragma unroll
        for (int s = 0; s < 8; ++s) v[s] = 0.f;
    } else if (VECTOR && k0 + 8 <= k) {
        const f32x4 lo = *reinterpret_cast<const f32x4*>(row + k0);
        const f32x4 hi = *reinterpret_cast<const f32x4*>(row + k0 + 4);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            v[s] = lo[s];
            v[4 + s] = hi[s];
        }
    } else {
#pragma unroll
        for (int s = 0; s < 8; ++s) v[s] = k0 + s < k ? row[k0 + s] : 0.f;
    }
    *reinterpret_cast<bf16x8*>(dst.at(batch, r, k0)) = round8(v);
}

template <bool VECTOR, bool SUMS>
__global__ __launch_bounds__(kThreads) void stage_transposed_kernel(const float* __restrict__ src, int64_t ld,
                                                                    int64_t rows, int64_t k, int64_t kp,
                                                                    int64_t src_stride, StageDst dst,
                                                                    float* __restrict__ sums) {
    __shared__ float tile[kTile * kPitch];  // [k][row]
    const int tid = threadIdx.x;
    const int64_t k_base = int64_t(blockIdx.x) * kTile;
    const int64_t r_base = int64_t(blockIdx.y) * kTile;
    const int64_t batch = blockIdx.z;
    const float* s = src + batch * src_stride;

    // Loads: thread t covers rows 4 (t % 16) .. +3 of k rows t / 16 + 16 i.
    const int c4 = 4 * (tid % 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int kk = tid / 16 + 16 * i;
        const int64_t kg = k_base + kk;
        const int64_t r = r_base + c4;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (kg < k) {
            const float* p = s + kg * ld + r;
            if (VECTOR && r + 4 <= rows) {
                const f32x4 x = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = x[j];
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = r + j < rows ? p[j] : 0.f;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) tile[kk * kPitch + c4 + j] = v[j];
    }
    __syncthreads();

    // Sums (one batch): thread t adds row r_base + t % 64 over k 16 (t / 64)
    // .. + 15 of the tile in order (k past K hold 0), and the four quarters
    // are added in order; partial [k tile][row].
    if constexpr (SUMS) {
        __shared__ float quarter_sums[4][kTile];
        const int row = tid % kTile, quarter = tid / kTile;
        float part = 0.f;
#pragma unroll
        for (int kk = 16 * quarter; kk < 16 * quarter + 16; ++kk) part = part + tile[kk * kPitch + row];
        quarter_sums[quarter][row] = part;
        __syncthreads();
        if (tid < kTile && r_base + tid < rows)
            sums[int64_t(blockIdx.x) * rows + r_base + tid] =
                ((quarter_sums[0][tid] + quarter_sums[1][tid]) + quarter_sums[2][tid]) + quarter_sums[3][tid];
    }

    // Stores: 8 lanes per row, lane l of a group writing k 8 (l % 8) .. +7.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int e = tid + kThreads * i;
        const int kgrp = e % 8;
        const int rr = e / 8;
        const int64_t r = r_base + rr;
        const int64_t k0 = k_base + 8 * kgrp;
        if (r < dst.rows_out() && k0 < kp) {
            float v[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) v[t] = tile[(8 * kgrp + t) * kPitch + rr];
            *reinterpret_cast<bf16x8*>(dst.at(batch, r, k0)) = round8(v);
        }
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

int64_t stage_sum_tiles(int64_t kp) { return (kp + kTile - 1) / kTile; }

namespace {

hipError_t launch_stage(const float* src, bool k_contiguous, int64_t ld, int64_t rows, int64_t k, int64_t kp,
                        int64_t batch, int64_t src_stride, const StageDst& dst, hipStream_t stream,
                        float* row_sums) {
    if (rows == 0 || kp == 0 || batch == 0) return hipSuccess;
    if (batch > 65535 || kp % 8 != 0 || kp < k) return hipErrorInvalidValue;
    if (row_sums != nullptr && (k_contiguous || batch != 1)) return hipErrorInvalidValue;
    const bool vector = ld % 4 == 0 && src_stride % 4 == 0 && aligned16(src);
    const int64_t rows_out = dst.rows_pad > 0 ? dst.rows_pad : rows;
    if (k_contiguous) {
        const int64_t work = rows_out * (kp / 8);
        if ((work + kThreads - 1) / kThreads > 0x7FFFFFFF) return hipErrorInvalidValue;
        const dim3 grid(unsigned((work + kThreads - 1) / kThreads), unsigned(batch));
        if (vector)
            hipLaunchKernelGGL(stage_rows_kernel<true>, grid, dim3(kThreads), 0, stream, src, ld, rows, k, kp,
                               src_stride, dst);
        else
            hipLaunchKernelGGL(stage_rows_kernel<false>, grid, dim3(kThreads), 0, stream, src, ld, rows, k, kp,
                               src_stride, dst);
    } else {
        const int64_t tiles_k = (kp + kTile - 1) / kTile;
        const int64_t tiles_r = (rows_out + kTile - 1) / kTile;
        if (tiles_r > 65535) return hipErrorInvalidValue;
        const dim3 grid{unsigned(tiles_k), unsigned(tiles_r), unsigned(batch)};
        if (row_sums != nullptr) {
            if (vector)
                hipLaunchKernelGGL((stage_transposed_kernel<true, true>), grid, dim3(kThreads), 0, stream, src, ld,
                                   rows, k, kp, src_stride, dst, row_sums);
            else
                hipLaunchKernelGGL((stage_transposed_kernel<false, true>), grid, dim3(kThreads), 0, stream, src, ld,
                                   rows, k, kp, src_stride, dst, row_sums);
        } else if (vector) {
            hipLaunchKernelGGL((stage_transposed_kernel<true, false>), grid, dim3(kThreads), 0, stream, src, ld, rows,
                               k, kp, src_stride, dst, nullptr);
        } else {
            hipLaunchKernelGGL((stage_transposed_kernel<false, false>), grid, dim3(kThreads), 0, stream, src, ld,
                               rows, k, kp, src_stride, dst, nullptr);
        }
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_stage_bf16(const float* src, bool k_contiguous, int64_t ld, int64_t rows, int64_t k, int64_t kp,
                             int64_t batch, int64_t src_stride, uint16_t* dst, hipStream_t stream,
                             float* row_sums) {
    return launch_stage(src, k_contiguous, ld, rows, k, kp, batch, src_stride, StageDst{dst, rows, kp, 0, false},
                        stream, row_sums);
}

hipError_t launch_stage_bf16_blocks(const float* src, bool k_contiguous, int64_t ld, int64_t rows, int64_t k,
                                    int64_t kp, int64_t rows_pad, bool quad, int64_t batch, int64_t src_stride,
                                    uint16_t* dst, hipStream_t stream, float* row_sums) {
    if (rows == 0 || kp == 0 || batch == 0) return hipSuccess;
    if (kp % 32 != 0 || rows_pad % 256 != 0 || rows_pad < rows) return hipErrorInvalidValue;
    return launch_stage(src, k_contiguous, ld, rows, k, kp, batch, src_stride, StageDst{dst, rows, kp, rows_pad, quad},
                        stream, row_sums);
}

}  // namespace sn

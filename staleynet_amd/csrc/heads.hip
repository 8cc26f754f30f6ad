// The attention head permutes on either side of the attention products
// (kernels/attention.rs:77-138, called at layers/attention.rs:202-214, :237,
// :262-264 and :289-317): split_heads copies each head's columns of
// the packed [batch * time, width] activations (from column_offset, e.g.
// the Q, K or V part of the fused QKV projection) into the head-major
// [batch, heads, time_capacity, head_dim] layout from time step time_offset
// on (which appends to a key/value cache); merge_heads copies them back and
// leaves the other packed columns alone. Pure index maps: bit-exact.
//
// A thread moves 4 consecutive elements of one head row (16-byte loads and
// stores) when head_dim, width, column_offset and the pointers allow it, one
// element otherwise, walking the source in its own order (below); a
// grid-stride loop over all moved elements serves layouts too large for that
// grid. HBM-bound: 8 bytes per moved element.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "gemm_internal.h"

namespace sn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

// Packed and head-major positions of moved element group `i` of `group`
// consecutive dims.
__device__ __forceinline__ void positions(const HeadLayoutArgs& l, int64_t i, int group, int64_t& packed,
                                          int64_t& head_major) {
    const int64_t groups_per_row = l.head_dim / group;
    const int64_t d = (i % groups_per_row) * group;
    const int64_t t = (i / groups_per_row) % l.time;
    const int64_t h = (i / (groups_per_row * l.time)) % l.heads;
    const int64_t b = i / (groups_per_row * l.time * l.heads);
    packed = (b * l.time + t) * l.width + l.column_offset + h * l.head_dim + d;
    head_major = ((b * l.heads + h) * l.time_capacity + l.time_offset + t) * l.head_dim + d;
}

template <bool SPLIT, int GROUP>
__global__ __launch_bounds__(kThreads) void permute_heads_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                                 HeadLayoutArgs l) {
    const int64_t total = l.batch * l.heads * l.time * (l.head_dim / GROUP);
    for (int64_t i = blockIdx.x * int64_t(kThreads) + threadIdx.x; i < total; i += int64_t(gridDim.x) * kThreads) {
        int64_t packed, head_major;
        positions(l, i, GROUP, packed, head_major);
        const int64_t from = SPLIT ? packed : head_major;
        const int64_t to = SPLIT ? head_major : packed;
        if constexpr (GROUP == 4)
            *reinterpret_cast<f32x4*>(dst + to) = *reinterpret_cast<const f32x4*>(src + from);
        else
            dst[to] = src[from];
    }
}

// The same copy walked in the source's order, the batch on the grid's z
// dimension: split_heads reads each packed row's head columns contiguously
// (x runs over (step, head, group)), merge_heads each head's rows (the head
// on y, x over (step, group)); the scattered side is the write, which the L2
// gathers. Two 32-bit divides per moved group instead of four 64-bit ones.
template <bool SPLIT, int GROUP>
__global__ __launch_bounds__(kThreads) void permute_head_rows_kernel(const float* __restrict__ src,
                                                                     float* __restrict__ dst, HeadLayoutArgs l) {
    const uint32_t groups_per_row = uint32_t(l.head_dim / GROUP);
    const uint32_t j = blockIdx.x * kThreads + threadIdx.x;
    int64_t t, h, d;
    if constexpr (SPLIT) {
        const uint32_t per_step = uint32_t(l.heads) * groups_per_row;
        if (j >= uint32_t(l.time) * per_step) return;
        const uint32_t step = j / per_step, rest = j - step * per_step;
        const uint32_t head = rest / groups_per_row;
        t = step;
        h = head;
        d = int64_t(rest - head * groups_per_row) * GROUP;
    } else {
        if (j >= uint32_t(l.time) * groups_per_row) return;
        const uint32_t step = j / groups_per_row;
        t = step;
        h = blockIdx.y;
        d = int64_t(j - step * groups_per_row) * GROUP;
    }
    const int64_t b = blockIdx.z;
    const int64_t packed = (b * l.time + t) * l.width + l.column_offset + h * l.head_dim + d;
    const int64_t head_major = ((b * l.heads + h) * l.time_capacity + l.time_offset + t) * l.head_dim + d;
    const int64_t from = SPLIT ? packed : head_major;
    const int64_t to = SPLIT ? head_major : packed;
    if constexpr (GROUP == 4)
        *reinterpret_cast<f32x4*>(dst + to) = *reinterpret_cast<const f32x4*>(src + from);
    else
        dst[to] = src[from];
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

hipError_t launch_permute_heads(bool split, const float* src, float* dst, const HeadLayoutArgs& l,
                                hipStream_t stream) {
    const int64_t elements = l.batch * l.heads * l.time * l.head_dim;
    if (elements == 0) return hipSuccess;
    const bool vector = l.head_dim % 4 == 0 && l.width % 4 == 0 && l.column_offset % 4 == 0 && aligned16(src) &&
                        aligned16(dst);
    const int64_t per_row_groups = vector ? l.head_dim / 4 : l.head_dim;
    const int64_t per_batch = l.time * l.heads * per_row_groups;  // split's x extent bounds merge's too
    if (per_batch < (int64_t(1) << 31) && l.heads <= 65535 && l.batch <= 65535) {
        const int64_t x = split ? per_batch : l.time * per_row_groups;
        const dim3 rows(unsigned((x + kThreads - 1) / kThreads), split ? 1u : unsigned(l.heads), unsigned(l.batch));
        if (vector) {
            if (split) hipLaunchKernelGGL((permute_head_rows_kernel<true, 4>), rows, dim3(kThreads), 0, stream, src, dst, l);
            else hipLaunchKernelGGL((permute_head_rows_kernel<false, 4>), rows, dim3(kThreads), 0, stream, src, dst, l);
        } else {
            if (split) hipLaunchKernelGGL((permute_head_rows_kernel<true, 1>), rows, dim3(kThreads), 0, stream, src, dst, l);
            else hipLaunchKernelGGL((permute_head_rows_kernel<false, 1>), rows, dim3(kThreads), 0, stream, src, dst, l);
        }
        return hipGetLastError();
    }
    const int64_t work = vector ? elements / 4 : elements;
    const dim3 grid(unsigned(std::min<int64_t>((work + kThreads - 1) / kThreads, 8192)));
    if (vector) {
        if (split) hipLaunchKernelGGL((permute_heads_kernel<true, 4>), grid, dim3(kThreads), 0, stream, src, dst, l);
        else hipLaunchKernelGGL((permute_heads_kernel<false, 4>), grid, dim3(kThreads), 0, stream, src, dst, l);
    } else {
        if (split) hipLaunchKernelGGL((permute_heads_kernel<true, 1>), grid, dim3(kThreads), 0, stream, src, dst, l);
        else hipLaunchKernelGGL((permute_heads_kernel<false, 1>), grid, dim3(kThreads), 0, stream, src, dst, l);
    }
    return hipGetLastError();
}

}  // namespace sn

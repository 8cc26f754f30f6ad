// Seeded synthetic inputs in device memory: element i of stream `stream`
// under `seed` is a normal deviate mean + std * z, z from the Box-Muller
// transform of two uniforms drawn by SplitMix64 (Steele, Lea and Flood,
// "Fast splittable pseudorandom number generators", OOPSLA 2014) at counter
// positions 2*(i/2) and 2*(i/2)+1. Counter-based, so any element can be
// produced independently and the same (seed, stream, count) always yields
// the same bytes. A bench/test utility with no reference counterpart (the
// reference draws its weights on the host, crates/staleynet-model/src/random.rs).
#include "staleynet_synth.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

namespace {

__host__ __device__ inline uint64_t splitmix64_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

__global__ __launch_bounds__(256) void fill_normal_kernel(float* out, uint64_t count, uint64_t base, float mean,
                                                          float stddev) {
    const uint64_t pairs = (count + 1) / 2;
    for (uint64_t pair = blockIdx.x * uint64_t(blockDim.x) + threadIdx.x; pair < pairs;
         pair += uint64_t(gridDim.x) * blockDim.x) {
        const uint64_t z1 = splitmix64_mix(base + (2 * pair + 1) * kGamma);
        const uint64_t z2 = splitmix64_mix(base + (2 * pair + 2) * kGamma);
        const float u1 = float((z1 >> 40) + 1) * (1.0f / 16777216.0f);  // (0, 1]
        const float u2 = float(z2 >> 40) * (1.0f / 16777216.0f);        // [0, 1)
        const float radius = sqrtf(-2.0f * logf(u1));
        float s, c;
        sincosf(6.28318530717958647692f * u2, &s, &c);
        out[2 * pair] = mean + stddev * (radius * c);
        if (2 * pair + 1 < count) out[2 * pair + 1] = mean + stddev * (radius * s);
    }
}

// Plain streaming copy, 16 bytes per lane per iteration: the known-size
// kernel that hardware byte counters are calibrated against.
__global__ __launch_bounds__(256) void copy_kernel(float4* __restrict__ dst, const float4* __restrict__ src,
                                                   uint64_t vectors) {
    for (uint64_t i = blockIdx.x * uint64_t(blockDim.x) + threadIdx.x; i < vectors;
         i += uint64_t(gridDim.x) * blockDim.x)
        dst[i] = src[i];
}

// Streaming read: each workgroup sums its grid-stride share of `src` (eight
// non-temporal 16-byte loads in flight per lane) and writes one float. The
// practical HBM read bandwidth that read-bound kernels are compared with.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void read_sum_kernel(const f32x4_t* __restrict__ src, uint64_t vectors,
                                                       float* __restrict__ sums) {
    __shared__ float partial[256];
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    uint64_t i = blockIdx.x * uint64_t(blockDim.x) + threadIdx.x;
    float s = 0.f;
    for (; i + 7 * stride < vectors; i += 8 * stride) {
        f32x4_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < 8; ++u) s += (v[u][0] + v[u][1]) + (v[u][2] + v[u][3]);
    }
    for (; i < vectors; i += stride) {
        const f32x4_t v = __builtin_nontemporal_load(src + i);
        s += (v[0] + v[1]) + (v[2] + v[3]);
    }
    partial[threadIdx.x] = s;
    __syncthreads();
    for (int half = 128; half > 0; half /= 2) {
        if (int(threadIdx.x) < half) partial[threadIdx.x] += partial[threadIdx.x + half];
        __syncthreads();
    }
    if (threadIdx.x == 0) sums[blockIdx.x] = partial[0];
}

}  // namespace

extern "C" int sn_read_sum(void* stream, const float* src, size_t count, float* sums, size_t sums_count) {
    if (count == 0) return 0;
    if (src == nullptr || sums == nullptr) return -1;
    if (count % 4 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0 || sums_count == 0 || sums_count > 65535)
        return -7;
    hipLaunchKernelGGL(read_sum_kernel, dim3(unsigned(sums_count)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       reinterpret_cast<const f32x4_t*>(src), uint64_t(count / 4), sums);
    return int(hipGetLastError());
}

extern "C" int sn_copy_device(void* stream, float* dst, const float* src, size_t count) {
    if (count == 0) return 0;
    if (dst == nullptr || src == nullptr) return -1;
    if (count % 4 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0)
        return -7;
    const uint64_t vectors = count / 4;
    const uint64_t grid = std::min<uint64_t>((vectors + 255) / 256, 8192);
    hipLaunchKernelGGL(copy_kernel, dim3(unsigned(grid)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       reinterpret_cast<float4*>(dst), reinterpret_cast<const float4*>(src), vectors);
    return int(hipGetLastError());
}

extern "C" int sn_fill_normal(void* stream, float* device, size_t count, uint64_t seed, uint64_t stream_id,
                              float mean, float stddev) {
    if (count == 0) return 0;
    if (device == nullptr) return -1;
    const uint64_t base = splitmix64_mix(seed) ^ splitmix64_mix(stream_id + 0x632BE59BD9B4E019ull);
    const uint64_t pairs = (count + 1) / 2;
    const uint64_t grid = std::min<uint64_t>((pairs + 255) / 256, 65536);
    hipLaunchKernelGGL(fill_normal_kernel, dim3(unsigned(grid)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       device, uint64_t(count), base, mean, stddev);
    return int(hipGetLastError());
}

// Pieces shared by the fused causal-attention kernels (attention.hip, the
// forward, the probability gradient and the decode form; attention_backward.hip,
// the gradients that recompute the probabilities): buffer addressing,
// direct-to-LDS loads, load-count waits, the exponential, the barrier that
// leaves loads in flight, and the per-head-dim LDS geometry.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <type_traits>

namespace sn {
namespace attn {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_void;

constexpr int kWaves = 4;
constexpr int kQueries = 32 * kWaves;  // per workgroup
constexpr int kKeys = 64;              // per LDS stage
constexpr int32_t kRecords = 0x7FFFFFFF;
constexpr int32_t kOutOfRange = int32_t(0x80000000u);
constexpr int32_t kRawBufferFormat = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, kRecords, kRawBufferFormat);
}

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, const void* lds, int32_t offset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void)lds, 16, offset, 0, 0, 0);
}

// Waits until at most PENDING of this wave's vector-memory loads are in
// flight (vmcnt; the other counters left at their maxima).
template <int PENDING>
__device__ __forceinline__ void wait_loads() {
    static_assert(PENDING >= 0 && PENDING < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (PENDING & 15) | ((PENDING >> 4) << 14));
}

// e^d as 2^(d log2 e) on the transcendental unit (v_exp_f32, about 1 ulp).
// d is a difference x - m already rounded as causal_softmax rounds it, so
// rounding d log2 e adds at most |d| 2^-24 to the exponent: a relative error
// under 2e-6 for every probability above e^-20, whatever the logits' size.
// d = -inf gives 0.
constexpr float kLog2e = 1.44269504088896340736f;
__device__ __forceinline__ float exp_of(float d) { return __builtin_amdgcn_exp2f(d * kLog2e); }

// Workgroup barrier that does not wait for loads still in flight (the
// direct-to-LDS loads of the next stage); LDS reads are completed first.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int H, int KEYS = kKeys>
struct Geometry {
    static constexpr int SLOTS = H / 4;                        // 16-byte chunks per row
    static constexpr int SWIZZLE = SLOTS < 16 ? SLOTS - 1 : 15;  // row bits XORed into the chunk index
    static constexpr int CHUNKS = H / 16;                      // 16-deep MFMA chunks over h
    static constexpr int OBLOCKS = H / 32;                     // 32-row accumulator blocks of O^T
    static constexpr int STAGE_SLOTS = KEYS * SLOTS;           // f32x4 per operand per stage
    static constexpr int LOADS = STAGE_SLOTS / (64 * kWaves);  // load instructions per wave per operand
    static_assert(H == 32 || H == 64 || H == 128, "head dims 32, 64, 128");
    static_assert(STAGE_SLOTS % (64 * kWaves) == 0, "whole load instructions per wave");
};

}  // namespace attn
}  // namespace sn

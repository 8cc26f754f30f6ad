// Decode-shaped products: few output rows against a row-major weight.
//
// The reference's autoregressive step (crates/staleynet-model/src/decode.rs:
// 123-161, layers/attention.rs:274-320) issues every Linear with M = the
// number of new positions (1 in `generate`), i.e. y[M, N] = x[M, K] W[K, N]
// with W row-major [K, N] (linear.rs:20-28). At M <= 16 a 128x128 matrix-core
// tile would leave most of its rows idle; the product is bound by reading W
// once from HBM, so this kernel streams W and is judged against 8 TB/s.
//
// Design (one launch, one memory round trip per workgroup):
//  * A workgroup of 4 waves owns 256 output columns and a 64-row slice of K;
//    each lane owns 4 consecutive columns. Every wave issues all 16 of its
//    row loads (16 bytes each, 1 KB contiguous per wave-row) before the
//    first multiply, so a workgroup's whole slice is in flight at once.
//  * x's slice is staged in LDS and read as a broadcast.
//  * The 4 waves' partial sums are added in wave order through LDS.
//  * K slices beyond the first go to separate workgroups. Each writes its
//    partial sums to the split-K workspace with device-coherent stores
//    (agent-scope atomics: written through to where every XCD reads them),
//    waits for them to complete and increments its column block's arrival
//    counter; the workgroup that arrives last reads the partials with
//    device-coherent loads, adds them in slice order, applies the
//    reference's combine and resets the counter. No workgroup waits for
//    another, the summation order is fixed, and no L2 write-back or
//    invalidate (a cost of ~100 us per launch here) is needed.
#include "gemm_common.h"

namespace sn {
namespace {

using gemm::f32x4;

constexpr int kThreads = 256;
constexpr int kColumns = 256;      // per workgroup: 64 lanes x 4
constexpr int kRowsPerWave = 16;   // loads in flight per lane
constexpr int kSlice = 4 * kRowsPerWave;
constexpr int kMaxRows = 16;

struct GemvArgs {
    const float* x;
    const float* w;
    float* y;
    float* ws;
    uint32_t* counters;
    int64_t m, n, k;
    int64_t stride_x, stride_w, stride_y;
    int32_t column_blocks;
    int32_t splits;
    int32_t accumulate;
    float scale;
};

template <int MT>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs args) {
    __shared__ __attribute__((aligned(16))) float x_slice[kSlice][MT];  // [row][m]: a row's MT multipliers together
    __shared__ f32x4 partial[MT][64];
    __shared__ int arrived_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int split = blockIdx.y;
    const int64_t batch = blockIdx.z;
    const int64_t n0 = int64_t(blockIdx.x) * kColumns;
    const int64_t k_begin = int64_t(split) * kSlice;
    const int slice = int(min(int64_t(kSlice), args.k - k_begin));

    const float* x = args.x + batch * args.stride_x;
    const float* w = args.w + batch * args.stride_w;

    // W first: one descriptor per workgroup (scalar registers), the lane's
    // row and column as its byte offset; rows past the slice read 0.
    const bool col_ok = n0 + 4 * lane < args.n;
    const __amdgpu_buffer_rsrc_t rsrc = gemm::buffer_of(w + k_begin * args.n + n0);
    f32x4 rows[kRowsPerWave];
#pragma unroll
    for (int u = 0; u < kRowsPerWave; ++u) {
        const int r = wave * kRowsPerWave + u;
        const bool ok = col_ok && r < slice;
        rows[u] = gemm::buffer_load4(rsrc, ok ? int32_t((int64_t(r) * args.n + 4 * lane) * 4) : gemm::kOutOfRange);
    }
    for (int e = tid; e < MT * kSlice; e += kThreads) {
        const int kk = e / MT;
        const int m = e % MT;
        x_slice[kk][m] = (m < args.m && kk < slice) ? x[m * args.k + k_begin + kk] : 0.f;
    }
    __syncthreads();

    f32x4 acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kRowsPerWave; ++u) {
        const float* xr = x_slice[wave * kRowsPerWave + u];
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[m] += xr[m] * rows[u];
    }

    // Wave-ordered sum of the four waves' partials.
    for (int turn = 0; turn < 4; ++turn) {
        if (wave == turn) {
#pragma unroll
            for (int m = 0; m < MT; ++m) partial[m][lane] = turn == 0 ? acc[m] : partial[m][lane] + acc[m];
        }
        __syncthreads();
    }

    const int64_t per_matrix = args.m * args.n;
    if (args.splits == 1) {
        for (int e = tid; e < MT * 64; e += kThreads) {
            const int m = e / 64;
            const int64_t c = n0 + 4 * (e % 64);
            if (m >= args.m || c >= args.n) continue;
            float* dst = args.y + batch * args.stride_y + m * args.n + c;
            const f32x4 sum = partial[m][e % 64];
#pragma unroll
            for (int j = 0; j < 4; ++j) gemm::write_output(dst + j, sum[j], args.scale, args.accumulate != 0);
        }
        return;
    }

    // Partial sums of this slice, written device-coherently; offsets from
    // the column block's origin in this slice's workspace matrix.
    const __amdgpu_buffer_rsrc_t mine = gemm::buffer_of(args.ws + (batch * args.splits + split) * per_matrix + n0);
    for (int e = tid; e < MT * 64; e += kThreads) {
        const int m = e / 64;
        const int l = e % 64;
        const bool inside = m < args.m && n0 + 4 * l < args.n;
        gemm::buffer_store4_coherent(mine, inside ? int32_t((m * args.n + 4 * l) * 4) : gemm::kOutOfRange,
                                     partial[m][l]);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are complete device-wide
    __syncthreads();
    uint32_t* counter = args.counters + batch * args.column_blocks + blockIdx.x;
    if (tid == 0)
        arrived_last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                       uint32_t(args.splits - 1);
    __syncthreads();
    if (!arrived_last) return;

    // Last to arrive: every slice's partials are complete; add them in slice
    // order (device-coherent loads) and apply the combine.
    const __amdgpu_buffer_rsrc_t all = gemm::buffer_of(args.ws + batch * args.splits * per_matrix + n0);
    for (int e = tid; e < MT * 64; e += kThreads) {
        const int m = e / 64;
        const int l = e % 64;
        const int64_t c = n0 + 4 * l;
        if (m >= args.m || c >= args.n) continue;
        f32x4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
        for (int s = 0; s < args.splits; ++s)
            sum += gemm::buffer_load4_coherent(all, int32_t((s * per_matrix + m * args.n + 4 * l) * 4));
        float* dst = args.y + batch * args.stride_y + m * args.n + c;
#pragma unroll
        for (int j = 0; j < 4; ++j) gemm::write_output(dst + j, sum[j], args.scale, args.accumulate != 0);
    }
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct GemvPlan {
    int column_blocks;
    int splits;
};

GemvPlan gemv_plan(const Problem& p) {
    GemvPlan plan;
    plan.column_blocks = int((p.n + kColumns - 1) / kColumns);
    plan.splits = int((p.k + kSlice - 1) / kSlice);
    return plan;
}

template <int MT>
hipError_t launch_rows(const Problem& p, const Env& env, const GemvPlan& plan, hipStream_t stream) {
    GemvArgs args;
    args.x = p.a;
    args.w = p.b;
    args.y = p.c;
    args.ws = env.workspace;
    args.counters = env.counters;
    args.m = p.m;
    args.n = p.n;
    args.k = p.k;
    args.stride_x = p.stride_a;
    args.stride_w = p.stride_b;
    args.stride_y = p.stride_c;
    args.column_blocks = plan.column_blocks;
    args.splits = plan.splits;
    args.accumulate = p.accumulate ? 1 : 0;
    args.scale = p.scale;
    hipLaunchKernelGGL(gemv_kernel<MT>, dim3(plan.column_blocks, plan.splits, unsigned(p.batch)), dim3(kThreads), 0,
                       stream, args);
    return hipGetLastError();
}

}  // namespace

bool gemv_applies(const Problem& p, const Env& env) {
    // Row-major x (K-contiguous) and row-major W (N-contiguous), aligned for
    // 16-byte loads; no mask; few rows; grid dimensions, counters and the
    // split-K workspace large enough.
    if (!(p.m >= 1 && p.m <= kMaxRows && p.k >= 1 && p.mask == SN_MASK_NONE && p.a_k_contiguous &&
          !p.b_k_contiguous && p.lda == p.k && p.ldb == p.n && p.n % 4 == 0 && p.stride_b % 4 == 0 &&
          gemm::aligned16(p.b) && p.batch <= 65535 &&
          (int64_t(kSlice) * p.n + kColumns) * 4 < gemm::kMaxBufferOffset))
        return false;
    const GemvPlan plan = gemv_plan(p);
    if (plan.splits == 1) return true;
    // Workspace offsets of one batch's partials must fit the 31-bit range.
    if (int64_t(plan.splits) * p.m * p.n * 4 >= gemm::kMaxBufferOffset) return false;
    const size_t partials = size_t(plan.splits) * size_t(p.batch) * size_t(p.m) * size_t(p.n) * sizeof(float);
    return plan.splits <= 65535 && partials <= env.workspace_bytes &&
           size_t(p.batch) * size_t(plan.column_blocks) <= env.counter_count;
}

hipError_t launch_gemv(const Problem& p, const Env& env, hipStream_t stream) {
    if (!gemv_applies(p, env)) return hipErrorNotSupported;
    const GemvPlan plan = gemv_plan(p);
    if (p.m == 1) return launch_rows<1>(p, env, plan, stream);
    if (p.m <= 2) return launch_rows<2>(p, env, plan, stream);
    if (p.m <= 4) return launch_rows<4>(p, env, plan, stream);
    if (p.m <= 8) return launch_rows<8>(p, env, plan, stream);
    return launch_rows<16>(p, env, plan, stream);
}

}  // namespace sn

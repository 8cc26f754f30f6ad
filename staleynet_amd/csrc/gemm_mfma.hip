// fp32 matrix-core GEMM for gfx950 (CDNA4): C_b = scale * op(A_b) op(B_b) (+ C_b).
//
// Replaces the reference's default kernel, matmul_blocked
// (crates/staleynet-cuda/src/kernels/matmul.rs:283-355), behind the same
// contract: any operand storage, strided batches, overwrite or accumulate,
// zero padding of partial tiles, row-major output with row stride N.
//
// Design (gfx950 first, not a translation of the reference's 64x64 SIMT tile):
//  * Matrix cores: v_mfma_f32_32x32x2_f32, a 32x32 fp32 block per 64-lane
//    wave per instruction (16 passes). A workgroup of 4 waves owns a
//    BM x BN output tile; each wave a (BM/WAVES_M) x (BN/WAVES_N) sub-tile
//    of FM x FN MFMA blocks accumulated in registers.
//  * LDS layout, per operand and stage: [BK/4 k-groups][ROWS + 1][4 floats].
//    A 16-byte slot holds four consecutive k of one row. Measured on gfx950:
//    b128 reads serve 16 lanes per clock and are conflict-free when those
//    lanes hit distinct slots mod 16; b128 writes serve 8 lanes per clock and
//    need distinct slots mod 8. Fragment reads walk consecutive rows of one
//    k-group (consecutive slots); stores put the 8 lanes of a write phase in
//    8 different k-groups, and the one-slot pad per k-group makes those 8
//    slots distinct mod 8. Every LDS access of the main loop is conflict-free.
//  * Fragments: within a 16-deep chunk, lane half h feeds k = 8h + s to
//    MFMA s (s = 0..7), i.e. k-groups 2h and 2h+1: two ds_read_b128 per
//    32-row fragment. A and B use the same assignment, so products pair.
//  * This kernel serves operands that 128-bit loads cannot: a base that is
//    not 16-byte aligned, or a contiguous dimension, leading dimension or
//    batch stride that is not a multiple of 4 floats. Global loads are then
//    scalar, coalesced along whichever dimension is contiguous in memory
//    (the scalar loaders in gemm_common.h), and edges are guarded per lane.
//    Aligned operands take gemm_dma.hip, which loads straight into LDS. One
//    kernel body serves NN, NT, TN and TT; an operand contiguous along M or
//    N is transposed in registers on its way into LDS.
//  * Double-buffered LDS; the next tile is prefetched into registers while
//    the current one is multiplied: one barrier per BK step.
//  * Grid: blockIdx.x enumerates (batch, split, tile), remapped so each XCD
//    (the dispatcher deals workgroups round-robin over 8 XCDs, each with its
//    own L2) receives a contiguous run of whole matrices or whole K splits,
//    each walked as a grouped raster. Split-K partial sums go to the
//    context's workspace and a second kernel adds them in split order
//    (deterministic).
//  * Masks: causal output tiles that are entirely masked are not multiplied;
//    causal left operands limit each tile's K range to the visible part.
#include "gemm_common.h"

namespace sn {
namespace gemm {
namespace {

template <class T>
__device__ __forceinline__ void multiply_tile(const float* __restrict__ lds_a, const float* __restrict__ lds_b,
                                              f32x16 (&acc)[T::FM][T::FN], int lane, int wave_m, int wave_n) {
    using PA = Planes<T::BM, T::BK>;
    using PB = Planes<T::BN, T::BK>;
    const int row = lane & 31;
    const int half = lane >> 5;
#pragma unroll
    for (int chunk = 0; chunk < T::BK / 16; ++chunk) {
        const int group = 4 * chunk + 2 * half;
        f32x4 a_lo[T::FM], a_hi[T::FM], b_lo[T::FN], b_hi[T::FN];
#pragma unroll
        for (int i = 0; i < T::FM; ++i) {
            const int r = wave_m * T::WTM + 32 * i + row;
            a_lo[i] = *reinterpret_cast<const f32x4*>(lds_a + 4 * (group * PA::PLANE + r));
            a_hi[i] = *reinterpret_cast<const f32x4*>(lds_a + 4 * ((group + 1) * PA::PLANE + r));
        }
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
            const int r = wave_n * T::WTN + 32 * j + row;
            b_lo[j] = *reinterpret_cast<const f32x4*>(lds_b + 4 * (group * PB::PLANE + r));
            b_hi[j] = *reinterpret_cast<const f32x4*>(lds_b + 4 * ((group + 1) * PB::PLANE + r));
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < T::FM; ++i)
#pragma unroll
                for (int j = 0; j < T::FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a_lo[i][s], b_lo[j][s], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < T::FM; ++i)
#pragma unroll
                for (int j = 0; j < T::FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a_hi[i][s], b_hi[j][s], acc[i][j], 0, 0, 0);
    }
}

template <class T, bool A_K, bool B_K, bool BUF>
__global__ __launch_bounds__(T::THREADS) void gemm_f32_kernel(Args args) {
    using PA = Planes<T::BM, T::BK>;
    using PB = Planes<T::BN, T::BK>;
    __shared__ __attribute__((aligned(16))) float lds_a[2][4 * PA::SLOTS];
    __shared__ __attribute__((aligned(16))) float lds_b[2][4 * PB::SLOTS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave / T::WAVES_N;
    const int wave_n = wave % T::WAVES_N;

    int batch_local, split, tm, tn;
    tile_coordinates(blockIdx.x, gridDim.x, args.tiles_m, args.tiles_n, args.splits, batch_local, split, tm, tn);
    const int64_t batch = args.batch_base + batch_local;
    const int64_t m0 = int64_t(tm) * T::BM;
    const int64_t n0 = int64_t(tn) * T::BN;

    const int64_t row_last = min(m0 + T::BM, args.m) - 1;
    const bool left_causal = args.mask == int(SN_MASK_CAUSAL_LEFT);
    float* c_batch = args.c + batch * args.stride_c;

    if (args.mask == int(SN_MASK_CAUSAL_OUTPUT) && n0 > row_last + args.query_offset) {
        // Every output of this tile is masked: the product is 0 there.
        if (!args.accumulate) zero_tile<T>(args, c_batch, m0, n0, tid);
        return;
    }

    int64_t k_begin = int64_t(split) * args.k_per_split;
    int64_t k_end = min(args.k, k_begin + args.k_per_split);
    if (left_causal) {
        if (A_K) {
            k_end = min(k_end, row_last + args.query_offset + 1);
        } else {
            const int64_t first = m0 - args.query_offset;
            if (first > k_begin) k_begin = first / T::BK * T::BK;
        }
    }

    const float* a = args.a + batch * args.stride_a;
    const float* b = args.b + batch * args.stride_b;

    LoaderFor<A_K, BUF, T::BM, T::BK, T::THREADS> load_a;
    LoaderFor<B_K, BUF, T::BN, T::BK, T::THREADS> load_b;
    load_a.init(args.lda, m0, args.m, tid);
    load_b.init(args.ldb, n0, args.n, tid);

    f32x16 acc[T::FM][T::FN];
#pragma unroll
    for (int i = 0; i < T::FM; ++i)
#pragma unroll
        for (int j = 0; j < T::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int steps = k_end > k_begin ? int((k_end - k_begin + T::BK - 1) / T::BK) : 0;
    if (steps > 0) {
        load_a.load(a, args.lda, m0, args.m, k_begin, args.k, tid);
        load_b.load(b, args.ldb, n0, args.n, k_begin, args.k, tid);
        if (left_causal) load_a.mask_keys_after_query(m0, k_begin, args.query_offset, tid);
        load_a.store(lds_a[0], tid);
        load_b.store(lds_b[0], tid);
        __syncthreads();
        for (int step = 0; step < steps; ++step) {
            const int cur = step & 1;
            const bool more = step + 1 < steps;
            const int64_t k_next = k_begin + int64_t(step + 1) * T::BK;
            if (more) {
                load_a.load(a, args.lda, m0, args.m, k_next, args.k, tid);
                load_b.load(b, args.ldb, n0, args.n, k_next, args.k, tid);
            }
            multiply_tile<T>(lds_a[cur], lds_b[cur], acc, lane, wave_m, wave_n);
            if (more) {
                if (left_causal) load_a.mask_keys_after_query(m0, k_next, args.query_offset, tid);
                load_a.store(lds_a[cur ^ 1], tid);
                load_b.store(lds_b[cur ^ 1], tid);
            }
            __syncthreads();
        }
    }

    const bool partial = args.splits > 1;
    float* out = partial ? args.ws + ((batch_local * int64_t(args.splits) + split) * args.m) * args.n : c_batch;
    write_tile<T, BUF>(args, acc, out, m0, n0, wave_m, wave_n, lane, partial);
}

// Adds the split partial sums of each output in split order, then applies
// the reference's combine.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, float* c, int64_t m,
                                                            int64_t n, int64_t batches, int splits,
                                                            int64_t stride_c, float scale, int accumulate,
                                                            const float* __restrict__ bias) {
    const int64_t per_matrix = m * n;
    const int64_t total = per_matrix * batches;
    for (int64_t idx = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; idx < total;
         idx += int64_t(gridDim.x) * blockDim.x) {
#pragma clang fp contract(off)
        const int64_t bat = idx / per_matrix;
        const int64_t e = idx % per_matrix;
        const float* src = ws + bat * splits * per_matrix + e;
        float sum = 0.f;
#pragma unroll 8
        for (int s = 0; s < splits; ++s) sum = sum + src[s * per_matrix];
        write_output(c + bat * stride_c + e, sum, scale, accumulate != 0, bias, e % n);
    }
}

// The same for 16-byte-aligned outputs with M*N a multiple of 4: four
// consecutive outputs per thread, 8 splits' 16-byte loads in flight
// (non-temporal: each partial is read once), and the output read (when
// accumulating) and written 16 bytes at a time; each element's combine is
// write_output's, rounded as it rounds.
__global__ __launch_bounds__(256) void splitk_reduce4_kernel(const f32x4* __restrict__ ws, float* c,
                                                             int64_t per_matrix, int64_t n, int64_t batches,
                                                             int splits, int64_t stride_c, float scale,
                                                             int accumulate, const float* __restrict__ bias) {
    const int64_t per_matrix4 = per_matrix / 4;
    const int64_t total = per_matrix4 * batches;
    for (int64_t idx = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; idx < total;
         idx += int64_t(gridDim.x) * blockDim.x) {
#pragma clang fp contract(off)
        const int64_t bat = idx / per_matrix4;
        const int64_t e4 = idx % per_matrix4;
        const f32x4* src = ws + bat * splits * per_matrix4 + e4;
        f32x4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
        for (int s = 0; s < splits; ++s) sum = sum + __builtin_nontemporal_load(src + s * per_matrix4);
        f32x4* dst = reinterpret_cast<f32x4*>(c + bat * stride_c + 4 * e4);
        const f32x4 prior = accumulate ? *dst : f32x4{0.f, 0.f, 0.f, 0.f};
        f32x4 out;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float scaled = scale * sum[j];
            float value = accumulate ? prior[j] + scaled : scaled;
            if (bias != nullptr) value = value + bias[(4 * e4 + j) % n];
            out[j] = value;
        }
        *dst = out;
    }
}

template <class T, bool A_K, bool B_K, bool BUF>
hipError_t launch_tiles(const Problem& p, const Env& env, const Plan& plan, hipStream_t stream) {
    const LaunchShape shape = tiled_shape<T>(p, plan, SN_PATH_NONE);
    if (shape.batches_per_launch < 1) return hipErrorInvalidConfiguration;
    Args args = make_args<T>(p, env, plan);
    const int64_t per_batch = int64_t(plan.tiles_m) * plan.tiles_n * plan.splits;
    const int64_t chunk = shape.batches_per_launch;
    for (int64_t first = 0; first < p.batch; first += chunk) {
        const int64_t count = std::min<int64_t>(chunk, p.batch - first);
        args.batch_base = first;
        hipLaunchKernelGGL((gemm_f32_kernel<T, A_K, B_K, BUF>), dim3(unsigned(count * per_batch)), dim3(T::THREADS), 0,
                           stream, args);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (plan.splits > 1) return launch_splitk_reduce(p, env, plan.splits, stream);
    return hipSuccess;
}

template <class T, bool A_K, bool B_K>
hipError_t dispatch_path(const Problem& p, const Env& env, const Plan& plan, hipStream_t stream) {
    // Operands that allow 128-bit loads never get here (gemm_dma.hip).
    return launch_tiles<T, A_K, B_K, false>(p, env, plan, stream);
}

template <class T>
hipError_t dispatch_layout(const Problem& p, const Env& env, hipStream_t stream) {
    const Plan plan = plan_for<T>(p, env);
    if (p.a_k_contiguous && p.b_k_contiguous) return dispatch_path<T, true, true>(p, env, plan, stream);
    if (p.a_k_contiguous) return dispatch_path<T, true, false>(p, env, plan, stream);
    if (p.b_k_contiguous) return dispatch_path<T, false, true>(p, env, plan, stream);
    return dispatch_path<T, false, false>(p, env, plan, stream);
}

using TileSquare = Tile<128, 128, 32, 2, 2>;  // 4 waves of 64x64
using TileNarrow = Tile<128, 64, 32, 4, 1>;   // N <= 64 (attention head dim): 3 workgroups per CU

bool use_narrow(const Problem& p) { return p.n <= 64; }

}  // namespace

hipError_t launch_splitk_reduce(const Problem& p, const Env& env, int splits, hipStream_t stream) {
    const int64_t total = p.m * p.n * p.batch;
    if ((p.m * p.n) % 4 == 0 && p.stride_c % 4 == 0 && aligned16(p.c)) {
        const int64_t grid = std::min<int64_t>((total / 4 + 255) / 256, int64_t(env.cu_count) * 16);
        hipLaunchKernelGGL(splitk_reduce4_kernel, dim3(unsigned(grid)), dim3(256), 0, stream,
                           reinterpret_cast<const f32x4*>(env.workspace), p.c, p.m * p.n, p.n, p.batch, splits,
                           p.stride_c, p.scale, p.accumulate ? 1 : 0, p.bias);
        return hipGetLastError();
    }
    const int64_t grid = std::min<int64_t>((total + 255) / 256, int64_t(env.cu_count) * 16);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(unsigned(grid)), dim3(256), 0, stream, env.workspace, p.c, p.m,
                       p.n, p.batch, splits, p.stride_c, p.scale, p.accumulate ? 1 : 0, p.bias);
    return hipGetLastError();
}

}  // namespace gemm

LaunchShape describe_gemm_f32(const Problem& p, const Env& env) {
    if (gemm::dma_applies(p, env)) return gemm::describe_f32_dma(p, env);
    if (gemm::use_narrow(p))
        return gemm::tiled_shape<gemm::TileNarrow>(p, gemm::plan_for<gemm::TileNarrow>(p, env), SN_PATH_F32_REGISTER);
    return gemm::tiled_shape<gemm::TileSquare>(p, gemm::plan_for<gemm::TileSquare>(p, env), SN_PATH_F32_REGISTER);
}

hipError_t launch_gemm_f32(const Problem& p, const Env& env, hipStream_t stream) {
    if (gemm::dma_applies(p, env)) return gemm::launch_gemm_f32_dma(p, env, stream);
    if (gemm::use_narrow(p)) return gemm::dispatch_layout<gemm::TileNarrow>(p, env, stream);
    return gemm::dispatch_layout<gemm::TileSquare>(p, env, stream);
}

size_t gemm_workspace_bytes(const Problem& p, bool bf16, const Env& env) {
    return bf16 ? describe_gemm_bf16(p, env).workspace_bytes : describe_gemm_f32(p, env).workspace_bytes;
}

}  // namespace sn

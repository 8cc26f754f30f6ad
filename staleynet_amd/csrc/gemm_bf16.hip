// bf16-input / fp32-accumulate matrix-core GEMM for gfx950, the MI355X
// counterpart of the reference's TF32 tensor-core kernel
// (crates/staleynet-cuda/src/kernels/matmul.rs:357-448): same contract as the
// fp32 kernel, inputs rounded once (to bf16, nearest-even) as they are staged
// into LDS, products summed in fp32. Tolerance 2e-2 in the reference's metric.
//
// The operands stay fp32 in HBM (the boundary hands over f32 tensors), so the
// global loads, schedule, split-K and masks are those of gemm_mfma.hip. The
// LDS stage is bf16 in [BK/8 k-octets][ROWS + PAD][8 bf16] 16-byte slots;
// each loader writes a group of four k as one 8-byte half slot, and PAD is
// chosen per loader layout so the 16 lanes of a b64 write phase hit
// distinct banks (gemm_common.h). v_mfma_f32_32x32x16_bf16 takes eight
// consecutive k per lane: in chunk c, lane half h reads octet 2c + h of its
// row, one ds_read_b128 per 32-row fragment.
#include "gemm_common.h"

namespace sn {
namespace gemm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <class T, class LA, class LB>
__device__ __forceinline__ void multiply_tile_bf16(const uint16_t* __restrict__ lds_a,
                                                   const uint16_t* __restrict__ lds_b, f32x16 (&acc)[T::FM][T::FN],
                                                   int lane, int wave_m, int wave_n) {
    using OA = OctetPlanes<T::BM, T::BK, LA::BF16_PAD>;
    using OB = OctetPlanes<T::BN, T::BK, LB::BF16_PAD>;
    const int row = lane & 31;
    const int half = lane >> 5;
#pragma unroll
    for (int chunk = 0; chunk < T::BK / 16; ++chunk) {
        const int octet = 2 * chunk + half;
        bf16x8 a[T::FM], b[T::FN];
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
            a[i] = *reinterpret_cast<const bf16x8*>(lds_a + 8 * (octet * OA::PLANE + wave_m * T::WTM + 32 * i + row));
#pragma unroll
        for (int j = 0; j < T::FN; ++j)
            b[j] = *reinterpret_cast<const bf16x8*>(lds_b + 8 * (octet * OB::PLANE + wave_n * T::WTN + 32 * j + row));
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
#pragma unroll
            for (int j = 0; j < T::FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
}

template <class T, bool A_K, bool B_K, bool BUF>
__global__ __launch_bounds__(T::THREADS) void gemm_bf16_kernel(Args args) {
    using LA = LoaderFor<A_K, BUF, T::BM, T::BK, T::THREADS>;
    using LB = LoaderFor<B_K, BUF, T::BN, T::BK, T::THREADS>;
    using OA = OctetPlanes<T::BM, T::BK, LA::BF16_PAD>;
    using OB = OctetPlanes<T::BN, T::BK, LB::BF16_PAD>;
    __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][8 * OA::SLOTS];
    __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][8 * OB::SLOTS];

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

    LA load_a;
    LB load_b;
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
        load_a.store_bf16(lds_a[0], tid);
        load_b.store_bf16(lds_b[0], tid);
        __syncthreads();
        for (int step = 0; step < steps; ++step) {
            const int cur = step & 1;
            const bool more = step + 1 < steps;
            const int64_t k_next = k_begin + int64_t(step + 1) * T::BK;
            if (more) {
                load_a.load(a, args.lda, m0, args.m, k_next, args.k, tid);
                load_b.load(b, args.ldb, n0, args.n, k_next, args.k, tid);
            }
            multiply_tile_bf16<T, LA, LB>(lds_a[cur], lds_b[cur], acc, lane, wave_m, wave_n);
            if (more) {
                if (left_causal) load_a.mask_keys_after_query(m0, k_next, args.query_offset, tid);
                load_a.store_bf16(lds_a[cur ^ 1], tid);
                load_b.store_bf16(lds_b[cur ^ 1], tid);
            }
            __syncthreads();
        }
    }

    const bool partial = args.splits > 1;
    float* out = partial ? args.ws + ((batch_local * int64_t(args.splits) + split) * args.m) * args.n : c_batch;
    write_tile<T, BUF>(args, acc, out, m0, n0, wave_m, wave_n, lane, partial);
}

template <class T, bool A_K, bool B_K, bool BUF>
hipError_t launch_tiles_bf16(const Problem& p, const Env& env, const Plan& plan, hipStream_t stream) {
    const LaunchShape shape = tiled_shape<T>(p, plan, SN_PATH_NONE);
    if (shape.batches_per_launch < 1) return hipErrorInvalidConfiguration;
    Args args = make_args<T>(p, env, plan);
    const int64_t per_batch = int64_t(plan.tiles_m) * plan.tiles_n * plan.splits;
    const int64_t chunk = shape.batches_per_launch;
    for (int64_t first = 0; first < p.batch; first += chunk) {
        const int64_t count = std::min<int64_t>(chunk, p.batch - first);
        args.batch_base = first;
        hipLaunchKernelGGL((gemm_bf16_kernel<T, A_K, B_K, BUF>), dim3(unsigned(count * per_batch)), dim3(T::THREADS), 0,
                           stream, args);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (plan.splits > 1) return launch_splitk_reduce(p, env, plan.splits, stream);
    return hipSuccess;
}

template <class T, bool A_K, bool B_K>
hipError_t dispatch_path_bf16(const Problem& p, const Env& env, const Plan& plan, hipStream_t stream) {
    if (buffers_ok<T>(p)) return launch_tiles_bf16<T, A_K, B_K, true>(p, env, plan, stream);
    return launch_tiles_bf16<T, A_K, B_K, false>(p, env, plan, stream);
}

template <class T>
hipError_t dispatch_layout_bf16(const Problem& p, const Env& env, hipStream_t stream) {
    const Plan plan = plan_for<T>(p, env);
    if (p.a_k_contiguous && p.b_k_contiguous) return dispatch_path_bf16<T, true, true>(p, env, plan, stream);
    if (p.a_k_contiguous) return dispatch_path_bf16<T, true, false>(p, env, plan, stream);
    if (p.b_k_contiguous) return dispatch_path_bf16<T, false, true>(p, env, plan, stream);
    return dispatch_path_bf16<T, false, false>(p, env, plan, stream);
}

using TileSquare = Tile<128, 128, 32, 2, 2>;
using TileNarrow = Tile<256, 64, 32, 4, 1>;

}  // namespace

}  // namespace gemm

LaunchShape describe_gemm_bf16(const Problem& p, const Env& env) {
    if (gemm::bf16_wide_applies(p, env)) return gemm::describe_bf16_wide(p, env);
    if (gemm::bf16_staged_applies(p, env)) return gemm::describe_bf16_staged(p, env);
    if (gemm::bf16_dma_applies(p, env)) return gemm::describe_bf16_dma(p, env);
    if (p.n <= 64)
        return gemm::tiled_shape<gemm::TileNarrow>(p, gemm::plan_for<gemm::TileNarrow>(p, env), SN_PATH_BF16_REGISTER);
    return gemm::tiled_shape<gemm::TileSquare>(p, gemm::plan_for<gemm::TileSquare>(p, env), SN_PATH_BF16_REGISTER);
}

hipError_t launch_gemm_bf16(const Problem& p, const Env& env, hipStream_t stream) {
    if (gemm::bf16_wide_applies(p, env)) return gemm::launch_gemm_bf16_wide(p, env, stream);
    if (gemm::bf16_staged_applies(p, env)) return gemm::launch_gemm_bf16_staged(p, env, stream);
    if (gemm::bf16_dma_applies(p, env)) return gemm::launch_gemm_bf16_dma(p, env, stream);
    if (p.n <= 64) return gemm::dispatch_layout_bf16<gemm::TileNarrow>(p, env, stream);
    return gemm::dispatch_layout_bf16<gemm::TileSquare>(p, env, stream);
}

}  // namespace sn

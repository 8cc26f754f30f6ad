// bf16-input GEMM that rounds the fp32 operands as it loads them: the role of
// the reference's TF32 tensor-core kernel (crates/staleynet-cuda/src/kernels/
// matmul.rs:357-448) for large aligned products, with no staging pass.
//
// The operands stay fp32 in HBM, so per FLOP this kernel reads twice the bytes
// a kernel on bf16 copies would; it makes up for it with the largest tile the
// registers allow and a deep prefetch, instead of paying a separate pass that
// reads every operand, writes a bf16 copy and reads that copy back.
//  * 256 x 256 output tile, eight waves (two per SIMD) of 64 x 128;
//  * 32 k per step (the fp32 loaders' geometry, gemm_common.h), two steps of
//    global loads in flight in two register sets (128 KB per CU), so the
//    loads of a step have two steps' MFMAs to arrive;
//  * each step rounds the next step's registers to bf16 (nearest-even,
//    v_cvt_pk_bf16_f32) into the other of two bf16 LDS stages, between its
//    two 16-deep MFMA chunks, and issues the loads of the step after next;
//  * one barrier per step, waiting on LDS only (the loads in flight are
//    waited for by count, never drained).
// The LDS stage layout, loaders and epilogue are those of the register-staged
// bf16 kernel (gemm_bf16.hip), with the LDS writes addressed from one base per
// lane; v_mfma_f32_32x32x16_bf16 takes eight consecutive k per lane, one
// ds_read_b128 per 32-row fragment.
#include "gemm_common.h"

namespace sn {
namespace gemm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

using WideTile = Tile<256, 256, 32, 4, 2>;

template <int PENDING>
__device__ __forceinline__ void wait_vector_loads() {
    static_assert(PENDING >= 0 && PENDING < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (PENDING & 15) | ((PENDING >> 4) << 14));
}

// Barrier for the LDS stage hand-off: this wave's LDS accesses complete
// (lgkmcnt(0)), the global loads in flight stay in flight.
__device__ __forceinline__ void stage_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Hides a value's origin from the compiler, so that addresses derived from it
// are formed where they are used (one base register, immediate offsets)
// instead of being precomputed per vector and held across the loop.
__device__ __forceinline__ void launder(int& x) { asm volatile("" : "+v"(x)); }

// The fp32 loaders (gemm_common.h) with the bf16 LDS write addressed from one
// per-lane base: vector v of a K-contiguous loader is row tid / 8 + v x
// (THREADS / 8), 16 x THREADS / 8 bytes further into the octet plane; block
// v of a row-contiguous loader is rows 4 (tid / 8 + v x THREADS / 8) .. + 3.
template <int ROWS, int BK, int THREADS>
struct WideKLoader : KContiguousBufferLoader<ROWS, BK, THREADS> {
    using Base = KContiguousBufferLoader<ROWS, BK, THREADS>;
    using Base::reg;
    static_assert(Base::TOTAL % THREADS == 0 && THREADS % Base::GROUPS == 0, "whole vectors per thread");
    __device__ __forceinline__ void store_bf16(uint16_t* lds, int tid) const {
        using O = OctetPlanes<ROWS, BK, Base::BF16_PAD>;
        const int g = tid % Base::GROUPS;
        int base = ((g / 2) * O::PLANE + tid / Base::GROUPS) * 16 + 8 * (g % 2);
        launder(base);
        char* p = reinterpret_cast<char*>(lds) + base;
#pragma unroll
        for (int v = 0; v < Base::PER_THREAD; ++v)
            *reinterpret_cast<u32x2*>(p + v * (THREADS / Base::GROUPS) * 16) = pack_bf16(reg[v]);
    }
};

template <int ROWS, int BK, int THREADS>
struct WideRowLoader : RowContiguousBufferLoader<ROWS, BK, THREADS> {
    using Base = RowContiguousBufferLoader<ROWS, BK, THREADS>;
    using Base::reg;
    static_assert(Base::TOTAL % THREADS == 0 && THREADS % Base::GROUPS == 0, "whole blocks per thread");
    __device__ __forceinline__ void store_bf16(uint16_t* lds, int tid) const {
        using O = OctetPlanes<ROWS, BK, Base::BF16_PAD>;
        const int g = tid % Base::GROUPS;
        int base = ((g / 2) * O::PLANE + 4 * (tid / Base::GROUPS)) * 16 + 8 * (g % 2);
        launder(base);
        char* p = reinterpret_cast<char*>(lds) + base;
#pragma unroll
        for (int v = 0; v < Base::PER_THREAD; ++v)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f32x4 t = {reg[v][0][e], reg[v][1][e], reg[v][2][e], reg[v][3][e]};
                *reinterpret_cast<u32x2*>(p + (4 * v * (THREADS / Base::GROUPS) + e) * 16) = pack_bf16(t);
            }
    }
};

template <bool K_CONTIGUOUS, int ROWS, int BK, int THREADS>
using WideLoaderFor = typename std::conditional<K_CONTIGUOUS, WideKLoader<ROWS, BK, THREADS>,
                                                WideRowLoader<ROWS, BK, THREADS>>::type;

// Vector-memory instructions one loader issues per step.
template <class L>
constexpr int loads_per_step() {
    return sizeof(L::reg) / sizeof(f32x4);
}

template <bool A_K, bool B_K>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_bf16_wide_kernel(Args args) {
    using T = WideTile;
    using LA = WideLoaderFor<A_K, T::BM, T::BK, T::THREADS>;
    using LB = WideLoaderFor<B_K, T::BN, T::BK, T::THREADS>;
    using OA = OctetPlanes<T::BM, T::BK, LA::BF16_PAD>;
    using OB = OctetPlanes<T::BN, T::BK, LB::BF16_PAD>;
    constexpr int kSetLoads = loads_per_step<LA>() + loads_per_step<LB>();
    __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][8 * OA::SLOTS];
    __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][8 * OB::SLOTS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave / T::WAVES_N;
    const int wave_n = wave % T::WAVES_N;
    const int row = lane & 31;
    const int half = lane >> 5;

    int batch_local, split, tm, tn;
    tile_coordinates(blockIdx.x, gridDim.x, args.tiles_m, args.tiles_n, args.splits, batch_local, split, tm, tn);
    const int64_t batch = args.batch_base + batch_local;
    const int64_t m0 = int64_t(tm) * T::BM;
    const int64_t n0 = int64_t(tn) * T::BN;
    const int64_t k_begin = int64_t(split) * args.k_per_split;
    const int64_t k_end = min(args.k, k_begin + args.k_per_split);
    const float* a = args.a + batch * args.stride_a;
    const float* b = args.b + batch * args.stride_b;

    // Two register sets per operand: set s holds the steps of parity s.
    LA la[2];
    LB lb[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        la[s].init(args.lda, m0, args.m, tid);
        lb[s].init(args.ldb, n0, args.n, tid);
    }

    f32x16 acc[T::FM][T::FN];
#pragma unroll
    for (int i = 0; i < T::FM; ++i)
#pragma unroll
        for (int j = 0; j < T::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Loads of step `step` into register set S; past the slice's end every
    // load is out of range (it reads zeros and keeps the counts the waits
    // assume).
    auto issue = [&](auto set, int step) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        const int64_t k0 = k_begin + int64_t(step) * T::BK;
        la[S].load(a, args.lda, m0, args.m, k0, k_end, tid);
        lb[S].load(b, args.ldb, n0, args.n, k0, k_end, tid);
    };
    // Rounds register set S into LDS stage S.
    auto stage = [&](auto set) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        la[S].store_bf16(lds_a[S], tid);
        lb[S].store_bf16(lds_b[S], tid);
    };
    // Fragments of one 16-deep chunk of LDS stage S, and its MFMAs.
    auto read_chunk = [&](auto set, int c, bf16x8 (&fa)[T::FM], bf16x8 (&fb)[T::FN]) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        const int octet = 2 * c + half;
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
            fa[i] = *reinterpret_cast<const bf16x8*>(lds_a[S] + 8 * (octet * OA::PLANE + wave_m * T::WTM + 32 * i + row));
#pragma unroll
        for (int j = 0; j < T::FN; ++j)
            fb[j] = *reinterpret_cast<const bf16x8*>(lds_b[S] + 8 * (octet * OB::PLANE + wave_n * T::WTN + 32 * j + row));
    };
    auto multiply_chunk = [&](const bf16x8 (&fa)[T::FM], const bf16x8 (&fb)[T::FN]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
#pragma unroll
            for (int j = 0; j < T::FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    };
    // One step from LDS stage S: the first chunk's fragments and MFMAs, the
    // next stage's hand-off (`between`: the other register set's loads
    // waited for by count, rounded into the other stage, then reloaded),
    // and the second chunk.
    auto step_from = [&](auto set, auto between) __attribute__((always_inline)) {
        bf16x8 fa0[T::FM], fb0[T::FN], fa1[T::FM], fb1[T::FN];
        read_chunk(set, 0, fa0, fb0);
        multiply_chunk(fa0, fb0);
        wait_vector_loads<kSetLoads>();
        between();
        read_chunk(set, 1, fa1, fb1);
        multiply_chunk(fa1, fb1);
    };

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    const int steps = k_end > k_begin ? int((k_end - k_begin + T::BK - 1) / T::BK) : 0;
    if (steps > 0) {
        issue(I0{}, 0);
        issue(I1{}, 1);
        wait_vector_loads<kSetLoads>();  // set 0 (step 0) is in
        stage(I0{});
        issue(I0{}, 2);
        stage_barrier();
        // Step s computes from stage s % 2 while set (s + 1) % 2, holding
        // step s + 1, is rounded into the other stage and reloaded with step
        // s + 3; set s % 2 (step s + 2) stays in flight.
        for (int s = 0; s < steps; s += 2) {
            step_from(I0{}, [&]() __attribute__((always_inline)) {
                stage(I1{});
                issue(I1{}, s + 3);
            });
            stage_barrier();
            if (s + 1 >= steps) break;
            step_from(I1{}, [&]() __attribute__((always_inline)) {
                stage(I0{});
                issue(I0{}, s + 4);
            });
            stage_barrier();
        }
        wait_vector_loads<0>();
    }

    const bool partial = args.splits > 1;
    float* c_batch = args.c + batch * args.stride_c;
    float* out = partial ? args.ws + ((batch_local * int64_t(args.splits) + split) * args.m) * args.n : c_batch;
    write_tile<T, true>(args, acc, out, m0, n0, wave_m, wave_n, lane, partial);
}

// Split-K under the launch model of plan_for: one workgroup per CU, and the
// per-CU rate the split counts were measured with.
Plan wide_plan(const Problem& p, const Env& env) {
    SplitCost cost;
    cost.workgroups_per_cu = 1;
    cost.flops_per_cu = 3.5e12;
    return plan_for<WideTile>(p, env, cost);
}

template <bool A_K, bool B_K>
hipError_t launch_wide(const Problem& p, const Env& env, const Plan& plan, hipStream_t stream) {
    const LaunchShape shape = tiled_shape<WideTile>(p, plan, SN_PATH_BF16_WIDE);
    if (shape.batches_per_launch < 1) return hipErrorInvalidConfiguration;
    Args args = make_args<WideTile>(p, env, plan);
    const int64_t per_batch = int64_t(plan.tiles_m) * plan.tiles_n * plan.splits;
    const int64_t chunk = shape.batches_per_launch;
    for (int64_t first = 0; first < p.batch; first += chunk) {
        const int64_t count = std::min<int64_t>(chunk, p.batch - first);
        args.batch_base = first;
        hipLaunchKernelGGL((gemm_bf16_wide_kernel<A_K, B_K>), dim3(unsigned(count * per_batch)),
                           dim3(WideTile::THREADS), 0, stream, args);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (plan.splits > 1) return launch_splitk_reduce(p, env, plan.splits, stream);
    return hipSuccess;
}

}  // namespace

// Unmasked products with 128-bit-loadable operands (buffers_ok) whose output
// fills at least a quarter of a 256 x 256 tile each way, in every layout but
// NN (a K-contiguous left operand times a row-contiguous right one: the
// forward Linear). Measured on c2's products, this kernel takes the weight
// gradients (TN) from 310-549 to 397-574 TFLOP/s and the input gradients
// (NT) from 464-616 to 512-775 against staging both operands as bf16
// (gemm_dma.hip), while the staged path stays 1-5 % ahead on NN, whose
// right operand (the weight) is small to stage and whose row-contiguous
// loads cost this kernel more LDS writes per step.
bool bf16_wide_applies(const Problem& p, const Env& env) {
    if (p.a_k_contiguous && !p.b_k_contiguous) return false;
    if (p.mask != SN_MASK_NONE || p.m < 128 || p.n < 128 || !buffers_ok<WideTile>(p)) return false;
    const Plan plan = wide_plan(p, env);
    return plan.splits <= 1 || size_t(plan.splits) * size_t(p.m) * size_t(p.n) * sizeof(float) <= env.workspace_bytes;
}

LaunchShape describe_bf16_wide(const Problem& p, const Env& env) {
    return tiled_shape<WideTile>(p, wide_plan(p, env), SN_PATH_BF16_WIDE);
}

hipError_t launch_gemm_bf16_wide(const Problem& p, const Env& env, hipStream_t stream) {
    const Plan plan = wide_plan(p, env);
    if (p.a_k_contiguous && p.b_k_contiguous) return launch_wide<true, true>(p, env, plan, stream);
    if (p.a_k_contiguous) return launch_wide<true, false>(p, env, plan, stream);
    if (p.b_k_contiguous) return launch_wide<false, true>(p, env, plan, stream);
    return launch_wide<false, false>(p, env, plan, stream);
}

}  // namespace gemm
}  // namespace sn

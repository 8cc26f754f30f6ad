// fp32 matrix-core GEMM fed by direct global -> LDS loads.
//
// Same contract, tiles, grid schedule, masks, split-K and epilogue as the
// kernel in gemm_mfma.hip (which remains the path for operands that are not
// 16-byte aligned); what changes is how operand tiles reach LDS:
//
//  * `buffer_load_dwordx4 ... lds`: each lane's 16 bytes go straight from
//    memory (through L2) to LDS at M0 + 16 * lane, with no trip through
//    VGPRs. The main loop therefore holds no prefetch registers, does no
//    in-register transposes and issues no ds_write; a K-step is 8 load
//    instructions per wave, one barrier and the MFMAs. Lanes whose offset is
//    past the buffer bound write zeros, which pads edge tiles and the last
//    partial K-step.
//  * Since a lane's 16 bytes land in lane order, the LDS layout is chosen by
//    which global 16 bytes each lane fetches:
//      K-contiguous operand (A in NN/NT, B in NT/TT): 8 slots of 16 bytes
//      (k-groups) per row, row-major, slot g of row r holding k-group
//      g ^ ((r >> 1) & 7). Fragment reads (two ds_read_b128 per 32-row
//      fragment and 16-deep chunk) then hit 16 distinct 16-byte bank groups
//      per phase: conflict-free.
//      Row-contiguous operand (B in NN/TN, A in TN/TT): the natural [k][row]
//      layout, one k row of the tile per 512 bytes. A fragment is eight
//      ds_read_b32 (consecutive rows across lanes: conflict-free).
//  * Two LDS stages (32 KB each for 128x128), double-buffered: after one
//    barrier per K-step the next step's loads are issued into the other
//    stage and the current one is multiplied while they fly. The loop is
//    unrolled by two so that each half reads one statically known stage
//    array, which keeps the compiler from waiting on the in-flight loads
//    into the other stage before its LDS reads.
//
// Within a 16-deep chunk, lane half h feeds k = 8h + s to MFMA s on both
// operands (the same pairing as gemm_mfma.hip).
#include "gemm_common.h"

namespace sn {
namespace gemm {
namespace {

typedef __attribute__((address_space(3))) void* lds_void;

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, const void* lds, int32_t offset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void)lds, 16, offset, 0, 0, 0);
}

// K-contiguous operand: ROWS rows of 32 k per stage, ROWS / 8 load
// instructions of 8 rows each, ROWS / 32 per wave.
template <int ROWS>
struct OperandK {
    static constexpr int PER_WAVE = ROWS / 32;
    int32_t offset[PER_WAVE];  // byte offset from the tile origin, row part
    int32_t group_k[PER_WAVE]; // the k-group (times 4) this lane fetches

    __device__ __forceinline__ void init(int64_t ld, int64_t row0, int64_t rows, int lane, int wave) {
#pragma unroll
        for (int t = 0; t < PER_WAVE; ++t) {
            const int q = wave * PER_WAVE + t;
            const int r = 8 * q + (lane >> 3);
            const int g = (lane & 7) ^ ((r >> 1) & 7);
            group_k[t] = 4 * g;
            offset[t] = row0 + r < rows ? int32_t((int64_t(r) * ld + 4 * g) * 4) : kOutOfRange;
        }
    }

    // Loads k = k0 .. k0 + 31 of the tile into `stage`; k >= k_limit reads 0.
    __device__ __forceinline__ void issue(const f32x4* stage, const float* origin, int64_t k0, int64_t k_limit,
                                          int wave) const {
        const __amdgpu_buffer_rsrc_t rsrc = buffer_of(origin + k0);
        const bool partial = k0 + 32 > k_limit;
#pragma unroll
        for (int t = 0; t < PER_WAVE; ++t) {
            const int q = wave * PER_WAVE + t;
            const int32_t off = partial && k0 + group_k[t] >= k_limit ? kOutOfRange : offset[t];
            dma16(rsrc, stage + 64 * q, off);
        }
    }

    // k = 16 c + 8 h + (0..7) of tile row r.
    __device__ __forceinline__ void fragment(const f32x4* stage, int r, int c, int h, float (&v)[8]) const {
        const int swz = (r >> 1) & 7;
        const int g = 4 * c + 2 * h;
        const f32x4 lo = stage[8 * r + (g ^ swz)];
        const f32x4 hi = stage[8 * r + ((g + 1) ^ swz)];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            v[s] = lo[s];
            v[4 + s] = hi[s];
        }
    }
};

// Row-contiguous operand: 32 k rows of ROWS contiguous values per stage,
// ROWS / 8 load instructions of 256 values (64 lanes x 4), ROWS / 32 per wave.
template <int ROWS>
struct OperandR {
    static constexpr int PER_WAVE = ROWS / 32;
    static constexpr int LANES_PER_K = ROWS / 4;   // lanes covering one k row
    static constexpr int K_PER_LOAD = 64 / LANES_PER_K;
    int32_t offset[PER_WAVE];
    int k_of[PER_WAVE];

    __device__ __forceinline__ void init(int64_t ld, int64_t row0, int64_t rows, int lane, int wave) {
#pragma unroll
        for (int t = 0; t < PER_WAVE; ++t) {
            const int q = wave * PER_WAVE + t;
            const int k = K_PER_LOAD * q + lane / LANES_PER_K;
            const int c = 4 * (lane % LANES_PER_K);
            k_of[t] = k;
            offset[t] = row0 + c < rows ? int32_t((int64_t(k) * ld + c) * 4) : kOutOfRange;
        }
    }

    // origin: the tile's first row at k = 0; loads k rows k0 .. k0 + 31.
    __device__ __forceinline__ void issue(const f32x4* stage, const float* origin, int64_t ld, int64_t k0,
                                          int64_t k_limit, int wave) const {
        const __amdgpu_buffer_rsrc_t rsrc = buffer_of(origin + k0 * ld);
        const bool partial = k0 + 32 > k_limit;
#pragma unroll
        for (int t = 0; t < PER_WAVE; ++t) {
            const int q = wave * PER_WAVE + t;
            const int32_t off = partial && k0 + k_of[t] >= k_limit ? kOutOfRange : offset[t];
            dma16(rsrc, stage + 64 * q, off);
        }
    }

    __device__ __forceinline__ void fragment(const f32x4* stage, int r, int c, int h, float (&v)[8]) const {
        const float* base = reinterpret_cast<const float*>(stage) + (16 * c + 8 * h) * ROWS + r;
#pragma unroll
        for (int s = 0; s < 8; ++s) v[s] = base[s * ROWS];
    }
};

template <bool K_CONTIGUOUS, int ROWS>
using OperandFor = typename std::conditional<K_CONTIGUOUS, OperandK<ROWS>, OperandR<ROWS>>::type;

// Multiplies one staged K-step: two 16-deep chunks. Chunk 0's fragments
// are read first; then `prefetch` starts the next K-step's loads into the
// other stage, and those loads and chunk 1's fragment reads are interleaved
// one per MFMA with chunk 0's MFMAs, so that the wave issues them in the
// MFMAs' shadow instead of stalling on them (left alone, the scheduler
// issues each LDS read just before its first MFMA and waits on it there).
template <class T, bool A_K, bool B_K, class Prefetch>
__device__ __forceinline__ void multiply_stage(const OperandFor<A_K, T::BM>& oa, const OperandFor<B_K, T::BN>& ob,
                                               const f32x4* sa, const f32x4* sb, f32x16 (&acc)[T::FM][T::FN],
                                               int lane, int wave_m, int wave_n, Prefetch&& prefetch) {
    static_assert(T::BK == 32, "two 16-deep chunks per stage");
    const int row = lane & 31;
    const int half = lane >> 5;
    float av[2][T::FM][8], bv[2][T::FN][8];
    auto read = [&](int c) {
#pragma unroll
        for (int i = 0; i < T::FM; ++i) oa.fragment(sa, wave_m * T::WTM + 32 * i + row, c, half, av[c][i]);
#pragma unroll
        for (int j = 0; j < T::FN; ++j) ob.fragment(sb, wave_n * T::WTN + 32 * j + row, c, half, bv[c][j]);
    };
    auto multiply = [&](int c) {
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int i = 0; i < T::FM; ++i)
#pragma unroll
                for (int j = 0; j < T::FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[c][i][s], bv[c][j][s], acc[i][j], 0, 0, 0);
    };
    constexpr int DS = T::FM * (A_K ? 2 : 4) + T::FN * (B_K ? 2 : 4);
    constexpr int VM = T::BM / 32 + T::BN / 32;
    constexpr int MF = 8 * T::FM * T::FN;
    read(0);
    __builtin_amdgcn_sched_barrier(0);
    prefetch();
    read(1);
    multiply(0);
    multiply(1);
#pragma unroll
    for (int x = 0; x < VM; ++x) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
#pragma unroll
    for (int x = 0; x < DS; ++x) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * MF - VM - DS, 0);
}

// Causal-left tiles on the diagonal: zeroes the staged A values of the
// stored [query, key] matrix where key > query + offset. A K-contiguous:
// row = query, k = key; A transposed: row = key, k = query.
template <class T, bool A_K>
__device__ __forceinline__ void mask_stage(f32x4* sa, int64_t m0, int64_t k0, int64_t offset, int tid) {
    float* values = reinterpret_cast<float*>(sa);
    for (int e = tid; e < T::BM * T::BK; e += T::THREADS) {
        const int r = e / T::BK;
        const int kk = e % T::BK;
        const int64_t row = m0 + r, k = k0 + kk;
        const int64_t key_minus_query = A_K ? k - row : row - k;
        if (key_minus_query > offset) {
            const int index = A_K ? 4 * (8 * r + ((kk >> 2) ^ ((r >> 1) & 7))) + (kk & 3) : kk * T::BM + r;
            values[index] = 0.f;
        }
    }
}

// Waves per SIMD that the two LDS stages allow (160 KB of LDS per CU).
template <class T>
constexpr int dma_waves_per_eu() {
    return (160 * 1024 / ((T::BM + T::BN) * T::BK * 4 * 2)) * (T::THREADS / 64) / 4;
}

__device__ __forceinline__ void wait_loads() {
    // vmcnt(0), expcnt and lgkmcnt left at their maxima (gfx9 encoding).
    __builtin_amdgcn_s_waitcnt(0x0F70);
}

template <class T, bool A_K, bool B_K>
// LDS (two stages) already caps a CU at two 128x128 workgroups (two waves
// per SIMD): let the register allocator use that budget instead of
// squeezing for occupancy it cannot reach.
__global__ __launch_bounds__(T::THREADS) __attribute__((amdgpu_waves_per_eu(1, dma_waves_per_eu<T>())))
void gemm_f32_dma_kernel(Args args) {
    constexpr int A_SLOTS = T::BM * T::BK / 4;
    constexpr int B_SLOTS = T::BN * T::BK / 4;
    __shared__ f32x4 a0[A_SLOTS], b0[B_SLOTS], a1[A_SLOTS], b1[B_SLOTS];

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

    // Tile origins at k = 0: K-contiguous rows start at row * ld, row-contiguous
    // tiles at their first row.
    const float* a = args.a + batch * args.stride_a + (A_K ? m0 * args.lda : m0);
    const float* b = args.b + batch * args.stride_b + (B_K ? n0 * args.ldb : n0);

    OperandFor<A_K, T::BM> oa;
    OperandFor<B_K, T::BN> ob;
    oa.init(args.lda, m0, args.m, lane, wave);
    ob.init(args.ldb, n0, args.n, lane, wave);

    f32x16 acc[T::FM][T::FN];
#pragma unroll
    for (int i = 0; i < T::FM; ++i)
#pragma unroll
        for (int j = 0; j < T::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    auto issue = [&](const f32x4* sa, const f32x4* sb, int64_t k0) {
        if constexpr (A_K) oa.issue(sa, a, k0, args.k, wave);
        else oa.issue(sa, a, args.lda, k0, args.k, wave);
        if constexpr (B_K) ob.issue(sb, b, k0, args.k, wave);
        else ob.issue(sb, b, args.ldb, k0, args.k, wave);
    };
    // One K-step: wait for this stage's loads (every wave's, via the
    // barrier, which also retires every read of the other stage), start the
    // next step's loads into the other stage, multiply this one.
    auto step_on = [&](f32x4* sa, f32x4* sb, const f32x4* na, const f32x4* nb, int64_t k0, bool more) {
        wait_loads();
        __syncthreads();
        // Causal-left: A values past the diagonal are zeroed in LDS on the
        // K-steps that reach it (A K-contiguous: keys past the tile's first
        // query; A transposed: queries before the tile's last key).
        if (left_causal && (A_K ? k0 + T::BK - 1 > m0 + args.query_offset : k0 + args.query_offset < row_last)) {
            mask_stage<T, A_K>(sa, m0, k0, args.query_offset, tid);
            __syncthreads();
        }
        multiply_stage<T, A_K, B_K>(oa, ob, sa, sb, acc, lane, wave_m, wave_n, [&] {
            if (more) issue(na, nb, k0 + T::BK);
        });
    };

    const int steps = k_end > k_begin ? int((k_end - k_begin + T::BK - 1) / T::BK) : 0;
    if (steps > 0) {
        issue(a0, b0, k_begin);
        // Pairs of steps that both prefetch (branch-free bodies), then the
        // last one or two steps.
        int step = 0;
        for (; step + 2 < steps; step += 2) {
            const int64_t k0 = k_begin + int64_t(step) * T::BK;
            step_on(a0, b0, a1, b1, k0, true);
            step_on(a1, b1, a0, b0, k0 + T::BK, true);
        }
        const int64_t k0 = k_begin + int64_t(step) * T::BK;
        if (steps - step == 2) {
            step_on(a0, b0, a1, b1, k0, true);
            step_on(a1, b1, a0, b0, k0 + T::BK, false);
        } else {
            step_on(a0, b0, a1, b1, k0, false);
        }
    }

    const bool partial = args.splits > 1;
    float* out = partial ? args.ws + ((batch_local * int64_t(args.splits) + split) * args.m) * args.n : c_batch;
    write_tile<T, true>(args, acc, out, m0, n0, wave_m, wave_n, lane, partial);
}

template <class T, bool A_K, bool B_K>
hipError_t launch_dma_tiles(const Problem& p, const Env& env, hipStream_t stream) {
    const Plan plan = plan_for<T>(p, env);
    Args args = make_args<T>(p, env, plan);
    const int64_t per_batch = int64_t(plan.tiles_m) * plan.tiles_n * plan.splits;
    const int64_t chunk = batches_per_launch(per_batch, T::THREADS, p.batch);
    if (chunk < 1) return hipErrorInvalidConfiguration;
    for (int64_t first = 0; first < p.batch; first += chunk) {
        const int64_t count = std::min<int64_t>(chunk, p.batch - first);
        args.batch_base = first;
        hipLaunchKernelGGL((gemm_f32_dma_kernel<T, A_K, B_K>), dim3(unsigned(count * per_batch)), dim3(T::THREADS),
                           0, stream, args);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (plan.splits > 1) return launch_splitk_reduce(p, env, plan.splits, stream);
    return hipSuccess;
}

template <class T>
hipError_t launch_dma_layout(const Problem& p, const Env& env, hipStream_t stream) {
    if (p.a_k_contiguous && p.b_k_contiguous) return launch_dma_tiles<T, true, true>(p, env, stream);
    if (p.a_k_contiguous) return launch_dma_tiles<T, true, false>(p, env, stream);
    if (p.b_k_contiguous) return launch_dma_tiles<T, false, true>(p, env, stream);
    return launch_dma_tiles<T, false, false>(p, env, stream);
}

using DmaSquare = Tile<128, 128, 32, 2, 2>;
using DmaNarrow = Tile<128, 64, 32, 4, 1>;

}  // namespace

// Operands 16-byte aligned with 16-byte-multiple leading dimensions and
// batch strides, and every per-lane offset of one K-step within the buffer
// offset range (the same conditions as the buffer-load path of gemm_mfma.hip).
bool dma_applies(const Problem& p) {
    return p.n <= 64 ? buffers_ok<DmaNarrow>(p) : buffers_ok<DmaSquare>(p);
}

hipError_t launch_gemm_f32_dma(const Problem& p, const Env& env, hipStream_t stream) {
    if (p.n <= 64) return launch_dma_layout<DmaNarrow>(p, env, stream);
    return launch_dma_layout<DmaSquare>(p, env, stream);
}

}  // namespace gemm
}  // namespace sn

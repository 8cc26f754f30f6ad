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
//    of FM x FN MFMA blocks, accumulated in registers.
//  * LDS: both operands are staged K-contiguous ([row][BK + 4] floats), so a
//    lane's eight fragment values for a 16-deep chunk are two ds_read_b128.
//    Within one chunk, lane half h feeds k = 8h + s to MFMA s (s = 0..7);
//    A and B use the same assignment, so every product pairs the right k.
//    The +4 float pad puts the 8 rows one b128 phase reads in distinct banks.
//  * Global loads: 128-bit, coalesced along whichever dimension is
//    contiguous in memory. An operand contiguous along M or N (left stored
//    transposed, right stored row-major) is loaded as KB x 4 blocks and
//    transposed in registers on the way into LDS, so one kernel body serves
//    NN, NT, TN and TT.
//  * Double-buffered LDS with the next tile prefetched into registers while
//    the current one is multiplied: one barrier per BK step.
//  * Grid: blockIdx.x enumerates output tiles, remapped so each XCD (the
//    dispatcher deals workgroups round-robin over 8 XCDs, each with its own
//    L2) receives a contiguous run of a grouped raster; y = matrix of the
//    batch; z = K split. Split-K partial sums go to the context's workspace
//    and a second kernel adds them in split order (deterministic).
//  * Masks: causal output tiles that are entirely masked are not multiplied;
//    causal left operands limit each tile's K range to the visible part.
#include "gemm_internal.h"
#include "staleynet_gemm.h"

#include <algorithm>

namespace sn {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kXcds = 8;
constexpr int kGroupM = 8;

struct Args {
    const float* a;
    const float* b;
    float* c;
    float* ws;
    int64_t m, n, k;
    int64_t lda, ldb;
    int64_t stride_a, stride_b, stride_c;
    int64_t k_per_split;
    int64_t batch_base;
    int64_t query_offset;
    int32_t tiles_m, tiles_n;
    int32_t splits;
    int32_t accumulate;
    int32_t mask;
    float scale;
};

template <int BM_, int BN_, int BK_, int WAVES_M_, int WAVES_N_>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_;
    static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
    static constexpr int THREADS = 64 * WAVES_M * WAVES_N;
    static constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    static constexpr int FM = WTM / 32, FN = WTN / 32;
    static constexpr int STRIDE = BK + 4;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile is whole 32x32 blocks");
    static_assert(BK % 16 == 0, "BK is whole 16-deep chunks");
};

// Stages a ROWS x BK tile of a K-contiguous operand (element (r, k) at
// base[r * ld + k]) through registers into LDS laid out [ROWS][BK + 4].
template <int ROWS, int BK, int THREADS, bool VEC>
struct KContiguousLoader {
    static constexpr int STRIDE = BK + 4;
    static constexpr int PER_ROW = BK / 4;
    static constexpr int TOTAL = ROWS * PER_ROW;
    static constexpr int PER_THREAD = (TOTAL + THREADS - 1) / THREADS;
    f32x4 reg[PER_THREAD];

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int64_t row0, int64_t rows,
                                         int64_t k0, int64_t k_end, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int r = idx / PER_ROW;
            const int kc = (idx % PER_ROW) * 4;
            const int64_t gr = row0 + r;
            const int64_t gk = k0 + kc;
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if ((TOTAL % THREADS == 0 || idx < TOTAL) && gr < rows) {
                const float* src = base + gr * ld + gk;
                if constexpr (VEC) {
                    if (gk < k_end) x = *reinterpret_cast<const f32x4*>(src);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (gk + e < k_end) x[e] = src[e];
                }
            }
            reg[v] = x;
        }
    }

    // Zeroes elements (r, k) with k > r + offset (causal [query, key] operand
    // stored row-major: r = query, k = key).
    __device__ __forceinline__ void mask_keys_after_query(int64_t row0, int64_t k0, int64_t offset, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int64_t gr = row0 + idx / PER_ROW;
            const int64_t gk = k0 + (idx % PER_ROW) * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (gk + e > gr + offset) reg[v][e] = 0.f;
        }
    }

    __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            if (TOTAL % THREADS == 0 || idx < TOTAL) {
                const int r = idx / PER_ROW;
                const int kc = (idx % PER_ROW) * 4;
                *reinterpret_cast<f32x4*>(lds + r * STRIDE + kc) = reg[v];
            }
        }
    }
};

// Stages a ROWS x BK tile of an operand contiguous along its rows (element
// (r, k) at base[k * ld + r]). Each thread loads KB consecutive k of four
// consecutive rows and writes them transposed, K-contiguous, into LDS.
template <int ROWS, int BK, int THREADS, bool VEC>
struct RowContiguousLoader {
    static constexpr int STRIDE = BK + 4;
    static constexpr int KB_WANTED = ROWS * BK / (4 * THREADS);
    static constexpr int KB = KB_WANTED >= 4 ? 4 : (KB_WANTED >= 2 ? 2 : 1);
    static constexpr int QR = ROWS / 4;
    static constexpr int QK = BK / KB;
    static constexpr int TOTAL = QR * QK;
    static constexpr int PER_THREAD = (TOTAL + THREADS - 1) / THREADS;
    static_assert(ROWS % 4 == 0 && BK % KB == 0, "tile is whole blocks");
    f32x4 reg[PER_THREAD][KB];

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int64_t row0, int64_t rows,
                                         int64_t k0, int64_t k_end, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int rq = idx % QR;
            const int kq = idx / QR;
            const int64_t gr = row0 + rq * 4;
#pragma unroll
            for (int kk = 0; kk < KB; ++kk) {
                const int64_t gk = k0 + kq * KB + kk;
                f32x4 x = {0.f, 0.f, 0.f, 0.f};
                if ((TOTAL % THREADS == 0 || idx < TOTAL) && gk < k_end) {
                    const float* src = base + gk * ld + gr;
                    if constexpr (VEC) {
                        if (gr < rows) x = *reinterpret_cast<const f32x4*>(src);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (gr + e < rows) x[e] = src[e];
                    }
                }
                reg[v][kk] = x;
            }
        }
    }

    // Zeroes elements (r, k) with r > k + offset (causal [query, key] operand
    // stored row-major and read transposed: r = key, k = query).
    __device__ __forceinline__ void mask_keys_after_query(int64_t row0, int64_t k0, int64_t offset, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int64_t gr = row0 + (idx % QR) * 4;
#pragma unroll
            for (int kk = 0; kk < KB; ++kk) {
                const int64_t gk = k0 + (idx / QR) * KB + kk;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (gr + e > gk + offset) reg[v][kk][e] = 0.f;
            }
        }
    }

    __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            if (TOTAL % THREADS == 0 || idx < TOTAL) {
                const int rq = idx % QR;
                const int kq = idx / QR;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float* dst = lds + (rq * 4 + e) * STRIDE + kq * KB;
                    if constexpr (KB == 4) {
                        f32x4 t = {reg[v][0][e], reg[v][1][e], reg[v][2][e], reg[v][3][e]};
                        *reinterpret_cast<f32x4*>(dst) = t;
                    } else if constexpr (KB == 2) {
                        typedef float f32x2 __attribute__((ext_vector_type(2)));
                        f32x2 t = {reg[v][0][e], reg[v][1][e]};
                        *reinterpret_cast<f32x2*>(dst) = t;
                    } else {
                        dst[0] = reg[v][0][e];
                    }
                }
            }
        }
    }
};

template <bool K_CONTIGUOUS, int ROWS, int BK, int THREADS, bool VEC>
using LoaderFor = typename std::conditional<K_CONTIGUOUS, KContiguousLoader<ROWS, BK, THREADS, VEC>,
                                            RowContiguousLoader<ROWS, BK, THREADS, VEC>>::type;

// Block id -> (tile row, tile column). Consecutive workgroup ids land on
// different XCDs, so ids are first regrouped so that each XCD holds one
// contiguous range, then that range walks a raster grouped kGroupM tile rows
// high, keeping the A rows and B columns an XCD reuses in its own L2.
__device__ __forceinline__ void tile_coordinates(int bid, int blocks, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int xcd = bid % kXcds;
    const int local = bid / kXcds;
    const int q = blocks / kXcds;
    const int r = blocks % kXcds;
    const int id = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + local;
    const int per_group = kGroupM * tiles_n;
    const int group = id / per_group;
    const int first_m = group * kGroupM;
    const int group_rows = min(tiles_m - first_m, kGroupM);
    const int within = id % per_group;
    tm = first_m + within % group_rows;
    tn = within / group_rows;
}

template <class T>
__device__ __forceinline__ void multiply_tile(const float* __restrict__ lds_a, const float* __restrict__ lds_b,
                                              f32x16 (&acc)[T::FM][T::FN], int lane, int wave_m, int wave_n) {
    const int row = lane & 31;
    const int half = lane >> 5;
#pragma unroll
    for (int chunk = 0; chunk < T::BK / 16; ++chunk) {
        f32x4 a_lo[T::FM], a_hi[T::FM], b_lo[T::FN], b_hi[T::FN];
#pragma unroll
        for (int i = 0; i < T::FM; ++i) {
            const float* pa = lds_a + (wave_m * T::WTM + 32 * i + row) * T::STRIDE + 16 * chunk + 8 * half;
            a_lo[i] = *reinterpret_cast<const f32x4*>(pa);
            a_hi[i] = *reinterpret_cast<const f32x4*>(pa + 4);
        }
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
            const float* pb = lds_b + (wave_n * T::WTN + 32 * j + row) * T::STRIDE + 16 * chunk + 8 * half;
            b_lo[j] = *reinterpret_cast<const f32x4*>(pb);
            b_hi[j] = *reinterpret_cast<const f32x4*>(pb + 4);
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

// The reference's combine (kernels/matmul.rs:166-168) with the product and
// the sum rounded separately, as the reference rounds them.
__device__ __forceinline__ void write_output(float* dst, float sum, float scale, bool accumulate) {
#pragma clang fp contract(off)
    const float scaled = scale * sum;
    *dst = accumulate ? *dst + scaled : scaled;
}

template <class T, bool A_K, bool B_K, bool VEC_A, bool VEC_B>
__global__ __launch_bounds__(T::THREADS) void gemm_f32_kernel(Args args) {
    __shared__ __attribute__((aligned(16))) float lds_a[2][T::BM * T::STRIDE];
    __shared__ __attribute__((aligned(16))) float lds_b[2][T::BN * T::STRIDE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave / T::WAVES_N;
    const int wave_n = wave % T::WAVES_N;

    int tm, tn;
    tile_coordinates(blockIdx.x, gridDim.x, args.tiles_m, args.tiles_n, tm, tn);
    const int64_t batch = args.batch_base + blockIdx.y;
    const int split = blockIdx.z;
    const int64_t m0 = int64_t(tm) * T::BM;
    const int64_t n0 = int64_t(tn) * T::BN;

    const int64_t row_last = min(m0 + T::BM, args.m) - 1;
    const bool output_causal = args.mask == int(SN_MASK_CAUSAL_OUTPUT);
    const bool left_causal = args.mask == int(SN_MASK_CAUSAL_LEFT);
    float* c_batch = args.c + batch * args.stride_c;

    if (output_causal && n0 > row_last + args.query_offset) {
        // Every output of this tile is masked: the product is 0 there.
        if (!args.accumulate) {
            for (int e = tid; e < T::BM * T::BN; e += T::THREADS) {
                const int64_t r = m0 + e / T::BN;
                const int64_t col = n0 + e % T::BN;
                if (r < args.m && col < args.n) c_batch[r * args.n + col] = 0.f;
            }
        }
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

    LoaderFor<A_K, T::BM, T::BK, T::THREADS, VEC_A> load_a;
    LoaderFor<B_K, T::BN, T::BK, T::THREADS, VEC_B> load_b;

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

    // Accumulator element r of a 32x32 block holds row 8(r/4) + 4*half + r%4
    // and column lane%32 of that block.
    const int col_in_block = lane & 31;
    const int half = lane >> 5;
    if (args.splits > 1) {
        float* part = args.ws + ((blockIdx.y * int64_t(args.splits) + split) * args.m) * args.n;
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
#pragma unroll
            for (int j = 0; j < T::FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t row = m0 + wave_m * T::WTM + 32 * i + 8 * (r / 4) + 4 * half + (r % 4);
                    const int64_t col = n0 + wave_n * T::WTN + 32 * j + col_in_block;
                    if (row < args.m && col < args.n) part[row * args.n + col] = acc[i][j][r];
                }
        return;
    }
    const bool accumulate = args.accumulate != 0;
#pragma unroll
    for (int i = 0; i < T::FM; ++i)
#pragma unroll
        for (int j = 0; j < T::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wave_m * T::WTM + 32 * i + 8 * (r / 4) + 4 * half + (r % 4);
                const int64_t col = n0 + wave_n * T::WTN + 32 * j + col_in_block;
                if (row < args.m && col < args.n) {
                    float* dst = c_batch + row * args.n + col;
                    if (output_causal && col > row + args.query_offset) {
                        if (!accumulate) *dst = 0.f;
                    } else {
                        write_output(dst, acc[i][j][r], args.scale, accumulate);
                    }
                }
            }
}

// Adds the split partial sums of each output in split order, then applies
// the reference's combine.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, float* c, int64_t m,
                                                            int64_t n, int64_t batches, int splits,
                                                            int64_t stride_c, float scale, int accumulate) {
    const int64_t per_matrix = m * n;
    const int64_t total = per_matrix * batches;
    for (int64_t idx = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; idx < total;
         idx += int64_t(gridDim.x) * blockDim.x) {
#pragma clang fp contract(off)
        const int64_t bat = idx / per_matrix;
        const int64_t e = idx % per_matrix;
        const float* src = ws + bat * splits * per_matrix + e;
        float sum = 0.f;
        for (int s = 0; s < splits; ++s) sum = sum + src[s * per_matrix];
        write_output(c + bat * stride_c + e, sum, scale, accumulate != 0);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// 128-bit loads need the contiguous dimension, the leading dimension and the
// batch stride to be multiples of 4 floats and the base 16-byte aligned.
bool vector_ok(const float* base, bool k_contiguous, int64_t rows, int64_t k, int64_t ld, int64_t stride) {
    const int64_t contiguous = k_contiguous ? k : rows;
    return aligned16(base) && contiguous % 4 == 0 && ld % 4 == 0 && stride % 4 == 0;
}

struct Plan {
    int tiles_m, tiles_n;
    int splits;
    int64_t k_per_split;
};

template <class T>
Plan plan_for(const Problem& p, const Env& env) {
    Plan plan;
    plan.tiles_m = int((p.m + T::BM - 1) / T::BM);
    plan.tiles_n = int((p.n + T::BN - 1) / T::BN);
    plan.splits = 1;
    plan.k_per_split = std::max<int64_t>(p.k, 1);
    const int64_t tiles = int64_t(plan.tiles_m) * plan.tiles_n * p.batch;
    // Products whose output tiles cannot fill every CU a few times over
    // (the K = 32768 weight gradients) split K instead, in BK-aligned slices
    // of at least 8 steps, as far as the workspace allows.
    const int64_t target = int64_t(env.cu_count) * 3;
    const int64_t k_steps = (p.k + T::BK - 1) / T::BK;
    if (p.mask == SN_MASK_NONE && tiles < target && k_steps >= 16 && p.batch == 1) {
        int64_t splits = std::min<int64_t>((target + tiles - 1) / tiles, k_steps / 8);
        const int64_t per_split_bytes = p.m * p.n * int64_t(sizeof(float));
        if (per_split_bytes > 0) splits = std::min<int64_t>(splits, int64_t(env.workspace_bytes) / per_split_bytes);
        if (splits >= 2) {
            const int64_t steps_per_split = (k_steps + splits - 1) / splits;
            plan.k_per_split = steps_per_split * T::BK;
            plan.splits = int((p.k + plan.k_per_split - 1) / plan.k_per_split);
        }
    }
    return plan;
}

template <class T, bool A_K, bool B_K, bool VEC_A, bool VEC_B>
hipError_t launch_tiles(const Problem& p, const Env& env, const Plan& plan, hipStream_t stream) {
    Args args;
    args.a = p.a;
    args.b = p.b;
    args.c = p.c;
    args.ws = env.workspace;
    args.m = p.m;
    args.n = p.n;
    args.k = p.k;
    args.lda = p.lda;
    args.ldb = p.ldb;
    args.stride_a = p.stride_a;
    args.stride_b = p.stride_b;
    args.stride_c = p.stride_c;
    args.k_per_split = plan.k_per_split;
    args.query_offset = p.query_offset;
    args.tiles_m = plan.tiles_m;
    args.tiles_n = plan.tiles_n;
    args.splits = plan.splits;
    args.accumulate = p.accumulate ? 1 : 0;
    args.mask = int(p.mask);
    args.scale = p.scale;
    const int64_t tile_count = int64_t(plan.tiles_m) * plan.tiles_n;
    // Work-items per grid dimension must stay below 2^32.
    if (tile_count * T::THREADS >= (int64_t(1) << 32)) return hipErrorInvalidConfiguration;
    const int blocks = int(tile_count);
    for (int64_t first = 0; first < p.batch; first += 65535) {
        const int64_t count = std::min<int64_t>(65535, p.batch - first);
        args.batch_base = first;
        hipLaunchKernelGGL((gemm_f32_kernel<T, A_K, B_K, VEC_A, VEC_B>), dim3(blocks, unsigned(count), plan.splits),
                           dim3(T::THREADS), 0, stream, args);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (plan.splits > 1) {
        const int64_t total = p.m * p.n * p.batch;
        const int64_t grid = std::min<int64_t>((total + 255) / 256, int64_t(env.cu_count) * 16);
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(unsigned(grid)), dim3(256), 0, stream, env.workspace, p.c, p.m,
                           p.n, p.batch, plan.splits, p.stride_c, p.scale, p.accumulate ? 1 : 0);
        return hipGetLastError();
    }
    return hipSuccess;
}

template <class T, bool A_K, bool B_K>
hipError_t dispatch_vec(const Problem& p, const Env& env, const Plan& plan, hipStream_t stream) {
    const bool va = vector_ok(p.a, A_K, p.m, p.k, p.lda, p.stride_a);
    const bool vb = vector_ok(p.b, B_K, p.n, p.k, p.ldb, p.stride_b);
    if (va && vb) return launch_tiles<T, A_K, B_K, true, true>(p, env, plan, stream);
    if (va) return launch_tiles<T, A_K, B_K, true, false>(p, env, plan, stream);
    if (vb) return launch_tiles<T, A_K, B_K, false, true>(p, env, plan, stream);
    return launch_tiles<T, A_K, B_K, false, false>(p, env, plan, stream);
}

template <class T>
hipError_t dispatch_layout(const Problem& p, const Env& env, hipStream_t stream) {
    const Plan plan = plan_for<T>(p, env);
    if (p.a_k_contiguous && p.b_k_contiguous) return dispatch_vec<T, true, true>(p, env, plan, stream);
    if (p.a_k_contiguous) return dispatch_vec<T, true, false>(p, env, plan, stream);
    if (p.b_k_contiguous) return dispatch_vec<T, false, true>(p, env, plan, stream);
    return dispatch_vec<T, false, false>(p, env, plan, stream);
}

using TileSquare = Tile<128, 128, 16, 2, 2>;  // 4 waves of 64x64
using TileNarrow = Tile<256, 64, 16, 4, 1>;   // N <= 64 (attention head dim)

bool use_narrow(const Problem& p) { return p.n <= 64; }

}  // namespace

size_t gemm_workspace_bytes(const Problem& p, bool bf16, const Env& env) {
    (void)bf16;
    const Plan plan = use_narrow(p) ? plan_for<TileNarrow>(p, env) : plan_for<TileSquare>(p, env);
    return plan.splits > 1 ? size_t(plan.splits) * size_t(p.m) * size_t(p.n) * sizeof(float) : 0;
}

hipError_t launch_gemm_f32(const Problem& p, const Env& env, hipStream_t stream) {
    if (use_narrow(p)) return dispatch_layout<TileNarrow>(p, env, stream);
    return dispatch_layout<TileSquare>(p, env, stream);
}

}  // namespace sn

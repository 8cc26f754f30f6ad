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
//  * Global loads are 128-bit and coalesced along whichever dimension is
//    contiguous in memory. A K-contiguous operand is read as 8 lanes per row
//    (128 contiguous bytes); an operand contiguous along M or N (left stored
//    transposed, right stored row-major) is read as 4x4 blocks, 8 lanes on
//    8 k-quads of one 4-row group, and transposed in registers on the way
//    into LDS. One kernel body serves NN, NT, TN and TT.
//  * Double-buffered LDS; the next tile is prefetched into registers while
//    the current one is multiplied: one barrier per BK step.
//  * Grid: blockIdx.x enumerates output tiles, remapped so each XCD (the
//    dispatcher deals workgroups round-robin over 8 XCDs, each with its own
//    L2) receives a contiguous run of whole K splits, each walked as a
//    grouped raster; y = matrix of the batch. Split-K partial sums go to the
//    context's workspace
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

// Buffer addressing: a 128-bit descriptor (base, record bound, format) in
// scalar registers plus a 32-bit per-lane byte offset. Loads at an offset
// past the bound return 0 and stores there are dropped, so edge tiles and
// partial K-steps select kOutOfRange instead of branching per lane.
constexpr int32_t kRecords = 0x7FFFFFFF;
constexpr int32_t kOutOfRange = int32_t(0x80000000u);
constexpr int32_t kRawBufferFormat = 0x00020000;  // 32-bit data format, gfx9 family
// Per-lane offsets stay below this many bytes (checked on the host).
constexpr int64_t kMaxBufferOffset = (int64_t(1) << 31) - 256;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, kRecords, kRawBufferFormat);
}

__device__ __forceinline__ f32x4 buffer_load4(__amdgpu_buffer_rsrc_t rsrc, int32_t offset) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, 0));
}

__device__ __forceinline__ float buffer_load1(__amdgpu_buffer_rsrc_t rsrc, int32_t offset) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, offset, 0, 0));
}

__device__ __forceinline__ void buffer_store1(__amdgpu_buffer_rsrc_t rsrc, int32_t offset, float value) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, value), rsrc, offset, 0, 0);
}

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
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile is whole 32x32 blocks");
    static_assert(BK == 32, "the loaders' lane mappings assume 8 k-groups per tile");
};

// LDS geometry of one operand tile: BK/4 planes (k-groups) of ROWS + 1
// slots; slot (g, r) holds k = 4g .. 4g+3 of row r.
template <int ROWS, int BK>
struct Planes {
    static constexpr int PLANE = ROWS + 1;
    static constexpr int GROUPS = BK / 4;
    static constexpr int SLOTS = GROUPS * PLANE;
};

// Operand loaders. Each stages a ROWS x BK tile of one operand per K-step
// through registers into the LDS layout above. `init` runs once per tile,
// `load` issues the global reads for the K-step starting at k0 (reading 0
// outside the matrix), `store` writes the registers to one LDS stage.
//
// K-contiguous operands (element (r, k) at base[r * ld + k]): vector v of a
// thread is row idx / 8, k-group idx % 8 (idx = tid + v * THREADS), so the 8
// lanes of a row read 128 contiguous bytes and write 8 different k-groups.
//
// Row-contiguous operands (element (r, k) at base[k * ld + r]): block v of a
// thread is k-quad idx % 8 and rows 4 * (idx / 8) .. +3, read as four 16-byte
// row pieces and written transposed, one slot per row.

// Scalar fallback for operands that are unaligned or too large for 32-bit
// buffer offsets: one bounds check per element.
template <int ROWS, int BK, int THREADS>
struct KContiguousScalarLoader {
    using P = Planes<ROWS, BK>;
    static constexpr int TOTAL = ROWS * P::GROUPS;
    static constexpr int PER_THREAD = (TOTAL + THREADS - 1) / THREADS;
    f32x4 reg[PER_THREAD];

    __device__ __forceinline__ void init(int64_t, int64_t, int64_t, int) {}

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int64_t row0, int64_t rows,
                                         int64_t k0, int64_t k_total, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int64_t gr = row0 + idx / P::GROUPS;
            const int64_t gk = k0 + (idx % P::GROUPS) * 4;
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if ((TOTAL % THREADS == 0 || idx < TOTAL) && gr < rows) {
                const float* src = base + gr * ld + gk;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (gk + e < k_total) x[e] = src[e];
            }
            reg[v] = x;
        }
    }

    // Zeroes elements (r, k) with k > r + offset (a causal [query, key]
    // operand stored row-major: r = query, k = key).
    __device__ __forceinline__ void mask_keys_after_query(int64_t row0, int64_t k0, int64_t offset, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int64_t gr = row0 + idx / P::GROUPS;
            const int64_t gk = k0 + (idx % P::GROUPS) * 4;
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
                const int slot = (idx % P::GROUPS) * P::PLANE + idx / P::GROUPS;
                *reinterpret_cast<f32x4*>(lds + 4 * slot) = reg[v];
            }
        }
    }
};

// 128-bit buffer loads; needs K % 4 == 0, ld % 4 == 0 and a 16-byte aligned
// base, so a vector is either wholly inside the matrix or wholly outside.
template <int ROWS, int BK, int THREADS>
struct KContiguousBufferLoader : KContiguousScalarLoader<ROWS, BK, THREADS> {
    using Base = KContiguousScalarLoader<ROWS, BK, THREADS>;
    using P = typename Base::P;
    using Base::PER_THREAD;
    using Base::TOTAL;
    using Base::reg;
    int32_t offset[PER_THREAD];  // bytes from the K-step's tile origin; kOutOfRange past the last row

    __device__ __forceinline__ void init(int64_t ld, int64_t row0, int64_t rows, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int r = idx / P::GROUPS;
            const bool valid = (TOTAL % THREADS == 0 || idx < TOTAL) && row0 + r < rows;
            offset[v] = valid ? int32_t((r * ld + (idx % P::GROUPS) * 4) * 4) : kOutOfRange;
        }
    }

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int64_t row0, int64_t,
                                         int64_t k0, int64_t k_total, int tid) {
        const __amdgpu_buffer_rsrc_t rsrc = buffer_of(base + row0 * ld + k0);
        const bool k_valid = k0 + (tid % P::GROUPS) * 4 < k_total;  // the same k-group for every v
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) reg[v] = buffer_load4(rsrc, k_valid ? offset[v] : kOutOfRange);
    }
};

template <int ROWS, int BK, int THREADS>
struct RowContiguousScalarLoader {
    using P = Planes<ROWS, BK>;
    static constexpr int TOTAL = P::GROUPS * (ROWS / 4);
    static constexpr int PER_THREAD = (TOTAL + THREADS - 1) / THREADS;
    static_assert(ROWS % 4 == 0, "tile is whole 4-row groups");
    f32x4 reg[PER_THREAD][4];  // [v][kk]: rows 4q..4q+3 at k = 4g + kk

    __device__ __forceinline__ void init(int64_t, int64_t, int64_t, int) {}

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int64_t row0, int64_t rows,
                                         int64_t k0, int64_t k_total, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int64_t gr = row0 + (idx / P::GROUPS) * 4;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const int64_t gk = k0 + (idx % P::GROUPS) * 4 + kk;
                f32x4 x = {0.f, 0.f, 0.f, 0.f};
                if ((TOTAL % THREADS == 0 || idx < TOTAL) && gk < k_total) {
                    const float* src = base + gk * ld + gr;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (gr + e < rows) x[e] = src[e];
                }
                reg[v][kk] = x;
            }
        }
    }

    // Zeroes elements (r, k) with r > k + offset (a causal [query, key]
    // operand stored row-major and read transposed: r = key, k = query).
    __device__ __forceinline__ void mask_keys_after_query(int64_t row0, int64_t k0, int64_t offset, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int64_t gr = row0 + (idx / P::GROUPS) * 4;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const int64_t gk = k0 + (idx % P::GROUPS) * 4 + kk;
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
                const int first = (idx % P::GROUPS) * P::PLANE + (idx / P::GROUPS) * 4;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    f32x4 t = {reg[v][0][e], reg[v][1][e], reg[v][2][e], reg[v][3][e]};
                    *reinterpret_cast<f32x4*>(lds + 4 * (first + e)) = t;
                }
            }
        }
    }
};

// 128-bit buffer loads; needs rows % 4 == 0, ld % 4 == 0 and a 16-byte
// aligned base.
template <int ROWS, int BK, int THREADS>
struct RowContiguousBufferLoader : RowContiguousScalarLoader<ROWS, BK, THREADS> {
    using Base = RowContiguousScalarLoader<ROWS, BK, THREADS>;
    using P = typename Base::P;
    using Base::PER_THREAD;
    using Base::TOTAL;
    using Base::reg;
    int32_t offset[PER_THREAD][4];  // bytes from the K-step's tile origin; kOutOfRange past the last row

    __device__ __forceinline__ void init(int64_t ld, int64_t row0, int64_t rows, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int r = (idx / P::GROUPS) * 4;
            const bool valid = (TOTAL % THREADS == 0 || idx < TOTAL) && row0 + r < rows;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                offset[v][kk] = valid ? int32_t((((idx % P::GROUPS) * 4 + kk) * ld + r) * 4) : kOutOfRange;
        }
    }

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int64_t row0, int64_t,
                                         int64_t k0, int64_t k_total, int tid) {
        const __amdgpu_buffer_rsrc_t rsrc = buffer_of(base + k0 * ld + row0);
        const int64_t k_first = k0 + (tid % P::GROUPS) * 4;  // the same k-quad for every v
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const bool k_valid = k_first + kk < k_total;
#pragma unroll
            for (int v = 0; v < PER_THREAD; ++v) reg[v][kk] = buffer_load4(rsrc, k_valid ? offset[v][kk] : kOutOfRange);
        }
    }
};

template <bool K_CONTIGUOUS, bool BUFFER, int ROWS, int BK, int THREADS>
using LoaderFor = typename std::conditional<
    K_CONTIGUOUS,
    typename std::conditional<BUFFER, KContiguousBufferLoader<ROWS, BK, THREADS>,
                              KContiguousScalarLoader<ROWS, BK, THREADS>>::type,
    typename std::conditional<BUFFER, RowContiguousBufferLoader<ROWS, BK, THREADS>,
                              RowContiguousScalarLoader<ROWS, BK, THREADS>>::type>::type;

// Block id -> (K split, tile row, tile column). Consecutive workgroup ids
// land on different XCDs, so ids are first regrouped so that each XCD holds
// one contiguous range; that range covers whole K splits in turn (the tiles
// of a split share its slices of A and B) and, within a split, walks a
// raster grouped kGroupM tile rows high, keeping the A rows and B columns an
// XCD reuses in its own L2.
__device__ __forceinline__ void tile_coordinates(int bid, int blocks, int tiles_m, int tiles_n, int& split, int& tm,
                                                 int& tn) {
    const int xcd = bid % kXcds;
    const int local = bid / kXcds;
    const int q = blocks / kXcds;
    const int r = blocks % kXcds;
    const int linear = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + local;
    const int tiles = tiles_m * tiles_n;
    split = linear / tiles;
    const int id = linear % tiles;
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

// The reference's combine (kernels/matmul.rs:166-168), the product and the
// sum rounded separately as the reference rounds them.
__device__ __forceinline__ void write_output(float* dst, float sum, float scale, bool accumulate) {
#pragma clang fp contract(off)
    const float scaled = scale * sum;
    *dst = accumulate ? *dst + scaled : scaled;
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

    int split, tm, tn;
    tile_coordinates(blockIdx.x, gridDim.x, args.tiles_m, args.tiles_n, split, tm, tn);
    const int64_t batch = args.batch_base + blockIdx.y;
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

    // Accumulator element r of a 32x32 block holds row 8(r/4) + 4*half + r%4
    // and column lane%32 of that block.
    const int col_in_block = lane & 31;
    const int half = lane >> 5;
    const bool accumulate = args.accumulate != 0;
    const bool partial = args.splits > 1;
    float* out = partial ? args.ws + ((blockIdx.y * int64_t(args.splits) + split) * args.m) * args.n : c_batch;
    if constexpr (BUF) {
        // Offsets from the tile origin; kOutOfRange drops stores outside the matrix.
        const __amdgpu_buffer_rsrc_t rsrc = buffer_of(out + m0 * args.n + n0);
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
#pragma unroll
            for (int j = 0; j < T::FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = wave_m * T::WTM + 32 * i + 8 * (r / 4) + 4 * half + (r % 4);
                    const int col = wave_n * T::WTN + 32 * j + col_in_block;
                    const bool inside = m0 + row < args.m && n0 + col < args.n;
                    const int32_t offset = inside ? int32_t((row * args.n + col) * 4) : kOutOfRange;
                    const float sum = acc[i][j][r];
                    if (partial) {
                        buffer_store1(rsrc, offset, sum);
                    } else if (output_causal && n0 + col > m0 + row + args.query_offset) {
                        if (!accumulate) buffer_store1(rsrc, offset, 0.f);
                    } else {
#pragma clang fp contract(off)
                        const float scaled = args.scale * sum;
                        buffer_store1(rsrc, offset, accumulate ? buffer_load1(rsrc, offset) + scaled : scaled);
                    }
                }
    } else {
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
#pragma unroll
            for (int j = 0; j < T::FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t row = m0 + wave_m * T::WTM + 32 * i + 8 * (r / 4) + 4 * half + (r % 4);
                    const int64_t col = n0 + wave_n * T::WTN + 32 * j + col_in_block;
                    if (row < args.m && col < args.n) {
                        float* dst = out + row * args.n + col;
                        if (partial) {
                            *dst = acc[i][j][r];
                        } else if (output_causal && col > row + args.query_offset) {
                            if (!accumulate) *dst = 0.f;
                        } else {
                            write_output(dst, acc[i][j][r], args.scale, accumulate);
                        }
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

// Buffer loads take 128 bits at a time, so the contiguous dimension, the
// leading dimension and the batch stride must be multiples of 4 floats and
// the base 16-byte aligned; per-lane offsets within one K-step tile must
// also fit the 31-bit range.
bool buffer_ok(const float* base, bool k_contiguous, int64_t rows, int64_t k, int64_t ld, int64_t stride,
               int tile_rows, int bk) {
    const int64_t contiguous = k_contiguous ? k : rows;
    const int64_t span = k_contiguous ? (int64_t(tile_rows) * ld + bk) * 4 : (int64_t(bk) * ld + tile_rows) * 4;
    return aligned16(base) && contiguous % 4 == 0 && ld % 4 == 0 && stride % 4 == 0 && span < kMaxBufferOffset;
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

template <class T, bool A_K, bool B_K, bool BUF>
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
    const int64_t tile_count = int64_t(plan.tiles_m) * plan.tiles_n * plan.splits;
    // Work-items per grid dimension must stay below 2^32.
    if (tile_count * T::THREADS >= (int64_t(1) << 32)) return hipErrorInvalidConfiguration;
    const int blocks = int(tile_count);
    for (int64_t first = 0; first < p.batch; first += 65535) {
        const int64_t count = std::min<int64_t>(65535, p.batch - first);
        args.batch_base = first;
        hipLaunchKernelGGL((gemm_f32_kernel<T, A_K, B_K, BUF>), dim3(blocks, unsigned(count)),
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
hipError_t dispatch_path(const Problem& p, const Env& env, const Plan& plan, hipStream_t stream) {
    const bool buffers = buffer_ok(p.a, A_K, p.m, p.k, p.lda, p.stride_a, T::BM, T::BK) &&
                         buffer_ok(p.b, B_K, p.n, p.k, p.ldb, p.stride_b, T::BN, T::BK) &&
                         (int64_t(T::BM) * p.n + T::BN) * 4 < kMaxBufferOffset;
    if (buffers) return launch_tiles<T, A_K, B_K, true>(p, env, plan, stream);
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
using TileNarrow = Tile<256, 64, 32, 4, 1>;   // N <= 64 (attention head dim)

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

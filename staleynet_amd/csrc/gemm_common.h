// Pieces shared by the fp32 and bf16 matrix-core GEMMs: buffer addressing,
// kernel arguments, the LDS geometry, the operand loaders, the tile
// schedule, split-K planning and the reference's combine. See
// gemm_mfma.hip for the design these serve.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "gemm_internal.h"
#include "staleynet_gemm.h"

namespace sn {
namespace gemm {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

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

// Cache policy of a buffer store: 0, or kStreaming (the non-temporal bit,
// NT): data written once and not read back by the kernel that writes it. On
// the bf16 256 x 256 kernel, whose fp32 output tile (256 KB per CU) is
// written at the end of every few hundred matrix-core cycles per K-step,
// streaming stores took NN 32768 x 16384 x 768 from 1269-1337 us to 1111 us
// (the output no longer displaces the operand panels the tiles share in L2).
constexpr int32_t kStreaming = 2;

template <int32_t POLICY = 0>
__device__ __forceinline__ void buffer_store1(__amdgpu_buffer_rsrc_t rsrc, int32_t offset, float value) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, value), rsrc, offset, 0, POLICY);
}

// Device-coherent 128-bit accesses (cache policy SC1: the device-scope bit
// the gfx942/gfx950 memory model sets on agent-scope atomic loads and
// stores). They are read and written where every XCD sees them, so data
// handed between workgroups on different XCDs needs no L2 write-back or
// invalidate, only completion ordering.
constexpr int32_t kDeviceCoherent = 16;

__device__ __forceinline__ f32x4 buffer_load4_coherent(__amdgpu_buffer_rsrc_t rsrc, int32_t offset) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, kDeviceCoherent));
}

__device__ __forceinline__ void buffer_store4_coherent(__amdgpu_buffer_rsrc_t rsrc, int32_t offset, f32x4 value) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, value), rsrc, offset, 0, kDeviceCoherent);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats -> two bf16 in one 32-bit word (element 0 in the low half):
// gfx950's v_cvt_pk_bf16_f32, which rounds by the MODE register's f32
// rounding mode (round to nearest, ties to even, by default) and keeps NaN a
// quiet NaN. One instruction per pair instead of a shift/add/compare
// sequence per element.
__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// Four floats as four bf16 packed into 8 bytes, element 0 in the low half.
__device__ __forceinline__ u32x2 pack_bf16(f32x4 x) {
    u32x2 packed;
    packed[0] = pack2_bf16(x[0], x[1]);
    packed[1] = pack2_bf16(x[2], x[3]);
    return packed;
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
    const float* bias;  // null, or one value per column added after the combine
    float* column_sums; // null, or the right operand's column sums over K, accumulated (see Problem)
    int32_t streaming_output;  // nonzero: the output tiles go out with kStreaming stores
    int32_t persistent_items;  // persistent kernels: the work items the grid loops over
};

template <int BM_, int BN_, int BK_, int WAVES_M_, int WAVES_N_>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_;
    static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
    static constexpr int THREADS = 64 * WAVES_M * WAVES_N;
    static constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    static constexpr int FM = WTM / 32, FN = WTN / 32;
    static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile is whole 32x32 blocks");
    static_assert(BK == 32, "the loaders' lane mappings assume 8 k-groups of 4 per tile");
};

// fp32 LDS geometry of one operand tile: BK/4 planes (k-groups) of ROWS + 1
// 16-byte slots; slot (g, r) holds k = 4g .. 4g+3 of row r.
template <int ROWS, int BK>
struct Planes {
    static constexpr int PLANE = ROWS + 1;
    static constexpr int GROUPS = BK / 4;
    static constexpr int SLOTS = GROUPS * PLANE;
};

// bf16 LDS geometry: BK/8 planes (k-octets) of ROWS + PAD 16-byte slots;
// slot (o, r) holds k = 8o .. 8o+7 of row r as bf16. A loader writes each
// group of four k as one 8-byte half-slot. PAD is chosen per loader so that
// the 16 lanes of a b64 write phase hit 16 distinct 8-byte banks.
template <int ROWS, int BK, int PAD>
struct OctetPlanes {
    static constexpr int PLANE = ROWS + PAD;
    static constexpr int OCTETS = BK / 8;
    static constexpr int SLOTS = OCTETS * PLANE;
};

// Operand loaders. Each stages a ROWS x BK tile of one operand per K-step
// through registers into LDS. `init` runs once per tile, `load` issues the
// global reads for the K-step starting at k0 (reading 0 outside the matrix),
// `store` writes one fp32 LDS stage, `store_bf16` one bf16 stage.
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
    static constexpr int GROUPS = BK / 4;
    static constexpr int TOTAL = ROWS * GROUPS;
    static constexpr int PER_THREAD = (TOTAL + THREADS - 1) / THREADS;
    // bf16 half-slot banks: 16 lanes = 2 rows x 8 k-groups.
    static constexpr int BF16_PAD = 2;
    f32x4 reg[PER_THREAD];

    __device__ __forceinline__ void init(int64_t, int64_t, int64_t, int) {}

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int64_t row0, int64_t rows,
                                         int64_t k0, int64_t k_total, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int64_t gr = row0 + idx / GROUPS;
            const int64_t gk = k0 + (idx % GROUPS) * 4;
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
            const int64_t gr = row0 + idx / GROUPS;
            const int64_t gk = k0 + (idx % GROUPS) * 4;
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
                const int slot = (idx % GROUPS) * P::PLANE + idx / GROUPS;
                *reinterpret_cast<f32x4*>(lds + 4 * slot) = reg[v];
            }
        }
    }

    __device__ __forceinline__ void store_bf16(uint16_t* lds, int tid) const {
        using O = OctetPlanes<ROWS, BK, BF16_PAD>;
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            if (TOTAL % THREADS == 0 || idx < TOTAL) {
                const int g = idx % GROUPS;
                const int slot = (g / 2) * O::PLANE + idx / GROUPS;
                *reinterpret_cast<u32x2*>(lds + 8 * slot + 4 * (g % 2)) = pack_bf16(reg[v]);
            }
        }
    }
};

// 128-bit buffer loads; needs K % 4 == 0, ld % 4 == 0 and a 16-byte aligned
// base, so a vector is either wholly inside the matrix or wholly outside.
template <int ROWS, int BK, int THREADS>
struct KContiguousBufferLoader : KContiguousScalarLoader<ROWS, BK, THREADS> {
    using Base = KContiguousScalarLoader<ROWS, BK, THREADS>;
    using Base::GROUPS;
    using Base::PER_THREAD;
    using Base::TOTAL;
    using Base::reg;
    int32_t offset[PER_THREAD];  // bytes from the K-step's tile origin; kOutOfRange past the last row

    __device__ __forceinline__ void init(int64_t ld, int64_t row0, int64_t rows, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int r = idx / GROUPS;
            const bool valid = (TOTAL % THREADS == 0 || idx < TOTAL) && row0 + r < rows;
            offset[v] = valid ? int32_t((r * ld + (idx % GROUPS) * 4) * 4) : kOutOfRange;
        }
    }

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int64_t row0, int64_t,
                                         int64_t k0, int64_t k_total, int tid) {
        const __amdgpu_buffer_rsrc_t rsrc = buffer_of(base + row0 * ld + k0);
        const bool k_valid = k0 + (tid % GROUPS) * 4 < k_total;  // the same k-group for every v
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) reg[v] = buffer_load4(rsrc, k_valid ? offset[v] : kOutOfRange);
    }
};

template <int ROWS, int BK, int THREADS>
struct RowContiguousScalarLoader {
    using P = Planes<ROWS, BK>;
    static constexpr int GROUPS = BK / 4;
    static constexpr int TOTAL = GROUPS * (ROWS / 4);
    static constexpr int PER_THREAD = (TOTAL + THREADS - 1) / THREADS;
    // bf16 half-slot banks: 16 lanes = 8 k-groups x 2 row quads.
    static constexpr int BF16_PAD = 1;
    static_assert(ROWS % 4 == 0, "tile is whole 4-row groups");
    f32x4 reg[PER_THREAD][4];  // [v][kk]: rows 4q..4q+3 at k = 4g + kk

    __device__ __forceinline__ void init(int64_t, int64_t, int64_t, int) {}

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int64_t row0, int64_t rows,
                                         int64_t k0, int64_t k_total, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int64_t gr = row0 + (idx / GROUPS) * 4;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const int64_t gk = k0 + (idx % GROUPS) * 4 + kk;
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
            const int64_t gr = row0 + (idx / GROUPS) * 4;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const int64_t gk = k0 + (idx % GROUPS) * 4 + kk;
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
                const int first = (idx % GROUPS) * P::PLANE + (idx / GROUPS) * 4;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    f32x4 t = {reg[v][0][e], reg[v][1][e], reg[v][2][e], reg[v][3][e]};
                    *reinterpret_cast<f32x4*>(lds + 4 * (first + e)) = t;
                }
            }
        }
    }

    __device__ __forceinline__ void store_bf16(uint16_t* lds, int tid) const {
        using O = OctetPlanes<ROWS, BK, BF16_PAD>;
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            if (TOTAL % THREADS == 0 || idx < TOTAL) {
                const int g = idx % GROUPS;
                const int first = (g / 2) * O::PLANE + (idx / GROUPS) * 4;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    f32x4 t = {reg[v][0][e], reg[v][1][e], reg[v][2][e], reg[v][3][e]};
                    *reinterpret_cast<u32x2*>(lds + 8 * (first + e) + 4 * (g % 2)) = pack_bf16(t);
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
    using Base::GROUPS;
    using Base::PER_THREAD;
    using Base::TOTAL;
    using Base::reg;
    int32_t offset[PER_THREAD][4];  // bytes from the K-step's tile origin; kOutOfRange past the last row

    __device__ __forceinline__ void init(int64_t ld, int64_t row0, int64_t rows, int tid) {
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int r = (idx / GROUPS) * 4;
            const bool valid = (TOTAL % THREADS == 0 || idx < TOTAL) && row0 + r < rows;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                offset[v][kk] = valid ? int32_t((((idx % GROUPS) * 4 + kk) * ld + r) * 4) : kOutOfRange;
        }
    }

    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int64_t row0, int64_t,
                                         int64_t k0, int64_t k_total, int tid) {
        const __amdgpu_buffer_rsrc_t rsrc = buffer_of(base + k0 * ld + row0);
        const int64_t k_first = k0 + (tid % GROUPS) * 4;  // the same k-quad for every v
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

// Block id -> (matrix of the batch, K split, tile row, tile column). The
// grid enumerates (batch, split, tile) with the batch outermost. Consecutive
// workgroup ids land on different XCDs, so ids are first regrouped so that
// each XCD holds one contiguous range: whole matrices of a batch (attention
// heads: every XCD gets the same mix of causally full and empty tiles, and a
// head's operands stay in one L2), or whole K splits of one product (the
// tiles of a split share its slices of A and B). Within a split the tiles
// are walked as a raster grouped kGroupM tile rows high, keeping the A rows
// and B columns an XCD reuses in its own L2.
// Host-callable too: the host planner (sn_tile_map) evaluates the same map.
__host__ __device__ inline void tile_coordinates(int bid, int blocks, int tiles_m, int tiles_n, int splits, int& batch,
                                                 int& split, int& tm, int& tn) {
    const int xcd = bid % kXcds;
    const int local = bid / kXcds;
    const int q = blocks / kXcds;
    const int r = blocks % kXcds;
    const int linear = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + local;
    const int tiles = tiles_m * tiles_n;
    batch = linear / (tiles * splits);
    const int in_batch = linear % (tiles * splits);
    split = in_batch / tiles;
    const int id = in_batch % tiles;
    const int per_group = kGroupM * tiles_n;
    const int group = id / per_group;
    const int first_m = group * kGroupM;
    const int group_rows = tiles_m - first_m < kGroupM ? tiles_m - first_m : kGroupM;
    const int within = id % per_group;
    tm = first_m + within % group_rows;
    tn = within / group_rows;
}

// Matrices of a batch per launch: the grid's x dimension holds
// batches x splits x tiles workgroups and must stay below 2^32 work-items.
// 0 when one matrix alone exceeds that.
inline int64_t batches_per_launch(int64_t per_batch, int threads, int64_t batch) {
    const int64_t fit = ((int64_t(1) << 32) - 1) / threads / per_batch;
    return fit < batch ? fit : batch;
}

// The launch of a tiled product under `plan`: matrices per launch (0 when
// one matrix alone is too large), the grid and the split-K partials. The
// tiled launchers take their grid from here.
template <class T>
LaunchShape tiled_shape(const Problem& p, int tiles_m, int tiles_n, int splits, int64_t k_per_split, uint32_t path) {
    LaunchShape s;
    s.path = path;
    s.threads = T::THREADS;
    s.tile_m = T::BM;
    s.tile_n = T::BN;
    s.tiles_m = tiles_m;
    s.tiles_n = tiles_n;
    s.splits = splits;
    s.k_per_split = k_per_split;
    const int64_t per_batch = int64_t(tiles_m) * tiles_n * splits;
    s.batches_per_launch = batches_per_launch(per_batch, T::THREADS, p.batch);
    s.workgroups = s.batches_per_launch * per_batch;
    s.launches = s.batches_per_launch > 0 ? (p.batch + s.batches_per_launch - 1) / s.batches_per_launch : 0;
    s.workspace_bytes = splits > 1 ? size_t(splits) * size_t(p.m) * size_t(p.n) * sizeof(float) : 0;
    return s;
}

// The reference's combine (kernels/matmul.rs:166-168), the product and the
// sum rounded separately as the reference rounds them; then, when fused,
// Linear's bias (kernels/elementwise.rs:62-68) as one more rounded add.
__device__ __forceinline__ void write_output(float* dst, float sum, float scale, bool accumulate,
                                             const float* bias = nullptr, int64_t col = 0) {
#pragma clang fp contract(off)
    const float scaled = scale * sum;
    float value = accumulate ? *dst + scaled : scaled;
    if (bias != nullptr) value = value + bias[col];
    *dst = value;
}

// Where a wave's accumulators sit in its WTM x WTN sub-tile. Element r of
// 32x32 block (i, j) in lane l is MFMA row q = 8(r/4) + 4(l/32) + r%4 and
// MFMA column l%32. Normally block i covers rows 32i .. 32i + 31 (row 32i +
// q) and block j columns 32j + l%32. A paired side (two blocks whose
// fragments a lane reads as adjacent rows of a row-contiguous operand, one
// 8-byte LDS read per k) interleaves them instead: block i covers rows
// 2q + i, block j columns 2(l%32) + j.
// QUAD_N: four column blocks whose columns interleave in fours instead
// (block j covers columns 4(l%32) + j of the wave's 128), so a lane's four
// outputs of a row are adjacent (one 16-byte store); the operand side reads
// its rows permuted to match (the wide bf16 kernel's right-operand stages).
template <bool PAIR_M, bool PAIR_N, bool QUAD_N = false>
struct TileMap {
    // Row within the wave's sub-tile: a per-lane part (half = l/32) and a
    // part per (block, element) that does not depend on the lane.
    __device__ __forceinline__ static constexpr int row_lane(int half) { return PAIR_M ? 8 * half : 4 * half; }
    __device__ __forceinline__ static constexpr int row_elem(int i, int r) {
        return PAIR_M ? 2 * (8 * (r / 4) + (r % 4)) + i : 32 * i + 8 * (r / 4) + (r % 4);
    }
    __device__ __forceinline__ static constexpr int col_lane(int col_in_block) {
        return QUAD_N ? 4 * col_in_block : PAIR_N ? 2 * col_in_block : col_in_block;
    }
    __device__ __forceinline__ static constexpr int col_elem(int j) { return PAIR_N || QUAD_N ? j : 32 * j; }
};

// Writes a wave's accumulators (TileMap gives each element's place).
// `partial` writes raw sums to the split-K workspace; otherwise the
// reference's combine, with causal-masked outputs written 0 (overwrite) or
// left alone (accumulate). POLICY: the buffer stores' cache policy.
// INTERIOR_ONLY: the caller guarantees an interior tile that reads nothing
// back (partial, or overwrite), so only that path is compiled. QUAD_N: see
// TileMap.
template <class T, bool BUF, bool PAIR_M = false, bool PAIR_N = false, int32_t POLICY = 0,
          bool INTERIOR_ONLY = false, bool QUAD_N = false>
__device__ __forceinline__ void write_tile(const Args& args, const f32x16 (&acc)[T::FM][T::FN], float* out,
                                           int64_t m0, int64_t n0, int wave_m, int wave_n, int lane, bool partial) {
    using Map = TileMap<PAIR_M, PAIR_N, QUAD_N>;
    static_assert(!PAIR_M || T::FM == 2, "pairs of row blocks");
    static_assert(!PAIR_N || T::FN == 2, "pairs of column blocks");
    static_assert(!QUAD_N || (T::FN == 4 && T::WTN == 128 && !PAIR_N), "fours of column blocks");
    const int col_in_block = lane & 31;
    const int half = lane >> 5;
    const bool accumulate = args.accumulate != 0;
    const bool output_causal = args.mask == int(SN_MASK_CAUSAL_OUTPUT);
    // The lane's first row and column within the tile.
    const int lane_row = wave_m * T::WTM + Map::row_lane(half);
    const int lane_col = wave_n * T::WTN + Map::col_lane(col_in_block);
    if constexpr (BUF) {
        // Offsets from the tile origin; kOutOfRange drops stores outside the matrix.
        const __amdgpu_buffer_rsrc_t rsrc = buffer_of(out + m0 * args.n + n0);
        // Interior tiles with nothing masked and nothing to read back (the
        // common case; uniform): one vector offset per lane and column block,
        // each element's row in a scalar offset, no per-element selects or
        // branches. The general path below costs ~20 instructions per element,
        // which at K = 64 outweighed the tile's MFMAs.
        const bool interior = INTERIOR_ONLY || (m0 + T::BM <= args.m && n0 + T::BN <= args.n);
        if (INTERIOR_ONLY || (interior && (partial || !accumulate))) {
            // Split-K partials are raw sums: scale 1, which is exact. Tiles
            // that cross the causal diagonal write 0 where masked (a compare
            // and a select per element, still no branch).
            const float scale = partial ? 1.f : args.scale;
            const bool any_masked = !partial && output_causal && n0 + T::BN - 1 > m0 + args.query_offset;
            // Fused bias (never with a mask): one value per lane and column block.
            const bool add_bias = !partial && args.bias != nullptr;
            float bias_value[T::FN];
#pragma unroll
            for (int j = 0; j < T::FN; ++j) bias_value[j] = add_bias ? args.bias[n0 + lane_col + Map::col_elem(j)] : 0.f;
            // col - row - offset of the lane's element at block (0, 0), r = 0.
            // (Clamped to 32 bits: beyond +-2^30 every element is on the same side.)
            const int64_t diagonal64 = n0 + lane_col - (m0 + lane_row) - args.query_offset;
            const int diagonal = int(max(min(diagonal64, int64_t(1) << 30), -(int64_t(1) << 30)));
            auto value_of = [&](int i, int j, int r) __attribute__((always_inline)) {
                float value = scale * acc[i][j][r];
                if (any_masked) value = diagonal + Map::col_elem(j) - Map::row_elem(i, r) > 0 ? 0.f : value;
                if (add_bias) value = value + bias_value[j];
                return value;
            };
            if constexpr (QUAD_N) {
                // The lane's four columns are adjacent: one 16-byte store per
                // row. The row goes into the vector offset, with a constant
                // scalar offset: with the row in an SGPR offset, a store's
                // data registers were rewritten by the next VALU instruction
                // before the store read them (the next row's values came out
                // in some lanes), a wait the compiler keeps only for stores
                // without a register scalar offset.
                typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
                const int32_t column_offset = int32_t((lane_row * args.n + lane_col) * 4);
#pragma unroll
                for (int i = 0; i < T::FM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int32_t row_offset = int32_t(Map::row_elem(i, r) * args.n * 4);
                        const u32x4_t quad = {__builtin_bit_cast(uint32_t, value_of(i, 0, r)),
                                              __builtin_bit_cast(uint32_t, value_of(i, 1, r)),
                                              __builtin_bit_cast(uint32_t, value_of(i, 2, r)),
                                              __builtin_bit_cast(uint32_t, value_of(i, 3, r))};
                        __builtin_amdgcn_raw_buffer_store_b128(quad, rsrc, column_offset + row_offset, 0, POLICY);
                    }
            } else if constexpr (PAIR_N) {
                // The lane's two columns are adjacent: one 8-byte store per element pair.
                typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
                const int32_t column_offset = int32_t((lane_row * args.n + lane_col) * 4);
#pragma unroll
                for (int i = 0; i < T::FM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int32_t row_offset = int32_t(Map::row_elem(i, r) * args.n * 4);
                        const u32x2_t pair = {__builtin_bit_cast(uint32_t, value_of(i, 0, r)),
                                              __builtin_bit_cast(uint32_t, value_of(i, 1, r))};
                        __builtin_amdgcn_raw_buffer_store_b64(pair, rsrc, column_offset, row_offset, POLICY);
                    }
            } else {
#pragma unroll
                for (int j = 0; j < T::FN; ++j) {
                    const int32_t column_offset = int32_t((lane_row * args.n + lane_col + Map::col_elem(j)) * 4);
#pragma unroll
                    for (int i = 0; i < T::FM; ++i)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int32_t row_offset = int32_t(Map::row_elem(i, r) * args.n * 4);
                            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, value_of(i, j, r)), rsrc,
                                                                  column_offset, row_offset, POLICY);
                        }
                }
            }
            return;
        }
        if constexpr (INTERIOR_ONLY) return;
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
#pragma unroll
            for (int j = 0; j < T::FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = lane_row + Map::row_elem(i, r);
                    const int col = lane_col + Map::col_elem(j);
                    const bool inside = m0 + row < args.m && n0 + col < args.n;
                    const int32_t offset = inside ? int32_t((row * args.n + col) * 4) : kOutOfRange;
                    const float sum = acc[i][j][r];
                    if (partial) {
                        buffer_store1<POLICY>(rsrc, offset, sum);
                    } else if (output_causal && n0 + col > m0 + row + args.query_offset) {
                        if (!accumulate) buffer_store1<POLICY>(rsrc, offset, 0.f);
                    } else {
#pragma clang fp contract(off)
                        const float scaled = args.scale * sum;
                        float value = accumulate ? buffer_load1(rsrc, offset) + scaled : scaled;
                        if (args.bias != nullptr && inside) value = value + args.bias[n0 + col];
                        buffer_store1<POLICY>(rsrc, offset, value);
                    }
                }
    } else {
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
#pragma unroll
            for (int j = 0; j < T::FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t row = m0 + lane_row + Map::row_elem(i, r);
                    const int64_t col = n0 + lane_col + Map::col_elem(j);
                    if (row < args.m && col < args.n) {
                        float* dst = out + row * args.n + col;
                        if (partial) {
                            *dst = acc[i][j][r];
                        } else if (output_causal && col > row + args.query_offset) {
                            if (!accumulate) *dst = 0.f;
                        } else {
                            write_output(dst, acc[i][j][r], args.scale, accumulate, args.bias, col);
                        }
                    }
                }
    }
}

// Writes zeros over a tile whose outputs are all causally masked: 16-byte
// stores (one vector offset per lane, rows in scalar offsets) for an interior
// tile of a 16-byte-aligned output, element stores otherwise.
template <class T>
__device__ __forceinline__ void zero_tile(const Args& args, float* c_batch, int64_t m0, int64_t n0, int tid) {
    const bool interior = m0 + T::BM <= args.m && n0 + T::BN <= args.n;
    const bool vectors = (args.n & 3) == 0 && (reinterpret_cast<uintptr_t>(c_batch) & 15) == 0;
    if (interior && vectors) {
        constexpr int kPerRow = T::BN / 4;                // 16-byte groups per tile row
        constexpr int kRowsPerRound = T::THREADS / kPerRow;
        const __amdgpu_buffer_rsrc_t rsrc = buffer_of(c_batch + m0 * args.n + n0);
        const int32_t lane_offset = int32_t(((tid / kPerRow) * args.n + 4 * (tid % kPerRow)) * 4);
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        // A product whose output streams out writes its zero tiles the same way.
        if (args.streaming_output) {
#pragma unroll
            for (int q = 0; q < T::BM / kRowsPerRound; ++q)
                __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, rsrc,
                                                       lane_offset + int32_t(q * kRowsPerRound * args.n * 4), 0,
                                                       kStreaming);
        } else {
#pragma unroll
            for (int q = 0; q < T::BM / kRowsPerRound; ++q)
                __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, rsrc, lane_offset,
                                                       int32_t(q * kRowsPerRound * args.n * 4), 0);
        }
        return;
    }
    for (int e = tid; e < T::BM * T::BN; e += T::THREADS) {
        const int64_t r = m0 + e / T::BN;
        const int64_t col = n0 + e % T::BN;
        if (r < args.m && col < args.n) c_batch[r * args.n + col] = 0.f;
    }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Buffer loads take 128 bits at a time, so the contiguous dimension, the
// leading dimension and the batch stride must be multiples of 4 floats and
// the base 16-byte aligned; per-lane offsets within one K-step tile must
// also fit the 31-bit range.
inline bool buffer_ok(const float* base, bool k_contiguous, int64_t rows, int64_t k, int64_t ld, int64_t stride,
                      int tile_rows, int bk) {
    const int64_t contiguous = k_contiguous ? k : rows;
    const int64_t span = k_contiguous ? (int64_t(tile_rows) * ld + bk) * 4 : (int64_t(bk) * ld + tile_rows) * 4;
    return aligned16(base) && contiguous % 4 == 0 && ld % 4 == 0 && stride % 4 == 0 && span < kMaxBufferOffset;
}

template <class T>
bool buffers_ok(const Problem& p) {
    return buffer_ok(p.a, p.a_k_contiguous, p.m, p.k, p.lda, p.stride_a, T::BM, T::BK) &&
           buffer_ok(p.b, p.b_k_contiguous, p.n, p.k, p.ldb, p.stride_b, T::BN, T::BK) &&
           (int64_t(T::BM) * p.n + T::BN) * 4 < kMaxBufferOffset;
}

struct Plan {
    int tiles_m, tiles_n;
    int splits;
    int64_t k_per_split;
};

// How a kernel instantiation occupies the device, for the split-K choice:
// workgroups resident per CU (LDS-limited), the FLOP rate one CU sustains
// on it, and the k values one K-step index counts (2 when the operands are
// bf16 pairs).
struct SplitCost {
    int workgroups_per_cu = 2;
    double flops_per_cu = 522e9;  // fp32 matrix cores at about 85 % of 157.3 TFLOP/s / 256 CUs
    int k_per_index = 1;
};

// Products whose output tiles cannot fill every CU four times over (the
// K = 32768 weight gradients: 36 to 768 tiles of 128x128) split K into
// BK-aligned slices of at least 8 steps, as far as the workspace allows. The
// count is the cheapest under a model of the launch, measured on the 111.5M model's
// weight gradients:
//  * workgroups are dealt evenly over the CUs; the busiest CU runs
//    ceil(tiles x slices / CUs) of them, workgroups_per_cu at a time, and
//    a last, partly filled group runs faster than a full one (about 0.7 of
//    its time when it is one of two);
//  * a workgroup costs its K-steps plus about 3 steps of start-up and
//    epilogue;
//  * the partial sums cost 8 bytes per slice and output (written, then
//    read by the reduce) at about 6 TB/s.
// Counts just past a whole number of groups leave a few workgroups running
// alone at the end; the former rule (about eight workgroups per CU) hit
// that on four of the five c2 weight gradients.
template <class T>
Plan plan_for(const Problem& p, const Env& env, const SplitCost& cost = SplitCost{}) {
    Plan plan;
    plan.tiles_m = int((p.m + T::BM - 1) / T::BM);
    plan.tiles_n = int((p.n + T::BN - 1) / T::BN);
    plan.splits = 1;
    plan.k_per_split = std::max<int64_t>(p.k, 1);
    const int64_t tiles = int64_t(plan.tiles_m) * plan.tiles_n * p.batch;
    const int64_t cus = std::max(env.cu_count, 1);
    const int64_t threshold = cus * 4;
    const int64_t k_steps = (p.k + T::BK - 1) / T::BK;
    if (p.mask != SN_MASK_NONE || tiles >= threshold || k_steps < 16 || p.batch != 1) return plan;
    int64_t max_splits = k_steps / 8;
    const int64_t per_split_bytes = p.m * p.n * int64_t(sizeof(float));
    if (per_split_bytes > 0) max_splits = std::min<int64_t>(max_splits, int64_t(env.workspace_bytes) / per_split_bytes);
    if (max_splits < 2) return plan;
    // One K-step of a full group of workgroups, and the partial-sum bytes
    // the reduce moves in that time.
    const int group = std::max(cost.workgroups_per_cu, 1);
    const double step_seconds = 2.0 * T::BM * T::BN * T::BK * cost.k_per_index * group / cost.flops_per_cu;
    const double reduce_bytes_per_step = 6e12 * step_seconds;
    auto time_of = [&](int64_t steps_per_split, int64_t splits) {
        const int64_t per_cu = (tiles * splits + cus - 1) / cus;
        const int64_t full = per_cu / group, rest = per_cu % group;
        const double groups = double(full) + (rest ? 1.0 - 0.3 * double(group - rest) / double(group - 1 > 0 ? group - 1 : 1) : 0.0);
        const double reduce = splits > 1 ? double(splits) * double(per_split_bytes) * 2.0 / reduce_bytes_per_step : 0.0;
        return groups * double(steps_per_split + 3) + reduce;
    };
    double best = time_of(k_steps, 1);
    for (int64_t want = 2; want <= max_splits; ++want) {
        const int64_t steps_per_split = (k_steps + want - 1) / want;
        const int64_t splits = (k_steps + steps_per_split - 1) / steps_per_split;
        const double t = time_of(steps_per_split, splits);
        if (t < best) {
            best = t;
            plan.k_per_split = steps_per_split * T::BK;
            plan.splits = int(splits);
        }
    }
    if (plan.splits > 1) plan.splits = int((p.k + plan.k_per_split - 1) / plan.k_per_split);
    return plan;
}

template <class T>
LaunchShape tiled_shape(const Problem& p, const Plan& plan, uint32_t path) {
    return tiled_shape<T>(p, plan.tiles_m, plan.tiles_n, plan.splits, plan.k_per_split, path);
}

template <class T>
Args make_args(const Problem& p, const Env& env, const Plan& plan) {
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
    args.batch_base = 0;
    args.query_offset = p.query_offset;
    args.tiles_m = plan.tiles_m;
    args.tiles_n = plan.tiles_n;
    args.splits = plan.splits;
    args.accumulate = p.accumulate ? 1 : 0;
    args.mask = int(p.mask);
    args.scale = p.scale;
    args.bias = p.bias;
    args.column_sums = p.column_sums;
    args.streaming_output = 0;
    args.persistent_items = 0;
    return args;
}

// The direct-to-LDS fp32 kernel (gemm_dma.hip): whether it serves `p`
// (aligned operands), its launch shape and its launcher.
bool dma_applies(const Problem& p, const Env& env);
LaunchShape describe_f32_dma(const Problem& p, const Env& env);
hipError_t launch_gemm_f32_dma(const Problem& p, const Env& env, hipStream_t stream);
// The bf16 variant of the direct-to-LDS kernel: whether it serves `p`, its
// launch shape (with the split-K workspace it uses) and its launcher.
bool bf16_dma_applies(const Problem& p, const Env& env);
LaunchShape describe_bf16_dma(const Problem& p, const Env& env);
hipError_t launch_gemm_bf16_dma(const Problem& p, const Env& env, hipStream_t stream);
// The 256 x 256 bf16 kernel that rounds fp32 operands as it loads them
// (gemm_bf16_wide.hip): whether it serves `p` (unmasked, aligned, large
// enough; partial sums fit), its launch shape and launcher.
bool bf16_wide_applies(const Problem& p, const Env& env);
LaunchShape describe_bf16_wide(const Problem& p, const Env& env);
hipError_t launch_gemm_bf16_wide(const Problem& p, const Env& env, hipStream_t stream);
// The fp32 direct-to-LDS product that also adds the right operand's column
// sums into p.column_sums (gemm_dma.hip): whether it serves `p` (batch 1,
// unmasked, no bias, right operand row-contiguous, aligned), its launch shape
// (workspace: the product's partial sums and N per K slice) and launcher.
bool f32_column_sums_applies(const Problem& p, const Env& env);
LaunchShape describe_f32_column_sums(const Problem& p, const Env& env);
hipError_t launch_gemm_f32_column_sums(const Problem& p, const Env& env, hipStream_t stream);
// The bf16 wide product that also adds the right operand's column sums into
// p.column_sums (gemm_bf16_wide.hip): whether it serves `p` (batch 1, no
// bias, right operand row-contiguous fp32 and not the one staged), its
// launch shape and launcher.
bool bf16_wide_column_sums_applies(const Problem& p, const Env& env);
LaunchShape describe_bf16_wide_column_sums(const Problem& p, const Env& env);
hipError_t launch_gemm_bf16_wide_column_sums(const Problem& p, const Env& env, hipStream_t stream);
// bf16 with both operands first staged as bf16 in the workspace (gemm_dma.hip):
// whether it serves `p` (unmasked, aligned, staged operands fit), its
// launch shape (workspace: staged operands and partial sums) and launcher.
bool bf16_staged_applies(const Problem& p, const Env& env);
LaunchShape describe_bf16_staged(const Problem& p, const Env& env);
hipError_t launch_gemm_bf16_staged(const Problem& p, const Env& env, hipStream_t stream);

// Adds the split-K partial sums in split order and applies the combine
// (defined in gemm_mfma.hip).
hipError_t launch_splitk_reduce(const Problem& p, const Env& env, int splits, hipStream_t stream);

}  // namespace gemm
}  // namespace sn

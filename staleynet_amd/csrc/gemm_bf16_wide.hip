// bf16-input GEMM that rounds fp32 operands as it loads them: the role of the
// reference's TF32 tensor-core kernel (crates/staleynet-cuda/src/kernels/
// matmul.rs:357-448) for large aligned products.
//
// The operands stay fp32 in HBM, so per FLOP this kernel reads twice the bytes
// a kernel on bf16 copies would; it makes up for it with the largest tile the
// registers allow and a deep prefetch, instead of paying a separate pass that
// reads every operand, writes a bf16 copy and reads that copy back. When one
// operand is much smaller than the other (the weight, in the Linear forward
// and input-gradient products), that one alone is rounded into the workspace
// first (launch_stage_bf16: cheap, and then read at 2 bytes an element by
// every tile row), and only the other is rounded as it loads.
//  * 256 x 256 output tile, eight waves (two per SIMD) of 64 x 128;
//  * 32 k per step (the fp32 loaders' geometry, gemm_common.h), two steps of
//    global loads in flight in two register sets (128 KB per CU with both
//    operands fp32, 96 KB with one staged), so the loads of a step have two
//    steps' MFMAs to arrive;
//  * each step rounds the next step's registers to bf16 (nearest-even,
//    v_cvt_pk_bf16_f32) into the other of two bf16 LDS stages, between its
//    two 16-deep MFMA chunks, and issues the loads of the step after next;
//  * one barrier per step, waiting on LDS only (the loads in flight are
//    waited for by count, never drained).
// The LDS stage layout, fp32 loaders and epilogue are those of the
// register-staged bf16 kernel (gemm_bf16.hip), with the LDS writes addressed
// from one base per lane; v_mfma_f32_32x32x16_bf16 takes eight consecutive k
// per lane, one ds_read_b128 per 32-row fragment.
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

// The right operand's stage rows in QUAD order (write_tile's QUAD_N map):
// LDS position p of each 128-row group (a wave's columns) holds the logical
// row quad_row(p), so that block j's fragment rows, positions 32 j + (0..31),
// are the rows 4 (0..31) + j whose outputs the epilogue stores side by side.
// The fragment reads are unchanged; the loaders place each row at
// quad_position of it (the inverse).
// (quad_row and quad_position: gemm_internal.h.)
static_assert(quad_position(quad_row(37)) == 37 && quad_row(quad_position(201)) == 201, "inverse maps");

// The fp32 loaders (gemm_common.h) with the bf16 LDS write addressed from one
// per-lane base: vector v of a K-contiguous loader is row tid / 8 + v x
// (THREADS / 8), 16 x THREADS / 8 bytes further into the octet plane; block
// v of a row-contiguous loader is rows 4 (tid / 8 + v x THREADS / 8) .. + 3.
// QUAD: the rows in quad order (a K-contiguous loader loads, for the same
// LDS slots, the rows quad_row of them; a row-contiguous one writes each of
// its four rows at quad_position of it).
template <int ROWS, int BK, int THREADS, bool QUAD = false>
struct WideKLoader : KContiguousBufferLoader<ROWS, BK, THREADS> {
    using Base = KContiguousBufferLoader<ROWS, BK, THREADS>;
    using Base::reg;
    // LDS slot of stage row r (the rows as they are).
    __device__ __forceinline__ static constexpr int row_slot(int r) { return r; }
    static_assert(Base::TOTAL % THREADS == 0 && THREADS % Base::GROUPS == 0, "whole vectors per thread");
    static_assert(!QUAD || ROWS % 128 == 0, "whole 128-row groups");
    __device__ __forceinline__ void init(int64_t ld, int64_t row0, int64_t rows, int tid) {
        if constexpr (!QUAD) {
            Base::init(ld, row0, rows, tid);
        } else {
#pragma unroll
            for (int v = 0; v < Base::PER_THREAD; ++v) {
                const int idx = tid + v * THREADS;
                const int r = quad_row(idx / Base::GROUPS);
                Base::offset[v] = row0 + r < rows ? int32_t((r * ld + (idx % Base::GROUPS) * 4) * 4) : kOutOfRange;
            }
        }
    }
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

template <int ROWS, int BK, int THREADS, bool QUAD = false, bool RUNS = true>
struct WideRowLoader : RowContiguousBufferLoader<ROWS, BK, THREADS> {
    using Base = RowContiguousBufferLoader<ROWS, BK, THREADS>;
    using Base::reg;
    static constexpr int GROUPS = Base::GROUPS;  // k-groups of 4 per step
    static_assert(GROUPS == 8 && ROWS % 64 == 0 && THREADS % (16 * GROUPS) == 0 && Base::TOTAL % THREADS == 0,
                  "whole 16-quad runs per k-group");
    // RUNS: lanes 16 j .. 16 j + 15 of a thread block take one k-group and
    // 16 consecutive row quads (256 contiguous bytes of each of that group's
    // four k-rows), so a wave instruction reads 4 k-rows x 256 bytes, where
    // 8 k-groups x 8 quads (thread i: k-group i % 8, quad i / 8; kept for the
    // column sums, whose 8 threads of a quad must be lanes of one wave) read
    // 8 rows' 128-byte pieces: the loads' cost follows the pieces more than
    // the bytes. RUNS thread index i: k-group (i / 16) % 8, quad 16 (i / 128)
    // + i % 16.
    __device__ __forceinline__ static constexpr int group_of(int i) { return RUNS ? (i / 16) % GROUPS : i % GROUPS; }
    __device__ __forceinline__ static constexpr int quad_index(int i) {
        return RUNS ? 16 * (i / (16 * GROUPS)) + i % 16 : i / GROUPS;
    }
    // Blocks v of a thread are THREADS / (16 GROUPS) x 16 quads apart: whole
    // 128-row groups, so block v's quad positions are block 0's plus a
    // constant (immediate offsets from one base), and its k-group is block 0's.
    static constexpr int QUADS_PER_BLOCK = THREADS / GROUPS;
    static_assert(!QUAD || ((4 * QUADS_PER_BLOCK) % 128 == 0 && ROWS % 128 == 0), "whole 128-row groups");
    // The row quad (rows 4 c .. 4 c + 3) a thread's block 0 holds, as placed
    // in LDS. In quad order the four rows of quad c land at positions 32 e +
    // c; quad index bits 0 and 2 are swapped, as the unswapped order's
    // 16-lane write phases conflicted when a phase held 8 k-groups x 2 quads
    // (the lanes of a wave still read the same row pieces).
    __device__ __forceinline__ static constexpr int quad_of(int q) {
        return QUAD ? (q & ~5) | ((q & 1) << 2) | ((q >> 2) & 1) : q;
    }
    // Rows as they are (QUAD off), the RUNS mapping puts a write phase's 16
    // lanes on rows 4 c + e of 16 consecutive quads, all on the same half of
    // their slots: slots 4 apart, 8 lanes to a bank. Row r then goes to slot
    // r ^ ((r / 8) % 4), which spreads those 16 rows over 8 bank pairs
    // (2-way, as in quad order) and keeps 8 consecutive rows, what a 16-byte
    // fragment read phase takes, on 8 distinct slots modulo 8 (no conflict).
    static constexpr bool ROW_SWIZZLE = !QUAD && RUNS;
    __device__ __forceinline__ static constexpr int row_slot(int r) { return ROW_SWIZZLE ? r ^ ((r >> 3) & 3) : r; }
    __device__ __forceinline__ void init(int64_t ld, int64_t row0, int64_t rows, int tid) {
#pragma unroll
        for (int v = 0; v < Base::PER_THREAD; ++v) {
            const int idx = tid + v * THREADS;
            const int r = 4 * quad_of(quad_index(idx));
            const bool valid = row0 + r < rows;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                Base::offset[v][kk] = valid ? int32_t(((group_of(idx) * 4 + kk) * ld + r) * 4) : kOutOfRange;
        }
    }
    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int64_t row0, int64_t,
                                         int64_t k0, int64_t k_total, int tid) {
        const __amdgpu_buffer_rsrc_t rsrc = buffer_of(base + k0 * ld + row0);
        const int64_t k_first = k0 + group_of(tid) * 4;  // the same k-group for every v
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const bool k_valid = k_first + kk < k_total;
#pragma unroll
            for (int v = 0; v < Base::PER_THREAD; ++v)
                reg[v][kk] = buffer_load4(rsrc, k_valid ? Base::offset[v][kk] : kOutOfRange);
        }
    }
    __device__ __forceinline__ void store_bf16(uint16_t* lds, int tid) const {
        using O = OctetPlanes<ROWS, BK, Base::BF16_PAD>;
        const int g = group_of(tid);
        const int c = quad_of(quad_index(tid));  // this thread's rows 4 c .. 4 c + 3 of block 0
        int base = ((g / 2) * O::PLANE + (QUAD ? quad_position(4 * c) : 4 * c)) * 16 + 8 * (g % 2);
        launder(base);
        char* p = reinterpret_cast<char*>(lds) + base;
        // ROW_SWIZZLE: row 4 c + e sits at slot 4 c + (e ^ x), x = (c / 2) % 4
        // (blocks v are whole 128-row groups apart, which the swizzle keeps).
        int x = ROW_SWIZZLE ? (c >> 1) & 3 : 0;
        launder(x);
#pragma unroll
        for (int v = 0; v < Base::PER_THREAD; ++v)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f32x4 t = {reg[v][0][e], reg[v][1][e], reg[v][2][e], reg[v][3][e]};
                // quad_position(4 c + e) = quad_position(4 c) + 32 e for e < 4.
                const int row = 4 * v * QUADS_PER_BLOCK + (QUAD ? 32 * e : ROW_SWIZZLE ? (e ^ x) : e);
                *reinterpret_cast<u32x2*>(p + row * 16) = pack_bf16(t);
            }
    }
};

static_assert(WideRowLoader<256, 32, 512, true>::quad_of(5) == 5 && WideRowLoader<256, 32, 512, true>::quad_of(1) == 4 &&
                  WideRowLoader<256, 32, 512, true>::quad_of(68) == 65,
              "quad index bits 0 and 2 swapped");

template <bool K_CONTIGUOUS, int ROWS, int BK, int THREADS, bool QUAD = false, bool RUNS = true>
using WideLoaderFor = typename std::conditional<K_CONTIGUOUS, WideKLoader<ROWS, BK, THREADS, QUAD>,
                                                WideRowLoader<ROWS, BK, THREADS, QUAD, RUNS>>::type;

// An operand already rounded to bf16 in the workspace, in the blocked layout
// of launch_stage_bf16_blocks: per 32-deep step, `ld` (rows_pad) rows of 32 k
// (64 bytes), in quad order when QUAD, zeros past the rows and K. Vector v of
// a thread is one 16-byte octet (8 consecutive k) of slot row tid / 4 + v x
// THREADS / 4, so a step's 256 rows of the tile are one contiguous 16 KB run
// (1 KB per wave instruction, where the row-by-row layout took 16 separate
// 64-byte pieces), and each lane writes its octet's LDS slot as it came.
// `base` points at the operand (batch offsets in floats).
template <int ROWS, int BK, int THREADS, bool QUAD = false>
struct StagedLoader {
    static constexpr int OCTETS = BK / 8;
    static constexpr int PER_THREAD = ROWS * OCTETS / THREADS;
    // A b128 write phase is 8 lanes (128 bytes over 32 banks): two rows x
    // four octets. A plane of 258 slots puts the octets 8 banks apart and the
    // rows 4: conflict-free. (Planes 4 slots longer put octets 0 and 2 on the
    // same banks; the counters showed it.)
    static constexpr int BF16_PAD = 2;
    static_assert(ROWS * OCTETS % THREADS == 0 && THREADS % OCTETS == 0, "whole slots per thread");
    static_assert(BK == 32 && ROWS % 128 == 0, "the blocked layout's 32-deep steps and whole quad groups");
    f32x4 reg[PER_THREAD];  // 8 bf16 each, as loaded
    __device__ __forceinline__ static constexpr int row_slot(int r) { return r; }

    // The layout is padded to whole tiles and already in quad order: every
    // offset is the same for every tile and step.
    __device__ __forceinline__ void init(int64_t, int64_t, int64_t, int) {}

    // A step past the slice's end reads zeros (out-of-range offsets), keeping
    // the counts the waits assume; a step inside it is whole (K is padded to
    // 32 with zeros and slices are whole steps).
    __device__ __forceinline__ void load(const float* __restrict__ base, int64_t ld, int64_t row0, int64_t,
                                         int64_t k0, int64_t k_end, int tid) {
        const uint16_t* tile = reinterpret_cast<const uint16_t*>(base) + (k0 / BK) * (ld * BK) + row0 * BK;
        const __amdgpu_buffer_rsrc_t rsrc = buffer_of(reinterpret_cast<const float*>(tile));
        const bool k_valid = k0 < k_end;
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v)
            reg[v] = buffer_load4(rsrc, k_valid ? int32_t((v * THREADS + tid) * 16) : kOutOfRange);
    }

    __device__ __forceinline__ void store_bf16(uint16_t* lds, int tid) const {
        using O = OctetPlanes<ROWS, BK, BF16_PAD>;
        int base = ((tid % OCTETS) * O::PLANE + tid / OCTETS) * 16;
        launder(base);
        char* p = reinterpret_cast<char*>(lds) + base;
#pragma unroll
        for (int v = 0; v < PER_THREAD; ++v) *reinterpret_cast<f32x4*>(p + v * (THREADS / OCTETS) * 16) = reg[v];
    }
};

// Which operand the workspace holds as bf16: none, the left or the right.
enum StagedSide { kStageNone = 0, kStageLeft = 1, kStageRight = 2 };

template <bool K_CONTIGUOUS, bool STAGED, int ROWS, int BK, int THREADS, bool QUAD = false, bool RUNS = true>
using OperandLoader = typename std::conditional<STAGED, StagedLoader<ROWS, BK, THREADS, QUAD>,
                                                WideLoaderFor<K_CONTIGUOUS, ROWS, BK, THREADS, QUAD, RUNS>>::type;

// Vector-memory instructions one loader issues per step.
template <class L>
constexpr int loads_per_step() {
    return sizeof(L::reg) / sizeof(f32x4);
}

// COLSUM: the first tile row also adds the right operand's column sums over
// K (row-contiguous fp32, not staged), from the fp32 values as loaded.
template <bool A_K, bool B_K, int SIDE, bool COLSUM = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_bf16_wide_kernel(Args args) {
    using T = WideTile;
    using LA = OperandLoader<A_K, SIDE == kStageLeft, T::BM, T::BK, T::THREADS>;
    using LB = OperandLoader<B_K, SIDE == kStageRight, T::BN, T::BK, T::THREADS, true, !COLSUM>;
    using OA = OctetPlanes<T::BM, T::BK, LA::BF16_PAD>;
    using OB = OctetPlanes<T::BN, T::BK, LB::BF16_PAD>;
    constexpr int kSetLoads = loads_per_step<LA>() + loads_per_step<LB>();
    if constexpr (COLSUM)
        static_assert(!B_K && SIDE != kStageRight && LB::PER_THREAD == 1 && LB::GROUPS == 8,
                      "column sums of a row-contiguous fp32 right operand, one 4-column block per thread");
    __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][8 * OA::SLOTS];
    __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][8 * OB::SLOTS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave / T::WAVES_N;
    const int wave_n = wave % T::WAVES_N;
    const int row = lane & 31;
    const int half = lane >> 5;
    const int a_row = LA::row_slot(row);  // where the A operand's loader put this lane's row

    int batch_local, split, tm, tn;
    tile_coordinates(blockIdx.x, gridDim.x, args.tiles_m, args.tiles_n, args.splits, batch_local, split, tm, tn);
    const int64_t batch = args.batch_base + batch_local;
    const int64_t m0 = int64_t(tm) * T::BM;
    const int64_t n0 = int64_t(tn) * T::BN;
    const int64_t k_begin = int64_t(split) * args.k_per_split;
    const int64_t k_end = min(args.k, k_begin + args.k_per_split);
    const float* a = args.a + batch * args.stride_a;
    const float* b = args.b + batch * args.stride_b;

    // NSETS register sets per operand: set j holds the steps s with s % NSETS
    // == j, loaded NSETS - 1 steps ahead of their hand-off to LDS. (A third
    // set, which fits when one operand is staged, measured no faster.)
    constexpr int NSETS = 2;
    LA la[NSETS];
    LB lb[NSETS];
#pragma unroll
    for (int j = 0; j < NSETS; ++j) {
        la[j].init(args.lda, m0, args.m, tid);
        lb[j].init(args.ldb, n0, args.n, tid);
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
    // Column sums (COLSUM, first tile row): thread t holds columns 4 q .. +3
    // (q = LB::quad_of(t / 8)) at k = 4 (t % 8) .. + 3 of every step, added here in k order as
    // each step is staged; the 8 threads of a column block are added at the
    // end in a fixed butterfly order.
    const bool colsum_tile = COLSUM && tm == 0;  // uniform over the workgroup
    float colsum[4] = {0.f, 0.f, 0.f, 0.f};
    // Rounds register set S into LDS stage L.
    auto stage = [&](auto set, auto lds) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        constexpr int L = decltype(lds)::value;
        if constexpr (COLSUM) {
            if (colsum_tile) {
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                    for (int e = 0; e < 4; ++e) colsum[e] = colsum[e] + lb[S].reg[0][kk][e];
            }
        }
        la[S].store_bf16(lds_a[L], tid);
        lb[S].store_bf16(lds_b[L], tid);
    };
    // Fragments of one 16-deep chunk of LDS stage S, and its MFMAs.
    auto read_chunk = [&](auto set, int c, bf16x8 (&fa)[T::FM], bf16x8 (&fb)[T::FN]) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        const int octet = 2 * c + half;
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
            fa[i] = *reinterpret_cast<const bf16x8*>(lds_a[S] + 8 * (octet * OA::PLANE + wave_m * T::WTM + 32 * i + a_row));
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
    // next stage's hand-off (`between`: the next step's register set waited
    // for by count, rounded into the other stage, then reloaded), and the
    // second chunk.
    auto step_from = [&](auto set, auto between) __attribute__((always_inline)) {
        bf16x8 fa0[T::FM], fb0[T::FN], fa1[T::FM], fb1[T::FN];
        read_chunk(set, 0, fa0, fb0);
        multiply_chunk(fa0, fb0);
        between();
        read_chunk(set, 1, fa1, fb1);
        multiply_chunk(fa1, fb1);
    };

    using I0 = std::integral_constant<int, 0>;
    const int steps = k_end > k_begin ? int((k_end - k_begin + T::BK - 1) / T::BK) : 0;
    // Step s (s % 2 == J) computes from LDS stage J while the set holding
    // step s + 1 is waited for (the later set stays in flight), rounded into
    // the other stage and reloaded with step s + 1 + NSETS.
    auto do_step = [&](auto j, int s) __attribute__((always_inline)) {
        constexpr int J = decltype(j)::value;
        using Stage = std::integral_constant<int, J % 2>;
        using NextSet = std::integral_constant<int, (J + 1) % NSETS>;
        using NextStage = std::integral_constant<int, (J + 1) % 2>;
        step_from(Stage{}, [&]() __attribute__((always_inline)) {
            wait_vector_loads<(NSETS - 1) * kSetLoads>();
            stage(NextSet{}, NextStage{});
            issue(NextSet{}, s + 1 + NSETS);
        });
        stage_barrier();
    };
    if (steps > 0) {
        issue(I0{}, 0);
        issue(std::integral_constant<int, 1>{}, 1);
        wait_vector_loads<(NSETS - 1) * kSetLoads>();  // set 0 (step 0) is in
        stage(I0{}, I0{});
        issue(I0{}, NSETS);
        stage_barrier();
        for (int s = 0; s < steps; s += 2) {
            do_step(std::integral_constant<int, 0>{}, s);
            if (s + 1 >= steps) break;
            do_step(std::integral_constant<int, 1>{}, s + 1);
        }
        wait_vector_loads<0>();
    }

    const bool partial = args.splits > 1;
    if constexpr (COLSUM) {
        if (colsum_tile) {
#pragma unroll
            for (int mask = 1; mask < 8; mask *= 2)
#pragma unroll
                for (int e = 0; e < 4; ++e) colsum[e] = colsum[e] + __shfl_xor(colsum[e], mask);
            if ((tid & 7) == 0) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int64_t c = n0 + 4 * LB::quad_of(tid / 8) + e;
                    if (c < args.n) {
                        if (partial)
                            args.ws[int64_t(args.splits) * args.m * args.n + int64_t(split) * args.n + c] = colsum[e];
                        else
                            args.column_sums[c] = args.column_sums[c] + colsum[e];
                    }
                }
            }
        }
    }
    float* c_batch = args.c + batch * args.stride_c;
    float* out = partial ? args.ws + ((batch_local * int64_t(args.splits) + split) * args.m) * args.n : c_batch;
    // The product goes out with streaming stores; split-K partials, which the
    // reduce reads back, with ordinary ones (measured 1 % faster over the set).
    if (partial)
        write_tile<T, true, false, false, 0, false, true>(args, acc, out, m0, n0, wave_m, wave_n, lane, partial);
    else
        write_tile<T, true, false, false, kStreaming, false, true>(args, acc, out, m0, n0, wave_m, wave_n, lane,
                                                                    partial);
}

// The same product as a persistent loop: each workgroup takes work items
// blockIdx.x, blockIdx.x + gridDim.x, ... (a matrix, K slice and 256 x 256
// tile, mapped by tile_coordinates as the one-tile launch maps its
// workgroups), for products whose tiles are all whole, read nothing back
// and have an even number of K-steps. The three loads a tile would issue
// past its last K-step (zeros, in the one-tile kernel) fetch the next item's
// first three K-steps instead, and its last step rounds the next item's
// first into LDS, so the next tile starts from data already in LDS and in
// registers. The tile's (streaming) output stores go out after those loads:
// load and store completions are counted in issue order (vmcnt), so the next
// tile's first two steps wait for their register sets with as many
// operations outstanding as were issued after them (the other set and the
// stores), and the stores drain under those two steps instead of ending the
// workgroup.
template <bool A_K, bool B_K, int SIDE>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_bf16_wide_persistent_kernel(
    Args args) {
    using T = WideTile;
    using LA = OperandLoader<A_K, SIDE == kStageLeft, T::BM, T::BK, T::THREADS>;
    using LB = OperandLoader<B_K, SIDE == kStageRight, T::BN, T::BK, T::THREADS, true>;
    using OA = OctetPlanes<T::BM, T::BK, LA::BF16_PAD>;
    using OB = OctetPlanes<T::BN, T::BK, LB::BF16_PAD>;
    constexpr int kSetLoads = loads_per_step<LA>() + loads_per_step<LB>();
    // Store instructions of the interior epilogue (one 16-byte store per row
    // of a lane's four adjacent columns), and the count the first two steps
    // of a tile wait down to: a set issued before the previous epilogue has
    // at least these many operations after it (the other set's loads and the
    // stores; a fused bias adds loads before the stores).
    constexpr int kStores = T::FM * 16;
    constexpr int kAfterEpilogue = kSetLoads + kStores;
    static_assert(kAfterEpilogue < 64, "vmcnt is 6 bits");
    __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][8 * OA::SLOTS];
    __shared__ __attribute__((aligned(16))) uint16_t lds_b[2][8 * OB::SLOTS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave / T::WAVES_N;
    const int wave_n = wave % T::WAVES_N;
    const int row = lane & 31;
    const int half = lane >> 5;
    const int a_row = LA::row_slot(row);  // where the A operand's loader put this lane's row
    const int items = args.persistent_items;
    const int stride = int(gridDim.x);

    struct Item {
        int tm, tn, batch_local, split;
    };
    auto item_of = [&](int w) {
        Item it;
        tile_coordinates(w, items, args.tiles_m, args.tiles_n, args.splits, it.batch_local, it.split, it.tm, it.tn);
        return it;
    };
    int w = int(blockIdx.x);
    if (w >= items) return;
    Item cur = item_of(w);

    constexpr int NSETS = 2;
    LA la[NSETS];
    LB lb[NSETS];
    // Whole tiles only (checked on the host): the loaders' offsets are the
    // same for every item.
#pragma unroll
    for (int j = 0; j < NSETS; ++j) {
        la[j].init(args.lda, 0, T::BM, tid);
        lb[j].init(args.ldb, 0, T::BN, tid);
    }
    // The item whose loads are being issued.
    const float* ld_a = args.a + (args.batch_base + cur.batch_local) * args.stride_a;
    const float* ld_b = args.b + (args.batch_base + cur.batch_local) * args.stride_b;
    int64_t ld_m0 = int64_t(cur.tm) * T::BM, ld_n0 = int64_t(cur.tn) * T::BN;
    int64_t ld_begin = int64_t(cur.split) * args.k_per_split;
    int64_t ld_end = min(args.k, ld_begin + args.k_per_split);
    auto switch_loads = [&](const Item& it) __attribute__((always_inline)) {
        ld_a = args.a + (args.batch_base + it.batch_local) * args.stride_a;
        ld_b = args.b + (args.batch_base + it.batch_local) * args.stride_b;
        ld_m0 = int64_t(it.tm) * T::BM;
        ld_n0 = int64_t(it.tn) * T::BN;
        ld_begin = int64_t(it.split) * args.k_per_split;
        ld_end = min(args.k, ld_begin + args.k_per_split);
    };

    f32x16 acc[T::FM][T::FN];
    // Loads of K-step `step` of the load item into register set S (past its
    // end: out of range, zeros).
    auto issue = [&](auto set, int step) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        const int64_t k0 = ld_begin + int64_t(step) * T::BK;
        la[S].load(ld_a, args.lda, ld_m0, args.m, k0, ld_end, tid);
        lb[S].load(ld_b, args.ldb, ld_n0, args.n, k0, ld_end, tid);
    };
    auto stage = [&](auto set, auto lds) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        constexpr int L = decltype(lds)::value;
        la[S].store_bf16(lds_a[L], tid);
        lb[S].store_bf16(lds_b[L], tid);
    };
    auto read_chunk = [&](auto set, int c, bf16x8 (&fa)[T::FM], bf16x8 (&fb)[T::FN]) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        const int octet = 2 * c + half;
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
            fa[i] = *reinterpret_cast<const bf16x8*>(lds_a[S] + 8 * (octet * OA::PLANE + wave_m * T::WTM + 32 * i + a_row));
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
    auto step_from = [&](auto set, auto between) __attribute__((always_inline)) {
        bf16x8 fa0[T::FM], fb0[T::FN], fa1[T::FM], fb1[T::FN];
        read_chunk(set, 0, fa0, fb0);
        multiply_chunk(fa0, fb0);
        between();
        read_chunk(set, 1, fa1, fb1);
        multiply_chunk(fa1, fb1);
    };
    // Step s (s % 2 == J) computes from LDS stage J while register set
    // (J + 1) % 2 (step s + 1 of the tile, or the next item's) is waited for,
    // rounded into the other stage and reloaded with `load_step` of the load
    // item. AFTER_STORES: the first two steps after an epilogue, whose sets
    // were issued before its stores.
    auto do_step = [&](auto j, int load_step, auto after_stores) __attribute__((always_inline)) {
        constexpr int J = decltype(j)::value;
        using Stage = std::integral_constant<int, J>;
        using NextSet = std::integral_constant<int, (J + 1) % NSETS>;
        using NextStage = std::integral_constant<int, (J + 1) % 2>;
        step_from(Stage{}, [&]() __attribute__((always_inline)) {
            if constexpr (decltype(after_stores)::value) wait_vector_loads<kAfterEpilogue>();
            else wait_vector_loads<(NSETS - 1) * kSetLoads>();
            stage(NextSet{}, NextStage{});
            issue(NextSet{}, load_step);
        });
        stage_barrier();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using Plain = std::false_type;
    using AfterStores = std::true_type;

    issue(I0{}, 0);
    issue(I1{}, 1);
    wait_vector_loads<(NSETS - 1) * kSetLoads>();  // set 0 (step 0) is in
    stage(I0{}, I0{});
    issue(I0{}, NSETS);
    stage_barrier();
    bool first = true;
    for (;;) {
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
#pragma unroll
            for (int j = 0; j < T::FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
        const int64_t k_begin = int64_t(cur.split) * args.k_per_split;
        const int steps = int((min(args.k, k_begin + args.k_per_split) - k_begin + T::BK - 1) / T::BK);
        const bool has_next = w + stride < items;
        const Item next = has_next ? item_of(w + stride) : cur;
        // Step s loads step s + 3: the tile's own while s + 3 < steps, then
        // the next item's 0, 1 and 2 (a load cursor switched once).
        auto load_step = [&](int s) __attribute__((always_inline)) {
            const int target = s + 1 + NSETS;
            if (target == steps && has_next) switch_loads(next);
            return target >= steps && has_next ? target - steps : target;
        };
        int s = 0;
        if (!first) {
            do_step(I0{}, load_step(0), AfterStores{});
            do_step(I1{}, load_step(1), AfterStores{});
            s = 2;
        }
        for (; s < steps; s += 2) {
            do_step(I0{}, load_step(s), Plain{});
            do_step(I1{}, load_step(s + 1), Plain{});
        }
        const bool partial = args.splits > 1;
        float* out = partial ? args.ws + ((cur.batch_local * int64_t(args.splits) + cur.split) * args.m) * args.n
                             : args.c + (args.batch_base + cur.batch_local) * args.stride_c;
        const int64_t m0 = int64_t(cur.tm) * T::BM, n0 = int64_t(cur.tn) * T::BN;
        if (partial)
            write_tile<T, true, false, false, 0, true, true>(args, acc, out, m0, n0, wave_m, wave_n, lane, partial);
        else
            write_tile<T, true, false, false, kStreaming, true, true>(args, acc, out, m0, n0, wave_m, wave_n, lane,
                                                                       partial);
        if (!has_next) break;
        w += stride;
        cur = next;
        first = false;
    }
    wait_vector_loads<0>();
}

// Split-K under the launch model of plan_for: one workgroup per CU, and the
// per-CU rate the split counts were measured with.
Plan wide_plan(const Problem& p, const Env& env) {
    SplitCost cost;
    cost.workgroups_per_cu = 1;
    cost.flops_per_cu = 3.5e12;
    return plan_for<WideTile>(p, env, cost);
}

// The operand the workspace holds as bf16, and the product as the kernel
// sees it (that operand K-contiguous bf16 in the workspace, ld = kp; the
// partial sums after it).
struct WideStaging {
    int side = kStageNone;
    int64_t kp = 0;        // K rounded up to a whole step
    int64_t rows_pad = 0;  // the staged operand's rows rounded up to a whole tile
    int64_t copies = 0;    // 1 when the operand is shared by the whole batch
    size_t bytes = 0;
    Problem q;
    Env rest;
};

size_t round256(size_t bytes) { return (bytes + 255) / 256 * 256; }

// Stages the operand with fewer elements (the weight, for the Linear
// products) when it has at most half the other's elements and fits beside
// the partial sums: rounding it once costs 6 bytes an element, while every
// tile row (or column) that reads it then fetches 2 bytes an element
// instead of 4. Measured on the 111.5M model's set (596 TFLOP/s against 558 with nothing
// staged): a quarter as the bound 595, any smaller operand 592 (the square
// weight gradients then pay the staging for no gain).
constexpr int kStageRatio = 2;
// ... and only when at least kStageMinReuse tiles of the other operand read
// the staged copy (tiles across the other output dimension, times the
// batches that share it). The weight of the forward and input-gradient
// products (128 tile rows at M = 32768) and x^T of the head's weight
// gradient (64 tile columns) repay their staging pass; x^T of the qkv and up
// weight gradients (9 and 12 tile columns: 100 MB of fp32 read, 50 MB
// written and read back, 33 us a pass) ran 5 % faster rounded as loaded
// (qkv TN 598-634 -> 647-652 TFLOP/s, up 634-643 -> 663-677), the down
// projection's dY (12 tile rows) the same either way. With STAGE_SUMS (the
// fused bias gradient) a right operand is staged whatever its reuse, as
// that pass also takes its column sums.
constexpr int64_t kStageMinReuse = 32;
WideStaging wide_staging(const Problem& p, const Env& env, bool stage_sums = false) {
    WideStaging st;
    st.q = p;
    st.rest = env;
    const int64_t a_copies = p.stride_a == 0 ? 1 : p.batch;
    const int64_t b_copies = p.stride_b == 0 ? 1 : p.batch;
    const double a_elems = double(p.m) * double(a_copies), b_elems = double(p.n) * double(b_copies);
    int side = kStageNone;
    if (b_elems * kStageRatio <= a_elems) side = kStageRight;
    else if (a_elems * kStageRatio <= b_elems) side = kStageLeft;
    if (side == kStageNone || env.workspace == nullptr || p.batch > 65535) return st;
    const int64_t rows = side == kStageLeft ? p.m : p.n;
    const int64_t copies = side == kStageLeft ? a_copies : b_copies;
    const int64_t reuse = (side == kStageLeft ? (p.n + WideTile::BN - 1) / WideTile::BN
                                              : (p.m + WideTile::BM - 1) / WideTile::BM) *
                          (copies == 1 ? p.batch : 1);
    if (reuse < kStageMinReuse && !(stage_sums && side == kStageRight)) return st;
    // The blocked layout (launch_stage_bf16_blocks): whole steps of K, whole
    // tiles of rows; `ld` of the staged operand is its padded row count.
    const int64_t kp = (p.k + WideTile::BK - 1) / WideTile::BK * WideTile::BK;
    constexpr int64_t kTileRows = WideTile::BM > WideTile::BN ? WideTile::BM : WideTile::BN;
    const int64_t rows_pad = (rows + kTileRows - 1) / kTileRows * kTileRows;
    const size_t bytes = round256(size_t(copies) * size_t(rows_pad) * size_t(kp) * 2);
    if (bytes >= env.workspace_bytes) return st;
    Problem q = p;
    const float* staged = env.workspace;
    if (side == kStageLeft) {
        q.a = staged;
        q.lda = rows_pad;
        q.stride_a = copies > 1 ? rows_pad * kp / 2 : 0;
        q.a_k_contiguous = true;
    } else {
        q.b = staged;
        q.ldb = rows_pad;
        q.stride_b = copies > 1 ? rows_pad * kp / 2 : 0;
        q.b_k_contiguous = true;
    }
    Env rest = env;
    rest.workspace = reinterpret_cast<float*>(reinterpret_cast<char*>(env.workspace) + bytes);
    rest.workspace_bytes = env.workspace_bytes - bytes;
    const Plan plan = wide_plan(q, rest);
    if (plan.splits > 1 && size_t(plan.splits) * size_t(p.m) * size_t(p.n) * sizeof(float) > rest.workspace_bytes)
        return st;
    st.side = side;
    st.kp = kp;
    st.rows_pad = rows_pad;
    st.copies = copies;
    st.bytes = bytes;
    st.q = q;
    st.rest = rest;
    return st;
}

// The grid of the persistent kernel for `p` (the product as the kernel sees
// it, with any staged operand), or 0 for the one-tile kernel: one launch,
// whole tiles that read nothing back, slices of an even number (at least
// four) of K-steps, and either two work items per CU or more, or more than
// one with tiles of at most kWidePersistentShortSteps K-steps (where the
// output write is a large share of a tile). One workgroup per CU, rounded
// down to whole XCDs. Measured on config 2's bf16 products against the
// one-tile kernel: NN qkv / up / head (K = 768, 4.5 to 32 tiles per CU)
// 664-668 -> 698-716, 736-746 -> 806-807, 760-770 -> 826-843 TFLOP/s; NT
// down (6 per CU) 752-765 -> 816-822; NN out (1.5 per CU, 24 K-steps)
// 537-567 -> 589-591; the 1.5-per-CU products with 72 to 512 K-steps
// (NN down, NT qkv / up / head) unchanged to 3 % slower, so they keep the
// one-tile kernel.
constexpr int64_t kWidePersistentShortSteps = 32;

int64_t wide_persistent_grid(const Problem& p, const Env& env, const Plan& plan, const LaunchShape& shape) {
    using T = WideTile;
    if (shape.batches_per_launch < p.batch || p.m % T::BM != 0 || p.n % T::BN != 0 ||
        (plan.splits == 1 && p.accumulate))
        return 0;
    const int64_t items = int64_t(plan.tiles_m) * plan.tiles_n * plan.splits * p.batch;
    const int64_t slots = int64_t(std::max(env.cu_count, 1)) / kXcds * kXcds;
    if (slots < kXcds || items <= slots || items > 0x7FFFFFFF) return 0;
    const int64_t steps = (plan.k_per_split + T::BK - 1) / T::BK;
    const int64_t last_steps = (p.k - int64_t(plan.splits - 1) * plan.k_per_split + T::BK - 1) / T::BK;
    if (steps % 2 != 0 || last_steps % 2 != 0 || last_steps < 4) return 0;
    if (items < 2 * slots && steps > kWidePersistentShortSteps) return 0;
    return slots;
}

template <bool A_K, bool B_K, int SIDE, bool COLSUM = false>
hipError_t launch_wide(const Problem& p, const Env& env, const Plan& plan, hipStream_t stream) {
    const LaunchShape shape = tiled_shape<WideTile>(p, plan, SN_PATH_BF16_WIDE);
    if (shape.batches_per_launch < 1) return hipErrorInvalidConfiguration;
    Args args = make_args<WideTile>(p, env, plan);
    if constexpr (!COLSUM) {
        const int64_t grid = wide_persistent_grid(p, env, plan, shape);
        if (grid > 0) {
            args.persistent_items = int32_t(int64_t(plan.tiles_m) * plan.tiles_n * plan.splits * p.batch);
            hipLaunchKernelGGL((gemm_bf16_wide_persistent_kernel<A_K, B_K, SIDE>), dim3(unsigned(grid)),
                               dim3(WideTile::THREADS), 0, stream, args);
            hipError_t err = hipGetLastError();
            if (err != hipSuccess) return err;
            if (plan.splits > 1) return launch_splitk_reduce(p, env, plan.splits, stream);
            return hipSuccess;
        }
    }
    const int64_t per_batch = int64_t(plan.tiles_m) * plan.tiles_n * plan.splits;
    const int64_t chunk = shape.batches_per_launch;
    for (int64_t first = 0; first < p.batch; first += chunk) {
        const int64_t count = std::min<int64_t>(chunk, p.batch - first);
        args.batch_base = first;
        hipLaunchKernelGGL((gemm_bf16_wide_kernel<A_K, B_K, SIDE, COLSUM>), dim3(unsigned(count * per_batch)),
                           dim3(WideTile::THREADS), 0, stream, args);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (plan.splits > 1) return launch_splitk_reduce(p, env, plan.splits, stream);
    return hipSuccess;
}

}  // namespace

// Unmasked products with 128-bit-loadable operands (buffers_ok) whose output
// fills at least a quarter of a 256 x 256 tile each way, and room for the
// partial sums. Measured on the 111.5M model's products against staging both operands as
// bf16 for the 128 x 256 kernel (gemm_dma.hip): weight gradients (TN)
// 310-549 -> 394-755 TFLOP/s, input gradients (NT) 464-616 -> 517-826,
// forward (NN) 430-601 -> 496-693.
//
// Products whose 256 x 256 plan leaves more than half the CUs idle (the 7.1M model's
// products: 2048 x 768 x 256 is 24 tiles) take the 128-wide kernels instead:
// the 7.1M model's bf16 set 52.0 -> 59.4 TFLOP/s, 2048 x 768 x 256 47 -> 55
// (a whole-device threshold cost the 111.5M model's set 7 %).
bool bf16_wide_applies(const Problem& p, const Env& env) {
    if (p.mask != SN_MASK_NONE || p.m < 128 || p.n < 128 || !buffers_ok<WideTile>(p)) return false;
    const WideStaging st = wide_staging(p, env);
    const Plan fill = wide_plan(st.q, st.rest);
    if (2 * int64_t(fill.tiles_m) * fill.tiles_n * fill.splits * p.batch < std::max(env.cu_count, 1)) return false;
    if (st.side != kStageNone) return true;
    const Plan plan = wide_plan(p, env);
    return plan.splits <= 1 || size_t(plan.splits) * size_t(p.m) * size_t(p.n) * sizeof(float) <= env.workspace_bytes;
}

LaunchShape describe_bf16_wide(const Problem& p, const Env& env) {
    const WideStaging st = wide_staging(p, env);
    const Plan plan = wide_plan(st.q, st.rest);
    LaunchShape shape = tiled_shape<WideTile>(st.q, plan, SN_PATH_BF16_WIDE);
    shape.persistent_grid = wide_persistent_grid(st.q, st.rest, plan, shape);
    shape.workspace_bytes += st.bytes;
    return shape;
}

hipError_t launch_gemm_bf16_wide(const Problem& p, const Env& env, hipStream_t stream) {
    const WideStaging st = wide_staging(p, env);
    const Problem& q = st.q;
    const Plan plan = wide_plan(q, st.rest);
    if (st.side == kStageLeft) {
        hipError_t err = launch_stage_bf16_blocks(p.a, p.a_k_contiguous, p.lda, p.m, p.k, st.kp, st.rows_pad, false,
                                                  st.copies, p.stride_a, reinterpret_cast<uint16_t*>(env.workspace),
                                                  stream);
        if (err != hipSuccess) return err;
        if (q.b_k_contiguous) return launch_wide<true, true, kStageLeft>(q, st.rest, plan, stream);
        return launch_wide<true, false, kStageLeft>(q, st.rest, plan, stream);
    }
    if (st.side == kStageRight) {
        hipError_t err = launch_stage_bf16_blocks(p.b, p.b_k_contiguous, p.ldb, p.n, p.k, st.kp, st.rows_pad, true,
                                                  st.copies, p.stride_b, reinterpret_cast<uint16_t*>(env.workspace),
                                                  stream);
        if (err != hipSuccess) return err;
        if (q.a_k_contiguous) return launch_wide<true, true, kStageRight>(q, st.rest, plan, stream);
        return launch_wide<false, true, kStageRight>(q, st.rest, plan, stream);
    }
    if (p.a_k_contiguous && p.b_k_contiguous) return launch_wide<true, true, kStageNone>(p, env, plan, stream);
    if (p.a_k_contiguous) return launch_wide<true, false, kStageNone>(p, env, plan, stream);
    if (p.b_k_contiguous) return launch_wide<false, true, kStageNone>(p, env, plan, stream);
    return launch_wide<false, false, kStageNone>(p, env, plan, stream);
}

// ---- The weight-gradient product with Linear's bias gradient -------------
//
// dY, the right operand of dW += x^T dY, is row-contiguous fp32. Unless it is
// the operand staged as bf16 (when it has at most half x's columns), every
// 256 x 32 slab of it passes through the registers as fp32 before rounding,
// and the first tile row sums its columns there. Each K slice also leaves N
// partial column sums after the product's partials, so the split count is
// chosen as if the workspace left after staging were M / (M + 1) of its size.
// When dY is the staged operand (the down projection: N <= M / 2), the
// staging pass, which reads all of dY as fp32 once, takes the sums instead:
// one partial per 64 k and column (stage_sum_tiles x N floats after the
// product's partials), added in k order by the finish kernel.

namespace {

size_t staged_sum_bytes(const WideStaging& st, const Problem& p) {
    return size_t(stage_sum_tiles(st.kp)) * size_t(p.n) * sizeof(float);
}

Plan wide_column_sums_plan(const WideStaging& st, const Problem& p) {
    Env e = st.rest;
    if (st.side == kStageRight) {
        const size_t sums = staged_sum_bytes(st, p);
        e.workspace_bytes = st.rest.workspace_bytes > sums ? st.rest.workspace_bytes - sums : 0;
    } else {
        e.workspace_bytes = st.rest.workspace_bytes / size_t(p.m + 1) * size_t(p.m);
    }
    return wide_plan(st.q, e);
}

// Workspace after the staged operand: the product's split partials, then the
// column sums' partials (per K slice, or per 64 k of the staging pass).
size_t product_partial_bytes(const Plan& plan, const Problem& p) {
    return plan.splits > 1 ? size_t(plan.splits) * size_t(p.m) * size_t(p.n) * sizeof(float) : 0;
}

size_t column_partial_bytes(const WideStaging& st, const Plan& plan, const Problem& p) {
    if (st.side == kStageRight) return staged_sum_bytes(st, p);
    return plan.splits > 1 ? size_t(plan.splits) * size_t(p.n) * sizeof(float) : 0;
}

}  // namespace

bool bf16_wide_column_sums_applies(const Problem& p, const Env& env) {
    if (p.batch != 1 || p.m < 1 || p.k < 1 || p.b_k_contiguous || p.bias != nullptr || !bf16_wide_applies(p, env))
        return false;
    const WideStaging st = wide_staging(p, env, true);
    const Plan plan = wide_column_sums_plan(st, p);
    return product_partial_bytes(plan, p) + column_partial_bytes(st, plan, p) <= st.rest.workspace_bytes;
}

LaunchShape describe_bf16_wide_column_sums(const Problem& p, const Env& env) {
    const WideStaging st = wide_staging(p, env, true);
    const Plan plan = wide_column_sums_plan(st, p);
    LaunchShape shape = tiled_shape<WideTile>(st.q, plan, SN_PATH_BF16_WIDE);
    // With dY staged, the staging pass takes the sums and the product runs
    // as launch_gemm_bf16_wide's (persistent where its tiles allow).
    if (st.side == kStageRight) shape.persistent_grid = wide_persistent_grid(st.q, st.rest, plan, shape);
    shape.workspace_bytes += st.bytes + column_partial_bytes(st, plan, p);
    return shape;
}

hipError_t launch_gemm_bf16_wide_column_sums(const Problem& p, const Env& env, hipStream_t stream) {
    const WideStaging st = wide_staging(p, env, true);
    const Problem& q = st.q;
    const Plan plan = wide_column_sums_plan(st, p);
    hipError_t err = hipSuccess;
    if (st.side == kStageRight) {
        float* sums = st.rest.workspace + product_partial_bytes(plan, p) / sizeof(float);
        err = launch_stage_bf16_blocks(p.b, false, p.ldb, p.n, p.k, st.kp, st.rows_pad, true, 1, p.stride_b,
                                       reinterpret_cast<uint16_t*>(env.workspace), stream, sums);
        if (err == hipSuccess)
            err = q.a_k_contiguous ? launch_wide<true, true, kStageRight>(q, st.rest, plan, stream)
                                   : launch_wide<false, true, kStageRight>(q, st.rest, plan, stream);
        if (err != hipSuccess) return err;
        return launch_column_sums_finish(sums, stage_sum_tiles(st.kp), p.n, p.column_sums, stream);
    }
    if (st.side == kStageLeft) {
        err = launch_stage_bf16_blocks(p.a, p.a_k_contiguous, p.lda, p.m, p.k, st.kp, st.rows_pad, false, st.copies,
                                       p.stride_a, reinterpret_cast<uint16_t*>(env.workspace), stream);
        if (err == hipSuccess) err = launch_wide<true, false, kStageLeft, true>(q, st.rest, plan, stream);
    } else {
        err = p.a_k_contiguous ? launch_wide<true, false, kStageNone, true>(p, env, plan, stream)
                               : launch_wide<false, false, kStageNone, true>(p, env, plan, stream);
    }
    if (err != hipSuccess || plan.splits == 1) return err;
    return launch_column_sums_finish(st.rest.workspace + int64_t(plan.splits) * p.m * p.n, plan.splits, p.n,
                                     p.column_sums, stream);
}

}  // namespace gemm
}  // namespace sn

// fp32 matrix-core GEMM fed by direct global -> LDS loads, and its
// bf16-input / fp32-accumulate variant.
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
//      ds_read_b32 (consecutive rows across lanes: conflict-free); when a
//      wave has two blocks on that side, they interleave their rows (block
//      i takes rows 2q + i) and a lane reads both blocks' values of a k in
//      one ds_read_b64 (the epilogue places the outputs accordingly:
//      TileMap). Measured on c2's fp32 set: NN +1 %, TN +1.5 %.
//  * Two or more LDS stages (32 KB each for 128x128), all in flight: a
//    stage is reloaded, STAGES steps ahead, as soon as every wave has read
//    it. The one barrier per K-step sits between its two 16-deep chunks, so
//    each chunk's fragments are read from LDS while the previous chunk is
//    multiplied and the matrix cores never wait on an LDS read.
//  * bf16 variant: the same fp32 stages; each lane rounds its fragments to
//    bf16 in registers and issues one 32x32x16 bf16 MFMA per block and chunk.
//
// Within a 16-deep chunk, lane half h feeds k = 8h + s to MFMA s on both
// operands (the same pairing as gemm_mfma.hip).
#include "gemm_common.h"

namespace sn {
namespace gemm {
namespace {

typedef __attribute__((address_space(3))) void* lds_void;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

// Eight floats rounded to bf16 (four v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16x8 to_bf16x8(const float (&v)[8]) {
    const f32x8 x = {v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
    return __builtin_convertvector(x, bf16x8);
}

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, const void* lds, int32_t offset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void)lds, 16, offset, 0, 0, 0);
}

// K-contiguous operand: ROWS rows of 32 k per stage, ROWS / 8 load
// instructions of 8 rows each, shared out over the WAVES waves.
template <int ROWS, int WAVES>
struct OperandK {
    static constexpr int PER_WAVE = ROWS / (8 * WAVES);
    static_assert(ROWS % (8 * WAVES) == 0, "whole load instructions per wave");
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
// ROWS / 8 load instructions of 256 values (64 lanes x 4), shared out over
// the WAVES waves.
template <int ROWS, int WAVES>
struct OperandR {
    static constexpr int PER_WAVE = ROWS / (8 * WAVES);
    static_assert(ROWS % (8 * WAVES) == 0 && ROWS <= 256, "whole load instructions per wave");
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

    // The fragments of two blocks that interleave their rows (TileMap's
    // pairs): rows r2 and r2 + 1 (r2 even) of each k in one 8-byte read, the
    // first to v0, the second to v1. Half the LDS read instructions of two
    // fragment() calls; lanes read consecutive 8-byte pieces (conflict-free).
    __device__ __forceinline__ void fragment_pair(const f32x4* stage, int r2, int c, int h, float (&v0)[8],
                                                  float (&v1)[8]) const {
        const float* base = reinterpret_cast<const float*>(stage) + (16 * c + 8 * h) * ROWS + r2;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const float2 p = *reinterpret_cast<const float2*>(base + s * ROWS);
            v0[s] = p.x;
            v1[s] = p.y;
        }
    }
};

// Whether a side's two 32-row (or 32-column) blocks are read as pairs: a
// row-contiguous operand with exactly two blocks per wave on that side.
template <class T, bool K_CONTIGUOUS, bool M_SIDE>
constexpr bool paired() {
    return !K_CONTIGUOUS && (M_SIDE ? T::FM : T::FN) == 2;
}

template <bool K_CONTIGUOUS, int ROWS, int WAVES>
using OperandFor =
    typename std::conditional<K_CONTIGUOUS, OperandK<ROWS, WAVES>, OperandR<ROWS, WAVES>>::type;

// One 16-deep chunk of a wave's fragments: FM A and FN B fragments, 8 values
// per lane (k = 16 c + 8 h + s for lane half h, s = 0..7).
template <class T>
struct Chunk {
    float a[T::FM][8];
    float b[T::FN][8];
};

template <class T, bool A_K, bool B_K>
__device__ __forceinline__ void read_chunk(const OperandFor<A_K, T::BM, T::THREADS / 64>& oa,
                                           const OperandFor<B_K, T::BN, T::THREADS / 64>& ob, const f32x4* sa,
                                           const f32x4* sb, int c, Chunk<T>& f, int lane, int wave_m, int wave_n) {
    const int row = lane & 31;
    const int half = lane >> 5;
    if constexpr (paired<T, A_K, true>()) {
        oa.fragment_pair(sa, wave_m * T::WTM + 2 * row, c, half, f.a[0], f.a[1]);
    } else {
#pragma unroll
        for (int i = 0; i < T::FM; ++i) oa.fragment(sa, wave_m * T::WTM + 32 * i + row, c, half, f.a[i]);
    }
    if constexpr (paired<T, B_K, false>()) {
        ob.fragment_pair(sb, wave_n * T::WTN + 2 * row, c, half, f.b[0], f.b[1]);
    } else {
#pragma unroll
        for (int j = 0; j < T::FN; ++j) ob.fragment(sb, wave_n * T::WTN + 32 * j + row, c, half, f.b[j]);
    }
}

// How the LDS stages feed the matrix cores.
//  kFeedF32: fp32 stages, eight v_mfma_f32_32x32x2_f32 per block, lane half
//    h feeding k = 8h + s to MFMA s.
//  kFeedRound: fp32 stages; the same eight values per lane are rounded to
//    bf16 (v_cvt_pk_bf16_f32, nearest-even) and feed one
//    v_mfma_f32_32x32x16_bf16, whose lane half h holds k = 8h .. 8h+7.
//  kFeedBf16: bf16 stages (operands converted before the product, both
//    K-contiguous). A stage row is the same 128 bytes, now 64 k, and the
//    kernel counts k in pairs; a lane's 8 words of a chunk are 16 bf16, k =
//    32c + 16h + (0..15), which feed two v_mfma_f32_32x32x16_bf16 (the
//    first 8 and the last 8).
// In every mode A and B are paired on the same k.
constexpr int kFeedF32 = 0;
constexpr int kFeedRound = 1;
constexpr int kFeedBf16 = 2;

template <class T, int FEED>
__device__ __forceinline__ void multiply_chunk(const Chunk<T>& f, f32x16 (&acc)[T::FM][T::FN]) {
    if constexpr (FEED == kFeedBf16) {
        bf16x8 a8[T::FM][2], b8[T::FN][2];
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
#pragma unroll
            for (int q = 0; q < 2; ++q)
                a8[i][q] = __builtin_bit_cast(
                    bf16x8, f32x4{f.a[i][4 * q], f.a[i][4 * q + 1], f.a[i][4 * q + 2], f.a[i][4 * q + 3]});
#pragma unroll
        for (int j = 0; j < T::FN; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q)
                b8[j][q] = __builtin_bit_cast(
                    bf16x8, f32x4{f.b[j][4 * q], f.b[j][4 * q + 1], f.b[j][4 * q + 2], f.b[j][4 * q + 3]});
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int i = 0; i < T::FM; ++i)
#pragma unroll
                for (int j = 0; j < T::FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8[i][q], b8[j][q], acc[i][j], 0, 0, 0);
    } else if constexpr (FEED == kFeedRound) {
        bf16x8 a8[T::FM], b8[T::FN];
#pragma unroll
        for (int i = 0; i < T::FM; ++i) a8[i] = to_bf16x8(f.a[i]);
#pragma unroll
        for (int j = 0; j < T::FN; ++j) b8[j] = to_bf16x8(f.b[j]);
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
#pragma unroll
            for (int j = 0; j < T::FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a8[i], b8[j], acc[i][j], 0, 0, 0);
    } else {
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int i = 0; i < T::FM; ++i)
#pragma unroll
                for (int j = 0; j < T::FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[i][s], f.b[j][s], acc[i][j], 0, 0, 0);
    }
}

// Orders one half-step for the scheduler: the chunk's conversions (bf16),
// then its MFMAs with the VM loads and DS fragment reads issued in their
// shadow, spread evenly (left alone, the scheduler issues each LDS read
// just before its first use and waits on it there).
template <class T, int FEED, int VM, int DS>
__device__ __forceinline__ void interleave() {
    constexpr int MF = (FEED == kFeedF32 ? 8 : FEED == kFeedBf16 ? 2 : 1) * T::FM * T::FN;
    if constexpr (FEED == kFeedRound) __builtin_amdgcn_sched_group_barrier(0x002, 4 * (T::FM + T::FN), 0);
#pragma unroll
    for (int x = 0; x < MF; ++x) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if constexpr (VM > 0)
            if (x * ((VM + MF - 1) / MF) < VM) __builtin_amdgcn_sched_group_barrier(0x020, (VM + MF - 1) / MF, 0);
        if (x * ((DS + MF - 1) / MF) < DS) __builtin_amdgcn_sched_group_barrier(0x100, (DS + MF - 1) / MF, 0);
    }
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

// Waves per SIMD that STAGES LDS stages allow (160 KB of LDS per CU), at
// most 4: 128 registers a lane (the 64 x 64 tile's LDS would allow 5, whose
// 96 registers spilled).
template <class T, int STAGES>
constexpr int dma_waves_per_eu() {
    const int by_lds = (160 * 1024 / ((T::BM + T::BN) * T::BK * 4 * STAGES)) * (T::THREADS / 64) / 4;
    return by_lds < 4 ? by_lds : 4;
}

// Waits until at most PENDING of this wave's vector-memory instructions are
// outstanding (vmcnt; expcnt and lgkmcnt left at their maxima; gfx9
// encoding: vmcnt bits 3:0 and 15:14).
template <int PENDING>
__device__ __forceinline__ void wait_loads() {
    static_assert(PENDING >= 0 && PENDING < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (PENDING & 15) | ((PENDING >> 4) << 14));
}

// Workgroup barrier for the stage hand-off. __syncthreads() fences every
// address space, and the compiler implements the fence by waiting for all of
// the wave's outstanding vector-memory loads, including the prefetches of
// later stages that are meant to stay in flight (an LDS-only fence does the
// same, since the direct-to-LDS loads are LDS writes). Here the stage's own
// loads are waited for explicitly (wait_loads), this wave's LDS writes
// (mask_stage) by lgkmcnt(0), and the empty asm statements keep the
// compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// One output tile (the whole of the kernels below); FEED selects what the
// stages hold and the matrix instruction they feed.
//
// STAGES LDS stages, all loading from the start: a stage is reloaded for
// the step STAGES ahead as soon as every wave has read it. One barrier per
// K-step, between its two 16-deep chunks (see the step halves below). At
// the barrier a wave waits until only the later stages' loads are still in
// flight (a wave's loads complete in order). Every step issues its loads
// unconditionally: loads past the tile's K range are out of bounds (no
// memory traffic, zeros), which keeps each step's load count, and so the
// wait count, fixed. The loop is unrolled by STAGES so that every LDS
// access names a statically known stage array; the compiler then never
// waits on loads into the other stages before its LDS reads.
template <class T, int STAGES, bool A_K, bool B_K, int FEED, bool COLSUM = false>
__device__ __forceinline__ void dma_tile(const Args& args) {
    static_assert(STAGES >= 2 && STAGES <= 4, "two to four LDS stages");
    static_assert(!COLSUM || (!B_K && FEED == kFeedF32), "column sums of a row-contiguous fp32 right operand");
    constexpr int WAVES = T::THREADS / 64;
    constexpr int A_SLOTS = T::BM * T::BK / 4;
    constexpr int B_SLOTS = T::BN * T::BK / 4;
    __shared__ f32x4 a0[A_SLOTS], b0[B_SLOTS], a1[A_SLOTS], b1[B_SLOTS];
    __shared__ f32x4 a2[STAGES > 2 ? A_SLOTS : 1], b2[STAGES > 2 ? B_SLOTS : 1];
    __shared__ f32x4 a3[STAGES > 3 ? A_SLOTS : 1], b3[STAGES > 3 ? B_SLOTS : 1];
    f32x4* const stage_a[4] = {a0, a1, a2, a3};
    f32x4* const stage_b[4] = {b0, b1, b2, b3};

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

    OperandFor<A_K, T::BM, WAVES> oa;
    OperandFor<B_K, T::BN, WAVES> ob;
    oa.init(args.lda, m0, args.m, lane, wave);
    ob.init(args.ldb, n0, args.n, lane, wave);

    f32x16 acc[T::FM][T::FN];
#pragma unroll
    for (int i = 0; i < T::FM; ++i)
#pragma unroll
        for (int j = 0; j < T::FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Loads stop at the tile's K end: a partial last step, and loads past
    // the last step, read zeros.
    auto issue = [&](const f32x4* sa, const f32x4* sb, int64_t k0) {
        if constexpr (A_K) oa.issue(sa, a, k0, k_end, wave);
        else oa.issue(sa, a, args.lda, k0, k_end, wave);
        if constexpr (B_K) ob.issue(sb, b, k0, k_end, wave);
        else ob.issue(sb, b, args.ldb, k0, k_end, wave);
    };
    // Causal-left: A values past the diagonal are zeroed in LDS on the
    // K-steps that reach it (A K-contiguous: keys past the tile's first
    // query; A transposed: queries before the tile's last key).
    auto mask_if_needed = [&](f32x4* sa, int64_t k0) {
        if (left_causal && (A_K ? k0 + T::BK - 1 > m0 + args.query_offset : k0 + args.query_offset < row_last)) {
            mask_stage<T, A_K>(sa, m0, k0, args.query_offset, tid);
            lds_barrier();
        }
    };
    constexpr int LOADS_PER_STEP = (T::BM + T::BN) / (8 * WAVES);
    // LDS read instructions per chunk (the compiler merges row-contiguous
    // reads in twos: ds_read2_b32, or ds_read2_b64 for pairs).
    constexpr int DS = (A_K ? 2 * T::FM : paired<T, A_K, true>() ? 4 : 4 * T::FM) +
                       (B_K ? 2 * T::FN : paired<T, B_K, false>() ? 4 : 4 * T::FN);
    Chunk<T> f0, f1;
    // A K-step on stage S is two halves around one barrier. Entered with
    // the stage's chunk 0 in f0, the first half reads chunk 1 into f1 while
    // chunk 0 is multiplied. Then `sync` waits for the next step's loads
    // (the later steps' stay in flight) and barriers: every wave's loads of
    // the next stage have landed and every wave has read all of stage S.
    // The second half starts the loads STAGES steps ahead into stage S and
    // reads the next stage's chunk 0 into f0 while chunk 1 is multiplied.
    // No LDS read is waited for with the matrix cores idle.
    // Column sums of the right operand (COLSUM; the workgroups of the first
    // tile row only): a stage holds B as [k][column], BN columns a k row;
    // thread t sums column t % BN over k rows (t / BN) x KPART .. + KPART - 1
    // of every stage, in k order, while the stage's MFMAs run.
    constexpr int PARTS = T::THREADS / T::BN;
    constexpr int KPART = T::BK / PARTS;
    static_assert(!COLSUM || (T::THREADS % T::BN == 0 && T::BK % PARTS == 0), "whole column parts");
    const bool colsum_tile = COLSUM && tm == 0;  // uniform over the workgroup
    float colsum = 0.f;
    auto first_half = [&](auto stage) {
        constexpr int S = decltype(stage)::value;
        __builtin_amdgcn_sched_barrier(0);
        read_chunk<T, A_K, B_K>(oa, ob, stage_a[S], stage_b[S], 1, f1, lane, wave_m, wave_n);
        multiply_chunk<T, FEED>(f0, acc);
        interleave<T, FEED, 0, DS>();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (COLSUM) {
            if (colsum_tile) {
                const float* column = reinterpret_cast<const float*>(stage_b[S]) + (tid / T::BN) * KPART * T::BN +
                                      tid % T::BN;
#pragma unroll
                for (int kk = 0; kk < KPART; ++kk) colsum = colsum + column[kk * T::BN];
            }
        }
    };
    auto sync = [&] {
        wait_loads<LOADS_PER_STEP * (STAGES - 2)>();
        lds_barrier();
    };
    auto second_half = [&](auto stage, int64_t k0) {
        constexpr int S = decltype(stage)::value;
        constexpr int N = (S + 1) % STAGES;
        mask_if_needed(stage_a[N], k0 + T::BK);
        __builtin_amdgcn_sched_barrier(0);
        issue(stage_a[S], stage_b[S], k0 + STAGES * T::BK);
        read_chunk<T, A_K, B_K>(oa, ob, stage_a[N], stage_b[N], 0, f0, lane, wave_m, wave_n);
        multiply_chunk<T, FEED>(f1, acc);
        interleave<T, FEED, LOADS_PER_STEP, DS>();
        __builtin_amdgcn_sched_barrier(0);
    };

    const int steps = k_end > k_begin ? int((k_end - k_begin + T::BK - 1) / T::BK) : 0;
    if (steps > 0) {
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I3 = std::integral_constant<int, 3>;
        // Every stage starts loading; step 0's chunk 0 is read and its
        // first half run. The loop then runs from barrier to barrier (second
        // half of step s, first half of step s + 1), so that the loads in
        // flight where it closes are the same on every iteration (none with
        // two stages): the compiler then tracks which stage each LDS read
        // may depend on instead of waiting for every load.
#pragma unroll
        for (int s = 0; s < STAGES; ++s) issue(stage_a[s], stage_b[s], k_begin + s * T::BK);
        wait_loads<LOADS_PER_STEP * (STAGES - 1)>();
        lds_barrier();
        mask_if_needed(stage_a[0], k_begin);
        read_chunk<T, A_K, B_K>(oa, ob, stage_a[0], stage_b[0], 0, f0, lane, wave_m, wave_n);
        first_half(I0{});
        sync();
        // Steps 0 .. steps - 2 close here in whole rounds of STAGES, then
        // the rest; the last step's second half ends the tile.
        int step = 0;
        for (; step + STAGES < steps; step += STAGES) {
            const int64_t k0 = k_begin + int64_t(step) * T::BK;
            second_half(I0{}, k0);
            first_half(I1{});
            sync();
            if constexpr (STAGES == 2) {
                second_half(I1{}, k0 + T::BK);
                first_half(I0{});
                sync();
            } else {
                second_half(I1{}, k0 + T::BK);
                first_half(I2{});
                sync();
                if constexpr (STAGES == 3) {
                    second_half(I2{}, k0 + 2 * T::BK);
                    first_half(I0{});
                    sync();
                } else {
                    second_half(I2{}, k0 + 2 * T::BK);
                    first_half(I3{});
                    sync();
                    second_half(I3{}, k0 + 3 * T::BK);
                    first_half(I0{});
                    sync();
                }
            }
        }
        // 0 .. STAGES - 1 more steps close, starting at stage 0; then the
        // last step, on stage `left`.
        const int left = steps - 1 - step;
        const int64_t k0 = k_begin + int64_t(step) * T::BK;
        if (left > 0) {
            second_half(I0{}, k0);
            first_half(std::integral_constant<int, 1 % STAGES>{});
            sync();
        }
        if constexpr (STAGES > 2)
            if (left > 1) {
                second_half(I1{}, k0 + T::BK);
                first_half(std::integral_constant<int, 2 % STAGES>{});
                sync();
            }
        if constexpr (STAGES > 3)
            if (left > 2) {
                second_half(I2{}, k0 + 2 * T::BK);
                first_half(std::integral_constant<int, 3 % STAGES>{});
                sync();
            }
        const int64_t k_last = k0 + int64_t(left) * T::BK;
        if (left == 0) second_half(I0{}, k_last);
        if constexpr (STAGES > 1)
            if (left == 1) second_half(std::integral_constant<int, 1 % STAGES>{}, k_last);
        if constexpr (STAGES > 2)
            if (left == 2) second_half(std::integral_constant<int, 2 % STAGES>{}, k_last);
        if constexpr (STAGES > 3)
            if (left == 3) second_half(std::integral_constant<int, 3 % STAGES>{}, k_last);
        // The loads issued past the last step are still writing (zeros)
        // into LDS: let them land before the workgroup can end.
        wait_loads<0>();
    }

    const bool partial = args.splits > 1;
    if constexpr (COLSUM) {
        if (colsum_tile) {
            // The column parts meet in LDS and are added in part order; the
            // sum over this slice of K is added to the sums (one slice) or
            // left for the reduce after the product's partial sums (several).
            lds_barrier();  // every wave is done with the stages
            float* parts = reinterpret_cast<float*>(stage_a[0]);
            parts[tid] = colsum;  // part tid / BN, column tid % BN
            lds_barrier();
            if (tid < T::BN) {
                float total = parts[tid];
#pragma unroll
                for (int q = 1; q < PARTS; ++q) total = total + parts[q * T::BN + tid];
                const int64_t c = n0 + tid;
                if (c < args.n) {
                    if (partial)
                        args.ws[int64_t(args.splits) * args.m * args.n + int64_t(split) * args.n + c] = total;
                    else
                        args.column_sums[c] = args.column_sums[c] + total;
                }
            }
        }
    }
    float* out = partial ? args.ws + ((batch_local * int64_t(args.splits) + split) * args.m) * args.n : c_batch;
    constexpr bool PM = paired<T, A_K, true>(), PN = paired<T, B_K, false>();
    if (args.streaming_output)
        write_tile<T, true, PM, PN, kStreaming>(args, acc, out, m0, n0, wave_m, wave_n, lane, partial);
    else
        write_tile<T, true, PM, PN>(args, acc, out, m0, n0, wave_m, wave_n, lane, partial);
}

// The fp32 tile schedule of dma_tile (two LDS stages, one barrier per K-step
// between its chunks) as a persistent loop: each workgroup takes work items
// blockIdx.x, blockIdx.x + gridDim.x, ... (a work item is a matrix, K slice
// and tile, mapped by tile_coordinates as the one-tile kernels map their
// workgroups) for unmasked products whose every tile has an even number of
// K-steps. The two loads a tile would issue past its last K-step (zeros, in
// dma_tile) fetch the next item's first two K-steps instead, so when a tile's
// last MFMAs are issued the next one's first stage is in LDS and its second
// in flight. Its output stores then go out behind those loads, and the next
// tile's first barrier waits for the loads only: load and store completions
// are counted in issue order (vmcnt), so waiting until at most as many
// operations are outstanding as the epilogue issued means every load before
// it has landed. The stores then drain under the next tile's first K-step,
// where the one-tile kernel ended the workgroup and started the next one's
// loads only after them.
template <class T, bool A_K, bool B_K>
__device__ __forceinline__ void dma_persistent(const Args& args) {
    constexpr int FEED = kFeedF32;
    constexpr int WAVES = T::THREADS / 64;
    constexpr int A_SLOTS = T::BM * T::BK / 4;
    constexpr int B_SLOTS = T::BN * T::BK / 4;
    __shared__ f32x4 a0[A_SLOTS], b0[B_SLOTS], a1[A_SLOTS], b1[B_SLOTS];
    f32x4* const stage_a[2] = {a0, a1};
    f32x4* const stage_b[2] = {b0, b1};

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_m = wave / T::WAVES_N;
    const int wave_n = wave % T::WAVES_N;
    const int items = args.persistent_items;
    const int stride = int(gridDim.x);

    // A work item's tile row and column, matrix and K slice.
    struct Item {
        int tm, tn, batch_local, split;
    };
    auto item_of = [&](int w) {
        Item it;
        tile_coordinates(w, items, args.tiles_m, args.tiles_n, args.splits, it.batch_local, it.split, it.tm, it.tn);
        return it;
    };
    auto k_begin_of = [&](const Item& it) { return int64_t(it.split) * args.k_per_split; };
    auto k_end_of = [&](const Item& it) { return min(args.k, k_begin_of(it) + args.k_per_split); };
    auto a_of = [&](const Item& it) {
        const int64_t m0 = int64_t(it.tm) * T::BM;
        return args.a + (args.batch_base + it.batch_local) * args.stride_a + (A_K ? m0 * args.lda : m0);
    };
    auto b_of = [&](const Item& it) {
        const int64_t n0 = int64_t(it.tn) * T::BN;
        return args.b + (args.batch_base + it.batch_local) * args.stride_b + (B_K ? n0 * args.ldb : n0);
    };

    int w = int(blockIdx.x);
    if (w >= items) return;
    Item cur = item_of(w);
    // The item whose loads are being issued: tile origins and K end.
    const float* ld_a = a_of(cur);
    const float* ld_b = b_of(cur);
    int64_t ld_end = k_end_of(cur);
    OperandFor<A_K, T::BM, WAVES> oa;
    OperandFor<B_K, T::BN, WAVES> ob;
    // Every tile is interior (checked on the host), so the row bounds of the
    // loaders' offsets are the same for every item.
    oa.init(args.lda, 0, T::BM, lane, wave);
    ob.init(args.ldb, 0, T::BN, lane, wave);
    auto issue = [&](const f32x4* sa, const f32x4* sb, int64_t k0) {
        if constexpr (A_K) oa.issue(sa, ld_a, k0, ld_end, wave);
        else oa.issue(sa, ld_a, args.lda, k0, ld_end, wave);
        if constexpr (B_K) ob.issue(sb, ld_b, k0, ld_end, wave);
        else ob.issue(sb, ld_b, args.ldb, k0, ld_end, wave);
    };

    constexpr int LOADS_PER_STEP = (T::BM + T::BN) / (8 * WAVES);
    constexpr int DS = (A_K ? 2 * T::FM : paired<T, A_K, true>() ? 4 : 4 * T::FM) +
                       (B_K ? 2 * T::FN : paired<T, B_K, false>() ? 4 : 4 * T::FN);
    constexpr bool PM = paired<T, A_K, true>(), PN = paired<T, B_K, false>();
    // Store instructions of write_tile's interior path, capped at what the
    // 6-bit count can hold (then at least the loads before them are done).
    constexpr int STORES = (PN ? 1 : T::FN) * T::FM * 16;
    constexpr int AFTER_STORES = STORES < 63 ? STORES : 63;
    Chunk<T> f0, f1;
    f32x16 acc[T::FM][T::FN];
    auto first_half = [&](auto stage) {
        constexpr int S = decltype(stage)::value;
        __builtin_amdgcn_sched_barrier(0);
        read_chunk<T, A_K, B_K>(oa, ob, stage_a[S], stage_b[S], 1, f1, lane, wave_m, wave_n);
        multiply_chunk<T, FEED>(f0, acc);
        interleave<T, FEED, 0, DS>();
        __builtin_amdgcn_sched_barrier(0);
    };
    auto sync = [&] {
        wait_loads<0>();
        lds_barrier();
    };
    // READ_NEXT: also read the next stage's chunk 0 (not for a tile's last
    // half: the next tile's first fragments are read after the epilogue, so
    // that they are not held in registers across it).
    auto second_half = [&](auto stage, int64_t k_load, auto read_next) {
        constexpr int S = decltype(stage)::value;
        constexpr int N = (S + 1) % 2;
        constexpr bool READ_NEXT = decltype(read_next)::value;
        __builtin_amdgcn_sched_barrier(0);
        issue(stage_a[S], stage_b[S], k_load);
        if constexpr (READ_NEXT) read_chunk<T, A_K, B_K>(oa, ob, stage_a[N], stage_b[N], 0, f0, lane, wave_m, wave_n);
        multiply_chunk<T, FEED>(f1, acc);
        interleave<T, FEED, LOADS_PER_STEP, READ_NEXT ? DS : DS / 2>();
        __builtin_amdgcn_sched_barrier(0);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using Read = std::true_type;
    using NoRead = std::false_type;

    {
        const int64_t k_begin = k_begin_of(cur);
        issue(a0, b0, k_begin);
        issue(a1, b1, k_begin + T::BK);
    }
    wait_loads<LOADS_PER_STEP>();
    lds_barrier();
    bool first = true;
    for (;;) {
        read_chunk<T, A_K, B_K>(oa, ob, a0, b0, 0, f0, lane, wave_m, wave_n);
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
#pragma unroll
            for (int j = 0; j < T::FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
        // Step 0's first half; then its second stage is waited for (issued
        // before the previous tile's stores, which may stay in flight).
        first_half(I0{});
        if (first) wait_loads<0>();
        else wait_loads<AFTER_STORES>();
        lds_barrier();
        const int64_t k_begin = k_begin_of(cur);
        const int steps = int((k_end_of(cur) - k_begin + T::BK - 1) / T::BK);
        int s = 0;
        for (; s + 2 < steps; s += 2) {
            const int64_t k0 = k_begin + int64_t(s) * T::BK;
            second_half(I0{}, k0 + 2 * T::BK, Read{});
            first_half(I1{});
            sync();
            second_half(I1{}, k0 + 3 * T::BK, Read{});
            first_half(I0{});
            sync();
        }
        // The tile's last two K-steps load the next item's first two (or,
        // for the workgroup's last item, nothing: offsets past the K end).
        const bool has_next = w + stride < items;
        int64_t k_next = ld_end;
        if (has_next) {
            const Item next = item_of(w + stride);
            ld_a = a_of(next);
            ld_b = b_of(next);
            ld_end = k_end_of(next);
            k_next = k_begin_of(next);
        }
        second_half(I0{}, k_next, Read{});
        first_half(I1{});
        sync();
        second_half(I1{}, has_next ? k_next + T::BK : k_next, NoRead{});

        const bool partial = args.splits > 1;
        float* out = partial ? args.ws + ((cur.batch_local * int64_t(args.splits) + cur.split) * args.m) * args.n
                             : args.c + (args.batch_base + cur.batch_local) * args.stride_c;
        write_tile<T, true, PM, PN, 0, true>(args, acc, out, int64_t(cur.tm) * T::BM, int64_t(cur.tn) * T::BN, wave_m,
                                            wave_n, lane, partial);
        if (!has_next) break;
        w += stride;
        cur = item_of(w);
        first = false;
    }
    wait_loads<0>();
}

// A tile shape with its number of LDS stages.
template <class T_, int STAGES_>
struct DmaConfig {
    using T = T_;
    static constexpr int STAGES = STAGES_;
};

// LDS (the stages) caps a CU's workgroups; registers are held to the same
// number of waves per SIMD (dma_waves_per_eu: two for the 128 x 128 tile,
// 256 registers a lane; three for 128 x 64; four for 64 x 64), so that the
// register file never lowers it further.
template <class C, bool A_K, bool B_K>
__global__ __launch_bounds__(C::T::THREADS)
__attribute__((amdgpu_waves_per_eu(dma_waves_per_eu<typename C::T, C::STAGES>(),
                                   dma_waves_per_eu<typename C::T, C::STAGES>())))
void gemm_f32_dma_kernel(Args args) {
    dma_tile<typename C::T, C::STAGES, A_K, B_K, kFeedF32>(args);
}

// The persistent form of the 128 x 128 fp32 tile (dma_persistent).
template <class C, bool A_K, bool B_K>
__global__ __launch_bounds__(C::T::THREADS)
__attribute__((amdgpu_waves_per_eu(dma_waves_per_eu<typename C::T, C::STAGES>(),
                                   dma_waves_per_eu<typename C::T, C::STAGES>())))
void gemm_f32_persistent_kernel(Args args) {
    dma_persistent<typename C::T, A_K, B_K>(args);
}

// The fp32 product with the right operand's column sums over K (Linear's
// weight and bias gradients in one pass).
template <class C, bool A_K>
__global__ __launch_bounds__(C::T::THREADS)
__attribute__((amdgpu_waves_per_eu(dma_waves_per_eu<typename C::T, C::STAGES>(),
                                   dma_waves_per_eu<typename C::T, C::STAGES>())))
void gemm_f32_dma_colsum_kernel(Args args) {
    dma_tile<typename C::T, C::STAGES, A_K, false, kFeedF32, true>(args);
}

// bf16-input / fp32-accumulate variant (SN_PRECISION_BF16): the same loads,
// LDS stages, schedule and epilogue; each lane rounds its fp32 fragments to
// bf16 just before the matrix instruction.
template <class C, bool A_K, bool B_K>
__global__ __launch_bounds__(C::T::THREADS)
__attribute__((amdgpu_waves_per_eu(dma_waves_per_eu<typename C::T, C::STAGES>(),
                                   dma_waves_per_eu<typename C::T, C::STAGES>())))
void gemm_bf16_dma_kernel(Args args) {
    dma_tile<typename C::T, C::STAGES, A_K, B_K, kFeedRound>(args);
}

// bf16 operands staged ahead of the product (both K-contiguous, k counted in
// pairs of bf16): the same loads, stages, schedule and epilogue, half the
// LDS bytes per FLOP.
template <class C>
__global__ __launch_bounds__(C::T::THREADS)
__attribute__((amdgpu_waves_per_eu(dma_waves_per_eu<typename C::T, C::STAGES>(),
                                   dma_waves_per_eu<typename C::T, C::STAGES>())))
void gemm_bf16_staged_kernel(Args args) {
    dma_tile<typename C::T, C::STAGES, true, true, kFeedBf16>(args);
}

// The split-K model's view of an instantiation: workgroups per CU from its
// LDS stages, and the rate one CU sustains on it (measured: fp32 at about
// 85 % of the matrix-core peak; bf16 from fp32 stages about 20 %, from bf16
// stages about 30 % of 2.5 PFLOP/s over 256 CUs).
template <class C, int FEED>
SplitCost split_cost() {
    using T = typename C::T;
    SplitCost cost;
    cost.workgroups_per_cu = std::max(1, dma_waves_per_eu<T, C::STAGES>() * 4 / (T::THREADS / 64));
    cost.flops_per_cu = FEED == kFeedF32 ? 522e9 : FEED == kFeedRound ? 1.95e12 : 2.9e12;
    cost.k_per_index = FEED == kFeedBf16 ? 2 : 1;
    return cost;
}

template <class C, int FEED>
Plan dma_plan(const Problem& p, const Env& env) {
    return plan_for<typename C::T>(p, env, split_cost<C, FEED>());
}

constexpr int64_t kStreamingMaxK = 128;

// The grid of the persistent fp32 kernel for `p` (a multiple of the XCD
// count, so that a workgroup's items stay on its XCD), or 0 when the product
// takes the one-tile kernel: masked products, several launches, tiles with an
// odd number of K-steps, or under two items per workgroup slot.
template <class C>
int64_t persistent_grid(const Problem& p, const Env& env, const Plan& plan, const LaunchShape& shape) {
    using T = typename C::T;
    if constexpr (C::STAGES != 2 || T::BM != 128 || T::BN != 128) return 0;
    // Interior tiles that read nothing back: write_tile's one store path.
    if (p.mask != SN_MASK_NONE || shape.batches_per_launch < p.batch || p.k <= kStreamingMaxK ||
        p.m % T::BM != 0 || p.n % T::BN != 0 || (plan.splits == 1 && p.accumulate))
        return 0;
    const int64_t items = int64_t(plan.tiles_m) * plan.tiles_n * plan.splits * p.batch;
    const int64_t per_cu = std::max(1, dma_waves_per_eu<T, C::STAGES>() * 4 / (T::THREADS / 64));
    const int64_t slots = int64_t(std::max(env.cu_count, 1)) * per_cu / kXcds * kXcds;
    if (slots < kXcds || items < 2 * slots || items > 0x7FFFFFFF) return 0;
    const int64_t steps = (plan.k_per_split + T::BK - 1) / T::BK;
    const int64_t last_steps = (p.k - int64_t(plan.splits - 1) * plan.k_per_split + T::BK - 1) / T::BK;
    if (steps % 2 != 0 || last_steps % 2 != 0 || last_steps < 2) return 0;
    return slots;
}

template <class C, bool A_K, bool B_K, int FEED>
hipError_t launch_dma_tiles(const Problem& p, const Env& env, hipStream_t stream) {
    using T = typename C::T;
    const Plan plan = dma_plan<C, FEED>(p, env);
    const LaunchShape shape = tiled_shape<T>(p, plan, SN_PATH_NONE);
    if (shape.batches_per_launch < 1) return hipErrorInvalidConfiguration;
    Args args = make_args<T>(p, env, plan);
    // Unsplit products with at most 128 inner elements write as many output
    // bytes as they read: their outputs, and the zero tiles of a causal
    // output mask, stream out. Measured on config 3's attention scores and
    // dP products (192 x 2048 x 2048 x 64), dense: 1.38-1.44 -> 1.25 ms and
    // 1.31-1.32 -> 1.17-1.19 ms; causal: 0.91 -> 0.81 ms and 0.88 -> 0.76 ms.
    // At K = 768 (the Linear products) streaming stores changed nothing
    // beyond noise.
    args.streaming_output = (p.mask == SN_MASK_NONE || p.mask == SN_MASK_CAUSAL_OUTPUT) && plan.splits == 1 &&
                                    p.k <= kStreamingMaxK
                                ? 1
                                : 0;
    if constexpr (FEED == kFeedF32 && C::STAGES == 2 && T::BM == 128 && T::BN == 128) {
        const int64_t grid = persistent_grid<C>(p, env, plan, shape);  // describe_f32_dma's choice
        if (grid > 0) {
            args.persistent_items = int32_t(int64_t(plan.tiles_m) * plan.tiles_n * plan.splits * p.batch);
            hipLaunchKernelGGL((gemm_f32_persistent_kernel<C, A_K, B_K>), dim3(unsigned(grid)), dim3(T::THREADS), 0,
                               stream, args);
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
        if constexpr (FEED == kFeedBf16)
            hipLaunchKernelGGL((gemm_bf16_staged_kernel<C>), dim3(unsigned(count * per_batch)), dim3(T::THREADS), 0,
                               stream, args);
        else if constexpr (FEED == kFeedRound)
            hipLaunchKernelGGL((gemm_bf16_dma_kernel<C, A_K, B_K>), dim3(unsigned(count * per_batch)),
                               dim3(T::THREADS), 0, stream, args);
        else
            hipLaunchKernelGGL((gemm_f32_dma_kernel<C, A_K, B_K>), dim3(unsigned(count * per_batch)),
                               dim3(T::THREADS), 0, stream, args);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (plan.splits > 1) return launch_splitk_reduce(p, env, plan.splits, stream);
    return hipSuccess;
}

template <class C, int FEED>
hipError_t launch_dma_layout(const Problem& p, const Env& env, hipStream_t stream) {
    if (p.a_k_contiguous && p.b_k_contiguous) return launch_dma_tiles<C, true, true, FEED>(p, env, stream);
    if (p.a_k_contiguous) return launch_dma_tiles<C, true, false, FEED>(p, env, stream);
    if (p.b_k_contiguous) return launch_dma_tiles<C, false, true, FEED>(p, env, stream);
    return launch_dma_tiles<C, false, false, FEED>(p, env, stream);
}

using DmaSquare = DmaConfig<Tile<128, 128, 32, 2, 2>, 2>;
using DmaNarrow = DmaConfig<Tile<128, 64, 32, 4, 1>, 2>;

// bf16 tiles. With fp32 operands in HBM the bf16 products are bound by the
// operand bytes each CU pulls from L2 per FLOP, so wide outputs take a
// 128x256 tile (8 waves of 64x64, three 48 KB stages, one workgroup per
// CU: 43 FLOP per loaded byte instead of 32). Outputs narrower than 2048
// columns have too few such tiles to fill the CUs and keep 128x128.
// Measured on the 111.5M set: 128x256 is 7-23 % faster at N >= 2304 and
// up to 40 % slower at N = 768.
using Bf16Square = DmaConfig<Tile<128, 128, 32, 2, 2>, 2>;
using Bf16Wide = DmaConfig<Tile<128, 256, 32, 2, 4>, 3>;
using Bf16Narrow = DmaNarrow;
constexpr int64_t kBf16WideColumns = 2048;

template <class C>
bool config_applies(const Problem& p) {
    return buffers_ok<typename C::T>(p);
}

// The tile configuration each direct-to-LDS family takes for `p`, handed
// to `f` (the launchers, applicability checks and launch shapes all choose
// through these).
// Products whose 128x128 plan (split K included) has fewer workgroups than
// the device has CUs take 64x64 tiles (four waves of 32x32, five workgroups
// per CU by LDS): the 7.1M model's products and the reference's published shapes
// (2048 x 768 x 256: 96 tiles of 128 x 128 on 256 CUs). Measured: the 7.1M model's
// set 43.6 -> 56.1 TFLOP/s, 2048 x 768 x 256 34 -> 54, 2048 x 1024 x 256
// 45 -> 68; the 42.9M and 111.5M models, whose plans fill the CUs, keep 128 x 128 (a
// 128 x 64 tile below 256 tiles lost 6 % on the 111.5M model's 768 x 768 weight
// gradient).
using DmaSmall = DmaConfig<Tile<64, 64, 32, 2, 2>, 2>;

// Products whose 128x128 plan leaves CU slots empty (under two workgroups
// per CU) with under 24 K-steps per workgroup take 64x64 tiles as well: the
// 128x128 plan there splits an already short K (or runs one workgroup per
// CU), and each workgroup's start-up and epilogue weigh on a few K-steps;
// four 64x64 workgroups per CU fill the device without splitting. Measured
// (fp32, one GPU's share of config 2 over 8 GPUs, M = 4096): NN and NT
// 4096 x 768 x 768 74-76 -> 104-107 TFLOP/s, TN 768 x 768 x 4096 83 -> 89;
// the 42.9M model's NN and NT 8192 x 512 x 512 99-103 -> 102-105. Longer
// slices keep 128x128 (the 111.5M model's 768 x 768 x 32768 weight
// gradient, 74 K-steps a workgroup: 127 TFLOP/s against 119 on 64x64).
constexpr int64_t kSmallTileMaxK = 768;

template <class F>
auto with_f32_dma_config(const Problem& p, const Env& env, F&& f) {
    if (p.n <= 64) return f(DmaNarrow{});
    const Plan square = dma_plan<DmaSquare, kFeedF32>(p, env);
    const int64_t workgroups = int64_t(square.tiles_m) * square.tiles_n * square.splits * p.batch;
    const int64_t cus = std::max(env.cu_count, 1);
    const bool short_slices = workgroups < 2 * cus && square.k_per_split < kSmallTileMaxK;
    return workgroups < cus || short_slices ? f(DmaSmall{}) : f(DmaSquare{});
}

// Small bf16 products (fewer 128 x 128 tiles than CUs: the 7.1M model's) skip
// the staging pass, whose two extra launches they cannot amortise, and take
// 64 x 64 tiles that round fp32 fragments as they are read: the 7.1M model's bf16
// set 60 -> 80 TFLOP/s, 2048 x 768 x 256 54 -> 74, 2048 x 1024 x 256 74 -> 108.
bool small_bf16(const Problem& p, const Env& env) {
    return ((p.m + 127) / 128) * ((p.n + 127) / 128) * p.batch < std::max(env.cu_count, 1);
}

template <class F>
auto with_bf16_dma_config(const Problem& p, const Env& env, F&& f) {
    if (p.n <= 64) return f(Bf16Narrow{});
    if (small_bf16(p, env)) return f(DmaSmall{});
    if (p.n >= kBf16WideColumns) return f(Bf16Wide{});
    return f(Bf16Square{});
}

}  // namespace

// Operands 16-byte aligned with 16-byte-multiple leading dimensions and
// batch strides, and every per-lane offset of one K-step within the buffer
// offset range (the same conditions as the buffer-load path of gemm_mfma.hip).
bool dma_applies(const Problem& p, const Env& env) {
    return with_f32_dma_config(p, env, [&](auto c) { return config_applies<decltype(c)>(p); });
}

bool bf16_dma_applies(const Problem& p, const Env& env) {
    return with_bf16_dma_config(p, env, [&](auto c) { return config_applies<decltype(c)>(p); });
}

LaunchShape describe_f32_dma(const Problem& p, const Env& env) {
    return with_f32_dma_config(p, env, [&](auto c) {
        using C = decltype(c);
        const Plan plan = dma_plan<C, kFeedF32>(p, env);
        LaunchShape s = tiled_shape<typename C::T>(p, plan, SN_PATH_F32_DIRECT);
        s.persistent_grid = persistent_grid<C>(p, env, plan, s);
        if (s.persistent_grid > 0) s.path = SN_PATH_F32_PERSISTENT;
        return s;
    });
}

LaunchShape describe_bf16_dma(const Problem& p, const Env& env) {
    return with_bf16_dma_config(p, env, [&](auto c) {
        using C = decltype(c);
        return tiled_shape<typename C::T>(p, dma_plan<C, kFeedRound>(p, env), SN_PATH_BF16_DIRECT);
    });
}

hipError_t launch_gemm_f32_dma(const Problem& p, const Env& env, hipStream_t stream) {
    return with_f32_dma_config(p, env, [&](auto c) { return launch_dma_layout<decltype(c), kFeedF32>(p, env, stream); });
}

hipError_t launch_gemm_bf16_dma(const Problem& p, const Env& env, hipStream_t stream) {
    return with_bf16_dma_config(p, env, [&](auto c) { return launch_dma_layout<decltype(c), kFeedRound>(p, env, stream); });
}

// ---- The weight-gradient product with Linear's bias gradient -------------

namespace {

// Each K slice also leaves N partial column sums after the product's M x N
// partials: the split count is chosen as if the workspace were M / (M + 1)
// of its size, so that both fit.
template <class C>
Plan column_sums_plan(const Problem& p, const Env& env) {
    Env e = env;
    e.workspace_bytes = env.workspace_bytes / size_t(p.m + 1) * size_t(p.m);
    return dma_plan<C, kFeedF32>(p, e);
}

template <class C, bool A_K>
hipError_t launch_column_sums_tiles(const Problem& p, const Env& env, hipStream_t stream) {
    using T = typename C::T;
    const Plan plan = column_sums_plan<C>(p, env);
    const Args args = make_args<T>(p, env, plan);
    const int64_t workgroups = int64_t(plan.tiles_m) * plan.tiles_n * plan.splits;
    hipLaunchKernelGGL((gemm_f32_dma_colsum_kernel<C, A_K>), dim3(unsigned(workgroups)), dim3(T::THREADS), 0, stream,
                       args);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || plan.splits == 1) return err;
    err = launch_splitk_reduce(p, env, plan.splits, stream);
    if (err != hipSuccess) return err;
    return launch_column_sums_finish(env.workspace + int64_t(plan.splits) * p.m * p.n, plan.splits, p.n,
                                     p.column_sums, stream);
}

}  // namespace

bool f32_column_sums_applies(const Problem& p, const Env& env) {
    return p.batch == 1 && p.m > 0 && p.k > 0 && p.mask == SN_MASK_NONE && !p.b_k_contiguous && p.bias == nullptr &&
           dma_applies(p, env);
}

LaunchShape describe_f32_column_sums(const Problem& p, const Env& env) {
    return with_f32_dma_config(p, env, [&](auto c) {
        using C = decltype(c);
        const Plan plan = column_sums_plan<C>(p, env);
        LaunchShape s = tiled_shape<typename C::T>(p, plan, SN_PATH_F32_DIRECT);
        if (plan.splits > 1) s.workspace_bytes += size_t(plan.splits) * size_t(p.n) * sizeof(float);
        return s;
    });
}

hipError_t launch_gemm_f32_column_sums(const Problem& p, const Env& env, hipStream_t stream) {
    return with_f32_dma_config(p, env, [&](auto c) {
        using C = decltype(c);
        return p.a_k_contiguous ? launch_column_sums_tiles<C, true>(p, env, stream)
                                : launch_column_sums_tiles<C, false>(p, env, stream);
    });
}

// ---- bf16 operands staged in the workspace -------------------------------

namespace {

// Where the staged operands go: A as [batch][m][kp] bf16 and B as
// [batch][n][kp], each from the workspace's start in 256-byte units; the
// product's split-K partial sums follow them.
struct Staging {
    int64_t kp = 0;          // K rounded up to 8 bf16 (one 16-byte slot)
    int64_t batches_a = 1;   // 1 when A is shared by every batch (stride 0)
    int64_t batches_b = 1;
    size_t a_bytes = 0, b_bytes = 0;
};

size_t round256(size_t bytes) { return (bytes + 255) / 256 * 256; }

Staging staging_for(const Problem& p) {
    Staging st;
    st.kp = (p.k + 7) / 8 * 8;
    st.batches_a = p.stride_a == 0 ? 1 : p.batch;
    st.batches_b = p.stride_b == 0 ? 1 : p.batch;
    st.a_bytes = round256(size_t(st.batches_a) * size_t(p.m) * size_t(st.kp) * 2);
    st.b_bytes = round256(size_t(st.batches_b) * size_t(p.n) * size_t(st.kp) * 2);
    return st;
}

// The product on the staged operands, k counted in pairs of bf16.
Problem staged_problem(const Problem& p, const Staging& st, const Env& env) {
    Problem q = p;
    const char* base = reinterpret_cast<const char*>(env.workspace);
    q.a = reinterpret_cast<const float*>(base);
    q.b = reinterpret_cast<const float*>(base + st.a_bytes);
    q.k = st.kp / 2;
    q.a_k_contiguous = true;
    q.b_k_contiguous = true;
    q.lda = st.kp / 2;
    q.ldb = st.kp / 2;
    q.stride_a = st.batches_a == 1 ? 0 : p.m * st.kp / 2;
    q.stride_b = st.batches_b == 1 ? 0 : p.n * st.kp / 2;
    return q;
}

// The workspace left for split-K partials after the staged operands.
Env staged_env(const Env& env, const Staging& st) {
    Env e = env;
    const size_t used = st.a_bytes + st.b_bytes;
    e.workspace = reinterpret_cast<float*>(reinterpret_cast<char*>(env.workspace) + used);
    e.workspace_bytes = env.workspace_bytes - used;
    return e;
}

using Bf16StagedSquare = DmaConfig<Tile<128, 128, 32, 2, 2>, 2>;
using Bf16StagedWide = DmaConfig<Tile<128, 256, 32, 2, 4>, 3>;

template <class F>
auto with_staged_config(const Problem& q, F&& f) {
    if (q.n >= kBf16WideColumns) return f(Bf16StagedWide{});
    return f(Bf16StagedSquare{});
}

}  // namespace

bool bf16_staged_applies(const Problem& p, const Env& env) {
    // Unmasked (the masked products keep their in-stage masking), operands
    // that the direct-to-LDS loads could read, n above the narrow tile, and
    // room for both staged operands.
    if (p.mask != SN_MASK_NONE || p.n <= 64 || p.k < 1 || env.workspace == nullptr || !bf16_dma_applies(p, env) ||
        small_bf16(p, env))
        return false;
    if (p.batch > 65535) return false;
    const Staging st = staging_for(p);
    if (st.a_bytes + st.b_bytes > env.workspace_bytes) return false;
    const Problem q = staged_problem(p, st, env);
    return with_staged_config(q, [&](auto c) { return config_applies<decltype(c)>(q) ? hipSuccess : hipErrorNotSupported; }) ==
           hipSuccess;
}

hipError_t launch_gemm_bf16_staged(const Problem& p, const Env& env, hipStream_t stream) {
    const Staging st = staging_for(p);
    const Problem q = staged_problem(p, st, env);
    uint16_t* a16 = reinterpret_cast<uint16_t*>(const_cast<float*>(q.a));
    uint16_t* b16 = reinterpret_cast<uint16_t*>(const_cast<float*>(q.b));
    hipError_t err = launch_stage_bf16(p.a, p.a_k_contiguous, p.lda, p.m, p.k, st.kp, st.batches_a, p.stride_a, a16,
                                       stream);
    if (err == hipSuccess)
        err = launch_stage_bf16(p.b, p.b_k_contiguous, p.ldb, p.n, p.k, st.kp, st.batches_b, p.stride_b, b16, stream);
    if (err != hipSuccess) return err;
    const Env rest = staged_env(env, st);
    return with_staged_config(q, [&](auto c) { return launch_dma_tiles<decltype(c), true, true, kFeedBf16>(q, rest, stream); });
}

LaunchShape describe_bf16_staged(const Problem& p, const Env& env) {
    const Staging st = staging_for(p);
    const Problem q = staged_problem(p, st, env);
    const Env rest = staged_env(env, st);
    LaunchShape shape = with_staged_config(q, [&](auto c) {
        using C = decltype(c);
        return tiled_shape<typename C::T>(q, dma_plan<C, kFeedBf16>(q, rest), SN_PATH_BF16_STAGED);
    });
    // The staged product counts k in pairs of bf16; its partial sums follow
    // the staged operands in the workspace.
    shape.k_per_split *= 2;
    shape.workspace_bytes += st.a_bytes + st.b_bytes;
    return shape;
}

}  // namespace gemm
}  // namespace sn

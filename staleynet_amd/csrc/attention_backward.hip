// Causal attention backward that recomputes the probabilities instead of
// reading them. The reference's backward (layers/attention.rs:220-267) reads
// the [queries, keys] probabilities P the forward kept and materialises dP
// and dS of the same size (3.2 GB each at config 3); here neither P nor dS
// exists in memory. From Q, K, V, dO, the forward's output O and its per-query
// softmax statistics (m, the maximum of the scaled visible scores, and l, the
// sum of e^(x - m); sn_causal_attention with stats), P = e^(s * scale - m) *
// (1 / l) is rebuilt where it is needed, as the forward's probability pass
// writes it, and the reference's three gradients come out:
//   dV = P^T dO                          (attention.rs:244-247)
//   dS = P * (dO V^T - D)                (the dP product and softmax_backward, :239-249)
//   dQ = scale (dS K),  dK = scale (dS^T Q)  (:250-260)
// with D per query = sum over h of dO * O (equal to softmax_backward's
// projection sum over keys of dP * P, since O = P V).
//
// Three launches, every sum taken in a fixed order (no atomics; reruns give
// the same bits):
//  * rows: per query {m, 1 / l, D} into the workspace (12 bytes);
//  * key blocks: a workgroup owns 128 keys of a head, a wave 32, with K and V
//    of its keys in LDS (head dims 32, 64) or registers (128); Q, dO and the
//    rows stream through LDS in 64-query stages, from the first query that
//    sees the block to the last. A wave computes S = Q K^T and dP = dO V^T
//    for 32 queries against its 32 keys: in the 32x32 accumulator lane l
//    holds column l % 32, its key, so P and dS are already laid out as the B
//    operands of dV^T += dO^T P and dK^T += Q^T dS (the forward's O^T +=
//    V^T P^T, transposed roles);
//  * dQ, one of two ways. Where the workspace holds them (head dims 32 and
//    64), the key kernel also writes each stage's dS to LDS and multiplies it
//    by the block's K, leaving per key block partial sums of dQ that a third
//    kernel adds up in block order: five products' MFMAs per pair in all.
//    Otherwise query blocks recompute S and dP in the layout of the forward
//    and the probability gradient (a lane owns a query): S^T = K Q^T and
//    dP^T = V dO^T against staged K and V, then dQ^T += K^T dS^T: seven
//    products' MFMAs per pair.
// Blocks wholly past a wave's causal horizon are skipped, and only those that
// cross it test each pair.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <type_traits>

#include "attention_common.h"
#include "gemm_internal.h"

namespace sn {
namespace {

using namespace attn;

constexpr int kKeyBlock = 32 * kWaves;  // keys per workgroup of the key kernel

// Waves per SIMD each kernel's registers are budgeted for. The query kernel
// takes the workgroups its LDS stages allow (the forward's rule). The key
// kernel keeps K and V of its key in registers beside the dV and dK
// accumulators (4 h / 2 floats per lane) and the 32 x 32 S and dP blocks:
// about 235 registers at h = 64, which two waves per SIMD (256 each) leave
// the compiler no room to schedule, so it takes one wave per SIMD there.
constexpr int backward_waves_per_simd(int h) { return h <= 32 ? 3 : h == 64 ? 2 : 1; }
constexpr int key_grad_waves_per_simd(int h) { return h <= 32 ? 2 : 1; }

// The row records: per head three planes of `plane` floats (queries rounded
// up to 4, so that every plane starts 16-byte aligned): m, 1 / l and D.
constexpr int64_t plane_of(int64_t queries) { return (queries + 3) / 4 * 4; }

struct RowsArgs {
    const float* d_out;
    const float* out;
    const float* stats;
    float* rows;
    int64_t queries;
    int64_t q_stride;
    int64_t total;  // heads x queries
};

// The row records of every query: 16 lanes per query, 4 of h each per pass,
// D summed per lane in h order and then over the lanes by a butterfly.
template <int H>
__global__ __launch_bounds__(256) void attention_rows_kernel(RowsArgs a) {
#pragma clang fp contract(off)
    const int64_t g = (int64_t(blockIdx.x) * 256 + threadIdx.x) / 16;
    const int li = threadIdx.x % 16;
    if (g >= a.total) return;  // whole 16-lane groups leave together
    const int64_t head = g / a.queries, q = g % a.queries;
    const float* dorow = a.d_out + head * a.q_stride + q * H;
    const float* orow = a.out + g * H;
    float d = 0.f;
#pragma unroll
    for (int c = 4 * li; c < H; c += 64) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(dorow + c);
        const f32x4 y = *reinterpret_cast<const f32x4*>(orow + c);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float product = x[s] * y[s];
            d = d + product;
        }
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) d = d + __shfl_xor(d, o);
    float* planes = a.rows + head * 3 * plane_of(a.queries) + q;
    if (li == 0) {
        planes[0] = a.stats[2 * g];
        planes[plane_of(a.queries)] = 1.f / a.stats[2 * g + 1];
        planes[2 * plane_of(a.queries)] = d;
    } else if (li < 4 && q == a.queries - 1 && q + li < plane_of(a.queries)) {
        // The last query's group also zeroes its head's padding slots (up to
        // three per plane), so the key kernels' whole 16-byte record loads
        // never bring in what the workspace held before.
        planes[li] = 0.f;
        planes[plane_of(a.queries) + li] = 0.f;
        planes[2 * plane_of(a.queries) + li] = 0.f;
    }
}

// The first query of the first stage of key block `block`: the first query
// that sees the block's first key, rounded down to a whole stage.
__host__ __device__ constexpr int64_t stage_begin(int64_t block, int64_t query_offset) {
    return (block * kKeyBlock - query_offset > 0 ? block * kKeyBlock - query_offset : 0) / kKeys * kKeys;
}

// The queries a key block's stages cover (from stage_begin to the last).
__host__ __device__ constexpr int64_t block_queries(int64_t block, int64_t queries, int64_t query_offset) {
    return stage_begin(block, query_offset) < queries ? queries - stage_begin(block, query_offset) : 0;
}

// dQ partial sums, when the key kernel computes them: per head, for each key
// block in order, one row of H floats per query its stages cover (the
// block's dS times its K rows, summed over its keys); block b's rows start
// after those of blocks 0 .. b - 1. Rows per head:
__host__ __device__ inline int64_t partial_rows(int64_t queries, int64_t keys, int64_t query_offset) {
    int64_t rows = 0;
    for (int64_t b = 0; b * kKeyBlock < keys; ++b) rows += block_queries(b, queries, query_offset);
    return rows;
}

struct KeyGradArgs {
    const float* q;
    const float* k;
    const float* v;
    const float* d_out;
    const float* rows;
    float* k_grad;
    float* v_grad;
    int64_t queries, keys;
    int64_t q_stride, kv_stride;
    int64_t query_offset;
    int64_t heads;
    float scale;
    float* partials;       // dQ partial sums (the LDS kernel's dQ form), else unused
    int64_t partial_rows;  // partial_rows() of the shape: rows per head
};

// Element (row, h = 32 b + col) of a stage whose 16-byte chunks are
// XOR-swizzled by row (slot (h / 4) ^ (row & SWIZZLE)), for the rows the
// accumulator pairing visits: row = 32 sub + 8 g + 4 half + j. Since col / 4
// and 4 half + j stay below 8, the XOR splits into a per-lane part, which
// depends on j only (lane_part(j), four registers), and a constant part, so
// every such read is one ds_read_b32 at an immediate offset from a lane base.
// Hides a value's origin from the compiler, so that addresses derived from
// it are formed where they are used (one VGPR base, immediate offsets)
// instead of being precomputed for every stage and chunk and held in
// registers across the loop.
__device__ __forceinline__ void launder(int& x) { asm volatile("" : "+v"(x)); }

// Byte offsets, from a stage's row 32 sub, of the 16-byte chunks lane (col,
// half) reads for the A operand of a 32-row product over h: chunk c, lo / hi
// = the h values 16c + 8 half + 0..3 / 4..7 of stage row col (swizzled).
template <int H>
struct ChunkReads {
    using G = Geometry<H>;
    int off[2 * G::CHUNKS];
    __device__ __forceinline__ ChunkReads(int col, int half) {
        const int swz = col & G::SWIZZLE;
#pragma unroll
        for (int c = 0; c < G::CHUNKS; ++c) {
            const int g = 4 * c + 2 * half;
            off[2 * c] = (col * G::SLOTS + (g ^ swz)) * 16;
            off[2 * c + 1] = (col * G::SLOTS + ((g + 1) ^ swz)) * 16;
        }
    }
    __device__ __forceinline__ void launder_all() {
#pragma unroll
        for (int i = 0; i < 2 * G::CHUNKS; ++i) launder(off[i]);
    }
    // 32 rows (32 sub .. of the stage) against the 32 columns held in `reg`.
    // The same, with the 32 columns' values read from LDS rows laid out as a
    // stage (`rows`: the first of the 32; row r's swizzle is r & SWIZZLE,
    // which is col & SWIZZLE for row 32 i + col, so the offsets are shared).
    __device__ __forceinline__ f32x16 product_lds(const f32x4* stage, int sub, const f32x4* rows) const {
        const char* base = reinterpret_cast<const char*>(stage) + 32 * sub * G::SLOTS * 16;
        const char* other = reinterpret_cast<const char*>(rows);
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
        for (int c = 0; c < G::CHUNKS; ++c) {
            const f32x4 lo = *reinterpret_cast<const f32x4*>(base + off[2 * c]);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(base + off[2 * c + 1]);
            const f32x4 ylo = *reinterpret_cast<const f32x4*>(other + off[2 * c]);
            const f32x4 yhi = *reinterpret_cast<const f32x4*>(other + off[2 * c + 1]);
            const float x[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            const float y[8] = {ylo[0], ylo[1], ylo[2], ylo[3], yhi[0], yhi[1], yhi[2], yhi[3]};
#pragma unroll
            for (int s = 0; s < 8; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x[s], y[s], acc, 0, 0, 0);
        }
        return acc;
    }
    __device__ __forceinline__ f32x16 product(const f32x4* stage, int sub, const float (&reg)[G::CHUNKS][8]) const {
        const char* base = reinterpret_cast<const char*>(stage) + 32 * sub * G::SLOTS * 16;
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
        for (int c = 0; c < G::CHUNKS; ++c) {
            const f32x4 lo = *reinterpret_cast<const f32x4*>(base + off[2 * c]);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(base + off[2 * c + 1]);
            const float x[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
            for (int s = 0; s < 8; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x[s], reg[c][s], acc, 0, 0, 0);
        }
        return acc;
    }
};

template <int H>
struct ColumnReads {
    using G = Geometry<H>;
    int base[4];  // floats, per j
    __device__ __forceinline__ ColumnReads(int col, int half) {
#pragma unroll
        for (int j = 0; j < 4; ++j) base[j] = 4 * half * H + 4 * ((col >> 2) ^ (4 * half + j)) + (col & 3);
    }
    // The constant part for (sub, g, j, b): row 32 sub + 8 g + j, chunk bit 3 flipped by g's
    // low bit where the swizzle reaches it (16 chunks or more per row).
    __device__ __forceinline__ void launder_all() {
#pragma unroll
        for (int j = 0; j < 4; ++j) launder(base[j]);
    }
    static constexpr int offset(int sub, int g, int j, int b) {
        return (32 * sub + 8 * g + j) * H + 32 * (G::SWIZZLE >= 15 ? (b ^ (g & 1)) : b);
    }
    __device__ __forceinline__ float read(const f32x4* stage, int sub, int g, int j, int b) const {
        return reinterpret_cast<const float*>(stage)[base[j] + offset(sub, g, j, b)];
    }
};
static_assert(Geometry<32>::SWIZZLE == 7 && Geometry<64>::SWIZZLE == 15 && Geometry<128>::SWIZZLE == 15,
              "ColumnReads assumes these swizzles");

template <int H>
__global__ __launch_bounds__(64 * kWaves)
__attribute__((amdgpu_waves_per_eu(key_grad_waves_per_simd(H), key_grad_waves_per_simd(H))))
void attention_key_grad_kernel(KeyGradArgs a) {
#pragma clang fp contract(off)
    using G = Geometry<H>;  // 64 queries per stage
    __shared__ f32x4 q_stage0[G::STAGE_SLOTS], q_stage1[G::STAGE_SLOTS];
    __shared__ f32x4 d_stage0[G::STAGE_SLOTS], d_stage1[G::STAGE_SLOTS];
    // Each wave loads its own copy of the stage's 64 row records (one load
    // instruction per wave per stage, so every wave's load count is the same):
    // 16-byte slots 0-15 hold m of the stage's queries, 16-31 their 1 / l,
    // 32-47 their D (lanes 48-63 load nothing).
    __shared__ f32x4 r_stage0[kWaves][64], r_stage1[kWaves][64];
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    auto q_of = [&](auto stage) __attribute__((always_inline)) -> f32x4* {
        if constexpr (decltype(stage)::value == 0) return q_stage0;
        else return q_stage1;
    };
    auto d_of = [&](auto stage) __attribute__((always_inline)) -> f32x4* {
        if constexpr (decltype(stage)::value == 0) return d_stage0;
        else return d_stage1;
    };
    auto r_of = [&](auto stage) __attribute__((always_inline)) -> f32x4* {
        if constexpr (decltype(stage)::value == 0) return r_stage0[0];
        else return r_stage1[0];
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31;  // this lane's key within the wave
    const int half = lane >> 5;

    // Key blocks in order: the first keys are seen by the most queries.
    const int64_t block = blockIdx.x;
    const int64_t head = block % a.heads;
    const int64_t k_first = (block / a.heads) * kKeyBlock;
    const int64_t k_wave = k_first + 32 * wave;
    const int64_t key = k_wave + col;
    const bool key_ok = key < a.keys;
    // Queries that see a key: q + query_offset >= key. Stages start at the
    // workgroup's first such query, rounded down to a stage.
    const int64_t q_seen = max(int64_t(0), k_first - a.query_offset);
    const int64_t q_begin = q_seen / kKeys * kKeys;
    const int stages_total = q_begin < a.queries ? int((a.queries - q_begin + kKeys - 1) / kKeys) : 0;

    const float* q_head = a.q + head * a.q_stride;
    const float* d_head = a.d_out + head * a.q_stride;
    const int64_t plane = plane_of(a.queries);
    const float* r_head = a.rows + head * 3 * plane;
    // Per lane, constant over the stages: the stage row each load instruction
    // fills and the byte offset of its 16 bytes from the stage's first row;
    // the records' plane piece. Each stage moves the descriptors' base.
    int32_t stage_row[G::LOADS], stage_off[G::LOADS];
#pragma unroll
    for (int u = 0; u < G::LOADS; ++u) {
        const int e = 64 * (wave * G::LOADS + u) + lane;
        const int row = e / G::SLOTS;
        stage_row[u] = row;
        stage_off[u] = (row * H + 4 * ((e % G::SLOTS) ^ (row & G::SWIZZLE))) * 4;
    }
    const int32_t record_off = int32_t(((lane / 16) * plane + 4 * (lane % 16)) * 4);

    // K and V of this lane's key: chunk c, MFMA s: h index 16c + 8 half + s.
    float kreg[G::CHUNKS][8], vreg[G::CHUNKS][8];
    {
        const int64_t row = head * a.kv_stride + (key_ok ? key : 0) * H;
#pragma unroll
        for (int c = 0; c < G::CHUNKS; ++c) {
            const f32x4 klo = *reinterpret_cast<const f32x4*>(a.k + row + 16 * c + 8 * half);
            const f32x4 khi = *reinterpret_cast<const f32x4*>(a.k + row + 16 * c + 8 * half + 4);
            const f32x4 vlo = *reinterpret_cast<const f32x4*>(a.v + row + 16 * c + 8 * half);
            const f32x4 vhi = *reinterpret_cast<const f32x4*>(a.v + row + 16 * c + 8 * half + 4);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                kreg[c][s] = key_ok ? klo[s] : 0.f;
                kreg[c][4 + s] = key_ok ? khi[s] : 0.f;
                vreg[c][s] = key_ok ? vlo[s] : 0.f;
                vreg[c][4 + s] = key_ok ? vhi[s] : 0.f;
            }
        }
    }

    // Q and dO rows of a stage, swizzled as the forward stages K; the rows'
    // records into this wave's copy.
    auto issue = [&](auto stage, int64_t q0) __attribute__((always_inline)) {
        f32x4* qs = q_of(stage);
        f32x4* ds = d_of(stage);
        const __amdgpu_buffer_rsrc_t q_rsrc = buffer_of(q_head + q0 * H);
        const __amdgpu_buffer_rsrc_t d_rsrc = buffer_of(d_head + q0 * H);
        const int32_t rows_left = int32_t(min(a.queries - q0, int64_t(kKeys)));  // wave-uniform
#pragma unroll
        for (int u = 0; u < G::LOADS; ++u) {
            const int32_t off = stage_row[u] < rows_left ? stage_off[u] : kOutOfRange;
            dma16(q_rsrc, qs + 64 * (wave * G::LOADS + u), off);
            dma16(d_rsrc, ds + 64 * (wave * G::LOADS + u), off);
        }
        // Four queries of plane lane / 16 (lanes 48-63 and queries past the end load nothing).
        const __amdgpu_buffer_rsrc_t r_rsrc = buffer_of(r_head + q0);
        dma16(r_rsrc, r_of(stage) + 64 * wave, lane < 48 && 4 * (lane % 16) < rows_left ? record_off : kOutOfRange);
    };
    ColumnReads<H> columns(col, half);
    ChunkReads<H> chunks(col, half);
    // dV^T and dK^T (rows h, column: this lane's key).
    f32x16 dv[G::OBLOCKS], dk[G::OBLOCKS];
#pragma unroll
    for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            dv[b][r] = 0.f;
            dk[b][r] = 0.f;
        }

    // One block of 32 queries (rows 32 sub .. of the stage, queries sub0 ..)
    // against the wave's keys. MASKED is false when every pair is visible
    // (the block's first query sees the wave's last key, all in range). P and
    // dS are formed four registers at a time (rows 32 sub + 8 g + 4 half +
    // 0..3, consecutive) and go straight into dV^T += dO^T P and dK^T += Q^T
    // dS: MFMA t = 4 g + j pairs the queries row_of(t) of the two lane halves;
    // lane l supplies dO (or Q) [row_of(half, t)][32 b + col].
    auto block_grad = [&](auto stage, auto masked, int sub, int64_t sub0) __attribute__((always_inline)) {
        constexpr bool MASKED = decltype(masked)::value;
        const f32x4* qs = q_of(stage);
        const f32x4* ds = d_of(stage);
        int record = 64 * wave + half;  // this lane's first record slot: 16-byte slot half of the wave's copy
        launder(record);
        const f32x4* rs = r_of(stage) + record;
        chunks.launder_all();
        columns.launder_all();
        const f32x16 s = chunks.product(qs, sub, kreg);
        __builtin_amdgcn_sched_barrier(0);
        const f32x16 dp = chunks.product(ds, sub, vreg);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            __builtin_amdgcn_sched_barrier(0);
            // Rows 32 sub + 8 g + 4 half .. + 3: slot (32 sub + 8 g) / 4 + half of each plane.
            const int slot = 8 * sub + 2 * g;
            const f32x4 m4 = rs[slot], il4 = rs[16 + slot], d4 = rs[32 + slot];
            float p[4], gr[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float shifted = s[4 * g + j] * a.scale - m4[j];
                const float pr = exp_of(shifted) * il4[j];
                const float difference = dp[4 * g + j] - d4[j];
                const float grad = pr * difference;
                if (MASKED) {
                    // Both terms are selected, not scaled by a zero p: a record
                    // slot past the last query may hold any bits, Inf and NaN included.
                    const int64_t query = sub0 + 8 * g + 4 * half + j;
                    const bool visible = key_ok && query < a.queries && key <= query + a.query_offset;
                    p[j] = visible ? pr : 0.f;
                    gr[j] = visible ? grad : 0.f;
                } else {
                    p[j] = pr;
                    gr[j] = grad;
                }
            }
#pragma unroll
            for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    dv[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(columns.read(ds, sub, g, j, b), p[j], dv[b], 0, 0, 0);
                    dk[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(columns.read(qs, sub, g, j, b), gr[j], dk[b], 0, 0, 0);
                }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    using Masked = std::true_type;
    using Whole = std::false_type;
    auto compute = [&](auto stage, int64_t q0) __attribute__((always_inline)) {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            const int64_t sub0 = q0 + 32 * sub;
            // Wave-uniform: a block none of whose queries sees the wave's first key is skipped.
            if (sub0 < a.queries && sub0 + 31 + a.query_offset >= k_wave && k_wave < a.keys) {
                if (sub0 + a.query_offset >= k_wave + 31 && sub0 + 32 <= a.queries && k_wave + 32 <= a.keys)
                    block_grad(stage, Whole{}, sub, sub0);
                else
                    block_grad(stage, Masked{}, sub, sub0);
            }
        }
    };
    // The forward's stage loop: both stages loading at the top of every pass
    // (loads past the last query read zeros), each waited for by count.
    constexpr int kStageLoads = 2 * G::LOADS + 1;
    issue(I0{}, q_begin);
    issue(I1{}, q_begin + kKeys);
    for (int st = 0; st < stages_total; st += 2) {
        const int64_t q0 = q_begin + int64_t(st) * kKeys;
        wait_loads<kStageLoads>();
        lds_barrier();
        compute(I0{}, q0);
        lds_barrier();
        issue(I0{}, q0 + 2 * kKeys);
        wait_loads<kStageLoads>();
        lds_barrier();
        if (st + 1 < stages_total) compute(I1{}, q0 + kKeys);
        lds_barrier();
        issue(I1{}, q0 + 3 * kKeys);
    }
    wait_loads<0>();  // the loads past the end land before the workgroup ends

    // dV = (dV^T)^T and dK = scale (dK^T)^T: lane l holds h rows 32 b + 4 half + 8 g + (0..3) of its key.
    if (key_ok) {
        float* vrow = a.v_grad + (head * a.keys + key) * H;
        float* krow = a.k_grad + (head * a.keys + key) * H;
#pragma unroll
        for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                f32x4 vo, ko;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    vo[s] = dv[b][4 * g + s];
                    ko[s] = a.scale * dk[b][4 * g + s];
                }
                *reinterpret_cast<f32x4*>(vrow + 32 * b + 4 * half + 8 * g) = vo;
                *reinterpret_cast<f32x4*>(krow + 32 * b + 4 * half + 8 * g) = ko;
            }
    }
}

// Key blocks with K and V in LDS, for head dims 32 and 64: eight waves, each
// taking a key group (32 keys) against a query half of every stage (wave w:
// half w / 4, stage rows 32 (w / 4) .. + 31). No wave holds K or V in registers, so
// two share each SIMD; the K and V rows are read from LDS by the same
// swizzled chunk reads as the stage rows. At the end the two halves' partial
// dV^T and dK^T meet in LDS and are added in a fixed order (half 0, then
// half 1): deterministic. (K, V and the stages of h = 128 exceed the LDS, so
// that head dim keeps the register kernel above.)
//
// With DQ the kernel also computes dQ, as partial sums per key block that
// attention_dq_sum_kernel adds up in block order, so that no query kernel has
// to recompute S and dP (five products' MFMAs per pair instead of seven). Each
// stage then ends in two more steps: the waves write their dS blocks to LDS,
// as the stage's [64 queries][128 keys], over the stage's own Q and dO rows
// (h = 64; h = 32 has LDS to spare for a buffer of its own); then wave w
// multiplies queries 16 (w % 4) .. + 15 of it by h columns (w / 4) H / 2 ..
// + H / 2 - 1 of the block's K (16 x 16 x 4 MFMAs over the 128 keys, in key
// order) and stores that part of the block's partial sums. The next stage's
// loads are issued after the stage's first barrier, into the buffer the stage
// before has finished with.
constexpr int kLdsKeyWaves = 8;

// The dS rows of a stage in LDS: row q holds the block's 128 keys, its 16-byte
// chunk c stored at c ^ ds_swizzle(q). Bijective on the low four bits of c for
// any 16 consecutive rows (the dQ step's reads, 16 rows at a time, cover all
// banks), and rows q and q + 4 (the two lane halves of a write) differ in bit 3
// (they fill opposite halves of the banks).
__device__ __forceinline__ int ds_swizzle(int q) { return (q & 15) ^ ((q & 4) << 1); }
constexpr int kDsRow = kKeyBlock;  // floats per dS row

template <int H, bool DQ = false>
__global__ __launch_bounds__(64 * kLdsKeyWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attention_key_grad_lds_kernel(KeyGradArgs a) {
#pragma clang fp contract(off)
    using G = Geometry<H>;  // 64 queries per stage
    constexpr int W = kLdsKeyWaves;
    constexpr int LOADS = G::STAGE_SLOTS / (64 * W);  // stage loads per wave and operand
    constexpr int KV_SLOTS = kKeyBlock * G::SLOTS;
    constexpr int KV_LOADS = KV_SLOTS / (64 * W);
    static_assert(H <= 64 && G::STAGE_SLOTS % (64 * W) == 0 && KV_SLOTS % (64 * W) == 0, "whole loads per wave");
    // Partial sums handed over at the end: 2 x OBLOCKS accumulators per lane
    // of the four half-1 waves, group g's in stage buffer g.
    constexpr int HANDOFF_FLOATS = 2 * G::OBLOCKS * 16 * 64;
    static_assert(HANDOFF_FLOATS <= G::STAGE_SLOTS * 4, "a group's hand-off fits in a stage buffer");
    // A stage's dS: 64 rows of the block's keys, over the stage's Q and dO
    // rows when those are large enough (h = 64), else in a buffer of its own.
    constexpr int DS_FLOATS = kKeys * kDsRow;
    constexpr bool DS_OVER_STAGE = 2 * G::STAGE_SLOTS * 4 >= DS_FLOATS;
    constexpr int DS_OWN = DQ && !DS_OVER_STAGE ? DS_FLOATS / 4 : 1;
    // Each stage's Q and dO rows are one LDS object, apart from the other
    // stage's: the compiler tracks the direct-to-LDS loads in flight per
    // object, so the reads of one stage do not wait for the loads into the
    // other (with one array for both stages it made every stage's first
    // read wait for the next stage's loads).
    __shared__ f32x4 kv_lds[2][KV_SLOTS];
    __shared__ f32x4 stage0[2][G::STAGE_SLOTS], stage1[2][G::STAGE_SLOTS];  // [Q, dO]
    __shared__ f32x4 r_stage0[W][64], r_stage1[W][64];
    __shared__ f32x4 ds_own[DS_OWN];
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    auto q_of = [&](auto stage) __attribute__((always_inline)) -> f32x4* {
        if constexpr (decltype(stage)::value == 0) return stage0[0];
        else return stage1[0];
    };
    auto d_of = [&](auto stage) __attribute__((always_inline)) -> f32x4* {
        if constexpr (decltype(stage)::value == 0) return stage0[1];
        else return stage1[1];
    };
    auto r_of = [&](auto stage) __attribute__((always_inline)) -> f32x4* {
        if constexpr (decltype(stage)::value == 0) return r_stage0[0];
        else return r_stage1[0];
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Key group and query half. Waves w and w + 4 share a SIMD: pairing group
    // g of half 0 with group 3 - g of half 1 spreads the blocks of the two
    // stages on the diagonal, where only groups up to the queries' reach
    // work, over the SIMDs (with group g in both halves, the first stage's
    // blocks fell on SIMDs 0 and 1 only).
    const int group = wave < 4 ? wave : 7 - wave;
    const int qh = wave / 4;
    const int col = lane & 31;
    const int half = lane >> 5;

    const int64_t block = blockIdx.x;
    const int64_t head = block % a.heads;
    const int64_t k_first = (block / a.heads) * kKeyBlock;
    const int64_t k_wave = k_first + 32 * group;
    const int64_t key = k_wave + col;
    const bool key_ok = key < a.keys;
    const int64_t q_seen = max(int64_t(0), k_first - a.query_offset);
    const int64_t q_begin = q_seen / kKeys * kKeys;
    const int stages_total = q_begin < a.queries ? int((a.queries - q_begin + kKeys - 1) / kKeys) : 0;

    const float* q_head = a.q + head * a.q_stride;
    const float* d_head = a.d_out + head * a.q_stride;
    const int64_t plane = plane_of(a.queries);
    const float* r_head = a.rows + head * 3 * plane;

    // K and V of the block's 128 keys into LDS, swizzled as the stages (rows
    // past the last key read zeros).
    {
        const __amdgpu_buffer_rsrc_t k_rsrc = buffer_of(a.k + head * a.kv_stride + k_first * H);
        const __amdgpu_buffer_rsrc_t v_rsrc = buffer_of(a.v + head * a.kv_stride + k_first * H);
        const int32_t rows_left = int32_t(min(a.keys - k_first, int64_t(kKeyBlock)));
#pragma unroll
        for (int u = 0; u < KV_LOADS; ++u) {
            const int e = 64 * (wave * KV_LOADS + u) + lane;
            const int row = e / G::SLOTS;
            const int32_t off = row < rows_left ? (row * H + 4 * ((e % G::SLOTS) ^ (row & G::SWIZZLE))) * 4 : kOutOfRange;
            dma16(k_rsrc, kv_lds[0] + 64 * (wave * KV_LOADS + u), off);
            dma16(v_rsrc, kv_lds[1] + 64 * (wave * KV_LOADS + u), off);
        }
    }
    int32_t stage_row[LOADS], stage_off[LOADS];
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
        const int e = 64 * (wave * LOADS + u) + lane;
        const int row = e / G::SLOTS;
        stage_row[u] = row;
        stage_off[u] = (row * H + 4 * ((e % G::SLOTS) ^ (row & G::SWIZZLE))) * 4;
    }
    const int32_t record_off = int32_t(((lane / 16) * plane + 4 * (lane % 16)) * 4);

    auto issue = [&](auto stage, int64_t q0) __attribute__((always_inline)) {
        f32x4* qs = q_of(stage);
        f32x4* ds = d_of(stage);
        const __amdgpu_buffer_rsrc_t q_rsrc = buffer_of(q_head + q0 * H);
        const __amdgpu_buffer_rsrc_t d_rsrc = buffer_of(d_head + q0 * H);
        const int32_t rows_left = int32_t(min(a.queries - q0, int64_t(kKeys)));  // wave-uniform
#pragma unroll
        for (int u = 0; u < LOADS; ++u) {
            const int32_t off = stage_row[u] < rows_left ? stage_off[u] : kOutOfRange;
            dma16(q_rsrc, qs + 64 * (wave * LOADS + u), off);
            dma16(d_rsrc, ds + 64 * (wave * LOADS + u), off);
        }
        const __amdgpu_buffer_rsrc_t r_rsrc = buffer_of(r_head + q0);
        dma16(r_rsrc, r_of(stage) + 64 * wave, lane < 48 && 4 * (lane % 16) < rows_left ? record_off : kOutOfRange);
    };
    ColumnReads<H> columns(col, half);
    ChunkReads<H> chunks(col, half);
    f32x16 dv[G::OBLOCKS], dk[G::OBLOCKS];
#pragma unroll
    for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            dv[b][r] = 0.f;
            dk[b][r] = 0.f;
        }

    // This wave's block of a stage: queries sub0 .. + 31 (rows 32 qh ..)
    // against its 32 keys, as the register kernel's block_grad; dS of row
    // 8 g + 4 half + j of the block into ds_out[4 g + j].
    auto block_grad = [&](auto stage, auto masked, int64_t sub0, float (&ds_out)[16]) __attribute__((always_inline)) {
        constexpr bool MASKED = decltype(masked)::value;
        const f32x4* qs = q_of(stage);
        const f32x4* ds = d_of(stage);
        int record = 64 * wave + half;
        launder(record);
        const f32x4* rs = r_of(stage) + record;
        int kv_row = 32 * group * G::SLOTS;
        launder(kv_row);
        chunks.launder_all();
        columns.launder_all();
        const f32x16 s = chunks.product_lds(qs, qh, kv_lds[0] + kv_row);
        __builtin_amdgcn_sched_barrier(0);
        const f32x16 dp = chunks.product_lds(ds, qh, kv_lds[1] + kv_row);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            __builtin_amdgcn_sched_barrier(0);
            const int slot = 8 * qh + 2 * g;
            const f32x4 m4 = rs[slot], il4 = rs[16 + slot], d4 = rs[32 + slot];
            float p[4], gr[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float shifted = s[4 * g + j] * a.scale - m4[j];
                const float pr = exp_of(shifted) * il4[j];
                const float difference = dp[4 * g + j] - d4[j];
                const float grad = pr * difference;
                if (MASKED) {
                    // Both terms are selected, not scaled by a zero p: a record
                    // slot past the last query may hold any bits, Inf and NaN included.
                    const int64_t query = sub0 + 8 * g + 4 * half + j;
                    const bool visible = key_ok && query < a.queries && key <= query + a.query_offset;
                    p[j] = visible ? pr : 0.f;
                    gr[j] = visible ? grad : 0.f;
                } else {
                    p[j] = pr;
                    gr[j] = grad;
                }
            }
#pragma unroll
            for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    dv[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(columns.read(ds, qh, g, j, b), p[j], dv[b], 0, 0, 0);
                    dk[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(columns.read(qs, qh, g, j, b), gr[j], dk[b], 0, 0, 0);
                }
#pragma unroll
            for (int j = 0; j < 4; ++j) ds_out[4 * g + j] = gr[j];
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    using Masked = std::true_type;
    using Whole = std::false_type;
    // The wave's block of the stage; dS stays 0 for a skipped block.
    auto compute = [&](auto stage, int64_t q0, float (&ds_out)[16]) __attribute__((always_inline)) {
        const int64_t sub0 = q0 + 32 * qh;
        // Wave-uniform: skipped when none of the block's queries sees the wave's first key.
        if (sub0 < a.queries && sub0 + 31 + a.query_offset >= k_wave && k_wave < a.keys) {
            if (sub0 + a.query_offset >= k_wave + 31 && sub0 + 32 <= a.queries && k_wave + 32 <= a.keys)
                block_grad(stage, Whole{}, sub0, ds_out);
            else
                block_grad(stage, Masked{}, sub0, ds_out);
        }
    };
    if constexpr (DQ) {
        // The dQ step's share of wave w: stage rows 16 (w % 4) + (lane % 16)
        // (B operand: dS[q][keys]) against h columns (w / 4) H / 2 + 16 t +
        // (lane % 16) of K (A operand), t < H / 32; MFMA 4 u + e pairs the
        // keys 16 u + 4 (lane / 16) + e. The 16 x 16 result in lane l:
        // h = 4 (l / 16) + r, query l % 16, four consecutive h per lane.
        constexpr int HT = H / 32;
        const int h_base = (wave / 4) * (H / 2);
        // Partial sums of this block: rows from its first stage's first query.
        int64_t rows_before = 0;
        for (int64_t b = 0; b < block / a.heads; ++b) rows_before += block_queries(b, a.queries, a.query_offset);
        const __amdgpu_buffer_rsrc_t p_rsrc =
            buffer_of(a.partials + (head * a.partial_rows + rows_before) * H);
        constexpr int STORES = HT;  // partial-sum stores per wave per stage
        auto dq_step = [&](auto stage, int64_t q0, const float (&ds_in)[16]) __attribute__((always_inline)) {
            float* dsm = DS_OVER_STAGE ? reinterpret_cast<float*>(q_of(stage)) : reinterpret_cast<float*>(ds_own);
            if constexpr (DS_OVER_STAGE) lds_barrier();  // every wave is done with the stage's Q and dO
            // dS row 32 qh + 8 g + 4 half + j, key 32 group + col.
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int q = 32 * qh + 8 * g + 4 * half + j, kl = 32 * group + col;
                    dsm[q * kDsRow + 4 * ((kl / 4) ^ ds_swizzle(q)) + (kl & 3)] = ds_in[4 * g + j];
                }
            lds_barrier();  // the stage's dS is whole
            // Byte offsets of the A reads (K row 4 lg + e of each 16-key step,
            // column h_base + 16 t + lq) and of the B reads (chunk 4 (u % 4) +
            // lg of dS row dq_row); u / 4 and the steps add immediates. Formed
            // here, from a laundered lane, rather than held through the stage.
            int l = lane;
            launder(l);
            const int lq = l % 16, lg = l / 16;
            const int dq_row = 16 * (wave % 4) + lq;  // stage row
            int k_off[4][HT], d_off[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma unroll
                for (int t = 0; t < HT; ++t) {
                    const int row = 4 * lg + e, h = h_base + 16 * t + lq;
                    k_off[e][t] = (row * H + 4 * ((h / 4) ^ (row & G::SWIZZLE)) + (h & 3)) * 4;
                }
                d_off[e] = (dq_row * kDsRow + 4 * ((4 * e + lg) ^ ds_swizzle(dq_row))) * 4;
            }
            f32x4 acc[HT];
#pragma unroll
            for (int t = 0; t < HT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            const char* kb = reinterpret_cast<const char*>(kv_lds[0]);
            const char* db = reinterpret_cast<const char*>(dsm);
#pragma unroll
            for (int u = 0; u < kDsRow / 16; ++u) {
                const f32x4 d4 = *reinterpret_cast<const f32x4*>(db + d_off[u % 4] + (u / 4) * 256);
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int t = 0; t < HT; ++t) {
                        const float kv = *reinterpret_cast<const float*>(kb + k_off[e][t] + u * 16 * H * 4);
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv, d4[e], acc[t], 0, 0, 0);
                    }
            }
            // Rows past the last query are dropped (out-of-range offsets).
            const int64_t q = q0 + dq_row;
            typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int t = 0; t < HT; ++t) {
                const int32_t off = q < a.queries ? int32_t(((q - q_begin) * H + h_base + 16 * t + 4 * lg) * 4)
                                                  : kOutOfRange;
                // The row offset rides in the vector offset, soffset 0: with a
                // scalar soffset the compiler may let the next VALU overwrite
                // the data registers before this 4-dword store has read them.
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[t]), p_rsrc, off, 0, 0);
            }
        };
        auto stage_dq = [&](auto stage, int64_t q0) __attribute__((always_inline)) {
            float dsv[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) dsv[i] = 0.f;
            compute(stage, q0, dsv);
            dq_step(stage, q0, dsv);
        };
        // Each stage starts once every wave is done with the stage before,
        // whose buffer then takes the next stage's loads (past the last query
        // they read zeros); it ends waiting for those loads, which leaves this
        // wave's partial-sum stores in flight. The waits and loads are
        // unconditional, so the compiler's count of the loads in flight stays
        // exact and it adds no waits of its own.
        issue(I0{}, q_begin);
        wait_loads<0>();  // K, V and the first stage
        for (int st = 0; st < stages_total; st += 2) {
            const int64_t q0 = q_begin + int64_t(st) * kKeys;
            lds_barrier();
            issue(I1{}, q0 + kKeys);
            stage_dq(I0{}, q0);
            wait_loads<STORES>();
            if (st + 1 >= stages_total) break;
            lds_barrier();
            issue(I0{}, q0 + 2 * kKeys);
            stage_dq(I1{}, q0 + kKeys);
            wait_loads<STORES>();
        }
    } else {
        // K and V go first, so the first wait (all but one stage's loads)
        // covers them too.
        constexpr int kStageLoads = 2 * LOADS + 1;
        float unused[16];
        issue(I0{}, q_begin);
        issue(I1{}, q_begin + kKeys);
        for (int st = 0; st < stages_total; st += 2) {
            const int64_t q0 = q_begin + int64_t(st) * kKeys;
            wait_loads<kStageLoads>();
            lds_barrier();
            compute(I0{}, q0, unused);
            lds_barrier();
            issue(I0{}, q0 + 2 * kKeys);
            wait_loads<kStageLoads>();
            lds_barrier();
            if (st + 1 < stages_total) compute(I1{}, q0 + kKeys, unused);
            lds_barrier();
            issue(I1{}, q0 + 3 * kKeys);
        }
    }
    wait_loads<0>();
    lds_barrier();  // every wave is done with the stages (and K, V)

    // Half 1 hands its partial sums to half 0 through the stages' space
    // (lane-consecutive, conflict-free); half 0 adds them and writes.
    float* handoff = reinterpret_cast<float*>(group < 2 ? stage0[group] : stage1[group - 2]) + lane;
    if (qh == 1) {
#pragma unroll
        for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                handoff[((2 * b) * 16 + r) * 64] = dv[b][r];
                handoff[((2 * b + 1) * 16 + r) * 64] = dk[b][r];
            }
    }
    lds_barrier();
    if (qh == 0 && key_ok) {
        float* vrow = a.v_grad + (head * a.keys + key) * H;
        float* krow = a.k_grad + (head * a.keys + key) * H;
#pragma unroll
        for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                f32x4 vo, ko;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const int r = 4 * g + s;
                    vo[s] = dv[b][r] + handoff[((2 * b) * 16 + r) * 64];
                    const float sum = dk[b][r] + handoff[((2 * b + 1) * 16 + r) * 64];
                    ko[s] = a.scale * sum;
                }
                *reinterpret_cast<f32x4*>(vrow + 32 * b + 4 * half + 8 * g) = vo;
                *reinterpret_cast<f32x4*>(krow + 32 * b + 4 * half + 8 * g) = ko;
            }
    }
}

struct QueryGradArgs {
    const float* q;
    const float* k;
    const float* v;
    const float* d_out;
    const float* rows;
    float* q_grad;
    int64_t queries, keys;
    int64_t q_stride, kv_stride;
    int64_t query_offset;
    int64_t heads;
    int32_t query_blocks;
    float scale;
};

template <int H>
__global__ __launch_bounds__(64 * kWaves)
__attribute__((amdgpu_waves_per_eu(backward_waves_per_simd(H), backward_waves_per_simd(H))))
void attention_query_grad_kernel(QueryGradArgs a) {
#pragma clang fp contract(off)
    using G = Geometry<H>;
    __shared__ f32x4 k_stage0[G::STAGE_SLOTS], k_stage1[G::STAGE_SLOTS];
    __shared__ f32x4 v_stage0[G::STAGE_SLOTS], v_stage1[G::STAGE_SLOTS];
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    auto k_of = [&](auto stage) __attribute__((always_inline)) -> f32x4* {
        if constexpr (decltype(stage)::value == 0) return k_stage0;
        else return k_stage1;
    };
    auto v_of = [&](auto stage) __attribute__((always_inline)) -> f32x4* {
        if constexpr (decltype(stage)::value == 0) return v_stage0;
        else return v_stage1;
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31;  // this lane's query within the wave
    const int half = lane >> 5;

    // Longest query blocks first, over all heads (the forward's order).
    const int64_t block = blockIdx.x;
    const int64_t head = block % a.heads;
    const int64_t query_block = a.query_blocks - 1 - block / a.heads;
    const int64_t q_first = query_block * kQueries;
    const int64_t q_wave = q_first + 32 * wave;
    const int64_t q = q_wave + col;
    const bool row_ok = q < a.queries;
    const int64_t wg_keys = min(a.keys, min(q_first + kQueries, a.queries) - 1 + a.query_offset + 1);
    const int64_t wave_keys = min(a.keys, q_wave + 31 + a.query_offset + 1);
    const int stages_total = int((wg_keys + kKeys - 1) / kKeys);

    const float* k_head = a.k + head * a.kv_stride;
    const float* v_head = a.v + head * a.kv_stride;
    // Per lane, constant over the stages: the stage row of each load and the
    // byte offset of its 16 bytes from the stage's first row.
    int32_t stage_row[G::LOADS], stage_off[G::LOADS];
#pragma unroll
    for (int u = 0; u < G::LOADS; ++u) {
        const int e = 64 * (wave * G::LOADS + u) + lane;
        const int row = e / G::SLOTS;
        stage_row[u] = row;
        stage_off[u] = (row * H + 4 * ((e % G::SLOTS) ^ (row & G::SWIZZLE))) * 4;
    }

    // Q and dO of this lane's query (chunk c, MFMA s: h index 16c + 8 half + s) and its row record.
    float qreg[G::CHUNKS][8], dreg[G::CHUNKS][8];
    f32x4 rec = {0.f, 0.f, 0.f, 0.f};
    {
        const int64_t row = head * a.q_stride + (row_ok ? q : 0) * H;
#pragma unroll
        for (int c = 0; c < G::CHUNKS; ++c) {
            const f32x4 qlo = *reinterpret_cast<const f32x4*>(a.q + row + 16 * c + 8 * half);
            const f32x4 qhi = *reinterpret_cast<const f32x4*>(a.q + row + 16 * c + 8 * half + 4);
            const f32x4 dlo = *reinterpret_cast<const f32x4*>(a.d_out + row + 16 * c + 8 * half);
            const f32x4 dhi = *reinterpret_cast<const f32x4*>(a.d_out + row + 16 * c + 8 * half + 4);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                qreg[c][s] = row_ok ? qlo[s] : 0.f;
                qreg[c][4 + s] = row_ok ? qhi[s] : 0.f;
                dreg[c][s] = row_ok ? dlo[s] : 0.f;
                dreg[c][4 + s] = row_ok ? dhi[s] : 0.f;
            }
        }
        if (row_ok) {
            const float* planes = a.rows + head * 3 * plane_of(a.queries) + q;
            rec = f32x4{planes[0], planes[plane_of(a.queries)], planes[2 * plane_of(a.queries)], 0.f};
        }
    }

    // K and V rows of a stage, both swizzled (K is read by chunks for S^T and
    // element by element for K^T).
    auto issue = [&](auto stage, int64_t key0) __attribute__((always_inline)) {
        f32x4* ks = k_of(stage);
        f32x4* vs = v_of(stage);
        const __amdgpu_buffer_rsrc_t k_rsrc = buffer_of(k_head + key0 * H);
        const __amdgpu_buffer_rsrc_t v_rsrc = buffer_of(v_head + key0 * H);
        const int32_t rows_left = int32_t(min(a.keys - key0, int64_t(kKeys)));  // wave-uniform
#pragma unroll
        for (int u = 0; u < G::LOADS; ++u) {
            const int32_t off = stage_row[u] < rows_left ? stage_off[u] : kOutOfRange;
            dma16(k_rsrc, ks + 64 * (wave * G::LOADS + u), off);
            dma16(v_rsrc, vs + 64 * (wave * G::LOADS + u), off);
        }
    };
    ColumnReads<H> columns(col, half);
    ChunkReads<H> chunks(col, half);
    // dQ^T (rows h, column: this lane's query).
    f32x16 dq[G::OBLOCKS];
#pragma unroll
    for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) dq[b][r] = 0.f;

    // dS^T of 32 keys (rows 32 sub + 8 g + 4 half + 0..3 of the stage, four
    // registers at a time) straight into dQ^T += K^T dS^T: MFMA t = 4 g + j
    // pairs the keys row_of(t) of the two lane halves; lane l supplies
    // K[row_of(half, t)][32 b + col].
    auto block_grad = [&](auto stage, auto masked, int sub, int64_t sub0) __attribute__((always_inline)) {
        constexpr bool MASKED = decltype(masked)::value;
        const f32x4* ks = k_of(stage);
        chunks.launder_all();
        columns.launder_all();
        const f32x16 s = chunks.product(ks, sub, qreg);
        __builtin_amdgcn_sched_barrier(0);
        const f32x16 dp = chunks.product(v_of(stage), sub, dreg);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            __builtin_amdgcn_sched_barrier(0);
            float gr[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float shifted = s[4 * g + j] * a.scale - rec[0];
                const float pr = exp_of(shifted) * rec[1];
                const float difference = dp[4 * g + j] - rec[2];
                const float grad = pr * difference;
                if (MASKED) {
                    const int64_t key = sub0 + 8 * g + 4 * half + j;
                    gr[j] = row_ok && key < a.keys && key <= q + a.query_offset ? grad : 0.f;
                } else {
                    gr[j] = grad;
                }
            }
#pragma unroll
            for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    dq[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(columns.read(ks, sub, g, j, b), gr[j], dq[b], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    using Masked = std::true_type;
    using Whole = std::false_type;
    const int64_t wave_horizon = q_wave + a.query_offset;  // last key the wave's first query sees
    auto compute = [&](auto stage, int64_t key0) __attribute__((always_inline)) {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            const int64_t sub0 = key0 + 32 * sub;
            if (sub0 < wave_keys) {  // wave-uniform
                if (sub0 + 31 <= wave_horizon && sub0 + 32 <= a.keys && q_wave + 32 <= a.queries)
                    block_grad(stage, Whole{}, sub, sub0);
                else
                    block_grad(stage, Masked{}, sub, sub0);
            }
        }
    };
    constexpr int kStageLoads = 2 * G::LOADS;
    issue(I0{}, 0);
    issue(I1{}, kKeys);
    for (int st = 0; st < stages_total; st += 2) {
        const int64_t key0 = int64_t(st) * kKeys;
        wait_loads<kStageLoads>();
        lds_barrier();
        compute(I0{}, key0);
        lds_barrier();
        issue(I0{}, key0 + 2 * kKeys);
        wait_loads<kStageLoads>();
        lds_barrier();
        if (st + 1 < stages_total) compute(I1{}, key0 + kKeys);
        lds_barrier();
        issue(I1{}, key0 + 3 * kKeys);
    }
    wait_loads<0>();

    // dQ = scale (dS K): lane l holds h rows 32 b + 4 half + 8 g + (0..3) of its query.
    if (row_ok) {
        float* qrow = a.q_grad + (head * a.queries + q) * H;
#pragma unroll
        for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                f32x4 out;
#pragma unroll
                for (int s = 0; s < 4; ++s) out[s] = a.scale * dq[b][4 * g + s];
                *reinterpret_cast<f32x4*>(qrow + 32 * b + 4 * half + 8 * g) = out;
            }
    }
}

struct DqSumArgs {
    const float* partials;
    float* q_grad;
    int64_t heads, queries, keys, query_offset, partial_rows;
    float scale;
};

// dQ = scale x the sum of the key blocks' partial sums, added in block order
// (the blocks whose stages cover the query; those are 0 .. some b, since a
// block's first stage starts no earlier than the block before's). One
// thread per 4 h of a query.
template <int H>
__global__ __launch_bounds__(256) void attention_dq_sum_kernel(DqSumArgs a) {
#pragma clang fp contract(off)
    constexpr int C = H / 4;
    const int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (t >= a.heads * a.queries * C) return;
    const int c = int(t % C);
    const int64_t row = t / C;  // head * queries + query
    const int64_t head = row / a.queries, q = row % a.queries;
    const float* base = a.partials + head * a.partial_rows * H + 4 * c;
    const int64_t blocks = (a.keys + kKeyBlock - 1) / kKeyBlock;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    int64_t before = 0;  // rows of the blocks before
    // Eight blocks' loads in flight at a time (non-temporal: each partial is
    // read once), added in block order.
    constexpr int kInFlight = 8;
    for (int64_t b = 0; b < blocks; b += kInFlight) {
        f32x4 x[kInFlight];
        bool ok[kInFlight];
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) {
            const int64_t first = stage_begin(b + u, a.query_offset);
            ok[u] = b + u < blocks && first <= q;
            x[u] = ok[u] ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(base + (before + q - first) * H))
                         : f32x4{0.f, 0.f, 0.f, 0.f};
            if (ok[u]) before += a.queries - first;
        }
#pragma unroll
        for (int u = 0; u < kInFlight; ++u)
            if (ok[u])
#pragma unroll
                for (int s = 0; s < 4; ++s) acc[s] = acc[s] + x[u][s];
        if (!ok[kInFlight - 1]) break;
    }
    f32x4 out;
#pragma unroll
    for (int s = 0; s < 4; ++s) out[s] = a.scale * acc[s];
    *reinterpret_cast<f32x4*>(a.q_grad + row * H + 4 * c) = out;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int H>
hipError_t launch_backward(const AttentionBackwardArgs& a, hipStream_t stream) {
    float* rows = a.workspace;
    const int64_t total = a.heads * a.queries;
    RowsArgs ra{a.d_out, a.out, a.stats, rows, a.queries, a.q_stride, total};
    hipLaunchKernelGGL(attention_rows_kernel<H>, dim3(unsigned((total * 16 + 255) / 256)), dim3(256), 0, stream, ra);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;

    KeyGradArgs ka{a.q, a.k, a.v, a.d_out, rows, a.k_grad, a.v_grad, a.queries, a.keys, a.q_stride,
                   a.kv_stride, a.query_offset, a.heads, a.scale, nullptr, 0};
    const int64_t key_blocks = (a.keys + kKeyBlock - 1) / kKeyBlock;
    if constexpr (H <= 64) {
        // dQ from the key kernel's partial sums when the workspace holds them
        // after the row records: for all heads at once, or in runs of heads
        // that still fill the device (512 workgroups or more); else the query
        // kernel recomputes S and dP for it.
        const size_t record_bytes = size_t(a.heads) * 3 * size_t(plane_of(a.queries)) * 4;
        const size_t partial_start = (record_bytes + 255) / 256 * 256;
        const int64_t prows = partial_rows(a.queries, a.keys, a.query_offset);
        const size_t per_head = size_t(prows) * H * 4;
        const size_t room = a.workspace_bytes > partial_start ? a.workspace_bytes - partial_start : 0;
        const int64_t run = per_head == 0 ? a.heads : int64_t(std::min(size_t(a.heads), room / per_head));
        if (run > 0 && (run == a.heads || run * key_blocks >= 512)) {
            float* partials = reinterpret_cast<float*>(reinterpret_cast<char*>(a.workspace) + partial_start);
            for (int64_t h0 = 0; h0 < a.heads; h0 += run) {
                const int64_t n = std::min(run, a.heads - h0);
                KeyGradArgs ra_ = ka;
                ra_.q = a.q + h0 * a.q_stride;
                ra_.d_out = a.d_out + h0 * a.q_stride;
                ra_.k = a.k + h0 * a.kv_stride;
                ra_.v = a.v + h0 * a.kv_stride;
                ra_.rows = rows + h0 * 3 * plane_of(a.queries);
                ra_.k_grad = a.k_grad + h0 * a.keys * H;
                ra_.v_grad = a.v_grad + h0 * a.keys * H;
                ra_.heads = n;
                ra_.partials = partials;
                ra_.partial_rows = prows;
                hipLaunchKernelGGL((attention_key_grad_lds_kernel<H, true>), dim3(unsigned(n * key_blocks)),
                                   dim3(64 * kLdsKeyWaves), 0, stream, ra_);
                err = hipGetLastError();
                if (err != hipSuccess) return err;
                DqSumArgs sa{partials, a.q_grad + h0 * a.queries * H, n, a.queries, a.keys, a.query_offset, prows,
                             a.scale};
                hipLaunchKernelGGL(attention_dq_sum_kernel<H>, dim3(unsigned((n * a.queries * (H / 4) + 255) / 256)),
                                   dim3(256), 0, stream, sa);
                err = hipGetLastError();
                if (err != hipSuccess) return err;
            }
            return hipSuccess;
        }
    }
    if constexpr (H <= 64)
        hipLaunchKernelGGL(attention_key_grad_lds_kernel<H>, dim3(unsigned(a.heads * key_blocks)),
                           dim3(64 * kLdsKeyWaves), 0, stream, ka);
    else
        hipLaunchKernelGGL(attention_key_grad_kernel<H>, dim3(unsigned(a.heads * key_blocks)), dim3(64 * kWaves), 0,
                           stream, ka);
    err = hipGetLastError();
    if (err != hipSuccess) return err;

    QueryGradArgs qa{a.q, a.k, a.v, a.d_out, rows, a.q_grad, a.queries, a.keys, a.q_stride, a.kv_stride,
                     a.query_offset, a.heads, int32_t((a.queries + kQueries - 1) / kQueries), a.scale};
    hipLaunchKernelGGL(attention_query_grad_kernel<H>, dim3(unsigned(a.heads * qa.query_blocks)), dim3(64 * kWaves),
                       0, stream, qa);
    return hipGetLastError();
}

}  // namespace

bool attention_backward_supported(const AttentionBackwardArgs& a) {
    const bool dims = a.head_dim == 32 || a.head_dim == 64 || a.head_dim == 128;
    const bool aligned = aligned16(a.q) && aligned16(a.k) && aligned16(a.v) && aligned16(a.out) &&
                         aligned16(a.d_out) && aligned16(a.q_grad) && aligned16(a.k_grad) && aligned16(a.v_grad) &&
                         aligned16(a.workspace) && (reinterpret_cast<uintptr_t>(a.stats) & 7) == 0 &&
                         a.q_stride % 4 == 0 && a.kv_stride % 4 == 0;
    // Per-head buffer offsets within 31 bits (the stage loads), the grids within 32 bits, and the
    // workspace large enough for the row records.
    const bool offsets = a.keys * a.head_dim * 4 < (int64_t(1) << 31) - 4096 &&
                         a.queries * a.head_dim * 4 < (int64_t(1) << 31) - 4096 &&
                         3 * plane_of(a.queries) * 4 < (int64_t(1) << 31) - 4096;
    const bool grids = a.heads * ((a.keys + kKeyBlock - 1) / kKeyBlock) < (int64_t(1) << 31) &&
                       a.heads * ((a.queries + kQueries - 1) / kQueries) < (int64_t(1) << 31) &&
                       a.heads * a.queries * 16 < (int64_t(1) << 32) - 256;
    const bool room = a.workspace != nullptr && size_t(a.heads) * 3 * size_t(plane_of(a.queries)) * 4 <= a.workspace_bytes;
    return dims && aligned && offsets && grids && room;
}

hipError_t launch_attention_backward(const AttentionBackwardArgs& a, hipStream_t stream) {
    if (a.heads == 0 || a.queries == 0 || a.keys == 0) return hipSuccess;
    switch (a.head_dim) {
        case 32: return launch_backward<32>(a, stream);
        case 64: return launch_backward<64>(a, stream);
        case 128: return launch_backward<128>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace sn

// Fused causal attention forward: O = causal_softmax(scale * Q K^T) V per
// head, without writing the [queries, keys] score matrix. The reference
// computes it as three calls (layers/attention.rs:206-213): the scores
// product (MatmulSpec::new(T, T, h).right_transposed(), batched over the
// heads), causal_softmax (kernels/attention.rs:140-183) and the mix product
// (MatmulSpec::new(T, h, T)); the probabilities it keeps for the backward
// are written here on request, so the backward (attention.rs:220-267) can
// run unchanged.
//
// Layout: Q [heads][queries][h] and K, V [heads][keys][h] (head-major, rows
// q_stride / kv_stride floats apart per head), O [heads][queries][h], P
// [heads][queries][keys]. Query q of a head sees keys 0 ..= q +
// query_offset (as causal_softmax with `queries` rows per matrix).
//
// Design (gfx950, fp32 matrix cores, v_mfma_f32_32x32x2f32):
//  * A workgroup of 4 waves owns 128 queries of one head; a wave owns 32.
//    K and V stream through LDS in blocks of 64 keys, two stages, loaded
//    straight from memory into LDS (buffer_load ... lds); K's 16-byte chunks
//    are XOR-swizzled by row so that fragment reads are conflict-free.
//  * A wave computes S^T = K Q^T for 32 keys at a time (keys along the
//    accumulator rows, its 32 queries along the columns, Q held in
//    registers). In the 32x32 accumulator, lane l holds column l % 32, so
//    every register of a lane belongs to the lane's query: the online
//    softmax (running max m, running sum l, O rescaled by exp(m_old -
//    m_new)) is per lane, with one exchange between the lane pair (l, l ^
//    32) that share a query, and the probabilities are already laid out as
//    the B operand of O^T += V^T P^T: no trip through LDS.
//  * Element arithmetic follows causal_softmax: s * scale, minus the
//    maximum, each rounded, then the exponential (as 2^(d log2 e) on the
//    transcendental unit); the sum is accumulated in a different order (per
//    32-key block, then rescaled), so parity is to the fp32 tolerance.
//  * Only the 32-key blocks on a wave's diagonal (or past the last key) test
//    keys against each query's horizon; the others skip the mask.
//  * P (optional) takes a second pass over K with the final m and l: p =
//    e^(s * scale - m) * (1 / l), 0 past the diagonal, so it matches the
//    probabilities causal_softmax leaves to the fp32 tolerance.
//  * Query blocks are launched longest first across all heads (the last
//    queries see the most keys).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <type_traits>

#include "attention_common.h"
#include "gemm_common.h"
#include "gemm_internal.h"


namespace sn {
namespace {

using namespace attn;

struct AttentionArgs {
    const float* q;
    const float* k;
    const float* v;
    float* o;
    float* p;      // null: no probabilities
    float* stats;  // null, or per query {m, l}: the maximum of its scaled visible scores and the sum of e^(x - m)
    int64_t queries, keys;
    int64_t q_stride, kv_stride;  // floats between heads
    int64_t query_offset;
    int64_t heads;
    int32_t query_blocks;
    float scale;
};

// Waves per SIMD the forward kernel's registers are budgeted for: as many
// workgroups as its LDS stages allow (64 KB at h = 64: two per CU).
constexpr int forward_waves_per_simd(int h) { return h <= 32 ? 3 : h == 64 ? 2 : 1; }

template <int H>
__global__ __launch_bounds__(64 * kWaves)
__attribute__((amdgpu_waves_per_eu(forward_waves_per_simd(H), forward_waves_per_simd(H))))
void causal_attention_kernel(AttentionArgs args) {
#pragma clang fp contract(off)
    constexpr int KEYS = kKeys;      // per LDS stage
    constexpr int SUBS = KEYS / 32;  // 32-key blocks per stage
    using G = Geometry<H, KEYS>;
    // Two LDS stages per operand, each its own array: every LDS access below
    // names its stage at compile time, so the compiler's wait counts leave the
    // other stage's loads in flight.
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

    // Longest query blocks first, over all heads: the heads' last query
    // blocks (which see the most keys), then the ones before, so that the
    // short blocks fill in at the end.
    const int64_t block = blockIdx.x;
    const int64_t head = block % args.heads;
    const int64_t query_block = args.query_blocks - 1 - block / args.heads;
    const int64_t q_first = query_block * kQueries;
    const int64_t q_wave = q_first + 32 * wave;
    const int64_t q = q_wave + col;
    // Keys this workgroup and this wave can see (exclusive ends).
    const int64_t wg_keys = min(args.keys, min(q_first + kQueries, args.queries) - 1 + args.query_offset + 1);
    const int64_t wave_keys = min(args.keys, q_wave + 31 + args.query_offset + 1);
    const int stages_total = int((wg_keys + KEYS - 1) / KEYS);

    const float* kh = args.k + head * args.kv_stride;
    const float* vh = args.v + head * args.kv_stride;
    const __amdgpu_buffer_rsrc_t k_rsrc = buffer_of(kh);
    const __amdgpu_buffer_rsrc_t v_rsrc = buffer_of(vh);

    // Q of this lane's query in registers: chunk c, MFMA s: h index 16c + 8 half + s.
    float qreg[G::CHUNKS][8];
    {
        // Lanes past the last query read query 0 and keep zeros.
        const bool ok = q < args.queries;
        const float* qrow = args.q + head * args.q_stride + (ok ? q : 0) * H;
#pragma unroll
        for (int c = 0; c < G::CHUNKS; ++c) {
            const f32x4 lo = *reinterpret_cast<const f32x4*>(qrow + 16 * c + 8 * half);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(qrow + 16 * c + 8 * half + 4);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                qreg[c][s] = ok ? lo[s] : 0.f;
                qreg[c][4 + s] = ok ? hi[s] : 0.f;
            }
        }
    }

    // Stage loads: instruction u of wave w covers rows 4 (w * LOADS + u) + lane / SLOTS' groups;
    // lane i writes LDS slot (row, i % SLOTS) of its 1 KB; for K that slot holds global chunk
    // (slot ^ swizzle(row)), for V chunk slot.
    auto issue = [&](auto stage, int64_t key0, bool with_v) __attribute__((always_inline)) {
        f32x4* ks = k_of(stage);
        f32x4* vs = v_of(stage);
#pragma unroll
        for (int u = 0; u < G::LOADS; ++u) {
            const int instr = wave * G::LOADS + u;
            const int e = 64 * instr + lane;  // f32x4 slot in the stage
            const int row = e / G::SLOTS;
            const int slot = e % G::SLOTS;
            const int64_t key = key0 + row;
            const int chunk_k = slot ^ (row & G::SWIZZLE);
            const int32_t k_off = key < args.keys ? int32_t((key * H + 4 * chunk_k) * 4) : kOutOfRange;
            dma16(k_rsrc, ks + 64 * instr, k_off);
            if (with_v) {
                const int32_t v_off = key < args.keys ? int32_t((key * H + 4 * slot) * 4) : kOutOfRange;
                dma16(v_rsrc, vs + 64 * instr, v_off);
            }
        }
    };

    // S^T for 32 keys (rows sub * 32 .. +31 of the stage) against this wave's queries.
    auto scores = [&](auto stage, int sub) __attribute__((always_inline)) {
        const f32x4* ks = k_of(stage);
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
        const int row = 32 * sub + col;
        const int swz = row & G::SWIZZLE;
#pragma unroll
        for (int c = 0; c < G::CHUNKS; ++c) {
            const int g = 4 * c + 2 * half;  // chunk of h = 16c + 8 half
            const f32x4 lo = ks[row * G::SLOTS + (g ^ swz)];
            const f32x4 hi = ks[row * G::SLOTS + ((g + 1) ^ swz)];
            const float kv[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
            for (int s = 0; s < 8; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[s], qreg[c][s], acc, 0, 0, 0);
        }
        return acc;
    };
    // Key of accumulator register r of this lane, within the 32-key sub-block.
    auto key_of = [&](int r) __attribute__((always_inline)) { return 4 * half + 8 * (r / 4) + (r % 4); };

    // Online softmax state of this lane's query, and O^T (rows h, column q).
    float m = -INFINITY, l = 0.f;
    f32x16 o[G::OBLOCKS];
#pragma unroll
    for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[b][r] = 0.f;

    // Last key of the 32-key block from sub0 that this lane's query sees, as
    // an offset within the block: -1 (none) .. 31 (all).
    auto visible_limit = [&](int64_t sub0) __attribute__((always_inline)) {
        const int64_t last = min(args.keys - 1, q + args.query_offset) - sub0;
        return int(max(int64_t(-1), min(int64_t(31), last)));
    };
    // Online softmax of one 32-key block (scores acc; keys sub0 .., block sub
    // of the stage) and its O^T += V^T P^T. MASKED is false when the wave's
    // first query sees the whole block (so every lane's query does): no
    // per-key test.
    auto softmax_and_mix = [&](auto stage, auto masked, int sub, const f32x16& acc, int64_t sub0)
                               __attribute__((always_inline)) {
        constexpr bool MASKED = decltype(masked)::value;
        float x[16];
        float block_max = -INFINITY;
        const int limit = MASKED ? visible_limit(sub0) : 31;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            x[r] = acc[r] * args.scale;
            if (MASKED) x[r] = key_of(r) <= limit ? x[r] : -INFINITY;
            block_max = fmaxf(block_max, x[r]);
        }
        block_max = fmaxf(block_max, __shfl_xor(block_max, 32));
        const float m_new = fmaxf(m, block_max);
        const float alpha = exp_of(m - m_new);
        float sum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            x[r] = exp_of(x[r] - m_new);  // now the probability numerator
            sum = sum + x[r];
        }
        sum = sum + __shfl_xor(sum, 32);
        l = l * alpha + sum;
        m = m_new;
        const float* vs = reinterpret_cast<const float*>(v_of(stage));
#pragma unroll
        for (int b = 0; b < G::OBLOCKS; ++b) {
#pragma unroll
            for (int r = 0; r < 16; ++r) o[b][r] = o[b][r] * alpha;
            // O^T rows 32 b .. +31 += V^T (rows h) P^T: MFMA t pairs keys key_of(t) of the two
            // lane halves; lane l supplies V[key_of(t)][32 b + col].
            const float* vrow = vs + (32 * sub) * H + 32 * b + col;
#pragma unroll
            for (int t = 0; t < 16; ++t)
                o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[key_of(t) * H], x[t], o[b], 0, 0, 0);
        }
    };
    // The stage's 32-key blocks that the wave's last query sees, one at a
    // time (scores, softmax, mix: the fewest registers live, so that two
    // workgroups share a CU at h = 64). A block is whole for the wave when
    // its first query sees every key of it (wave-uniform).
    using Masked = std::true_type;
    using Whole = std::false_type;
    const int64_t wave_horizon = q_wave + args.query_offset;  // last key the wave's first query sees
    auto compute = [&](auto stage, int64_t key0) __attribute__((always_inline)) {
#pragma unroll
        for (int sub = 0; sub < SUBS; ++sub) {
            const int64_t sub0 = key0 + 32 * sub;
            if (sub0 < wave_keys) {  // wave-uniform
                const f32x16 s = scores(stage, sub);
                if (sub0 + 31 <= wave_horizon && sub0 + 32 <= args.keys)
                    softmax_and_mix(stage, Whole{}, sub, s, sub0);
                else
                    softmax_and_mix(stage, Masked{}, sub, s, sub0);
            }
        }
    };
    // The stage loop runs from barrier to barrier with both stages loading
    // at the top of every iteration (loads past the last key read zeros), so
    // the loads in flight are the same on every pass and each stage is
    // waited for by count: a stage's loads are done when only the other
    // stage's are still in flight.
    constexpr int kStageLoads = 2 * G::LOADS;
    issue(I0{}, 0, true);
    issue(I1{}, KEYS, true);
    for (int st = 0; st < stages_total; st += 2) {
        const int64_t key0 = int64_t(st) * KEYS;
        wait_loads<kStageLoads>();
        lds_barrier();
        compute(I0{}, key0);
        lds_barrier();
        issue(I0{}, key0 + 2 * KEYS, true);
        wait_loads<kStageLoads>();
        lds_barrier();
        if (st + 1 < stages_total) compute(I1{}, key0 + KEYS);
        lds_barrier();
        issue(I1{}, key0 + 3 * KEYS, true);
    }
    wait_loads<0>();  // the loads past the end land before the stages are reused

    // The row statistics the recomputing backward needs (both lanes of a query hold the same m, l).
    if (args.stats != nullptr && q < args.queries && half == 0)
        *reinterpret_cast<float2*>(args.stats + 2 * (head * args.queries + q)) = make_float2(m, l);
    // O = O^T / l: lane l holds h rows 32 b + 4 half + 8 (r / 4) + (r % 4) of its query.
    if (q < args.queries) {
        float* orow = args.o + (head * args.queries + q) * H;
#pragma unroll
        for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                f32x4 out;
#pragma unroll
                for (int s = 0; s < 4; ++s) out[s] = o[b][4 * g + s] / l;
                *reinterpret_cast<f32x4*>(orow + 32 * b + 4 * half + 8 * g) = out;
            }
    }
    if (args.p == nullptr) return;

    // Probabilities: a second pass over K with the final m and l; 0 past the diagonal.
    float* prow = args.p + (head * args.queries + q) * args.keys;
    const bool row_ok = q < args.queries;
    const bool vector_rows = (args.keys & 3) == 0;
    const float inv_l = 1.f / l;
    auto probabilities_of = [&](auto stage, int64_t key0) __attribute__((always_inline)) {
#pragma unroll
        for (int sub = 0; sub < SUBS; ++sub) {
            const int64_t sub0 = key0 + 32 * sub;
            if (sub0 >= args.keys) continue;
            f32x16 acc;
            if (sub0 < wave_keys) {
                acc = scores(stage, sub);
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[r] = 0.f;
            }
            const int limit = visible_limit(sub0);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float pv[4];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const float shifted = acc[4 * g + s] * args.scale - m;
                    pv[s] = key_of(4 * g + s) <= limit ? exp_of(shifted) * inv_l : 0.f;
                }
                const int64_t key = sub0 + 4 * half + 8 * g;
                if (row_ok) {
                    if (vector_rows && key + 4 <= args.keys) {
                        *reinterpret_cast<f32x4*>(prow + key) = f32x4{pv[0], pv[1], pv[2], pv[3]};
                    } else {
#pragma unroll
                        for (int s = 0; s < 4; ++s)
                            if (key + s < args.keys) prow[key + s] = pv[s];
                    }
                }
            }
        }
    };
    // The same stage loop over K alone. The probability stores are vector
    // memory operations too: each wait also covers the stores issued since,
    // which only makes it wait longer, never too little.
    issue(I0{}, 0, false);
    issue(I1{}, KEYS, false);
    for (int st = 0; st < stages_total; st += 2) {
        const int64_t key0 = int64_t(st) * KEYS;
        wait_loads<G::LOADS>();
        lds_barrier();
        probabilities_of(I0{}, key0);
        lds_barrier();
        issue(I0{}, key0 + 2 * KEYS, false);
        wait_loads<G::LOADS>();
        lds_barrier();
        if (st + 1 < stages_total) probabilities_of(I1{}, key0 + KEYS);
        lds_barrier();
        issue(I1{}, key0 + 3 * KEYS, false);
    }
    wait_loads<0>();
    // Keys past every query of the workgroup: zeros, each row filled by the
    // whole workgroup with contiguous stores.
    const int64_t zero_from = int64_t(stages_total) * KEYS;
    if (zero_from < args.keys) {
        const int64_t rows = min(int64_t(kQueries), args.queries - q_first);
        for (int64_t r = 0; r < rows; ++r) {
            float* zrow = args.p + (head * args.queries + q_first + r) * args.keys;
            if (vector_rows) {
                for (int64_t e = zero_from + 4 * tid; e < args.keys; e += 4 * 64 * kWaves)
                    *reinterpret_cast<f32x4*>(zrow + e) = f32x4{0.f, 0.f, 0.f, 0.f};
            } else {
                for (int64_t e = zero_from + tid; e < args.keys; e += 64 * kWaves) zrow[e] = 0.f;
            }
        }
    }
}

// The probability gradient of the same attention, fused: what the reference's
// backward (layers/attention.rs:238-248) computes with the dP product
// (MatmulSpec::new(T, T, h).right_transposed(): dP = dO V^T) and
// softmax_backward(P, dP) (kernels/attention.rs:185-207): dS = P * (dP -
// D) with D = sum over keys of dP * P per query, in one pass that never
// writes dP. D is taken as sum over h of dO * O (the same quantity, since O =
// P V), from the forward's output O. The layout is the forward's: a wave
// computes dP^T = V dO^T for 32 keys against its 32 queries (dO in
// registers), so lane l reads and writes its own query's row of P and dS.
// Keys past each query's horizon get 0, as P is 0 there.
struct ScoreGradArgs {
    const float* d_out;   // dO [heads][queries][h]
    const float* v;       // V [heads][keys][h], kv_stride apart
    const float* out;     // O [heads][queries][h]
    const float* p;       // P [heads][queries][keys]
    float* grad;          // dS, same layout as P
    const float* k;       // K [heads][keys][h], kv_stride apart (with q_grad)
    float* q_grad;        // null, or dQ = scale dS K [heads][queries][h]
    int64_t queries, keys;
    int64_t q_stride, kv_stride;
    int64_t query_offset;
    int64_t heads;
    int32_t query_blocks;
    float scale;
};

// PREFETCH (rows of P 16-byte aligned: keys a multiple of 4): each stage's P
// values are loaded with the stage, into one of two register sets, so that
// they are waited for by count with the stage's V; otherwise they are loaded
// where they are used.
// QGRAD: the query gradient of the backward's next call (attention.rs:250-253,
// MatmulSpec::new(T, h, T).scaled(scale): dQ = scale dS K) is accumulated too.
// Each lane's dS values are already the B operand of dQ^T += K^T dS^T (the
// forward's O^T += V^T P^T): K is staged beside V, unswizzled.
// Waves per SIMD the gradient kernel's registers are budgeted for where the
// compiler's own choice would leave one workgroup per CU although the LDS
// stages fit two (h = 64 with K staged: 264 -> 240 registers; h = 128
// without: 272 -> 256). A budget of three spills.
constexpr int score_grad_waves_per_simd(int h, bool qgrad) {
    return (h == 64 && qgrad) || (h == 128 && !qgrad) ? 2 : 1;
}

template <int H, bool PREFETCH, bool QGRAD>
__global__ __launch_bounds__(64 * kWaves)
__attribute__((amdgpu_waves_per_eu(score_grad_waves_per_simd(H, QGRAD), score_grad_waves_per_simd(H, QGRAD))))
void attention_score_grad_kernel(ScoreGradArgs args) {
#pragma clang fp contract(off)
    using G = Geometry<H>;
    constexpr int K_SLOTS = QGRAD ? G::STAGE_SLOTS : 1;
    __shared__ f32x4 v_stage0[G::STAGE_SLOTS], v_stage1[G::STAGE_SLOTS];
    __shared__ f32x4 k_stage0[K_SLOTS], k_stage1[K_SLOTS];
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    auto v_of = [&](auto stage) __attribute__((always_inline)) -> f32x4* {
        if constexpr (decltype(stage)::value == 0) return v_stage0;
        else return v_stage1;
    };
    auto k_of = [&](auto stage) __attribute__((always_inline)) -> f32x4* {
        if constexpr (decltype(stage)::value == 0) return k_stage0;
        else return k_stage1;
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31;
    const int half = lane >> 5;

    const int64_t block = blockIdx.x;
    const int64_t head = block % args.heads;
    const int64_t query_block = args.query_blocks - 1 - block / args.heads;
    const int64_t q_first = query_block * kQueries;
    const int64_t q_wave = q_first + 32 * wave;
    const int64_t q = q_wave + col;
    const int64_t wg_keys = min(args.keys, min(q_first + kQueries, args.queries) - 1 + args.query_offset + 1);
    const int64_t wave_keys = min(args.keys, q_wave + 31 + args.query_offset + 1);
    const int stages_total = int((wg_keys + kKeys - 1) / kKeys);
    const bool row_ok = q < args.queries;

    const __amdgpu_buffer_rsrc_t v_rsrc = buffer_of(args.v + head * args.kv_stride);
    const __amdgpu_buffer_rsrc_t k_rsrc = buffer_of(QGRAD ? args.k + head * args.kv_stride : args.v);

    // dO of this lane's query in registers (the forward's Q pattern) and D.
    float dreg[G::CHUNKS][8];
    float d_row;
    {
        const int64_t row = head * args.q_stride + (row_ok ? q : 0) * H;
        const int64_t out_row = (head * args.queries + (row_ok ? q : 0)) * H;
        float partial = 0.f;
#pragma unroll
        for (int c = 0; c < G::CHUNKS; ++c) {
            const f32x4 lo = *reinterpret_cast<const f32x4*>(args.d_out + row + 16 * c + 8 * half);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(args.d_out + row + 16 * c + 8 * half + 4);
            const f32x4 olo = *reinterpret_cast<const f32x4*>(args.out + out_row + 16 * c + 8 * half);
            const f32x4 ohi = *reinterpret_cast<const f32x4*>(args.out + out_row + 16 * c + 8 * half + 4);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                dreg[c][s] = row_ok ? lo[s] : 0.f;
                dreg[c][4 + s] = row_ok ? hi[s] : 0.f;
                const float a = dreg[c][s] * olo[s];
                partial = partial + a;
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const float a = dreg[c][4 + s] * ohi[s];
                partial = partial + a;
            }
        }
        d_row = partial + __shfl_xor(partial, 32);
    }

    auto issue = [&](auto stage, int64_t key0) __attribute__((always_inline)) {
        f32x4* vs = v_of(stage);
        f32x4* ks = k_of(stage);
#pragma unroll
        for (int u = 0; u < G::LOADS; ++u) {
            const int instr = wave * G::LOADS + u;
            const int e = 64 * instr + lane;
            const int row = e / G::SLOTS;
            const int slot = e % G::SLOTS;
            const int64_t key = key0 + row;
            const int chunk = slot ^ (row & G::SWIZZLE);
            dma16(v_rsrc, vs + 64 * instr, key < args.keys ? int32_t((key * H + 4 * chunk) * 4) : kOutOfRange);
            if constexpr (QGRAD)
                dma16(k_rsrc, ks + 64 * instr, key < args.keys ? int32_t((key * H + 4 * slot) * 4) : kOutOfRange);
        }
    };
    // dP^T for 32 keys (rows sub * 32 .. +31 of the stage) against this wave's queries.
    auto products = [&](auto stage, int sub) __attribute__((always_inline)) {
        const f32x4* vs = v_of(stage);
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
        const int row = 32 * sub + col;
        const int swz = row & G::SWIZZLE;
#pragma unroll
        for (int c = 0; c < G::CHUNKS; ++c) {
            const int g = 4 * c + 2 * half;
            const f32x4 lo = vs[row * G::SLOTS + (g ^ swz)];
            const f32x4 hi = vs[row * G::SLOTS + ((g + 1) ^ swz)];
            const float vv[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
            for (int s = 0; s < 8; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[s], dreg[c][s], acc, 0, 0, 0);
        }
        return acc;
    };

    const float* prow = args.p + (head * args.queries + q) * args.keys;
    float* grow = args.grad + (head * args.queries + q) * args.keys;
    const bool vector_rows = (args.keys & 3) == 0;
    // P of a stage for the prefetching form: 2 blocks x 4 groups of 4 keys.
    const __amdgpu_buffer_rsrc_t p_rsrc = buffer_of(args.p + head * args.queries * args.keys);
    auto load_p = [&](int64_t key0, f32x4 (&pr)[2][4]) __attribute__((always_inline)) {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int64_t key = key0 + 32 * sub + 4 * half + 8 * g;
                const int32_t off = row_ok && key < args.keys ? int32_t((q * args.keys + key) * 4) : kOutOfRange;
                pr[sub][g] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(p_rsrc, off, 0, 0));
            }
    };
    // dQ^T (rows h, column q) when QGRAD.
    f32x16 dq[QGRAD ? G::OBLOCKS : 1];
#pragma unroll
    for (int b = 0; b < (QGRAD ? G::OBLOCKS : 1); ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) dq[b][r] = 0.f;
    auto gradients_of = [&](auto stage, int64_t key0, const f32x4 (&pr)[2][4]) __attribute__((always_inline)) {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            const int64_t sub0 = key0 + 32 * sub;
            if (sub0 >= args.keys) continue;  // wave-uniform
            const bool computed = sub0 < wave_keys;  // wave-uniform
            f32x16 acc;
            if (computed) {
                acc = products(stage, sub);
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[r] = 0.f;
            }
            // dS of this lane's 16 keys (0 for a lane past the last query).
            float ds[16];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int64_t key = sub0 + 4 * half + 8 * g;
                float pv[4] = {0.f, 0.f, 0.f, 0.f};
                if constexpr (PREFETCH) {
#pragma unroll
                    for (int s = 0; s < 4; ++s) pv[s] = pr[sub][g][s];
                } else if (row_ok) {
                    if (vector_rows && key + 4 <= args.keys) {
                        const f32x4 x = *reinterpret_cast<const f32x4*>(prow + key);
#pragma unroll
                        for (int s = 0; s < 4; ++s) pv[s] = x[s];
                    } else {
#pragma unroll
                        for (int s = 0; s < 4; ++s) pv[s] = key + s < args.keys ? prow[key + s] : 0.f;
                    }
                }
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const bool visible = row_ok && key + s <= q + args.query_offset;
                    const float difference = acc[4 * g + s] - d_row;
                    ds[4 * g + s] = visible ? pv[s] * difference : 0.f;
                }
                if (row_ok) {
                    if (vector_rows && key + 4 <= args.keys) {
                        *reinterpret_cast<f32x4*>(grow + key) =
                            f32x4{ds[4 * g], ds[4 * g + 1], ds[4 * g + 2], ds[4 * g + 3]};
                    } else {
#pragma unroll
                        for (int s = 0; s < 4; ++s)
                            if (key + s < args.keys) grow[key + s] = ds[4 * g + s];
                    }
                }
            }
            if constexpr (QGRAD) {
                if (computed) {
                    // dQ^T rows 32 b .. +31 += K^T dS^T: MFMA t pairs keys key_of(t) of the two
                    // lane halves; lane l supplies K[key_of(t)][32 b + col].
                    const float* ks = reinterpret_cast<const float*>(k_of(stage));
#pragma unroll
                    for (int b = 0; b < G::OBLOCKS; ++b) {
                        const float* krow = ks + (32 * sub) * H + 32 * b + col;
#pragma unroll
                        for (int t = 0; t < 16; ++t) {
                            const int key = 4 * half + 8 * (t / 4) + (t % 4);
                            dq[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(krow[key * H], ds[t], dq[b], 0, 0, 0);
                        }
                    }
                }
            }
        }
    };
    // The forward's stage loop (both stages loading at the top of every pass;
    // loads past the last key read zeros), with each stage's P loaded beside
    // its V in the prefetching form. The dS stores (and P loads in the other
    // form) are vector memory operations too; a wait by count then only waits
    // longer.
    constexpr int kStageLoads = G::LOADS * (QGRAD ? 2 : 1) + (PREFETCH ? 8 : 0);
    f32x4 p0[2][4], p1[2][4];
    issue(I0{}, 0);
    if constexpr (PREFETCH) load_p(0, p0);
    issue(I1{}, kKeys);
    if constexpr (PREFETCH) load_p(kKeys, p1);
    for (int st = 0; st < stages_total; st += 2) {
        const int64_t key0 = int64_t(st) * kKeys;
        wait_loads<kStageLoads>();
        lds_barrier();
        gradients_of(I0{}, key0, p0);
        lds_barrier();
        issue(I0{}, key0 + 2 * kKeys);
        if constexpr (PREFETCH) load_p(key0 + 2 * kKeys, p0);
        wait_loads<kStageLoads>();
        lds_barrier();
        if (st + 1 < stages_total) gradients_of(I1{}, key0 + kKeys, p1);
        lds_barrier();
        issue(I1{}, key0 + 3 * kKeys);
        if constexpr (PREFETCH) load_p(key0 + 3 * kKeys, p1);
    }
    wait_loads<0>();
    if constexpr (QGRAD) {
        // dQ = scale (dS K): lane l holds h rows 32 b + 4 half + 8 g + (0..3) of its query.
        if (row_ok) {
            float* qrow = args.q_grad + (head * args.queries + q) * H;
#pragma unroll
            for (int b = 0; b < G::OBLOCKS; ++b)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    f32x4 out;
#pragma unroll
                    for (int s = 0; s < 4; ++s) out[s] = args.scale * dq[b][4 * g + s];
                    *reinterpret_cast<f32x4*>(qrow + 32 * b + 4 * half + 8 * g) = out;
                }
        }
    }
    // Keys past every query of the workgroup: zeros.
    const int64_t zero_from = int64_t(stages_total) * kKeys;
    if (zero_from < args.keys) {
        const int64_t rows = min(int64_t(kQueries), args.queries - q_first);
        for (int64_t r = 0; r < rows; ++r) {
            float* zrow = args.grad + (head * args.queries + q_first + r) * args.keys;
            if (vector_rows) {
                for (int64_t e = zero_from + 4 * tid; e < args.keys; e += 4 * 64 * kWaves)
                    *reinterpret_cast<f32x4*>(zrow + e) = f32x4{0.f, 0.f, 0.f, 0.f};
            } else {
                for (int64_t e = zero_from + tid; e < args.keys; e += 64 * kWaves) zrow[e] = 0.f;
            }
        }
    }
}

// Decode-shaped attention: a few queries per head (a decode step's one new
// position, or a handful) against a long run of cached keys, without the
// probabilities. The query-block kernel above would give each head one
// workgroup, reading the whole cache alone, with 31 of every 32 MFMA columns
// empty. Here the keys are split into 128-key chunks, one workgroup each:
//  * 256 threads; a key row of h floats is read by h / 4 lanes (16 bytes
//    each), so a pass covers 1024 / h rows and a chunk takes h / 16 passes,
//    every K and V load issued before the first use;
//  * a score is a lane's 4-term dot product summed over the row's lanes by
//    an xor butterfly (every lane ends with the same value), scaled and
//    masked as causal_softmax does; the chunk's maximum m_c, sum l_c of
//    e^(x - m_c) and partial O_c = sum of e^(x - m_c) V follow by the same
//    butterflies over the rows of a wave, then over the four waves through
//    LDS, in a fixed order;
//  * each chunk writes (O_c, m_c, l_c) per query to the workspace with
//    device-coherent stores, waits for them, and bumps its head's arrival
//    counter; the last chunk to arrive merges them, O = sum e^(m_c - m) O_c
//    / sum e^(m_c - m) l_c with m the largest m_c (kept as a running
//    maximum, the sums rescaled as it grows), all its threads folding chunks
//    in a fixed order, and resets the counter. Deterministic: no atomics on
//    data.
constexpr int kDecodeKeys = 128;    // keys per workgroup (64: 10.4 us, 32: 13.1 us at a full 1408 cache)
constexpr int kDecodeQueries = 4;   // most queries per head
constexpr int kDecodeThreads = 256;

template <int H>
struct DecodeGeometry {
    static constexpr int LANES = H / 4;                       // lanes per key row
    static constexpr int ROWS = kDecodeThreads / LANES;       // rows per pass
    static constexpr int PASSES = kDecodeKeys / ROWS;         // passes per chunk
    static constexpr int RECORD = H + 4;                      // floats per (chunk, query): O_c, m_c, l_c, pad
    static_assert(PASSES * ROWS == kDecodeKeys && LANES <= 64, "whole passes");
};

struct DecodeArgs {
    const float* q;
    const float* k;
    const float* v;
    float* o;
    float* ws;           // [heads][chunks][NQ][RECORD]
    uint32_t* counters;  // [heads], zero between calls
    int64_t queries, keys;
    int64_t q_stride, kv_stride;
    int64_t query_offset;
    int32_t chunks;
    float scale;
};

// NQ: queries per head the registers and records are laid out for (1, 2 or
// 4; the launch picks the least that holds a.queries).
template <int H, int NQ>
__global__ __launch_bounds__(kDecodeThreads) void decode_attention_kernel(DecodeArgs a) {
#pragma clang fp contract(off)
    using D = DecodeGeometry<H>;
    __shared__ float wave_values[4][NQ];
    __shared__ f32x4 wave_out[4][NQ][H / 4];
    __shared__ bool arrived_last;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int li = tid % D::LANES;    // 16-byte piece of the row
    const int slot = tid / D::LANES;  // row within a pass
    const int64_t head = blockIdx.y;
    const int chunk = blockIdx.x;
    const int64_t key0 = int64_t(chunk) * kDecodeKeys;
    const int nq = int(a.queries);

    const float* kh = a.k + head * a.kv_stride;
    const float* vh = a.v + head * a.kv_stride;
    const float* qh = a.q + head * a.q_stride;
    // Keys the last query sees: rows of the cache past them (an unwritten
    // tail, possibly NaN or Inf) are never read, since 0 * NaN would leak.
    const int64_t visible = min(a.keys, a.queries + a.query_offset);
    f32x4 kr[D::PASSES], vr[D::PASSES], qr[NQ];
#pragma unroll
    for (int i = 0; i < D::PASSES; ++i) {
        const int64_t key = key0 + i * D::ROWS + slot;
        const bool ok = key < visible;
        kr[i] = ok ? *reinterpret_cast<const f32x4*>(kh + key * H + 4 * li) : f32x4{0.f, 0.f, 0.f, 0.f};
        vr[i] = ok ? *reinterpret_cast<const f32x4*>(vh + key * H + 4 * li) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < NQ; ++j)
        qr[j] = j < nq ? *reinterpret_cast<const f32x4*>(qh + j * H + 4 * li) : f32x4{0.f, 0.f, 0.f, 0.f};

    // Scaled, masked scores; the chunk's maximum per query.
    float x[D::PASSES][NQ];
    float m_c[NQ];
#pragma unroll
    for (int j = 0; j < NQ; ++j) m_c[j] = -INFINITY;
#pragma unroll
    for (int i = 0; i < D::PASSES; ++i) {
        const int64_t key = key0 + i * D::ROWS + slot;
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
            float dot = kr[i][0] * qr[j][0];
#pragma unroll
            for (int e = 1; e < 4; ++e) dot = dot + kr[i][e] * qr[j][e];
#pragma unroll
            for (int o = 1; o < D::LANES; o <<= 1) dot = dot + __shfl_xor(dot, o);
            const bool visible = j < nq && key < a.keys && key <= j + a.query_offset;
            x[i][j] = visible ? dot * a.scale : -INFINITY;
            m_c[j] = fmaxf(m_c[j], x[i][j]);
        }
    }
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
#pragma unroll
        for (int o = D::LANES; o < 64; o <<= 1) m_c[j] = fmaxf(m_c[j], __shfl_xor(m_c[j], o));
        if (lane == 0) wave_values[wave][j] = m_c[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NQ; ++j)
        m_c[j] = fmaxf(fmaxf(wave_values[0][j], wave_values[1][j]), fmaxf(wave_values[2][j], wave_values[3][j]));
    __syncthreads();

    // e^(x - m_c), the chunk's sums and partial outputs (0 for a query that
    // sees none of the chunk's keys).
    float l_c[NQ];
    f32x4 o_c[NQ];
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
        l_c[j] = 0.f;
        o_c[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < D::PASSES; ++i) {
            const float e = m_c[j] == -INFINITY ? 0.f : exp_of(x[i][j] - m_c[j]);
            l_c[j] = l_c[j] + e;
#pragma unroll
            for (int d = 0; d < 4; ++d) o_c[j][d] = o_c[j][d] + e * vr[i][d];
        }
#pragma unroll
        for (int o = D::LANES; o < 64; o <<= 1) {
            l_c[j] = l_c[j] + __shfl_xor(l_c[j], o);
#pragma unroll
            for (int d = 0; d < 4; ++d) o_c[j][d] = o_c[j][d] + __shfl_xor(o_c[j][d], o);
        }
        if (lane == 0) wave_values[wave][j] = l_c[j];
        if (lane < D::LANES) wave_out[wave][j][li] = o_c[j];
    }
    __syncthreads();

    // One chunk: it is the whole answer, O = O_c / l_c.
    if (a.chunks == 1) {
        if (tid < nq * (H / 4)) {
            const int j = tid / (H / 4), piece = tid % (H / 4);
            const f32x4 sum = ((wave_out[0][j][piece] + wave_out[1][j][piece]) + wave_out[2][j][piece]) +
                              wave_out[3][j][piece];
            const float l_sum = ((wave_values[0][j] + wave_values[1][j]) + wave_values[2][j]) + wave_values[3][j];
            f32x4 out;
#pragma unroll
            for (int d = 0; d < 4; ++d) out[d] = sum[d] / l_sum;
            *reinterpret_cast<f32x4*>(a.o + (head * a.queries + j) * H + 4 * piece) = out;
        }
        return;
    }

    // This chunk's records, device-coherent: thread t writes query t / (h / 4),
    // 16-byte piece t % (h / 4) of O_c; thread j < NQ also m_c, l_c.
    const __amdgpu_buffer_rsrc_t mine = gemm::buffer_of(a.ws + (head * a.chunks + chunk) * NQ * D::RECORD);
    if (tid < NQ * (H / 4)) {
        const int j = tid / (H / 4), piece = tid % (H / 4);
        const f32x4 sum = ((wave_out[0][j][piece] + wave_out[1][j][piece]) + wave_out[2][j][piece]) +
                          wave_out[3][j][piece];
        gemm::buffer_store4_coherent(mine, int32_t((j * D::RECORD + 4 * piece) * 4), sum);
    }
    if (tid < NQ) {
        const float l_sum = ((wave_values[0][tid] + wave_values[1][tid]) + wave_values[2][tid]) + wave_values[3][tid];
        gemm::buffer_store4_coherent(mine, int32_t((tid * D::RECORD + H) * 4), f32x4{m_c[tid], l_sum, 0.f, 0.f});
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's record stores are complete device-wide
    __syncthreads();
    uint32_t* counter = a.counters + head;
    if (tid == 0)
        arrived_last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                       uint32_t(a.chunks - 1);
    __syncthreads();
    if (!arrived_last) return;

    // Last to arrive: merge the chunks. Thread group g (h / 4 threads, one
    // 16-byte piece of O each) folds chunks g, g + GROUPS, ... in order
    // (device-coherent loads, 8 chunks' records in flight at a time),
    // rescaling its running sums to each new maximum; group 0 then folds the
    // groups' results in group order. Deterministic. Every query sees key 0,
    // so group 0's maximum is finite from its first chunk on, and a group
    // with no chunk (or only chunks a query does not reach) contributes 0.
    constexpr int PIECES = H / 4;
    constexpr int GROUPS = kDecodeThreads / PIECES;
    constexpr int kBatch = 8;
    __shared__ f32x4 group_out[GROUPS][PIECES];
    __shared__ float group_m[GROUPS], group_l[GROUPS];
    const int piece = tid % PIECES, g = tid / PIECES;
    const __amdgpu_buffer_rsrc_t all = gemm::buffer_of(a.ws + head * a.chunks * NQ * D::RECORD);
    auto fold = [](float& m, float& l, f32x4& acc, float m_c, float l_c, const f32x4& part)
                    __attribute__((always_inline)) {
        const float m_new = fmaxf(m, m_c);
        if (m_new == -INFINITY) return;  // nothing seen yet on either side
        const float kept = exp_of(m - m_new);
        const float w = exp_of(m_c - m_new);
        l = l * kept + w * l_c;
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[d] = acc[d] * kept + w * part[d];
        m = m_new;
    };
    for (int j = 0; j < nq; ++j) {
        float m = -INFINITY, l = 0.f;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int c0 = g; c0 < a.chunks; c0 += kBatch * GROUPS) {
            f32x4 ml[kBatch], part[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int c = c0 + u * GROUPS;
                const bool ok = c < a.chunks;
                ml[u] = gemm::buffer_load4_coherent(all, ok ? int32_t(((c * NQ + j) * D::RECORD + H) * 4)
                                                            : gemm::kOutOfRange);
                part[u] = gemm::buffer_load4_coherent(all, ok ? int32_t(((c * NQ + j) * D::RECORD + 4 * piece) * 4)
                                                              : gemm::kOutOfRange);
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (c0 + u * GROUPS < a.chunks) fold(m, l, acc, ml[u][0], ml[u][1], part[u]);
        }
        group_out[g][piece] = acc;
        if (piece == 0) {
            group_m[g] = m;
            group_l[g] = l;
        }
        __syncthreads();
        if (g == 0) {
            float mm = -INFINITY, ll = 0.f;
            f32x4 total = {0.f, 0.f, 0.f, 0.f};
            for (int k = 0; k < GROUPS; ++k) fold(mm, ll, total, group_m[k], group_l[k], group_out[k][piece]);
            f32x4 out;
#pragma unroll
            for (int d = 0; d < 4; ++d) out[d] = total[d] / ll;
            *reinterpret_cast<f32x4*>(a.o + (head * a.queries + j) * H + 4 * piece) = out;
        }
        __syncthreads();
    }
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

namespace {

// Chunks of the decode form for `a`, or 0 when the query-block kernel runs:
// probabilities requested, more than kDecodeQueries queries, or no room for
// the records and counters.
int64_t decode_chunks(const CausalAttentionArgs& a) {
    if (a.p != nullptr || a.stats != nullptr || a.queries > kDecodeQueries || a.heads > 65535) return 0;
    const int64_t visible = std::min(a.keys, a.queries + a.query_offset);  // keys the last query sees
    const int64_t chunks = (visible + kDecodeKeys - 1) / kDecodeKeys;
    const int64_t record_bytes = int64_t(kDecodeQueries) * (a.head_dim + 4) * 4;
    if (chunks < 1 || chunks > 65535 || chunks * record_bytes >= gemm::kMaxBufferOffset) return 0;
    if (size_t(a.heads) > a.counter_count || a.counters == nullptr || a.workspace == nullptr ||
        size_t(a.heads * chunks * record_bytes) > a.workspace_bytes)
        return 0;
    return chunks;
}

}  // namespace

hipError_t launch_causal_attention(const CausalAttentionArgs& a, hipStream_t stream) {
    if (a.heads == 0 || a.queries == 0) return hipSuccess;
    if (const int64_t chunks = decode_chunks(a); chunks > 0) {
        DecodeArgs args;
        args.q = a.q;
        args.k = a.k;
        args.v = a.v;
        args.o = a.o;
        args.ws = a.workspace;
        args.counters = a.counters;
        args.queries = a.queries;
        args.keys = a.keys;
        args.q_stride = a.q_stride;
        args.kv_stride = a.kv_stride;
        args.query_offset = a.query_offset;
        args.chunks = int32_t(chunks);
        args.scale = a.scale;
        const dim3 grid(unsigned(chunks), unsigned(a.heads));
        auto launch = [&](auto h) {
            constexpr int H = decltype(h)::value;
            if (a.queries == 1)
                hipLaunchKernelGGL((decode_attention_kernel<H, 1>), grid, dim3(kDecodeThreads), 0, stream, args);
            else if (a.queries == 2)
                hipLaunchKernelGGL((decode_attention_kernel<H, 2>), grid, dim3(kDecodeThreads), 0, stream, args);
            else
                hipLaunchKernelGGL((decode_attention_kernel<H, 4>), grid, dim3(kDecodeThreads), 0, stream, args);
        };
        switch (a.head_dim) {
            case 32: launch(std::integral_constant<int, 32>{}); break;
            case 64: launch(std::integral_constant<int, 64>{}); break;
            case 128: launch(std::integral_constant<int, 128>{}); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    AttentionArgs args;
    args.q = a.q;
    args.k = a.k;
    args.v = a.v;
    args.o = a.o;
    args.p = a.p;
    args.stats = a.stats;
    args.queries = a.queries;
    args.keys = a.keys;
    args.q_stride = a.q_stride;
    args.kv_stride = a.kv_stride;
    args.query_offset = a.query_offset;
    args.heads = a.heads;
    args.query_blocks = int32_t((a.queries + kQueries - 1) / kQueries);
    args.scale = a.scale;
    const dim3 grid(unsigned(a.heads * args.query_blocks));
    switch (a.head_dim) {
        case 32: hipLaunchKernelGGL(causal_attention_kernel<32>, grid, dim3(64 * kWaves), 0, stream, args); break;
        case 64: hipLaunchKernelGGL(causal_attention_kernel<64>, grid, dim3(64 * kWaves), 0, stream, args); break;
        case 128: hipLaunchKernelGGL(causal_attention_kernel<128>, grid, dim3(64 * kWaves), 0, stream, args); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool causal_attention_supported(const CausalAttentionArgs& a) {
    const bool dims = a.head_dim == 32 || a.head_dim == 64 || a.head_dim == 128;
    const bool aligned = aligned16(a.q) && aligned16(a.k) && aligned16(a.v) && aligned16(a.o) &&
                         (a.p == nullptr || aligned16(a.p)) &&
                         (a.stats == nullptr || (reinterpret_cast<uintptr_t>(a.stats) & 7) == 0) &&
                         a.q_stride % 4 == 0 && a.kv_stride % 4 == 0;
    // Per-head buffer offsets (keys x h floats) within 31 bits; the grid within 32 bits.
    const bool offsets = a.keys * a.head_dim * 4 < (int64_t(1) << 31) - 4096;
    const int64_t query_blocks = (a.queries + kQueries - 1) / kQueries;
    const bool grid = a.heads * query_blocks < (int64_t(1) << 31);
    return dims && aligned && offsets && grid;
}

hipError_t launch_attention_score_grad(const AttentionScoreGradArgs& a, hipStream_t stream) {
    if (a.heads == 0 || a.queries == 0) return hipSuccess;
    ScoreGradArgs args;
    args.d_out = a.d_out;
    args.v = a.v;
    args.out = a.out;
    args.p = a.p;
    args.grad = a.grad;
    args.k = a.k;
    args.q_grad = a.q_grad;
    args.scale = a.scale;
    args.queries = a.queries;
    args.keys = a.keys;
    args.q_stride = a.q_stride;
    args.kv_stride = a.kv_stride;
    args.query_offset = a.query_offset;
    args.heads = a.heads;
    args.query_blocks = int32_t((a.queries + kQueries - 1) / kQueries);
    const dim3 grid(unsigned(a.heads * args.query_blocks));
    // Prefetching needs 16-byte P rows and a head's P within 31-bit offsets.
    const bool prefetch = a.keys % 4 == 0 && a.queries * a.keys * 4 < (int64_t(1) << 31) - 4096;
    auto launch_q = [&](auto h, auto pf, auto qg) {
        hipLaunchKernelGGL((attention_score_grad_kernel<decltype(h)::value, decltype(pf)::value, decltype(qg)::value>),
                           grid, dim3(64 * kWaves), 0, stream, args);
    };
    using T = std::true_type;
    using F = std::false_type;
    auto launch = [&](auto h, auto pf) {
        if (a.q_grad != nullptr) launch_q(h, pf, T{});
        else launch_q(h, pf, F{});
    };
    switch (a.head_dim) {
        case 32: prefetch ? launch(std::integral_constant<int, 32>{}, T{}) : launch(std::integral_constant<int, 32>{}, F{}); break;
        case 64: prefetch ? launch(std::integral_constant<int, 64>{}, T{}) : launch(std::integral_constant<int, 64>{}, F{}); break;
        case 128: prefetch ? launch(std::integral_constant<int, 128>{}, T{}) : launch(std::integral_constant<int, 128>{}, F{}); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool attention_score_grad_supported(const AttentionScoreGradArgs& a) {
    const bool dims = a.head_dim == 32 || a.head_dim == 64 || a.head_dim == 128;
    const bool aligned = aligned16(a.d_out) && aligned16(a.v) && aligned16(a.out) && aligned16(a.p) &&
                         aligned16(a.grad) && (a.q_grad == nullptr || (aligned16(a.q_grad) && aligned16(a.k))) &&
                         a.q_stride % 4 == 0 && a.kv_stride % 4 == 0;
    const bool offsets = a.keys * a.head_dim * 4 < (int64_t(1) << 31) - 4096;
    const int64_t query_blocks = (a.queries + kQueries - 1) / kQueries;
    const bool grid = a.heads * query_blocks < (int64_t(1) << 31);
    return dims && aligned && offsets && grid;
}

}  // namespace sn

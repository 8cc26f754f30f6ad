// Decode-shaped products: few output rows against a row-major weight.
//
// The reference's autoregressive step (crates/staleynet-model/src/decode.rs:
// 123-161, layers/attention.rs:274-320) issues every Linear with M = the
// number of new positions (1 in `generate`), i.e. y[M, N] = x[M, K] W[K, N]
// with W row-major [K, N] (linear.rs:20-28). At M <= 16 a 128x128 matrix-core
// tile would leave most of its rows idle; the product is bound by reading W
// once from HBM, so this kernel streams W and is judged against 8 TB/s.
//
// Design (one launch). Reads, not arithmetic, set the time, and an MI355X CU
// sustains only about 16 GB/s of loads (its outstanding misses over the
// memory latency), so the first rule is to keep every CU streaming:
//  * A workgroup of 4 waves (8 on the matrix-core path) owns a slab of 64
//    columns; a lane owns 4
//    consecutive columns, 16 lanes read one 256-byte row piece and one wave
//    load covers 4 rows. A single row of x against a weight that K is split
//    for takes 32-column slabs instead (8 lanes per 128-byte piece, 8 rows
//    per wave load): twice the workgroups per slice. A pass is 16 (8 for 3-4 rows of x) 16-byte
//    loads in flight per lane, rows dealt to the waves in groups of 4; the
//    next pass's loads are issued before the current one is multiplied (two
//    register sets, loads issued unconditionally so that the compiler's
//    wait counts stay exact).
//  * x's rows of the pass are staged in LDS (double-buffered with the passes)
//    and read as broadcasts. A pass's x loads are issued before its W loads:
//    load counters complete in order, so writing x to LDS then never waits
//    for W.
//  * Up to 4 rows of x: FMAs on the VALU, then the partial sums of a wave's
//    row lanes are added with cross-lane moves. 5 to 16 rows: each wave load
//    of W (4 rows x 64 columns) feeds four v_mfma_f32_16x16x4f32, one per
//    column of a lane's 4, with x's 4 rows as the A operand; the matrix core
//    sums the 4 rows. Then the waves' partial sums are added in wave order
//    through LDS: a fixed order.
//  * With a slab per CU or more (the 16-codebook head: 256 slabs), each slab
//    streams the whole of K. Narrower weights (768 to 3072 columns: 12 to 48
//    slabs) split K into slices of whole 16-row groups, for 128-192
//    workgroups. Every slice but the last of a slab writes its partial sums
//    into zeroed slots with device-coherent stores (agent scope: written
//    through to where every XCD reads them) and ends. The last slice, the
//    slab's highest workgroup id and so the last dispatched, polls the slots
//    with device-coherent loads until all are written, adds them in slice
//    order with its own, applies the reference's combine and zeroes the
//    slots. The summation order is fixed, no L2 write-back or invalidate (a
//    cost of ~100 us per launch here) is needed, and the hand-off costs one
//    store's flight and one polling round trip. (An arrival counter, read
//    by whichever slice finishes last, cost a store acknowledgement, an
//    atomic and a load round trip: about half of a layer product's time.)
//    The grid is far smaller than what the device holds at once, so every
//    slice a last slice waits for is resident or done; the polling still
//    ends at a deadline, so every wave exits whatever happens.
#include "gemm_common.h"

namespace sn {
namespace {

using gemm::f32x4;

// Waves per workgroup: 4 on the VALU paths (one per SIMD), 8 on the
// matrix-core path, whose MFMAs (a quarter of a pass's time at 16 rows) then
// run on one wave of a SIMD while the other waits for its loads.
template <int MT>
constexpr int waves_for();
constexpr int kMaxRows = 16;
// Cache policy of the W loads: non-temporal (each weight byte is read once
// per launch). A streaming-read probe on MI355X reaches 6.5 TB/s with it and
// 5.9 TB/s without; here it is worth 3-7 % per product.
constexpr int32_t kNontemporal = 2;
// Slabs (times batches) from which K is never split: one per CU. Below
// that, reads need more CUs than slabs: an MI355X CU sustains only about
// 16 GB/s of loads (its outstanding misses over the memory latency), so a
// 768-wide weight streamed by 12 slabs would take 4x longer than its split
// hand-off costs.
constexpr int kUnsplitSlabs = 256;
// Workgroups a split plan aims for. Each slice adds a partial sum to write
// and read back, so fewer than one per CU: measured on the c4 layer weights,
// 128 (M <= 4) and 192 (M = 16) beat both 48 and 512.
constexpr int kSplitTargetFewRows = 128;
constexpr int kSplitTargetFewRowsNarrow = 96;
constexpr int kNarrowSlabs = 16;
constexpr int kSplitTargetManyRows = 192;
constexpr int kMinSliceGroups = 8;
// One row of x against one weight that K gets split for (the layer products
// of a decode step): 32-column slabs, 8 lanes per 128-byte row piece, so
// twice the workgroups stream a slice of the same length. On the c4 layer
// weights at M = 1 (graph replay) the products took 4.9 / 5.6 / 6.2 / 6.8 us
// (out / qkv / up / down) against 5.3 / 6.2 / 6.4 / 7.6 with 64 columns;
// 16-column slabs were slower for each. Split from fewer than 96 such slabs
// (the 3072-wide up product, 96 slabs, took 6.2 us whole against 6.4 in two
// slices) into slices for about 192 workgroups.
constexpr int kNarrowLanes = 8;
constexpr int kUnsplitNarrowSlabs = 96;
constexpr int kSplitTargetNarrow = 192;

// Rows of x from which the products go to the matrix cores: 16 output rows
// cost one v_mfma_f32_16x16x4f32 per 4 rows x 16 columns of W, where the
// VALU would spend 16 FMAs per W value and hold 16 accumulators per column.
template <int MT>
constexpr bool uses_mfma() { return MT >= 8; }

// Loads in flight per lane (measured on the c4 weights): for one or two rows
// of x, 16 when a slab streams the whole of K (the head) and 8 when K is split
// into slices of a few hundred rows (the layer weights, 2-9 % over 16); 8 for
// four rows, whose x values and accumulators need the registers (two waves
// per SIMD throughout; 4 lost up to 8 %). On the matrix cores (8 waves)
// shorter passes did better still: 4 loads for a whole K (the head: 4.1 TB/s
// against 3.7 with 8), 2 for slices (3-7 % over 4; the head lost 12 % with 2).
template <int MT>
constexpr int loads_for(bool split) {
    return MT <= 2 ? (split ? 8 : 16) : !uses_mfma<MT>() ? 8 : split ? 2 : 4;
}
template <int MT>
constexpr int waves_for() { return uses_mfma<MT>() ? 8 : 4; }
// Rows of W one pass covers: waves x loads x rows per wave load.
template <int MT, int LPR, int LOADS>
constexpr int pass_rows() { return waves_for<MT>() * LOADS * (64 / LPR); }

// The hand-off's encoding of a partial sum in a slot word: the bitwise NOT
// of its bits, with every NaN first made the canonical quiet NaN. The only
// bits that encode to 0 (an empty slot) are 0xFFFFFFFF, a NaN, which never
// gets stored, so an empty slot and a written one cannot be confused. (The
// whole vector is reinterpreted at once: clang's __builtin_bit_cast of an
// ext_vector element reads element 0, whatever the subscript.)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4 handoff_encode(f32x4 v) {
    u32x4 bits = __builtin_bit_cast(u32x4, v);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float x = v[j];
        if (x != x) bits[j] = 0x7FC00000u;
    }
    return __builtin_bit_cast(f32x4, ~bits);
}
__device__ __forceinline__ bool handoff_filled(f32x4 v) {
    const u32x4 bits = __builtin_bit_cast(u32x4, v);
    return bits[0] != 0u && bits[1] != 0u && bits[2] != 0u && bits[3] != 0u;
}
__device__ __forceinline__ f32x4 handoff_decode(f32x4 v) { return __builtin_bit_cast(f32x4, ~__builtin_bit_cast(u32x4, v)); }
// Slices polled per batch of loads, and the polling deadline in ticks of
// the 100 MHz clock s_memrealtime reads (0.5 s).
constexpr int kHandoffBatch = 16;
constexpr uint64_t kHandoffDeadlineTicks = 50000000ull;

struct GemvArgs {
    const float* x;
    const float* w;
    float* y;
    uint32_t* handoff;  // zero-initialized slots, (splits - 1) x m x 64 words per column block and batch
    int64_t m, n, k;
    int64_t k_limit;       // keys actually multiplied: k, or the last row's horizon + 1 (causal left)
    int64_t query_offset;  // causal left: x[m][k] counts only for k <= m + query_offset
    int32_t causal_left;
    int64_t stride_x, stride_w, stride_y;
    int64_t k_per_split;
    int32_t column_blocks;
    int32_t splits;
    int32_t accumulate;
    float scale;
    const float* bias;  // null, or Linear's bias added after the combine
};

// MT: rows of x the instantiation holds; LPR: lanes per row piece (the slab
// is 4 * LPR columns wide); LOADS: loads in flight per lane (loads_for).
template <int MT, int LPR, int LOADS>
__global__ __launch_bounds__(64 * waves_for<MT>()) void gemv_kernel(GemvArgs args) {
    constexpr int kWaves = waves_for<MT>();
    constexpr int kThreads = 64 * kWaves;
    constexpr int kLoads = LOADS;
    constexpr int kRowsPerLoad = 64 / LPR;
    constexpr int kColumns = 4 * LPR;
    constexpr int kPassRows = pass_rows<MT, LPR, LOADS>();
    // x of a pass as [row][m], rows kXStride floats apart: an odd stride (for
    // two or more rows of x) puts the consecutive rows that a wave's lanes
    // write on distinct banks.
    constexpr int kXStride = MT == 1 ? 1 : MT + 1;
    __shared__ __attribute__((aligned(16))) float x_pass[2][kPassRows][kXStride];
    __shared__ f32x4 partial[kWaves][MT][LPR];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int row_lane = lane / LPR;  // which row of a wave load
    const int col_lane = lane % LPR;
    const int split = blockIdx.y;
    const int64_t batch = blockIdx.z;
    const int64_t n0 = int64_t(blockIdx.x) * kColumns;
    const int64_t k_begin = int64_t(split) * args.k_per_split;
    const int64_t k_end = min(args.k_limit, k_begin + args.k_per_split);
    const int passes = int((k_end - k_begin + kPassRows - 1) / kPassRows);

    const float* x = args.x + batch * args.stride_x;
    const float* w = args.w + batch * args.stride_w;
    const bool col_ok = n0 + 4 * col_lane < args.n;
    const int32_t lane_offset = col_ok ? int32_t((int64_t(row_lane) * args.n + 4 * col_lane) * 4) : gemm::kOutOfRange;
    // Rows of a pass are dealt to the waves in groups of kRowsPerLoad:
    // load u of wave v reads rows (kWaves u + v) * kRowsPerLoad + row_lane, so a
    // short slice still spreads over all four waves. Wave-uniform: this
    // wave's first row and the byte distance between a lane's loads.
    const int32_t wave_row = __builtin_amdgcn_readfirstlane(wave) * kRowsPerLoad;
    const int32_t wave_offset = int32_t(int64_t(wave_row) * args.n * 4);
    const int32_t load_stride = int32_t(int64_t(kWaves * kRowsPerLoad) * args.n * 4);

    // Loads of one pass: one descriptor per pass and a scalar offset per
    // load; rows past the slice read 0 (only the last pass of a slice can
    // have any).
    auto load_pass = [&](int64_t k0, f32x4 (&rows)[kLoads]) {
        const __amdgpu_buffer_rsrc_t rsrc = gemm::buffer_of(w + k0 * args.n + n0);
        const bool full = k0 + kPassRows <= k_end;
#pragma unroll
        for (int u = 0; u < kLoads; ++u) {
            const int32_t voffset =
                full || k0 + kWaves * kRowsPerLoad * u + wave_row + row_lane < k_end ? lane_offset : gemm::kOutOfRange;
            rows[u] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voffset, u * load_stride + wave_offset, kNontemporal));
        }
    };
    // x values of a pass: each thread loads kXPerThread of them into
    // registers (issued before that pass's W loads, so that waiting for them
    // never waits for W) and later writes them to the pass's LDS buffer.
    // Branch-free buffer loads: values past the slice or past M read 0.
    // Element e of the pass is row e % kPassRows of x's row e / kPassRows, so
    // a wave's lanes read 64 consecutive k of one row of x (256 contiguous
    // bytes; with the row index fastest a wave load touched up to 64 lines).
    // A pass of fewer x values than threads leaves the last threads idle.
    constexpr int kXElems = kPassRows * MT;
    constexpr int kXPerThread = (kXElems + kThreads - 1) / kThreads;
    static_assert(kPassRows % 64 == 0, "a wave's x lanes stay within one row of x");
    auto x_in_pass = [&](int e) { return kXElems % kThreads == 0 || e < kXElems; };
    const __amdgpu_buffer_rsrc_t x_rsrc = gemm::buffer_of(x);
    auto load_x = [&](int64_t k0, float (&xs)[kXPerThread]) {
#pragma unroll
        for (int i = 0; i < kXPerThread; ++i) {
            const int e = tid + i * kThreads;
            const int r = e % kPassRows;
            const int m = e / kPassRows;
            // Causal left: the stored left matrix is 0 past row m's horizon
            // (the tiled kernels zero it in LDS the same way).
            const bool ok = x_in_pass(e) && m < args.m && k0 + r < k_end &&
                            (!args.causal_left || k0 + r <= m + args.query_offset);
            xs[i] = gemm::buffer_load1(x_rsrc, ok ? int32_t((m * args.k + k0 + r) * 4) : gemm::kOutOfRange);
        }
    };
    auto store_x = [&](const float (&xs)[kXPerThread], int buf) {
#pragma unroll
        for (int i = 0; i < kXPerThread; ++i) {
            const int e = tid + i * kThreads;
            if (x_in_pass(e)) x_pass[buf][e % kPassRows][e / kPassRows] = xs[i];
        }
    };

    f32x4 acc[uses_mfma<MT>() ? 1 : MT];
#pragma unroll
    for (int m = 0; m < (uses_mfma<MT>() ? 1 : MT); ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Matrix-core accumulators: macc[c][r] = row 4 * (lane / 16) + r, column
    // n0 + 4 * (lane % 16) + c of this wave's partial sum.
    f32x4 macc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) macc[c] = f32x4{0.f, 0.f, 0.f, 0.f};

    // One pass: start the next pass's x and W loads, then (after the barrier
    // that publishes this pass's x and retires the other x buffer) multiply
    // this pass, x values read one load ahead, and stage the next pass's x.
    auto pass = [&](int p, const f32x4 (&cur)[kLoads], f32x4 (&next)[kLoads]) {
        const int64_t k0 = k_begin + int64_t(p) * kPassRows;
        // Unconditional: past the last pass every load is out of range and
        // fetches nothing. (Skipping them on a branch would make the compiler
        // assume, where the paths join, that this pass's W loads are the most
        // recent, and wait for the next pass's loads before multiplying.)
        float xs[kXPerThread];
        load_x(k0 + kPassRows, xs);
        load_pass(k0 + kPassRows, next);
        __syncthreads();
        const float* xr = x_pass[p & 1][wave_row + row_lane];
        if constexpr (uses_mfma<MT>()) {
            // Load u holds W rows r .. r + 3 (r its first row, lane / 16 =
            // row_lane picks one) and 64 columns, 4 per lane. For component
            // c, lane l supplies B[k = l / 16][j = l % 16] = W[r + k][n0 +
            // 4j + c]; the A operand is x[m = l % 16][r + l / 16] (0 past
            // MT). One MFMA per component adds those 4 rows into the 16 x 16
            // block of columns n0 + 4j + c.
            float xa[kLoads];
#pragma unroll
            for (int u = 0; u < kLoads; ++u)
                xa[u] = (lane & 15) < MT ? xr[u * kWaves * kRowsPerLoad * kXStride + (lane & 15)] : 0.f;
#pragma unroll
            for (int u = 0; u < kLoads; ++u)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    macc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[u], cur[u][c], macc[c], 0, 0, 0);
        } else {
            float xv[MT], xn[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) xv[m] = xr[m];
#pragma unroll
            for (int u = 0; u < kLoads; ++u) {
                if (u + 1 < kLoads) {
#pragma unroll
                    for (int m = 0; m < MT; ++m) xn[m] = xr[(u + 1) * kWaves * kRowsPerLoad * kXStride + m];
                }
#pragma unroll
                for (int m = 0; m < MT; ++m) acc[m] += xv[m] * cur[u];
#pragma unroll
                for (int m = 0; m < MT; ++m) xv[m] = xn[m];
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        store_x(xs, (p + 1) & 1);
    };

    f32x4 ra[kLoads], rb[kLoads];
    {
        float xs[kXPerThread];
        load_x(k_begin, xs);
        load_pass(k_begin, ra);
        store_x(xs, 0);
    }
    for (int p = 0; p < passes; p += 2) {
        pass(p, ra, rb);
        if (p + 1 < passes) pass(p + 1, rb, ra);
    }

    if constexpr (uses_mfma<MT>()) {
        // Lane l holds rows 4 (l / 16) .. +3 of columns 4 (l % 16) .. +3
        // (col_lane = l % 16, as LPR = 16 here).
        static_assert(LPR == 16, "16 lanes per 64-column row piece");
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * row_lane + r;
            if (m < MT) partial[wave][m][col_lane] = f32x4{macc[0][r], macc[1][r], macc[2][r], macc[3][r]};
        }
    } else {
        // The row lanes of a wave hold the same columns: add them (xor LPR,
        // 2 LPR, .. 32), then the waves in order through LDS.
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float v = acc[m][j];
#pragma unroll
                for (int step = LPR; step < 64; step *= 2) v += __shfl_xor(v, step);
                acc[m][j] = v;
            }
        if (row_lane == 0) {
#pragma unroll
            for (int m = 0; m < MT; ++m) partial[wave][m][col_lane] = acc[m];
        }
    }
    __syncthreads();

    // One thread per (m, column group): the wave-ordered sum of the slab.
    const int om = tid / LPR;
    const int oc = tid % LPR;
    const bool owner = tid < MT * LPR;
    f32x4 slab_sum = {0.f, 0.f, 0.f, 0.f};
    if (owner) {
        slab_sum = partial[0][om][oc];
#pragma unroll
        for (int v = 1; v < kWaves; ++v) slab_sum += partial[v][om][oc];
    }
    const int64_t out_col = n0 + 4 * oc;
    const bool out_ok = owner && om < args.m && out_col < args.n;

    if (args.splits == 1) {
        if (out_ok) {
            float* dst = args.y + batch * args.stride_y + om * args.n + out_col;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                gemm::write_output(dst + j, slab_sum[j], args.scale, args.accumulate != 0, args.bias, out_col + j);
        }
        return;
    }

    // Split K: the slices hand their partial sums to the column block's last
    // slice, the highest workgroup id of the block (so the last dispatched,
    // after every slice it waits for). Slots are M x (slab width) words per slice,
    // zero between calls; a slice writes its encoded partials device-
    // coherently and ends, and the last slice polls them (device-coherent
    // loads) until every word is non-zero, adds them in slice order with its
    // own last, applies the combine and clears the slots. One one-way store
    // and one polling round trip, where an arrival counter costs a store
    // acknowledgement, an atomic and a load round trip.
    const int last = args.splits - 1;
    const int64_t slice_words = args.m * kColumns;
    uint32_t* slots = args.handoff + (batch * args.column_blocks + blockIdx.x) * int64_t(last) * slice_words;
    const int32_t chunk = int32_t((om * kColumns + 4 * oc) * 4);  // this owner's 16 bytes within a slice's slot
    if (split < last) {
        if (owner && om < args.m)  // every column of the slab, zeros past n: each slot word gets written
            gemm::buffer_store4_coherent(gemm::buffer_of(reinterpret_cast<float*>(slots + split * slice_words)), chunk,
                                         handoff_encode(slab_sum));
        return;
    }
    if (!(owner && om < args.m)) return;
    const __amdgpu_buffer_rsrc_t all = gemm::buffer_of(reinterpret_cast<float*>(slots));
    const int32_t slice_bytes = int32_t(slice_words * 4);
    // Polling ends at a deadline (0.5 s of the 100 MHz real-time clock, far
    // past any slice's arrival) so that every wave exits whatever happens; a
    // slot still empty then reads as a NaN partial.
    const uint64_t deadline = __builtin_amdgcn_s_memrealtime() + kHandoffDeadlineTicks;
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < last; s0 += kHandoffBatch) {
        f32x4 part[kHandoffBatch];
        uint32_t pending = 0;
#pragma unroll
        for (int u = 0; u < kHandoffBatch; ++u) {
            part[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (s0 + u < last) pending |= 1u << u;
        }
        while (pending != 0) {
            // Every pending slot's load in flight at once, then the checks.
            f32x4 got[kHandoffBatch];
#pragma unroll
            for (int u = 0; u < kHandoffBatch; ++u)
                got[u] = gemm::buffer_load4_coherent(
                    all, (pending >> u) & 1u ? (s0 + u) * slice_bytes + chunk : gemm::kOutOfRange);
#pragma unroll
            for (int u = 0; u < kHandoffBatch; ++u) {
                if (((pending >> u) & 1u) && handoff_filled(got[u])) {
                    part[u] = got[u];
                    pending &= ~(1u << u);
                }
            }
            if (pending != 0 && __builtin_amdgcn_s_memrealtime() > deadline) break;
        }
#pragma unroll
        for (int u = 0; u < kHandoffBatch; ++u) {
            if (s0 + u < last) {
                sum += handoff_decode(part[u]);
                gemm::buffer_store4_coherent(all, (s0 + u) * slice_bytes + chunk, f32x4{0.f, 0.f, 0.f, 0.f});
            }
        }
    }
    sum += slab_sum;
    if (out_ok) {
        float* dst = args.y + batch * args.stride_y + om * args.n + out_col;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            gemm::write_output(dst + j, sum[j], args.scale, args.accumulate != 0, args.bias, out_col + j);
    }
}

struct GemvPlan {
    int lanes_per_row;  // lanes per row piece: 16 (64-column slabs) or kNarrowLanes
    int narrow_loads;   // loads in flight per lane on the 32-column slabs
    int column_blocks;
    int splits;
    int64_t k_per_split;
    int64_t pass_rows;
};

// Rows of a pass for the instantiation launch_width picks for m rows.
template <int LPR>
int64_t pass_rows_for(int64_t m, bool split) {
    if (m <= 2) return split ? pass_rows<2, LPR, loads_for<2>(true)>() : pass_rows<2, LPR, loads_for<2>(false)>();
    if (m <= 4) return pass_rows<4, LPR, loads_for<4>(false)>();
    if (m <= 8)
        return split ? pass_rows<8, LPR, loads_for<8>(true)>() : pass_rows<8, LPR, loads_for<8>(false)>();
    return split ? pass_rows<16, LPR, loads_for<16>(true)>() : pass_rows<16, LPR, loads_for<16>(false)>();
}

// Keys a product multiplies: all K, or with a causal left mask up to the last
// row's horizon (the left matrix is 0 past it, and the right operand's rows
// there, such as an unwritten cache tail, are not read).
int64_t keys_used(const Problem& p) {
    if (p.mask != SN_MASK_CAUSAL_LEFT) return p.k;
    return std::max<int64_t>(1, std::min(p.k, p.m - 1 + p.query_offset + 1));
}

GemvPlan gemv_plan(const Problem& p) {
    const int64_t k = keys_used(p);
    GemvPlan plan;
    plan.lanes_per_row = 16;
    plan.column_blocks = int((p.n + 63) / 64);
    if (p.m == 1 && p.batch == 1 && plan.column_blocks < kUnsplitSlabs) {
        plan.lanes_per_row = kNarrowLanes;
        plan.column_blocks = int((p.n + 4 * kNarrowLanes - 1) / (4 * kNarrowLanes));
    }
    const bool narrow = plan.lanes_per_row == kNarrowLanes;
    const int64_t slabs = int64_t(plan.column_blocks) * p.batch;
    int64_t rows_per_split = std::max<int64_t>(k, 1);
    if (slabs < (narrow ? kUnsplitNarrowSlabs : kUnsplitSlabs)) {
        // Enough slices for about `target` workgroups, each a whole
        // number of 16-row groups (4 waves x 4 rows; on the 8-wave path a
        // slice's last group may leave waves idle).
        const int64_t groups = (std::max<int64_t>(k, 1) + 15) / 16;
        // Narrow weights (16 column blocks or fewer: the 768-wide out and down
        // products) do better with fewer, longer slices when there are few rows.
        const int64_t target = narrow ? kSplitTargetNarrow
                               : p.m > 4 ? kSplitTargetManyRows
                               : slabs <= kNarrowSlabs ? kSplitTargetFewRowsNarrow : kSplitTargetFewRows;
        // Slices of at least 8 groups (128 rows): the 768-deep out product
        // took 5-11 % less time in 6 slices than in 8 (M = 1) or 16 (M = 16).
        const int64_t want =
            std::max<int64_t>(1, std::min<int64_t>(groups / kMinSliceGroups, (target + slabs - 1) / slabs));
        rows_per_split = 16 * ((groups + want - 1) / want);
    }
    plan.k_per_split = rows_per_split;
    plan.splits = int((std::max<int64_t>(k, 1) + rows_per_split - 1) / rows_per_split);
    // A pass no longer than a slice: 8 loads (256 rows) from 256-row slices,
    // else 4 (the 128-row slices of the out product: 4.9 us against 5.1+).
    plan.narrow_loads = rows_per_split >= 256 ? 8 : 4;
    plan.pass_rows = !narrow                  ? pass_rows_for<16>(p.m, plan.splits > 1)
                     : plan.narrow_loads == 8 ? pass_rows<1, kNarrowLanes, 8>()
                                              : pass_rows<1, kNarrowLanes, 4>();
    return plan;
}

size_t handoff_words(const Problem& p, const GemvPlan& plan) {
    return size_t(p.batch) * size_t(plan.column_blocks) * size_t(plan.splits - 1) * size_t(p.m) * 4 *
           size_t(plan.lanes_per_row);
}

template <int MT, int LPR, int LOADS>
hipError_t launch_rows(const Problem& p, const Env& env, const GemvPlan& plan, hipStream_t stream) {
    GemvArgs args;
    args.x = p.a;
    args.w = p.b;
    args.y = p.c;
    args.handoff = env.handoff;
    args.m = p.m;
    args.n = p.n;
    args.k = p.k;
    args.k_limit = keys_used(p);
    args.query_offset = p.query_offset;
    args.causal_left = p.mask == SN_MASK_CAUSAL_LEFT ? 1 : 0;
    args.stride_x = p.stride_a;
    args.stride_w = p.stride_b;
    args.stride_y = p.stride_c;
    args.k_per_split = plan.k_per_split;
    args.column_blocks = plan.column_blocks;
    args.splits = plan.splits;
    args.accumulate = p.accumulate ? 1 : 0;
    args.scale = p.scale;
    args.bias = p.bias;
    hipLaunchKernelGGL((gemv_kernel<MT, LPR, LOADS>), dim3(plan.column_blocks, plan.splits, unsigned(p.batch)),
                       dim3(64 * waves_for<MT>()), 0, stream, args);
    return hipGetLastError();
}

template <int LPR>
hipError_t launch_width(const Problem& p, const Env& env, const GemvPlan& plan, hipStream_t stream) {
    const bool split = plan.splits > 1;
    if (p.m == 1)
        return split ? launch_rows<1, LPR, loads_for<1>(true)>(p, env, plan, stream)
                     : launch_rows<1, LPR, loads_for<1>(false)>(p, env, plan, stream);
    if (p.m <= 2)
        return split ? launch_rows<2, LPR, loads_for<2>(true)>(p, env, plan, stream)
                     : launch_rows<2, LPR, loads_for<2>(false)>(p, env, plan, stream);
    if (p.m <= 4) return launch_rows<4, LPR, loads_for<4>(false)>(p, env, plan, stream);
    if (p.m <= 8)
        return split ? launch_rows<8, LPR, loads_for<8>(true)>(p, env, plan, stream)
                     : launch_rows<8, LPR, loads_for<8>(false)>(p, env, plan, stream);
    return split ? launch_rows<16, LPR, loads_for<16>(true)>(p, env, plan, stream)
                 : launch_rows<16, LPR, loads_for<16>(false)>(p, env, plan, stream);
}

// Few-row products against a K-contiguous right operand (right_transposed):
// the decode step's attention scores against the cache (attention.rs:307-310,
// MatmulSpec::new(n, capacity, h).right_transposed()), where each output is
// the dot product of one of x's rows with one of B's rows. The tiled kernels
// would spend a 128x128 tile per 128 keys on a single row. Here 16 lanes read
// a row of B 16 bytes at a time (a 256-thread workgroup covers 64 rows of B
// in 4 passes), each lane keeps 4-term dot products per row of x, and an xor
// butterfly over the 16 lanes sums them. Outputs past a causal mask's
// horizon are written 0 (or left alone when accumulating); rows of B past
// the last row's horizon are not read.
constexpr int kNtRows = 64;      // rows of B per workgroup
constexpr int kNtMaxRows = 4;    // rows of x

struct GemvNtArgs {
    const float* x;  // [m][k], rows k floats apart
    const float* w;  // B stored [n][k], rows ldb floats apart
    float* y;        // [m][n]
    int64_t m, n, k, ldb;
    int64_t n_limit;  // rows of B any output needs (n, or the last row's horizon + 1 under the mask)
    int64_t stride_x, stride_w, stride_y;
    int64_t query_offset;
    int32_t causal;
    int32_t accumulate;
    float scale;
};

template <int MT>
__global__ __launch_bounds__(256) void gemv_nt_kernel(GemvNtArgs a) {
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const int li = tid % 16;    // 16-byte piece of a row
    const int slot = tid / 16;  // row of B within a pass
    const int64_t batch = blockIdx.y;
    const int64_t n_base = int64_t(blockIdx.x) * kNtRows;
    const float* x = a.x + batch * a.stride_x;
    const float* w = a.w + batch * a.stride_w;
    float* y = a.y + batch * a.stride_y;
    float acc[4][MT];
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int j = 0; j < MT; ++j) acc[p][j] = 0.f;
    for (int64_t k0 = 4 * li; k0 < a.k; k0 += 64) {
        f32x4 xv[MT];
#pragma unroll
        for (int j = 0; j < MT; ++j)
            xv[j] = j < a.m ? *reinterpret_cast<const f32x4*>(x + j * a.k + k0) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int64_t row = n_base + 16 * p + slot;
            if (row < a.n_limit) {
                const f32x4 bv = *reinterpret_cast<const f32x4*>(w + row * a.ldb + k0);
#pragma unroll
                for (int j = 0; j < MT; ++j) {
                    float d = bv[0] * xv[j][0];
#pragma unroll
                    for (int e = 1; e < 4; ++e) d = d + bv[e] * xv[j][e];
                    acc[p][j] = acc[p][j] + d;
                }
            }
        }
    }
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int j = 0; j < MT; ++j)
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) acc[p][j] = acc[p][j] + __shfl_xor(acc[p][j], o);
    // Lane j of each row's 16 writes x row j's output for that row of B.
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int64_t row = n_base + 16 * p + slot;
#pragma unroll
        for (int j = 0; j < MT; ++j) {
            if (li != j || j >= a.m || row >= a.n) continue;
            float* dst = y + j * a.n + row;
            if (a.causal && row > j + a.query_offset) {
                if (!a.accumulate) *dst = 0.f;
            } else {
                gemm::write_output(dst, acc[p][j], a.scale, a.accumulate != 0);
            }
        }
    }
}

}  // namespace

bool gemv_applies(const Problem& p, const Env& env) {
    // Row-major x (K-contiguous) and row-major W (N-contiguous), aligned for
    // 16-byte loads; no mask or a causal left mask; few rows; grid
    // dimensions and the hand-off slots large enough; a pass's
    // offsets within 31 bits.
    if (!(p.m >= 1 && p.m <= kMaxRows && p.k >= 1 && (p.mask == SN_MASK_NONE || p.mask == SN_MASK_CAUSAL_LEFT) &&
          p.a_k_contiguous &&
          !p.b_k_contiguous && p.lda == p.k && p.ldb == p.n && p.n % 4 == 0 && p.stride_b % 4 == 0 &&
          gemm::aligned16(p.b) && p.batch <= 65535 && p.n < (int64_t(1) << 30)))
        return false;
    const GemvPlan plan = gemv_plan(p);
    if ((plan.pass_rows * p.n + 64) * 4 >= gemm::kMaxBufferOffset) return false;
    if (p.m * p.k * 4 >= gemm::kMaxBufferOffset) return false;  // x's offsets
    if (plan.splits == 1) return true;
    // The hand-off slots (splits - 1 slices of m x (slab width) words per column block
    // and batch) must fit the environment's; their byte offsets then stay
    // within 31 bits.
    return plan.splits <= 65535 && env.handoff != nullptr && handoff_words(p, plan) <= env.handoff_words;
}

bool gemv_nt_applies(const Problem& p) {
    // Row-major x, B stored [n][k] (right transposed), both 16-byte aligned
    // with k and the strides multiples of 4; at most kNtMaxRows rows; no mask
    // or a causal output mask; no fused bias; the grid within limits.
    return p.m >= 1 && p.m <= kNtMaxRows && p.k >= 1 && p.k % 4 == 0 &&
           (p.mask == SN_MASK_NONE || p.mask == SN_MASK_CAUSAL_OUTPUT) && p.bias == nullptr && p.a_k_contiguous &&
           p.b_k_contiguous && p.lda == p.k && p.ldb % 4 == 0 && p.stride_a % 4 == 0 && p.stride_b % 4 == 0 &&
           gemm::aligned16(p.a) && gemm::aligned16(p.b) && p.batch <= 65535 &&
           (p.n + kNtRows - 1) / kNtRows <= 0x7FFFFFFF;
}

hipError_t launch_gemv_nt(const Problem& p, hipStream_t stream) {
    if (!gemv_nt_applies(p)) return hipErrorNotSupported;
    GemvNtArgs a;
    a.x = p.a;
    a.w = p.b;
    a.y = p.c;
    a.m = p.m;
    a.n = p.n;
    a.k = p.k;
    a.ldb = p.ldb;
    a.n_limit = p.mask == SN_MASK_CAUSAL_OUTPUT ? std::min(p.n, p.m - 1 + p.query_offset + 1) : p.n;
    a.stride_x = p.stride_a;
    a.stride_w = p.stride_b;
    a.stride_y = p.stride_c;
    a.query_offset = p.query_offset;
    a.causal = p.mask == SN_MASK_CAUSAL_OUTPUT ? 1 : 0;
    a.accumulate = p.accumulate ? 1 : 0;
    a.scale = p.scale;
    const dim3 grid(unsigned((p.n + kNtRows - 1) / kNtRows), unsigned(p.batch));
    if (p.m == 1)
        hipLaunchKernelGGL(gemv_nt_kernel<1>, grid, dim3(256), 0, stream, a);
    else if (p.m == 2)
        hipLaunchKernelGGL(gemv_nt_kernel<2>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(gemv_nt_kernel<4>, grid, dim3(256), 0, stream, a);
    return hipGetLastError();
}

LaunchShape describe_gemv(const Problem& p) {
    const GemvPlan plan = gemv_plan(p);
    LaunchShape s;
    s.path = SN_PATH_FEW_ROWS;
    s.threads = p.m <= 4 ? 64 * waves_for<4>() : 64 * waves_for<16>();
    s.tile_m = int32_t(p.m);
    s.tile_n = 4 * plan.lanes_per_row;
    s.tiles_m = 1;
    s.tiles_n = plan.column_blocks;
    s.splits = plan.splits;
    s.k_per_split = plan.k_per_split;
    s.batches_per_launch = p.batch;
    s.workgroups = int64_t(plan.column_blocks) * plan.splits * p.batch;
    s.launches = 1;
    s.workspace_bytes = 0;  // the split hand-off uses its own zeroed slots, not the workspace
    return s;
}

LaunchShape describe_gemv_nt(const Problem& p) {
    LaunchShape s;
    s.path = SN_PATH_FEW_ROWS_NT;
    s.threads = 256;
    s.tile_m = int32_t(p.m);
    s.tile_n = kNtRows;
    s.tiles_m = 1;
    s.tiles_n = int32_t((p.n + kNtRows - 1) / kNtRows);
    s.splits = 1;
    s.k_per_split = p.k;
    s.batches_per_launch = p.batch;
    s.workgroups = int64_t(s.tiles_n) * p.batch;
    s.launches = 1;
    return s;
}

hipError_t launch_gemv(const Problem& p, const Env& env, hipStream_t stream) {
    if (!gemv_applies(p, env)) return hipErrorNotSupported;
    const GemvPlan plan = gemv_plan(p);
    if (plan.lanes_per_row == kNarrowLanes)
        return plan.narrow_loads == 8 ? launch_rows<1, kNarrowLanes, 8>(p, env, plan, stream)
                                      : launch_rows<1, kNarrowLanes, 4>(p, env, plan, stream);
    return launch_width<16>(p, env, plan, stream);
}

}  // namespace sn

// The routing of a product to a kernel family, shared by sn_matmul's
// launch and the host-side planner, and the planner's view of the tiled
// kernels' workgroup map. The reference launches its one selected kernel on
// a grid from `launch::matmul_tiles` / `matmul_blocks`
// (crates/staleynet-cuda/src/launch.rs:28-48); here the family depends on
// the shape (few rows, alignment) and the precision, and each family plans
// its own grid.
#include "gemm_common.h"

namespace sn {

namespace {

enum class Family { Simple, FewRows, FewRowsNt, Tiled };

// SN_KERNEL_SIMPLE runs everything in the reference's order; otherwise fp32
// products with few rows take the decode kernels, and the rest the tiled
// kernels of the requested precision.
Family family_of(const Problem& p, uint32_t kernel, const Env& env) {
    if (kernel == SN_KERNEL_SIMPLE) return Family::Simple;
    const bool bf16 = kernel == SN_KERNEL_MFMA_BF16;
    if (!bf16 && gemv_applies(p, env)) return Family::FewRows;
    if (!bf16 && gemv_nt_applies(p)) return Family::FewRowsNt;
    return Family::Tiled;
}

}  // namespace

LaunchShape describe_matmul(const Problem& p, uint32_t kernel, const Env& env) {
    if (p.m == 0 || p.n == 0) return LaunchShape{};
    switch (family_of(p, kernel, env)) {
        case Family::Simple: return describe_gemm_simple(p);
        case Family::FewRows: return describe_gemv(p);
        case Family::FewRowsNt: return describe_gemv_nt(p);
        case Family::Tiled: break;
    }
    return kernel == SN_KERNEL_MFMA_BF16 ? describe_gemm_bf16(p, env) : describe_gemm_f32(p, env);
}

hipError_t launch_matmul(const Problem& p, uint32_t kernel, const Env& env, hipStream_t stream) {
    if (p.m == 0 || p.n == 0) return hipSuccess;
    switch (family_of(p, kernel, env)) {
        case Family::Simple: return launch_gemm_simple(p, stream);
        case Family::FewRows: return launch_gemv(p, env, stream);
        case Family::FewRowsNt: return launch_gemv_nt(p, stream);
        case Family::Tiled: break;
    }
    return kernel == SN_KERNEL_MFMA_BF16 ? launch_gemm_bf16(p, env, stream) : launch_gemm_f32(p, env, stream);
}

ColumnSumsFusion column_sums_fusion(const Problem& p, uint32_t kernel, const Env& env) {
    if (family_of(p, kernel, env) != Family::Tiled) return ColumnSumsFusion::None;
    if (kernel == SN_KERNEL_MFMA_F32 && gemm::f32_column_sums_applies(p, env)) return ColumnSumsFusion::F32Direct;
    if (kernel == SN_KERNEL_MFMA_BF16 && gemm::bf16_wide_column_sums_applies(p, env))
        return ColumnSumsFusion::Bf16Wide;
    return ColumnSumsFusion::None;
}

LaunchShape describe_matmul_column_sums(const Problem& p, uint32_t kernel, const Env& env) {
    if (p.n == 0) return LaunchShape{};
    switch (column_sums_fusion(p, kernel, env)) {
        case ColumnSumsFusion::F32Direct: return gemm::describe_f32_column_sums(p, env);
        case ColumnSumsFusion::Bf16Wide: return gemm::describe_bf16_wide_column_sums(p, env);
        case ColumnSumsFusion::None: break;
    }
    Problem product = p;
    product.column_sums = nullptr;
    LaunchShape s = describe_matmul(product, kernel, env);
    s.workspace_bytes = std::max(s.workspace_bytes, column_sums_workspace_bytes(p.k, p.n, env));
    return s;
}

hipError_t launch_matmul_column_sums(const Problem& p, uint32_t kernel, const Env& env, hipStream_t stream) {
    if (p.n == 0) return hipSuccess;
    switch (column_sums_fusion(p, kernel, env)) {
        case ColumnSumsFusion::F32Direct: return gemm::launch_gemm_f32_column_sums(p, env, stream);
        case ColumnSumsFusion::Bf16Wide: return gemm::launch_gemm_bf16_wide_column_sums(p, env, stream);
        case ColumnSumsFusion::None: break;
    }
    Problem product = p;
    product.column_sums = nullptr;
    hipError_t err = launch_matmul(product, kernel, env, stream);
    if (err != hipSuccess) return err;
    // The stored right operand is [K][N] (row-contiguous, one matrix).
    return launch_column_sums(p.b, p.k, p.n, p.column_sums, env, stream);
}

}  // namespace sn

extern "C" int sn_tile_map(uint32_t workgroups, uint32_t tiles_m, uint32_t tiles_n, uint32_t splits,
                           uint32_t* matrix, uint32_t* slice, uint32_t* tile_row, uint32_t* tile_col) {
    if (matrix == nullptr || slice == nullptr || tile_row == nullptr || tile_col == nullptr) return SN_ERR_NULL_ARGUMENT;
    if (workgroups == 0 || tiles_m == 0 || tiles_n == 0 || splits == 0 || workgroups > 0x7FFFFFFFu ||
        uint64_t(tiles_m) * tiles_n * splits > 0x7FFFFFFFu)
        return SN_ERR_OVERFLOW;
    for (uint32_t w = 0; w < workgroups; ++w) {
        int batch, split, tm, tn;
        sn::gemm::tile_coordinates(int(w), int(workgroups), int(tiles_m), int(tiles_n), int(splits), batch, split, tm,
                                   tn);
        matrix[w] = uint32_t(batch);
        slice[w] = uint32_t(split);
        tile_row[w] = uint32_t(tm);
        tile_col[w] = uint32_t(tn);
    }
    return SN_OK;
}

// One thread per output, k summed in order with every product and sum
// rounded separately: the arithmetic of the reference's CPU loop
// (crates/staleynet-cuda/src/reference.rs:19-38) and of its matmul_naive
// kernel (crates/staleynet-cuda/src/kernels/matmul.rs:206-233). Selected by
// SN_KERNEL_SIMPLE as an on-device cross-check; not a performance path.
#include "gemm_internal.h"
#include "staleynet_gemm.h"

#include <algorithm>

namespace sn {
namespace {

struct SimpleArgs {
    const float* a;
    const float* b;
    float* c;
    int64_t m, n, k, lda, ldb, stride_a, stride_b, stride_c, batch_base, query_offset;
    int32_t a_k_contiguous, b_k_contiguous, accumulate, mask;
    float scale;
    const float* bias;
};

__global__ __launch_bounds__(256) void gemm_simple_kernel(SimpleArgs p) {
    // hipcc contracts a * b + c into one fused multiply-add by default; the
    // reference rounds the product and the sum separately.
#pragma clang fp contract(off)
    const int64_t col = int64_t(blockIdx.x) * 16 + threadIdx.x;
    const int64_t row = int64_t(blockIdx.y) * 16 + threadIdx.y;
    const int64_t batch = p.batch_base + blockIdx.z;
    if (row >= p.m || col >= p.n) return;
    float* dst = p.c + batch * p.stride_c + row * p.n + col;
    if (p.mask == int(SN_MASK_CAUSAL_OUTPUT) && col > row + p.query_offset) {
        if (!p.accumulate) *dst = 0.f;
        return;
    }
    const float* a = p.a + batch * p.stride_a;
    const float* b = p.b + batch * p.stride_b;
    float sum = 0.f;
    for (int64_t k = 0; k < p.k; ++k) {
        float x = p.a_k_contiguous ? a[row * p.lda + k] : a[k * p.lda + row];
        if (p.mask == int(SN_MASK_CAUSAL_LEFT)) {
            const bool visible = p.a_k_contiguous ? k <= row + p.query_offset : row <= k + p.query_offset;
            if (!visible) x = 0.f;
        }
        const float y = p.b_k_contiguous ? b[col * p.ldb + k] : b[k * p.ldb + col];
        const float product = x * y;
        sum = sum + product;
    }
    const float scaled = p.scale * sum;
    float value = p.accumulate ? *dst + scaled : scaled;
    if (p.bias != nullptr) value = value + p.bias[col];
    *dst = value;
}

}  // namespace

LaunchShape describe_gemm_simple(const Problem& p) {
    LaunchShape s;
    s.path = SN_PATH_REFERENCE_ORDER;
    s.threads = 256;
    s.tile_m = 16;
    s.tile_n = 16;
    s.tiles_m = int32_t((p.m + 15) / 16);
    s.tiles_n = int32_t((p.n + 15) / 16);
    s.splits = 1;
    s.k_per_split = p.k;
    s.batches_per_launch = std::min<int64_t>(65535, p.batch);
    s.workgroups = int64_t(s.tiles_m) * s.tiles_n * s.batches_per_launch;
    s.launches = (p.batch + 65534) / 65535;
    return s;
}

hipError_t launch_gemm_simple(const Problem& p, hipStream_t stream) {
    SimpleArgs args{p.a, p.b, p.c, p.m, p.n, p.k, p.lda, p.ldb, p.stride_a, p.stride_b, p.stride_c, 0,
                    p.query_offset, p.a_k_contiguous, p.b_k_contiguous, p.accumulate, int32_t(p.mask), p.scale,
                    p.bias};
    if ((p.m + 15) / 16 > 65535 || (p.n + 15) / 16 * 16 >= (int64_t(1) << 32)) return hipErrorInvalidConfiguration;
    const dim3 grid(unsigned((p.n + 15) / 16), unsigned((p.m + 15) / 16), 1);
    for (int64_t first = 0; first < p.batch; first += 65535) {
        args.batch_base = first;
        const dim3 g(grid.x, grid.y, unsigned(std::min<int64_t>(65535, p.batch - first)));
        hipLaunchKernelGGL(gemm_simple_kernel, g, dim3(16, 16), 0, stream, args);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

}  // namespace sn

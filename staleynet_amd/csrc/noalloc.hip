// sn_matmul_noalloc: sn_matmul for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc). It has no counterpart in the reference. Here the
// kernels' scratch (split-K partial sums and bf16 staged operands, arrival
// counters, and the decode kernel's hand-off slots) lives in a file-scope
// device array instead of a context's workspace:
//  * every device the library runs on holds its own copy of the array from
//    the moment the code object loads until the process ends;
//  * on the first call on a device (with that device current) its address
//    is looked up with hipGetSymbolAddress and kept per device; the array's
//    name in host code is only a stand-in, never a device address. That
//    set-up puts no work on any stream, so a first call made under stream
//    capture records only the product's own kernels;
//  * the counters and hand-off slots must be zero between calls: the array
//    has static storage and no initializer, so the code object's loader
//    zero-fills it, and every kernel that increments a counter or fills a
//    slot resets it before it ends; the partial sums are written before
//    they are read within each call;
//  * every call on a device shares that device's array, so calls that
//    overlap on one device (two streams, two threads) race.
// Products whose plan would split K into more partial sums than the array
// holds take fewer slices (the planner caps them by the workspace size), so
// results stay within the fp32 tolerance of sn_matmul's and are
// bit-identical whenever both plans agree.
#include <mutex>

#include "gemm_common.h"

namespace {

constexpr size_t kScratchCounters = 16384;                              // as a context has
constexpr size_t kScratchCounterBytes = kScratchCounters * sizeof(uint32_t);  // 64 KiB
constexpr size_t kScratchHandoffBytes = sn::kHandoffWords * sizeof(uint32_t);  // 4 MiB
constexpr size_t kScratchWorkspaceBytes = SN_NOALLOC_WORKSPACE_BYTES;   // 64 MiB
static_assert((kScratchCounterBytes + kScratchHandoffBytes) % 256 == 0, "the workspace part stays 256-byte aligned");

static __device__ __align__(256)
    unsigned char scratch[kScratchCounterBytes + kScratchHandoffBytes + kScratchWorkspaceBytes];

constexpr int kMaxDevices = 64;

struct DeviceScratch {
    std::once_flag once;
    hipError_t status = hipSuccess;
    unsigned char* ptr = nullptr;  // this device's copy of `scratch`
    int cu_count = 256;
};

DeviceScratch g_devices[kMaxDevices];

// Set-up of `device` (current on the calling thread), once: the device
// address of its `scratch` and its compute-unit count. Nothing is enqueued.
// A failure is kept and returned by every later call.
DeviceScratch& scratch_of(int device) {
    DeviceScratch& d = g_devices[device];
    std::call_once(d.once, [&] {
        void* ptr = nullptr;
        hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        int cus = 0;
        if (err == hipSuccess) err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
        if (err == hipSuccess) {
            d.ptr = static_cast<unsigned char*>(ptr);
            d.cu_count = cus > 0 ? cus : 256;
        }
        d.status = err;
    });
    return d;
}

}  // namespace

extern "C" int sn_matmul_noalloc(const sn_matmul_spec* spec, const float* left, size_t left_len, const float* right,
                                 size_t right_len, float* output, size_t output_len, void* stream) {
    const int rc = sn::check_matmul_call(spec, left, left_len, right, right_len, nullptr, 0, output, output_len);
    if (rc != SN_OK) return rc;
    if (spec->rows == 0 || spec->cols == 0) return SN_OK;
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) return int(err);
    if (device < 0 || device >= kMaxDevices) return SN_ERR_NO_DEVICE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    DeviceScratch& d = scratch_of(device);
    if (d.status != hipSuccess) return int(d.status);
    sn::Env env;
    env.counters = reinterpret_cast<uint32_t*>(d.ptr);
    env.counter_count = kScratchCounters;
    env.handoff = reinterpret_cast<uint32_t*>(d.ptr + kScratchCounterBytes);
    env.handoff_words = sn::kHandoffWords;
    env.workspace = reinterpret_cast<float*>(d.ptr + kScratchCounterBytes + kScratchHandoffBytes);
    env.workspace_bytes = kScratchWorkspaceBytes;
    env.cu_count = d.cu_count;
    const sn::Problem p = sn::problem_of(spec, left, right, output, nullptr);
    const uint32_t kernel = spec->precision == SN_PRECISION_BF16 ? SN_KERNEL_MFMA_BF16 : SN_KERNEL_MFMA_F32;
    if (sn::describe_matmul(p, kernel, env).workspace_bytes > env.workspace_bytes) return SN_ERR_WORKSPACE;
    err = sn::launch_matmul(p, kernel, env, s);
    return err == hipSuccess ? SN_OK : int(err);
}

// Decode-shaped products (few output rows). Filled in by the GEMV kernels;
// until then every product goes to the tiled kernels.
#include "gemm_internal.h"

namespace sn {

bool gemv_applies(const Problem&) { return false; }

hipError_t launch_gemv(const Problem&, const Env&, hipStream_t) { return hipErrorNotSupported; }

}  // namespace sn

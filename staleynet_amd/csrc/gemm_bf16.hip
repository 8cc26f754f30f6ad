// bf16-input / fp32-accumulate matrix-core GEMM (filled in next).
#include "gemm_internal.h"

namespace sn {

hipError_t launch_gemm_bf16(const Problem&, const Env&, hipStream_t) { return hipErrorNotSupported; }

}  // namespace sn

// Instantiations of the fused argmax GEMV kernel for f16_t base logits (one
// translation unit per base dtype keeps the build parallel).
#include "fused_argmax_fp8.h"
#include "fused_argmax_gemv.h"

namespace dels {

hipError_t launch_gemv_f16(const ArgmaxKArgs& ka, bool packed, int prior_kind, hipStream_t s) {
    return launch_gemv_for_base<f16_t>(ka, packed, prior_kind, s);
}

hipError_t launch_gemv8_f16(const ArgmaxKArgs& ka, int prior_kind, hipStream_t s) {
    return launch_gemv8_for_base<f16_t>(ka, prior_kind, s);
}

}  // namespace dels

// Instantiations of the fused decode-step kernel (rank projection + argmax,
// M <= 16) for f16_t base logits; one translation unit per base dtype.
#include "lowrank_decode.h"

namespace dels {

hipError_t launch_decode_f16(const DecodeKArgs& ka, int ksteps, int prior_kind, hipStream_t s, bool gru) {
    return launch_decode_for_base<f16_t>(ka, ksteps, prior_kind, s, gru);
}

hipError_t launch_decode8_f16(const DecodeKArgs& ka, int prior_kind, hipStream_t s) {
    return launch_decode8_for_base<f16_t>(ka, prior_kind, s);
}

}  // namespace dels

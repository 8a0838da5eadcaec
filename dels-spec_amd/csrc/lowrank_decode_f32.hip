// Instantiations of the fused decode-step kernel (rank projection + argmax,
// M <= 16) for float base logits; one translation unit per base dtype.
#include "lowrank_decode.h"

namespace dels {

hipError_t launch_decode_f32(const DecodeKArgs& ka, int ksteps, int prior_kind, hipStream_t s, bool gru) {
    return launch_decode_for_base<float>(ka, ksteps, prior_kind, s, gru);
}

hipError_t launch_decode8_f32(const DecodeKArgs& ka, int prior_kind, hipStream_t s) {
    return launch_decode8_for_base<float>(ka, prior_kind, s);
}

}  // namespace dels

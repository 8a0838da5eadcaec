// Instantiations of the batched (MFMA-tiled) fused argmax kernel for float base
// logits (one translation unit per base dtype keeps the build parallel).
#include "fused_argmax_tiled.h"

namespace dels {

hipError_t launch_tiled_f32(const TiledKArgs& ka, int ksteps, int prior_kind, int gx, int gy, hipStream_t s) {
    return launch_tiled_for_base<float>(ka, ksteps, prior_kind, gx, gy, s);
}

}  // namespace dels

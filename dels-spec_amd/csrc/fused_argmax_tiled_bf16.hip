// Instantiations of the batched (MFMA-tiled) fused argmax kernel for bf16_t base
// logits (one translation unit per base dtype keeps the build parallel).
#include "fused_argmax_tiled.h"

namespace dels {

hipError_t launch_tiled_bf16(const TiledKArgs& ka, int ksteps, int prior_kind, int gx, int gy, hipStream_t s) {
    return launch_tiled_for_base<bf16_t>(ka, ksteps, prior_kind, gx, gy, s);
}

}  // namespace dels

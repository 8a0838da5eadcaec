// Instantiations of the batched (MFMA-tiled) fused argmax kernels (bf16 and e4m3 B) for f16_t base
// logits (one translation unit per base dtype keeps the build parallel).
#include "fused_argmax_tiled.h"
#include "fused_argmax_tiled8.h"

namespace dels {

hipError_t launch_tiled_f16(const TiledKArgs& ka, int ksteps, int prior_kind, int gx, int gy, hipStream_t s) {
    return launch_tiled_for_base<f16_t>(ka, ksteps, prior_kind, gx, gy, s);
}

hipError_t launch_tiled8_f16(const TiledKArgs& ka, int ks8, int prior_kind, int gx, int gy, hipStream_t s) {
    return launch_tiled8_for_base<f16_t>(ka, ks8, prior_kind, gx, gy, s);
}

}  // namespace dels

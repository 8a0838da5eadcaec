// Host side of the fused combine + argmax: workspace layout and dispatch to
// the per-dtype instantiations of the GEMV kernel (fused_argmax_gemv.h).
#include <algorithm>

#include "fused_argmax_gemv.h"

namespace dels {

size_t argmax_data_bytes(int64_t /*M*/, int64_t /*r*/, int64_t /*V*/) { return 0; }

bool argmax_supported(int64_t M, int64_t r, int64_t /*V*/) { return r >= 8 && r <= 512 && M <= kMaxKeyRows; }

hipError_t launch_fused_argmax(const ArgmaxArgs& a, void* ws, hipStream_t s) {
    ArgmaxKArgs ka{};
    ka.rank = a.rank; ka.ldrank = a.ldrank;
    ka.B = a.B; ka.ldb = a.ldb;
    ka.base = a.base; ka.ldbase = a.ldbase;
    ka.prior = a.prior;
    ka.alpha = a.alpha; ka.alpha_stride = a.alpha_stride;
    ka.beta = a.beta; ka.beta_stride = a.beta_stride;
    ka.M = a.M; ka.r = a.r; ka.V = a.V;
    ka.ksteps = (a.r + 31) / 32;
    ka.out_ids = a.out_ids; ka.out_score = a.out_score; ka.ld_out = a.ld_out;
    char* w = static_cast<char*>(ws);
    ka.counter = reinterpret_cast<unsigned int*>(w + kCountersOff);
    ka.keys = reinterpret_cast<unsigned long long*>(w + kKeysOff);
    // one 128-byte line per row while the rows fit the key area, else packed
    ka.key_stride = (int64_t)a.M * 128 <= (int64_t)(kCtrlBytes - kKeysOff) ? 16 : 1;
    // prior kind: 0 none, 1 fp32, 2 bf16, 3 fp16
    const int pk = a.prior == nullptr ? 0 : (a.prior_dtype == 1 ? 2 : (a.prior_dtype == 2 ? 3 : 1));
    if (a.base_dtype == 1) return launch_gemv_bf16(ka, a.b_packed, pk, s);
    if (a.base_dtype == 2) return launch_gemv_f16(ka, a.b_packed, pk, s);
    return launch_gemv_f32(ka, a.b_packed, pk, s);
}

}  // namespace dels

// Host-side internal interface between the C ABI (capi.hip) and the kernel
// launchers (skinny_gemm.hip, fused_argmax.hip).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dels {

// ---- skinny GEMM: rank projection and fused GRU step -----------------------

struct SkinnyPlan {
    int wm, wn;        // 16x16 MFMA sub-tiles per wave (rows x cols)
    int m_wg, n_wg;    // workgroup grid (row tiles, col tiles)
    int ksplit;        // workgroups sharing one output tile along K
    int ksteps;        // ceil(K / 32)
    size_t counter_bytes, partial_bytes;
};

// rows: M; cols: N (rank) or G (GRU, three gate tiles per column tile).
SkinnyPlan plan_skinny(int64_t rows, int64_t K, int64_t cols, bool gru);
size_t skinny_ws_bytes(const SkinnyPlan& p);

struct RankArgs {
    const uint16_t* h; int64_t ldh;
    const uint16_t* A; int64_t lda;
    const uint16_t* bias; int act;
    int M, d, r;
    uint16_t* rank; int64_t ldrank;
};
hipError_t launch_rank_proj(const RankArgs& a, const SkinnyPlan& p, void* ws, hipStream_t s);

struct GruArgs {
    const uint16_t* gi_table; int64_t ld_gi; int64_t table_rows;
    const int64_t* tokens; int64_t tok_stride;
    const uint16_t* h_in; int64_t ldh_in;
    const uint16_t* w_hh; const uint16_t* b_hh;
    int batch, G;
    uint16_t* h_out; int64_t ldh_out;
};
hipError_t launch_gru_step(const GruArgs& a, const SkinnyPlan& p, void* ws, hipStream_t s);

// ---- fused combine + argmax -------------------------------------------------

struct ArgmaxArgs {
    const uint16_t* rank; int64_t ldrank;
    const uint16_t* B; int64_t ldb;
    const void* base; int64_t ldbase; int base_dtype;
    const void* prior; int prior_dtype;
    const float* alpha; int64_t alpha_stride;
    const float* beta; int64_t beta_stride;
    int M, r, V;
    int64_t* out_ids; float* out_score; int64_t ld_out;
};
size_t argmax_ws_bytes(int64_t M, int64_t r, int64_t V);
bool argmax_supported(int64_t M, int64_t r, int64_t V);
hipError_t launch_fused_argmax(const ArgmaxArgs& a, void* ws, hipStream_t s);

// ---- workspace fill ---------------------------------------------------------
hipError_t launch_fill_zero(void* ws, size_t bytes, hipStream_t s);

// Device properties of the current device (cached per device id).
int device_cu_count();

}  // namespace dels

// Host-side internal interface between the C ABI (capi.hip) and the kernel
// launchers (skinny_gemm.hip, fused_argmax.hip).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dels {

// ---- workspace layout ---------------------------------------------------------
// Every entry point lays its workspace out the same way:
//  * [0, kCtrlBytes): the control area -- cross-workgroup counters at
//    [0, 32 KiB) and argmax keys at [32 KiB, 64 KiB).  Kernels return it to
//    zero before they finish, except the last 128-byte line of the counters,
//    whose words persist between calls (the fused decode step's launch
//    generation).
//  * [kDecodeOff, kDataOff): the fused decode step's tagged words (rank
//    partials and the published rank).  Reserved in every layout and written
//    by the decode kernels only, so each word holds zero or the tag of an
//    earlier decode launch on this workspace -- never leftover data of another
//    entry point that could pass for the current launch's tag.
//  * [kResidentOff, kDataOff): the resident rollout's tagged words (the state
//    and the rank of each step) and argmax slot words, written by that kernel
//    only, for the same reason.
//  * [kDataOff, ...): data regions of the other kernels (split-K partials, the
//    rank, quantised operands); they may hold anything between calls.
// Calls with different shapes or entry points can therefore share one
// workspace (one at a time).
constexpr size_t kCtrlBytes = 65536;
constexpr size_t kCountersOff = 0;
constexpr int kMaxCounters = 8160;             // counters that kernels return to zero
constexpr int kDecodeGenWord = 8160;           // the decode step's launch generation (persists)
constexpr size_t kKeysOff = 32768;
constexpr int kMaxKeyRows = 4096;

inline constexpr size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

constexpr int kDecodeWGs = 256;                // grid of the fused decode step (one workgroup per CU)
constexpr int kDecodeMaxRank = 512;            // largest rank r the decode step takes
// one 256-word partial per workgroup, then 16 rows x r/2 words of the rank
constexpr size_t kDecodeWordBytes = align256((size_t)kDecodeWGs * 256 * 8) +
                                    align256((size_t)16 * (kDecodeMaxRank / 2) * 8);
constexpr size_t kDecodeOff = kCtrlBytes;

// The rollout with B resident on chip (rollout_resident.hip): r = 256, G <= 1024,
// batch <= 16, 64 .. 256 workgroups; its words {tag, two bf16} of the state
// (16 rows x G/2 words at most) and of the rank (16 x r/2), each producer's
// words on 128-byte lines of their own, then the argmax slot words [2][nwg][16].
constexpr int kResidentRank = 256;
constexpr int kResidentMaxG = 1024;
constexpr int kResidentLdsTiles = 6;           // vocabulary tiles per workgroup in LDS beyond the registers
constexpr int kResidentMaxSteps = 64;
constexpr int kResidentMaxWGs = 256;
constexpr size_t kResidentHWordBytes = align256((size_t)16 * (kResidentMaxG / 2) * 8);
constexpr size_t kResidentRankWordBytes = align256((size_t)16 * (kResidentRank / 2) * 8);
constexpr size_t kResidentSlotBytes = align256((size_t)2 * 16 * kResidentMaxWGs * 8);
constexpr size_t kResidentWordBytes = kResidentHWordBytes + kResidentRankWordBytes + kResidentSlotBytes;
constexpr size_t kResidentOff = kDecodeOff + kDecodeWordBytes;
constexpr size_t kDataOff = kResidentOff + kResidentWordBytes;

// ---- skinny GEMM: rank projection and fused GRU step -----------------------

// Rows from which the rank projection uses the LDS-tiled kernel.
constexpr int kRankTiledMinRows = 64;

struct SkinnyPlan {
    bool tiled;        // rank projection by the LDS-tiled kernel (many rows)
    int tm, tn;        // its output tile (rows x cols)
    int wm, wn;        // 16x16 MFMA sub-tiles per wave (rows x cols)
    int m_wg, n_wg;    // workgroup grid (row tiles, col tiles)
    int ksplit;        // workgroups sharing one output tile along K
    int ksteps;        // ceil(K / 32)
    size_t partial_bytes;
};

// rows: M; cols: N (rank) or G (GRU, three gate tiles per column tile).
SkinnyPlan plan_skinny(int64_t rows, int64_t K, int64_t cols, bool gru);
// Bytes of the data region the plan needs (its counters live in the control area).
size_t skinny_data_bytes(const SkinnyPlan& p);
bool skinny_supported(const SkinnyPlan& p);

struct RankArgs {
    const uint16_t* h; int64_t ldh;
    const uint16_t* A; int64_t lda; bool a_packed;
    const float* a_scale = nullptr;   // non-null: A is e4m3 in K32 blocks, this its per-column scale [r]
    const uint16_t* bias; int act;
    int M, d, r;
    uint16_t* rank; int64_t ldrank;
    // non-null (rank_proj_quantizes): the rank is also written quantised per row
    // to e4m3 ([M][r] bytes) with its per-row scale [M], as the e4m3 tiled argmax takes it
    uint8_t* rank_q = nullptr;
    float* rank_qscale = nullptr;
};
// Whether launch_rank_proj with plan p can also write the rank quantised per
// row to e4m3 (the LDS-tiled GEMM with split K, r = 256 or 512).
bool rank_proj_quantizes(const SkinnyPlan& p, int64_t r);
// `ws` is the workspace base (control area); partials go to ws + data_off.
hipError_t launch_rank_proj(const RankArgs& a, const SkinnyPlan& p, void* ws, size_t data_off, hipStream_t s);

struct GruArgs {
    const uint16_t* gi_table; int64_t ld_gi; int64_t table_rows;
    const int64_t* tokens; int64_t tok_stride;
    const uint16_t* h_in; int64_t ldh_in;
    const uint16_t* w_hh; bool w_packed; const uint16_t* b_hh;
    int batch, G;
    uint16_t* h_out; int64_t ldh_out;
};
hipError_t launch_gru_step(const GruArgs& a, const SkinnyPlan& p, void* ws, size_t data_off, hipStream_t s);

// ---- fused combine + argmax -------------------------------------------------

struct ArgmaxArgs {
    const uint16_t* rank; int64_t ldrank;
    // non-null: row m of the rank is row rank_rows[m * rank_rows_stride] of the
    // [rank_rows_count, r] table `rank` (bf16 argmax only)
    const int64_t* rank_rows = nullptr;
    int64_t rank_rows_stride = 0, rank_rows_count = 0;
    const uint16_t* B; int64_t ldb; bool b_packed;
    const float* b_scale = nullptr;   // non-null: B is e4m3 in K128 blocks, this its per-row scale [V]
    // e4m3 tiled argmax only: the rank quantised per row is already at the
    // argmax's data offset (rank_proj_quantizes), no quantisation launch
    bool rank_quantized = false;
    const void* base; int64_t ldbase; int base_dtype;
    const void* prior; int prior_dtype;
    const float* alpha; int64_t alpha_stride;
    const float* beta; int64_t beta_stride;
    int M, r, V;
    int64_t* out_ids; float* out_score; int64_t ld_out;
};
// Data-region bytes the argmax needs beyond the control area (counter + keys):
// the per-chunk partials of the tiled kernel.
size_t argmax_data_bytes(int64_t M, int64_t r, int64_t V);
bool argmax_supported(int64_t M, int64_t r, int64_t V);
// `ws` is the workspace base (control area); partials go to ws + data_off.
hipError_t launch_fused_argmax(const ArgmaxArgs& a, void* ws, size_t data_off, hipStream_t s);

// Plain per-row argmax of logits [M, V] (dtype 0 fp32, 1 bf16, 2 fp16), M <= kMaxKeyRows.
hipError_t launch_argmax_rows(const void* x, int64_t ldx, int dtype, int M, int V, int64_t* out_ids,
                              float* out_score, int64_t ld_out, void* ws, hipStream_t s);

// Temperature sampling of logits [M, V] (dtype as launch_argmax_rows): Gumbel-max
// over Philox4x32-10 bits at counter (v/4, m, offset) and key seed; M <= kMaxKeyRows.
hipError_t launch_sample_rows(const void* x, int64_t ldx, int dtype, int M, int V, float temperature, uint64_t seed,
                              uint64_t offset, int64_t* out_ids, float* out_score, int64_t ld_out, void* ws,
                              hipStream_t s);

// fp8 argmax (b_scale set): r in {128, 256, 512}, any M up to kMaxKeyRows.
bool argmax_fp8_supported(int64_t M, int64_t r);
size_t argmax_fp8_data_bytes(int64_t M, int64_t r, int64_t V);
// Whether launch_fused_argmax_fp8 runs the e4m3 tiled kernel for `a` (which
// reads the rank quantised per row from the start of its data region).
bool fp8_argmax_tiled(const ArgmaxArgs& a);
hipError_t launch_fused_argmax_fp8(const ArgmaxArgs& a, void* ws, size_t data_off, hipStream_t s);

// ---- target LM head of a draft block: base = bf16(hidden . W^T), argmax rows fused ----
// K blocks per chunk of the LM head's K-chunk-major W layout (dels_pack_lm_head).
constexpr int kLmHeadKChunk = 4;
// W [V, K] in MFMA-16 blocks, K-chunk-major, K a multiple of 256; rows m with argmax_period > 0
// and m % argmax_period == 0 are argmaxed (ids/scores at row m / argmax_period of
// out_*) instead of stored.  Keys and counter in the control area of `ws`.
bool lm_head_supported(int64_t M, int64_t K, int64_t V, int64_t argmax_period);
hipError_t launch_lm_head(const void* hidden, int64_t ldh, const void* W, int M, int K, int V, void* base,
                          int64_t ldo, int argmax_period, int64_t* out_ids, float* out_score, int64_t ld_out,
                          void* ws, hipStream_t s);

// ---- Domino correction step (SiLU(z + s) . fc2^T (+ bias), alpha, base, argmax) ----

constexpr int kDominoMaxE = 2048;              // largest correction-MLP width (LDS operands)

struct DominoArgs {
    const uint16_t* z; int64_t ldz;            // [M, E] bf16: fc1's hidden-state part of this step
    const uint16_t* s; int64_t lds;            // [M, E] bf16: fc1's GRU-state part
    const uint16_t* W;                         // fc2 weight [V, E], MFMA-16 blocks
    const void* bias; int bias_dtype;          // fc2 bias [V] (nullptr: none), dtype code as base
    const void* base; int64_t ldbase; int base_dtype;
    float alpha;
    int middle;                                // DELS_MIDDLE_*: the elementwise layer between fc1 and fc2
    int M, E, V;
    int64_t* out_ids; float* out_score; int64_t ld_out;
};
bool domino_supported(int64_t M, int64_t E, int64_t V);
size_t domino_lds_bytes(int64_t E);
// keys and counter in the control area of `ws`
hipError_t launch_domino_argmax(const DominoArgs& a, void* ws, hipStream_t s);

// ---- fused decode step: rank projection + argmax in one launch (M <= 16) --------

// Both weights packed, r/32 in {2, 4, 8, 16}, d a multiple of 32 and at most
// 32 K blocks per split of the rank projection.
bool decode_eligible(int64_t M, int64_t d, int64_t r, bool a_packed, bool b_packed);

// ---- the rollout with B resident on chip (one launch for every step) -------------
struct ResidentRolloutArgs {
    const uint16_t* w_hh; const uint16_t* b_hh;
    const uint16_t* A; const uint16_t* rank_b; int act;
    const uint16_t* B;
    const uint16_t* gi_table; int64_t ld_gi; int64_t table_rows;
    const int64_t* prefix; int64_t ld_prefix;
    const void* base; int64_t ld_base; int base_dtype;
    const void* prior; int prior_dtype;
    const float* alpha; const float* beta;
    int64_t batch, G, V, steps;
    int64_t* out_ids; float* out_scores; int64_t ld_out;   // row m, step s at [m * ld_out + s]
};
bool rollout_resident_eligible(int64_t batch, int64_t G, int64_t r, int64_t V, int64_t steps, bool packed);
hipError_t launch_rollout_resident(const ResidentRolloutArgs& a, void* ws, hipStream_t s);
int resident_spin_limit();
int set_resident_spin_limit(int limit);   // returns the previous limit
int set_rollout_resident(int enable);   // returns the previous setting (1 = used where eligible)
bool rollout_resident_enabled();
// The fp8 decode step (A e4m3 K32, B e4m3 K128): as above with r in {128, 256, 512}.
bool decode8_eligible(int64_t M, int64_t d, int64_t r);
// A rollout step with the local head's GRU fused into the decode launch:
// h = GRU(gi_table[tokens], h_prev) is computed in the launch (and written to
// h_out), then the draft step runs on it (ra.h is not read).
struct DecodeGru {
    const uint16_t* gi_table; int64_t ld_gi, table_rows;   // [rows, 3G] bf16
    const int64_t* tokens; int64_t tok_stride;
    const uint16_t* w_hh;        // [3G, G] in MFMA-16 blocks
    const uint16_t* b_hh;        // [3G] or NULL
    const uint16_t* h_prev;      // [M, G], row stride G
    uint16_t* h_out;             // [M, G], row stride G
};
// decode_eligible (bf16, packed), G a multiple of 32 up to 2048, and room in the
// grid for G/16 GRU workgroups next to the rank workgroups.
bool decode_gru_eligible(int64_t M, int64_t G, int64_t r);
// fp8 when ra.a_scale and aa.b_scale are set (decode8_eligible), bf16 otherwise;
// with `gru` (bf16 only, decode_gru_eligible) a fused rollout step.
// The tagged words go to [kDecodeOff, kDataOff) of `ws`.
hipError_t launch_lowrank_decode(const RankArgs& ra, const ArgmaxArgs& aa, void* ws, hipStream_t s,
                                 const DecodeGru* gru = nullptr);
// Polls of the rank-ready count before a workgroup computes the rank itself
// (test hook; returns the previous value).
int set_decode_spin_limit(int limit);

// ---- workspace fill and operand packing ---------------------------------------
hipError_t launch_fill_zero(void* ws, size_t bytes, hipStream_t s);

// MFMA-16 block layout: 16-row x 32-column blocks of 1 KiB in wave64 lane order.
inline int64_t packed_row_blocks(int64_t rows) { return (rows + 15) / 16; }
inline int64_t packed_col_blocks(int64_t cols) { return (cols + 31) / 32; }
inline size_t packed_bytes(int64_t rows, int64_t cols) {
    return (size_t)packed_row_blocks(rows) * packed_col_blocks(cols) * 1024;
}
// kchunk > 0: K-chunk-major block order (the LM head's layout), see pack.hip.
hipError_t launch_pack_mfma16(const uint16_t* W, int64_t ldw, int64_t rows, int64_t cols, uint16_t* P,
                              hipStream_t s, int64_t kchunk = 0);
// e4m3 layouts: K128 (16 x 128 blocks of 2 KiB, the fp8 argmax's B) and K32
// (16 x 32 blocks of 512 bytes, the fp8 rank projection's A).
enum : int { FP8_K128 = 2, FP8_K32 = 3 };
inline size_t packed_fp8_bytes(int64_t rows, int64_t cols, int layout) {
    const int64_t kb = layout == FP8_K128 ? 128 : 32;
    return (size_t)((rows + 15) / 16) * (size_t)((cols + kb - 1) / kb) * (size_t)(16 * kb);
}
hipError_t launch_pack_fp8(const uint8_t* W, int64_t ldw, int64_t rows, int64_t cols, int layout, uint8_t* P,
                           hipStream_t s);

// Device properties of the current device (cached per device id).
int device_cu_count();

}  // namespace dels

// C ABI of the DeLS draft-token selection path (declared in include/dels.h).
//
// Host-side argument checking, workspace layout and kernel dispatch.  Nothing
// here allocates device memory or synchronises the caller's stream; the only
// objects the library creates are the hipGraph/hipGraphExec (and the capture
// stream) owned by a dels_graph_create handle.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <initializer_list>
#include <mutex>
#include <string>

#include "../../include/dels.h"
#include "dels_internal.h"

namespace dels {

// The rollout's rank projection reads only G x r weights: below this hidden
// size two launches (rank GEMM with K whole, then the argmax GEMV) finish
// sooner than the one-launch decode step, whose device-wide rank hand-off
// costs a fixed few microseconds.  At G = 1024, r = 256 the decode step is
// ahead (draft block of batch 8, block 16: 727.9 -> 719.2 us).
constexpr int kRolloutDecodeMinG = 1024;

static thread_local std::string g_last_error;

static int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

static int hip_fail(hipError_t e, const char* what) {
    return fail(DELS_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int device_cu_count() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 1;
        cache[dev] = n;
    }
    return cache[dev];
}

__global__ void fill_zero_kernel(uint32_t* p, size_t words) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < words; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

hipError_t launch_fill_zero(void* ws, size_t bytes, hipStream_t s) {
    const size_t words = bytes / 4;
    if (words == 0) return hipSuccess;
    const int blocks = (int)std::min<size_t>(1024, (words + 255) / 256);
    hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, s, static_cast<uint32_t*>(ws), words);
    return hipGetLastError();
}

static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
static inline bool valid_dtype(int d) { return d == DELS_DTYPE_F32 || d == DELS_DTYPE_BF16 || d == DELS_DTYPE_F16; }
static inline size_t dtype_size(int d) { return d == DELS_DTYPE_F32 ? 4 : 2; }

// Checks of a bf16 row-major operand: non-null, 16-byte aligned, ld % 8 == 0, ld >= cols.
// Extents every entry point keeps within: rows, batch, batch * steps, r, G and
// E in [0, 2^24), hidden sizes (d, D, K) in [0, 2^26), V in [0, 2^31 - 1).
// Within them all size arithmetic stays below 2^60; the size queries answer 0
// for a shape outside them, and check_ws() refuses a need of 0.
static bool rows_ok(int64_t x) { return x >= 0 && x < (int64_t(1) << 24); }
static bool inner_ok(int64_t x) { return x >= 0 && x < (int64_t(1) << 26); }
static bool vocab_ok(int64_t x) { return x >= 0 && x < INT32_MAX; }
// Leading dimensions and strides (in elements) lie in [0, 2^40), so that every
// element offset the kernels form stays far inside 64 bits.
static bool ld_ok(std::initializer_list<int64_t> xs) {
    for (int64_t x : xs)
        if (x < 0 || x >= (int64_t(1) << 40)) return false;
    return true;
}

static int check_bf16_matrix(const void* p, int64_t ld, int64_t cols, const char* name) {
    if (!p) return fail(DELS_ERR_INVALID_ARGUMENT, "%s is NULL", name);
    if (!ld_ok({ld})) return fail(DELS_ERR_INVALID_ARGUMENT, "%s: leading dimension %lld out of range", name,
                                  (long long)ld);
    if (ld < cols) return fail(DELS_ERR_INVALID_ARGUMENT, "%s: leading dimension %lld < columns %lld", name,
                               (long long)ld, (long long)cols);
    if (!aligned16(p) || (ld % 8) != 0)
        return fail(DELS_ERR_ALIGNMENT, "%s must be 16-byte aligned with a leading dimension divisible by 8", name);
    return DELS_OK;
}

// Checks of a bf16 weight operand in either layout.
static int check_weight(const void* p, int64_t ld, int64_t cols, int layout, const char* name) {
    if (layout == DELS_LAYOUT_ROWMAJOR) return check_bf16_matrix(p, ld, cols, name);
    if (layout == DELS_LAYOUT_FP8_K128 || layout == DELS_LAYOUT_FP8_K32) {
        if (!p) return fail(DELS_ERR_INVALID_ARGUMENT, "%s is NULL", name);
        if (!aligned16(p)) return fail(DELS_ERR_ALIGNMENT, "packed fp8 %s must be 16-byte aligned", name);
        return DELS_OK;
    }
    if (layout != DELS_LAYOUT_MFMA16) return fail(DELS_ERR_INVALID_ARGUMENT, "%s: unknown layout %d", name, layout);
    if (!p) return fail(DELS_ERR_INVALID_ARGUMENT, "%s is NULL", name);
    if (!aligned16(p)) return fail(DELS_ERR_ALIGNMENT, "packed %s must be 16-byte aligned", name);
    return DELS_OK;
}

// ---- workspace layouts -------------------------------------------------------

// Every layout starts with the control area and the decode words, [0, kDataOff).
struct LowrankLayout {
    size_t rank_off, part_off, argmax_off, total;
    SkinnyPlan plan;
};

static LowrankLayout lowrank_layout(int64_t M, int64_t d, int64_t r, int64_t V) {
    LowrankLayout L{};
    L.plan = plan_skinny(M, d, r, false);
    L.rank_off = kDataOff;
    L.part_off = L.rank_off + align256((size_t)M * r * 2);
    L.argmax_off = L.part_off + skinny_data_bytes(L.plan);
    // room for the bf16 argmax and for the e4m3 one (which also keeps the quantised rank)
    L.total = L.argmax_off + align256(std::max(argmax_data_bytes(M, r, V), argmax_fp8_data_bytes(M, r, V)));
    return L;
}

struct RolloutLayout {
    size_t part_off, argmax_off, total;   // the steps' kernels run in turn and share the partials
    SkinnyPlan rank_plan, gru_plan;
};

static RolloutLayout rollout_layout(int64_t batch, int64_t G, int64_t r, int64_t V) {
    RolloutLayout L{};
    L.rank_plan = plan_skinny(batch, G, r, false);
    L.gru_plan = plan_skinny(batch, G, G, true);
    L.part_off = kDataOff;
    L.argmax_off = L.part_off + std::max(skinny_data_bytes(L.rank_plan), skinny_data_bytes(L.gru_plan));
    L.total = L.argmax_off + align256(argmax_data_bytes(batch, r, V));
    return L;
}

// ---- argument checks shared by several entry points ----------------------------

static int check_argmax_args(const void* rank, int64_t ldrank, const void* B, int64_t ldb, int b_layout,
                             const void* base, int64_t ldbase, int base_dtype,
                             const void* prior, int prior_dtype,
                             const float* alpha, int64_t alpha_stride,
                             const float* beta, int64_t beta_stride,
                             int64_t M, int64_t r, int64_t V,
                             const int64_t* out_ids, int64_t ld_out, bool check_rank) {
    if (M < 0 || r <= 0 || V <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "bad shape M=%lld r=%lld V=%lld",
                                               (long long)M, (long long)r, (long long)V);
    if (V >= INT32_MAX || M >= INT32_MAX) return fail(DELS_ERR_UNSUPPORTED, "M and V must be < 2^31-1");
    if (r % 8 != 0) return fail(DELS_ERR_UNSUPPORTED, "rank dimension r=%lld must be a multiple of 8", (long long)r);
    if (!argmax_supported(M, r, V)) return fail(DELS_ERR_UNSUPPORTED, "rank dimension r=%lld not supported (8..512)",
                                                (long long)r);
    if (M == 0) return DELS_OK;   // nothing to read or write
    int rc;
    if (check_rank && (rc = check_bf16_matrix(rank, ldrank, r, "rank")) != DELS_OK) return rc;
    if ((rc = check_weight(B, ldb, r, b_layout, "B (low-rank LM head)")) != DELS_OK) return rc;
    if (!base) return fail(DELS_ERR_INVALID_ARGUMENT, "base logits pointer is NULL");
    if (!valid_dtype(base_dtype)) return fail(DELS_ERR_INVALID_ARGUMENT, "unknown base dtype %d", base_dtype);
    if (M > 1 && ldbase < V) return fail(DELS_ERR_INVALID_ARGUMENT, "base leading dimension %lld < V %lld",
                                         (long long)ldbase, (long long)V);
    if (prior && !valid_dtype(prior_dtype)) return fail(DELS_ERR_INVALID_ARGUMENT, "unknown prior dtype %d", prior_dtype);
    if (!alpha || !beta) return fail(DELS_ERR_INVALID_ARGUMENT, "alpha/beta pointers must be non-NULL");
    if (alpha_stride < 0 || beta_stride < 0) return fail(DELS_ERR_INVALID_ARGUMENT, "negative alpha/beta stride");
    if (!ld_ok({ldbase, alpha_stride, beta_stride, ld_out}))
        return fail(DELS_ERR_INVALID_ARGUMENT, "leading dimension or stride out of range");
    if (!out_ids) return fail(DELS_ERR_INVALID_ARGUMENT, "out_ids is NULL");
    if (M > 1 && ld_out < 1) return fail(DELS_ERR_INVALID_ARGUMENT, "ld_out must be >= 1");
    return DELS_OK;
}

static int check_ws(const void* ws, size_t ws_bytes, size_t need) {
    if (need == 0) return fail(DELS_ERR_UNSUPPORTED, "shape past the supported extents");
    if (!ws) return fail(DELS_ERR_WORKSPACE, "workspace is NULL (%zu bytes needed)", need);
    if ((reinterpret_cast<uintptr_t>(ws) & 255u) != 0) return fail(DELS_ERR_WORKSPACE, "workspace must be 256-byte aligned");
    if (ws_bytes < need) return fail(DELS_ERR_WORKSPACE, "workspace too small: %zu bytes given, %zu needed", ws_bytes, need);
    return DELS_OK;
}

static int check_gru_args(const void* gi_table, int64_t ld_gi, int64_t table_rows, const int64_t* tokens,
                          const void* h_in, int64_t ldh_in, const void* w_hh, int w_layout, int64_t batch,
                          int64_t G, const void* h_out, int64_t ldh_out) {
    if (batch < 0 || G <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "bad GRU shape batch=%lld G=%lld",
                                         (long long)batch, (long long)G);
    if (batch > 64) return fail(DELS_ERR_UNSUPPORTED, "GRU step supports batch <= 64 (got %lld)", (long long)batch);
    if (G >= (1 << 24)) return fail(DELS_ERR_UNSUPPORTED, "GRU hidden size too large");
    if (G % 8 != 0) return fail(DELS_ERR_UNSUPPORTED, "GRU hidden size %lld must be a multiple of 8", (long long)G);
    if (batch == 0) return DELS_OK;
    if (!gi_table || table_rows <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "GRU input table is NULL or empty");
    if (ld_gi < 3 * G) return fail(DELS_ERR_INVALID_ARGUMENT, "GRU input table leading dimension < 3G");
    if (!ld_ok({ld_gi, ldh_out})) return fail(DELS_ERR_INVALID_ARGUMENT, "GRU leading dimension out of range");
    if (!tokens) return fail(DELS_ERR_INVALID_ARGUMENT, "token ids pointer is NULL");
    int rc;
    if (h_in && (rc = check_bf16_matrix(h_in, ldh_in, G, "h_in")) != DELS_OK) return rc;
    if ((rc = check_weight(w_hh, G, G, w_layout, "W_hh")) != DELS_OK) return rc;
    if (w_layout == DELS_LAYOUT_MFMA16 && G % 16 != 0)
        return fail(DELS_ERR_UNSUPPORTED, "packed W_hh needs a hidden size divisible by 16");
    if (!h_out) return fail(DELS_ERR_INVALID_ARGUMENT, "h_out is NULL");
    if (batch > 1 && ldh_out < G) return fail(DELS_ERR_INVALID_ARGUMENT, "h_out leading dimension < G");
    if (h_in && h_in == h_out) return fail(DELS_ERR_INVALID_ARGUMENT, "h_in and h_out must not alias");
    return DELS_OK;
}

// ---- rollout ---------------------------------------------------------------------

static int check_rollout(const dels_rollout* p) {
    if (!p) return fail(DELS_ERR_INVALID_ARGUMENT, "rollout parameters are NULL");
    if (p->steps <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "rollout requires steps > 0, got %lld", (long long)p->steps);
    if (p->batch <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "rollout requires batch > 0");
    if (!rows_ok(p->steps) || !rows_ok(p->r) || !vocab_ok(p->V))
        return fail(DELS_ERR_UNSUPPORTED, "rollout: steps and r below 2^24, V below 2^31-1");
    if (p->act != DELS_ACT_IDENTITY && p->act != DELS_ACT_SILU)
        return fail(DELS_ERR_INVALID_ARGUMENT, "unknown rank activation %d", p->act);
    if (p->ld_prefix < 0 || !ld_ok({p->ld_prefix, p->ld_out}))
        return fail(DELS_ERR_INVALID_ARGUMENT, "rollout ld_prefix / ld_out out of range");
    if (p->ld_out != 0 && p->ld_out < p->steps)
        return fail(DELS_ERR_INVALID_ARGUMENT, "rollout ld_out %lld < steps %lld", (long long)p->ld_out,
                    (long long)p->steps);
    int rc = check_gru_args(p->gi_table, p->ld_gi, p->table_rows, p->prefix_ids, p->h_a, p->G, p->w_hh,
                            p->weights_layout, p->batch, p->G, p->h_b, p->G);
    if (rc != DELS_OK) return rc;
    if ((rc = check_bf16_matrix(p->h_b, p->G, p->G, "h_b")) != DELS_OK) return rc;
    if ((rc = check_weight(p->rank_w, p->G, p->G, p->weights_layout, "rank_w")) != DELS_OK) return rc;
    if (p->ld_base != 0 && p->ld_base < p->steps * p->V)
        return fail(DELS_ERR_INVALID_ARGUMENT, "rollout ld_base %lld < steps * V", (long long)p->ld_base);
    if ((rc = check_argmax_args(p->rank, p->r, p->lm_w, p->r, p->weights_layout, p->base,
                                p->ld_base ? p->ld_base : p->steps * p->V, p->base_dtype, p->prior,
                                p->prior_dtype, p->alpha, 0, p->beta, 0, p->batch, p->r, p->V, p->out_ids,
                                p->ld_out ? p->ld_out : p->steps, true)) != DELS_OK)
        return rc;
    const RolloutLayout L = rollout_layout(p->batch, p->G, p->r, p->V);
    if (!skinny_supported(L.rank_plan) || !skinny_supported(L.gru_plan))
        return fail(DELS_ERR_UNSUPPORTED, "rollout shape needs too many workgroup tiles");
    return check_ws(p->ws, p->ws_bytes, L.total);
}

static int enqueue_rollout(const dels_rollout* p, hipStream_t s) {
    const RolloutLayout L = rollout_layout(p->batch, p->G, p->r, p->V);
    char* ws = static_cast<char*>(p->ws);
    const int B = (int)p->batch, G = (int)p->G, r = (int)p->r, V = (int)p->V;
    const int64_t ldp = p->ld_prefix ? p->ld_prefix : 1;         // prefix id of row b at [b * ldp]
    const int64_t ldo = p->ld_out ? p->ld_out : p->steps;        // id of row b, step s at [b * ldo + s]

    GruArgs g{};
    g.gi_table = static_cast<const uint16_t*>(p->gi_table);
    g.ld_gi = p->ld_gi;
    g.table_rows = p->table_rows;
    g.w_hh = static_cast<const uint16_t*>(p->w_hh);
    g.w_packed = p->weights_layout == DELS_LAYOUT_MFMA16;
    g.b_hh = static_cast<const uint16_t*>(p->b_hh);
    g.batch = B;
    g.G = G;

    uint16_t* h_cur = static_cast<uint16_t*>(p->h_a);
    uint16_t* h_next = static_cast<uint16_t*>(p->h_b);
    const size_t esz = dtype_size(p->base_dtype);
    const bool packed = p->weights_layout == DELS_LAYOUT_MFMA16;
    if (rollout_resident_enabled() && rollout_resident_eligible(B, G, r, V, p->steps, packed)) {
        // every step in one launch with B held on chip (rollout_resident.hip)
        ResidentRolloutArgs ra{};
        ra.w_hh = g.w_hh; ra.b_hh = g.b_hh;
        ra.A = static_cast<const uint16_t*>(p->rank_w); ra.rank_b = static_cast<const uint16_t*>(p->rank_b);
        ra.act = p->act;
        ra.B = static_cast<const uint16_t*>(p->lm_w);
        ra.gi_table = g.gi_table; ra.ld_gi = g.ld_gi; ra.table_rows = g.table_rows;
        ra.prefix = p->prefix_ids; ra.ld_prefix = ldp;
        ra.base = p->base; ra.ld_base = p->ld_base ? p->ld_base : p->steps * (int64_t)V;
        ra.base_dtype = p->base_dtype;
        ra.prior = p->prior; ra.prior_dtype = p->prior_dtype;
        ra.alpha = p->alpha; ra.beta = p->beta;
        ra.batch = B; ra.G = G; ra.V = V; ra.steps = p->steps;
        ra.out_ids = p->out_ids; ra.out_scores = p->out_scores; ra.ld_out = ldo;
        hipError_t e = launch_rollout_resident(ra, ws, s);
        return e == hipSuccess ? DELS_OK : hip_fail(e, "resident rollout launch");
    }
    const bool use_decode = G >= kRolloutDecodeMinG && decode_eligible(B, G, r, packed, packed);
    // every step advances the GRU inside its decode launch, the first one from
    // the zero state on the prefix ids: no GRU launch at all
    const bool fuse_gru = use_decode && decode_gru_eligible(B, G, r);
    hipError_t e = hipSuccess;
    if (!fuse_gru) {
        // h0 = GRU(gi_table[prefix], 0)   (code/kernel/dels.py:426-433)
        g.tokens = p->prefix_ids;
        g.tok_stride = ldp;
        g.h_in = nullptr;
        g.ldh_in = G;
        g.h_out = h_cur;
        g.ldh_out = G;
        e = launch_gru_step(g, L.gru_plan, ws, L.part_off, s);
        if (e != hipSuccess) return hip_fail(e, "GRU step launch");
    }
    for (int step = 0; step < p->steps; ++step) {
        RankArgs ra{};
        ra.h = h_cur; ra.ldh = G;
        ra.A = static_cast<const uint16_t*>(p->rank_w); ra.lda = G;
        ra.a_packed = p->weights_layout == DELS_LAYOUT_MFMA16;
        ra.bias = static_cast<const uint16_t*>(p->rank_b); ra.act = p->act;
        ra.M = B; ra.d = G; ra.r = r;
        ra.rank = static_cast<uint16_t*>(p->rank); ra.ldrank = r;

        ArgmaxArgs aa{};
        aa.rank = static_cast<const uint16_t*>(p->rank); aa.ldrank = r;
        aa.B = static_cast<const uint16_t*>(p->lm_w); aa.ldb = r;
        aa.b_packed = p->weights_layout == DELS_LAYOUT_MFMA16;
        aa.base = static_cast<const char*>(p->base) + (size_t)step * V * esz;
        aa.ldbase = p->ld_base ? p->ld_base : p->steps * (int64_t)V;
        aa.base_dtype = p->base_dtype;
        aa.prior = p->prior; aa.prior_dtype = p->prior_dtype;
        aa.alpha = p->alpha + step; aa.alpha_stride = 0;
        aa.beta = p->beta + step; aa.beta_stride = 0;
        aa.M = B; aa.r = r; aa.V = V;
        aa.out_ids = p->out_ids + step;
        aa.out_score = p->out_scores ? p->out_scores + step : nullptr;
        aa.ld_out = ldo;

        if (fuse_gru) {
            // h = GRU(gi_table[previous ids], h) -- step 0: GRU(gi_table[prefix], 0)
            // (code/kernel/dels.py:426-433) --, rank projection and argmax in one launch
            DecodeGru dg{};
            dg.gi_table = g.gi_table; dg.ld_gi = g.ld_gi; dg.table_rows = g.table_rows;
            dg.w_hh = g.w_hh; dg.b_hh = g.b_hh;
            if (step == 0) {
                dg.tokens = p->prefix_ids; dg.tok_stride = ldp;
                dg.h_prev = nullptr; dg.h_out = h_cur;
                ra.h = h_cur;
            } else {
                dg.tokens = p->out_ids + (step - 1); dg.tok_stride = ldo;
                dg.h_prev = h_cur; dg.h_out = h_next;
                ra.h = h_next;
            }
            e = launch_lowrank_decode(ra, aa, ws, s, &dg);
            if (e != hipSuccess) return hip_fail(e, "fused rollout step launch");
            if (step > 0) std::swap(h_cur, h_next);
        } else if (use_decode) {
            // rank projection and argmax in one launch
            e = launch_lowrank_decode(ra, aa, ws, s);
            if (e != hipSuccess) return hip_fail(e, "fused decode step launch");
        } else {
            e = launch_rank_proj(ra, L.rank_plan, ws, L.part_off, s);
            if (e != hipSuccess) return hip_fail(e, "rank projection launch");
            e = launch_fused_argmax(aa, ws, L.argmax_off, s);
            if (e != hipSuccess) return hip_fail(e, "fused argmax launch");
        }

        if (step + 1 < p->steps && !fuse_gru) {
            g.tokens = p->out_ids + step;
            g.tok_stride = ldo;
            g.h_in = h_cur;
            g.h_out = h_next;
            e = launch_gru_step(g, L.gru_plan, ws, L.part_off, s);
            if (e != hipSuccess) return hip_fail(e, "GRU step launch");
            std::swap(h_cur, h_next);
        }
    }
    return DELS_OK;
}

struct GraphHandle {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

// One eager run of `enqueue` on a private stream (resolves per-kernel launch
// configuration outside capture), then the same work captured into a graph.
template <typename Enqueue>
static int capture_graph(Enqueue enqueue, void** graph_out) {
    hipStream_t cs = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&cs, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_fail(e, "capture stream creation");
    int rc = enqueue(cs);
    if (rc == DELS_OK && (e = hipStreamSynchronize(cs)) != hipSuccess) rc = hip_fail(e, "warm-up run");
    hipGraph_t graph = nullptr;
    if (rc == DELS_OK) {
        e = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) {
            rc = hip_fail(e, "hipStreamBeginCapture");
        } else {
            rc = enqueue(cs);
            hipError_t e2 = hipStreamEndCapture(cs, &graph);
            if (rc == DELS_OK && e2 != hipSuccess) rc = hip_fail(e2, "hipStreamEndCapture");
        }
    }
    hipGraphExec_t exec = nullptr;
    if (rc == DELS_OK && (e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0)) != hipSuccess)
        rc = hip_fail(e, "hipGraphInstantiate");
    (void)hipStreamDestroy(cs);
    if (rc != DELS_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    *graph_out = new GraphHandle{graph, exec};
    return DELS_OK;
}

// ---- Markov rollout ----------------------------------------------------------------

static int check_markov(const dels_markov_rollout* p) {
    if (!p) return fail(DELS_ERR_INVALID_ARGUMENT, "Markov rollout parameters are NULL");
    if (p->steps <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "Markov rollout requires steps > 0, got %lld",
                                   (long long)p->steps);
    if (p->batch <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "Markov rollout requires batch > 0");
    if (!rows_ok(p->steps) || !rows_ok(p->r) || !vocab_ok(p->V))
        return fail(DELS_ERR_UNSUPPORTED, "Markov rollout: steps and r below 2^24, V below 2^31-1");
    if (!p->prev_ids) return fail(DELS_ERR_INVALID_ARGUMENT, "prev_ids is NULL");
    if (p->table_rows <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "embedding table is empty");
    int rc = check_bf16_matrix(p->embedding, p->ld_embedding, p->r, "embedding");
    if (rc != DELS_OK) return rc;
    if (p->ld_base != 0 && p->ld_base < p->steps * p->V)
        return fail(DELS_ERR_INVALID_ARGUMENT, "Markov rollout ld_base %lld < steps * V", (long long)p->ld_base);
    if ((rc = check_argmax_args(nullptr, p->r, p->lm_w, p->r, p->lm_layout, p->base,
                                p->ld_base ? p->ld_base : p->steps * p->V, p->base_dtype, p->prior, p->prior_dtype,
                                p->alpha, 0, p->beta, 0, p->batch, p->r, p->V, p->out_ids, p->steps, false)) != DELS_OK)
        return rc;
    return check_ws(p->ws, p->ws_bytes, kDataOff + align256(argmax_data_bytes(p->batch, p->r, p->V)));
}

static ArgmaxArgs gather_args(const int64_t* tokens, int64_t tok_stride, const void* E, int64_t lde,
                              int64_t table_rows, const void* B, int64_t ldb, int b_layout, const void* base,
                              int64_t ldbase, int base_dtype, const void* prior, int prior_dtype, const float* alpha,
                              int64_t alpha_stride, const float* beta, int64_t beta_stride, int64_t M, int64_t r,
                              int64_t V, int64_t* out_ids, float* out_score, int64_t ld_out) {
    ArgmaxArgs a{};
    a.rank = static_cast<const uint16_t*>(E); a.ldrank = lde;
    a.rank_rows = tokens; a.rank_rows_stride = tok_stride; a.rank_rows_count = table_rows;
    a.B = static_cast<const uint16_t*>(B); a.ldb = ldb; a.b_packed = b_layout == DELS_LAYOUT_MFMA16;
    a.base = base; a.ldbase = ldbase; a.base_dtype = base_dtype;
    a.prior = prior; a.prior_dtype = prior_dtype;
    a.alpha = alpha; a.alpha_stride = alpha_stride;
    a.beta = beta; a.beta_stride = beta_stride;
    a.M = (int)M; a.r = (int)r; a.V = (int)V;
    a.out_ids = out_ids; a.out_score = out_score; a.ld_out = ld_out;
    return a;
}

static int enqueue_markov(const dels_markov_rollout* p, hipStream_t s) {
    const size_t esz = dtype_size(p->base_dtype);
    const int64_t ldbase = p->ld_base ? p->ld_base : p->steps * p->V;
    for (int64_t step = 0; step < p->steps; ++step) {
        // token_s: the previous token for the first step, then the step before's pick
        const int64_t* tok = step == 0 ? p->prev_ids : p->out_ids + (step - 1);
        const int64_t tok_stride = step == 0 ? 1 : p->steps;
        ArgmaxArgs a = gather_args(tok, tok_stride, p->embedding, p->ld_embedding, p->table_rows, p->lm_w, p->r,
                                   p->lm_layout, static_cast<const char*>(p->base) + (size_t)step * p->V * esz,
                                   ldbase, p->base_dtype, p->prior, p->prior_dtype, p->alpha + step, 0,
                                   p->beta + step, 0, p->batch, p->r, p->V, p->out_ids + step,
                                   p->out_scores ? p->out_scores + step : nullptr, p->steps);
        hipError_t e = launch_fused_argmax(a, p->ws, kDataOff, s);
        if (e != hipSuccess) return hip_fail(e, "Markov argmax launch");
    }
    return DELS_OK;
}

// ---- scratch of the allocation-free draft step ------------------------------------
//
// dels_lowrank_argmax_noalloc runs dels_lowrank_argmax with its workspace in
// this file-scope device array instead of caller memory.  Every GPU the
// library runs on holds its own copy until the process ends.  In host code the
// name `scratch` is only a host-side stand-in: the device address of each
// GPU's copy comes from hipGetSymbolAddress (with that GPU current) and is
// kept per device; only that address is ever passed to kernels.
static __device__ __align__(256) unsigned char scratch[DELS_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxScratchDevices];   // device address of `scratch` per device; null until set up
}  // namespace

// The current device's scratch address.  On the device's first call: look the
// address up, then zero the array once with the fill kernel on `s`, ahead of
// the call's own kernels (the workspace contract: zeroed before first use).
// That fill must not be captured -- a graph would replay it and reset the
// decode step's launch generation on every replay -- so a first call under
// stream capture is refused.
static int scratch_address(hipStream_t s, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxScratchDevices) return fail(DELS_ERR_UNSUPPORTED, "device id %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
        if ((e = hipStreamIsCapturing(s, &status)) != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
        if (status != hipStreamCaptureStatusNone)
            return fail(DELS_ERR_INVALID_ARGUMENT,
                        "the first dels_lowrank_argmax_noalloc call on a device clears its scratch array and "
                        "must not be captured: make one call outside stream capture first");
        void* addr = nullptr;
        if ((e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch))) != hipSuccess)
            return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if ((e = launch_fill_zero(addr, DELS_NOALLOC_SCRATCH_BYTES, s)) != hipSuccess)
            return hip_fail(e, "scratch zero fill launch");
        g_scratch_addr[dev] = addr;
    }
    *out = g_scratch_addr[dev];
    return DELS_OK;
}

// ---- Domino correction rollout ---------------------------------------------------

struct DominoLayout {
    size_t part_off, total;   // the projections and GRU steps run in turn and share the partials
    SkinnyPlan z_plan, s_plan, gru_plan;
};

static DominoLayout domino_layout(int64_t batch, int64_t steps, int64_t D, int64_t G, int64_t E) {
    DominoLayout L{};
    L.z_plan = plan_skinny(batch * steps, D, E, false);
    L.s_plan = plan_skinny(batch, G, E, false);
    L.gru_plan = plan_skinny(batch, G, G, true);
    L.part_off = kDataOff;
    L.total = L.part_off + std::max(skinny_data_bytes(L.z_plan),
                                    std::max(skinny_data_bytes(L.s_plan), skinny_data_bytes(L.gru_plan)));
    return L;
}

static int check_domino_step(const void* z, int64_t ldz, const void* sv, int64_t lds, const void* fc2_w,
                             const void* fc2_bias, int fc2_bias_dtype, const void* base, int64_t ldbase,
                             int base_dtype, float alpha, int middle, int64_t M, int64_t E, int64_t V,
                             const int64_t* out_ids, int64_t ld_out) {
    if (M < 0 || E <= 0 || V <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "bad shape M=%lld E=%lld V=%lld",
                                                (long long)M, (long long)E, (long long)V);
    if (V >= INT32_MAX || M > kMaxKeyRows) return fail(DELS_ERR_UNSUPPORTED, "Domino step: M <= %d, V < 2^31-1",
                                                       kMaxKeyRows);
    if (E % 32 != 0 || E > kDominoMaxE)
        return fail(DELS_ERR_UNSUPPORTED, "Domino step: E=%lld must be a multiple of 32 and at most %d",
                    (long long)E, kDominoMaxE);
    if (!(alpha == alpha)) return fail(DELS_ERR_INVALID_ARGUMENT, "guidance alpha is NaN");
    if (middle < DELS_MIDDLE_SILU || middle > DELS_MIDDLE_SIGMOID)
        return fail(DELS_ERR_INVALID_ARGUMENT, "unknown Domino middle layer %d (DELS_MIDDLE_*)", middle);
    if (M == 0) return DELS_OK;
    if (!z || !sv) return fail(DELS_ERR_INVALID_ARGUMENT, "z or s is NULL");
    if ((M > 1 && (ldz < E || lds < E)) || ldz < 0 || lds < 0)
        return fail(DELS_ERR_INVALID_ARGUMENT, "z/s leading dimension < E");
    if (!ld_ok({ldz, lds, ldbase, ld_out})) return fail(DELS_ERR_INVALID_ARGUMENT, "leading dimension out of range");
    if (!fc2_w) return fail(DELS_ERR_INVALID_ARGUMENT, "fc2 weight is NULL");
    if (!aligned16(fc2_w)) return fail(DELS_ERR_ALIGNMENT, "packed fc2 weight must be 16-byte aligned");
    if (fc2_bias && !valid_dtype(fc2_bias_dtype)) return fail(DELS_ERR_INVALID_ARGUMENT, "unknown fc2 bias dtype %d",
                                                               fc2_bias_dtype);
    if (!base) return fail(DELS_ERR_INVALID_ARGUMENT, "base logits pointer is NULL");
    if (!valid_dtype(base_dtype)) return fail(DELS_ERR_INVALID_ARGUMENT, "unknown base dtype %d", base_dtype);
    if (M > 1 && ldbase < V) return fail(DELS_ERR_INVALID_ARGUMENT, "base leading dimension %lld < V %lld",
                                         (long long)ldbase, (long long)V);
    if (!out_ids) return fail(DELS_ERR_INVALID_ARGUMENT, "out_ids is NULL");
    if (M > 1 && ld_out < 1) return fail(DELS_ERR_INVALID_ARGUMENT, "ld_out must be >= 1");
    return DELS_OK;
}

static DominoArgs domino_args(const void* z, int64_t ldz, const void* sv, int64_t lds, const void* fc2_w,
                              const void* fc2_bias, int fc2_bias_dtype, const void* base, int64_t ldbase,
                              int base_dtype, float alpha, int middle, int64_t M, int64_t E, int64_t V,
                              int64_t* out_ids, float* out_score, int64_t ld_out) {
    DominoArgs d{};
    d.z = static_cast<const uint16_t*>(z); d.ldz = ldz;
    d.s = static_cast<const uint16_t*>(sv); d.lds = lds;
    d.W = static_cast<const uint16_t*>(fc2_w);
    d.bias = fc2_bias; d.bias_dtype = fc2_bias_dtype;
    d.base = base; d.ldbase = ldbase; d.base_dtype = base_dtype;
    d.alpha = alpha;
    d.middle = middle;
    d.M = (int)M; d.E = (int)E; d.V = (int)V;
    d.out_ids = out_ids; d.out_score = out_score; d.ld_out = ld_out;
    return d;
}

static int check_domino_rollout(const dels_domino_rollout* p) {
    if (!p) return fail(DELS_ERR_INVALID_ARGUMENT, "Domino rollout parameters are NULL");
    if (p->steps <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "rollout requires steps > 0, got %lld",
                                   (long long)p->steps);
    if (p->batch <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "rollout requires batch > 0");
    if (p->prefix_len <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "Domino rollout requires prefix_len > 0");
    if (p->D <= 0 || p->D % 8 != 0) return fail(DELS_ERR_UNSUPPORTED, "hidden size D must be a positive multiple of 8");
    if (!rows_ok(p->steps) || !rows_ok(p->batch) || !rows_ok(p->batch * p->steps) || !inner_ok(p->D) ||
        !rows_ok(p->E) || !vocab_ok(p->V))
        return fail(DELS_ERR_UNSUPPORTED, "Domino rollout: batch * steps and E below 2^24, D below 2^26, "
                    "V below 2^31-1");
    int rc = check_gru_args(p->gi_table, p->ld_gi, p->table_rows, p->prefix_ids, p->h_a, p->G, p->w_hh,
                            p->weights_layout, p->batch, p->G, p->h_b, p->G);
    if (rc != DELS_OK) return rc;
    if ((rc = check_bf16_matrix(p->h_b, p->G, p->G, "h_b")) != DELS_OK) return rc;
    if ((rc = check_weight(p->w_z, p->D, p->D, p->weights_layout, "w_z")) != DELS_OK) return rc;
    if ((rc = check_weight(p->w_s, p->G, p->G, p->weights_layout, "w_s")) != DELS_OK) return rc;
    if ((rc = check_bf16_matrix(p->hiddens, p->D, p->D, "hiddens")) != DELS_OK) return rc;
    if ((rc = check_bf16_matrix(p->z, p->E, p->E, "z scratch")) != DELS_OK) return rc;
    if ((rc = check_bf16_matrix(p->s, p->E, p->E, "s scratch")) != DELS_OK) return rc;
    if (p->ld_base != 0 && p->ld_base < p->steps * p->V)
        return fail(DELS_ERR_INVALID_ARGUMENT, "rollout ld_base %lld < steps * V", (long long)p->ld_base);
    if ((rc = check_domino_step(p->z, p->steps * p->E, p->s, p->E, p->fc2_w, p->fc2_bias, p->fc2_bias_dtype, p->base,
                                p->ld_base ? p->ld_base : p->steps * p->V, p->base_dtype, p->alpha, p->middle,
                                p->batch, p->E, p->V, p->out_ids, p->steps)) != DELS_OK)
        return rc;
    const DominoLayout L = domino_layout(p->batch, p->steps, p->D, p->G, p->E);
    if (!skinny_supported(L.z_plan) || !skinny_supported(L.s_plan) || !skinny_supported(L.gru_plan))
        return fail(DELS_ERR_UNSUPPORTED, "Domino rollout shape needs too many workgroup tiles");
    return check_ws(p->ws, p->ws_bytes, L.total);
}

static int enqueue_domino(const dels_domino_rollout* p, hipStream_t s) {
    const DominoLayout L = domino_layout(p->batch, p->steps, p->D, p->G, p->E);
    char* ws = static_cast<char*>(p->ws);
    const int B = (int)p->batch, S = (int)p->steps, G = (int)p->G, E = (int)p->E, V = (int)p->V;
    const bool packed = p->weights_layout == DELS_LAYOUT_MFMA16;

    // z = F.linear(parallel_hiddens, w_z, fc1_bias) for every step at once  (code/kernel/domino.py:386-390)
    RankArgs rz{};
    rz.h = static_cast<const uint16_t*>(p->hiddens); rz.ldh = p->D;
    rz.A = static_cast<const uint16_t*>(p->w_z); rz.lda = p->D; rz.a_packed = packed;
    rz.bias = static_cast<const uint16_t*>(p->fc1_bias); rz.act = DELS_ACT_IDENTITY;
    rz.M = B * S; rz.d = (int)p->D; rz.r = E;
    rz.rank = static_cast<uint16_t*>(p->z); rz.ldrank = E;
    hipError_t e = launch_rank_proj(rz, L.z_plan, ws, L.part_off, s);
    if (e != hipSuccess) return hip_fail(e, "z projection launch");

    GruArgs g{};
    g.gi_table = static_cast<const uint16_t*>(p->gi_table);
    g.ld_gi = p->ld_gi;
    g.table_rows = p->table_rows;
    g.w_hh = static_cast<const uint16_t*>(p->w_hh);
    g.w_packed = packed;
    g.b_hh = static_cast<const uint16_t*>(p->b_hh);
    g.batch = B;
    g.G = G;
    g.ldh_in = G;
    g.ldh_out = G;

    // h = prefix_gru(embed_tokens(prefix_ids)) from h = 0, one cell per prefix id  (392-396)
    uint16_t* h_cur = static_cast<uint16_t*>(p->h_a);
    uint16_t* h_next = static_cast<uint16_t*>(p->h_b);
    for (int64_t j = 0; j < p->prefix_len; ++j) {
        g.tokens = p->prefix_ids + j;
        g.tok_stride = p->prefix_len;
        g.h_in = j == 0 ? nullptr : h_cur;
        g.h_out = j == 0 ? h_cur : h_next;
        e = launch_gru_step(g, L.gru_plan, ws, L.part_off, s);
        if (e != hipSuccess) return hip_fail(e, "GRU step launch");
        if (j > 0) std::swap(h_cur, h_next);
    }

    const size_t esz = dtype_size(p->base_dtype);
    for (int t = 0; t < S; ++t) {
        // s = F.linear(h, w_s)   (400-402)
        RankArgs rs{};
        rs.h = h_cur; rs.ldh = G;
        rs.A = static_cast<const uint16_t*>(p->w_s); rs.lda = G; rs.a_packed = packed;
        rs.bias = nullptr; rs.act = DELS_ACT_IDENTITY;
        rs.M = B; rs.d = G; rs.r = E;
        rs.rank = static_cast<uint16_t*>(p->s); rs.ldrank = E;
        e = launch_rank_proj(rs, L.s_plan, ws, L.part_off, s);
        if (e != hipSuccess) return hip_fail(e, "s projection launch");

        // the fused correction step on z[:, t], s and base[:, t]   (404-410, 419)
        const DominoArgs d = domino_args(static_cast<const char*>(p->z) + (size_t)t * E * 2, (int64_t)S * E, p->s, E,
                                         p->fc2_w, p->fc2_bias, p->fc2_bias_dtype,
                                         static_cast<const char*>(p->base) + (size_t)t * V * esz,
                                         p->ld_base ? p->ld_base : (int64_t)S * V, p->base_dtype, p->alpha,
                                         p->middle, B, E, V,
                                         p->out_ids + t, p->out_scores ? p->out_scores + t : nullptr, S);
        e = launch_domino_argmax(d, ws, s);
        if (e != hipSuccess) return hip_fail(e, "Domino step launch");

        if (t + 1 < S) {   // GRU step on the chosen ids   (421-428)
            g.tokens = p->out_ids + t;
            g.tok_stride = S;
            g.h_in = h_cur;
            g.h_out = h_next;
            e = launch_gru_step(g, L.gru_plan, ws, L.part_off, s);
            if (e != hipSuccess) return hip_fail(e, "GRU step launch");
            std::swap(h_cur, h_next);
        }
    }
    return DELS_OK;
}

}  // namespace dels

using namespace dels;

extern "C" {

int dels_abi_version(void) { return DELS_ABI_VERSION; }

const char* dels_strerror(int status) {
    switch (status) {
        case DELS_OK: return "success";
        case DELS_ERR_INVALID_ARGUMENT: return "invalid argument";
        case DELS_ERR_UNSUPPORTED: return "unsupported shape or type";
        case DELS_ERR_ALIGNMENT: return "misaligned operand";
        case DELS_ERR_WORKSPACE: return "workspace missing, misaligned or too small";
        case DELS_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

const char* dels_last_error(void) { return g_last_error.c_str(); }

int dels_workspace_init(void* ws, size_t ws_bytes, void* stream) {
    if (ws_bytes == 0) return DELS_OK;
    if (!ws) return fail(DELS_ERR_WORKSPACE, "workspace is NULL");
    if ((reinterpret_cast<uintptr_t>(ws) & 255u) != 0 || (ws_bytes % 4) != 0)
        return fail(DELS_ERR_WORKSPACE, "workspace must be 256-byte aligned with a size divisible by 4");
    hipError_t e = launch_fill_zero(ws, ws_bytes, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "workspace fill launch");
}

size_t dels_packed_bytes(int64_t rows, int64_t cols) {
    if (rows <= 0 || cols <= 0 || !vocab_ok(rows) || !inner_ok(cols)) return 0;
    return packed_bytes(rows, cols);
}

int dels_pack_operand(const void* W, int64_t ldw, int64_t rows, int64_t cols, void* packed, size_t packed_bytes_,
                      void* stream) {
    if (rows < 0 || cols < 0) return fail(DELS_ERR_INVALID_ARGUMENT, "bad shape to pack");
    if (!vocab_ok(rows) || !inner_ok(cols)) return fail(DELS_ERR_UNSUPPORTED, "pack: rows below 2^31-1, cols below 2^26");
    if (rows == 0 || cols == 0) return DELS_OK;
    int rc = check_bf16_matrix(W, ldw, cols, "W (to pack)");
    if (rc != DELS_OK) return rc;
    if (!packed || !aligned16(packed)) return fail(DELS_ERR_ALIGNMENT, "packed output must be 16-byte aligned");
    if (packed_bytes_ < packed_bytes(rows, cols))
        return fail(DELS_ERR_INVALID_ARGUMENT, "packed output too small: %zu bytes given, %zu needed", packed_bytes_,
                    packed_bytes(rows, cols));
    hipError_t e = launch_pack_mfma16(static_cast<const uint16_t*>(W), ldw, rows, cols, static_cast<uint16_t*>(packed),
                                      static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "pack launch");
}

size_t dels_rank_proj_ws_bytes(int64_t M, int64_t d, int64_t r) {
    if (!rows_ok(M) || !inner_ok(d) || !rows_ok(r)) return 0;
    return kDataOff + skinny_data_bytes(plan_skinny(std::max<int64_t>(M, 1), std::max<int64_t>(d, 1),
                                                      std::max<int64_t>(r, 1), false));
}

int dels_rank_proj(const void* h, int64_t ldh, const void* A, int64_t lda, int a_layout, const void* bias, int act,
                   int64_t M, int64_t d, int64_t r, void* rank, int64_t ldrank, void* ws, size_t ws_bytes,
                   void* stream) {
    if (M < 0 || d <= 0 || r <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "bad rank projection shape");
    if (M >= (1 << 24) || d >= (1 << 26) || r >= (1 << 24)) return fail(DELS_ERR_UNSUPPORTED, "shape too large");
    if (d % 8 != 0) return fail(DELS_ERR_UNSUPPORTED, "hidden size d=%lld must be a multiple of 8", (long long)d);
    if (act != DELS_ACT_IDENTITY && act != DELS_ACT_SILU)
        return fail(DELS_ERR_INVALID_ARGUMENT, "Unsupported DeLS rank_activation code %d", act);
    if (M == 0) return DELS_OK;
    int rc;
    if ((rc = check_bf16_matrix(h, ldh, d, "h")) != DELS_OK) return rc;
    if ((rc = check_weight(A, lda, d, a_layout, "A (rank projection)")) != DELS_OK) return rc;
    if (!rank) return fail(DELS_ERR_INVALID_ARGUMENT, "rank output is NULL");
    if (ldrank < r) return fail(DELS_ERR_INVALID_ARGUMENT, "rank leading dimension < r");
    const SkinnyPlan p = plan_skinny(M, d, r, false);
    if (!skinny_supported(p)) return fail(DELS_ERR_UNSUPPORTED, "rank projection shape needs too many tiles");
    if ((rc = check_ws(ws, ws_bytes, kDataOff + skinny_data_bytes(p))) != DELS_OK) return rc;
    RankArgs ra{};
    ra.h = static_cast<const uint16_t*>(h); ra.ldh = ldh;
    ra.A = static_cast<const uint16_t*>(A); ra.lda = lda; ra.a_packed = a_layout == DELS_LAYOUT_MFMA16;
    ra.bias = static_cast<const uint16_t*>(bias); ra.act = act;
    ra.M = (int)M; ra.d = (int)d; ra.r = (int)r;
    ra.rank = static_cast<uint16_t*>(rank); ra.ldrank = ldrank;
    hipError_t e = launch_rank_proj(ra, p, ws, kDataOff, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "rank projection launch");
}

size_t dels_fused_argmax_ws_bytes(int64_t M, int64_t r, int64_t V) {
    if (!rows_ok(M) || !rows_ok(r) || !vocab_ok(V)) return 0;
    return kDataOff + align256(argmax_data_bytes(M, r, V));
}

int dels_fused_argmax(const void* rank, int64_t ldrank, const void* B, int64_t ldb, int b_layout, const void* base,
                      int64_t ldbase, int base_dtype, const void* prior, int prior_dtype, const float* alpha,
                      int64_t alpha_stride, const float* beta, int64_t beta_stride, int64_t M, int64_t r,
                      int64_t V, int64_t* out_ids, float* out_score, int64_t ld_out, void* ws, size_t ws_bytes,
                      void* stream) {
    int rc = check_argmax_args(rank, ldrank, B, ldb, b_layout, base, ldbase, base_dtype, prior, prior_dtype, alpha,
                               alpha_stride, beta, beta_stride, M, r, V, out_ids, ld_out, true);
    if (rc != DELS_OK) return rc;
    if (M == 0) return DELS_OK;
    if ((rc = check_ws(ws, ws_bytes, dels_fused_argmax_ws_bytes(M, r, V))) != DELS_OK) return rc;
    ArgmaxArgs a{};
    a.rank = static_cast<const uint16_t*>(rank); a.ldrank = ldrank;
    a.B = static_cast<const uint16_t*>(B); a.ldb = ldb; a.b_packed = b_layout == DELS_LAYOUT_MFMA16;
    a.base = base; a.ldbase = ldbase; a.base_dtype = base_dtype;
    a.prior = prior; a.prior_dtype = prior_dtype;
    a.alpha = alpha; a.alpha_stride = alpha_stride;
    a.beta = beta; a.beta_stride = beta_stride;
    a.M = (int)M; a.r = (int)r; a.V = (int)V;
    a.out_ids = out_ids; a.out_score = out_score; a.ld_out = ld_out;
    hipError_t e = launch_fused_argmax(a, ws, kDataOff, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "fused argmax launch");
}

int dels_debug_set_decode_spin_limit(int limit) { return set_decode_spin_limit(limit); }
int dels_debug_set_rollout_resident(int enable) { return set_rollout_resident(enable); }
int dels_debug_set_resident_spin_limit(int limit) { return set_resident_spin_limit(limit); }

size_t dels_lowrank_argmax_ws_bytes(int64_t M, int64_t d, int64_t r, int64_t V) {
    if (!rows_ok(M) || !inner_ok(d) || !rows_ok(r) || !vocab_ok(V)) return 0;
    return lowrank_layout(std::max<int64_t>(M, 1), std::max<int64_t>(d, 1), std::max<int64_t>(r, 1),
                          std::max<int64_t>(V, 1)).total;
}

int dels_lowrank_argmax(const void* h, int64_t ldh, const void* A, int64_t lda, int a_layout, const void* bias,
                        int act, const void* B, int64_t ldb, int b_layout, const void* base, int64_t ldbase, int base_dtype,
                        const void* prior, int prior_dtype, const float* alpha, int64_t alpha_stride,
                        const float* beta, int64_t beta_stride, int64_t M, int64_t d, int64_t r, int64_t V,
                        int64_t* out_ids, float* out_score, int64_t ld_out, void* ws, size_t ws_bytes,
                        void* stream) {
    int rc = check_argmax_args(nullptr, r, B, ldb, b_layout, base, ldbase, base_dtype, prior, prior_dtype, alpha,
                               alpha_stride, beta, beta_stride, M, r, V, out_ids, ld_out, false);
    if (rc != DELS_OK) return rc;
    if (d <= 0 || d % 8 != 0 || !inner_ok(d))
        return fail(DELS_ERR_UNSUPPORTED, "hidden size d=%lld must be a positive multiple of 8 below 2^26",
                                          (long long)d);
    if (act != DELS_ACT_IDENTITY && act != DELS_ACT_SILU)
        return fail(DELS_ERR_INVALID_ARGUMENT, "Unsupported DeLS rank_activation code %d", act);
    if (M == 0) return DELS_OK;
    if ((rc = check_bf16_matrix(h, ldh, d, "h")) != DELS_OK) return rc;
    if ((rc = check_weight(A, lda, d, a_layout, "A (rank projection)")) != DELS_OK) return rc;
    const LowrankLayout L = lowrank_layout(M, d, r, V);
    if (!skinny_supported(L.plan)) return fail(DELS_ERR_UNSUPPORTED, "rank projection shape needs too many tiles");
    if ((rc = check_ws(ws, ws_bytes, L.total)) != DELS_OK) return rc;
    char* w = static_cast<char*>(ws);
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint16_t* rank = reinterpret_cast<uint16_t*>(w + L.rank_off);

    RankArgs ra{};
    ra.h = static_cast<const uint16_t*>(h); ra.ldh = ldh;
    ra.A = static_cast<const uint16_t*>(A); ra.lda = lda; ra.a_packed = a_layout == DELS_LAYOUT_MFMA16;
    ra.bias = static_cast<const uint16_t*>(bias); ra.act = act;
    ra.M = (int)M; ra.d = (int)d; ra.r = (int)r;
    ra.rank = rank; ra.ldrank = r;
    ArgmaxArgs a{};
    a.rank = rank; a.ldrank = r;
    a.B = static_cast<const uint16_t*>(B); a.ldb = ldb; a.b_packed = b_layout == DELS_LAYOUT_MFMA16;
    a.base = base; a.ldbase = ldbase; a.base_dtype = base_dtype;
    a.prior = prior; a.prior_dtype = prior_dtype;
    a.alpha = alpha; a.alpha_stride = alpha_stride;
    a.beta = beta; a.beta_stride = beta_stride;
    a.M = (int)M; a.r = (int)r; a.V = (int)V;
    a.out_ids = out_ids; a.out_score = out_score; a.ld_out = ld_out;
    hipError_t e;
    if (decode_eligible(M, d, r, ra.a_packed, a.b_packed)) {
        // few rows, packed weights: rank projection and argmax in one launch
        e = launch_lowrank_decode(ra, a, ws, s);
        return e == hipSuccess ? DELS_OK : hip_fail(e, "fused decode step launch");
    }
    e = launch_rank_proj(ra, L.plan, ws, L.part_off, s);
    if (e != hipSuccess) return hip_fail(e, "rank projection launch");
    e = launch_fused_argmax(a, ws, L.argmax_off, s);
    return e == hipSuccess ? DELS_OK : hip_fail(e, "fused argmax launch");
}

int dels_lowrank_argmax_noalloc(const void* h, int64_t ldh, const void* A, int64_t lda, int a_layout,
                                const void* bias, int act, const void* B, int64_t ldb, int b_layout,
                                const void* base, int64_t ldbase, int base_dtype, const void* prior,
                                int prior_dtype, const float* alpha, int64_t alpha_stride, const float* beta,
                                int64_t beta_stride, int64_t M, int64_t d, int64_t r, int64_t V, int64_t* out_ids,
                                float* out_score, int64_t ld_out, void* stream) {
    const size_t need = dels_lowrank_argmax_ws_bytes(M, d, r, V);
    if (need > DELS_NOALLOC_SCRATCH_BYTES)
        return fail(DELS_ERR_WORKSPACE,
                    "dels_lowrank_argmax_noalloc: M=%lld d=%lld r=%lld V=%lld needs %zu bytes of scratch, more "
                    "than the %zu-byte array; call dels_lowrank_argmax with a workspace instead",
                    (long long)M, (long long)d, (long long)r, (long long)V, need,
                    (size_t)DELS_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    const int rc = scratch_address(static_cast<hipStream_t>(stream), &ws);
    if (rc != DELS_OK) return rc;
    return dels_lowrank_argmax(h, ldh, A, lda, a_layout, bias, act, B, ldb, b_layout, base, ldbase, base_dtype,
                               prior, prior_dtype, alpha, alpha_stride, beta, beta_stride, M, d, r, V, out_ids,
                               out_score, ld_out, ws, DELS_NOALLOC_SCRATCH_BYTES, stream);
}

// ---- fp8 variant ---------------------------------------------------------------

static int check_scale(const float* p, const char* name) {
    if (!p) return fail(DELS_ERR_INVALID_ARGUMENT, "%s is NULL", name);
    if ((reinterpret_cast<uintptr_t>(p) & 3u) != 0) return fail(DELS_ERR_ALIGNMENT, "%s must be 4-byte aligned", name);
    return DELS_OK;
}

static bool fp8_rank_ok(int64_t r) { return r == 128 || r == 256 || r == 512; }

size_t dels_packed_fp8_bytes(int64_t rows, int64_t cols, int layout) {
    if (rows <= 0 || cols <= 0 || !vocab_ok(rows) || !inner_ok(cols)) return 0;
    if (layout != DELS_LAYOUT_FP8_K128 && layout != DELS_LAYOUT_FP8_K32) return 0;
    return packed_fp8_bytes(rows, cols, layout == DELS_LAYOUT_FP8_K128 ? FP8_K128 : FP8_K32);
}

int dels_pack_operand_fp8(const void* Wq, int64_t ldw, int64_t rows, int64_t cols, int layout, void* packed,
                          size_t packed_bytes_, void* stream) {
    if (rows < 0 || cols < 0) return fail(DELS_ERR_INVALID_ARGUMENT, "bad shape to pack");
    if (layout != DELS_LAYOUT_FP8_K128 && layout != DELS_LAYOUT_FP8_K32)
        return fail(DELS_ERR_INVALID_ARGUMENT, "unknown fp8 layout %d", layout);
    if (!vocab_ok(rows) || !inner_ok(cols)) return fail(DELS_ERR_UNSUPPORTED, "pack: rows below 2^31-1, cols below 2^26");
    if (rows == 0 || cols == 0) return DELS_OK;
    if (!Wq) return fail(DELS_ERR_INVALID_ARGUMENT, "W (to pack) is NULL");
    if (rows > 1 && ldw < cols) return fail(DELS_ERR_INVALID_ARGUMENT, "W leading dimension %lld < cols %lld",
                                            (long long)ldw, (long long)cols);
    if (!packed || !aligned16(packed)) return fail(DELS_ERR_ALIGNMENT, "packed output must be 16-byte aligned");
    const size_t need = dels_packed_fp8_bytes(rows, cols, layout);
    if (packed_bytes_ < need)
        return fail(DELS_ERR_INVALID_ARGUMENT, "packed output too small: %zu bytes given, %zu needed", packed_bytes_,
                    need);
    hipError_t e = launch_pack_fp8(static_cast<const uint8_t*>(Wq), ldw, rows, cols,
                                   layout == DELS_LAYOUT_FP8_K128 ? FP8_K128 : FP8_K32, static_cast<uint8_t*>(packed),
                                   static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "fp8 pack launch");
}

size_t dels_fused_argmax_fp8_ws_bytes(int64_t M, int64_t r, int64_t V) {
    if (!rows_ok(M) || !rows_ok(r) || !vocab_ok(V)) return 0;
    return kDataOff + align256(argmax_fp8_data_bytes(M, r, V));
}

static void fill_argmax_fp8(ArgmaxArgs& a, const void* Bq, const float* b_scale, const void* base, int64_t ldbase,
                            int base_dtype, const void* prior, int prior_dtype, const float* alpha,
                            int64_t alpha_stride, const float* beta, int64_t beta_stride, int64_t M, int64_t r,
                            int64_t V, int64_t* out_ids, float* out_score, int64_t ld_out) {
    a.B = static_cast<const uint16_t*>(Bq); a.ldb = 0; a.b_packed = true;
    a.b_scale = b_scale;
    a.base = base; a.ldbase = ldbase; a.base_dtype = base_dtype;
    a.prior = prior; a.prior_dtype = prior_dtype;
    a.alpha = alpha; a.alpha_stride = alpha_stride;
    a.beta = beta; a.beta_stride = beta_stride;
    a.M = (int)M; a.r = (int)r; a.V = (int)V;
    a.out_ids = out_ids; a.out_score = out_score; a.ld_out = ld_out;
}

int dels_fused_argmax_fp8(const void* rank, int64_t ldrank, const void* Bq, const float* b_scale, const void* base,
                          int64_t ldbase, int base_dtype, const void* prior, int prior_dtype, const float* alpha,
                          int64_t alpha_stride, const float* beta, int64_t beta_stride, int64_t M, int64_t r,
                          int64_t V, int64_t* out_ids, float* out_score, int64_t ld_out, void* ws, size_t ws_bytes,
                          void* stream) {
    int rc = check_argmax_args(rank, ldrank, Bq, 0, DELS_LAYOUT_FP8_K128, base, ldbase, base_dtype, prior,
                               prior_dtype, alpha, alpha_stride, beta, beta_stride, M, r, V, out_ids, ld_out, true);
    if (rc != DELS_OK) return rc;
    if (!fp8_rank_ok(r)) return fail(DELS_ERR_UNSUPPORTED, "fp8 argmax needs r in {128, 256, 512} (got %lld)",
                                     (long long)r);
    if (!argmax_fp8_supported(M, r)) return fail(DELS_ERR_UNSUPPORTED, "fp8 argmax: too many rows");
    if (M == 0) return DELS_OK;
    if ((rc = check_scale(b_scale, "b_scale")) != DELS_OK) return rc;
    if ((rc = check_ws(ws, ws_bytes, dels_fused_argmax_fp8_ws_bytes(M, r, V))) != DELS_OK) return rc;
    ArgmaxArgs a{};
    a.rank = static_cast<const uint16_t*>(rank); a.ldrank = ldrank;
    fill_argmax_fp8(a, Bq, b_scale, base, ldbase, base_dtype, prior, prior_dtype, alpha, alpha_stride, beta,
                    beta_stride, M, r, V, out_ids, out_score, ld_out);
    hipError_t e = launch_fused_argmax_fp8(a, ws, kDataOff, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "fp8 fused argmax launch");
}

size_t dels_lowrank_argmax_fp8_ws_bytes(int64_t M, int64_t d, int64_t r, int64_t V) {
    return dels_lowrank_argmax_ws_bytes(M, d, r, V);
}

int dels_lowrank_argmax_fp8(const void* h, int64_t ldh, const void* Aq, const float* a_scale, const void* bias,
                            int act, const void* Bq, const float* b_scale, const void* base, int64_t ldbase,
                            int base_dtype, const void* prior, int prior_dtype, const float* alpha,
                            int64_t alpha_stride, const float* beta, int64_t beta_stride, int64_t M, int64_t d,
                            int64_t r, int64_t V, int64_t* out_ids, float* out_score, int64_t ld_out, void* ws,
                            size_t ws_bytes, void* stream) {
    int rc = check_argmax_args(nullptr, r, Bq, 0, DELS_LAYOUT_FP8_K128, base, ldbase, base_dtype, prior, prior_dtype,
                               alpha, alpha_stride, beta, beta_stride, M, r, V, out_ids, ld_out, false);
    if (rc != DELS_OK) return rc;
    if (!fp8_rank_ok(r)) return fail(DELS_ERR_UNSUPPORTED, "fp8 argmax needs r in {128, 256, 512} (got %lld)",
                                     (long long)r);
    if (!argmax_fp8_supported(M, r)) return fail(DELS_ERR_UNSUPPORTED, "fp8 argmax: too many rows");
    if (d <= 0 || d % 8 != 0 || !inner_ok(d))
        return fail(DELS_ERR_UNSUPPORTED, "hidden size d=%lld must be a positive multiple of 8 below 2^26",
                                          (long long)d);
    if (act != DELS_ACT_IDENTITY && act != DELS_ACT_SILU)
        return fail(DELS_ERR_INVALID_ARGUMENT, "Unsupported DeLS rank_activation code %d", act);
    if (M == 0) return DELS_OK;
    if ((rc = check_bf16_matrix(h, ldh, d, "h")) != DELS_OK) return rc;
    if ((rc = check_weight(Aq, 0, d, DELS_LAYOUT_FP8_K32, "A_q (rank projection)")) != DELS_OK) return rc;
    if ((rc = check_scale(a_scale, "a_scale")) != DELS_OK) return rc;
    if ((rc = check_scale(b_scale, "b_scale")) != DELS_OK) return rc;
    const LowrankLayout L = lowrank_layout(M, d, r, V);
    if (!skinny_supported(L.plan)) return fail(DELS_ERR_UNSUPPORTED, "rank projection shape needs too many tiles");
    if ((rc = check_ws(ws, ws_bytes, L.total)) != DELS_OK) return rc;
    char* w = static_cast<char*>(ws);
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint16_t* rank = reinterpret_cast<uint16_t*>(w + L.rank_off);
    RankArgs ra{};
    ra.h = static_cast<const uint16_t*>(h); ra.ldh = ldh;
    ra.A = static_cast<const uint16_t*>(Aq); ra.lda = 0; ra.a_packed = true;
    ra.a_scale = a_scale;
    ra.bias = static_cast<const uint16_t*>(bias); ra.act = act;
    ra.M = (int)M; ra.d = (int)d; ra.r = (int)r;
    ra.rank = rank; ra.ldrank = r;
    ArgmaxArgs a{};
    a.rank = rank; a.ldrank = r;
    fill_argmax_fp8(a, Bq, b_scale, base, ldbase, base_dtype, prior, prior_dtype, alpha, alpha_stride, beta,
                    beta_stride, M, r, V, out_ids, out_score, ld_out);
    hipError_t e;
    if (decode8_eligible(M, d, r)) {
        e = launch_lowrank_decode(ra, a, ws, s);
        return e == hipSuccess ? DELS_OK : hip_fail(e, "fp8 fused decode step launch");
    }
    if (fp8_argmax_tiled(a) && rank_proj_quantizes(L.plan, r)) {
        // the rank epilogue also writes the rank quantised per row where the
        // e4m3 tiled argmax reads it: no quantisation launch
        ra.rank_q = reinterpret_cast<uint8_t*>(w + L.argmax_off);
        ra.rank_qscale = reinterpret_cast<float*>(w + L.argmax_off + align256((size_t)M * r));
        a.rank_quantized = true;
    }
    e = launch_rank_proj(ra, L.plan, ws, L.part_off, s);
    if (e != hipSuccess) return hip_fail(e, "fp8 rank projection launch");
    e = launch_fused_argmax_fp8(a, ws, L.argmax_off, s);
    return e == hipSuccess ? DELS_OK : hip_fail(e, "fp8 fused argmax launch");
}

size_t dels_argmax_rows_ws_bytes(int64_t, int64_t) { return kDataOff; }

int dels_argmax_rows(const void* x, int64_t ldx, int dtype, int64_t M, int64_t V, int64_t* out_ids, float* out_score,
                     int64_t ld_out, void* ws, size_t ws_bytes, void* stream) {
    if (M < 0 || V <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "bad shape M=%lld V=%lld", (long long)M, (long long)V);
    if (M > kMaxKeyRows || V >= INT32_MAX) return fail(DELS_ERR_UNSUPPORTED, "argmax rows: M <= %d and V < 2^31-1",
                                                       kMaxKeyRows);
    if (M == 0) return DELS_OK;
    if (!x) return fail(DELS_ERR_INVALID_ARGUMENT, "logits pointer is NULL");
    if (!valid_dtype(dtype)) return fail(DELS_ERR_INVALID_ARGUMENT, "unknown logits dtype %d", dtype);
    if (M > 1 && ldx < V) return fail(DELS_ERR_INVALID_ARGUMENT, "logits leading dimension %lld < V %lld",
                                      (long long)ldx, (long long)V);
    if (!out_ids) return fail(DELS_ERR_INVALID_ARGUMENT, "out_ids is NULL");
    if (M > 1 && ld_out < 1) return fail(DELS_ERR_INVALID_ARGUMENT, "ld_out must be >= 1");
    if (!ld_ok({ldx, ld_out})) return fail(DELS_ERR_INVALID_ARGUMENT, "leading dimension out of range");
    int rc = check_ws(ws, ws_bytes, kDataOff);
    if (rc != DELS_OK) return rc;
    hipError_t e = launch_argmax_rows(x, ldx, dtype, (int)M, (int)V, out_ids, out_score, ld_out, ws,
                                      static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "argmax rows launch");
}

size_t dels_sample_rows_ws_bytes(int64_t, int64_t) { return kDataOff; }

int dels_sample_rows(const void* x, int64_t ldx, int dtype, int64_t M, int64_t V, float temperature, uint64_t seed,
                     uint64_t offset, int64_t* out_ids, float* out_score, int64_t ld_out, void* ws, size_t ws_bytes,
                     void* stream) {
    if (!(temperature == temperature) || temperature == __builtin_inff())
        return fail(DELS_ERR_INVALID_ARGUMENT, "temperature must be finite");
    // sample() takes the argmax below 1e-5 (code/dflash.py:32-33)
    if (temperature < 1e-5f)
        return dels_argmax_rows(x, ldx, dtype, M, V, out_ids, out_score, ld_out, ws, ws_bytes, stream);
    if (M < 0 || V <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "bad shape M=%lld V=%lld", (long long)M, (long long)V);
    if (M > kMaxKeyRows || V >= INT32_MAX) return fail(DELS_ERR_UNSUPPORTED, "sample rows: M <= %d and V < 2^31-1",
                                                       kMaxKeyRows);
    if (M == 0) return DELS_OK;
    if (!x) return fail(DELS_ERR_INVALID_ARGUMENT, "logits pointer is NULL");
    if (!valid_dtype(dtype)) return fail(DELS_ERR_INVALID_ARGUMENT, "unknown logits dtype %d", dtype);
    if (M > 1 && ldx < V) return fail(DELS_ERR_INVALID_ARGUMENT, "logits leading dimension %lld < V %lld",
                                      (long long)ldx, (long long)V);
    if (!out_ids) return fail(DELS_ERR_INVALID_ARGUMENT, "out_ids is NULL");
    if (M > 1 && ld_out < 1) return fail(DELS_ERR_INVALID_ARGUMENT, "ld_out must be >= 1");
    if (!ld_ok({ldx, ld_out})) return fail(DELS_ERR_INVALID_ARGUMENT, "leading dimension out of range");
    int rc = check_ws(ws, ws_bytes, kDataOff);
    if (rc != DELS_OK) return rc;
    hipError_t e = launch_sample_rows(x, ldx, dtype, (int)M, (int)V, temperature, seed, offset, out_ids, out_score,
                                      ld_out, ws, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "sample rows launch");
}

size_t dels_gru_step_ws_bytes(int64_t batch, int64_t G) {
    if (!rows_ok(batch) || !rows_ok(G)) return 0;
    return kDataOff + skinny_data_bytes(plan_skinny(std::max<int64_t>(batch, 1), std::max<int64_t>(G, 1),
                                                      std::max<int64_t>(G, 1), true));
}

int dels_gru_step(const void* gi_table, int64_t ld_gi, int64_t table_rows, const int64_t* tokens,
                  int64_t tok_stride, const void* h_in, int64_t ldh_in, const void* w_hh, int w_layout,
                  const void* b_hh,
                  int64_t batch, int64_t G, void* h_out, int64_t ldh_out, void* ws, size_t ws_bytes,
                  void* stream) {
    int rc = check_gru_args(gi_table, ld_gi, table_rows, tokens, h_in, ldh_in, w_hh, w_layout, batch, G, h_out,
                            ldh_out);
    if (rc != DELS_OK) return rc;
    if (!ld_ok({tok_stride})) return fail(DELS_ERR_INVALID_ARGUMENT, "token stride out of range");
    if (batch == 0) return DELS_OK;
    const SkinnyPlan p = plan_skinny(batch, G, G, true);
    if (!skinny_supported(p)) return fail(DELS_ERR_UNSUPPORTED, "GRU shape needs too many tiles");
    if ((rc = check_ws(ws, ws_bytes, kDataOff + skinny_data_bytes(p))) != DELS_OK) return rc;
    GruArgs g{};
    g.gi_table = static_cast<const uint16_t*>(gi_table); g.ld_gi = ld_gi; g.table_rows = table_rows;
    g.tokens = tokens; g.tok_stride = tok_stride;
    g.h_in = static_cast<const uint16_t*>(h_in); g.ldh_in = ldh_in;
    g.w_hh = static_cast<const uint16_t*>(w_hh); g.w_packed = w_layout == DELS_LAYOUT_MFMA16;
    g.b_hh = static_cast<const uint16_t*>(b_hh);
    g.batch = (int)batch; g.G = (int)G;
    g.h_out = static_cast<uint16_t*>(h_out); g.ldh_out = ldh_out;
    hipError_t e = launch_gru_step(g, p, ws, kDataOff, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "GRU step launch");
}

size_t dels_rollout_ws_bytes(int64_t batch, int64_t G, int64_t r, int64_t V) {
    if (!rows_ok(batch) || !rows_ok(G) || !rows_ok(r) || !vocab_ok(V)) return 0;
    return rollout_layout(std::max<int64_t>(batch, 1), std::max<int64_t>(G, 1), std::max<int64_t>(r, 1),
                          std::max<int64_t>(V, 1)).total;
}

int dels_rollout_enqueue(const dels_rollout* p, void* stream) {
    int rc = check_rollout(p);
    if (rc != DELS_OK) return rc;
    return enqueue_rollout(p, static_cast<hipStream_t>(stream));
}

int dels_graph_create(const dels_rollout* p, void** graph_out) {
    if (!graph_out) return fail(DELS_ERR_INVALID_ARGUMENT, "graph_out is NULL");
    *graph_out = nullptr;
    int rc = check_rollout(p);
    if (rc != DELS_OK) return rc;
    return capture_graph([p](hipStream_t s) { return enqueue_rollout(p, s); }, graph_out);
}

size_t dels_gather_argmax_ws_bytes(int64_t M, int64_t r, int64_t V) { return dels_fused_argmax_ws_bytes(M, r, V); }

int dels_gather_argmax(const int64_t* tokens, int64_t tok_stride, const void* E, int64_t lde, int64_t table_rows,
                       const void* B, int64_t ldb, int b_layout, const void* base, int64_t ldbase, int base_dtype,
                       const void* prior, int prior_dtype, const float* alpha, int64_t alpha_stride,
                       const float* beta, int64_t beta_stride, int64_t M, int64_t r, int64_t V, int64_t* out_ids,
                       float* out_score, int64_t ld_out, void* ws, size_t ws_bytes, void* stream) {
    int rc = check_argmax_args(nullptr, r, B, ldb, b_layout, base, ldbase, base_dtype, prior, prior_dtype, alpha,
                               alpha_stride, beta, beta_stride, M, r, V, out_ids, ld_out, false);
    if (rc != DELS_OK) return rc;
    if (M == 0) return DELS_OK;
    if (!tokens) return fail(DELS_ERR_INVALID_ARGUMENT, "token ids pointer is NULL");
    if (table_rows <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "embedding table is empty");
    if (!ld_ok({tok_stride})) return fail(DELS_ERR_INVALID_ARGUMENT, "token stride out of range");
    if ((rc = check_bf16_matrix(E, lde, r, "E (embedding table)")) != DELS_OK) return rc;
    if ((rc = check_ws(ws, ws_bytes, dels_gather_argmax_ws_bytes(M, r, V))) != DELS_OK) return rc;
    ArgmaxArgs a = gather_args(tokens, tok_stride, E, lde, table_rows, B, ldb, b_layout, base, ldbase, base_dtype,
                               prior, prior_dtype, alpha, alpha_stride, beta, beta_stride, M, r, V, out_ids,
                               out_score, ld_out);
    hipError_t e = launch_fused_argmax(a, ws, kDataOff, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "gather argmax launch");
}

size_t dels_markov_rollout_ws_bytes(int64_t batch, int64_t r, int64_t V) {
    if (!rows_ok(batch) || !rows_ok(r) || !vocab_ok(V)) return 0;
    return kDataOff + align256(argmax_data_bytes(std::max<int64_t>(batch, 1), std::max<int64_t>(r, 1),
                                                 std::max<int64_t>(V, 1)));
}

int dels_markov_rollout_enqueue(const dels_markov_rollout* p, void* stream) {
    int rc = check_markov(p);
    if (rc != DELS_OK) return rc;
    return enqueue_markov(p, static_cast<hipStream_t>(stream));
}

int dels_markov_graph_create(const dels_markov_rollout* p, void** graph_out) {
    if (!graph_out) return fail(DELS_ERR_INVALID_ARGUMENT, "graph_out is NULL");
    *graph_out = nullptr;
    int rc = check_markov(p);
    if (rc != DELS_OK) return rc;
    return capture_graph([p](hipStream_t s) { return enqueue_markov(p, s); }, graph_out);
}

size_t dels_lm_head_ws_bytes(int64_t, int64_t, int64_t) { return kDataOff; }

int dels_pack_lm_head(const void* W, int64_t ldw, int64_t rows, int64_t cols, void* packed, size_t packed_bytes_,
                      void* stream) {
    if (rows < 0 || cols < 0) return fail(DELS_ERR_INVALID_ARGUMENT, "bad shape to pack");
    if (!vocab_ok(rows) || !inner_ok(cols)) return fail(DELS_ERR_UNSUPPORTED, "pack: rows below 2^31-1, cols below 2^26");
    if (cols % (32 * kLmHeadKChunk) != 0)
        return fail(DELS_ERR_UNSUPPORTED, "LM head layout: cols=%lld must be a multiple of %d", (long long)cols,
                    32 * kLmHeadKChunk);
    if (rows == 0 || cols == 0) return DELS_OK;
    int rc = check_bf16_matrix(W, ldw, cols, "W (to pack)");
    if (rc != DELS_OK) return rc;
    if (!packed || !aligned16(packed)) return fail(DELS_ERR_ALIGNMENT, "packed output must be 16-byte aligned");
    if (packed_bytes_ < packed_bytes(rows, cols))
        return fail(DELS_ERR_INVALID_ARGUMENT, "packed output too small: %zu bytes given, %zu needed", packed_bytes_,
                    packed_bytes(rows, cols));
    hipError_t e = launch_pack_mfma16(static_cast<const uint16_t*>(W), ldw, rows, cols, static_cast<uint16_t*>(packed),
                                      static_cast<hipStream_t>(stream), kLmHeadKChunk);
    return e == hipSuccess ? DELS_OK : hip_fail(e, "pack launch");
}

int dels_lm_head(const void* hidden, int64_t ldh, const void* W, int64_t M, int64_t K, int64_t V, void* base,
                 int64_t ldo, int64_t argmax_period, int64_t* out_ids, float* out_score, int64_t ld_out, void* ws,
                 size_t ws_bytes, void* stream) {
    if (M < 0 || K <= 0 || V <= 0) return fail(DELS_ERR_INVALID_ARGUMENT, "bad LM head shape M=%lld K=%lld V=%lld",
                                                (long long)M, (long long)K, (long long)V);
    if (argmax_period < 0) return fail(DELS_ERR_INVALID_ARGUMENT, "argmax_period must be >= 0");
    if (M == 0) return DELS_OK;
    if (!lm_head_supported(M, K, V, argmax_period))
        return fail(DELS_ERR_UNSUPPORTED, "LM head: K=%lld must be a multiple of 256, M <= 8192, V < 2^31-1 and "
                    "at most %d argmax rows", (long long)K, kMaxKeyRows);
    int rc;
    if ((rc = check_bf16_matrix(hidden, ldh, K, "hidden")) != DELS_OK) return rc;
    if (((M - 1) * ldh + K) * 2 >= (int64_t(1) << 31))
        return fail(DELS_ERR_UNSUPPORTED, "LM head: the hidden rows must span less than 2 GiB");
    if (!W) return fail(DELS_ERR_INVALID_ARGUMENT, "W is NULL");
    if (!aligned16(W)) return fail(DELS_ERR_ALIGNMENT, "packed W must be 16-byte aligned");
    if (base && M > 1 && ldo < V) return fail(DELS_ERR_INVALID_ARGUMENT, "base leading dimension %lld < V %lld",
                                              (long long)ldo, (long long)V);
    if (!ld_ok({ldo, ld_out})) return fail(DELS_ERR_INVALID_ARGUMENT, "leading dimension out of range");
    if (argmax_period > 0) {
        if (!out_ids) return fail(DELS_ERR_INVALID_ARGUMENT, "out_ids is NULL");
        if (ld_out < 1) return fail(DELS_ERR_INVALID_ARGUMENT, "ld_out must be >= 1");
    }
    if ((rc = check_ws(ws, ws_bytes, kDataOff)) != DELS_OK) return rc;
    hipError_t e = launch_lm_head(hidden, ldh, W, (int)M, (int)K, (int)V, base, ldo, (int)argmax_period, out_ids,
                                  out_score, ld_out, ws, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "LM head launch");
}

size_t dels_domino_argmax_ws_bytes(int64_t, int64_t, int64_t) { return kDataOff; }

int dels_domino_argmax(const void* z, int64_t ldz, const void* sv, int64_t lds, const void* fc2_w,
                       const void* fc2_bias, int fc2_bias_dtype, const void* base, int64_t ldbase, int base_dtype,
                       float alpha, int middle, int64_t M, int64_t E, int64_t V, int64_t* out_ids, float* out_score,
                       int64_t ld_out, void* ws, size_t ws_bytes, void* stream) {
    int rc = check_domino_step(z, ldz, sv, lds, fc2_w, fc2_bias, fc2_bias_dtype, base, ldbase, base_dtype, alpha,
                               middle, M, E, V, out_ids, ld_out);
    if (rc != DELS_OK) return rc;
    if (M == 0) return DELS_OK;
    if ((rc = check_ws(ws, ws_bytes, kDataOff)) != DELS_OK) return rc;
    const DominoArgs d = domino_args(z, ldz, sv, lds, fc2_w, fc2_bias, fc2_bias_dtype, base, ldbase, base_dtype, alpha,
                                     middle, M, E, V, out_ids, out_score, ld_out);
    hipError_t e = launch_domino_argmax(d, ws, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "Domino step launch");
}

size_t dels_domino_rollout_ws_bytes(int64_t batch, int64_t steps, int64_t D, int64_t G, int64_t E, int64_t V) {
    if (!rows_ok(batch) || !rows_ok(steps) || !rows_ok(batch * steps) || !inner_ok(D) || !rows_ok(G) ||
        !rows_ok(E) || !vocab_ok(V))
        return 0;
    return domino_layout(std::max<int64_t>(batch, 1), std::max<int64_t>(steps, 1), std::max<int64_t>(D, 1),
                         std::max<int64_t>(G, 1), std::max<int64_t>(E, 1)).total;
}

int dels_domino_rollout_enqueue(const dels_domino_rollout* p, void* stream) {
    int rc = check_domino_rollout(p);
    if (rc != DELS_OK) return rc;
    return enqueue_domino(p, static_cast<hipStream_t>(stream));
}

int dels_domino_graph_create(const dels_domino_rollout* p, void** graph_out) {
    if (!graph_out) return fail(DELS_ERR_INVALID_ARGUMENT, "graph_out is NULL");
    *graph_out = nullptr;
    int rc = check_domino_rollout(p);
    if (rc != DELS_OK) return rc;
    return capture_graph([p](hipStream_t s) { return enqueue_domino(p, s); }, graph_out);
}

int dels_graph_launch(void* graph, void* stream) {
    if (!graph) return fail(DELS_ERR_INVALID_ARGUMENT, "graph handle is NULL");
    GraphHandle* h = static_cast<GraphHandle*>(graph);
    hipError_t e = hipGraphLaunch(h->exec, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? DELS_OK : hip_fail(e, "hipGraphLaunch");
}

int dels_graph_destroy(void* graph) {
    if (!graph) return DELS_OK;
    GraphHandle* h = static_cast<GraphHandle*>(graph);
    hipError_t e1 = h->exec ? hipGraphExecDestroy(h->exec) : hipSuccess;
    hipError_t e2 = h->graph ? hipGraphDestroy(h->graph) : hipSuccess;
    delete h;
    if (e1 != hipSuccess) return hip_fail(e1, "hipGraphExecDestroy");
    if (e2 != hipSuccess) return hip_fail(e2, "hipGraphDestroy");
    return DELS_OK;
}

}  // extern "C"

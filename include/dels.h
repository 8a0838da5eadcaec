/*
 * dels.h -- C ABI of the MI355X (gfx950) draft-token selection path of DeLS-Spec.
 *
 * The path: for each draft row m,
 *     rank_m  = bf16(act(bf16(h_m . A^T + bias)))
 *     s[m, v] = fp32(rank_m . B[v]) * alpha_m + base[m, v] - beta_m * prior[v]
 *               (evaluated as two fused multiply-adds, each rounded once)
 *     id_m    = lowest v attaining max_v s[m, v];  score_m = s[m, id_m]
 * without writing the [M, V] logits to memory, plus the GRU local-head step
 * that feeds the next draft position and a hipGraph of the whole suffix
 * rollout.  Paths cited below are relative to the dt-3t/DeLS-Spec repository.
 *
 * Conventions
 *  - Every pointer argument except `ws` scratch bookkeeping is a device
 *    pointer owned by the caller; the library never allocates, frees or keeps
 *    a pointer past the call (graph handles excepted, see dels_graph_*).
 *  - Matrices are row-major with a leading dimension (`ld*`, in elements) and
 *    unit column stride.  bf16 operands (h, A, B, rank, GRU weights) must be
 *    16-byte aligned with ld % 8 == 0.
 *  - `stream` is a hipStream_t (pass torch.cuda.current_stream().cuda_stream);
 *    all work is stream-ordered, nothing synchronises the host, so every entry
 *    point may be captured into a hipGraph.
 *  - Workspace (`ws`): caller-owned device memory of at least the size the
 *    matching *_ws_bytes() function returns, 256-byte aligned, zero-filled
 *    once before first use (dels_workspace_init).  Every entry point lays it
 *    out alike: a 64 KiB control area that kernels return to the state they
 *    found it in -- zeros, apart from one word that the fused decode step and
 *    the one-launch rollout advance once per launch (a launch generation) -- so no call needs a
 *    memset; then 544 KiB that only the fused decode step writes (its rank
 *    hand-off words, each tagged with a launch generation) and 144 KiB that
 *    only the one-launch rollout writes (its state and rank words, tagged with
 *    the launch generation and the step, and its argmax slot words, which each
 *    launch clears before use); then data regions that may hold
 *    anything between calls.  One workspace may therefore serve
 *    every entry point and shape in turn; calls that share it must not
 *    overlap in time (same stream is fine).
 *  - Extents: rows, batch, batch * steps, r, G and E below 2^24, hidden sizes
 *    (d, D, K) below 2^26, V below 2^31 - 1, leading dimensions and strides
 *    in [0, 2^40) elements.  Calls outside them fail their checks, and the
 *    *_ws_bytes() / *_packed_*bytes() queries return 0 for such shapes.
 *  - Return value: DELS_OK (0) or a negative DELS_ERR_* code; no exception
 *    crosses the ABI.  dels_strerror() names a code, dels_last_error() gives
 *    the detail of the calling thread's last failure.
 */
#ifndef DELS_H
#define DELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DELS_ABI_VERSION 3

/* status codes */
#define DELS_OK 0
#define DELS_ERR_INVALID_ARGUMENT (-1)
#define DELS_ERR_UNSUPPORTED (-2)
#define DELS_ERR_ALIGNMENT (-3)
#define DELS_ERR_WORKSPACE (-4)
#define DELS_ERR_HIP (-5)

/* element types of base logits / prior */
#define DELS_DTYPE_F32 0
#define DELS_DTYPE_BF16 1
#define DELS_DTYPE_F16 2

/* rank activations (code/dels.py:14) */
#define DELS_ACT_IDENTITY 0
#define DELS_ACT_SILU 1

/*
 * Middle layer of the Domino correction MLP (the layers between fc1 and fc2 of
 * embed_proj, code/kernel/domino.py:15-51, 404-431), applied elementwise in
 * fp32 to p = z + s.  SILU is the reference's fused case (0, so a zeroed
 * rollout struct keeps it); the others are the modules its unfused step runs:
 * nn.Identity, nn.ReLU, nn.GELU() (erf), nn.GELU(approximate="tanh"),
 * nn.Tanh, nn.Sigmoid.
 */
#define DELS_MIDDLE_SILU 0
#define DELS_MIDDLE_IDENTITY 1
#define DELS_MIDDLE_RELU 2
#define DELS_MIDDLE_GELU 3
#define DELS_MIDDLE_GELU_TANH 4
#define DELS_MIDDLE_TANH 5
#define DELS_MIDDLE_SIGMOID 6

/*
 * Weight layouts.  DELS_LAYOUT_ROWMAJOR: [rows, cols] row-major with a leading
 * dimension.  DELS_LAYOUT_MFMA16: the "MFMA-16 block" layout written by
 * dels_pack_operand -- the matrix is cut into 16-row x 32-column blocks (rows
 * padded to 16, columns to 32, with zeros), blocks stored row-block-major, and
 * each 1 KiB block in wave64 lane order (lane l holds the 8 elements of row
 * l%16 at columns 8*(l/16)..+7 of the block), so every 16-byte-per-lane load of
 * an MFMA operand reads one contiguous KiB of HBM.  Leading dimensions are
 * ignored for packed operands.
 */
#define DELS_LAYOUT_ROWMAJOR 0
#define DELS_LAYOUT_MFMA16 1
/*
 * fp8 weight layouts (OCP float8 e4m3fn bytes; no counterpart in the
 * reference, whose weights are bf16 -- the fp8 configuration stores A and B as
 * e4m3 with a per-output-channel fp32 scale).  Written by dels_pack_operand_fp8
 * from row-major e4m3 bytes, zero-padded:
 *   DELS_LAYOUT_FP8_K128: 16-row x 128-column blocks of 2 KiB, row-block-major,
 *     each as two 1 KiB halves [half][lane][16 bytes], lane l holding row l%16,
 *     columns 32*(l/16) + 16*half .. +15 of the block (the low-rank LM head B);
 *   DELS_LAYOUT_FP8_K32: the MFMA16 block order with one byte per element,
 *     16-row x 32-column blocks of 512 bytes (the rank projection weight A).
 */
#define DELS_LAYOUT_FP8_K128 2
#define DELS_LAYOUT_FP8_K32 3

int dels_abi_version(void);
const char* dels_strerror(int status);
const char* dels_last_error(void);

/* Zero-fill a workspace on `stream` with a fill kernel (capture-safe). */
int dels_workspace_init(void* ws, size_t ws_bytes, void* stream);

/*
 * Repack a bf16 [rows, cols] row-major weight into the MFMA-16 block layout
 * (no counterpart in the reference, whose runner keeps .contiguous() copies of
 * the same weights, code/kernel/dels.py:260-276).  `packed` must hold
 * dels_packed_bytes(rows, cols) bytes and be 16-byte aligned.
 */
size_t dels_packed_bytes(int64_t rows, int64_t cols);
int dels_pack_operand(const void* W, int64_t ldw, int64_t rows, int64_t cols,
                      void* packed, size_t packed_bytes, void* stream);

/*
 * Rank projection rank = bf16(act(bf16(h . A^T + bias)))  [M, r] bf16.
 * Replaces F.linear(h_state, rank_weight, rank_bias) + F.silu in
 * DeLSGraphRunner._forward_impl (code/kernel/dels.py:437-443) and
 * DeLSLocalHead.logits_from_hidden's rank_proj (code/dels.py:334-339).
 *   h [M, d] bf16 (ldh), A [r, d] bf16 (lda), bias [r] bf16 or NULL.
 */
size_t dels_rank_proj_ws_bytes(int64_t M, int64_t d, int64_t r);
int dels_rank_proj(const void* h, int64_t ldh, const void* A, int64_t lda, int a_layout,
                   const void* bias, int act, int64_t M, int64_t d, int64_t r,
                   void* rank, int64_t ldrank, void* ws, size_t ws_bytes, void* stream);

/*
 * Fused low-rank LM-head combine + vocabulary argmax, given rank.
 * Replaces _fused_low_rank_argmax_kernel + _reduce_argmax_kernel as launched
 * by DeLSGraphRunner._argmax_step_triton (code/kernel/dels.py:15-138, 375-423).
 *   rank  [M, r] bf16 (ldrank)          B     [V, r] bf16 (ldb, b_layout)
 *   base  [M, V] base_dtype (ldbase)    prior [V] prior_dtype, or NULL
 *   alpha/beta: fp32 device arrays read at alpha[m*alpha_stride] (stride 0
 *   broadcasts one value).  The prior term is applied to row m only when
 *   prior != NULL and beta_m != 0 (code/kernel/dels.py:81-88, 382).
 *   out_ids[m*ld_out] int64, out_score[m*ld_out] fp32 (out_score may be NULL).
 * Ties go to the lowest vocabulary index; a row whose scores are all -inf
 * returns id 0 with score -inf.
 */
size_t dels_fused_argmax_ws_bytes(int64_t M, int64_t r, int64_t V);
int dels_fused_argmax(const void* rank, int64_t ldrank, const void* B, int64_t ldb, int b_layout,
                      const void* base, int64_t ldbase, int base_dtype,
                      const void* prior, int prior_dtype,
                      const float* alpha, int64_t alpha_stride,
                      const float* beta, int64_t beta_stride,
                      int64_t M, int64_t r, int64_t V,
                      int64_t* out_ids, float* out_score, int64_t ld_out,
                      void* ws, size_t ws_bytes, void* stream);

/*
 * Rank projection followed by the fused argmax: one draft step of the
 * reference's Triton path (code/kernel/dels.py:437-446).  The bf16 rank
 * lives in the workspace.
 */
size_t dels_lowrank_argmax_ws_bytes(int64_t M, int64_t d, int64_t r, int64_t V);
int dels_lowrank_argmax(const void* h, int64_t ldh, const void* A, int64_t lda, int a_layout,
                        const void* bias, int act,
                        const void* B, int64_t ldb, int b_layout,
                        const void* base, int64_t ldbase, int base_dtype,
                        const void* prior, int prior_dtype,
                        const float* alpha, int64_t alpha_stride,
                        const float* beta, int64_t beta_stride,
                        int64_t M, int64_t d, int64_t r, int64_t V,
                        int64_t* out_ids, float* out_score, int64_t ld_out,
                        void* ws, size_t ws_bytes, void* stream);

/*
 * dels_lowrank_argmax without a workspace argument: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under
 * hipGraph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * workspace is a file-scope device array of DELS_NOALLOC_SCRATCH_BYTES that
 * every GPU the library runs on holds until the process ends; the call
 * allocates nothing.  Shapes whose dels_lowrank_argmax_ws_bytes() exceeds the
 * array are refused with DELS_ERR_WORKSPACE (16 MiB covers M <= 512 at
 * d = 4096, r = 512).  All calls on one GPU share its array: calls that
 * overlap in time on one GPU race (serialise them, e.g. on one stream).  The
 * first call on a device clears the array once on `stream` and must not be
 * made under stream capture; later calls may be captured.
 */
#define DELS_NOALLOC_SCRATCH_BYTES (16u << 20)
int dels_lowrank_argmax_noalloc(const void* h, int64_t ldh, const void* A, int64_t lda, int a_layout,
                                const void* bias, int act,
                                const void* B, int64_t ldb, int b_layout,
                                const void* base, int64_t ldbase, int base_dtype,
                                const void* prior, int prior_dtype,
                                const float* alpha, int64_t alpha_stride,
                                const float* beta, int64_t beta_stride,
                                int64_t M, int64_t d, int64_t r, int64_t V,
                                int64_t* out_ids, float* out_score, int64_t ld_out, void* stream);

/*
 * Test hook (no counterpart in the reference).  With M <= 16 rows and both
 * weights in the MFMA-16 layout, dels_lowrank_argmax runs the rank projection
 * and the argmax in one launch whose workgroups wait (bounded) for each other's
 * rank tiles; a workgroup that polls `limit` times without seeing them computes
 * the rank itself.  Sets that poll limit for later launches (0 forces the local
 * computation) and returns the previous one.  Not thread-safe.
 */
int dels_debug_set_decode_spin_limit(int limit);

/*
 * Test hook (no counterpart in the reference).  Where the shape allows it
 * (weights in the MFMA-16 layout, r = 256, batch <= 16, G <= 1024 a multiple of
 * twice the CU count, the vocabulary's share fitting a CU), dels_rollout_enqueue
 * and dels_graph_create run every step of the rollout in one launch that keeps
 * the low-rank head resident on chip; enable = 0 selects the per-step launches
 * instead (for later calls), 1 restores the default.  Returns the previous
 * setting.  Not thread-safe.
 */
int dels_debug_set_rollout_resident(int enable);
/* Test hook: the waits of that one-launch rollout re-read each other's results
 * at most `limit` times (default 65536) before the launch gives up; a launch
 * that gives up writes -1 ids for the steps it could not finish, and the next
 * launch starts clean.  Returns the previous limit.  Not thread-safe. */
int dels_debug_set_resident_spin_limit(int limit);

/*
 * Plain argmax of each row of logits: sample() at temperature 0
 * (code/dflash.py:31-33; torch.argmax over the vocabulary), as used for the
 * first draft position (code/dflash.py:473).  x [M, V] with row stride ldx,
 * dtype DELS_DTYPE_*; out_ids[m*ld_out] int64, out_score[m*ld_out] fp32 (or
 * NULL).  Ties go to the lowest index; NaN ranks above every number, so a
 * row holding NaN gives the index of its first NaN (score NaN), as
 * torch.argmax does; a row of -inf gives id 0 and score -inf.
 */
size_t dels_argmax_rows_ws_bytes(int64_t M, int64_t V);
int dels_argmax_rows(const void* x, int64_t ldx, int dtype, int64_t M, int64_t V,
                     int64_t* out_ids, float* out_score, int64_t ld_out,
                     void* ws, size_t ws_bytes, void* stream);

/*
 * dels_sample_rows: sample() at temperature > 0 (code/dflash.py:31-38:
 * softmax(logits / T) then torch.multinomial, one draw per row), for logits
 * [M, V] (dtype and layout as dels_argmax_rows).  Computed as a Gumbel-max:
 *   y = round_dtype(fp32(x) / T),  u = ((bits >> 9) + 0.5) * 2^-23,
 *   id = argmax_v (y[v] - log(-log(u[v]))),  score = that maximum,
 * where bits is word v%4 of Philox4x32-10 at counter (v/4, m, offset low,
 * offset high) and key (seed low, seed high).  The ids are distributed as
 * softmax(y) draws and depend only on (seed, offset, row, logits).
 * temperature < 1e-5 is dels_argmax_rows, as in the reference; NaN or inf
 * temperatures are rejected.  Where torch.multinomial raises (a row with NaN
 * or +inf, or of -inf only) this returns the argmax rule's id instead.
 */
size_t dels_sample_rows_ws_bytes(int64_t M, int64_t V);
int dels_sample_rows(const void* x, int64_t ldx, int dtype, int64_t M, int64_t V,
                     float temperature, uint64_t seed, uint64_t offset,
                     int64_t* out_ids, float* out_score, int64_t ld_out,
                     void* ws, size_t ws_bytes, void* stream);

/*
 * fp8 variant (no counterpart in the reference: the fp8 configuration of the
 * same draft step, with e4m3 weights and per-output-channel fp32 scales).
 *
 * dels_pack_operand_fp8: row-major e4m3 bytes W [rows, cols] (ldw bytes) into
 * `layout` (DELS_LAYOUT_FP8_K128 or _K32); `packed` holds
 * dels_packed_fp8_bytes(rows, cols, layout) bytes, 16-byte aligned.
 *
 * dels_fused_argmax_fp8: the fused argmax of dels_fused_argmax with
 *   B_q [V, r] e4m3 (DELS_LAYOUT_FP8_K128) and b_scale [V] fp32; each rank row
 *   is quantised in the kernel to e4m3 with scale sR = absmax / 448 and
 *     dot[m, v] = fp32(R_q[m] . B_q[v]) * sR[m] * b_scale[v]
 *   (rounded after each product), then the same combine and argmax.
 *   r must be 128, 256 or 512.
 *
 * dels_lowrank_argmax_fp8: rank = bf16(act(bf16(fp32(h . A_q^T) * a_scale +
 *   bias))) with A_q [r, d] e4m3 (DELS_LAYOUT_FP8_K32) and a_scale [r] fp32,
 *   then dels_fused_argmax_fp8.  One launch for M <= 16 (d a multiple of 32).
 */
size_t dels_packed_fp8_bytes(int64_t rows, int64_t cols, int layout);
int dels_pack_operand_fp8(const void* Wq, int64_t ldw, int64_t rows, int64_t cols, int layout,
                          void* packed, size_t packed_bytes, void* stream);
size_t dels_fused_argmax_fp8_ws_bytes(int64_t M, int64_t r, int64_t V);
int dels_fused_argmax_fp8(const void* rank, int64_t ldrank, const void* Bq, const float* b_scale,
                          const void* base, int64_t ldbase, int base_dtype,
                          const void* prior, int prior_dtype,
                          const float* alpha, int64_t alpha_stride,
                          const float* beta, int64_t beta_stride,
                          int64_t M, int64_t r, int64_t V,
                          int64_t* out_ids, float* out_score, int64_t ld_out,
                          void* ws, size_t ws_bytes, void* stream);
size_t dels_lowrank_argmax_fp8_ws_bytes(int64_t M, int64_t d, int64_t r, int64_t V);
int dels_lowrank_argmax_fp8(const void* h, int64_t ldh, const void* Aq, const float* a_scale,
                            const void* bias, int act, const void* Bq, const float* b_scale,
                            const void* base, int64_t ldbase, int base_dtype,
                            const void* prior, int prior_dtype,
                            const float* alpha, int64_t alpha_stride,
                            const float* beta, int64_t beta_stride,
                            int64_t M, int64_t d, int64_t r, int64_t V,
                            int64_t* out_ids, float* out_score, int64_t ld_out,
                            void* ws, size_t ws_bytes, void* stream);

/*
 * One GRU local-head step h_out = GRUCell(gi_table[tokens], h_in).
 * Replaces DeLSGraphRunner._gru_cell / _fused_gru_cell_kernel plus the
 * input-table gather (code/kernel/dels.py:140-211, 359-373, 432, 461).
 *   gi_table [table_rows, 3G] bf16 (ld_gi) = F.linear(E, W_ih, b_ih);
 *   tokens[b*tok_stride] int64 (clamped to [0, table_rows) before use);
 *   h_in [batch, G] bf16 (ldh_in) or NULL for a zero state;
 *   w_hh [3G, G] bf16 in w_layout, b_hh [3G] bf16 or NULL; h_out [batch, G] bf16.
 * Gate order (r, z, n) as torch.nn.GRU; gh = bf16(h . W_hh^T + b_hh).
 */
size_t dels_gru_step_ws_bytes(int64_t batch, int64_t G);
int dels_gru_step(const void* gi_table, int64_t ld_gi, int64_t table_rows,
                  const int64_t* tokens, int64_t tok_stride,
                  const void* h_in, int64_t ldh_in,
                  const void* w_hh, int w_layout, const void* b_hh,
                  int64_t batch, int64_t G,
                  void* h_out, int64_t ldh_out,
                  void* ws, size_t ws_bytes, void* stream);

/*
 * The DeLS suffix rollout of DeLSGraphRunner._forward_impl
 * (code/kernel/dels.py:425-467): h = GRU(gi_table[prefix], 0); then for each
 * step s: rank projection, fused argmax against base[:, s, :] with
 * alpha[s]/beta[s], out_ids[:, s] = id, and a GRU step on that id unless s is
 * the last step.  All buffers are caller-owned device memory.
 */
typedef struct dels_rollout {
    const void* gi_table;   /* [table_rows, 3G] bf16 */
    int64_t ld_gi;
    int64_t table_rows;
    const void* w_hh;       /* [3G, G] bf16 */
    const void* b_hh;       /* [3G] bf16 or NULL */
    const void* rank_w;     /* [r, G] bf16 */
    const void* rank_b;     /* [r] bf16 or NULL */
    int act;                /* DELS_ACT_* */
    const void* lm_w;       /* [V, r] bf16 */
    const void* prior;      /* [V] or NULL */
    int prior_dtype;
    const float* alpha;     /* [steps] fp32 */
    const float* beta;      /* [steps] fp32 */
    int64_t batch, steps, G, r, V;
    int weights_layout;     /* DELS_LAYOUT_* of w_hh, rank_w and lm_w */
    const int64_t* prefix_ids; /* [batch] int64: row b at prefix_ids[b * ld_prefix] */
    const void* base;       /* [batch, steps, V]: row b, step s at base + (b * ld_base + s * V) */
    int base_dtype;
    int64_t ld_base;        /* elements between batch rows of base (0: steps * V) */
    int64_t* out_ids;       /* [batch, steps] int64: row b, step s at out_ids[b * ld_out + s] */
    float* out_scores;      /* [batch, steps] fp32 or NULL, rows ld_out apart as out_ids */
    void* h_a;              /* [batch, G] bf16 state buffers (ping-pong) */
    void* h_b;
    void* rank;             /* [batch, r] bf16 scratch for the rank (unused when the
                               step runs as one fused launch: packed weights, batch <= 16) */
    void* ws;
    size_t ws_bytes;
    int64_t ld_prefix;      /* elements between batch rows of prefix_ids (0: 1) */
    int64_t ld_out;         /* elements between batch rows of out_ids / out_scores (0: steps; else >= steps) */
} dels_rollout;

size_t dels_rollout_ws_bytes(int64_t batch, int64_t G, int64_t r, int64_t V);
/* (A draft step feeds base_logits[:, 1:k, :] of its [batch, k, V] logits in place: ld_base = k * V.) */
int dels_rollout_enqueue(const dels_rollout* p, void* stream);

/*
 * hipGraph of the rollout: replaces the torch.cuda.CUDAGraph capture and
 * replay of DeLSGraphRunner (code/kernel/dels.py:320-329, 477).  The graph
 * bakes in the pointers of `p`; the handle owns only the graph objects.
 * dels_graph_launch and dels_graph_destroy also take the handles of
 * dels_markov_graph_create.
 */
int dels_graph_create(const dels_rollout* p, void** graph_out);
int dels_graph_launch(void* graph, void* stream);
int dels_graph_destroy(void* graph);

/*
 * Target LM head of a draft block (code/dflash.py:468, target.lm_head(
 * parallel_hiddens)), with sample() of chosen rows fused (code/dflash.py:475):
 *   base[m, v] = bf16(hidden[m] . W[v])   (fp32 accumulate, one rounding).
 * hidden [M, K] bf16 (leading dimension ldh, 16-byte aligned, ldh % 8 == 0);
 * W [V, K] bf16 packed by dels_pack_lm_head; K a multiple of 256.
 * With argmax_period > 0, rows m with m % argmax_period == 0 are not stored:
 * out_ids[j * ld_out] (and out_score) receive the argmax of row j*argmax_period
 * over its bf16 values (lowest index on ties, first NaN wins), as
 * sample(base[:, :1]) of a [batch, argmax_period, V] block.  Every other row
 * goes to base (leading dimension ldo) when base is not NULL.
 */
size_t dels_lm_head_ws_bytes(int64_t M, int64_t K, int64_t V);
/* dels_pack_lm_head: W [rows, cols] bf16 row-major into the LM head's layout --
 * the MFMA-16 blocks in K-chunk-major order (4 blocks of 32 K per chunk: the
 * 4 KiB of a 16-row tile in one chunk, then the next tile of the same chunk);
 * cols a multiple of 128; `packed` holds dels_packed_bytes(rows, cols) bytes. */
int dels_pack_lm_head(const void* W, int64_t ldw, int64_t rows, int64_t cols, void* packed, size_t packed_bytes,
                      void* stream);
int dels_lm_head(const void* hidden, int64_t ldh, const void* W, int64_t M, int64_t K, int64_t V,
                 void* base, int64_t ldo, int64_t argmax_period,
                 int64_t* out_ids, float* out_score, int64_t ld_out,
                 void* ws, size_t ws_bytes, void* stream);

/*
 * Domino correction step (DraftCorrectionGraphRunner._fused_step_triton,
 * code/kernel/domino.py:58-173, 438-482): for rows m < M of z and s [M, E]
 * bf16 (the hidden-state and GRU-state parts of the correction MLP's first
 * layer),
 *   mid[m, k] = f(p),  p = fp32(z[m, k]) + fp32(s[m, k])   (fp32; f the
 *               middle layer, DELS_MIDDLE_*: SILU is p * sigmoid(p))
 *   dot[m, v] = fp32(mid[m] . fc2[v])   (+ fc2_bias[v] when given)
 *   id_m = lowest argmax_v fma(dot[m, v], alpha, base[m, v]).
 * fc2 [V, E] bf16 in the MFMA-16 layout (dels_pack_operand); E a multiple of
 * 32, at most 2048; fc2_bias [V] of fc2_bias_dtype or NULL; base [M, V] with
 * leading dimension ldbase.  mid enters the matrix cores as two bf16 parts
 * (hi + lo, 2^-17 relative).
 */
size_t dels_domino_argmax_ws_bytes(int64_t M, int64_t E, int64_t V);
int dels_domino_argmax(const void* z, int64_t ldz, const void* s, int64_t lds, const void* fc2_w,
                       const void* fc2_bias, int fc2_bias_dtype,
                       const void* base, int64_t ldbase, int base_dtype, float alpha, int middle,
                       int64_t M, int64_t E, int64_t V,
                       int64_t* out_ids, float* out_score, int64_t ld_out,
                       void* ws, size_t ws_bytes, void* stream);

/*
 * The Domino correction rollout of DraftCorrectionGraphRunner._forward_impl
 * (code/kernel/domino.py:379-436):
 *   z = F.linear(hiddens [batch * steps, D], w_z, fc1_bias)       (bf16)
 *   h = GRU over the prefix ids from h = 0 (gi_table rows, one cell per id)
 *   for each step t: s = F.linear(h, w_s); out_ids[:, t] = the correction
 *   step on z[:, t], s and base[:, t, :]; then a GRU step on that id unless
 *   t is the last step.
 * gi_table = F.linear(embed_tokens.weight, W_ih, b_ih) as in the DeLS rollout.
 */
typedef struct dels_domino_rollout {
    const void* gi_table;   /* [table_rows, 3G] bf16 */
    int64_t ld_gi;
    int64_t table_rows;
    const void* w_hh;       /* [3G, G] bf16 (weights_layout) */
    const void* b_hh;       /* [3G] bf16 or NULL */
    const void* w_z;        /* [E, D] bf16 (weights_layout): fc1.weight[:, :D] */
    const void* fc1_bias;   /* [E] bf16 or NULL */
    const void* w_s;        /* [E, G] bf16 (weights_layout): fc1.weight[:, D:] */
    const void* fc2_w;      /* [V, E] bf16, MFMA-16 layout */
    const void* fc2_bias;   /* [V] or NULL */
    int fc2_bias_dtype;
    float alpha;            /* guidance alpha */
    int64_t batch, steps, prefix_len, D, G, E, V;
    int weights_layout;     /* DELS_LAYOUT_* of w_hh, w_z and w_s */
    const int64_t* prefix_ids; /* [batch, prefix_len] int64 */
    const void* hiddens;    /* [batch, steps, D] bf16, contiguous */
    const void* base;       /* [batch, steps, V]: row b, step t at base + (b * ld_base + t * V) */
    int base_dtype;
    int64_t ld_base;        /* 0: steps * V */
    int64_t* out_ids;       /* [batch, steps] int64 */
    float* out_scores;      /* [batch, steps] fp32 or NULL */
    void* h_a;              /* [batch, G] bf16 state buffers (ping-pong) */
    void* h_b;
    void* z;                /* [batch * steps, E] bf16 scratch */
    void* s;                /* [batch, E] bf16 scratch */
    void* ws;
    size_t ws_bytes;
    int middle;             /* DELS_MIDDLE_* of the correction MLP's middle layer (0: SiLU) */
} dels_domino_rollout;

size_t dels_domino_rollout_ws_bytes(int64_t batch, int64_t steps, int64_t D, int64_t G, int64_t E, int64_t V);
int dels_domino_rollout_enqueue(const dels_domino_rollout* p, void* stream);
/* hipGraph of the rollout (torch.cuda.graph of code/kernel/domino.py:364-377); launch and
 * destroy with dels_graph_launch / dels_graph_destroy. */
int dels_domino_graph_create(const dels_domino_rollout* p, void** graph_out);

/*
 * Markov DeLS step: the rank of row m is a row of a table, rank_m =
 * E[tokens[m]] (F.embedding(current_token, embedding_weight)), followed by the
 * fused argmax of dels_fused_argmax.  Replaces _fused_markov_argmax_kernel +
 * _reduce_argmax_kernel with the embedding gather of
 * MarkovDeLSGraphRunner._forward_impl (code/kernel/markov_dels.py:15-138,
 * 216-258, 261-268); the gather is the kernels' rank load, no separate launch.
 *   tokens[m*tok_stride] int64, clamped to [0, table_rows);
 *   E [table_rows, r] bf16 row-major (lde % 8 == 0, 16-byte aligned);
 *   the rest as dels_fused_argmax (B [V, r] bf16 in b_layout).
 */
size_t dels_gather_argmax_ws_bytes(int64_t M, int64_t r, int64_t V);
int dels_gather_argmax(const int64_t* tokens, int64_t tok_stride, const void* E, int64_t lde,
                       int64_t table_rows, const void* B, int64_t ldb, int b_layout,
                       const void* base, int64_t ldbase, int base_dtype,
                       const void* prior, int prior_dtype,
                       const float* alpha, int64_t alpha_stride,
                       const float* beta, int64_t beta_stride,
                       int64_t M, int64_t r, int64_t V,
                       int64_t* out_ids, float* out_score, int64_t ld_out,
                       void* ws, size_t ws_bytes, void* stream);

/*
 * The Markov rollout of MarkovDeLSGraphRunner._forward_impl
 * (code/kernel/markov_dels.py:261-278): token_0 = prev_ids; for each step s,
 * out_ids[:, s] = dels_gather_argmax(token_s) against base[:, s, :] with
 * alpha[s]/beta[s], and token_{s+1} = out_ids[:, s].  One launch per step.
 */
typedef struct dels_markov_rollout {
    const void* embedding;  /* [table_rows, r] bf16 row-major */
    int64_t ld_embedding;
    int64_t table_rows;
    const void* lm_w;       /* [V, r] bf16 */
    int lm_layout;          /* DELS_LAYOUT_ROWMAJOR (ld = r) or DELS_LAYOUT_MFMA16 */
    const void* prior;      /* [V] or NULL */
    int prior_dtype;
    const float* alpha;     /* [steps] fp32 */
    const float* beta;      /* [steps] fp32 */
    int64_t batch, steps, r, V;
    const int64_t* prev_ids; /* [batch] int64 */
    const void* base;       /* [batch, steps, V]: row b, step s at base + (b * ld_base + s * V) */
    int base_dtype;
    int64_t ld_base;        /* elements between batch rows of base (0: steps * V) */
    int64_t* out_ids;       /* [batch, steps] int64 */
    float* out_scores;      /* [batch, steps] fp32 or NULL */
    void* ws;
    size_t ws_bytes;
} dels_markov_rollout;

size_t dels_markov_rollout_ws_bytes(int64_t batch, int64_t r, int64_t V);
int dels_markov_rollout_enqueue(const dels_markov_rollout* p, void* stream);
int dels_markov_graph_create(const dels_markov_rollout* p, void** graph_out);

#ifdef __cplusplus
}
#endif

#endif /* DELS_H */

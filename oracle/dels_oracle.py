"""CPU oracle: a numpy restatement of DeLS-Spec's draft-token selection path.

TEST INFRASTRUCTURE ONLY -- what the HIP path is tested against, never shipped and
never called by the package.  Every function cites the reference lines it
restates (paths relative to the dt-3t/DeLS-Spec repository root).

Arithmetic contract restated here (the "Triton semantics" of the fused path,
``code/kernel/dels.py:42-138``):

    rank_m  = bf16(act(bf16(h_m . A^T + bias)))            # F.linear in bf16
    dot     = sum_r fp32(B[v, r]) * fp32(rank_m[r])         # fp32 accumulate
    s[m, v] = dot * alpha_m + base[m, v] - beta_m * prior[v]  (prior term only
              when a prior is given and beta_m != 0)
    id_m    = min{v : s[m, v] == max_u s[m, u]}             # lowest index wins
    score_m = s[m, id_m]

The dot product is evaluated in float64 and rounded once to float32 (the
reference's fp32 accumulation order is compiler-defined, so no fixed order can
be "the" reference; the exact dot is the common target).  The combine is two
fused multiply-adds, each rounded once to float32:

    s = fma(dot, alpha_m, base[m, v]);   s = fma(-beta_m, prior[v], s)

which is how the reference's Triton kernel computes ``acc *= ALPHA; acc +=
base`` and ``acc -= BETA * baseline`` (Triton compiles with floating-point
contraction enabled by default, so a multiply feeding an add becomes one fma).

Pinning (see tests/test_oracle_*.py): bf16/e4m3 rounding against torch's own
casts; rank projection against torch.nn.functional.linear/silu; the fused
argmax against closed forms (alpha=beta=0, B=0, constant base), a pure-Python
brute force on tiny shapes, planted maxima and ties, and permutation
invariance; the GRU cell against torch.nn.GRU(bias=False); the prior against
its closed form on tiny count vectors.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "bf16_round",
    "f32_to_bf16_bits",
    "bf16_bits_to_f32",
    "e4m3_round",
    "quantize_rows_e4m3",
    "quantize_rank_e4m3",
    "fma_f32",
    "sigmoid_f32",
    "silu_f32",
    "rank_proj",
    "fused_argmax",
    "score_at",
    "lowrank_argmax",
    "eager_argmax_bf16",
    "gru_input_table",
    "gru_cell",
    "rollout",
    "markov_rollout",
    "unigram_log_prior",
    "rank_proj_fp8",
    "fused_argmax_fp8",
    "score_at_fp8",
    "lowrank_argmax_fp8",
    "check_parity",
]

_F32 = np.float32
_F64 = np.float64


# --------------------------------------------------------------------------
# Number formats
# --------------------------------------------------------------------------

def f32_to_bf16_bits(x) -> np.ndarray:
    """Round float32 to bfloat16 (round-to-nearest-even) and return the bits.

    NaN stays NaN (quiet); overflow rounds to +-inf, as torch's
    ``tensor.to(torch.bfloat16)`` does.
    """
    x = np.ascontiguousarray(x, dtype=_F32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = r.copy()
        r[nan] = ((u[nan] >> np.uint64(16)).astype(np.uint16) | np.uint16(0x0040))
    return r


def bf16_bits_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(_F32)


def bf16_round(x) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16 (kept as float32)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x)).reshape(np.shape(x))


_E4M3_MAX = 448.0


def e4m3_round(x) -> np.ndarray:
    """Round to the OCP float8 e4m3fn grid (bias 7, no inf, max 448).

    Round-to-nearest-even; finite values beyond +-448 saturate (the absmax
    scaling used here never produces them).  Returned as float32.
    """
    x = np.asarray(x, dtype=_F64)
    a = np.abs(x)
    _, ex = np.frexp(a)                     # a = f * 2**ex, f in [0.5, 1)
    e = np.maximum(ex - 1, -6)              # normal exponent, floored at subnormal range
    quantum = np.ldexp(1.0, e - 3)          # 3 mantissa bits
    q = np.round(a / quantum) * quantum     # np.round: half to even
    q = np.minimum(q, _E4M3_MAX)
    q = np.where(a == 0, 0.0, q)
    return (np.sign(x) * q).astype(_F32)


def quantize_rows_e4m3(w) -> tuple[np.ndarray, np.ndarray]:
    """Per-row (per-output-channel) absmax e4m3 quantisation.

    Returns ``(q, scale)`` with ``q`` on the e4m3 grid (float32 values) and
    ``w ~= q * scale[:, None]``; ``scale = absmax / 448`` (1.0 for an all-zero
    row).  This is the fp8 storage format of the fp8 variant of the path.
    """
    w = np.asarray(w, dtype=_F32)
    amax = np.abs(w).max(axis=1)
    scale = np.where(amax > 0, amax / _F32(_E4M3_MAX), _F32(1.0)).astype(_F32)
    q = e4m3_round(w / scale[:, None])
    return q, scale


def sigmoid_f32(x) -> np.ndarray:
    x = np.asarray(x, dtype=_F32)
    with np.errstate(over="ignore"):
        return (_F32(1.0) / (_F32(1.0) + np.exp(-x))).astype(_F32)


def silu_f32(x) -> np.ndarray:
    x = np.asarray(x, dtype=_F32)
    with np.errstate(over="ignore"):
        return (x / (_F32(1.0) + np.exp(-x))).astype(_F32)


def fma_f32(a, b, c) -> np.ndarray:
    """``a * b + c`` for float32 operands, rounded once to float32 (round to nearest even).

    The product of two float32 values is exact in float64; the sum is rounded
    to float64 *to odd* (the TwoSum residual says whether it was exact, and an
    inexact even result steps one float64 ulp towards the residual), and the
    odd-rounded float64 is then rounded to float32.  Rounding to odd in a format
    with at least two more bits makes the second rounding correct (Boldo and
    Melquiond, "When double rounding is odd", 2005).  inf/NaN operands follow
    IEEE arithmetic.
    """
    a = np.asarray(a, _F32).astype(_F64)
    b = np.asarray(b, _F32).astype(_F64)
    c = np.asarray(c, _F32).astype(_F64)
    with np.errstate(invalid="ignore", over="ignore"):
        p = a * b
        s = p + c
        bb = s - p
        err = (p - (s - bb)) + (c - bb)          # exact residual of s = fl64(p + c)
        finite = np.isfinite(s) & np.isfinite(err)
        even = (s.view(np.uint64) & np.uint64(1)) == 0
        bump = finite & (err != 0) & even
        s = np.where(bump, np.nextafter(s, np.where(err > 0, np.inf, -np.inf)), s)
    return s.astype(_F32)


def _dot_f32(a, b) -> np.ndarray:
    """``a @ b.T`` evaluated in float64, rounded once to float32."""
    return (np.asarray(a, _F64) @ np.asarray(b, _F64).T).astype(_F32)


# --------------------------------------------------------------------------
# a4: rank projection  (code/kernel/dels.py:437-443, code/dels.py:334-339)
# --------------------------------------------------------------------------

def rank_proj(h, A, bias=None, act: str = "identity") -> np.ndarray:
    """``rank = act(F.linear(h, A, bias))`` with bf16 outputs.

    ``F.linear`` on bf16 tensors accumulates in fp32, adds the bias and rounds
    to bf16 once; ``F.silu`` on a bf16 tensor evaluates in fp32 and rounds to
    bf16 again (code/kernel/dels.py:437-439).
    """
    pre = _dot_f32(h, A)
    if bias is not None:
        pre = (pre + np.asarray(bias, _F32)[None, :]).astype(_F32)
    rank = bf16_round(pre)
    if act == "silu":
        rank = bf16_round(silu_f32(rank))
    elif act != "identity":
        raise ValueError(f"Unsupported DeLS rank_activation={act!r}.")
    return rank


# --------------------------------------------------------------------------
# a1 + a2: fused combine and argmax  (code/kernel/dels.py:42-98, 100-138)
# --------------------------------------------------------------------------

def _combine(dot, base, prior, alpha, beta):
    """fp32 combine of one [M, C] chunk (code/kernel/dels.py:68-90), as two fmas."""
    s = fma_f32(dot, alpha[:, None], base)                  # acc *= ALPHA; acc += base   (68-79)
    if prior is not None:                                   # if HAS_BASELINE             (81-88)
        use = beta != 0
        if use.any():
            sp = fma_f32(-beta[:, None], prior[None, :], s)  # acc -= BETA * baseline
            s = np.where(use[:, None], sp, s)
    return s


def _rowvec(x, M):
    x = np.asarray(x, dtype=_F32).reshape(-1)
    if x.size == 1:
        x = np.full(M, x[0], dtype=_F32)
    if x.size != M:
        raise ValueError(f"per-row vector has {x.size} entries, expected {M}")
    return x


def fused_argmax(rank, B, base, prior, alpha, beta, *, chunk: int = 8192):
    """Argmax over the vocabulary of the fp32 combined score.

    Returns ``(ids int64[M], score f32[M], second f32[M])``: the winning
    index (lowest index among equal maxima; an all ``-inf`` row gives 0, as
    the reference's strict ``>`` cross-tile update does,
    code/kernel/dels.py:114-138), its score, and the largest score at any
    other index (the top-2 runner-up, used by the parity margin rule).
    """
    rank = np.asarray(rank, _F32)
    B = np.asarray(B, _F32)
    base = np.asarray(base, _F32)
    M, V = base.shape
    alpha = _rowvec(alpha, M)
    beta = _rowvec(beta, M)
    prior = None if prior is None else np.asarray(prior, _F32).reshape(-1)
    best = np.full(M, -np.inf, _F32)
    idx = np.zeros(M, np.int64)
    second = np.full(M, -np.inf, _F32)
    rows = np.arange(M)
    r64 = rank.astype(_F64)
    for v0 in range(0, V, chunk):
        v1 = min(V, v0 + chunk)
        dot = (r64 @ B[v0:v1].astype(_F64).T).astype(_F32)
        s = _combine(dot, base[:, v0:v1], None if prior is None else prior[v0:v1], alpha, beta)
        i1 = np.argmax(s, axis=1)
        c1 = s[rows, i1].copy()
        s[rows, i1] = -np.inf
        c2 = s.max(axis=1) if s.shape[1] > 1 else np.full(M, -np.inf, _F32)
        take = c1 > best
        second = np.where(take, np.maximum(best, c2), np.maximum(second, c1)).astype(_F32)
        idx = np.where(take, i1 + v0, idx)
        best = np.where(take, c1, best).astype(_F32)
    return idx.astype(np.int64), best, second


def score_at(rank, B, base, prior, alpha, beta, ids) -> np.ndarray:
    """The fp32 combined score of row m at vocabulary index ``ids[m]``."""
    rank = np.asarray(rank, _F32)
    base = np.asarray(base, _F32)
    M = base.shape[0]
    ids = np.asarray(ids, np.int64).reshape(-1)
    alpha = _rowvec(alpha, M)
    beta = _rowvec(beta, M)
    Bv = np.asarray(B, _F32)[ids]
    dot = np.einsum("mk,mk->m", rank.astype(_F64), Bv.astype(_F64)).astype(_F32)
    s = fma_f32(dot, alpha, base[np.arange(M), ids])
    if prior is not None:
        p = np.asarray(prior, _F32).reshape(-1)[ids]
        s = np.where(beta != 0, fma_f32(-beta, p, s), s)
    return s.astype(_F32)


def lowrank_argmax(h, A, bias, act, B, base, prior, alpha, beta, **kw):
    """Rank projection followed by the fused argmax (code/kernel/dels.py:437-446)."""
    rank = rank_proj(h, A, bias, act)
    return (rank,) + fused_argmax(rank, B, base, prior, alpha, beta, **kw)


# --------------------------------------------------------------------------
# a6: eager bf16 combine  (code/kernel/dels.py:447-456, code/dflash.py:516-529)
# --------------------------------------------------------------------------

def eager_argmax_bf16(rank, B, base, prior, alpha, beta) -> np.ndarray:
    """The reference's non-Triton path: every op in bf16, then argmax.

    ``short = F.linear(rank, B)`` rounds to bf16; ``long + alpha*short`` and
    ``- beta*prior`` each round to bf16 (torch evaluates bf16 elementwise ops
    in fp32 and rounds once per op).
    """
    base = bf16_round(np.asarray(base, _F32))
    M = base.shape[0]
    alpha = _rowvec(alpha, M)
    beta = _rowvec(beta, M)
    short = bf16_round(_dot_f32(rank, B))
    final = bf16_round(base + bf16_round(alpha[:, None] * short))
    if prior is not None:
        p = bf16_round(np.asarray(prior, _F32).reshape(1, -1))
        use = beta != 0
        final = np.where(use[:, None], bf16_round(final - bf16_round(beta[:, None] * p)), final)
    return np.argmax(final, axis=1).astype(np.int64)


# --------------------------------------------------------------------------
# a8: GRU local-head step  (code/kernel/dels.py:265-268, 359-373, 202-205)
# --------------------------------------------------------------------------

def gru_input_table(E, W_ih, b_ih=None) -> np.ndarray:
    """``gi_table = F.linear(E, W_ih, b_ih)`` in bf16 (code/kernel/dels.py:265-268)."""
    t = _dot_f32(E, W_ih)
    if b_ih is not None:
        t = (t + np.asarray(b_ih, _F32)[None, :]).astype(_F32)
    return bf16_round(t)


def gru_cell(gi, h, W_hh, b_hh=None) -> np.ndarray:
    """One GRU step as the graph runner computes it.

    ``gh = F.linear(h, W_hh, b_hh)`` rounds to bf16 (code/kernel/dels.py:365);
    the gates are evaluated in fp32 with PyTorch's (r, z, n) order and
    ``tanh(x) = 2*sigmoid(2x) - 1`` (code/kernel/dels.py:202-205); the new
    state is stored in bf16 (207-211).
    """
    gi = np.asarray(gi, _F32)
    h = np.asarray(h, _F32)
    G = h.shape[1]
    gh = _dot_f32(h, W_hh)
    if b_hh is not None:
        gh = (gh + np.asarray(b_hh, _F32)[None, :]).astype(_F32)
    gh = bf16_round(gh)
    i_r, i_z, i_n = gi[:, :G], gi[:, G:2 * G], gi[:, 2 * G:3 * G]
    h_r, h_z, h_n = gh[:, :G], gh[:, G:2 * G], gh[:, 2 * G:3 * G]
    r = sigmoid_f32(i_r + h_r)
    z = sigmoid_f32(i_z + h_z)
    n = (_F32(2.0) * sigmoid_f32(_F32(2.0) * (i_n + r * h_n)) - _F32(1.0)).astype(_F32)
    h_new = ((_F32(1.0) - z) * n + z * h).astype(_F32)
    return bf16_round(h_new)


# --------------------------------------------------------------------------
# a7: suffix rollout of the graph runner  (code/kernel/dels.py:425-467)
# --------------------------------------------------------------------------

def rollout(prefix_ids, base, *, gi_table=None, W_hh, b_hh, A, rank_bias, act, B,
            prior, alphas, betas, forced_ids=None, embed=None, W_ih=None, b_ih=None):
    """The DeLS suffix rollout, step by step.

    ``h0 = GRU(gi_table[prefix], 0)``; for each step: rank projection, fused
    argmax against ``base[:, step]``, then (unless last) a GRU step on the
    chosen token.  With ``forced_ids`` the GRU is fed those tokens instead of
    the oracle's own picks (teacher forcing), so a device rollout can be
    checked step by step on its own history.  Instead of the full input table,
    ``embed``/``W_ih``/``b_ih`` may be given: the rows are then computed when
    gathered (each row is independent, so the values are the same).

    Returns ``(ids, scores, seconds)``, each ``[batch, steps]``.
    """
    prefix_ids = np.asarray(prefix_ids, np.int64).reshape(-1)
    base = np.asarray(base, _F32)
    nb, steps, V = base.shape
    G = np.asarray(W_hh).shape[1]

    def gi_rows(tok):
        if gi_table is not None:
            return np.asarray(gi_table, _F32)[tok]
        return gru_input_table(np.asarray(embed, _F32)[tok], W_ih, b_ih)

    h = np.zeros((nb, G), _F32)
    h = gru_cell(gi_rows(prefix_ids), h, W_hh, b_hh)
    ids = np.zeros((nb, steps), np.int64)
    scores = np.zeros((nb, steps), _F32)
    seconds = np.zeros((nb, steps), _F32)
    for s in range(steps):
        rank = rank_proj(h, A, rank_bias, act)
        i, sc, sec = fused_argmax(rank, B, base[:, s, :], prior,
                                  np.full(nb, alphas[s], _F32), np.full(nb, betas[s], _F32))
        ids[:, s], scores[:, s], seconds[:, s] = i, sc, sec
        tok = i if forced_ids is None else np.asarray(forced_ids, np.int64)[:, s]
        if s + 1 < steps:
            h = gru_cell(gi_rows(tok), h, W_hh, b_hh)
    return ids, scores, seconds


def markov_rollout(prev_ids, base, *, E, B, prior, alphas, betas, forced_ids=None):
    """The Markov DeLS rollout (code/kernel/markov_dels.py:261-278).

    ``token_0 = prev_ids``; for each step s the rank is the table row
    ``E[token_s]`` (F.embedding; ids clamped into the table), the fused argmax
    against ``base[:, s]`` with ``alphas[s]``/``betas[s]`` picks ``out[:, s]``,
    and ``token_{s+1} = out[:, s]`` (or ``forced_ids[:, s]``, teacher forcing).
    Returns ``(ids, scores, seconds)``, each ``[batch, steps]``.
    """
    tok = np.asarray(prev_ids, np.int64).reshape(-1)
    base = np.asarray(base, _F32)
    E = np.asarray(E, _F32)
    nb, steps, V = base.shape
    ids = np.zeros((nb, steps), np.int64)
    scores = np.zeros((nb, steps), _F32)
    seconds = np.zeros((nb, steps), _F32)
    for s in range(steps):
        rank = E[np.clip(tok, 0, E.shape[0] - 1)]
        i, sc, sec = fused_argmax(rank, B, base[:, s, :], prior, np.full(nb, alphas[s], _F32),
                                  np.full(nb, betas[s], _F32))
        ids[:, s], scores[:, s], seconds[:, s] = i, sc, sec
        tok = i if forced_ids is None else np.asarray(forced_ids, np.int64)[:, s]
    return ids, scores, seconds


# --------------------------------------------------------------------------
# a9: unigram log-prior  (code/dels.py:66-90)
# --------------------------------------------------------------------------

def unigram_log_prior(counts, vocab_size: int, smoothing: float = 1.0) -> np.ndarray:
    """Normalised log unigram probabilities from token counts (float64).

    Counts are zero-padded to ``vocab_size``; with ``smoothing > 0`` the
    result is ``log(c + s) - log(sum(c + s))``; with ``smoothing == 0`` zero
    counts are floored to the smallest log-probability of a seen token.
    """
    if smoothing < 0:
        raise ValueError("smoothing must be non-negative.")
    c = np.asarray(counts, _F64).reshape(-1)
    if c.size > vocab_size:
        raise ValueError(
            f"Unigram baseline vocab size {c.size} exceeds runtime vocab size {vocab_size}.")
    if c.size < vocab_size:
        c = np.concatenate([c, np.zeros(vocab_size - c.size, _F64)])
    if smoothing == 0.0:
        nz = c > 0
        if not nz.any():
            raise ValueError("Unigram baseline has no positive counts.")
        out = np.full(vocab_size, -np.inf, _F64)
        out[nz] = np.log(c[nz]) - np.log(c.sum())
        out[~nz] = out[nz].min()
        return out
    sm = c + float(smoothing)
    return np.log(sm) - np.log(sm.sum())


# --------------------------------------------------------------------------
# fp8 variant (no counterpart in the reference: the format of the fp8
# configuration -- e4m3fn weights with per-output-channel fp32 scales)
# --------------------------------------------------------------------------

def rank_proj_fp8(h, A_q, A_scale, bias=None, act: str = "identity") -> np.ndarray:
    """Rank projection with e4m3 weights: ``bf16(act(bf16(scale_n * h.A_q[n])))``."""
    pre = (_dot_f32(h, A_q) * np.asarray(A_scale, _F32)[None, :]).astype(_F32)
    if bias is not None:
        pre = (pre + np.asarray(bias, _F32)[None, :]).astype(_F32)
    rank = bf16_round(pre)
    if act == "silu":
        rank = bf16_round(silu_f32(rank))
    elif act != "identity":
        raise ValueError(f"Unsupported DeLS rank_activation={act!r}.")
    return rank


def fused_argmax_fp8(rank, B_q, B_scale, base, prior, alpha, beta, *, chunk: int = 8192):
    """fp8 argmax on a given rank: each rank row quantised to e4m3, then an fp8 x fp8 contraction.

    ``R_q, sR = quantize_rank_e4m3(rank)``;
    ``dot[m, v] = fp32(fp32(R_q[m] . B_q[v]) * sR[m]) * sB[v]`` followed by the
    same fp32 combine and argmax as the bf16 path (``fused_argmax``).  Returns
    ``(ids, best, second)``.
    """
    R_q, R_scale = quantize_rank_e4m3(rank)
    base = np.asarray(base, _F32)
    M, V = base.shape
    alpha = _rowvec(alpha, M)
    beta = _rowvec(beta, M)
    prior = None if prior is None else np.asarray(prior, _F32).reshape(-1)
    B_q = np.asarray(B_q, _F32)
    B_scale = np.asarray(B_scale, _F32)
    best = np.full(M, -np.inf, _F32)
    idx = np.zeros(M, np.int64)
    second = np.full(M, -np.inf, _F32)
    rows = np.arange(M)
    for v0 in range(0, V, chunk):
        v1 = min(V, v0 + chunk)
        raw = _dot_f32(R_q, B_q[v0:v1])
        dot = ((raw * R_scale[:, None]).astype(_F32) * B_scale[None, v0:v1]).astype(_F32)
        s = _combine(dot, base[:, v0:v1], None if prior is None else prior[v0:v1], alpha, beta)
        i1 = np.argmax(s, axis=1)
        c1 = s[rows, i1].copy()
        s[rows, i1] = -np.inf
        c2 = s.max(axis=1) if s.shape[1] > 1 else np.full(M, -np.inf, _F32)
        take = c1 > best
        second = np.where(take, np.maximum(best, c2), np.maximum(second, c1)).astype(_F32)
        idx = np.where(take, i1 + v0, idx)
        best = np.where(take, c1, best).astype(_F32)
    return idx.astype(np.int64), best, second


def quantize_rank_e4m3(rank) -> tuple[np.ndarray, np.ndarray]:
    """Per-row e4m3 quantisation of the rank inside the fp8 kernels.

    ``inv = fp32(448 / absmax)``, ``q = e4m3(fp32(rank * inv))`` and
    ``scale = fp32(absmax / 448)`` (1 and zeros for an all-zero row): one
    division per row instead of one per element, so the rounding differs from
    ``quantize_rows_e4m3`` (``w / scale``) by at most one fp32 ulp of the
    quotient before the e4m3 rounding.
    """
    w = np.asarray(rank, dtype=_F32)
    amax = np.abs(w).max(axis=1)
    nz = amax > 0
    safe = np.where(nz, amax, _F32(1.0)).astype(_F32)
    inv = np.where(nz, (_F32(_E4M3_MAX) / safe).astype(_F32), _F32(1.0)).astype(_F32)
    scale = np.where(nz, (safe / _F32(_E4M3_MAX)).astype(_F32), _F32(1.0)).astype(_F32)
    q = e4m3_round((w * inv[:, None]).astype(_F32))
    return q, scale


def score_at_fp8(rank, B_q, B_scale, base, prior, alpha, beta, ids) -> np.ndarray:
    """The fp8 path's combined score of row m at vocabulary index ``ids[m]``."""
    R_q, R_scale = quantize_rank_e4m3(rank)
    base = np.asarray(base, _F32)
    M = base.shape[0]
    ids = np.asarray(ids, np.int64).reshape(-1)
    alpha = _rowvec(alpha, M)
    beta = _rowvec(beta, M)
    Bv = np.asarray(B_q, _F32)[ids]
    raw = np.einsum("mk,mk->m", R_q.astype(_F64), Bv.astype(_F64)).astype(_F32)
    dot = ((raw * R_scale).astype(_F32) * np.asarray(B_scale, _F32)[ids]).astype(_F32)
    s = fma_f32(dot, alpha, base[np.arange(M), ids])
    if prior is not None:
        p = np.asarray(prior, _F32).reshape(-1)[ids]
        s = np.where(beta != 0, fma_f32(-beta, p, s), s)
    return s.astype(_F32)


def lowrank_argmax_fp8(h, A_q, A_scale, bias, act, B_q, B_scale, base, prior, alpha, beta,
                       *, chunk: int = 8192):
    """fp8 variant of a whole step: ``rank_proj_fp8`` then ``fused_argmax_fp8``.

    Returns ``(rank, ids, best, second)``.
    """
    rank = rank_proj_fp8(h, A_q, A_scale, bias, act)
    idx, best, second = fused_argmax_fp8(rank, B_q, B_scale, base, prior, alpha, beta, chunk=chunk)
    return rank, idx, best, second


# --------------------------------------------------------------------------
# Parity rule: ids exact where the top-2 margin exceeds 1e-3 relative; the
# winning score within 1e-2 absolute.
# --------------------------------------------------------------------------

def check_parity(dev_ids, dev_scores, ref_ids, ref_scores, ref_second, dev_pick_scores=None,
                 *, rel_margin: float = 1e-3, score_atol: float = 1e-2) -> dict:
    """Compare device results with the oracle under the parity rule.

    ``dev_pick_scores`` (optional) are the oracle's scores at the device's
    chosen ids: where the margin is too small for the id to be pinned, the
    device's pick must still be a near-maximum under the oracle.
    Returns a dict of counts and the indices of failing rows.
    """
    dev_ids = np.asarray(dev_ids, np.int64).reshape(-1)
    ref_ids = np.asarray(ref_ids, np.int64).reshape(-1)
    ref_scores = np.asarray(ref_scores, _F64).reshape(-1)
    ref_second = np.asarray(ref_second, _F64).reshape(-1)
    scale = np.maximum(np.abs(ref_scores), 1e-30)
    with np.errstate(invalid="ignore"):               # inf - inf on all -inf rows
        margin = (ref_scores - ref_second) / scale
        pinned = margin > rel_margin
        id_bad = pinned & (dev_ids != ref_ids)
        res = {"rows": int(dev_ids.size), "pinned": int(pinned.sum()),
               "id_mismatch_pinned": int(id_bad.sum()), "bad_rows": np.nonzero(id_bad)[0].tolist()}
        if dev_scores is not None:
            ds = np.asarray(dev_scores, _F64).reshape(-1)
            both_inf = np.isinf(ds) & np.isinf(ref_scores) & (np.sign(ds) == np.sign(ref_scores))
            sc_bad = ~both_inf & ~(np.abs(ds - ref_scores) <= score_atol)
            res["score_bad"] = int(sc_bad.sum())
            res["score_bad_rows"] = np.nonzero(sc_bad)[0].tolist()
            finite = ~both_inf
            res["max_score_err"] = float(np.max(np.abs(ds - ref_scores)[finite])) if finite.any() else 0.0
        if dev_pick_scores is not None:
            ps = np.asarray(dev_pick_scores, _F64).reshape(-1)
            slack = rel_margin * scale + 1e-6
            near_bad = ~pinned & ~(ps >= ref_scores - slack) & ~np.isinf(ref_scores)
            res["unpinned_far_pick"] = int(near_bad.sum())
    return res

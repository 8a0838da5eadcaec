"""Error bounds that turn "ids agree wherever the margin allows" into a checkable rule.

TEST INFRASTRUCTURE ONLY -- used by tests/ to compare a path that rounds
differently from the fp32 oracle (the fp8 configuration, the reference's eager
bf16 fallback) with it, never shipped.  Paths are relative to the
dt-3t/DeLS-Spec repository.

Both checks follow one argument.  Let ``s`` be the fp32-semantics score of the
fused path (``code/kernel/dels.py:42-98``) and ``t`` another path's score of
the same row, with ``|t[v] - s[v]| <= E[v]`` for every vocabulary entry ``v``.
If ``t`` picks ``g`` and ``s`` picks ``b`` (``b`` maximises ``s``), then

    s[b] - s[g] <= (t[b] + E[b]) - (t[g] - E[g]) <= E[b] + E[g]      (t[g] >= t[b])

so a pick that violates this is a defect, not rounding; and on a row whose
top-2 margin of ``s`` exceeds ``2 max_v E[v]`` the two ids must be equal.

Pinned in tests/test_oracle_bounds.py: on brute-forced small cases the bound
dominates the true difference at every entry, and leaving out any one of its
terms lets a constructed case escape it.
"""

from __future__ import annotations

import numpy as np

from .dels_oracle import _rowvec, quantize_rank_e4m3

_F32 = np.float32
_F64 = np.float64
_U = 2.0 ** -24            # fp32 unit roundoff
_UB = 2.0 ** -8            # bf16 unit roundoff (8 bits of precision)

__all__ = ["fp8_error_bound", "fp8_bound_at", "rank_order_slack", "eager_bf16_error_bound", "eager_bound_at",
           "pick_consistent"]


def _abs64(x):
    return np.abs(np.asarray(x, _F64))


def _rank_terms(rank_bf16, rank_fp8):
    """|eR|, |rank| and |rank_used| per row (float64): ``rank_used`` is what the fp8 MFMA contracts."""
    R_q, sR = quantize_rank_e4m3(rank_fp8)
    used = np.asarray(R_q, _F64) * np.asarray(sR, _F64)[:, None]
    return np.abs(used - np.asarray(rank_bf16, _F64)), _abs64(rank_bf16), np.abs(used)


def _vocab_terms(B, B_q, B_scale):
    """|B| + |eB|, |eB| and |B_deq| per vocabulary row (float64), ``B_deq`` the dequantised e4m3 B."""
    Bc = np.asarray(B, _F64)
    Bd = np.asarray(B_q, _F64) * np.asarray(B_scale, _F64)[:, None]
    aeB = np.abs(Bd - Bc)
    return np.abs(Bc) + aeB, aeB, np.abs(Bd)


def _fp8_bound_from(aeR, arank, aused, aB_eB, aeB, aBd, alpha, base_abs, prior_term_abs):
    """E = |alpha| (|eR|.(|B| + |eB|) + |rank|.|eB|)             (quantisation: (rank + eR).(B + eB) - rank.B)
         + |alpha| (r + 4) u |rank_used|.|B_deq|                    (fp32 accumulation and the two scale products)
         + 4 u (|base| + |beta prior| + |alpha| |rank_used|.|B_deq|) + 1e-30   (the combine's roundings, both paths)
    """
    r = aeR.shape[1]
    q = aeR @ aB_eB.T + arank @ aeB.T
    mag = aused @ aBd.T
    a = np.abs(alpha)[:, None]
    return a * q * (1 + 1e-12) + a * (r + 4) * _U * mag + 4 * _U * (base_abs + prior_term_abs + a * mag) + 1e-30


def _prior_term_abs(prior, beta, cols=None):
    if prior is None:
        return 0.0
    p = _abs64(np.asarray(prior, _F32).reshape(-1))
    if cols is not None:
        p = p[cols]
        return np.abs(beta) * p
    return np.abs(beta)[:, None] * p[None, :]


def fp8_error_bound(rank_bf16, rank_fp8, B, B_q, B_scale, base, prior, alpha, beta, *, chunk: int = 8192):
    """Per row, ``max_v E[m, v]``: a bound on |fp8 score - bf16-oracle score| over the whole vocabulary.

    ``rank_bf16`` is the bf16 path's rank (``rank_proj`` with the bf16 A);
    ``rank_fp8`` the fp8 path's (``rank_proj_fp8`` with the e4m3 A), which the
    fp8 kernels quantise per row (``quantize_rank_e4m3``); ``B`` the bf16
    low-rank head, ``B_q``/``B_scale`` its e4m3 values and per-row scales.
    """
    base = np.asarray(base, _F32)
    M, V = base.shape
    alpha = _rowvec(alpha, M).astype(_F64)
    beta = _rowvec(beta, M).astype(_F64)
    aeR, arank, aused = _rank_terms(rank_bf16, rank_fp8)
    out = np.zeros(M, _F64)
    for v0 in range(0, V, chunk):
        v1 = min(V, v0 + chunk)
        aB_eB, aeB, aBd = _vocab_terms(B[v0:v1], B_q[v0:v1], B_scale[v0:v1])
        pt = _prior_term_abs(None if prior is None else np.asarray(prior, _F32).reshape(-1)[v0:v1], beta)
        E = _fp8_bound_from(aeR, arank, aused, aB_eB, aeB, aBd, alpha, _abs64(base[:, v0:v1]), pt)
        out = np.maximum(out, E.max(axis=1))
    return out


def fp8_bound_at(rank_bf16, rank_fp8, B, B_q, B_scale, base, prior, alpha, beta, cols):
    """``E[m, cols[m]]`` for one vocabulary entry per row (the same bound as ``fp8_error_bound``)."""
    base = np.asarray(base, _F32)
    M = base.shape[0]
    cols = np.asarray(cols, np.int64).reshape(-1)
    alpha = _rowvec(alpha, M).astype(_F64)
    beta = _rowvec(beta, M).astype(_F64)
    aeR, arank, aused = _rank_terms(rank_bf16, rank_fp8)
    aB_eB, aeB, aBd = _vocab_terms(np.asarray(B)[cols], np.asarray(B_q)[cols], np.asarray(B_scale)[cols])
    r = aeR.shape[1]
    q = np.einsum("mk,mk->m", aeR, aB_eB) + np.einsum("mk,mk->m", arank, aeB)
    mag = np.einsum("mk,mk->m", aused, aBd)
    a = np.abs(alpha)
    pt = 0.0 if prior is None else np.abs(beta) * _abs64(np.asarray(prior, _F32).reshape(-1)[cols])
    return a * q * (1 + 1e-12) + a * (r + 4) * _U * mag + 4 * _U * (_abs64(base[np.arange(M), cols]) + pt + a * mag) \
        + 1e-30


# --------------------------------------------------------------------------
# The reference's eager bf16 step (code/kernel/dels.py:447-456,
# code/dflash.py:516-529) against the fp32 fused semantics
# --------------------------------------------------------------------------

def _eager_bound_from(a_dot, a_mag, base_abs, prior_term_abs, r):
    """Every eager op rounds to bf16 once (relative error <= u_b = 2^-8 of its result):

        short  = bf16(rank . B)               <= u_b |dot| (+ fp32 accumulation  r u |rank|.|B|)
        scaled = bf16(alpha * short)          <= u_b |alpha short|
        base16 = bf16(base)                   <= u_b |base|
        logits = bf16(base16 + scaled)        <= u_b |logits|
        pb     = bf16(beta * bf16(prior))     <= u_b |beta prior| (twice)
        final  = bf16(logits - pb)            <= u_b |final|

    with every intermediate magnitude at most ``(1 + 2^-6)`` times the sum of
    the absolute inputs: ``E = u_b (1 + 2^-6) (4 a + 3 |base| + 3 |beta p|) +
    (r + 2) u a_mag`` where ``a = |alpha dot|``; the second term also covers the
    fp32 path's own accumulation.
    """
    return _UB * (1 + 2.0 ** -6) * (4 * a_dot + 3 * base_abs + 3 * prior_term_abs) + 2 * (r + 2) * _U * a_mag + 1e-30


def rank_order_slack(h, A, rank) -> np.ndarray:
    """Per rank element, a bound on how far two bf16 ranks ``bf16(h . A^T)`` computed in
    different fp32 summation orders can differ (identity activation, no bias).

    Each fp32 sum is within ``eps = gamma_d |h|.|A|^T`` of the exact dot product
    (``gamma_d = d u / (1 - d u)``, any order); each bf16 rounding adds at most
    half an ulp: ``D = 2 eps + ulp_bf16(|rank| + 2 eps)``.
    """
    h = _abs64(h)
    A = _abs64(A)
    d = h.shape[1]
    gamma = d * _U / (1 - d * _U)
    eps = gamma * (h @ A.T)
    mag = _abs64(rank) * (1 + 2.0 ** -8) + 2 * eps       # the largest fp32 sum either path can round
    _, ex = np.frexp(np.maximum(mag, 2.0 ** -133))        # mag = f 2^ex, f in [0.5, 1): ulp = 2^(ex - 8)
    return 2 * eps + np.ldexp(1.0, ex - 8)


def eager_bf16_error_bound(rank, B, base, prior, alpha, beta, *, rank_slack=None, chunk: int = 8192):
    """Per row, ``max_v E[m, v]``: a bound on |eager bf16 score - fp32 fused score| over the vocabulary.

    ``rank_slack`` (``[M, r]``, optional) bounds how far the two paths' ranks may
    differ element by element; it adds ``|alpha| rank_slack.|B|^T``.
    """
    base = np.asarray(base, _F32)
    M, V = base.shape
    alpha = _rowvec(alpha, M).astype(_F64)
    beta = _rowvec(beta, M).astype(_F64)
    rank = np.asarray(rank, _F64)
    arank = np.abs(rank)
    r = rank.shape[1]
    out = np.zeros(M, _F64)
    for v0 in range(0, V, chunk):
        v1 = min(V, v0 + chunk)
        Bc = np.asarray(B[v0:v1], _F64)
        a_dot = np.abs(alpha)[:, None] * np.abs(rank @ Bc.T)
        a_mag = np.abs(alpha)[:, None] * (arank @ np.abs(Bc).T)
        pt = _prior_term_abs(None if prior is None else np.asarray(prior, _F32).reshape(-1)[v0:v1], beta)
        E = _eager_bound_from(a_dot, a_mag, _abs64(base[:, v0:v1]), pt, r)
        if rank_slack is not None:
            E = E + np.abs(alpha)[:, None] * (_abs64(rank_slack) @ np.abs(Bc).T) * (1 + 1e-12)
        out = np.maximum(out, E.max(axis=1))
    return out


def eager_bound_at(rank, B, base, prior, alpha, beta, cols, *, rank_slack=None):
    """``E[m, cols[m]]`` of ``eager_bf16_error_bound`` for one vocabulary entry per row."""
    base = np.asarray(base, _F32)
    M = base.shape[0]
    cols = np.asarray(cols, np.int64).reshape(-1)
    alpha = _rowvec(alpha, M).astype(_F64)
    beta = _rowvec(beta, M).astype(_F64)
    rank = np.asarray(rank, _F64)
    Bv = np.asarray(B, _F64)[cols]
    a_dot = np.abs(alpha) * np.abs(np.einsum("mk,mk->m", rank, Bv))
    a_mag = np.abs(alpha) * np.einsum("mk,mk->m", np.abs(rank), np.abs(Bv))
    pt = 0.0 if prior is None else np.abs(beta) * _abs64(np.asarray(prior, _F32).reshape(-1)[cols])
    E = _eager_bound_from(a_dot, a_mag, _abs64(base[np.arange(M), cols]), pt, rank.shape[1])
    if rank_slack is not None:
        E = E + np.abs(alpha) * np.einsum("mk,mk->m", _abs64(rank_slack), np.abs(Bv)) * (1 + 1e-12)
    return E


def pick_consistent(s_at_ref, s_at_other, e_ref, e_other):
    """True where another path's pick ``g`` is explainable by rounding: ``s[b] - s[g] <= E[b] + E[g]``.

    ``s_at_ref``/``s_at_other`` are one path's scores at its own pick ``b`` and at
    the other path's pick ``g``; ``e_ref``/``e_other`` the bounds at those entries.
    """
    d = np.asarray(s_at_ref, _F64) - np.asarray(s_at_other, _F64)
    return d <= np.asarray(e_ref, _F64) + np.asarray(e_other, _F64)

"""CPU oracle of the Domino correction path (code/kernel/domino.py).

TEST INFRASTRUCTURE ONLY -- the reference the HIP Domino kernel and rollout are tested against.

Step semantics restated from _fused_mlp_bias_argmax_kernel and
_reduce_argmax_kernel (code/kernel/domino.py:58-173):

    p        = fp32(z[m, k]) + fp32(s[m, k])                (fp32 add, 93-96)
    mid      = fp32(p * sigmoid(p))                         (SiLU as p * sigmoid(p), 97)
               or, for another middle layer f of the correction MLP (the
               reference's unfused step, 404-431), fp32(f(p)) with f
               evaluated in float64: Identity, ReLU, GELU (erf or tanh
               form, as nn.GELU defines them), Tanh, Sigmoid
    dot      = sum_k fp32(fc2[v, k]) * mid[k]               (fp32 accumulate, 99-110)
    dot      = fp32(dot + fc2_bias[v])                      (when a bias is given, 112-116)
    score    = fma(dot, alpha, base[m, v])                  (acc *= ALPHA; acc += base, 118-129)
    id_m     = lowest index of the maximum                  (tl.argmax per block, strict > across blocks)

The dot is evaluated in float64 and rounded once (the reference's fp32
accumulation order is compiler-defined).  The rollout restates
DraftCorrectionGraphRunner._forward_impl (379-436) with the GRU prefix run as
one table-gather cell per prefix id.

Pinning (tests/test_oracle_domino.py): the step against torch's own modules
(nn.Sequential(Linear, SiLU, Linear) on the concatenated [z_h, s_h] in fp32,
the reference's unfused formula, code/dflash.py:619-626) on the margin rule,
closed forms (alpha = 0 gives argmax(base); fc2 = 0 gives argmax(alpha * bias
+ base)), and a pure-Python brute force on tiny shapes; the rollout against
torch.nn.GRUCell + the same modules, teacher-forced.  Every other middle
layer against its torch module in float64 (elementwise) and through the
same nn.Sequential(Linear, module, Linear) step comparison.
"""

from __future__ import annotations

import numpy as np

from .dels_oracle import _rowvec, fma_f32, gru_cell, gru_input_table, rank_proj, sigmoid_f32

__all__ = ["MIDDLES", "domino_mid", "domino_step", "domino_rollout"]

_F32 = np.float32
_F64 = np.float64

# the middle layers of the correction MLP the kernels fuse, by name
MIDDLES = ("silu", "identity", "relu", "gelu", "gelu_tanh", "tanh", "sigmoid")


def _middle_f64(p: np.ndarray, middle: str) -> np.ndarray:
    """A middle layer other than SiLU on float64 values (nn.Identity, nn.ReLU, nn.GELU(),
    nn.GELU(approximate="tanh"), nn.Tanh, nn.Sigmoid)."""
    from scipy.special import erf

    if middle == "identity":
        return p
    if middle == "relu":
        return np.where(p > 0, p, np.where(np.isnan(p), p, 0.0))
    if middle == "gelu":
        return 0.5 * p * (1.0 + erf(p / np.sqrt(2.0)))
    if middle == "gelu_tanh":
        return 0.5 * p * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (p + 0.044715 * p ** 3)))
    if middle == "tanh":
        return np.tanh(p)
    if middle == "sigmoid":
        return 1.0 / (1.0 + np.exp(-p))
    raise ValueError(f"unknown middle layer {middle!r}")


def domino_mid(z, s, middle: str = "silu") -> np.ndarray:
    """``mid = f(p)`` with ``p = fp32(z) + fp32(s)``: SiLU as ``p * sigmoid(p)`` in fp32
    (code/kernel/domino.py:93-97), any other middle layer evaluated in float64 and
    rounded once to fp32."""
    p = (np.asarray(z, _F32) + np.asarray(s, _F32)).astype(_F32)
    if middle == "silu":
        return (p * sigmoid_f32(p)).astype(_F32)
    with np.errstate(over="ignore"):
        return _middle_f64(p.astype(_F64), middle).astype(_F32)


def domino_step(z, s, fc2, fc2_bias, base, alpha, *, middle: str = "silu", chunk: int = 8192):
    """One correction step.  Returns ``(ids int64[M], best f32[M], second f32[M])``."""
    mid = domino_mid(z, s, middle).astype(_F64)
    fc2 = np.asarray(fc2, _F32)
    base = np.asarray(base, _F32)
    M, V = base.shape
    alpha = _rowvec(alpha, M)
    bias = None if fc2_bias is None else np.asarray(fc2_bias, _F32).reshape(-1)
    best = np.full(M, -np.inf, _F32)
    idx = np.zeros(M, np.int64)
    second = np.full(M, -np.inf, _F32)
    rows = np.arange(M)
    for v0 in range(0, V, chunk):
        v1 = min(V, v0 + chunk)
        dot = (mid @ fc2[v0:v1].astype(_F64).T).astype(_F32)
        if bias is not None:
            dot = (dot + bias[None, v0:v1]).astype(_F32)
        sc = fma_f32(dot, alpha[:, None], base[:, v0:v1])
        i1 = np.argmax(sc, axis=1)
        c1 = sc[rows, i1].copy()
        sc[rows, i1] = -np.inf
        c2 = sc.max(axis=1) if sc.shape[1] > 1 else np.full(M, -np.inf, _F32)
        take = c1 > best
        second = np.where(take, np.maximum(best, c2), np.maximum(second, c1)).astype(_F32)
        idx = np.where(take, i1 + v0, idx)
        best = np.where(take, c1, best).astype(_F32)
    return idx.astype(np.int64), best, second


def domino_rollout(prefix_ids, hiddens, base, *, W_hh, b_hh, w_z, fc1_bias, w_s, fc2, fc2_bias, alpha,
                   gi_table=None, embed=None, W_ih=None, b_ih=None, forced_ids=None, middle: str = "silu"):
    """The Domino correction rollout (code/kernel/domino.py:379-436).

    ``z = F.linear(hiddens, w_z, fc1_bias)`` (bf16); ``h`` = the GRU over
    ``prefix_ids [batch, P]`` from zero (one table-gather cell per id); per
    step ``s = F.linear(h, w_s)`` (bf16), the correction step on ``z[:, t]``,
    ``s`` and ``base[:, t]``, then a GRU cell on the chosen id (or on
    ``forced_ids[:, t]``: teacher forcing) unless it is the last step.
    The input table is ``gi_table``, or its rows are computed when gathered
    from ``embed``/``W_ih``/``b_ih`` (each row is independent: same values).
    Returns ``(ids, scores, seconds)``, each ``[batch, steps]``.
    """
    prefix_ids = np.asarray(prefix_ids, np.int64)
    hiddens = np.asarray(hiddens, _F32)
    base = np.asarray(base, _F32)
    nb, steps, V = base.shape
    D = hiddens.shape[2]
    G = np.asarray(W_hh).shape[1]

    def gi_rows(tok):
        if gi_table is not None:
            return np.asarray(gi_table, _F32)[tok]
        return gru_input_table(np.asarray(embed, _F32)[tok], W_ih, b_ih)

    z = rank_proj(hiddens.reshape(nb * steps, D), w_z, fc1_bias, "identity").reshape(nb, steps, -1)
    h = np.zeros((nb, G), _F32)
    for j in range(prefix_ids.shape[1]):
        h = gru_cell(gi_rows(prefix_ids[:, j]), h, W_hh, b_hh)
    ids = np.zeros((nb, steps), np.int64)
    scores = np.zeros((nb, steps), _F32)
    seconds = np.zeros((nb, steps), _F32)
    for t in range(steps):
        s = rank_proj(h, w_s, None, "identity")
        i, sc, sec = domino_step(z[:, t], s, fc2, fc2_bias, base[:, t], np.full(nb, alpha, _F32), middle=middle)
        ids[:, t], scores[:, t], seconds[:, t] = i, sc, sec
        tok = i if forced_ids is None else np.asarray(forced_ids, np.int64)[:, t]
        if t + 1 < steps:
            h = gru_cell(gi_rows(tok), h, W_hh, b_hh)
    return ids, scores, seconds


def gru_table(embed, W_ih, b_ih=None) -> np.ndarray:
    """The runner's input table ``F.linear(embed_tokens.weight, W_ih, b_ih)`` in bf16 (328-333)."""
    return gru_input_table(embed, W_ih, b_ih)


__all__.append("gru_table")


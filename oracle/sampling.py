"""CPU oracle of temperature sampling (code/dflash.py:31-38).

TEST INFRASTRUCTURE ONLY -- the reference the HIP sampling kernel is tested against.

The reference draws ``torch.multinomial(softmax(logits / T), 1)``.  The GPU
path draws the same distribution by a Gumbel-max, and this module restates it
exactly so that the GPU's ids can be compared one for one:

    y[m, v]  = round_dtype(fp32(x[m, v]) / fp32(T))       # logits / temperature
    bits     = word v % 4 of Philox4x32-10(counter=(v // 4, m, off_lo, off_hi),
                                           key=(seed_lo, seed_hi))
    u        = ((bits >> 9) + 0.5) * 2**-23
    g        = fp32(-log(-log(u)))                          # evaluated in float64
    id_m     = argmax_v fp32(y + g)                         # lowest index on ties

Pinning (tests/test_oracle_sampling.py): Philox4x32-10 against the published
known-answer vectors of Random123 (Salmon et al., SC 2011); the Gumbel-max
against the softmax distribution (chi-square over many seeds); temperature
below 1e-5 against ``torch.argmax``.
"""

from __future__ import annotations

import numpy as np

__all__ = ["philox4x32_10", "sampling_bits", "gumbel_from_bits", "tempered_logits", "perturbed_scores", "sample_rows"]

_M0, _M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
_W0, _W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)


def philox4x32_10(c0, c1, c2, c3, k0, k1):
    """Philox4x32 with 10 rounds on uint32 arrays (broadcast); returns the four output words."""
    c = [np.asarray(x, dtype=np.uint32) for x in (c0, c1, c2, c3)]
    k0 = np.asarray(k0, dtype=np.uint32)
    k1 = np.asarray(k1, dtype=np.uint32)
    with np.errstate(over="ignore"):
        for r in range(10):
            if r:
                k0 = (k0 + _W0).astype(np.uint32)
                k1 = (k1 + _W1).astype(np.uint32)
            p0 = c[0].astype(np.uint64) * _M0
            p1 = c[2].astype(np.uint64) * _M1
            hi0, lo0 = (p0 >> np.uint64(32)).astype(np.uint32), p0.astype(np.uint32)
            hi1, lo1 = (p1 >> np.uint64(32)).astype(np.uint32), p1.astype(np.uint32)
            c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
    return c


def sampling_bits(M: int, V: int, seed: int, offset: int = 0) -> np.ndarray:
    """uint32 [M, V]: the Philox word of every (row, vocabulary index)."""
    G = (V + 3) // 4
    words = philox4x32_10(np.arange(G, dtype=np.uint32)[None, :], np.arange(M, dtype=np.uint32)[:, None],
                          np.uint32(offset & 0xFFFFFFFF), np.uint32((offset >> 32) & 0xFFFFFFFF),
                          np.uint32(seed & 0xFFFFFFFF), np.uint32((seed >> 32) & 0xFFFFFFFF))
    stack = np.stack([np.broadcast_to(w, (M, G)) for w in words], axis=-1)   # [M, G, 4]: element 4g + q
    return stack.reshape(M, 4 * G)[:, :V].copy()


def gumbel_from_bits(bits) -> np.ndarray:
    """Gumbel noise, float32: ``-log(-log(u))`` with ``u = ((bits >> 9) + 0.5) * 2**-23``, in float64, rounded once."""
    u = ((np.asarray(bits, np.uint32) >> np.uint32(9)).astype(np.float64) + 0.5) * 2.0 ** -23
    return (-np.log(-np.log(u))).astype(np.float32)


def tempered_logits(x, temperature: float, dtype: str = "float32") -> np.ndarray:
    """``logits / temperature`` as torch computes it for a tensor of ``dtype``: fp32 division, one rounding."""
    y = (np.asarray(x, np.float32) / np.float32(temperature)).astype(np.float32)
    if dtype == "bfloat16":
        from .dels_oracle import bf16_round
        y = bf16_round(y)
    elif dtype == "float16":
        y = y.astype(np.float16).astype(np.float32)
    return y


def perturbed_scores(x, temperature: float, seed: int, offset: int = 0, dtype: str = "float32") -> np.ndarray:
    """float32 [M, V]: ``fp32(y + g)``, the scores the draw maximises."""
    x = np.asarray(x, np.float32)
    M, V = x.shape
    y = tempered_logits(x, temperature, dtype)
    with np.errstate(invalid="ignore"):
        return (y + gumbel_from_bits(sampling_bits(M, V, seed, offset))).astype(np.float32)


def sample_rows(x, temperature: float, seed: int, offset: int = 0, dtype: str = "float32"):
    """Oracle of one draw per row.  Returns ``(ids int64[M], score f32[M], second f32[M])``: the
    winning perturbed score and the largest one at any other index (for the margin rule)."""
    s = perturbed_scores(x, temperature, seed, offset, dtype)
    M, V = s.shape
    nan = np.isnan(s)
    key = np.where(nan, np.inf, s)
    ids = np.argmax(key, axis=1)
    first_nan = nan.any(axis=1)
    ids = np.where(first_nan, np.argmax(nan, axis=1), ids)
    rows = np.arange(M)
    best = s[rows, ids]
    s2 = s.copy()
    s2[rows, ids] = -np.inf
    second = np.where(np.isnan(s2), -np.inf, s2).max(axis=1) if V > 1 else np.full(M, -np.inf, np.float32)
    return ids.astype(np.int64), best.astype(np.float32), second.astype(np.float32)

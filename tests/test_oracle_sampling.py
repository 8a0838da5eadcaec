"""CPU tests pinning the sampling oracle (code/dflash.py:31-38) and its host-side checks."""

import numpy as np
import pytest
import torch

from oracle import sampling as S


# Published known-answer vectors of Philox4x32-10 (Random123, kat_vectors):
# counter (4 words), key (2 words) -> output (4 words).
PHILOX_KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff, 0xffffffff, 0xffffffff, 0xffffffff), (0xffffffff, 0xffffffff),
     (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX_KAT)
def test_philox_known_answers(ctr, key, want):
    got = S.philox4x32_10(*ctr, *key)
    assert [int(w) for w in got] == list(want)


def test_bits_layout_and_streams():
    """Element v of row m is word v % 4 of the counter (v // 4, m, offset); seeds,
    offsets and rows give different streams; 64-bit seeds and offsets use both halves."""
    b = S.sampling_bits(3, 13, seed=(7 << 32) | 5, offset=(3 << 32) | 9)
    for m in range(3):
        for v in range(13):
            assert int(b[m, v]) == int(S.philox4x32_10(v // 4, m, 9, 3, 5, 7)[v % 4])
    base = S.sampling_bits(4, 64, seed=1)
    for other in (S.sampling_bits(4, 64, seed=2), S.sampling_bits(4, 64, seed=1, offset=1),
                  S.sampling_bits(4, 64, seed=1 | (1 << 32)), S.sampling_bits(4, 64, seed=1, offset=1 << 32)):
        assert (other != base).mean() > 0.99
    assert (base[0] != base[1]).mean() > 0.99


def test_gumbel_noise_is_finite_and_standard():
    """u stays inside (0, 1) for every 32-bit pattern (the extremes included), and the
    noise has the standard Gumbel mean (Euler's gamma) and variance (pi^2 / 6)."""
    ext = S.gumbel_from_bits(np.array([0, 511, 512, 0xFFFFFE00, 0xFFFFFFFF], np.uint32))
    assert np.all(np.isfinite(ext))
    g = S.gumbel_from_bits(S.sampling_bits(64, 4096, seed=11)).astype(np.float64).ravel()
    assert abs(g.mean() - 0.5772156649) < 0.01
    assert abs(g.var() - np.pi ** 2 / 6) < 0.03


@pytest.mark.parametrize("temperature", [0.5, 1.0, 2.5])
def test_gumbel_max_draws_follow_softmax(temperature):
    """Many rows holding the same logits (each row its own Philox stream) give ids whose
    frequencies match softmax(logits / T): a chi-square test at p > 1e-6."""
    from scipy.stats import chisquare

    rng = np.random.default_rng(3)
    V, N = 12, 60000
    x = (rng.standard_normal(V) * 1.5).astype(np.float32)
    ids, _, _ = S.sample_rows(np.broadcast_to(x, (N, V)).copy(), temperature, seed=1234)
    p = torch.softmax(torch.tensor(x, dtype=torch.float64) / temperature, dim=-1).numpy()
    counts = np.bincount(ids, minlength=V)
    assert chisquare(counts, p * N).pvalue > 1e-6


def test_tempered_logits_round_like_torch():
    """logits / temperature in the logits' dtype: torch's bf16 and fp16 tensor-by-scalar division."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(4096) * 7).astype(np.float32)
    for dt, name in ((torch.bfloat16, "bfloat16"), (torch.float16, "float16"), (torch.float32, "float32")):
        xt = torch.tensor(x).to(dt)
        for T in (0.3, 0.7, 1.9):
            want = (xt / T).float().numpy()
            got = S.tempered_logits(xt.float().numpy(), T, name)
            np.testing.assert_array_equal(got, want)


def test_sample_rows_ties_nan_and_planted_winner():
    """A logit far above the rest wins every draw; a NaN wins as in torch.argmax; the margin
    outputs bracket the winner."""
    x = np.zeros((3, 50), np.float32)
    x[0, 17] = 200.0
    x[1, 5] = np.nan
    x[1, 9] = np.nan
    ids, best, second = S.sample_rows(x, 1.0, seed=9)
    assert ids[0] == 17 and ids[1] == 5
    assert best[0] > second[0] + 150
    assert best[2] >= second[2]

"""GPU tests of temperature sampling (code/dflash.py:31-38) against the oracle."""

import numpy as np
import pytest
import torch

from oracle import sampling as S

pytestmark = pytest.mark.gpu

_NAMES = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}


def _check_against_oracle(x_cpu, T, seed, offset, ids, score):
    """ids equal the oracle's wherever its top-2 margin exceeds 1e-5 relative; elsewhere the
    device's pick is within that margin of the maximum; scores agree to 4e-6 relative."""
    name = _NAMES[x_cpu.dtype]
    s = S.perturbed_scores(x_cpu.float().numpy(), T, seed, offset, name)
    rid, rbest, rsecond = S.sample_rows(x_cpu.float().numpy(), T, seed, offset, name)
    ids = ids.cpu().numpy()
    score = score.cpu().numpy()
    rows = np.arange(len(ids))
    tol = 1e-5 * np.maximum(1.0, np.abs(rbest))
    pinned = (rbest - rsecond) > tol
    assert np.array_equal(ids[pinned], rid[pinned]), np.nonzero(ids != rid)
    assert np.all(s[rows, ids] >= rbest - tol)
    np.testing.assert_allclose(score, s[rows, ids], rtol=4e-6, atol=4e-6)
    return pinned.mean()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,V,T,seed,offset", [
    (16, 151936, 0.7, 1, 0),
    (5, 1001, 1.3, (123 << 32) | 77, (5 << 32) | 3),
    (3, 3, 2.0, 42, 1),
    (40, 4099, 0.05, 7, 0),
])
def test_sample_rows_matches_oracle(pkg, dev, dtype, M, V, T, seed, offset):
    g = torch.Generator().manual_seed(M * 1000 + V)
    x = (torch.randn(M, V, generator=g) * 3).to(dtype)
    ids, score = pkg.sample_rows(x.to(dev), T, seed, offset)
    torch.cuda.synchronize()
    frac = _check_against_oracle(x, T, seed, offset, ids, score)
    assert frac > 0.9


def test_sample_rows_strided_rows_and_outputs(pkg, dev):
    g = torch.Generator().manual_seed(4)
    big = torch.randn(6, 3000, generator=g).to(torch.bfloat16)
    x = big[::2, :2500]                                   # row stride 6000, 2500 columns
    out_ids = torch.full((3, 2), -1, dtype=torch.int64, device=dev)
    out_sc = torch.zeros(3, 2, dtype=torch.float32, device=dev)
    pkg.sample_rows(big.to(dev)[::2, :2500], 0.9, 55, 0, out_ids=out_ids[:, 1],
                    out_score=out_sc[:, 1])
    torch.cuda.synchronize()
    _check_against_oracle(x.contiguous(), 0.9, 55, 0, out_ids[:, 1], out_sc[:, 1])
    assert torch.all(out_ids[:, 0] == -1)


def test_draws_follow_softmax_on_gpu(pkg, dev):
    """4096 rows of the same 12 logits: frequencies match softmax(x / T) (chi-square p > 1e-6)."""
    from scipy.stats import chisquare

    x = torch.tensor([0.3, -1.0, 2.2, 0.0, 1.1, -0.4, 0.9, 1.7, -2.0, 0.5, 1.3, 0.1])
    N, T = 4096, 0.8
    counts = np.zeros(12)
    for seed in range(4):
        ids, _ = pkg.sample_rows(x.expand(N, 12).contiguous().to(dev), T, 1000 + seed)
        counts += np.bincount(ids.cpu().numpy(), minlength=12)
    p = torch.softmax(x.double() / T, -1).numpy()
    assert chisquare(counts, p * counts.sum()).pvalue > 1e-6


def test_low_temperature_is_argmax_and_repeatable(pkg, dev):
    g = torch.Generator().manual_seed(8)
    x = torch.randn(7, 5000, generator=g).to(torch.bfloat16).to(dev)
    ids0, _ = pkg.sample_rows(x, 1e-6, 3)
    assert torch.equal(ids0.cpu(), torch.argmax(x.float().cpu(), dim=-1))
    a, _ = pkg.sample_rows(x, 1.0, 99, 4)
    b, _ = pkg.sample_rows(x, 1.0, 99, 4)
    c, _ = pkg.sample_rows(x, 1.0, 99, 5)
    assert torch.equal(a, b)
    assert not torch.equal(a, c)


def test_sample_mirrors_reference_call(pkg, dev):
    """sample(logits [bsz, seq, V], temperature): argmax below 1e-5, a seeded draw above."""
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(2, 5, 777, generator=g).to(torch.bfloat16).to(dev)
    assert torch.equal(pkg.sample(logits).cpu(), torch.argmax(logits.float().cpu(), dim=-1))
    torch.manual_seed(17)
    d1 = pkg.sample(logits, 0.8)
    torch.manual_seed(17)
    d2 = pkg.sample(logits, 0.8)
    assert d1.shape == (2, 5) and d1.dtype == torch.int64 and torch.equal(d1, d2)
    ids, sc = pkg.sample_rows(logits.reshape(10, 777), 0.8, 321)
    assert torch.equal(pkg.sample(logits, 0.8, seed=321).reshape(-1), ids)


def test_bad_temperature_is_an_error(pkg, dev):
    x = torch.zeros(2, 10, device=dev)
    with pytest.raises(RuntimeError, match="temperature"):
        pkg.sample_rows(x, float("nan"), 1)

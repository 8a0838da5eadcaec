"""GPU parity of the MFMA-tiled argmax kernel at many rows (M >= 256, packed B, 16-bit base).

The tiled kernel takes the fused argmax (code/kernel/dels.py:15-138) for M >= 64
rows with B in the MFMA-16 layout; with 16-bit base logits it reads them in
whole 128-byte lines (two 32-column tiles per chunk), so a chunk can end inside
a workgroup's last tile and the vocabulary can end in half a tile.  Checked
against the oracle under the parity rule, on ragged row groups, a vocabulary
that ends in half a tile, every prior kind, ties across tiles, waves and
workgroups, all -inf rows, beta = 0 rows beside an infinite prior, strided base
views, the Markov gathered rank, and exact dot products (bit-identical scores).
"""

import numpy as np
import pytest
import torch

import oracle
from test_gpu_parity import assert_parity, f

pytestmark = pytest.mark.gpu

MANY_ROW_CASES = [
    # M, r, V, base dtype, prior dtype (None: no prior)
    (257, 512, 151936, torch.bfloat16, torch.bfloat16),   # one row in the third row group
    (384, 256, 20016, torch.bfloat16, torch.float16),     # V % 32 == 16: the last tile is half masked
    (300, 256, 50000, torch.float16, torch.float32),
    (512, 512, 151936, torch.bfloat16, None),
    (1000, 512, 30016, torch.float16, torch.bfloat16),
    (4096, 256, 4112, torch.bfloat16, torch.bfloat16),    # the most rows a call takes: 32 row groups
]


@pytest.mark.parametrize("M,r,V,bdt,pdt", MANY_ROW_CASES)
def test_tiled_many_rows_argmax_random(pkg, dev, M, r, V, bdt, pdt):
    print(f"case tiled argmax many rows M={M} r={r} V={V} base={bdt} prior={pdt}", flush=True)
    x = pkg.synth.lowrank_inputs(M, 64, r, V, base_dtype=bdt, prior_dtype=pdt or torch.float32,
                                 per_position=True, seed=M * 7 + r + V)
    rank = (torch.randn(M, r, generator=torch.Generator().manual_seed(M + V)) * 1.5).to(torch.bfloat16)
    prior = x.prior if pdt is not None else None
    beta = x.beta.clone()
    beta[::5] = 0.0                                   # rows without the prior term
    Bp = pkg.pack_operand(x.B.to(dev))
    args = (rank.to(dev), Bp, x.base.to(dev), None if prior is None else prior.to(dev), x.alpha.to(dev), beta.to(dev))
    ids, score = pkg.fused_argmax(*args)
    torch.cuda.synchronize()
    ids, score = ids.clone(), score.clone()
    assert_parity(ids, score, f(rank), f(x.B), f(x.base), None if prior is None else f(prior), f(x.alpha), f(beta))
    ids2, score2 = pkg.fused_argmax(*args)
    torch.cuda.synchronize()
    assert torch.equal(ids2, ids) and torch.equal(score2, score)


def test_tiled_many_rows_argmax_repeat_is_bitwise_stable(pkg, dev):
    M, r, V = 512, 512, 151936
    x = pkg.synth.config_inputs("qwen3_8b_m512", seed=3)
    rank = (torch.randn(M, r, generator=torch.Generator().manual_seed(4)) * 1.3).to(torch.bfloat16).to(dev)
    Bp = pkg.pack_operand(x.B.to(dev))
    args = (rank, Bp, x.base.to(dev), x.prior.to(dev), x.alpha.to(dev), x.beta.to(dev))
    first = None
    for _ in range(10):
        ids, score = pkg.fused_argmax(*args)
        torch.cuda.synchronize()
        if first is None:
            first = (ids.clone(), score.clone())
        else:
            assert torch.equal(ids, first[0]) and torch.equal(score, first[1])
    assert_parity(first[0], first[1], f(rank), f(x.B), f(x.base), f(x.prior), f(x.alpha), f(x.beta))


@pytest.mark.parametrize("r,bdt", [(512, torch.bfloat16), (256, torch.float16)])
def test_tiled_many_rows_argmax_ties_inf_strided(pkg, dev, r, bdt):
    """rank = 0, so scores are base - beta * prior exactly.  Ties inside a lane, across
    the two halves of a tile, across waves, across vocabulary streams and across the
    whole vocabulary go to the lowest index; an all -inf row gives id 0 and -inf; a
    beta = 0 row ignores an infinite prior that drives a beta = 1 row away; the base
    is a strided view (ldbase > V); the last row group is ragged."""
    M, V, ld = 300, 30000, 30016                # V % 32 == 16: the last tile is half masked
    g = torch.Generator().manual_seed(5)
    rank = torch.zeros(M, r, dtype=torch.bfloat16)
    B = (torch.randn(V, r, generator=g) * 0.02).to(torch.bfloat16)
    full = torch.randn(M, ld, generator=g).to(bdt)
    base = full[:, :V]
    alpha = torch.ones(M)
    beta = torch.zeros(M)
    prior = torch.zeros(V)
    plant = {
        0: [(29990, 50.0), (17, 50.0)],          # across the vocabulary: 17
        1: [(5000, 40.0), (5001, 40.0)],         # inside one lane's 16 columns: 5000
        3: [(15, 30.0), (16, 30.0)],             # across the two halves of a tile: 15
        4: [(64, 20.0), (32, 20.0)],             # tiles of two waves: 32
        8: [(29999, 9.0), (29985, 9.0)],         # inside the half-masked last tile: 29985
        299: [(7, 60.0), (29000, 60.0)],         # last (ragged) row group
    }
    for m, pts in plant.items():
        for v, val in pts:
            base[m, v] = val
    base[2, :] = -float("inf")                   # all -inf: id 0
    prior[123] = float("inf")
    beta[5] = 1.0
    base[5, 123] = 1e4                           # beta = 1: driven to -inf
    base[6, 123] = 1e4                           # beta = 0: kept
    Bp = pkg.pack_operand(B.to(dev))
    based = full.to(dev)[:, :V]
    assert based.stride(0) == ld
    ids, score = pkg.fused_argmax(rank.to(dev), Bp, based, prior.to(dev), alpha.to(dev), beta.to(dev))
    torch.cuda.synchronize()
    ids = ids.cpu().numpy()
    score = score.cpu().numpy()
    want = {0: 17, 1: 5000, 3: 15, 4: 32, 8: 29985, 299: 7, 2: 0, 6: 123}
    for m, v in want.items():
        assert ids[m] == v, (m, ids[m], v)
    assert score[2] == -np.inf and ids[5] != 123
    ref = oracle.fused_argmax(f(rank), f(B), f(base), f(prior), f(alpha), f(beta))
    assert np.array_equal(ids, ref[0])
    assert np.array_equal(score, ref[1])


def test_tiled_many_rows_argmax_exact_dots_are_bit_identical(pkg, dev):
    """Integer ranks and B in multiples of 1/64: every dot product is exact in fp32, so
    the kernel's scores must equal the oracle's bit for bit (same two-fma combine)."""
    M, r, V = 320, 256, 20000
    rng = np.random.default_rng(8)
    rank = rng.integers(-3, 4, (M, r)).astype(np.float32)
    B = (rng.integers(-64, 65, (V, r)) / 64).astype(np.float32)
    base = oracle.bf16_round((rng.standard_normal((M, V)) * 3).astype(np.float32))
    prior = oracle.bf16_round(np.log(rng.dirichlet(np.ones(V))).astype(np.float32))
    alpha = rng.uniform(0.05, 0.6, M).astype(np.float32)
    beta = rng.uniform(0.0, 0.6, M).astype(np.float32)
    beta[::3] = 0.0
    t = lambda a, dt=torch.float32: torch.from_numpy(a).to(dt).to(dev)  # noqa: E731
    ids, score = pkg.fused_argmax(t(rank, torch.bfloat16), pkg.pack_operand(t(B, torch.bfloat16)),
                                  t(base, torch.bfloat16), t(prior, torch.bfloat16), t(alpha), t(beta))
    torch.cuda.synchronize()
    rid, rsc, _ = oracle.fused_argmax(rank, B, base, prior, alpha, beta)
    np.testing.assert_array_equal(ids.cpu().numpy(), rid)
    np.testing.assert_array_equal(score.cpu().numpy(), rsc)


def test_tiled_many_rows_gather_argmax_markov_rows(pkg, dev):
    """The Markov step's gathered rank (row m = embedding[token_m]) at M >= 256."""
    M, r, V, rows = 512, 256, 30016, 4000
    g = torch.Generator().manual_seed(9)
    E = torch.randn(rows, r, generator=g).to(torch.bfloat16)
    W = (torch.randn(V, r, generator=g) * 0.05).to(torch.bfloat16)
    base = (torch.randn(M, V, generator=g) * 3).to(torch.bfloat16)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0).to(torch.bfloat16)
    alpha = torch.rand(M, generator=g) * 0.6
    beta = torch.rand(M, generator=g) * 0.6
    tok = torch.randint(-3, rows + 3, (M,), generator=g)      # out-of-table ids clamp to the ends
    ids, score = pkg.gather_argmax(tok.to(dev), E.to(dev), pkg.pack_operand(W.to(dev)), base.to(dev), prior.to(dev),
                                   alpha.to(dev), beta.to(dev))
    torch.cuda.synchronize()
    rank = f(E)[np.clip(tok.numpy(), 0, rows - 1)]
    assert_parity(ids, score, rank, f(W), f(base), f(prior), f(alpha), f(beta))


def test_many_rows_argmax_with_views_the_tiled_kernel_cannot_stream(pkg, dev):
    """At M >= 64 the tiled kernel moves base and prior rows with 16- and 4-byte
    direct-to-LDS loads; views without that alignment -- a base starting one
    element into its rows (ldbase % 8 != 0) and a 16-bit prior starting one
    element into its buffer -- go to the GEMV kernel instead, with the same result."""
    M, r, V = 80, 512, 30016
    g = torch.Generator().manual_seed(21)
    x = pkg.synth.lowrank_inputs(M, 64, r, V, base_dtype=torch.bfloat16, prior_dtype=torch.bfloat16,
                                 per_position=True, seed=21)
    rank = (torch.randn(M, r, generator=g) * 1.5).to(torch.bfloat16)
    full = torch.zeros(M, V + 3, dtype=torch.bfloat16)
    full[:, 1:V + 1] = x.base
    pbuf = torch.zeros(V + 1, dtype=torch.bfloat16)
    pbuf[1:] = x.prior
    based = full.to(dev)[:, 1:V + 1]
    priord = pbuf.to(dev)[1:]
    assert based.data_ptr() % 16 != 0 and based.stride(0) % 8 != 0 and priord.data_ptr() % 4 != 0
    Bp = pkg.pack_operand(x.B.to(dev))
    ids, score = pkg.fused_argmax(rank.to(dev), Bp, based, priord, x.alpha.to(dev), x.beta.to(dev))
    torch.cuda.synchronize()
    assert_parity(ids, score, f(rank), f(x.B), f(x.base), f(x.prior), f(x.alpha), f(x.beta))

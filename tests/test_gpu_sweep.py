"""A seeded sweep of whole draft steps (rank projection + fused combine/argmax)
over shapes, dtypes and weight layouts, each against the oracle with the
parity rule of test_gpu_parity.  The draws cover every kernel regime: the
one-launch decode step (M <= 16, packed weights), the GEMV argmax (row-major
B or 17 <= M < 64), the MFMA-tiled argmax (M >= 64, packed B), the skinny and
the LDS-tiled rank projections, ragged vocabularies, hidden sizes that do not
divide into the K slices, and the e4m3 variant.  Each case runs twice in a
row on one workspace: the second launch must reproduce the first bit for bit
(the decode step's tagged hand-off words of one launch never pass for the
next one's).
"""

import numpy as np
import pytest
import torch

import oracle
from test_gpu_fp8 import assert_parity_fp8, fp8_weight
from test_gpu_parity import assert_parity, f

pytestmark = pytest.mark.gpu

_DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _draw(seed):
    rng = np.random.default_rng(seed)
    M = int(rng.choice([1, 3, 7, 12, 16, 16, 24, 40, 64, 96, 130]))
    r = int(rng.choice([64, 128, 256, 512]))
    d = int(32 * rng.integers(2, 97))                  # 64 .. 3072, often not a multiple of 128
    V = int(rng.integers(500, 40000))
    if rng.random() < 0.5:
        V -= V % 16                                    # a multiple of the 16-row tile (and of 8)
    bdt = _DTYPES[int(rng.integers(0, 3))]
    pdt = None if rng.random() < 0.25 else _DTYPES[int(rng.integers(0, 3))]
    act = "silu" if rng.random() < 0.5 else "identity"
    bias = bool(rng.random() < 0.5)
    packed = bool(rng.random() < 0.75)
    return M, d, r, V, bdt, pdt, act, bias, packed


@pytest.mark.parametrize("seed", range(24))
def test_lowrank_argmax_sweep(pkg, dev, seed):
    M, d, r, V, bdt, pdt, act, bias, packed = _draw(seed)
    print(f"case sweep seed={seed} M={M} d={d} r={r} V={V} base={bdt} prior={pdt} {act} bias={bias} "
          f"packed={packed}", flush=True)
    x = pkg.synth.lowrank_inputs(M, d, r, V, base_dtype=bdt, prior_dtype=pdt or torch.float32, per_position=True,
                                 seed=1000 + seed)
    g = torch.Generator().manual_seed(seed)
    rb = (torch.randn(r, generator=g) * 0.5).to(torch.bfloat16) if bias else None
    xd = x.to(dev)
    A, B = (pkg.pack_operand(xd.A), pkg.pack_operand(xd.B)) if packed else (xd.A, xd.B)
    prior = xd.prior if pdt is not None else None
    args = (xd.h, A, B, xd.base, prior, xd.alpha, xd.beta)
    kw = dict(act=act, rank_bias=None if rb is None else rb.to(dev))
    ids, score = pkg.lowrank_argmax(*args, **kw)
    torch.cuda.synchronize()
    ids, score = ids.clone(), score.clone()
    rank = oracle.rank_proj(f(x.h), f(x.A), None if rb is None else f(rb), act)
    assert_parity(ids, score, rank, f(x.B), f(x.base), None if pdt is None else f(x.prior), f(x.alpha),
                  f(x.beta))
    ids2, score2 = pkg.lowrank_argmax(*args, **kw)
    torch.cuda.synchronize()
    assert torch.equal(ids2, ids) and torch.equal(score2, score)


@pytest.mark.parametrize("seed", range(8))
def test_lowrank_argmax_fp8_sweep(pkg, dev, seed):
    rng = np.random.default_rng(500 + seed)
    M = int(rng.choice([2, 9, 16, 33, 64, 150]))
    r = int(rng.choice([128, 256, 512]))
    d = int(32 * rng.integers(2, 97))
    V = int(rng.integers(1000, 40000))
    V -= V % 16
    bdt = _DTYPES[int(rng.integers(0, 3))]
    pdt = None if rng.random() < 0.25 else _DTYPES[int(rng.integers(0, 3))]
    act = "silu" if rng.random() < 0.5 else "identity"
    bias = bool(rng.random() < 0.5)
    print(f"case fp8 sweep seed={seed} M={M} d={d} r={r} V={V} base={bdt} prior={pdt} {act} bias={bias}",
          flush=True)
    g = torch.Generator().manual_seed(2000 + seed)
    h = torch.randn(M, d, generator=g).bfloat16()
    A, Aq, sA = fp8_weight(pkg, (torch.randn(r, d, generator=g) * 0.02).to(dev), "k32")
    B, Bq, sB = fp8_weight(pkg, (torch.randn(V, r, generator=g) * 0.02).to(dev), "k128")
    rb = (torch.randn(r, generator=g) * 0.1).bfloat16() if bias else None
    base = (torch.randn(M, V, generator=g) * 3).to(bdt)
    prior = torch.randn(V, generator=g).to(pdt) if pdt is not None else None
    alpha = (torch.rand(M, generator=g) * 0.6 + 0.2).float()
    beta = (torch.rand(M, generator=g) * 0.6).float()
    args = (h.to(dev), A, B, base.to(dev), None if prior is None else prior.to(dev), alpha.to(dev), beta.to(dev))
    kw = dict(act=act, rank_bias=None if rb is None else rb.to(dev))
    ids, score = pkg.lowrank_argmax_fp8(*args, **kw)
    torch.cuda.synchronize()
    ids, score = ids.clone(), score.clone()
    rank, rid, rsc, rsec = oracle.lowrank_argmax_fp8(f(h), Aq, sA, None if rb is None else f(rb), act, Bq, sB,
                                                     f(base), None if prior is None else f(prior), f(alpha),
                                                     f(beta))
    assert_parity_fp8(ids, score, rank, Bq, sB, f(base), None if prior is None else f(prior), f(alpha), f(beta),
                      ref=(rid, rsc, rsec))
    ids2, score2 = pkg.lowrank_argmax_fp8(*args, **kw)
    torch.cuda.synchronize()
    assert torch.equal(ids2, ids) and torch.equal(score2, score)

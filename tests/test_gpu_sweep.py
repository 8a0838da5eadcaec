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


@pytest.mark.parametrize("seed", list(range(16)) + [-1])
def test_graph_runner_rollout_sweep(pkg, dev, seed):
    """Seeded rollouts over batch, steps, hidden size (below, at and above the
    hidden size where the GRU runs inside the decode launch, up to its limit
    2048), rank, activation, rank bias and prior, teacher-forced against the
    oracle as test_graph_runner_rollout, and replayed bit for bit.  Seed -1:
    the largest fused-GRU grid (16 rows, G = 2048, r = 512: 128 rank and 128
    GRU workgroups)."""
    from test_gpu_parity import _Head

    rng = np.random.default_rng(900 + seed)
    nb = int(rng.choice([1, 2, 5, 8, 13, 16]))
    steps = int(rng.choice([1, 2, 3, 5, 9]))
    V = int(rng.integers(1000, 30000))
    E = int(rng.choice([16, 32, 64]))
    G = int(rng.choice([64, 256, 1024, 1536, 2048]))
    r = int(rng.choice([64, 128, 256, 512]))
    act = "silu" if rng.random() < 0.5 else "identity"
    rank_bias = bool(rng.random() < 0.5)
    with_prior = bool(rng.random() < 0.6)
    if seed == -1:
        nb, steps, V, E, G, r, act, rank_bias, with_prior = 16, 4, 20011, 32, 2048, 512, "silu", True, True
    std = 0.02 if G >= 1024 else 0.1
    print(f"case rollout sweep seed={seed} nb={nb} steps={steps} V={V} E={E} G={G} r={r} {act} "
          f"bias={rank_bias} prior={with_prior}", flush=True)
    head = _Head(V, E, G, r, act, rank_bias, seed=3000 + seed, std=std).to(dev)
    g = torch.Generator().manual_seed(4000 + seed)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0) if with_prior else None
    alphas = [float(a) for a in rng.uniform(0.05, 0.6, steps)]
    betas = [float(b) for b in rng.uniform(0.0, 0.5, steps)] if with_prior else [0.0] * steps
    runner = pkg.DeLSGraphRunner(local_head=head, batch_size=nb, steps=steps, vocab_size=V, alpha_values=alphas,
                                 beta_values=betas, baseline_logits=prior, device=dev)
    prefix = torch.randint(0, V, (nb, 1), generator=g)
    base = (torch.randn(nb, steps, V, generator=g) * 3).to(torch.bfloat16)
    out = runner(prefix.to(dev), base.to(dev)).clone()
    scores = runner.static_scores.clone()
    torch.cuda.synchronize()
    out2 = runner(prefix.to(dev), base.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(out2, out)
    dev_ids = out.cpu().numpy()
    rid, rsc, rsec = oracle.rollout(
        prefix.numpy().reshape(-1), f(base), embed=f(head.embed_tokens.weight), W_ih=f(head.prefix_gru.weight_ih_l0),
        W_hh=f(head.prefix_gru.weight_hh_l0), b_hh=None,
        A=f(head.rank_proj.weight), rank_bias=f(head.rank_proj.bias) if rank_bias else None, act=act,
        B=f(head.low_rank_lm_head.weight), prior=f(prior.to(torch.bfloat16)) if with_prior else None,
        alphas=alphas, betas=betas, forced_ids=dev_ids)
    res = oracle.check_parity(dev_ids.reshape(-1), f(scores).reshape(-1), rid.reshape(-1), rsc.reshape(-1),
                              rsec.reshape(-1))
    # the device's bf16 GRU state may differ from the oracle's by an ulp: allow score drift of 2e-2
    assert res["id_mismatch_pinned"] == 0, res
    assert res["max_score_err"] < 2e-2, res
    runner.close()


@pytest.mark.parametrize("nb,steps,G,r,V", [(8, 5, 1024, 256, 30011),     # GRU inside every decode launch
                                             (3, 4, 256, 128, 20011)])      # the GRU step kernel between launches
def test_graph_runner_rollout_with_gru_bias(pkg, dev, nb, steps, G, r, V):
    """A local head whose GRU has biases (b_ih folded into the input table, b_hh
    into gh, and gh = b_hh at the zero-state first step), teacher-forced against
    the oracle with both biases."""
    from test_gpu_parity import _Head

    print(f"case rollout gru bias nb={nb} steps={steps} G={G} r={r} V={V}", flush=True)
    E = 64
    head = _Head(V, E, G, r, "silu", True, seed=77 + G, std=0.02 if G >= 1024 else 0.1, gru_bias=True).to(dev)
    g = torch.Generator().manual_seed(78 + G)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0)
    alphas = [1.0 + 0.05 * i for i in range(steps)]
    betas = [0.05] * steps
    runner = pkg.DeLSGraphRunner(local_head=head, batch_size=nb, steps=steps, vocab_size=V, alpha_values=alphas,
                                 beta_values=betas, baseline_logits=prior, device=dev)
    prefix = torch.randint(0, V, (nb, 1), generator=g)
    # small base logits: the low-rank term, and with it the GRU state, decides the ids
    base = (torch.randn(nb, steps, V, generator=g) * 0.05).to(torch.bfloat16)
    out = runner(prefix.to(dev), base.to(dev)).clone()
    scores = runner.static_scores.clone()
    torch.cuda.synchronize()
    dev_ids = out.cpu().numpy()
    gru = head.prefix_gru
    rid, rsc, rsec = oracle.rollout(
        prefix.numpy().reshape(-1), f(base), embed=f(head.embed_tokens.weight), W_ih=f(gru.weight_ih_l0),
        b_ih=f(gru.bias_ih_l0), W_hh=f(gru.weight_hh_l0), b_hh=f(gru.bias_hh_l0),
        A=f(head.rank_proj.weight), rank_bias=f(head.rank_proj.bias), act="silu",
        B=f(head.low_rank_lm_head.weight), prior=f(prior.to(torch.bfloat16)), alphas=alphas, betas=betas,
        forced_ids=dev_ids)
    res = oracle.check_parity(dev_ids.reshape(-1), f(scores).reshape(-1), rid.reshape(-1), rsc.reshape(-1),
                              rsec.reshape(-1))
    assert res["id_mismatch_pinned"] == 0, res
    assert res["max_score_err"] < 2e-2, res
    # without b_hh the oracle picks other ids: the device's ids show that the bias reaches its GRU
    rid0, _, _ = oracle.rollout(
        prefix.numpy().reshape(-1), f(base), embed=f(head.embed_tokens.weight), W_ih=f(gru.weight_ih_l0),
        b_ih=f(gru.bias_ih_l0), W_hh=f(gru.weight_hh_l0), b_hh=None,
        A=f(head.rank_proj.weight), rank_bias=f(head.rank_proj.bias), act="silu",
        B=f(head.low_rank_lm_head.weight), prior=f(prior.to(torch.bfloat16)), alphas=alphas, betas=betas,
        forced_ids=dev_ids)
    assert not np.array_equal(rid0, dev_ids)
    runner.close()


@pytest.mark.parametrize("seed", range(8))
def test_gather_argmax_sweep(pkg, dev, seed):
    """The Markov path's gathered-rank argmax over seeded shapes (GEMV and
    MFMA-tiled regimes, either layout, every base/prior dtype)."""
    rng = np.random.default_rng(1200 + seed)
    M = int(rng.choice([1, 4, 16, 33, 64, 100]))
    r = int(rng.choice([32, 64, 128, 256, 512]))
    V = int(rng.integers(500, 40000))
    if rng.random() < 0.5:
        V -= V % 32
    packed = bool(rng.random() < 0.6)
    bdt = _DTYPES[int(rng.integers(0, 3))]
    pdt = _DTYPES[int(rng.integers(0, 3))]
    rows = int(rng.integers(50, 3000))
    print(f"case gather sweep seed={seed} M={M} r={r} V={V} packed={packed} base={bdt} prior={pdt} rows={rows}",
          flush=True)
    g = torch.Generator().manual_seed(5000 + seed)
    E = torch.randn(rows, r, generator=g).to(torch.bfloat16)
    W = (torch.randn(V, r, generator=g) * 0.05).to(torch.bfloat16)
    base = (torch.randn(M, V, generator=g) * 3).to(bdt)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0).to(pdt)
    alpha = torch.rand(M, generator=g) * 0.6
    beta = torch.rand(M, generator=g) * 0.6
    tok = torch.randint(-3, rows + 3, (M,), generator=g)      # out-of-table ids clamp to the ends
    Wd = W.to(dev)
    args = (tok.to(dev), E.to(dev), pkg.pack_operand(Wd) if packed else Wd, base.to(dev), prior.to(dev),
            alpha.to(dev), beta.to(dev))
    ids, score = pkg.gather_argmax(*args)
    torch.cuda.synchronize()
    ids, score = ids.clone(), score.clone()
    rank = f(E)[np.clip(tok.numpy(), 0, rows - 1)]
    assert_parity(ids, score, rank, f(W), f(base), f(prior), f(alpha), f(beta))
    ids2, score2 = pkg.gather_argmax(*args)
    torch.cuda.synchronize()
    assert torch.equal(ids2, ids) and torch.equal(score2, score)


@pytest.mark.parametrize("seed", range(8))
def test_domino_argmax_sweep(pkg, dev, seed):
    """The Domino correction step over seeded shapes and dtypes against the oracle."""
    from oracle import domino as DO

    rng = np.random.default_rng(1300 + seed)
    M = int(rng.choice([1, 3, 8, 16, 29]))
    E = int(32 * rng.integers(1, 65))
    V = int(rng.integers(100, 40000))
    bias_dt = [None, torch.bfloat16, torch.float32][int(rng.integers(0, 3))]
    base_dt = _DTYPES[int(rng.integers(0, 3))]
    alpha = float(rng.uniform(0.1, 1.5))
    print(f"case domino sweep seed={seed} M={M} E={E} V={V} bias={bias_dt} base={base_dt} alpha={alpha:.3f}",
          flush=True)
    g = torch.Generator().manual_seed(6000 + seed)
    z = torch.randn(M, E, generator=g).to(torch.bfloat16)
    s = torch.randn(M, E, generator=g).to(torch.bfloat16)
    fc2 = (torch.randn(V, E, generator=g) * 0.02).to(torch.bfloat16)
    base = (torch.randn(M, V, generator=g) * 3).to(base_dt)
    bias = torch.randn(V, generator=g).to(bias_dt) if bias_dt is not None else None
    ids, score = pkg.domino_argmax(z.to(dev), s.to(dev), pkg.pack_operand(fc2.to(dev)), base.to(dev), alpha,
                                   bias.to(dev) if bias is not None else None)
    torch.cuda.synchronize()
    rid, rbest, rsec = DO.domino_step(f(z), f(s), f(fc2), None if bias is None else f(bias), f(base), alpha)
    res = oracle.check_parity(ids.cpu().numpy(), score.cpu().numpy(), rid, rbest, rsec, score_atol=1e-4)
    assert res["id_mismatch_pinned"] == 0 and res["score_bad"] == 0, res

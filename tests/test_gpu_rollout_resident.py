"""GPU tests of the rollout that keeps the low-rank head resident on chip: every
step in one launch (dels_rollout_enqueue / dels_graph_create where the shape
allows it: weights in the MFMA-16 layout, r = 256, batch <= 16, G a power of two
up to 1024 with an even number of GRU units per CU).

Each rollout is teacher-forced against the oracle on the device's own ids
(code/kernel/dels.py:425-467) under the parity rule, graph replays must
repeat bit for bit, and the same rollout through the per-step launches must
pass the same check.  The bounded waits are exercised from the host: with
their re-read limit at zero the launch gives up, writes -1 ids, and the next
launch on the same workspace is correct again.
"""

import numpy as np
import pytest
import torch

import oracle
from test_gpu_parity import _Head

pytestmark = pytest.mark.gpu


def f(t):
    return t.detach().float().cpu().numpy()


# nb, steps, G, r, V, base dtype, with prior, activation, rank bias, GRU biases
CASES = [
    (8, 14, 1024, 256, 151936, torch.bfloat16, True, "silu", False, False),   # the draft block's rollout
    (1, 3, 1024, 256, 4099, torch.float32, False, "identity", True, True),    # few tiles: most workgroups none
    (16, 5, 512, 256, 30011, torch.float16, True, "silu", True, True),        # 16 rows, 2 GRU units per CU
    (3, 1, 1024, 256, 20011, torch.bfloat16, True, "silu", False, False),     # one step: no GRU after it
    (5, 6, 1024, 256, 100003, torch.bfloat16, True, "silu", False, True),     # ragged vocabulary, LDS tiles
]


def _rollout(pkg, dev, head, nb, steps, V, prior, alphas, betas, prefix, base, resident):
    lib = pkg._lib.load()
    prev = lib.dels_debug_set_rollout_resident(1 if resident else 0)
    try:
        runner = pkg.DeLSGraphRunner(local_head=head, batch_size=nb, steps=steps, vocab_size=V, alpha_values=alphas,
                                     beta_values=betas, baseline_logits=prior, device=dev)
    finally:
        lib.dels_debug_set_rollout_resident(prev)
    out = runner(prefix.to(dev), base.to(dev)).clone()
    scores = runner.static_scores.clone()
    again = runner(prefix.to(dev), base.to(dev)).clone()
    again_scores = runner.static_scores.clone()
    torch.cuda.synchronize()
    runner.close()
    return out, scores, again, again_scores


@torch.inference_mode()
def _eager(runner, prefix, base):
    runner.static_prefix_ids.copy_(prefix)
    runner.static_base_logits.copy_(base)
    runner.enqueue_eager()
    return runner.static_out.clone()


def _check_against_oracle(head, prefix, base, prior, alphas, betas, act, ids, scores, gru_bias, rank_bias):
    gru = head.prefix_gru
    dev_ids = ids.cpu().numpy()
    rid, rsc, rsec = oracle.rollout(
        prefix.numpy().reshape(-1), f(base), embed=f(head.embed_tokens.weight), W_ih=f(gru.weight_ih_l0),
        b_ih=f(gru.bias_ih_l0) if gru_bias else None, W_hh=f(gru.weight_hh_l0),
        b_hh=f(gru.bias_hh_l0) if gru_bias else None, A=f(head.rank_proj.weight),
        rank_bias=f(head.rank_proj.bias) if rank_bias else None, act=act, B=f(head.low_rank_lm_head.weight),
        prior=f(prior.to(torch.bfloat16)) if prior is not None else None, alphas=alphas, betas=betas,
        forced_ids=dev_ids)
    res = oracle.check_parity(dev_ids.reshape(-1), f(scores).reshape(-1), rid.reshape(-1), rsc.reshape(-1),
                              rsec.reshape(-1))
    assert res["id_mismatch_pinned"] == 0, res
    assert res["max_score_err"] < 2e-2, res
    return res


@pytest.mark.parametrize("nb,steps,G,r,V,bdt,with_prior,act,rank_bias,gru_bias", CASES)
def test_resident_rollout_against_oracle(pkg, dev, nb, steps, G, r, V, bdt, with_prior, act, rank_bias, gru_bias):
    print(f"case resident rollout nb={nb} steps={steps} G={G} r={r} V={V} base={bdt} prior={with_prior} "
          f"act={act}", flush=True)
    E = 64
    head = _Head(V, E, G, r, act, rank_bias, seed=90 + V % 97, std=0.02 if G >= 1024 else 0.05,
                 gru_bias=gru_bias).to(dev)
    g = torch.Generator().manual_seed(91 + nb)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0) if with_prior else None
    alphas = [0.8 + 0.05 * i for i in range(steps)]
    betas = [0.1 * (i % 3) for i in range(steps)] if with_prior else [0.0] * steps
    prefix = torch.randint(0, V, (nb, 1), generator=g)
    base = (torch.randn(nb, steps, V, generator=g) * 0.5).to(bdt)
    ids, scores, ids2, scores2 = _rollout(pkg, dev, head, nb, steps, V, prior, alphas, betas, prefix, base, True)
    assert torch.equal(ids, ids2) and torch.equal(scores, scores2), "replays differ"
    assert bool((ids >= 0).all()), "the one-launch rollout gave up"
    _check_against_oracle(head, prefix, base, prior, alphas, betas, act, ids, scores, gru_bias, rank_bias)
    # the per-step launches on the same inputs pass the same check
    pids, pscores, _, _ = _rollout(pkg, dev, head, nb, steps, V, prior, alphas, betas, prefix, base, False)
    _check_against_oracle(head, prefix, base, prior, alphas, betas, act, pids, pscores, gru_bias, rank_bias)


def _largest_resident_vocab(cus):
    """The largest vocabulary the one-launch rollout takes on `cus` CUs (r = 256): its 16
    rank workgroups hold 8 waves x 4 tiles of 16 vocabulary rows in registers, every other
    workgroup those and 6 more tiles in LDS."""
    return (16 * 32 + (cus - 16) * 38) * 16


def test_resident_rollout_at_the_largest_vocabulary(pkg, dev):
    """Every workgroup holding all the tiles it can, the last one ragged (V % 16 = 7)."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    V = _largest_resident_vocab(cus) - 9
    test_resident_rollout_against_oracle(pkg, dev, 2, 4, 1024, 256, V, torch.bfloat16, True, "silu", False, False)


def test_resident_rollout_gives_up_cleanly_and_recovers(pkg, dev):
    """With the waits' re-read limit at zero the launch cannot finish: it writes -1
    ids and still ends; the next launch (limit restored) on the same workspace
    matches the oracle -- the control area was left clean."""
    nb, steps, G, r, V = 4, 4, 1024, 256, 30011
    print(f"case resident rollout give-up nb={nb} steps={steps} G={G} V={V}", flush=True)
    head = _Head(V, 64, G, r, "silu", False, seed=5, std=0.02).to(dev)
    g = torch.Generator().manual_seed(6)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0)
    alphas, betas = [1.0] * steps, [0.1] * steps
    prefix = torch.randint(0, V, (nb, 1), generator=g)
    base = (torch.randn(nb, steps, V, generator=g) * 0.5).to(torch.bfloat16)
    lib = pkg._lib.load()
    runner = pkg.DeLSGraphRunner(local_head=head, batch_size=nb, steps=steps, vocab_size=V, alpha_values=alphas,
                                 beta_values=betas, baseline_logits=prior, device=dev)
    prev = lib.dels_debug_set_resident_spin_limit(0)
    try:
        # the graph holds the launch's arguments: run the rollout eagerly with the limit at zero
        bad = _eager(runner, prefix.to(dev), base.to(dev))
        torch.cuda.synchronize()
    finally:
        lib.dels_debug_set_resident_spin_limit(prev)
    assert bool((bad == -1).any()), bad
    ids = _eager(runner, prefix.to(dev), base.to(dev))
    scores = runner.static_scores.clone()
    torch.cuda.synchronize()
    assert bool((ids >= 0).all())
    _check_against_oracle(head, prefix, base, prior, alphas, betas, "silu", ids, scores, False, False)
    runner.close()


@pytest.mark.parametrize("resident", [True, False])
def test_strided_prefix_ids_and_outputs(pkg, dev, resident):
    """Prefix ids read from a column of a wider tensor (ld_prefix) and ids/scores written
    into columns of wider tensors (ld_out), as the draft block writes its rollout into its
    own output: the same values as the contiguous rollout, nothing written beside them."""
    import ctypes
    nb, steps, G, r, V = 4, 5, 1024, 256, 30011
    print(f"case strided rollout nb={nb} steps={steps} resident={resident}", flush=True)
    head = _Head(V, 64, G, r, "silu", False, seed=21, std=0.02).to(dev)
    g = torch.Generator().manual_seed(22)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0)
    alphas, betas = [0.9] * steps, [0.2] * steps
    prefix = torch.randint(0, V, (nb, 1), generator=g)
    base = (torch.randn(nb, steps, V, generator=g) * 0.5).to(torch.bfloat16)
    lib = pkg._lib.load()
    prev = lib.dels_debug_set_rollout_resident(1 if resident else 0)
    try:
        runner = pkg.DeLSGraphRunner(local_head=head, batch_size=nb, steps=steps, vocab_size=V, alpha_values=alphas,
                                     beta_values=betas, baseline_logits=prior, device=dev)
        want = runner(prefix.to(dev), base.to(dev)).clone()
        want_sc = runner.static_scores.clone()
        big_prefix = torch.full((nb, 3), -5, dtype=torch.int64, device=dev)
        big_prefix[:, 1] = prefix[:, 0].to(dev)
        big_out = torch.full((nb, steps + 3), -7, dtype=torch.int64, device=dev)
        big_sc = torch.full((nb, steps + 3), -7.0, dtype=torch.float32, device=dev)
        p = runner._rollout_params(runner.static_base_logits, steps * V, big_prefix[:, 1], big_out[:, 2:2 + steps],
                                   big_sc[:, 2:2 + steps], runner._ws)
        assert p.ld_prefix == 3 and p.ld_out == steps + 3
        pkg._lib.check(lib.dels_rollout_enqueue(ctypes.byref(p), torch.cuda.current_stream(dev).cuda_stream),
                       "dels_rollout_enqueue")
        torch.cuda.synchronize()
    finally:
        lib.dels_debug_set_rollout_resident(prev)
    assert torch.equal(big_out[:, 2:2 + steps], want) and torch.equal(big_sc[:, 2:2 + steps], want_sc)
    assert bool((big_out[:, :2] == -7).all()) and bool((big_out[:, 2 + steps:] == -7).all())
    assert bool((big_sc[:, :2] == -7.0).all()) and bool((big_sc[:, 2 + steps:] == -7.0).all())
    runner.close()

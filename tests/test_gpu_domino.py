"""GPU tests of the Domino correction step and runner (code/kernel/domino.py) against the oracle."""

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from oracle import domino as DO

pytestmark = pytest.mark.gpu


def _f(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("M,E,V,bias_dt,base_dt", [
    (1, 1024, 151936, None, torch.bfloat16),
    (16, 512, 151936, torch.bfloat16, torch.float32),
    (5, 96, 1001, torch.float32, torch.bfloat16),
    (37, 2048, 4099, None, torch.float16),
    (20, 64, 33, torch.bfloat16, torch.bfloat16),
])
def test_domino_step_matches_oracle(pkg, dev, M, E, V, bias_dt, base_dt):
    g = torch.Generator().manual_seed(M * 7 + E)
    z = torch.randn(M, E, generator=g).to(torch.bfloat16)
    s = torch.randn(M, E, generator=g).to(torch.bfloat16)
    fc2 = (torch.randn(V, E, generator=g) * 0.02).to(torch.bfloat16)
    base = (torch.randn(M, V, generator=g) * 3).to(base_dt)
    bias = torch.randn(V, generator=g).to(bias_dt) if bias_dt is not None else None
    alpha = 0.7
    ids, score = pkg.domino_argmax(z.to(dev), s.to(dev), pkg.pack_operand(fc2.to(dev)), base.to(dev), alpha,
                                   bias.to(dev) if bias is not None else None)
    torch.cuda.synchronize()
    rid, rbest, rsec = DO.domino_step(_f(z), _f(s), _f(fc2), None if bias is None else _f(bias), _f(base), alpha)
    res = oracle.check_parity(ids.cpu().numpy(), score.cpu().numpy(), rid, rbest, rsec, score_atol=1e-4)
    assert res["id_mismatch_pinned"] == 0 and res["score_bad"] == 0, res


@pytest.mark.parametrize("middle,M,E,V", [(m, 8, 512, 30011) for m in DO.MIDDLES if m != "silu"] +
                         [("gelu", 16, 1024, 151936)])
def test_domino_step_middle_layers_match_oracle(pkg, dev, middle, M, E, V):
    """The fused step with each middle layer of the correction MLP that the reference runs as
    its unfused step (code/kernel/domino.py:404-431), against the oracle's fp32 formula."""
    print(f"case domino step middle={middle} M={M} E={E} V={V}", flush=True)
    g = torch.Generator().manual_seed(M * 5 + E + len(middle))
    z = torch.randn(M, E, generator=g).to(torch.bfloat16)
    s = torch.randn(M, E, generator=g).to(torch.bfloat16)
    fc2 = (torch.randn(V, E, generator=g) * 0.1).to(torch.bfloat16)   # the MLP term outweighs base
    base = (torch.randn(M, V, generator=g) * 3).to(torch.bfloat16)
    bias = torch.randn(V, generator=g).to(torch.bfloat16)
    ids, score = pkg.domino_argmax(z.to(dev), s.to(dev), pkg.pack_operand(fc2.to(dev)), base.to(dev), 0.9,
                                   bias.to(dev), middle=middle)
    torch.cuda.synchronize()
    rid, rbest, rsec = DO.domino_step(_f(z), _f(s), _f(fc2), _f(bias), _f(base), 0.9, middle=middle)
    res = oracle.check_parity(ids.cpu().numpy(), score.cpu().numpy(), rid, rbest, rsec, score_atol=1e-4)
    assert res["id_mismatch_pinned"] == 0 and res["score_bad"] == 0, res


def test_domino_step_strided_inputs_and_outputs(pkg, dev):
    g = torch.Generator().manual_seed(3)
    M, E, V = 6, 128, 5000
    zz = torch.randn(M, 3, E, generator=g).to(torch.bfloat16)      # z[:, 1] of a [M, steps, E] tensor
    s = torch.randn(M, E, generator=g).to(torch.bfloat16)
    fc2 = (torch.randn(V, E, generator=g) * 0.05).to(torch.bfloat16)
    base3 = (torch.randn(M, 4, V, generator=g) * 3).to(torch.bfloat16)
    out = torch.full((M, 3), -1, dtype=torch.int64, device=dev)
    sc = torch.zeros(M, 3, dtype=torch.float32, device=dev)
    zd, bd = zz.to(dev), base3.to(dev)
    pkg.domino_argmax(zd[:, 1], s.to(dev), fc2.to(dev), bd[:, 2], 1.3, out_ids=out[:, 1], out_score=sc[:, 1])
    torch.cuda.synchronize()
    rid, rbest, rsec = DO.domino_step(_f(zz[:, 1]), _f(s), _f(fc2), None, _f(base3[:, 2]), 1.3)
    res = oracle.check_parity(out[:, 1].cpu().numpy(), sc[:, 1].cpu().numpy(), rid, rbest, rsec, score_atol=1e-4)
    assert res["id_mismatch_pinned"] == 0 and res["score_bad"] == 0, res
    assert torch.all(out[:, 0] == -1) and torch.all(out[:, 2] == -1)


class _Draft(nn.Module):
    def __init__(self, D, G, E, V, fc1_bias, fc2_bias, g, gru_bias=False, middle=None):
        super().__init__()
        self.embed_proj = nn.Sequential(nn.Linear(D + G, E, bias=fc1_bias), middle if middle is not None else nn.SiLU(),
                                        nn.Linear(E, V, bias=fc2_bias))
        self.prefix_gru = nn.GRU(D, G, num_layers=1, batch_first=True, bias=gru_bias)
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, generator=g) * 0.02)


class _Target(nn.Module):
    def __init__(self, V, D, g):
        super().__init__()
        self.model = nn.Module()
        self.model.embed_tokens = nn.Embedding(V, D)
        with torch.no_grad():
            self.model.embed_tokens.weight.copy_(torch.randn(V, D, generator=g))


@pytest.mark.parametrize("B,S,P,D,G,E,V,fc1_bias,fc2_bias,gru_bias,middle", [
    (2, 6, 2, 256, 128, 256, 3001, True, True, False, "silu"),
    (1, 14, 2, 4096, 1024, 1024, 151936, False, False, False, "silu"),
    (3, 5, 3, 512, 256, 512, 20011, True, False, True, "silu"),     # GRU with b_ih and b_hh
    (2, 6, 2, 256, 128, 256, 3001, True, True, False, "gelu"),      # middles the reference runs unfused
    (3, 5, 2, 512, 256, 512, 20011, True, False, True, "gelu_tanh"),
    (2, 4, 2, 256, 128, 256, 3001, False, True, False, "relu"),
])
def test_runner_rollout_teacher_forced(pkg, dev, B, S, P, D, G, E, V, fc1_bias, fc2_bias, gru_bias, middle):
    """The hipGraph rollout against the oracle's, fed the device's own ids (each step is then
    checked on its own history): ids under the margin rule, scores within 1e-3."""
    print(f"case domino rollout B={B} S={S} P={P} D={D} G={G} E={E} V={V} gru_bias={gru_bias} middle={middle}",
          flush=True)
    g = torch.Generator().manual_seed(11 + V)
    module = {"silu": nn.SiLU(), "gelu": nn.GELU(), "gelu_tanh": nn.GELU(approximate="tanh"), "relu": nn.ReLU()}
    draft = _Draft(D, G, E, V, fc1_bias, fc2_bias, g, gru_bias, module[middle]).to(torch.bfloat16)
    target = _Target(V, D, g).to(torch.bfloat16)
    runner = pkg.DraftCorrectionGraphRunner(draft_model=draft.to(dev), target_model=target.to(dev), batch_size=B,
                                            steps=S, hidden_dim=D, gru_hidden_dim=G, vocab_size=V,
                                            prefix_token_count=P, device=dev, guidance_alpha=0.8)
    assert runner._can_triton_fuse
    prefix = torch.randint(0, V, (B, P), generator=g)
    hiddens = torch.randn(B, S, D, generator=g).to(torch.bfloat16)
    base = (torch.randn(B, S, V, generator=g) * 3).to(torch.bfloat16)
    out = runner(prefix.to(dev), hiddens.to(dev), base.to(dev), 0.8)
    torch.cuda.synchronize()
    assert out.shape == (B, S) and out.dtype == torch.int64
    ids = out.cpu().numpy()
    W1 = _f(draft.embed_proj[0].weight)
    ref_ids, ref_sc, ref_sec = DO.domino_rollout(
        prefix.numpy(), _f(hiddens), _f(base), W_hh=_f(draft.prefix_gru.weight_hh_l0),
        b_hh=_f(draft.prefix_gru.bias_hh_l0) if gru_bias else None,
        b_ih=_f(draft.prefix_gru.bias_ih_l0) if gru_bias else None,
        w_z=W1[:, :D], fc1_bias=None if not fc1_bias else _f(draft.embed_proj[0].bias), w_s=W1[:, D:],
        fc2=_f(draft.embed_proj[2].weight), fc2_bias=None if not fc2_bias else _f(draft.embed_proj[2].bias),
        alpha=0.8, embed=_f(target.model.embed_tokens.weight), W_ih=_f(draft.prefix_gru.weight_ih_l0),
        forced_ids=ids, middle=middle)
    scores = runner.static_scores.cpu().numpy()
    res = oracle.check_parity(ids.reshape(-1), scores.reshape(-1), ref_ids.reshape(-1), ref_sc.reshape(-1),
                              ref_sec.reshape(-1), score_atol=1e-3)
    assert res["id_mismatch_pinned"] == 0 and res["score_bad"] == 0, res
    # a replay equals the same rollout launched kernel by kernel; new inputs give new ids
    runner.enqueue_eager()
    torch.cuda.synchronize()
    assert np.array_equal(runner.static_out.cpu().numpy(), ids)
    with pytest.raises(ValueError, match="fixed domino guidance alpha"):
        runner(prefix.to(dev), hiddens.to(dev), base.to(dev), 0.5)
    base2 = (torch.randn(B, S, V, generator=g) * 3).to(torch.bfloat16)
    out2 = runner(prefix.to(dev), hiddens.to(dev), base2.to(dev))
    assert not torch.equal(out2, out)
    runner.close()

"""GPU parity of the Markov DeLS path (code/kernel/markov_dels.py): the gathered-rank
argmax (dels_gather_argmax) and MarkovDeLSGraphRunner, against the oracle."""

import numpy as np
import pytest
import torch

import oracle
from test_gpu_parity import assert_parity, f

pytestmark = pytest.mark.gpu


class _MarkovHead(torch.nn.Module):
    """The attributes MarkovDeLSGraphRunner reads (as MarkovDeLSLocalHead holds them)."""

    def __init__(self, E, W):
        super().__init__()
        self.embedding_weight = torch.nn.Parameter(E, requires_grad=False)
        self.lm_head_weight = torch.nn.Parameter(W, requires_grad=False)
        self.vocab_size = int(W.shape[0])
        self.rank = int(W.shape[1])


@pytest.mark.parametrize("M,r,V,packed,bdt", [(8, 256, 151936, False, torch.bfloat16),
                                              (8, 256, 151936, True, torch.float32),
                                              (80, 256, 30011, True, torch.bfloat16),   # MFMA-tiled path
                                              (5, 96, 4099, False, torch.float16)])
def test_gather_argmax(pkg, dev, M, r, V, packed, bdt):
    print(f"case gather_argmax M={M} r={r} V={V} packed={packed}", flush=True)
    g = torch.Generator().manual_seed(M + r)
    rows = 777
    E = torch.randn(rows, r, generator=g).to(torch.bfloat16)
    W = (torch.randn(V, r, generator=g) * 0.05).to(torch.bfloat16)
    base = (torch.randn(M, V, generator=g) * 3).to(bdt)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0).to(bdt)
    alpha = torch.rand(M, generator=g) * 0.6
    beta = torch.rand(M, generator=g) * 0.6
    beta[1] = 0.0
    tok_full = torch.randint(0, rows, (M, 3), generator=g)
    tok_full[0, 1] = -5                       # out of the table: clamped to row 0
    tok_full[2, 1] = rows + 3                 # clamped to the last row
    tok = tok_full[:, 1]                      # a strided column of token ids
    Wd = W.to(dev)
    ids, score = pkg.gather_argmax(tok_full.to(dev)[:, 1], E.to(dev), pkg.pack_operand(Wd) if packed else Wd,
                                   base.to(dev), prior.to(dev), alpha.to(dev), beta.to(dev))
    torch.cuda.synchronize()
    rank = f(E)[np.clip(tok.numpy(), 0, rows - 1)]
    assert_parity(ids, score, rank, f(W), f(base), f(prior), f(alpha), f(beta))


def test_markov_runner_follows_the_chain(pkg, dev):
    """The oracle's closed-form chain (orthonormal E, B[pi(t)] = 10 E[t]): the device
    rollout must visit pi^(s+1)(prev) exactly."""
    print("case markov runner chain", flush=True)
    rng = np.random.default_rng(4)
    V, r, nb, steps = 60, 64, 4, 9
    Q, _ = np.linalg.qr(rng.standard_normal((r, r)))
    E = Q[:V].astype(np.float32)
    pi = rng.permutation(V)
    W = np.zeros((V, r), np.float32)
    W[pi] = 10 * E
    head = _MarkovHead(torch.from_numpy(E).bfloat16(), torch.from_numpy(W).bfloat16()).to(dev)
    runner = pkg.MarkovDeLSGraphRunner(local_head=head, batch_size=nb, steps=steps, vocab_size=V,
                                       alpha_values=[1.0] * steps, beta_values=[0.0] * steps, baseline_logits=None,
                                       device=dev)
    prev = torch.tensor([[0], [7], [59], [31]])
    base = torch.from_numpy((rng.standard_normal((nb, steps, V)) * 0.1).astype(np.float32)).bfloat16()
    out = runner(prev.to(dev), base.to(dev)).cpu().numpy()
    want = np.zeros((nb, steps), np.int64)
    t = prev.numpy().reshape(-1)
    for s in range(steps):
        t = pi[t]
        want[:, s] = t
    np.testing.assert_array_equal(out, want)
    runner.close()


@pytest.mark.parametrize("nb,steps,V,r,head_dtype", [(8, 14, 151936, 256, torch.bfloat16),
                                                     (3, 5, 20011, 128, torch.float32)])
def test_markov_runner_rollout(pkg, dev, nb, steps, V, r, head_dtype):
    print(f"case markov runner nb={nb} steps={steps} V={V} r={r}", flush=True)
    g = torch.Generator().manual_seed(V + r)
    E = (torch.randn(V, r, generator=g) * 0.5).to(head_dtype)
    W = (torch.randn(V, r, generator=g) * 0.05).to(head_dtype)
    head = _MarkovHead(E, W).to(dev)
    prior = pkg.synth.zipf_log_prior(V).float()
    ab = torch.rand(2, steps, generator=g) * 0.6
    alphas, betas = ab[0].tolist(), ab[1].tolist()
    betas[2] = 0.0
    runner = pkg.MarkovDeLSGraphRunner(local_head=head, batch_size=nb, steps=steps, vocab_size=V,
                                       alpha_values=alphas, beta_values=betas, baseline_logits=prior, device=dev)
    assert runner._can_triton_fuse and runner.rank == r
    prev = torch.randint(0, V, (nb, 1), generator=g)
    base = (torch.randn(nb, steps, V, generator=g) * 3).to(head_dtype)
    out = runner(prev.to(dev), base.to(dev))
    scores = runner.static_scores.clone()
    out2 = runner(prev.to(dev), base.to(dev))
    runner.enqueue_eager()
    torch.cuda.synchronize()
    torch.testing.assert_close(out2, out, rtol=0, atol=0)
    torch.testing.assert_close(runner.static_out, out, rtol=0, atol=0)
    dev_ids = out.cpu().numpy()
    bf = torch.bfloat16
    rid, rsc, rsec = oracle.markov_rollout(prev.numpy().reshape(-1), f(base.to(head_dtype)), E=f(E.to(bf)),
                                           B=f(W.to(bf)), prior=f(prior.to(head_dtype)),
                                           alphas=np.array(alphas, np.float32), betas=np.array(betas, np.float32),
                                           forced_ids=dev_ids)
    res = oracle.check_parity(dev_ids.reshape(-1), f(scores).reshape(-1), rid.reshape(-1), rsc.reshape(-1),
                              rsec.reshape(-1))
    assert res["id_mismatch_pinned"] == 0 and res["score_bad"] == 0 and res["pinned"] >= 0.9 * res["rows"], res
    runner.close()

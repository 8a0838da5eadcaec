"""GPU tests of the plain row argmax (sample() at temperature 0) and of the whole
draft block as one graph (target LM head GEMM, first-position argmax, rollout).

The LM head is either the library GEMM (hipBLASLt through torch.mm) followed
by the row argmax, or the hand-written dels_lm_head with the first-position
argmax fused (position-0 logits are never stored); its bf16 output is checked
against a float32 product within bf16 rounding, the first ids against
torch.argmax of the same LM head's values (for the fused head a launch that
stores every row), and the rollout on the device's own base logits
(teacher-forced on the device's ids, as for DeLSGraphRunner).
"""

import numpy as np
import pytest
import torch

import oracle
from test_gpu_parity import _Head

pytestmark = pytest.mark.gpu


def f(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("M,V,dtype,stride_pad", [(8, 151936, torch.bfloat16, 0), (5, 4099, torch.float32, 7),
                                                  (33, 20011, torch.float16, 0), (1, 1, torch.float32, 0),
                                                  # 16-byte pieces: strided rows, and chunks of several rounds
                                                  (6, 30000, torch.float32, 4), (7, 65536, torch.float16, 8),
                                                  (5, 300000, torch.float32, 0)])
def test_argmax_rows(pkg, dev, M, V, dtype, stride_pad):
    """Ids as torch.argmax on the CPU (code/dflash.py:31-33): lowest index of the
    maximum, the first NaN of a row wins, an all -inf row gives 0."""
    print(f"case argmax_rows M={M} V={V} {dtype}", flush=True)
    g = torch.Generator().manual_seed(M + V)
    full = (torch.randn(M, V + stride_pad, generator=g) * 3).to(dtype)
    x = full[:, :V]
    if M > 4 and V > 10:
        x[0, 3] = x[0, V - 2] = 100.0                   # equal maxima: the lower index wins
        x[1].fill_(-float("inf"))                        # all -inf -> 0
        x[2, 7] = x[2, V - 1] = float("nan")             # the first NaN wins over the maximum
        x[2, 1] = 1000.0
        x[3, V - 1] = float("nan")                       # a NaN in the vocabulary tail
        x[4, 0] = -float("nan")                          # a NaN with the sign bit set counts the same
    ids, score = pkg.argmax_rows(x.to(dev))
    torch.cuda.synchronize()
    ref = torch.argmax(x, dim=-1).numpy()
    np.testing.assert_array_equal(ids.cpu().numpy(), ref)
    want = f(x)[np.arange(M), ref]
    got = score.cpu().numpy()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(got[~np.isnan(want)], want[~np.isnan(want)])


@pytest.mark.parametrize("lm_head", ["library", "fused"])
@pytest.mark.parametrize("B,k,d,V,E,G,r,act,with_prior", [(3, 6, 256, 5003, 32, 64, 64, "silu", True),
                                                          (8, 15, 512, 30000, 64, 128, 256, "identity", False)])
def test_draft_step(pkg, dev, B, k, d, V, E, G, r, act, with_prior, lm_head):
    print(f"case draft_step B={B} k={k} d={d} V={V} G={G} r={r} lm_head={lm_head}", flush=True)
    head = _Head(V, E, G, r, act, False, seed=B + V, std=0.2).to(dev)
    g = torch.Generator().manual_seed(7)
    W = (torch.randn(V, d, generator=g) * 0.05).bfloat16()
    prior = torch.log_softmax(torch.randn(V, generator=g), 0) if with_prior else None
    steps = k - 1
    alphas = [0.1 + 0.05 * i for i in range(steps)]
    betas = [0.3 if with_prior else 0.0] * steps
    step = pkg.DeLSDraftStep(local_head=head, lm_head_weight=W.to(dev), batch_size=B, k_draft=k, vocab_size=V,
                             alpha_values=alphas, beta_values=betas, baseline_logits=prior, device=dev,
                             lm_head=lm_head)
    hid = (torch.randn(B, k, d, generator=g)).bfloat16()
    out = step(hid.to(dev))
    torch.cuda.synchronize()
    base = step.static_base.clone()
    # replays and the eager path give the same ids
    out2 = step(hid.to(dev))
    step.enqueue_eager()
    torch.cuda.synchronize()
    torch.testing.assert_close(out2, out, rtol=0, atol=0)
    torch.testing.assert_close(step.static_out, out, rtol=0, atol=0)
    assert out.shape == (B, k) and out.dtype == torch.int64
    # the GEMM is the LM head: base = bf16(hidden . W^T) (positions 1.. stored)
    ref_base = (f(hid).reshape(B * k, d) @ f(W).T).reshape(B, k, V)
    np.testing.assert_allclose(f(base)[:, 1:], ref_base[:, 1:], rtol=2e-2, atol=2e-2)
    # first position: argmax of the LM head's own bf16 logits of position 0 (the fused
    # head does not store them: a second launch of the same kernel stores every row)
    if lm_head == "fused":
        full, _, _ = pkg.lm_head(hid.to(dev).reshape(B * k, d), step._w_p)
        torch.cuda.synchronize()
        full = full.reshape(B, k, V)
        torch.testing.assert_close(full[:, 1:], base[:, 1:], rtol=0, atol=0)
    else:
        full = base
    np.testing.assert_array_equal(out[:, 0].cpu().numpy(), torch.argmax(full[:, 0, :].cpu(), dim=-1).numpy())
    bn = f(base)
    # the rollout on base[:, 1:], teacher-forced on the device's own ids
    prior_np = f(prior.to(torch.bfloat16)) if with_prior else None
    dev_ids = out[:, 1:].cpu().numpy()
    rid, rsc, rsec = oracle.rollout(
        out[:, 0].cpu().numpy(), bn[:, 1:, :], embed=f(head.embed_tokens.weight), W_ih=f(head.prefix_gru.weight_ih_l0),
        W_hh=f(head.prefix_gru.weight_hh_l0), b_hh=None, A=f(head.rank_proj.weight), rank_bias=None, act=act,
        B=f(head.low_rank_lm_head.weight), prior=prior_np, alphas=alphas, betas=betas, forced_ids=dev_ids)
    res = oracle.check_parity(dev_ids.reshape(-1), f(step.static_rest_scores).reshape(-1), rid.reshape(-1),
                              rsc.reshape(-1), rsec.reshape(-1))
    assert res["id_mismatch_pinned"] == 0, res
    assert res["max_score_err"] < 2e-2, res
    step.close()


@pytest.mark.parametrize("lm_head", ["library", "fused"])
def test_draft_step_full_size(pkg, dev, lm_head):
    """The whole draft block at the size the bench times: batch 8, block 16 (k_draft 15,
    14 DeLS steps), W [151936, 4096], local head E = G = 1024, r = 256, silu, bf16 base,
    the Zipf prior and per-step alpha/beta (synth.draft_block_workload).  The LM-head
    GEMM against a float32 CPU product on a sample of rows, the first position against
    torch.argmax, and the 14-step rollout teacher-forced against the oracle."""
    print(f"case draft_step full size B=8 k=15 d=4096 V=151936 G=1024 r=256 lm_head={lm_head}", flush=True)
    wl = pkg.synth.draft_block_workload(dev)
    B, k, d, V = wl.batch, wl.k_draft, wl.d, wl.V
    head = wl.head
    step = pkg.DeLSDraftStep(local_head=head, lm_head_weight=wl.W, batch_size=B, k_draft=k, vocab_size=V,
                             alpha_values=wl.alphas, beta_values=wl.betas, baseline_logits=wl.prior, device=dev,
                             lm_head=lm_head)
    hid = wl.hiddens(1)[0]
    out = step(hid)
    torch.cuda.synchronize()
    base = step.static_base.clone()
    out2 = step(hid)
    torch.cuda.synchronize()
    torch.testing.assert_close(out2, out, rtol=0, atol=0)
    # LM head on a row sample (rows (b, position) of the [B*k, V] product; position 0
    # rows are argmaxed in the kernel, not stored)
    rows = [1, 17, 44, 77, 119]
    hid_rows = f(hid).reshape(B * k, d)[rows]
    W_np = f(wl.W)
    ref_rows = hid_rows @ W_np.T
    got_rows = f(base).reshape(B * k, V)[rows]
    np.testing.assert_allclose(got_rows, ref_rows, rtol=1e-2, atol=2e-3)      # bf16 output rounding
    del W_np
    # first draft position: torch.argmax of the LM head's own bf16 logits of position 0
    if lm_head == "fused":
        full, _, _ = pkg.lm_head(hid.reshape(B * k, d), step._w_p)
        torch.cuda.synchronize()
        full = full.reshape(B, k, V)
        torch.testing.assert_close(full[:, 1:], base[:, 1:], rtol=0, atol=0)
    else:
        full = base
    np.testing.assert_array_equal(out[:, 0].cpu().numpy(), torch.argmax(full[:, 0, :].cpu(), dim=-1).numpy())
    del full
    # the rollout over base[:, 1:], teacher-forced on the device's own ids
    bn = f(base)
    dev_ids = out[:, 1:].cpu().numpy()
    prior_np = f(wl.prior.to(torch.bfloat16))
    rid, rsc, rsec = oracle.rollout(
        out[:, 0].cpu().numpy(), bn[:, 1:, :], embed=f(head.embed_tokens.weight),
        W_ih=f(head.prefix_gru.weight_ih_l0), W_hh=f(head.prefix_gru.weight_hh_l0), b_hh=None,
        A=f(head.rank_proj.weight), rank_bias=None, act=head.rank_activation, B=f(head.low_rank_lm_head.weight),
        prior=prior_np, alphas=wl.alphas, betas=wl.betas, forced_ids=dev_ids)
    res = oracle.check_parity(dev_ids.reshape(-1), f(step.static_rest_scores).reshape(-1), rid.reshape(-1),
                              rsc.reshape(-1), rsec.reshape(-1))
    assert res["rows"] == B * (k - 1) and res["pinned"] >= 0.9 * res["rows"], res
    assert res["id_mismatch_pinned"] == 0, res
    assert res["score_bad"] == 0, res
    step.close()



def test_default_lm_head_is_the_hand_written_one_where_it_applies(pkg, dev):
    """lm_head="auto" (the default) takes the hand-written LM head when the hidden size is
    a multiple of 256, the library GEMM otherwise; both give the same first ids here."""
    V = 5003
    head = _Head(V, 32, 64, 64, "silu", False, seed=5, std=0.2).to(dev)
    g = torch.Generator().manual_seed(11)
    firsts = []
    for d, fused in ((256, True), (200, False)):
        print(f"case draft_step default lm_head d={d}", flush=True)
        W = (torch.randn(V, d, generator=g) * 0.05).bfloat16()
        st = pkg.DeLSDraftStep(local_head=head, lm_head_weight=W.to(dev), batch_size=2, k_draft=3, vocab_size=V,
                               alpha_values=[0.1, 0.2], beta_values=[0.0, 0.0], baseline_logits=None, device=dev)
        assert st._fused_head is fused
        hid = torch.randn(2, 3, d, generator=g).bfloat16()
        out = st(hid.to(dev))
        torch.cuda.synchronize()
        ref = (hid.float().reshape(6, d) @ W.float().T).reshape(2, 3, V)[:, 0]
        firsts.append((out[:, 0].cpu(), ref))
        st.close()
    for got, ref in firsts:
        top2 = torch.topk(ref, 2, dim=-1).values
        pinned = (top2[:, 0] - top2[:, 1]) > 0.05 * top2[:, 0].abs()
        assert torch.equal(got[pinned], torch.argmax(ref, dim=-1)[pinned])

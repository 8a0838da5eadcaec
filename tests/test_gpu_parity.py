"""GPU parity: the gfx950 kernels (through the C ABI) against the CPU oracle.

Parity rule: ids bit-exact wherever the oracle's top-2 margin exceeds 1e-3
relative; elsewhere the device's pick must be a near-maximum under the oracle;
the winning score within 1e-2 absolute.  bf16 outputs (rank, GRU state) may
differ from the oracle by one bf16 ulp only where fp32 accumulation order
straddles a rounding boundary.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def f(t):
    return t.detach().float().cpu().numpy()


def from_bits(b, dev):
    return torch.from_numpy(np.ascontiguousarray(b).astype(np.int16)).view(torch.bfloat16).to(dev)


def assert_parity(ids, score, rank_np, B_np, base_np, prior_np, alpha, beta, ref=None):
    ids = ids.cpu().numpy()
    score = score.cpu().numpy()
    if ref is None:
        ref = oracle.fused_argmax(rank_np, B_np, base_np, prior_np, alpha, beta)
    rid, rsc, rsec = ref
    pick = oracle.score_at(rank_np, B_np, base_np, prior_np, alpha, beta, np.clip(ids, 0, B_np.shape[0] - 1))
    res = oracle.check_parity(ids, score, rid, rsc, rsec, pick)
    bad = sorted(set(res["bad_rows"]) | set(res["score_bad_rows"]))[:8]
    detail = [(int(m), int(ids[m]), int(rid[m]), float(score[m]), float(rsc[m]), float(pick[m]), float(rsec[m]))
              for m in bad]   # (row, dev id, ref id, dev score, ref score, ref score at dev id, ref runner-up)
    assert res["id_mismatch_pinned"] == 0, (res, detail)
    assert res["score_bad"] == 0, (res, detail)
    assert res["unpinned_far_pick"] == 0, (res, detail)
    return res


def bf16_ulps(a, b):
    """Distance in bf16 ulps between two arrays of bf16-representable fp32 values."""
    ia = oracle.f32_to_bf16_bits(a).astype(np.int32)
    ib = oracle.f32_to_bf16_bits(b).astype(np.int32)
    # map sign-magnitude to a monotone integer line
    ia = np.where(ia & 0x8000, -(ia & 0x7FFF), ia)
    ib = np.where(ib & 0x8000, -(ib & 0x7FFF), ib)
    return np.abs(ia - ib)


# ------------------------------------------------------------------ fused argmax

ARGMAX_CASES = [
    # M, r, V, base dtype, prior dtype (None: no prior), per-row alpha/beta
    (1, 64, 1000, torch.float32, torch.float32, True),
    (4, 8, 17, torch.bfloat16, torch.bfloat16, True),
    (3, 96, 4099, torch.bfloat16, None, True),
    (16, 256, 151936, torch.float32, torch.float32, False),
    (16, 512, 151936, torch.float32, torch.float32, True),
    (17, 128, 5000, torch.float16, torch.float32, True),
    (40, 512, 20011, torch.bfloat16, torch.bfloat16, True),
]


@pytest.mark.parametrize("M,r,V,bdt,pdt,per_row", ARGMAX_CASES)
def test_fused_argmax_random(pkg, dev, M, r, V, bdt, pdt, per_row):
    print(f"case fused_argmax M={M} r={r} V={V} base={bdt} prior={pdt}", flush=True)
    x = pkg.synth.lowrank_inputs(M, 64, r, V, base_dtype=bdt, prior_dtype=pdt or torch.float32,
                                 per_position=per_row, seed=M * 7 + r)
    rank = (torch.randn(M, r, generator=torch.Generator().manual_seed(M + V)) * 2).to(torch.bfloat16)
    prior = x.prior if pdt is not None else None
    ids, score = pkg.fused_argmax(rank.to(dev), x.B.to(dev), x.base.to(dev),
                                  None if prior is None else prior.to(dev), x.alpha.to(dev), x.beta.to(dev))
    torch.cuda.synchronize()
    assert_parity(ids, score, f(rank), f(x.B), f(x.base), None if prior is None else f(prior),
                  f(x.alpha), f(x.beta))


# Many rows with B packed: the MFMA-tiled kernel (256-row groups, vocabulary
# chunks, per-chunk partials).  Ragged row groups (M % 256), a ragged last
# vocabulary tile (V % 16 = 8), every base dtype, every prior kind and r in
# {128, 256, 512}.
TILED_CASES = [
    # M, r, V, base dtype, prior dtype (None: no prior), per-row alpha/beta
    (64, 128, 4096, torch.float32, torch.float32, True),
    (100, 256, 20008, torch.bfloat16, torch.bfloat16, True),
    (256, 512, 30000, torch.float16, None, True),
    (300, 512, 50008, torch.bfloat16, torch.float32, True),
    (512, 512, 151936, torch.bfloat16, torch.bfloat16, True),
    (512, 512, 151936, torch.float32, torch.bfloat16, True),    # the batched shape with fp32 base logits
    (512, 256, 151936, torch.float32, torch.float16, False),
]


@pytest.mark.parametrize("M,r,V,bdt,pdt,per_row", TILED_CASES)
def test_fused_argmax_tiled_random(pkg, dev, M, r, V, bdt, pdt, per_row):
    print(f"case fused_argmax tiled M={M} r={r} V={V} base={bdt} prior={pdt}", flush=True)
    x = pkg.synth.lowrank_inputs(M, 64, r, V, base_dtype=bdt, prior_dtype=pdt or torch.float32,
                                 per_position=per_row, seed=M * 5 + r)
    rank = (torch.randn(M, r, generator=torch.Generator().manual_seed(M + V)) * 2).to(torch.bfloat16)
    prior = x.prior if pdt is not None else None
    Bp = pkg.pack_operand(x.B.to(dev))
    ids, score = pkg.fused_argmax(rank.to(dev), Bp, x.base.to(dev),
                                  None if prior is None else prior.to(dev), x.alpha.to(dev), x.beta.to(dev))
    torch.cuda.synchronize()
    assert_parity(ids, score, f(rank), f(x.B), f(x.base), None if prior is None else f(prior),
                  f(x.alpha), f(x.beta))
    # same inputs, row-major B: the GEMV kernel must agree on every pinned row
    ids2, score2 = pkg.fused_argmax(rank.to(dev), x.B.to(dev), x.base.to(dev),
                                    None if prior is None else prior.to(dev), x.alpha.to(dev), x.beta.to(dev))
    torch.cuda.synchronize()
    assert_parity(ids2, score2, f(rank), f(x.B), f(x.base), None if prior is None else f(prior),
                  f(x.alpha), f(x.beta))


def test_fused_argmax_tiled_repeat_is_bitwise_stable(pkg, dev):
    """Back-to-back calls of the tiled kernel return bit-identical ids and
    scores (a guard for the cross-wave hand-off of the LDS stage buffers)."""
    M, r, V = 512, 256, 151936
    x = pkg.synth.lowrank_inputs(M, 64, r, V, base_dtype=torch.float32, prior_dtype=torch.float16,
                                 per_position=False, seed=11)
    rank = (torch.randn(M, r, generator=torch.Generator().manual_seed(12)) * 2).to(torch.bfloat16).to(dev)
    Bp = pkg.pack_operand(x.B.to(dev))
    base, prior, al, be = x.base.to(dev), x.prior.to(dev), x.alpha.to(dev), x.beta.to(dev)
    first = None
    for _ in range(12):
        ids, score = pkg.fused_argmax(rank, Bp, base, prior, al, be)
        torch.cuda.synchronize()
        if first is None:
            first = (ids.clone(), score.clone())
        else:
            assert torch.equal(ids, first[0]) and torch.equal(score, first[1])
    assert_parity(first[0], first[1], f(rank), f(x.B), f(x.base), f(x.prior), f(x.alpha), f(x.beta))


def test_fused_argmax_tiled_ties_inf_strided(pkg, dev):
    """Tiled kernel edge cases: ties across vocabulary chunks and row groups go
    to the lowest index, an all -inf row gives id 0, a row with beta = 0 skips
    an infinite prior, and a strided base view (ldbase > V) is read correctly."""
    M, r, V, ld = 320, 128, 12000, 12008
    g = torch.Generator().manual_seed(3)
    rank = torch.zeros(M, r, dtype=torch.bfloat16)
    B = (torch.randn(V, r, generator=g) * 0.02).to(torch.bfloat16)
    big = torch.randn(M, ld, generator=g).float()
    base_full = big.clone()
    base = base_full[:, :V]                   # strided view: ldbase = 12008
    alpha = torch.ones(M)
    beta = torch.zeros(M)
    prior = torch.zeros(V)
    # rank = 0: scores are base - beta * prior exactly
    base[0, 11990] = 50.0
    base[0, 17] = 50.0                        # tie across chunks: 17 wins
    base[1, 5000] = 40.0
    base[1, 5001] = 40.0                      # tie inside a tile
    base[2, :] = -float("inf")                # all -inf: id 0
    base[300, 7] = 60.0                       # second row group
    base[300, 11999] = 60.0
    prior[123] = float("inf")                 # only rows with beta != 0 see it
    beta[5] = 1.0
    base[5, 123] = 1e6                        # row 5: beta = 1 drives index 123 to -inf
    base[6, 123] = 1e6                        # row 6: beta = 0 keeps it
    Bp = pkg.pack_operand(B.to(dev))
    based = base_full.to(dev)[:, :V]
    assert based.stride(0) == ld
    ids, score = pkg.fused_argmax(rank.to(dev), Bp, based, prior.to(dev), alpha.to(dev), beta.to(dev))
    torch.cuda.synchronize()
    ids = ids.cpu().numpy()
    score = score.cpu().numpy()
    assert ids[0] == 17 and score[0] == 50.0
    assert ids[1] == 5000 and score[1] == 40.0
    assert ids[2] == 0 and score[2] == -np.inf
    assert ids[300] == 7 and score[300] == 60.0
    assert ids[5] != 123 and ids[6] == 123
    ref = oracle.fused_argmax(f(rank), f(B), f(base), f(prior), f(alpha), f(beta))
    rows = np.r_[3:5, 7:300, 301:M]
    assert np.array_equal(ids[rows], ref[0][rows])


def test_fused_argmax_strided_base_and_outputs(pkg, dev):
    g = torch.Generator().manual_seed(5)
    nb, steps, V, r = 3, 5, 3001, 64
    base3 = (torch.randn(nb, steps, V, generator=g) * 3).to(torch.bfloat16)
    B = (torch.randn(V, r, generator=g) * 0.05).to(torch.bfloat16)
    rank = torch.randn(nb, r, generator=g).to(torch.bfloat16)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0).to(torch.bfloat16)
    out_ids = torch.full((nb, steps), -1, dtype=torch.int64, device=dev)
    out_sc = torch.zeros(nb, steps, dtype=torch.float32, device=dev)
    base_d = base3.to(dev)
    for s in range(steps):
        pkg.fused_argmax(rank.to(dev), B.to(dev), base_d[:, s, :], prior.to(dev), 0.3, 0.2,
                         out_ids=out_ids[:, s], out_score=out_sc[:, s])
    torch.cuda.synchronize()
    for s in range(steps):
        assert_parity(out_ids[:, s], out_sc[:, s], f(rank), f(B), f(base3[:, s, :]), f(prior), 0.3, 0.2)


def test_fused_argmax_ties_inf_and_skipped_prior(pkg, dev):
    g = torch.Generator().manual_seed(6)
    M, r, V = 6, 128, 151936
    B = (torch.randn(V, r, generator=g) * 0.02).to(torch.bfloat16)
    rank = torch.randn(M, r, generator=g).to(torch.bfloat16)
    base = torch.randn(M, V, generator=g) * 3
    prior = torch.log_softmax(torch.randn(V, generator=g), 0)
    alpha = torch.full((M,), 0.3)
    beta = torch.full((M,), 0.4)
    planted = [5, 77777, 150000, V - 1]
    B[planted] = 0
    prior[planted] = 0
    base[0, 5] = base[0, 150000] = 100.0      # tie across far-apart workgroups -> 5
    base[1, V - 1] = 100.0                    # last vocabulary entry
    base[2, :] = float("-inf")                # all -inf -> id 0, score -inf
    alpha[2] = 0.0
    base[3, 77777] = base[3, 150000] = 100.0  # tie -> 77777
    prior_inf = prior.clone()
    prior_inf[1234] = float("inf")            # poisons only rows whose beta is used
    beta[4] = 0.0
    ids, score = pkg.fused_argmax(rank.to(dev), B.to(dev), base.to(dev), prior_inf.to(dev), alpha.to(dev),
                                  beta.to(dev))
    ids, score = ids.cpu(), score.cpu()
    assert ids[0].item() == 5 and ids[1].item() == V - 1 and ids[3].item() == 77777
    assert ids[2].item() == 0 and score[2].item() == float("-inf")
    assert score[0].item() == 100.0
    ref = oracle.fused_argmax(f(rank), f(B), f(base), f(prior_inf), f(alpha), f(beta))
    assert ids[4].item() == ref[0][4] and abs(score[4].item() - ref[1][4]) < 1e-2 and np.isfinite(score[4].item())


def test_fused_argmax_repeated_calls_reset_workspace(pkg, dev):
    x = pkg.synth.lowrank_inputs(16, 64, 256, 30000, seed=9)
    rank = torch.randn(16, 256, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).to(dev)
    args = (x.B.to(dev), x.base.to(dev), x.prior.to(dev), x.alpha.to(dev), x.beta.to(dev))
    first = pkg.fused_argmax(rank, *args)
    first = (first[0].clone(), first[1].clone())
    for _ in range(4):
        again = pkg.fused_argmax(rank, *args)
        torch.testing.assert_close(again[0], first[0], rtol=0, atol=0)
        torch.testing.assert_close(again[1], first[1], rtol=0, atol=0)
    # a smaller problem right after a larger one on the same workspace
    small = pkg.fused_argmax(rank[:3], x.B[:100].to(dev), x.base[:3, :100].to(dev), x.prior[:100].to(dev),
                             x.alpha[:3].to(dev), x.beta[:3].to(dev))
    torch.cuda.synchronize()
    assert_parity(small[0], small[1], f(rank[:3]), f(x.B[:100]), f(x.base[:3, :100]), f(x.prior[:100]),
                  f(x.alpha[:3]), f(x.beta[:3]))


def test_fused_argmax_vocab_of_one_and_empty_batch(pkg, dev):
    rank = torch.ones(2, 8, dtype=torch.bfloat16, device=dev)
    B = torch.ones(1, 8, dtype=torch.bfloat16, device=dev)
    base = torch.tensor([[1.0], [-2.0]], device=dev)
    ids, score = pkg.fused_argmax(rank, B, base, None, 0.5, 0.0)
    assert ids.tolist() == [0, 0] and score.tolist() == [5.0, 2.0]
    ids, score = pkg.fused_argmax(rank[:0], B, base[:0], None, 0.5, 0.0)
    assert ids.numel() == 0


@pytest.mark.parametrize("layout", ["rowmajor", "packed"])
def test_shared_workspace_across_entry_points_and_shapes(pkg, dev, layout):
    """Entry points with different workspace layouts interleaved on one stream's workspace.

    With packed weights the draft step is the one-launch decode kernel, whose
    tagged words live in a region of the workspace that no other entry point
    writes: the region is checked unchanged across the other calls."""
    print(f"case shared workspace {layout}", flush=True)
    x = pkg.synth.lowrank_inputs(16, 1024, 128, 20000, seed=21)
    xd = x.to(dev)
    if layout == "packed":
        xd.A, xd.B = pkg.pack_operand(xd.A), pkg.pack_operand(xd.B)
    want = pkg.lowrank_argmax(xd.h, xd.A, xd.B, xd.base, xd.prior, xd.alpha, xd.beta)
    want = (want[0].clone(), want[1].clone())
    ref = oracle.lowrank_argmax(f(x.h), f(x.A), None, x.act, f(x.B), f(x.base), f(x.prior), f(x.alpha),
                                f(x.beta))
    assert_parity(want[0], want[1], ref[0], f(x.B), f(x.base), f(x.prior), f(x.alpha), f(x.beta), ref=ref[1:])
    reserved = slice(65536, 65536 + 544 * 1024)   # the decode step's tagged words
    g = torch.Generator().manual_seed(22)
    big_h = torch.randn(512, 2048, generator=g).to(torch.bfloat16).to(dev)
    big_A = (torch.randn(384, 2048, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    table = torch.randn(50, 3 * 256, generator=g).to(torch.bfloat16).to(dev)
    w_hh = (torch.randn(3 * 256, 256, generator=g) * 0.05).to(torch.bfloat16).to(dev)
    tok = torch.arange(40, dtype=torch.int64, device=dev) % 50
    h40 = torch.randn(40, 256, generator=g).to(torch.bfloat16).to(dev)
    big_B = pkg.pack_operand((torch.randn(3000, 384, generator=g) * 0.02).to(torch.bfloat16).to(dev))
    big_base = torch.randn(512, 3000, generator=g).to(dev)

    def others():
        rk = pkg.rank_proj(big_h, big_A, None, "silu")        # large split-K partial region
        pkg.gru_step(table, tok, h40, w_hh)                   # different tile count
        pkg.fused_argmax(rk, big_B, big_base, None, 0.5, 0.0)  # tiled argmax, M=512

    others()                                                  # grows the stream's workspace to its final size
    for _ in range(2):
        got = pkg.lowrank_argmax(xd.h, xd.A, xd.B, xd.base, xd.prior, xd.alpha, xd.beta)
        ws = pkg.ops.workspace(dev, 0)
        torch.cuda.synchronize()
        before = ws[reserved].clone()
        others()
        torch.cuda.synchronize()
        assert pkg.ops.workspace(dev, 0).data_ptr() == ws.data_ptr()
        assert torch.equal(ws[reserved], before)
        got = pkg.lowrank_argmax(xd.h, xd.A, xd.B, xd.base, xd.prior, xd.alpha, xd.beta)
        torch.testing.assert_close(got[0], want[0], rtol=0, atol=0)
        torch.testing.assert_close(got[1], want[1], rtol=0, atol=0)


# ------------------------------------------------------------------ MFMA-16 packed layout

def _pack_reference(W):
    """The documented block layout, restated with numpy (uint16 bf16 bits)."""
    rows, cols = W.shape
    rb, cb = -(-rows // 16), -(-cols // 32)
    Wp = np.zeros((rb * 16, cb * 32), np.uint16)
    Wp[:rows, :cols] = W
    out = np.zeros((rb, cb, 64, 8), np.uint16)
    for lane in range(64):
        out[:, :, lane, :] = Wp.reshape(rb, 16, cb, 32)[:, lane % 16, :, 8 * (lane // 16):8 * (lane // 16) + 8]
    return out.reshape(-1)


@pytest.mark.parametrize("rows,cols", [(16, 32), (37, 72), (151936, 512), (3 * 1024, 1024), (5, 8)])
def test_pack_operand_layout(pkg, dev, rows, cols):
    g = torch.Generator().manual_seed(rows + cols)
    W = torch.randn(rows, cols + 8, generator=g).to(torch.bfloat16)[:, :cols]   # strided source
    P = pkg.pack_operand(W.to(dev))
    got = P.data.cpu().view(torch.int16).numpy().view(np.uint16)
    want = _pack_reference(W.contiguous().view(torch.int16).numpy().view(np.uint16))
    np.testing.assert_array_equal(got[:want.size], want)


@pytest.mark.parametrize("M,r,V,bdt", [(16, 512, 151936, torch.float32), (5, 96, 4099, torch.bfloat16),
                                       (40, 256, 20011, torch.bfloat16)])
def test_packed_equals_rowmajor(pkg, dev, M, r, V, bdt):
    print(f"case packed vs rowmajor M={M} r={r} V={V}", flush=True)
    x = pkg.synth.lowrank_inputs(M, 1024, r, V, base_dtype=bdt, prior_dtype=bdt, seed=M + r, act="silu")
    xd = x.to(dev)
    Ap, Bp = pkg.pack_operand(xd.A), pkg.pack_operand(xd.B)
    # same rank, B row-major vs packed: the same kernel family and K order -> identical
    rank_row = pkg.rank_proj(xd.h, xd.A, None, "silu").clone()
    fa_row = pkg.fused_argmax(rank_row, xd.B, xd.base, xd.prior, xd.alpha, xd.beta)
    fa_row = (fa_row[0].clone(), fa_row[1].clone())
    fa_pk = pkg.fused_argmax(rank_row, Bp, xd.base, xd.prior, xd.alpha, xd.beta)
    torch.testing.assert_close(fa_pk[0], fa_row[0], rtol=0, atol=0)
    torch.testing.assert_close(fa_pk[1], fa_row[1], rtol=0, atol=0)
    # packed A may run a different rank-projection kernel: equal up to accumulation order
    rank_pk = pkg.rank_proj(xd.h, Ap, None, "silu")
    assert (bf16_ulps(f(rank_pk), f(rank_row)) > 0).mean() < 2e-3
    pk = pkg.lowrank_argmax(xd.h, Ap, Bp, xd.base, xd.prior, xd.alpha, xd.beta, act="silu")
    torch.cuda.synchronize()
    rank = oracle.rank_proj(f(x.h), f(x.A), None, "silu")
    assert_parity(pk[0], pk[1], rank, f(x.B), f(x.base), f(x.prior), f(x.alpha), f(x.beta))
    assert_parity(fa_row[0], fa_row[1], f(rank_row), f(x.B), f(x.base), f(x.prior), f(x.alpha), f(x.beta))


def test_packed_gru_equals_rowmajor(pkg, dev):
    g = torch.Generator().manual_seed(31)
    nb, G, rows = 8, 1024, 100
    table = torch.randn(rows, 3 * G, generator=g).to(torch.bfloat16).to(dev)
    w_hh = (torch.randn(3 * G, G, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    h = torch.randn(nb, G, generator=g).to(torch.bfloat16).to(dev)
    tok = torch.randint(0, rows, (nb,), generator=g).to(dev)
    a = pkg.gru_step(table, tok, h, w_hh).clone()
    b = pkg.gru_step(table, tok, h, pkg.pack_operand(w_hh))
    torch.testing.assert_close(b, a, rtol=0, atol=0)


# ------------------------------------------------------------------ rank projection

@pytest.mark.parametrize("M,d,r,act,bias", [(16, 4096, 512, "identity", False), (16, 2560, 256, "silu", False),
                                            (5, 1024, 64, "silu", True), (40, 512, 136, "identity", True),
                                            (512, 4096, 512, "silu", False), (100, 1000, 136, "identity", True),
                                            (64, 4096, 256, "silu", True)])
def test_rank_proj(pkg, dev, M, d, r, act, bias):
    print(f"case rank_proj M={M} d={d} r={r} act={act} bias={bias}", flush=True)
    g = torch.Generator().manual_seed(M + d + r)
    h = torch.randn(M, d, generator=g).to(torch.bfloat16)
    A = (torch.randn(r, d, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(r, generator=g) * 0.1).to(torch.bfloat16) if bias else None
    got = f(pkg.rank_proj(h.to(dev), A.to(dev), None if b is None else b.to(dev), act))
    ref = oracle.rank_proj(f(h), f(A), None if b is None else f(b), act)
    # one bf16 ulp of the result, plus the fp32 accumulation-order bound on the
    # pre-activation (|error| <= ~1e-6 * sum|h||A| for these K), which matters
    # only for results close to zero
    mag = np.abs(f(h)).astype(np.float64) @ np.abs(f(A)).astype(np.float64).T
    pre = f(h).astype(np.float64) @ f(A).astype(np.float64).T
    # one bf16 ulp of the output, plus one of the pre-activation carried through
    # silu (slope <= 1.1), plus the accumulation-order bound
    ulp = np.abs(ref) * 2.0 ** -7 + (1.1 * np.abs(pre) * 2.0 ** -7 if act == "silu" else 0.0)
    tol = ulp + 2e-6 * mag + 1e-30
    err = np.abs(got - ref)
    bad = err > tol
    if bad.any():
        idx = np.argwhere(bad)[:8]
        detail = [(int(i), int(j), float(got[i, j]), float(ref[i, j]), float(mag[i, j])) for i, j in idx]
        raise AssertionError(f"{int(bad.sum())} rank elements out of tolerance, e.g. (row, col, got, ref, mag) "
                             f"{detail}")
    assert (bf16_ulps(got, ref) > 0).mean() < 2e-3


def test_rank_proj_tiled_packed_equals_rowmajor(pkg, dev):
    """Many rows (the LDS-tiled rank GEMM): the MFMA-16 blocked A gives the same
    rank as row-major A (same kernel, same K order), ragged rows, columns and K."""
    M, d, r = 300, 1000, 200
    g = torch.Generator().manual_seed(21)
    h = torch.randn(M, d, generator=g).to(torch.bfloat16).to(dev)
    A = (torch.randn(r, d, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    b = (torch.randn(r, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    row = pkg.rank_proj(h, A, b, "silu").clone()
    pk = pkg.rank_proj(h, pkg.pack_operand(A), b, "silu")
    torch.cuda.synchronize()
    torch.testing.assert_close(pk, row, rtol=0, atol=0)
    ref = oracle.rank_proj(f(h), f(A), f(b), "silu")
    assert (bf16_ulps(f(row), ref) > 0).mean() < 2e-3


def test_rank_proj_tiled_into_unaligned_view(pkg, dev):
    """The LDS-tiled rank GEMM (split K + epilogue kernel) writing into an
    output view whose rows are not 4- or 8-byte aligned gives the same rank as
    into a contiguous tensor."""
    M, d, r = 128, 1024, 64
    g = torch.Generator().manual_seed(5)
    h = torch.randn(M, d, generator=g).to(torch.bfloat16).to(dev)
    A = (torch.randn(r, d, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    want = pkg.rank_proj(h, A, None, "silu").clone()
    big = torch.zeros(M, r + 3, dtype=torch.bfloat16, device=dev)
    view = big[:, 1:r + 1]                     # row stride r + 3 (odd), start offset 2 bytes
    got = pkg.rank_proj(h, A, None, "silu", out=view)
    torch.cuda.synchronize()
    torch.testing.assert_close(got, want, rtol=0, atol=0)
    assert big[:, 0].abs().sum().item() == 0 and big[:, r + 1:].abs().sum().item() == 0


# ------------------------------------------------------------------ end-to-end draft step

@pytest.mark.parametrize("name", ["qwen3_4b_m16", "qwen3_8b_m16"])
def test_lowrank_argmax_configs(pkg, dev, name):
    print(f"case lowrank_argmax {name}", flush=True)
    x = pkg.synth.config_inputs(name)
    xd = x.to(dev)
    ids, score = pkg.lowrank_argmax(xd.h, xd.A, xd.B, xd.base, xd.prior, xd.alpha, xd.beta, act=x.act)
    torch.cuda.synchronize()
    rank = oracle.rank_proj(f(x.h), f(x.A), None, x.act)
    assert_parity(ids, score, rank, f(x.B), f(x.base), f(x.prior), f(x.alpha), f(x.beta))


# Few rows with both weights packed: the one-launch decode step (split rank
# projection over all workgroups, then the argmax stream).  Every r it takes,
# d that does and does not divide evenly over the K splits, 1..16 rows, bias,
# silu, every base dtype and prior kind.
DECODE_CASES = [
    # M, d, r, act, bias, base dtype, prior dtype (None: no prior), V
    (16, 4096, 512, "identity", False, torch.float32, torch.float32, 151936),
    (16, 2560, 256, "silu", True, torch.bfloat16, torch.bfloat16, 151936),
    (5, 1024, 128, "silu", False, torch.float16, None, 20011),
    (1, 352, 64, "identity", True, torch.float32, torch.float16, 5003),
    (9, 4096, 512, "silu", True, torch.bfloat16, torch.float32, 30000),
]


@pytest.mark.parametrize("M,d,r,act,bias,bdt,pdt,V", DECODE_CASES)
def test_lowrank_decode_step(pkg, dev, M, d, r, act, bias, bdt, pdt, V):
    print(f"case decode M={M} d={d} r={r} {act} bias={bias} base={bdt} prior={pdt} V={V}", flush=True)
    x = pkg.synth.lowrank_inputs(M, d, r, V, base_dtype=bdt, prior_dtype=pdt or torch.float32, per_position=True,
                                 seed=M + d + r)
    g = torch.Generator().manual_seed(d)
    rb = (torch.randn(r, generator=g) * 0.5).to(torch.bfloat16) if bias else None
    xd = x.to(dev)
    Ap, Bp = pkg.pack_operand(xd.A), pkg.pack_operand(xd.B)
    prior = xd.prior if pdt is not None else None
    ids, score = pkg.lowrank_argmax(xd.h, Ap, Bp, xd.base, prior, xd.alpha, xd.beta, act=act,
                                    rank_bias=None if rb is None else rb.to(dev))
    torch.cuda.synchronize()
    rank = oracle.rank_proj(f(x.h), f(x.A), None if rb is None else f(rb), act)
    assert_parity(ids, score, rank, f(x.B), f(x.base), None if prior is None else f(x.prior), f(x.alpha),
                  f(x.beta))


def test_lowrank_decode_repeat_and_local_rank_fallback(pkg, dev):
    """Back-to-back decode steps are bit-identical (the rank words of one launch
    never pass for the next one's), and with the rank poll limit forced to
    zero -- every workgroup computes the rank itself, as when the
    grid is not co-resident -- the results still meet the parity rule."""
    M, d, r, V = 16, 4096, 512, 151936
    x = pkg.synth.config_inputs("qwen3_8b_m16")
    xd = x.to(dev)
    Ap, Bp = pkg.pack_operand(xd.A), pkg.pack_operand(xd.B)
    first = None
    for _ in range(10):
        ids, score = pkg.lowrank_argmax(xd.h, Ap, Bp, xd.base, xd.prior, xd.alpha, xd.beta, act=x.act)
        torch.cuda.synchronize()
        if first is None:
            first = (ids.clone(), score.clone())
        else:
            assert torch.equal(ids, first[0]) and torch.equal(score, first[1])
    rank = oracle.rank_proj(f(x.h), f(x.A), None, x.act)
    ref = oracle.fused_argmax(rank, f(x.B), f(x.base), f(x.prior), f(x.alpha), f(x.beta))
    assert_parity(first[0], first[1], rank, f(x.B), f(x.base), f(x.prior), f(x.alpha), f(x.beta), ref=ref)
    lib = pkg._lib.load()
    prev = lib.dels_debug_set_decode_spin_limit(0)
    try:
        ids2, score2 = pkg.lowrank_argmax(xd.h, Ap, Bp, xd.base, xd.prior, xd.alpha, xd.beta, act=x.act)
        torch.cuda.synchronize()
    finally:
        lib.dels_debug_set_decode_spin_limit(prev)
    assert_parity(ids2, score2, rank, f(x.B), f(x.base), f(x.prior), f(x.alpha), f(x.beta), ref=ref)
    # the local computation sums the same K-slice partials in the same order
    assert torch.equal(ids2, first[0]) and torch.equal(score2, first[1])
    # and the normal path again, on the workspace the fallback call used
    ids3, score3 = pkg.lowrank_argmax(xd.h, Ap, Bp, xd.base, xd.prior, xd.alpha, xd.beta, act=x.act)
    torch.cuda.synchronize()
    assert torch.equal(ids3, first[0]) and torch.equal(score3, first[1])


@pytest.mark.parametrize("layout", ["rowmajor", "packed"])
def test_lowrank_argmax_m512_rows(pkg, dev, layout):
    """The batched-verification shape (M=512, d=4096, r=512, V=151936, bf16 base and prior):
    every one of the 512 rows against the oracle, with row-major and packed weights."""
    print(f"case lowrank_argmax M=512 {layout}", flush=True)
    x = pkg.synth.config_inputs("qwen3_8b_m512")
    xd = x.to(dev)
    A, B = (xd.A, xd.B) if layout == "rowmajor" else (pkg.pack_operand(xd.A), pkg.pack_operand(xd.B))
    ids, score = pkg.lowrank_argmax(xd.h, A, B, xd.base, xd.prior, xd.alpha, xd.beta, act=x.act)
    torch.cuda.synchronize()
    rank = oracle.rank_proj(f(x.h), f(x.A), None, x.act)
    res = assert_parity(ids, score, rank, f(x.B), f(x.base), f(x.prior), f(x.alpha), f(x.beta))
    assert res["rows"] == 512 and res["pinned"] >= 500


def _exact_dot_case(M, d, r, V, seed):
    """Inputs whose rank and dot products are exact in fp32 under any summation order.

    h and A in {-1, 0, 1} (A sparse) give an integer rank of magnitude <= 256
    (exact in bf16); B holds multiples of 1/64 in [-1, 1]; every partial sum of
    rank . B[v] is then a multiple of 1/64 below 2**15, i.e. within fp32's 24
    bits, so MFMA accumulation order cannot change it.  The combine's roundings
    are then the only ones left.
    """
    rng = np.random.default_rng(seed)
    h = rng.integers(-1, 2, (M, d)).astype(np.float32)
    A = (rng.integers(-1, 2, (r, d)) * (rng.random((r, d)) < 1 / 32)).astype(np.float32)
    B = (rng.integers(-64, 65, (V, r)) / 64).astype(np.float32)
    base = (rng.standard_normal((M, V)) * 3).astype(np.float32)
    prior = np.log(rng.dirichlet(np.ones(V))).astype(np.float32)
    alpha = rng.uniform(0.05, 0.6, M).astype(np.float32)
    beta = rng.uniform(0.05, 0.6, M).astype(np.float32)
    beta[::5] = 0.0                                      # rows without the prior term
    return h, A, B, base, prior, alpha, beta


def test_combine_rounding_is_the_same_on_every_path(pkg, dev):
    """The combine s = fma(-beta, prior, fma(dot, alpha, base)) is rounded the same way by the
    one-launch decode step (M <= 16), the GEMV kernel (M < 64) and the MFMA-tiled kernel
    (M >= 64) as by the oracle: with exact dot products the scores agree bit for bit, on rows
    where rounding the products separately would give different scores."""
    M, d, r, V = 64, 256, 128, 20011
    h, A, B, base, prior, alpha, beta = _exact_dot_case(M, d, r, V, seed=31)
    rank = oracle.rank_proj(h, A)
    assert np.array_equal(rank, h @ A.T)                 # the integer rank is exact
    ids, best, _ = oracle.fused_argmax(rank, B, base, prior, alpha, beta)
    # the same winners rounded as two separate products and sums
    dot = (rank.astype(np.float64) * B[ids].astype(np.float64)).sum(1).astype(np.float32)
    two = ((dot * alpha).astype(np.float32) + base[np.arange(M), ids]).astype(np.float32)
    two = np.where(beta != 0, (two - (beta * prior[ids]).astype(np.float32)).astype(np.float32), two)
    differs = two != best
    assert differs[:16].sum() >= 2 and differs[:40].sum() >= 4 and differs.sum() >= 8, differs.sum()

    hd = torch.from_numpy(h).to(torch.bfloat16).to(dev)
    Ap = pkg.pack_operand(torch.from_numpy(A).to(torch.bfloat16).to(dev))
    Bd = torch.from_numpy(B).to(torch.bfloat16).to(dev)
    Bp = pkg.pack_operand(Bd)
    rd = torch.from_numpy(rank).to(torch.bfloat16).to(dev)
    based = torch.from_numpy(base).to(dev)
    priord = torch.from_numpy(prior).to(dev)
    al = torch.from_numpy(alpha).to(dev)
    be = torch.from_numpy(beta).to(dev)
    runs = {
        "decode M=16": pkg.lowrank_argmax(hd[:16], Ap, Bp, based[:16], priord, al[:16], be[:16]),
        "gemv M=40": pkg.fused_argmax(rd[:40], Bp, based[:40], priord, al[:40], be[:40]),
        "gemv row-major M=40": pkg.fused_argmax(rd[:40], Bd, based[:40], priord, al[:40], be[:40]),
        "tiled M=64": pkg.fused_argmax(rd, Bp, based, priord, al, be),
    }
    torch.cuda.synchronize()
    for name, (gi, gs) in runs.items():
        n = gi.numel()
        np.testing.assert_array_equal(gi.cpu().numpy(), ids[:n], err_msg=name)
        np.testing.assert_array_equal(gs.cpu().numpy(), best[:n], err_msg=name)


# ------------------------------------------------------------------ golden fixtures

@pytest.mark.parametrize("name", ["argmax_ragged_silu_f32.npz", "argmax_bf16_identity.npz",
                                  "argmax_noprior_m20.npz"])
def test_golden_argmax(pkg, dev, name):
    z = np.load(os.path.join(GOLDEN, name))
    act = str(z["act"])
    base = torch.from_numpy(z["base"])
    prior = torch.from_numpy(z["prior"])
    if bool(z["base_bf16"]):
        base, prior = base.to(torch.bfloat16), prior.to(torch.bfloat16)
    prior_d = prior.to(dev) if bool(z["with_prior"]) else None
    ids, score = pkg.lowrank_argmax(from_bits(z["h"], dev), from_bits(z["A"], dev), from_bits(z["B"], dev),
                                    base.to(dev), prior_d, torch.from_numpy(z["alpha"]).to(dev),
                                    torch.from_numpy(z["beta"]).to(dev), act=act)
    torch.cuda.synchronize()
    rank = oracle.bf16_bits_to_f32(z["rank"]).reshape(z["rank"].shape)
    B = oracle.bf16_bits_to_f32(z["B"]).reshape(z["B"].shape)
    assert_parity(ids, score, rank, B, f(base), f(prior) if prior_d is not None else None, z["alpha"], z["beta"],
                  ref=(z["ids"], z["score"], z["second"]))


@pytest.mark.parametrize("name", ["gru_b4_g32.npz", "gru_b17_g48_bias.npz"])
def test_golden_gru(pkg, dev, name):
    z = np.load(os.path.join(GOLDEN, name))
    b_hh = from_bits(z["b_hh"], dev) if z["b_hh"].size else None
    tok = torch.from_numpy(z["tokens"]).to(dev)
    for h_key, out_key in (("h", "h_out"), (None, "h_out_zero")):
        h = from_bits(z[h_key], dev) if h_key else None
        out = pkg.gru_step(from_bits(z["table"], dev), tok, h, from_bits(z["W_hh"], dev), b_hh)
        torch.cuda.synchronize()
        ref = oracle.bf16_bits_to_f32(z[out_key]).reshape(z[out_key].shape)
        ulps = bf16_ulps(f(out), ref)
        assert ulps.max() <= 1 and (ulps > 0).mean() < 0.02, (name, out_key, ulps.max(), (ulps > 0).mean())


# ------------------------------------------------------------------ GRU step

@pytest.mark.parametrize("nb,G", [(1, 1024), (8, 1024), (33, 256), (64, 128)])
def test_gru_step(pkg, dev, nb, G):
    print(f"case gru_step nb={nb} G={G}", flush=True)
    g = torch.Generator().manual_seed(nb * G)
    rows = 300
    table = torch.randn(rows, 3 * G, generator=g).to(torch.bfloat16)
    w_hh = (torch.randn(3 * G, G, generator=g) * 0.02).to(torch.bfloat16)
    b_hh = (torch.randn(3 * G, generator=g) * 0.1).to(torch.bfloat16)
    h = torch.randn(nb, G, generator=g).to(torch.bfloat16)
    tok_full = torch.randint(0, rows, (nb, 4), generator=g)
    tok = tok_full[:, 2]                       # a strided column of token ids
    out = pkg.gru_step(table.to(dev), tok_full.to(dev)[:, 2], h.to(dev), w_hh.to(dev), b_hh.to(dev))
    torch.cuda.synchronize()
    ref = oracle.gru_cell(f(table)[tok.numpy()], f(h), f(w_hh), f(b_hh))
    ulps = bf16_ulps(f(out), ref)
    assert ulps.max() <= 1 and (ulps > 0).mean() < 0.01


# ------------------------------------------------------------------ rollout runner

class _Head(torch.nn.Module):
    """Duck-typed local head: the attributes DeLSGraphRunner reads."""

    def __init__(self, V, E, G, r, act, rank_bias, seed, std=0.2, gru_bias=False):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.embed_tokens = torch.nn.Embedding(V, E)
        self.prefix_gru = torch.nn.GRU(E, G, num_layers=1, batch_first=True, bias=gru_bias)
        self.rank_proj = torch.nn.Linear(G, r, bias=rank_bias)
        self.low_rank_lm_head = torch.nn.Linear(r, V, bias=False)
        self.rank_activation = act
        with torch.no_grad():
            self.embed_tokens.weight.copy_(torch.randn(V, E, generator=g))
            self.prefix_gru.weight_ih_l0.copy_(torch.randn(3 * G, E, generator=g) * std)
            self.prefix_gru.weight_hh_l0.copy_(torch.randn(3 * G, G, generator=g) * std)
            if gru_bias:
                self.prefix_gru.bias_ih_l0.copy_(torch.randn(3 * G, generator=g) * 0.3)
                self.prefix_gru.bias_hh_l0.copy_(torch.randn(3 * G, generator=g) * 0.3)
            self.rank_proj.weight.copy_(torch.randn(r, G, generator=g) * std)
            if rank_bias:
                self.rank_proj.bias.copy_(torch.randn(r, generator=g) * 0.1)
            self.low_rank_lm_head.weight.copy_(torch.randn(V, r, generator=g) * std)
        self.to(torch.bfloat16)


@pytest.mark.parametrize("nb,steps,V,E,G,r,act,rank_bias,with_prior,std",
                         [(1, 14, 5003, 32, 64, 64, "silu", False, True, 0.2),
                          (3, 6, 2000, 16, 128, 96, "identity", True, True, 0.2),
                          (8, 4, 151936, 64, 1024, 256, "silu", False, False, 0.02)])
def test_graph_runner_rollout(pkg, dev, nb, steps, V, E, G, r, act, rank_bias, with_prior, std):
    print(f"case runner nb={nb} steps={steps} V={V} G={G} r={r}", flush=True)
    head = _Head(V, E, G, r, act, rank_bias, seed=nb + V, std=std).to(dev)
    g = torch.Generator().manual_seed(11)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0) if with_prior else None
    alphas = [0.1 + 0.05 * i for i in range(steps)]
    betas = [0.3 if with_prior else 0.0] * steps
    if with_prior:
        betas[1] = 0.0
    runner = pkg.DeLSGraphRunner(local_head=head, batch_size=nb, steps=steps, vocab_size=V, alpha_values=alphas,
                                 beta_values=betas, baseline_logits=prior, device=dev)
    assert runner._can_triton_fuse
    prefix = torch.randint(0, V, (nb, 1), generator=g)
    base = (torch.randn(nb, steps, V, generator=g) * 3).to(torch.bfloat16)
    out = runner(prefix.to(dev), base.to(dev))
    scores = runner.static_scores.clone()
    torch.cuda.synchronize()
    assert out.shape == (nb, steps) and out.dtype == torch.int64
    # replay again and run the same kernels eagerly: identical ids (deterministic kernels)
    out2 = runner(prefix.to(dev), base.to(dev))
    runner.enqueue_eager()
    torch.testing.assert_close(out2, out, rtol=0, atol=0)
    torch.testing.assert_close(runner.static_out, out, rtol=0, atol=0)
    # oracle, teacher-forced with the device's own ids so each step is checked on its own history
    prior_np = f(prior.to(torch.bfloat16)) if with_prior else None
    dev_ids = out.cpu().numpy()
    rid, rsc, rsec = oracle.rollout(
        prefix.numpy().reshape(-1), f(base), embed=f(head.embed_tokens.weight), W_ih=f(head.prefix_gru.weight_ih_l0),
        W_hh=f(head.prefix_gru.weight_hh_l0), b_hh=None,
        A=f(head.rank_proj.weight), rank_bias=f(head.rank_proj.bias) if rank_bias else None, act=act,
        B=f(head.low_rank_lm_head.weight), prior=prior_np, alphas=alphas, betas=betas, forced_ids=dev_ids)
    res = oracle.check_parity(dev_ids.reshape(-1), f(scores).reshape(-1), rid.reshape(-1), rsc.reshape(-1),
                              rsec.reshape(-1))
    # the device's bf16 GRU state may differ from the oracle's by an ulp: allow score drift of 2e-2
    assert res["id_mismatch_pinned"] == 0, res
    assert res["max_score_err"] < 2e-2, res
    runner.close()


def test_rollout_fused_gru_local_fallback_bit_identical(pkg, dev):
    """At hidden size 1024 the rollout advances the GRU inside the decode launch of steps 1..
    (GRU workgroups publish the new state as tagged words, the rank workgroups read them).  With
    the re-read limit forced to zero every workgroup computes the state and the rank itself, as
    when the grid is not co-resident: the same partial sums in the same order, so the same bits.
    The rollout itself meets the oracle in test_graph_runner_rollout."""
    print("case fused GRU rollout, local fallback", flush=True)
    V, E, G, r, nb, steps = 30011, 64, 1024, 256, 8, 4
    head = _Head(V, E, G, r, "silu", True, seed=21, std=0.02).to(dev)
    g = torch.Generator().manual_seed(5)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0)
    runner = pkg.DeLSGraphRunner(local_head=head, batch_size=nb, steps=steps, vocab_size=V,
                                 alpha_values=[0.2] * steps, beta_values=[0.1] * steps, baseline_logits=prior,
                                 device=dev)
    prefix = torch.randint(0, V, (nb, 1), generator=g).to(dev)
    base = (torch.randn(nb, steps, V, generator=g) * 3).to(torch.bfloat16).to(dev)
    out = runner(prefix, base).clone()
    sc = runner.static_scores.clone()
    torch.cuda.synchronize()
    lib = pkg._lib.load()
    prev = lib.dels_debug_set_decode_spin_limit(0)
    try:
        runner.enqueue_eager()
        torch.cuda.synchronize()
    finally:
        lib.dels_debug_set_decode_spin_limit(prev)
    assert torch.equal(runner.static_out, out) and torch.equal(runner.static_scores, sc)
    # and the tagged path again on the workspace the fallback used
    runner.enqueue_eager()
    torch.cuda.synchronize()
    assert torch.equal(runner.static_out, out) and torch.equal(runner.static_scores, sc)
    runner.close()


@pytest.mark.parametrize("head_dtype", [torch.float32, torch.float16])
def test_graph_runner_accepts_fp32_and_fp16_heads(pkg, dev, head_dtype):
    """A float32 or float16 local head runs as the same head converted once to bf16: base
    logits and prior stay in the head's dtype, the streamed weights are bf16."""
    print(f"case runner head dtype {head_dtype}", flush=True)
    V, E, G, r, nb, steps = 3001, 32, 64, 64, 2, 5
    head = _Head(V, E, G, r, "silu", False, seed=5).to(dev)           # bf16 weights
    other = _Head(V, E, G, r, "silu", False, seed=5).to(dev).to(head_dtype)
    with torch.no_grad():                                              # the same values in the wider dtype
        for p, q in zip(head.parameters(), other.parameters()):
            q.copy_(p.to(head_dtype))
    g = torch.Generator().manual_seed(3)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0).to(head_dtype)
    kw = dict(batch_size=nb, steps=steps, vocab_size=V, alpha_values=[0.3] * steps, beta_values=[0.2] * steps,
              device=dev)
    prefix = torch.randint(0, V, (nb, 1), generator=g).to(dev)
    base = (torch.randn(nb, steps, V, generator=g) * 3).to(head_dtype).to(dev)
    r_other = pkg.DeLSGraphRunner(local_head=other, baseline_logits=prior, **kw)
    assert r_other.static_base_logits.dtype == head_dtype
    out = r_other(prefix, base)
    sc = r_other.static_scores.clone()
    # the bf16 head's rollout over the same base logits and prior, kept in head_dtype
    r_bf16 = pkg.DeLSGraphRunner(local_head=head, baseline_logits=prior, **kw)
    with torch.inference_mode():
        r_bf16.static_base_logits = base.clone()
        r_bf16.baseline_logits = prior.to(dev).contiguous()
        r_bf16.static_prefix_ids.copy_(prefix)
        p = r_bf16._rollout_params(r_bf16.static_base_logits, steps * V, r_bf16.static_prefix_ids,
                                   r_bf16.static_out, r_bf16.static_scores, r_bf16._ws)
        pkg._lib.check(pkg._lib.load().dels_rollout_enqueue(ctypes.byref(p), torch.cuda.current_stream().cuda_stream),
                       "dels_rollout_enqueue")
    torch.cuda.synchronize()
    torch.testing.assert_close(r_bf16.static_out, out, rtol=0, atol=0)
    torch.testing.assert_close(r_bf16.static_scores, sc, rtol=0, atol=0)
    r_other.close()
    r_bf16.close()


def _fp32_reference_rollout(head, prefix, base, prior, alphas, betas, forced):
    """The reference runner's rollout for an fp32 head, every buffer fp32 (code/kernel/dels.py:252,
    260-276, 425-467), on the CPU with torch's own GRU cell: per step the fp32 scores
    ``act(F.linear(h, A, b)) . B^T * alpha + base - beta * prior``; the GRU fed ``forced``."""
    gru = head.prefix_gru
    cell = torch.nn.GRUCell(gru.input_size, gru.hidden_size, bias=gru.bias)
    with torch.no_grad():
        cell.weight_ih.copy_(gru.weight_ih_l0)
        cell.weight_hh.copy_(gru.weight_hh_l0)
        if gru.bias:
            cell.bias_ih.copy_(gru.bias_ih_l0)
            cell.bias_hh.copy_(gru.bias_hh_l0)
    emb = head.embed_tokens.weight
    nb, steps, V = base.shape
    scores = torch.empty(nb, steps, V)
    with torch.no_grad():
        h = cell(emb[prefix.reshape(-1)], torch.zeros(nb, gru.hidden_size))
        for s in range(steps):
            rank = torch.nn.functional.linear(h, head.rank_proj.weight, head.rank_proj.bias)
            if head.rank_activation == "silu":
                rank = torch.nn.functional.silu(rank)
            sc = rank @ head.low_rank_lm_head.weight.t() * alphas[s] + base[:, s]
            if betas[s] != 0.0:
                sc = sc - betas[s] * prior
            scores[:, s] = sc
            if s + 1 < steps:
                h = cell(emb[forced[:, s]], h)
    return scores


@pytest.mark.parametrize("nb,steps,V,E,G,r,std", [(4, 6, 20011, 32, 256, 128, 0.06),
                                                  (8, 5, 30011, 64, 1024, 256, 0.02)])
def test_graph_runner_fp32_head_against_fp32_reference(pkg, dev, nb, steps, V, E, G, r, std):
    """An fp32 local head with weights that bf16 cannot represent.  The reference keeps
    every buffer in fp32; this runner streams the weights in bf16.  Teacher-forced on the
    device's ids, every step's id must equal the fp32 reference's wherever the reference's
    top-2 margin exceeds 2^-5 of the row's low-rank magnitude ``alpha max_v |rank|.|B_v|``
    (a budget for bf16 weights, state and rank: each rounds by at most 2^-9 relative);
    elsewhere the device's pick must be a near-maximum.  Prints the overall agreement."""
    print(f"case fp32 head vs fp32 reference nb={nb} steps={steps} V={V} G={G} r={r}", flush=True)
    g = torch.Generator().manual_seed(900 + G)
    head = _Head(V, E, G, r, "silu", True, seed=901 + G, std=std).float()
    with torch.no_grad():                                   # fp32 values off the bf16 grid
        for p in head.parameters():
            p.add_(torch.randn(p.shape, generator=g) * p.abs().mean() * 2 ** -8)
    prior = torch.log_softmax(torch.randn(V, generator=g), 0)
    alphas = [0.25 + 0.05 * i for i in range(steps)]
    betas = [0.3] * steps
    runner = pkg.DeLSGraphRunner(local_head=head.to(dev), batch_size=nb, steps=steps, vocab_size=V,
                                 alpha_values=alphas, beta_values=betas, baseline_logits=prior, device=dev)
    prefix = torch.randint(0, V, (nb, 1), generator=g)
    base = torch.randn(nb, steps, V, generator=g) * 3
    out = runner(prefix.to(dev), base.to(dev)).cpu()
    runner.close()
    head = head.cpu()
    ref = _fp32_reference_rollout(head, prefix, base, prior, alphas, betas, out)
    top2 = torch.topk(ref, 2, dim=-1).values.double()
    margin = top2[..., 0] - top2[..., 1]
    with torch.no_grad():
        pick = torch.gather(ref, 2, out.unsqueeze(-1)).squeeze(-1).double()
        ref_ids = torch.argmax(ref, dim=-1)
        # the low-rank magnitude per (row, step) along the teacher-forced history
        mags = torch.empty(nb, steps)
        gru = head.prefix_gru
        cell = torch.nn.GRUCell(gru.input_size, gru.hidden_size, bias=gru.bias)
        cell.load_state_dict({"weight_ih": gru.weight_ih_l0, "weight_hh": gru.weight_hh_l0})
        h = cell(head.embed_tokens.weight[prefix.reshape(-1)], torch.zeros(nb, G))
        for s in range(steps):
            rank = torch.nn.functional.silu(torch.nn.functional.linear(h, head.rank_proj.weight, head.rank_proj.bias))
            mags[:, s] = (rank.abs() @ head.low_rank_lm_head.weight.abs().t()).amax(dim=1) * alphas[s]
            if s + 1 < steps:
                h = cell(head.embed_tokens.weight[out[:, s]], h)
    budget = mags.double() * 2 ** -5
    pinned = margin > budget
    match = out == ref_ids
    print(f"  fp32 head: id agreement {match.double().mean():.4f} ({int(match.sum())}/{match.numel()}), pinned "
          f"{int(pinned.sum())}, pinned agreement {match[pinned].double().mean():.4f}", flush=True)
    assert bool(match[pinned].all()), torch.nonzero(pinned & ~match)
    assert bool((pick >= top2[..., 0] - budget).all())
    assert int(pinned.sum()) >= match.numel() // 4


def test_runner_driven_by_position_mix_head(pkg, dev, tmp_path):
    """A block-prefix position-mix joint checkpoint drives the runner as the reference's
    benchmark wires it (code/benchmark.py:356-387, 471-480): its gates are the alpha/beta
    schedules (alpha_beta_schedules), its baseline_logits buffer the prior.  Teacher-forced
    rollout against the oracle."""
    print("case runner from a position-mix joint head", flush=True)
    V, E, G, r, nb, block = 6007, 48, 128, 64, 3, 16
    steps = block - 2
    g = torch.Generator().manual_seed(41)

    class Inner(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.embed_tokens = torch.nn.Embedding.from_pretrained(torch.randn(V, E, generator=g), freeze=True)

    class Target(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.model = Inner()
            self.lm_head = torch.nn.Linear(E, V, bias=False)

    gates = torch.rand(steps, 2, generator=g) * 0.6
    gates[3, 1] = 0.0                                       # a position without the prior term
    pre = "local_head_model."
    state = {pre + "prefix_gru.weight_ih_l0": torch.randn(3 * G, E, generator=g) * 0.2,
             pre + "prefix_gru.weight_hh_l0": torch.randn(3 * G, G, generator=g) * 0.2,
             pre + "rank_proj.weight": torch.randn(r, G, generator=g) * 0.2,
             pre + "low_rank_lm_head.weight": torch.randn(V, r, generator=g) * 0.2,
             "position_gates": gates,
             "baseline_logits": torch.log_softmax(torch.randn(V, generator=g), 0)}
    cfg = {"method": "block_prefix_position_mix_joint",
           "local_head_config": dict(vocab_size=V, embed_dim=E, gru_hidden_dim=G, low_rank_dim=r,
                                     rank_activation="silu")}
    path = str(tmp_path / "block_prefix_position_mix_joint.pt")
    torch.save({"model_config": cfg, "model_state_dict": state}, path)
    head = pkg.PositionMixJointHead.from_checkpoint(checkpoint_path=path, target_model=Target(), block_size=block,
                                                    dtype=torch.bfloat16, device=dev)
    alphas, betas = head.alpha_beta_schedules()
    runner = pkg.DeLSGraphRunner(local_head=head, batch_size=nb, steps=steps, vocab_size=V, alpha_values=alphas,
                                 beta_values=betas, baseline_logits=head.baseline_logits, device=dev)
    prefix = torch.randint(0, V, (nb, 1), generator=g)
    base = (torch.randn(nb, steps, V, generator=g) * 3).to(torch.bfloat16)
    out = runner(prefix.to(dev), base.to(dev))
    torch.cuda.synchronize()
    dev_ids = out.cpu().numpy()
    rid, rsc, rsec = oracle.rollout(
        prefix.numpy().reshape(-1), f(base), embed=f(head.embed_tokens.weight), W_ih=f(head.prefix_gru.weight_ih_l0),
        W_hh=f(head.prefix_gru.weight_hh_l0), b_hh=None, A=f(head.rank_proj.weight), rank_bias=None, act="silu",
        B=f(head.low_rank_lm_head.weight), prior=f(head.baseline_logits).reshape(-1),
        alphas=np.array(alphas, np.float32), betas=np.array(betas, np.float32), forced_ids=dev_ids)
    res = oracle.check_parity(dev_ids.reshape(-1), f(runner.static_scores).reshape(-1), rid.reshape(-1),
                              rsc.reshape(-1), rsec.reshape(-1))
    assert res["id_mismatch_pinned"] == 0 and res["pinned"] >= 0.9 * res["rows"], res
    assert res["max_score_err"] < 2e-2, res
    runner.close()


def test_golden_rollout(pkg, dev):
    z = np.load(os.path.join(GOLDEN, "rollout_b2_s6.npz"))
    V, E = z["emb"].shape
    G = z["W_hh"].shape[1]
    r = z["A"].shape[0]
    nb, steps = z["ids"].shape
    head = _Head(V, E, G, r, str(z["act"]), False, seed=0).to(dev)
    with torch.no_grad():
        head.embed_tokens.weight.copy_(from_bits(z["emb"], dev))
        head.prefix_gru.weight_ih_l0.copy_(from_bits(z["W_ih"], dev))
        head.prefix_gru.weight_hh_l0.copy_(from_bits(z["W_hh"], dev))
        head.rank_proj.weight.copy_(from_bits(z["A"], dev))
        head.low_rank_lm_head.weight.copy_(from_bits(z["B"], dev))
    prior = from_bits(z["prior"], dev)
    runner = pkg.DeLSGraphRunner(local_head=head, batch_size=nb, steps=steps, vocab_size=V,
                                 alpha_values=z["alphas"].tolist(), beta_values=z["betas"].tolist(),
                                 baseline_logits=prior, device=dev)
    base = from_bits(z["base"], dev)
    out = runner(torch.from_numpy(z["prefix"]).view(nb, 1).to(dev), base)
    torch.cuda.synchronize()
    res = oracle.check_parity(out.cpu().numpy().reshape(-1), f(runner.static_scores).reshape(-1),
                              z["ids"].reshape(-1), z["scores"].reshape(-1), z["seconds"].reshape(-1))
    assert res["id_mismatch_pinned"] == 0 and res["max_score_err"] < 2e-2, res
    runner.close()


# ------------------------------------------------------------------ error paths

def test_errors_are_raised_not_faulted(pkg, dev):
    B = torch.zeros(100, 64, dtype=torch.bfloat16, device=dev)
    rank = torch.zeros(2, 64, dtype=torch.bfloat16, device=dev)
    base = torch.zeros(2, 100, device=dev)
    with pytest.raises(ValueError):
        pkg.fused_argmax(rank, B, base[:, :50])
    with pytest.raises(TypeError):
        pkg.fused_argmax(rank.float(), B, base)
    with pytest.raises(ValueError, match="no CPU fallback"):
        pkg.fused_argmax(rank.cpu(), B, base)
    # misaligned operand: caught by the C ABI
    big = torch.zeros(2, 72, dtype=torch.bfloat16, device=dev)
    with pytest.raises(pkg._lib.DelsError, match="aligned"):
        pkg.fused_argmax(big[:, 1:65], B, base)
    with pytest.raises(pkg._lib.DelsError, match="not supported"):
        pkg.fused_argmax(torch.zeros(2, 1024, dtype=torch.bfloat16, device=dev),
                         torch.zeros(100, 1024, dtype=torch.bfloat16, device=dev), base)

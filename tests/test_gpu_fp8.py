"""GPU parity of the fp8 variant (e4m3 weights with per-channel scales) against the oracle.

Same parity rule as the bf16 path: ids bit-exact wherever the oracle's top-2
margin exceeds 1e-3 relative, elsewhere a near-maximum pick; the winning score
within 1e-2 absolute.  The weights are quantised once on the device
(``quantize_e4m3_rows``) and the oracle is given the same e4m3 values and
scales, so the comparison covers the kernels' in-kernel rank quantisation,
contraction and combine.
"""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def f(t):
    return t.detach().float().cpu().numpy()


def e4m3_values(q_u8):
    """uint8 e4m3fn codes (torch, any device) -> float32 numpy."""
    return q_u8.cpu().view(torch.float8_e4m3fn).float().numpy()


def fp8_weight(pkg, W, layout):
    q, s = pkg.quantize_e4m3_rows(W)
    return pkg.pack_operand_fp8(q, s, layout), e4m3_values(q), f(s)


def assert_parity_fp8(ids, score, rank_np, Bq, sB, base_np, prior_np, alpha, beta, ref):
    ids = ids.cpu().numpy()
    score = score.cpu().numpy()
    rid, rsc, rsec = ref
    pick = oracle.score_at_fp8(rank_np, Bq, sB, base_np, prior_np, alpha, beta, np.clip(ids, 0, Bq.shape[0] - 1))
    res = oracle.check_parity(ids, score, rid, rsc, rsec, pick)
    bad = sorted(set(res["bad_rows"]) | set(res["score_bad_rows"]))[:8]
    detail = [(int(m), int(ids[m]), int(rid[m]), float(score[m]), float(rsc[m]), float(pick[m]), float(rsec[m]))
              for m in bad]
    assert res["id_mismatch_pinned"] == 0, (res, detail)
    assert res["score_bad"] == 0, (res, detail)
    assert res["unpinned_far_pick"] == 0, (res, detail)
    return res


# ------------------------------------------------------------------ packing

def _pack_ref(W, layout):
    """The fp8 block layouts of include/dels.h, built on the CPU from row-major bytes."""
    rows, cols = W.shape
    kb = 128 if layout == "k128" else 32
    rb, cb = -(-rows // 16), -(-cols // kb)
    Wp = np.zeros((rb * 16, cb * kb), np.uint8)
    Wp[:rows, :cols] = W
    out = []
    for bi in range(rb):
        for bj in range(cb):
            blk = Wp[bi * 16:(bi + 1) * 16, bj * kb:(bj + 1) * kb]
            if layout == "k128":
                for half in range(2):
                    for lane in range(64):
                        c0 = 32 * (lane // 16) + 16 * half
                        out.append(blk[lane % 16, c0:c0 + 16])
            else:
                for lane in range(64):
                    c0 = 8 * (lane // 16)
                    out.append(blk[lane % 16, c0:c0 + 8])
    return np.concatenate(out)


@pytest.mark.parametrize("rows,cols,layout", [(37, 300, "k128"), (16, 128, "k128"), (37, 72, "k32"),
                                              (512, 4096, "k32")])
def test_pack_fp8_layout(pkg, dev, rows, cols, layout):
    print(f"case pack_fp8 {rows}x{cols} {layout}", flush=True)
    g = torch.Generator().manual_seed(rows * cols)
    W = torch.randint(0, 256, (rows, cols), dtype=torch.uint8, generator=g)
    pw = pkg.pack_operand_fp8(W.to(dev), torch.ones(rows, device=dev), layout)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(pw.data.cpu().numpy(), _pack_ref(W.numpy(), layout))


# ------------------------------------------------------------------ in-kernel e4m3 rounding

@pytest.mark.parametrize("r", [128, 256])   # r=128: the fp8 GEMV; r=256 (>= 64 rows): the fp8 tiled kernel
def test_rank_quantisation_is_exact_e4m3_rounding(pkg, dev, r):
    """Each rank row holds +-448 (so its scale is exactly 1) and one probe value;
    B selects the probe column and the base masks every other vocabulary entry,
    so the returned score is the kernel's e4m3 rounding of the probe.  Probes:
    every e4m3 value, every midpoint between neighbours (ties to even), the
    subnormal range, values that saturate, and random bf16 values."""
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    grid = codes[np.isfinite(codes)]
    pos = np.sort(grid[grid >= 0])
    mids = ((pos[1:].astype(np.float64) + pos[:-1]) / 2).astype(np.float32)
    rng = np.random.default_rng(41)
    rand = (rng.standard_normal(300) * np.exp2(rng.integers(-12, 9, 300))).astype(np.float32)
    probes = np.concatenate([pos, -pos, mids, -mids, rng.uniform(0, 2 ** -6, 100).astype(np.float32),
                             np.array([447.5, 448.0, -448.0, 0.0], np.float32), rand]).astype(np.float32)
    probes = torch.from_numpy(probes).bfloat16().float().numpy()     # the rank is bf16
    probes = probes[np.abs(probes) <= 448.0]
    P = probes.size
    V = 4
    rank = np.zeros((P, r), np.float32)
    rank[:, 0] = np.where(np.arange(P) % 2 == 0, 448.0, -448.0)
    rank[:, 1] = probes
    Bq = np.zeros((V, r), np.uint8)
    Bq[0, 1] = 0x38                                                   # e4m3 1.0 at the probe column
    B = pkg.pack_operand_fp8(torch.from_numpy(Bq).to(dev), torch.ones(V, device=dev), "k128")
    base = np.full((P, V), -1e30, np.float32)
    base[:, 0] = 0.0
    ids, score = pkg.fused_argmax_fp8(torch.from_numpy(rank).bfloat16().to(dev), B, torch.from_numpy(base).to(dev),
                                      None, 1.0, 0.0)
    torch.cuda.synchronize()
    assert (ids.cpu().numpy() == 0).all()
    np.testing.assert_array_equal(score.cpu().numpy(), oracle.e4m3_round(probes))


# ------------------------------------------------------------------ fused argmax (rank given)

FP8_ARGMAX_CASES = [
    (16, 512, 151936, torch.float32, torch.float32),
    (5, 128, 20011, torch.bfloat16, torch.bfloat16),
    (40, 256, 30000, torch.float16, None),
    (100, 512, 50000, torch.bfloat16, torch.float32),
    (1, 128, 4099, torch.float32, None),
    # >= 64 rows, r in {256, 512}: the fp8 MFMA-tiled kernel (ragged row groups, every base dtype)
    (300, 256, 30000, torch.bfloat16, torch.bfloat16),
    (64, 512, 20008, torch.float32, torch.float32),
    (512, 512, 151936, torch.bfloat16, torch.bfloat16),
]


@pytest.mark.parametrize("M,r,V,bdt,pdt", FP8_ARGMAX_CASES)
def test_fused_argmax_fp8(pkg, dev, M, r, V, bdt, pdt):
    print(f"case fused_argmax_fp8 M={M} r={r} V={V}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + r + V)
    rank = (torch.randn(M, r, generator=g)).bfloat16()
    W = torch.randn(V, r, generator=g) * 0.02
    B, Bq, sB = fp8_weight(pkg, W.to(dev), "k128")
    base = (torch.randn(M, V, generator=g) * 3).to(bdt)
    prior = torch.randn(V, generator=g).to(pdt) if pdt is not None else None
    alpha = (torch.rand(M, generator=g) * 0.6 + 0.2).float()
    beta = (torch.rand(M, generator=g) * 0.6).float()
    if M > 2:
        beta[1] = 0.0
    ids, score = pkg.fused_argmax_fp8(rank.to(dev), B, base.to(dev), prior.to(dev) if prior is not None else None,
                                      alpha.to(dev), beta.to(dev))
    torch.cuda.synchronize()
    args = (f(rank), Bq, sB, f(base), f(prior) if prior is not None else None, f(alpha), f(beta))
    ref = oracle.fused_argmax_fp8(*args)
    assert_parity_fp8(ids, score, *args, ref=ref)


# ------------------------------------------------------------------ whole step

FP8_STEP_CASES = [
    # M, d, r, act, bias, base dtype, prior dtype, V    (M <= 16: one decode launch)
    (16, 4096, 512, "identity", False, torch.float32, torch.float32, 151936),
    (5, 1024, 128, "silu", True, torch.bfloat16, None, 20011),
    (9, 2560, 256, "silu", False, torch.float16, torch.float16, 30000),
    (40, 512, 256, "identity", True, torch.float32, torch.float32, 30000),   # rank GEMM + fp8 argmax
    (96, 1000, 128, "silu", True, torch.bfloat16, torch.bfloat16, 20011),    # LDS-tiled rank GEMM, e4m3 A
    # the batched-verification shape: e4m3 rank GEMM, row quantisation, fp8 MFMA-tiled argmax
    (512, 4096, 512, "identity", False, torch.bfloat16, torch.bfloat16, 151936),
    # the rank quantised per row inside the split-K rank epilogue, ragged last workgroup
    # of rows (r = 256: four rows per workgroup; r = 512: two)
    (130, 2048, 256, "silu", True, torch.bfloat16, torch.float32, 30000),
    (257, 1024, 512, "identity", False, torch.float16, None, 30000),
]


def _step_inputs(pkg, dev, M, d, r, act, bias, bdt, pdt, V, seed):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(M, d, generator=g).bfloat16()
    A, Aq, sA = fp8_weight(pkg, (torch.randn(r, d, generator=g) * 0.02).to(dev), "k32")
    B, Bq, sB = fp8_weight(pkg, (torch.randn(V, r, generator=g) * 0.02).to(dev), "k128")
    rb = (torch.randn(r, generator=g) * 0.1).bfloat16() if bias else None
    base = (torch.randn(M, V, generator=g) * 3).to(bdt)
    prior = torch.randn(V, generator=g).to(pdt) if pdt is not None else None
    alpha = (torch.rand(M, generator=g) * 0.6 + 0.2).float()
    beta = (torch.rand(M, generator=g) * 0.6).float()
    return h, A, Aq, sA, B, Bq, sB, rb, base, prior, alpha, beta


@pytest.mark.parametrize("M,d,r,act,bias,bdt,pdt,V", FP8_STEP_CASES)
def test_lowrank_argmax_fp8(pkg, dev, M, d, r, act, bias, bdt, pdt, V):
    print(f"case lowrank_argmax_fp8 M={M} d={d} r={r} V={V}", flush=True)
    h, A, Aq, sA, B, Bq, sB, rb, base, prior, alpha, beta = _step_inputs(pkg, dev, M, d, r, act, bias, bdt, pdt, V,
                                                                          M + d + r)
    ids, score = pkg.lowrank_argmax_fp8(h.to(dev), A, B, base.to(dev), prior.to(dev) if prior is not None else None,
                                        alpha.to(dev), beta.to(dev), act=act,
                                        rank_bias=rb.to(dev) if rb is not None else None)
    torch.cuda.synchronize()
    rank, rid, rsc, rsec = oracle.lowrank_argmax_fp8(f(h), Aq, sA, f(rb) if rb is not None else None, act, Bq, sB,
                                                     f(base), f(prior) if prior is not None else None, f(alpha),
                                                     f(beta))
    assert_parity_fp8(ids, score, rank, Bq, sB, f(base), f(prior) if prior is not None else None, f(alpha), f(beta),
                      ref=(rid, rsc, rsec))


def test_lowrank_argmax_fp8_repeat_and_local_rank_fallback(pkg, dev):
    M, d, r, V = 16, 4096, 512, 151936
    h, A, Aq, sA, B, Bq, sB, rb, base, prior, alpha, beta = _step_inputs(pkg, dev, M, d, r, "identity", False,
                                                                          torch.float32, torch.float32, V, 5)
    xs = (h.to(dev), A, B, base.to(dev), prior.to(dev), alpha.to(dev), beta.to(dev))
    first = None
    for _ in range(6):
        ids, score = pkg.lowrank_argmax_fp8(*xs)
        torch.cuda.synchronize()
        if first is None:
            first = (ids.clone(), score.clone())
        else:
            assert torch.equal(ids, first[0]) and torch.equal(score, first[1])
    rank, rid, rsc, rsec = oracle.lowrank_argmax_fp8(f(h), Aq, sA, None, "identity", Bq, sB, f(base), f(prior),
                                                     f(alpha), f(beta))
    assert_parity_fp8(first[0], first[1], rank, Bq, sB, f(base), f(prior), f(alpha), f(beta), ref=(rid, rsc, rsec))
    lib = pkg._lib.load()
    prev = lib.dels_debug_set_decode_spin_limit(0)
    try:
        ids2, score2 = pkg.lowrank_argmax_fp8(*xs)
        torch.cuda.synchronize()
    finally:
        lib.dels_debug_set_decode_spin_limit(prev)
    assert_parity_fp8(ids2, score2, rank, Bq, sB, f(base), f(prior), f(alpha), f(beta), ref=(rid, rsc, rsec))
    # the local computation sums the same K-slice partials in the same order
    assert torch.equal(ids2, first[0]) and torch.equal(score2, first[1])
    ids3, score3 = pkg.lowrank_argmax_fp8(*xs)
    torch.cuda.synchronize()
    assert torch.equal(ids3, first[0]) and torch.equal(score3, first[1])

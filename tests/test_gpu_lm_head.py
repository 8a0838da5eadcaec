"""GPU tests of the hand-written target LM head, dels_lm_head (code/dflash.py:468,
target.lm_head(parallel_hiddens), with sample() of position 0 fused, :475).

Each stored value is checked against the float64 product of the same bf16
operands under a bound that holds for any fp32 accumulation order followed by
one rounding to bf16:

    |got - ref| <= 2^-8 |ref| + (1 + 2^-8) K 2^-24 (|h| . |W|^T) + 2^-133

(bf16 unit roundoff 2^-8, fp32 recursive summation gamma_K <= K 2^-24 with
margin), and the check is made to fail by a planted error on the CPU.  The
argmax rows must equal torch.argmax of the same kernel's values from a launch
that stores every row (the kernel is deterministic: same values bit for bit),
and the float64 argmax wherever its top-2 gap exceeds twice the bound.
Shapes cover one and several row groups of 128, one and several passes over a
workgroup's vocabulary tiles (40 tiles per pass), a partial last tile, a
strided output without 8-byte rows, and every row an argmax row.
"""

import numpy as np
import pytest
import torch


def _bound(h64, W64, ref, K):
    mag = np.abs(h64) @ np.abs(W64).T
    return 2.0**-8 * np.abs(ref) + (1 + 2.0**-8) * K * 2.0**-24 * mag + 2.0**-133


def _within(got, ref, bound):
    return np.abs(got - ref) <= bound


def test_bound_rejects_a_planted_error():
    """CPU: the bound is tight enough that a value off by a few bf16 ulps fails it."""
    g = np.random.default_rng(3)
    K = 512
    h = g.standard_normal((4, K)).astype(np.float32)
    W = (g.standard_normal((50, K)) * 0.05).astype(np.float32)
    h64 = torch.from_numpy(h).bfloat16().double().numpy()
    W64 = torch.from_numpy(W).bfloat16().double().numpy()
    ref = h64 @ W64.T
    got = torch.from_numpy(ref.astype(np.float32)).bfloat16().double().numpy()
    b = _bound(h64, W64, ref, K)
    assert _within(got, ref, b).all()
    bad = got.copy()
    bad[1, 7] = ref[1, 7] * (1 + 3 * 2.0**-8)
    assert not _within(bad, ref, b)[1, 7]


# (M, K, V, argmax_period, strided_out)
CASES = [
    (120, 4096, 20011, 15, False),    # a draft block's rows, partial last tile
    (1, 256, 5003, 0, False),
    (7, 512, 5003, 1, False),         # every row an argmax row: nothing stored
    (129, 512, 30000, 16, True),      # two row groups, output rows of odd length
    (300, 256, 20011, 0, False),      # three row groups
    (128, 1024, 151936, 0, False),    # the full vocabulary: 37-38 tiles per workgroup, one pass
    (4096, 256, 6000, 7, False),      # 32 row groups, 8 workgroups per group: two passes each
]


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,V,period,strided", CASES)
def test_lm_head_values_and_argmax(pkg, dev, M, K, V, period, strided):
    print(f"case lm_head M={M} K={K} V={V} period={period} strided_out={strided}", flush=True)
    g = torch.Generator().manual_seed(M + K + V)
    h = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(V, K, generator=g) * 0.05).bfloat16()
    Wp = pkg.pack_lm_head(W.to(dev))
    hd = h.to(dev)
    out = None
    if strided:
        out = torch.full((M, V + 3), 7.0, dtype=torch.bfloat16, device=dev)[:, :V]
    got, ids, sc = pkg.lm_head(hd, Wp, out=out, argmax_period=period)
    full, _, _ = pkg.lm_head(hd, Wp)          # every row stored
    again, _, _ = pkg.lm_head(hd, Wp)
    torch.cuda.synchronize()
    assert torch.equal(full, again), "repeat launches differ"

    h64 = h.double().numpy()
    W64 = W.double().numpy()
    ref = h64 @ W64.T
    bound = _bound(h64, W64, ref, K)
    f = full.double().cpu().numpy()
    ok = _within(f, ref, bound)
    assert ok.all(), f"{(~ok).sum()} values outside the bound, worst {np.abs(f - ref)[~ok].max()}"

    argmax_rows = np.arange(0, M, period) if period > 0 else np.array([], dtype=np.int64)
    stored = np.setdiff1d(np.arange(M), argmax_rows)
    if period != 1:
        gs = got.double().cpu().numpy()
        # stored rows are the full launch's values bit for bit
        np.testing.assert_array_equal(gs[stored], f[stored])
        if strided:
            # argmax rows are left untouched
            untouched = got[torch.as_tensor(argmax_rows, device=dev)] if len(argmax_rows) else None
            if untouched is not None:
                assert bool((untouched == 7.0).all())
    else:
        assert got is None
    if period > 0:
        ids = ids.cpu().numpy()
        assert ids.shape == (len(argmax_rows),)
        want = torch.argmax(full[torch.as_tensor(argmax_rows, device=dev)].cpu(), dim=-1).numpy()
        np.testing.assert_array_equal(ids, want)
        np.testing.assert_array_equal(sc.cpu().numpy(), f[argmax_rows, want].astype(np.float32))
        # against the float64 product where the top-2 gap exceeds twice the bound
        r = ref[argmax_rows]
        top2 = np.sort(r, axis=1)[:, -2:]
        pinned = (top2[:, 1] - top2[:, 0]) > 2 * bound[argmax_rows].max(axis=1)
        np.testing.assert_array_equal(ids[pinned], np.argmax(r, axis=1)[pinned])
        assert pinned.sum() >= max(1, len(argmax_rows) // 2), pinned.sum()

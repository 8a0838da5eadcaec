"""Pins the oracle's number formats and elementwise math against torch's own routines."""

import numpy as np
import torch
import torch.nn.functional as F

import oracle


def _edge_f32():
    rng = np.random.default_rng(0)
    vals = [
        rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-8, 8, 20000).astype(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, 3.0e38, -3.0e38, 3.4028235e38, 1e-40, -1e-40, 1e-45,
                  np.inf, -np.inf], np.float32),
    ]
    # exact bf16 halfway points (ties to even) and their neighbours
    base = (rng.integers(0, 1 << 16, 4000).astype(np.uint32) << 16) | 0x8000
    halfway = base.view(np.float32)
    with np.errstate(invalid="ignore"):
        vals += [halfway, np.nextafter(halfway, np.float32(np.inf)), np.nextafter(halfway, np.float32(-np.inf))]
    return np.concatenate(vals).astype(np.float32)


def test_bf16_round_matches_torch():
    x = _edge_f32()
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = oracle.bf16_round(x)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)          # NaN payloads may differ
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_bf16_round_nan_and_bits_roundtrip():
    x = np.array([np.nan, -np.nan, 1.5], np.float32)
    got = oracle.bf16_round(x)
    assert np.isnan(got[0]) and np.isnan(got[1]) and got[2] == 1.5
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    f = oracle.bf16_bits_to_f32(bits)
    finite = np.isfinite(f)
    np.testing.assert_array_equal(oracle.f32_to_bf16_bits(f[finite]), bits[finite])


def test_e4m3_round_matches_torch():
    rng = np.random.default_rng(1)
    grid = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    grid = grid[np.isfinite(grid)]
    # every representable value, random values in range, and exact midpoints between neighbours
    s = np.sort(np.unique(grid))
    mids = ((s[1:].astype(np.float64) + s[:-1]) / 2).astype(np.float32)
    x = np.concatenate([grid, rng.uniform(-448, 448, 20000).astype(np.float32),
                        rng.standard_normal(20000).astype(np.float32) * 0.01, mids]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).float().numpy()
    got = oracle.e4m3_round(x)
    np.testing.assert_array_equal(got, ref)


def test_quantize_rows_e4m3_scale():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((64, 96)) * 0.02).astype(np.float32)
    w[3] = 0.0
    q, s = oracle.quantize_rows_e4m3(w)
    assert s[3] == 1.0 and np.all(q[3] == 0)
    np.testing.assert_allclose(np.abs(q).max(axis=1)[np.arange(64) != 3], 448.0)
    # dequantised values are within half an e4m3 ulp (2^-4 relative) of the input
    deq = q * s[:, None]
    assert np.all(np.abs(deq - w) <= np.abs(w) * 2 ** -4 + s[:, None] * 2 ** -10)


def test_sigmoid_silu_match_torch():
    x = np.linspace(-30, 30, 40001).astype(np.float32)
    t = torch.from_numpy(x)
    np.testing.assert_allclose(oracle.sigmoid_f32(x), torch.sigmoid(t).numpy(), rtol=3e-7, atol=1e-30)
    np.testing.assert_allclose(oracle.silu_f32(x), F.silu(t).numpy(), rtol=3e-7, atol=1e-30)


def _e4m3_grid():
    g = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    return g[np.isfinite(g)]


def test_fused_argmax_fp8_reduces_to_bf16_path_on_the_grid():
    # rank rows and B rows on the e4m3 grid with absmax 448: both scales are 1
    # and quantisation is the identity, so the fp8 argmax is the bf16 one exactly
    rng = np.random.default_rng(31)
    grid = _e4m3_grid()
    grid = grid[np.abs(grid) <= 448]
    M, r, V = 6, 128, 700
    rank = rng.choice(grid, (M, r)).astype(np.float32)
    rank[:, 5] = 448.0
    Bq = rng.choice(grid, (V, r)).astype(np.float32)
    Bq[:, 0] = -448.0
    base = (rng.standard_normal((M, V)) * 3).astype(np.float32)
    prior = rng.standard_normal(V).astype(np.float32)
    alpha = rng.uniform(0, 1e-4, M).astype(np.float32)
    beta = np.array([0.3, 0, 0.1, 0.2, 0, 0.5], np.float32)
    got = oracle.fused_argmax_fp8(rank, Bq, np.ones(V, np.float32), base, prior, alpha, beta)
    ref = oracle.fused_argmax(rank, Bq, base, prior, alpha, beta)
    for g, e in zip(got, ref):
        np.testing.assert_array_equal(g, e)
    np.testing.assert_array_equal(oracle.score_at_fp8(rank, Bq, np.ones(V, np.float32), base, prior, alpha, beta,
                                                      got[0]), got[1])


def test_fused_argmax_fp8_brute_force_with_torch_casts():
    # tiny shapes: quantise with torch's float8 cast, score every (m, v) in
    # float64 with the stated rounding points, take the first maximum
    rng = np.random.default_rng(32)
    M, r, V = 3, 128, 37
    rank = torch.from_numpy((rng.standard_normal((M, r)) * 0.7).astype(np.float32)).bfloat16().float().numpy()
    rank[1] = 0.0                                    # an all-zero row: scale 1, zero dot
    Bq = _e4m3_grid()[rng.integers(0, 200, (V, r))].astype(np.float32)
    sB = rng.uniform(1e-4, 1e-3, V).astype(np.float32)
    base = (rng.standard_normal((M, V)) * 0.05).astype(np.float32)
    alpha = np.array([1.0, 0.5, 2.0], np.float32)
    ids, best, _ = oracle.fused_argmax_fp8(rank, Bq, sB, base, None, alpha, 0.0)
    for m in range(M):
        amax = np.float32(np.abs(rank[m]).max())
        sR = np.float32(amax / np.float32(448.0)) if amax > 0 else np.float32(1.0)
        inv = np.float32(np.float32(448.0) / amax) if amax > 0 else np.float32(1.0)
        rq = torch.from_numpy((rank[m] * inv).astype(np.float32)).to(torch.float8_e4m3fn).float().numpy()
        scores = []
        for v in range(V):
            raw = np.float32(sum(float(a) * float(b) for a, b in zip(rq, Bq[v])))
            dot = np.float32(np.float32(raw * sR) * sB[v])
            scores.append(np.float32(np.float32(dot * alpha[m]) + base[m, v]))
        scores = np.array(scores, np.float32)
        assert ids[m] == int(np.argmax(scores)), m
        assert best[m] == scores.max(), m


def test_fused_argmax_fp8_scale_equivariance():
    # multiplying B row v by 2^k changes only its scale: identical ids and scores
    rng = np.random.default_rng(33)
    M, r, V = 4, 256, 300
    rank = (rng.standard_normal((M, r))).astype(np.float32)
    W = (rng.standard_normal((V, r)) * 0.02).astype(np.float32)
    q, s = oracle.quantize_rows_e4m3(W)
    k = rng.integers(-4, 5, V).astype(np.float32)
    q2, s2 = oracle.quantize_rows_e4m3(W * np.exp2(k)[:, None])
    np.testing.assert_array_equal(q2, q)
    np.testing.assert_array_equal(s2, (s * np.exp2(k)).astype(np.float32))
    base = (rng.standard_normal((M, V))).astype(np.float32)
    a = oracle.fused_argmax_fp8(rank, q, s * np.exp2(k), base, None, 0.5, 0.0)
    b = oracle.fused_argmax_fp8(rank, q2, s2, base, None, 0.5, 0.0)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


def test_quantize_rank_e4m3_against_torch_and_division_form():
    rng = np.random.default_rng(34)
    rank = torch.from_numpy((rng.standard_normal((40, 512)) * 3).astype(np.float32)).bfloat16().float().numpy()
    rank[7] = 0.0
    q, s = oracle.quantize_rank_e4m3(rank)
    assert s[7] == 1.0 and np.all(q[7] == 0)
    amax = np.abs(rank).max(axis=1)
    inv = np.where(amax > 0, np.float32(448.0) / np.where(amax > 0, amax, 1), 1).astype(np.float32)
    ref = torch.from_numpy((rank * inv[:, None]).astype(np.float32)).to(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(q, ref)
    np.testing.assert_array_equal(np.abs(q).max(axis=1)[np.arange(40) != 7], 448.0)
    # against the per-element division form: equal but for rare quotients within an fp32 ulp of a midpoint
    qd, sd = oracle.quantize_rows_e4m3(rank)
    np.testing.assert_array_equal(s, sd)
    assert (q != qd).mean() < 1e-3

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

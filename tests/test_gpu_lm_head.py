"""GPU tests of the hand-written LM head (code/dflash.py:468) with the fused argmax of
chosen rows (sample() of position 0, code/dflash.py:475).

The product is checked against a float64 product of the same bf16 operands
(torch on the GPU): every stored value within one bf16 ulp of bf16(reference)
plus the fp32 accumulation allowance 2^-16 * sum_k |h_k w_k| (which matters
only where the sum cancels to near zero), and bit-equal to bf16(reference) for
all but a few values.  The fused argmax is checked bit for bit against
torch.argmax of the kernel's own stored values (a second launch that stores
every row), which fixes the tie and NaN rules exactly.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _bf16_ulp(x):
    a = np.abs(x).astype(np.float32)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return np.exp2(e - 7)


def _ref(hidden, W):
    """(float64 product, sum of |terms|) of the bf16 operands."""
    with torch.no_grad():
        return hidden.double() @ W.double().T, hidden.double().abs() @ W.double().abs().T


@pytest.mark.parametrize("M,K,V,period", [(120, 4096, 151936, 15), (37, 256, 1001, 5), (130, 512, 4099, 0),
                                          (1, 768, 33, 1), (64, 1024, 20000, 16)])
def test_lm_head_matches_fp32_product_and_argmax(pkg, dev, M, K, V, period):
    print(f"case lm_head M={M} K={K} V={V} period={period}", flush=True)
    g = torch.Generator(device=dev).manual_seed(M * 31 + V)
    hidden = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    W = (torch.randn(V, K, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    Wp = pkg.pack_lm_head(W)
    full, _, _ = pkg.lm_head(hidden, Wp)                       # every row stored
    torch.cuda.synchronize()
    ref, mag = _ref(hidden, W)
    ref_b = ref.to(torch.bfloat16).float().cpu().numpy()
    tol = _bf16_ulp(ref_b) * 1.01 + mag.cpu().numpy() * 2.0 ** -16
    del ref, mag
    got = full.float().cpu().numpy()
    diff = np.abs(got - ref_b)
    assert np.all(diff <= tol), float((diff / tol).max())
    assert np.mean(diff == 0) > 0.99
    if period == 0:
        return
    part, ids, sc = pkg.lm_head(hidden, Wp, argmax_period=period)
    torch.cuda.synchronize()
    arows = np.arange(0, M, period)
    want = torch.argmax(full[arows].cpu(), dim=-1).numpy()
    np.testing.assert_array_equal(ids.cpu().numpy(), want)
    np.testing.assert_array_equal(sc.cpu().numpy(), got[arows, want])
    if period > 1:
        keep = np.setdiff1d(np.arange(M), arows)
        np.testing.assert_array_equal(part.float().cpu().numpy()[keep], got[keep])


def test_lm_head_ties_nan_and_strided_output(pkg, dev):
    """Equal maxima: the lowest index; a NaN in hidden makes the row all NaN (0 * NaN), whose
    argmax is then index 0 with a NaN score (as torch.argmax); an unaligned, strided output
    buffer takes the element-wise stores."""
    M, K, V = 9, 256, 3000
    hidden = torch.zeros(M, K, dtype=torch.bfloat16, device=dev)
    W = torch.zeros(V, K, dtype=torch.bfloat16, device=dev)
    hidden[:, 0] = 1.0
    W[17, 0] = 5.0
    W[2900, 0] = 5.0                      # tie with 17: 17 wins
    hidden[3, 1] = float("nan")           # row 3: every product is NaN -> id 0
    out = torch.full((M, V + 3), 7.0, dtype=torch.bfloat16, device=dev)[:, 1:V + 1]
    _, ids, sc = pkg.lm_head(hidden, W, out=out, argmax_period=3)
    torch.cuda.synchronize()
    got = ids.cpu().numpy()
    assert got[0] == 17 and got[2] == 17 and got[1] == 0, got
    assert torch.isnan(sc[1]).item()
    o = out.float().cpu().numpy()
    np.testing.assert_array_equal(o[1, [17, 2900]], [5.0, 5.0])
    assert np.all(o[[0, 3, 6]] == 7.0)     # argmax rows are not stored

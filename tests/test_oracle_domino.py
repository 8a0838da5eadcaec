"""CPU tests pinning the Domino oracle (code/kernel/domino.py) and the runner's host-side checks."""

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from oracle import domino as DO


def _bf16(t):
    return t.to(torch.bfloat16).float()


# the middle layers the kernels fuse, as the torch modules a model would hold
MIDDLE_MODULES = {"silu": nn.SiLU(), "identity": nn.Identity(), "relu": nn.ReLU(), "gelu": nn.GELU(),
                  "gelu_tanh": nn.GELU(approximate="tanh"), "tanh": nn.Tanh(), "sigmoid": nn.Sigmoid()}


def _mlp(D, G, E, V, fc2_bias, seed, middle="silu"):
    g = torch.Generator().manual_seed(seed)
    mlp = nn.Sequential(nn.Linear(D + G, E, bias=False), MIDDLE_MODULES[middle], nn.Linear(E, V, bias=fc2_bias))
    with torch.no_grad():
        mlp[0].weight.copy_(_bf16(torch.randn(E, D + G, generator=g) * 0.05))
        mlp[2].weight.copy_(_bf16(torch.randn(V, E, generator=g) * 0.05))
        if fc2_bias:
            mlp[2].bias.copy_(_bf16(torch.randn(V, generator=g)))
    return mlp


@pytest.mark.parametrize("fc2_bias,middle", [(False, "silu"), (True, "silu")] +
                         [(True, m) for m in DO.MIDDLES if m != "silu"])
def test_step_matches_torch_modules(fc2_bias, middle):
    """The reference's unfused formula on torch modules in fp32 (code/dflash.py:619-626,
    code/kernel/domino.py:404-431): base + alpha * embed_proj(cat[z_h, s_h]) with the given
    middle module -- against the oracle fed with the two halves of the first layer, under
    the margin rule."""
    D, G, E, V, M, alpha = 48, 32, 64, 997, 9, 0.8
    mlp = _mlp(D, G, E, V, fc2_bias, seed=1, middle=middle)
    g = torch.Generator().manual_seed(2)
    zh, sh = torch.randn(M, D, generator=g), torch.randn(M, G, generator=g)
    base = torch.randn(M, V, generator=g) * 3
    with torch.no_grad():
        logits = base + alpha * mlp(torch.cat([zh, sh], dim=-1))
    want = torch.argmax(logits, dim=-1).numpy()
    W1 = mlp[0].weight.detach().numpy()
    z = (zh.double() @ torch.tensor(W1[:, :D]).double().T).float().numpy()
    s = (sh.double() @ torch.tensor(W1[:, D:]).double().T).float().numpy()
    bias = mlp[2].bias.detach().numpy() if fc2_bias else None
    ids, best, second = DO.domino_step(z, s, mlp[2].weight.detach().numpy(), bias, base.numpy(), alpha,
                                       middle=middle)
    res = oracle.check_parity(want, logits.gather(1, torch.tensor(want)[:, None])[:, 0].numpy(), ids, best, second)
    assert res["id_mismatch_pinned"] == 0 and res["score_bad"] == 0, res


@pytest.mark.parametrize("middle", [m for m in DO.MIDDLES if m != "silu"])
def test_middle_layers_match_torch_modules_elementwise(middle):
    """Each middle layer of the oracle against its torch module evaluated in float64 on the
    same fp32 inputs (ordinary values, zeros, large magnitudes): equal after rounding to fp32
    within one fp32 ulp, or 1e-12 absolute (the two float64 formulas may differ in their last
    bits, and the tanh form of GELU cancels to ~1e-16 for large negative inputs)."""
    rng = np.random.default_rng(11)
    p = np.concatenate([rng.standard_normal(4000) * 3, [0.0, -0.0, 1e-30, -1e-30, 12.5, -12.5, 40.0, -40.0]])
    p = p.astype(np.float32)
    got = DO.domino_mid(p, np.zeros_like(p), middle)
    want = MIDDLE_MODULES[middle](torch.tensor(p, dtype=torch.float64)).numpy().astype(np.float32)
    np.testing.assert_allclose(got, want, rtol=1.2e-7, atol=1e-12)
    # a planted mistake the check must see: GELU with x / 2 for the erf argument instead of x / sqrt(2)
    if middle == "gelu":
        from scipy.special import erf
        wrong = (0.5 * p.astype(np.float64) * (1 + erf(p.astype(np.float64) / 2))).astype(np.float32)
        assert not np.allclose(wrong, want, rtol=1.2e-7, atol=1e-12)


def test_middle_name_of_modules(pkg):
    """The runner's map from the correction MLP's middle modules to the fused kernel's codes."""
    from importlib import import_module
    mn = import_module(pkg.__name__ + ".domino_runner").middle_name
    for name, mod in MIDDLE_MODULES.items():
        assert mn(mod) == name and mn(nn.Sequential(mod)) == name
    assert mn(nn.Sequential()) == "identity"
    assert mn(nn.LeakyReLU()) is None and mn(nn.Sequential(nn.SiLU(), nn.Dropout())) is None


def test_step_closed_forms():
    rng = np.random.default_rng(3)
    M, E, V = 5, 32, 300
    z, s = rng.standard_normal((M, E)).astype(np.float32), rng.standard_normal((M, E)).astype(np.float32)
    fc2 = (rng.standard_normal((V, E)) * 0.1).astype(np.float32)
    base = (rng.standard_normal((M, V)) * 3).astype(np.float32)
    bias = rng.standard_normal(V).astype(np.float32)
    ids, best, _ = DO.domino_step(z, s, fc2, bias, base, 0.0)          # alpha 0: argmax(base)
    np.testing.assert_array_equal(ids, base.argmax(1))
    np.testing.assert_array_equal(best, base.max(1))
    ids, _, _ = DO.domino_step(z, s, np.zeros_like(fc2), bias, base, 0.5)  # fc2 0: argmax(0.5 bias + base)
    np.testing.assert_array_equal(ids, (0.5 * bias[None, :] + base).argmax(1))
    base[:, 7] = base.max() + 100                                      # planted winner, tail and head
    ids, _, _ = DO.domino_step(z, s, fc2, None, base, 1.0)
    assert np.all(ids == 7)


def test_step_brute_force_tiny():
    """A pure-Python evaluation (float64 loops) of the restated formula on tiny shapes."""
    rng = np.random.default_rng(4)
    M, E, V = 3, 5, 11
    z, s = rng.standard_normal((M, E)).astype(np.float32), rng.standard_normal((M, E)).astype(np.float32)
    fc2 = rng.standard_normal((V, E)).astype(np.float32)
    base = (rng.standard_normal((M, V)) * 3).astype(np.float32)
    bias = rng.standard_normal(V).astype(np.float32)
    ids, best, second = DO.domino_step(z, s, fc2, bias, base, 0.6)
    import math
    for m in range(M):
        mid = []
        for k in range(E):
            p = float(z[m, k]) + float(s[m, k])
            mid.append(p / (1.0 + math.exp(-p)))
        sc = [(sum(float(fc2[v, k]) * mid[k] for k in range(E)) + float(bias[v])) * 0.6 + float(base[m, v])
              for v in range(V)]
        top = max(range(V), key=lambda v: (sc[v], -v))
        assert ids[m] == top
        assert abs(best[m] - sc[top]) < 1e-4 * max(1.0, abs(sc[top]))


def test_rollout_matches_torch_gru_and_modules_teacher_forced():
    """The rollout (code/kernel/domino.py:379-436) against nn.GRU + nn.Embedding + the MLP in
    fp32, fed the same ids: where torch's top-2 margin exceeds 0.05 the ids agree."""
    D, G, E, V, B, S, P, alpha = 32, 16, 32, 211, 3, 5, 2, 0.9
    mlp = _mlp(D, G, E, V, False, seed=5)
    g = torch.Generator().manual_seed(6)
    gru = nn.GRU(D, G, num_layers=1, batch_first=True, bias=False)
    emb = nn.Embedding(V, D)
    with torch.no_grad():
        gru.weight_ih_l0.copy_(_bf16(torch.randn(3 * G, D, generator=g) * 0.2))
        gru.weight_hh_l0.copy_(_bf16(torch.randn(3 * G, G, generator=g) * 0.2))
        emb.weight.copy_(_bf16(torch.randn(V, D, generator=g)))
    prefix = torch.randint(0, V, (B, P), generator=g)
    hiddens = _bf16(torch.randn(B, S, D, generator=g))
    base = _bf16(torch.randn(B, S, V, generator=g) * 3)
    with torch.no_grad():
        _, h = gru(emb(prefix))
        ids_t, margins = [], []
        for t in range(S):
            logits = base[:, t] + alpha * mlp(torch.cat([hiddens[:, t], h[0]], dim=-1))
            top2 = torch.topk(logits, 2, dim=-1).values
            margins.append((top2[:, 0] - top2[:, 1]).numpy())
            cur = torch.argmax(logits, dim=-1)
            ids_t.append(cur.numpy())
            _, h = gru(emb(cur)[:, None, :], h)
    ids_t, margins = np.stack(ids_t, 1), np.stack(margins, 1)
    W1 = mlp[0].weight.detach().numpy()
    ids, _, _ = DO.domino_rollout(prefix.numpy(), hiddens.numpy(), base.numpy(),
                                  W_hh=gru.weight_hh_l0.detach().numpy(), b_hh=None, w_z=W1[:, :D], fc1_bias=None,
                                  w_s=W1[:, D:], fc2=mlp[2].weight.detach().numpy(), fc2_bias=None, alpha=alpha,
                                  embed=emb.weight.detach().numpy(), W_ih=gru.weight_ih_l0.detach().numpy(),
                                  forced_ids=ids_t)
    pinned = margins > 0.05
    assert pinned.mean() > 0.8
    np.testing.assert_array_equal(ids[pinned], ids_t[pinned])


class _Draft(nn.Module):
    def __init__(self, embed_proj, D=32, G=16):
        super().__init__()
        self.embed_proj = embed_proj
        self.prefix_gru = nn.GRU(D, G, batch_first=True, bias=False)


class _Target(nn.Module):
    def __init__(self, V=64, D=32):
        super().__init__()
        self.model = nn.Module()
        self.model.embed_tokens = nn.Embedding(V, D)


@pytest.mark.parametrize("embed_proj,exc,msg", [
    (nn.Linear(48, 64), TypeError, "to be nn.Sequential"),
    (nn.Sequential(nn.Linear(48, 64)), ValueError, "at least two layers"),
    (nn.Sequential(nn.SiLU(), nn.Linear(48, 64)), ValueError, "first layer must be nn.Linear"),
    (nn.Sequential(nn.Linear(48, 64), nn.SiLU()), ValueError, "last layer must be nn.Linear"),
    (nn.Sequential(nn.Linear(40, 64), nn.SiLU(), nn.Linear(64, 64)), ValueError, "input dim mismatch"),
    (nn.Sequential(nn.Linear(48, 64), nn.LeakyReLU(), nn.Linear(64, 64)), ValueError, "fuses a middle layer"),
])
def test_runner_argument_checks(pkg, embed_proj, exc, msg):
    """The reference's checks and messages (code/kernel/domino.py:15-51, 268-275), raised before
    any GPU work."""
    with pytest.raises(exc, match=msg):
        pkg.DraftCorrectionGraphRunner(draft_model=_Draft(embed_proj), target_model=_Target(), batch_size=1, steps=3,
                                       hidden_dim=32, gru_hidden_dim=16, vocab_size=64, prefix_token_count=2,
                                       device="cuda")


def test_unwrap_correction_mlp(pkg):
    fc1, mid, fc2 = pkg.unwrap_correction_mlp(nn.Sequential(nn.Linear(4, 8), nn.SiLU(), nn.Linear(8, 3)))
    assert isinstance(fc1, nn.Linear) and isinstance(fc2, nn.Linear) and isinstance(mid, nn.Sequential)
    _, mid2, _ = pkg.unwrap_correction_mlp(nn.Sequential(nn.Linear(4, 8), nn.Linear(8, 3)))
    assert isinstance(mid2, nn.Identity)

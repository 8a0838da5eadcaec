"""CPU tests of the local-head modules' checkpoint loaders and host-side helpers.

The reference ships no checkpoints (and none can be fetched), so every file
here is synthetic, written by the test in the formats the reference's loaders
read (code/dels.py:115-138, 208-305, 381-426, 489-604).  Each test checks the
loaded module against the tensors that went into the file, with the folds
(target LM head x rank_to_hidden, target embedding x down_proj) recomputed
in float64 numpy.
"""

import numpy as np
import pytest
import torch

import oracle

V, E, G, R, H = 40, 12, 16, 8, 24   # vocabulary, embedding, GRU hidden, rank, target hidden


class _Inner(torch.nn.Module):
    def __init__(self, emb):
        super().__init__()
        self.embed_tokens = torch.nn.Embedding.from_pretrained(emb, freeze=True)


class _Target(torch.nn.Module):
    """A stand-in target model: ``model.embed_tokens`` and ``lm_head``."""

    def __init__(self, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.model = _Inner(torch.randn(V, E, generator=g))
        self.lm_head = torch.nn.Linear(H, V, bias=False)
        with torch.no_grad():
            self.lm_head.weight.copy_(torch.randn(V, H, generator=g) * 0.1)


def _rnn_state(seed=1, *, lm_head=True, up=False, prefix=""):
    g = torch.Generator().manual_seed(seed)
    sd = {
        prefix + "prefix_gru.weight_ih_l0": torch.randn(3 * G, E, generator=g) * 0.1,
        prefix + "prefix_gru.weight_hh_l0": torch.randn(3 * G, G, generator=g) * 0.1,
        prefix + "rank_proj.weight": torch.randn(R, G, generator=g) * 0.1,
    }
    if lm_head:
        sd[prefix + "low_rank_lm_head.weight"] = torch.randn(V, R, generator=g) * 0.1
    if up:
        sd[prefix + "rank_to_hidden.weight"] = torch.randn(H, R, generator=g) * 0.1
    return sd


def _config(**kw):
    c = dict(vocab_size=V, embed_dim=E, gru_hidden_dim=G, low_rank_dim=R, rank_activation="silu")
    c.update(kw)
    return c


def _save(tmp_path, name, obj):
    p = tmp_path / name
    torch.save(obj, p)
    return str(p)


def _f64(t):
    return t.detach().to(torch.float64).numpy()


# ------------------------------------------------------------------ a11: target LM-head fold

def test_fuse_target_lm_head_matches_fp32_product(pkg):
    """fuse_target_lm_head_ folds W_target [V, H] . rank_to_hidden [H, R] in fp32 and rounds
    once to the head's dtype (code/dels.py:307-322)."""
    tgt = _Target()
    head = pkg.DeLSLocalHead(target_model=tgt, vocab_size=V, embed_dim=E, gru_hidden_dim=G, low_rank_dim=R,
                             lm_head_mode="target_lm_head", rank_activation="identity", dtype=torch.bfloat16,
                             device="cpu", target_lm_head=tgt.lm_head)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        head.rank_to_hidden.weight.copy_(torch.randn(H, R, generator=g) * 0.1)
    Wt, U = _f64(head.target_lm_head.weight), _f64(head.rank_to_hidden.weight)
    head.fuse_target_lm_head_()
    want = oracle.bf16_round((Wt @ U).astype(np.float32))
    got = head.low_rank_lm_head.weight.detach().float().numpy()
    ulps = np.abs(oracle.f32_to_bf16_bits(got).astype(np.int32) - oracle.f32_to_bf16_bits(want).astype(np.int32))
    assert ulps.max() <= 1 and (ulps > 0).mean() < 0.05
    assert head.lm_head_mode == "low_rank" and head.rank_to_hidden is None and head.target_lm_head is None
    before = head.low_rank_lm_head.weight.clone()
    head.fuse_target_lm_head_()                              # no-op once folded
    assert torch.equal(head.low_rank_lm_head.weight, before)


# ------------------------------------------------------------------ f1: DeLS RNN head files

def test_dels_checkpoint_low_rank(pkg, tmp_path):
    sd = _rnn_state()
    sd["target_lm_head.weight"] = torch.zeros(V, H)          # frozen target copy: skipped
    path = _save(tmp_path, "local_head.pt", {"model_config": _config(shift_label=True), "model_state_dict": sd})
    head = pkg.DeLSLocalHead.from_checkpoint(checkpoint_path=path, target_model=_Target(), dtype=torch.float32,
                                             device="cpu")
    for k in ("prefix_gru.weight_ih_l0", "prefix_gru.weight_hh_l0", "rank_proj.weight", "low_rank_lm_head.weight"):
        assert torch.equal(head.state_dict()[k], sd[k]), k
    assert head.pure_draft_prefix_len == 1 and head.shift_label is True
    assert head.rank_activation == "silu" and head.lm_head_mode == "low_rank"
    assert pkg.detect_local_head_checkpoint_kind(path) == "dels"


def test_dels_checkpoint_target_lm_head_is_folded(pkg, tmp_path):
    tgt = _Target()
    sd = _rnn_state(lm_head=False, up=True)
    path = _save(tmp_path, "local_head.pt", {"model_config": _config(lm_head_mode="target_lm_head"),
                                             "model_state_dict": sd})
    head = pkg.DeLSLocalHead.from_checkpoint(checkpoint_path=path, target_model=tgt, dtype=torch.float32,
                                             device="cpu")
    want = _f64(tgt.lm_head.weight) @ _f64(sd["rank_to_hidden.weight"])
    np.testing.assert_allclose(head.low_rank_lm_head.weight.detach().numpy(), want, rtol=1e-5, atol=1e-6)
    assert head.lm_head_mode == "low_rank"


def test_dels_checkpoint_merged_lm_head(pkg, tmp_path):
    sd = _rnn_state(lm_head=False, up=True)
    merged = torch.randn(V, R, generator=torch.Generator().manual_seed(9))
    path = _save(tmp_path, "local_head.pt", {"model_config": _config(lm_head_mode="target_lm_head"),
                                             "model_state_dict": sd})
    for payload in ({"weight": merged}, merged):
        mpath = _save(tmp_path, "merged_lm_head.pt", payload)
        head = pkg.DeLSLocalHead.from_checkpoint(checkpoint_path=path, target_model=_Target(), dtype=torch.float32,
                                                 device="cpu", merged_lm_head_path=mpath)
        assert torch.equal(head.low_rank_lm_head.weight, merged) and head.lm_head_mode == "low_rank"


def test_dels_checkpoint_direct_vocab(pkg, tmp_path):
    sd = _rnn_state()
    sd["embed_tokens.weight"] = torch.randn(V, E, generator=torch.Generator().manual_seed(3))
    for cfg in (_config(rnn_parameterization="direct_vocab"), _config(architecture="direct_vocab_rnn")):
        path = _save(tmp_path, "merged_rnn_local_head.pt", {"model_config": cfg, "model_state_dict": sd})
        tgt = _Target()
        head = pkg.DeLSLocalHead.from_checkpoint(checkpoint_path=path, target_model=tgt, dtype=torch.float32,
                                                 device="cpu")
        assert torch.equal(head.embed_tokens.weight, sd["embed_tokens.weight"])
        assert head.embed_tokens is not tgt.model.embed_tokens and head.pure_draft_prefix_len == 0
    no_emb = {k: v for k, v in sd.items() if k != "embed_tokens.weight"}
    path = _save(tmp_path, "bad.pt", {"model_config": _config(rnn_parameterization="direct_vocab"),
                                      "model_state_dict": no_emb})
    with pytest.raises(ValueError, match="no embed_tokens.weight"):
        pkg.DeLSLocalHead.from_checkpoint(checkpoint_path=path, target_model=_Target(), dtype=torch.float32,
                                          device="cpu")


@pytest.mark.parametrize("mutate,msg", [
    (lambda sd: sd.update({"embed_down_proj.weight": torch.zeros(E, H)}), "embed_down_proj"),
    (lambda sd: sd.update({"extra.weight": torch.zeros(3)}), "Unexpected local-head tensor extra.weight"),
    (lambda sd: sd.update({"rank_proj.weight": torch.zeros(R + 1, G)}), "Unexpected local-head tensor"),
    (lambda sd: sd.pop("rank_proj.weight"), "missing=\\['rank_proj.weight'\\]"),
])
def test_dels_checkpoint_errors(pkg, tmp_path, mutate, msg):
    sd = _rnn_state()
    mutate(sd)
    path = _save(tmp_path, "local_head.pt", {"model_config": _config(), "model_state_dict": sd})
    with pytest.raises(ValueError, match=msg):
        pkg.DeLSLocalHead.from_checkpoint(checkpoint_path=path, target_model=_Target(), dtype=torch.float32,
                                          device="cpu")
    path = _save(tmp_path, "no_config.pt", {"model_state_dict": sd})
    with pytest.raises(ValueError, match="model_config and model_state_dict"):
        pkg.DeLSLocalHead.from_checkpoint(checkpoint_path=path, target_model=_Target(), dtype=torch.float32,
                                          device="cpu")


class _Opaque:
    """An object torch.load(weights_only=True) refuses to rebuild."""


def test_checkpoints_are_read_without_unpickling_code(pkg, tmp_path):
    path = _save(tmp_path, "local_head.pt", {"model_config": _Opaque(), "model_state_dict": _rnn_state()})
    with pytest.raises(ValueError, match="weights_only=True"):
        pkg.detect_local_head_checkpoint_kind(path)
    with pytest.raises(ValueError, match="weights_only=True"):
        pkg.DeLSLocalHead.from_checkpoint(checkpoint_path=path, target_model=_Target(), dtype=torch.float32,
                                          device="cpu")


def test_detect_checkpoint_kind(pkg, tmp_path):
    cases = {
        "dels_gru_keys.pt": ({"model_config": {}, "model_state_dict": _rnn_state()}, "dels"),
        "dels_config.pt": ({"model_config": _config(), "model_state_dict": {}}, "dels"),
        "markov_factored.pt": ({"model_config": {"rank": R},
                                "model_state_dict": {"down_proj": torch.zeros(E, R), "up_proj": torch.zeros(R, H),
                                                     "prefix_gru.x": torch.zeros(1)}}, "markov"),
        "markov_merged.pt": ({"embedding_weight": torch.zeros(V, R), "lm_head_weight": torch.zeros(V, R)}, "markov"),
    }
    for name, (payload, kind) in cases.items():
        assert pkg.detect_local_head_checkpoint_kind(_save(tmp_path, name, payload)) == kind, name
    with pytest.raises(ValueError, match="Cannot identify local-head checkpoint type"):
        pkg.detect_local_head_checkpoint_kind(_save(tmp_path, "other.pt", {"weights": torch.zeros(2)}))


# ------------------------------------------------------------------ f2's head: Markov files

def test_markov_checkpoints(pkg, tmp_path):
    tgt = _Target()
    g = torch.Generator().manual_seed(11)
    emb, lm = torch.randn(V, R, generator=g), torch.randn(V, R, generator=g)
    merged = pkg.MarkovDeLSLocalHead.from_checkpoint(
        checkpoint_path=_save(tmp_path, "merged_markov_local_head.pt", {"embedding_weight": emb,
                                                                        "lm_head_weight": lm}),
        target_model=tgt, dtype=torch.float32, device="cpu")
    assert torch.equal(merged.embedding_weight, emb) and torch.equal(merged.lm_head_weight, lm)
    assert merged.vocab_size == V and merged.rank == R
    tok = torch.tensor([[3], [7]])
    np.testing.assert_allclose(merged.logits_from_token(tok).detach().numpy(),
                               (_f64(emb)[tok.numpy()] @ _f64(lm).T), rtol=1e-5, atol=1e-5)
    down, up = torch.randn(E, R, generator=g), torch.randn(R, H, generator=g)
    fact = pkg.MarkovDeLSLocalHead.from_checkpoint(
        checkpoint_path=_save(tmp_path, "markov_local_head.pt", {"model_config": {"rank": R},
                                                                 "model_state_dict": {"down_proj": down,
                                                                                      "up_proj": up}}),
        target_model=tgt, dtype=torch.float32, device="cpu")
    np.testing.assert_allclose(fact.embedding_weight.detach().numpy(), _f64(tgt.model.embed_tokens.weight) @ _f64(down),
                               rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(fact.lm_head_weight.detach().numpy(), _f64(tgt.lm_head.weight) @ _f64(up).T,
                               rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError, match="Unexpected Markov rank"):
        pkg.MarkovDeLSLocalHead.from_checkpoint(
            checkpoint_path=_save(tmp_path, "m2.pt", {"model_config": {"rank": R + 1},
                                                      "model_state_dict": {"down_proj": down, "up_proj": up}}),
            target_model=tgt, dtype=torch.float32, device="cpu")
    with pytest.raises(ValueError, match="down_proj and up_proj"):
        pkg.MarkovDeLSLocalHead.from_checkpoint(
            checkpoint_path=_save(tmp_path, "m3.pt", {"model_config": {}, "model_state_dict": {"down_proj": down}}),
            target_model=tgt, dtype=torch.float32, device="cpu")
    with pytest.raises(ValueError, match="rank mismatch"):
        pkg.MarkovDeLSLocalHead(embedding_weight=emb, lm_head_weight=lm[:, :-1], dtype=torch.float32, device="cpu")


# ------------------------------------------------------------------ a12: position-mix joint head

def _position_ckpt(gates, baseline, *, up=False, **cfg):
    sd = _rnn_state(lm_head=not up, up=up, prefix="local_head_model.")
    sd["local_head_model.embed_tokens.weight"] = torch.zeros(V, E)     # frozen target copy
    sd["position_gates"] = gates
    sd["baseline_logits"] = baseline
    sd["trainer_step"] = torch.tensor(7)                                # training-only state
    c = {"method": "block_prefix_position_mix_joint",
         "local_head_config": _config(lm_head_mode="target_lm_head" if up else "low_rank")}
    c.update(cfg)
    return {"model_config": c, "model_state_dict": sd}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_position_mix_gates_are_the_schedules(pkg, tmp_path, dtype):
    """alpha_beta_schedules() returns the gates' columns as the runner's alpha/beta
    (code/dels.py:612-615); baseline_logits is the persistent [1, 1, V] buffer."""
    g = torch.Generator().manual_seed(21)
    gates = torch.rand(14, 2, generator=g) * 0.6
    baseline = torch.log_softmax(torch.randn(V, generator=g), 0)
    path = _save(tmp_path, "block_prefix_position_mix_joint.pt", _position_ckpt(gates, baseline))
    head = pkg.PositionMixJointHead.from_checkpoint(checkpoint_path=path, target_model=_Target(), block_size=16,
                                                    dtype=dtype, device="cpu")
    alphas, betas = head.alpha_beta_schedules()
    assert len(alphas) == len(betas) == 14
    np.testing.assert_array_equal(np.array(alphas, np.float32), gates[:, 0].to(dtype).float().numpy())
    np.testing.assert_array_equal(np.array(betas, np.float32), gates[:, 1].to(dtype).float().numpy())
    assert head.baseline_logits.shape == (1, 1, V) and head.baseline_logits.dtype == dtype
    assert torch.equal(head.baseline_logits.reshape(-1), baseline.to(dtype))
    assert "baseline_logits" in head.state_dict()                       # persistent buffer
    assert head.rnn_input == "block_prefix" and head.pure_draft_prefix_len == 1
    # the schedules drive a runner's argument checks as lists of the right length
    assert pkg.parse_scalar_schedule(alphas, 14, name="DeLS alpha") == alphas


def test_position_mix_suffix_length_and_fold(pkg, tmp_path):
    tgt = _Target()
    gates = torch.rand(15, 2)
    path = _save(tmp_path, "p.pt", _position_ckpt(gates, torch.zeros(V), up=True, dflash_shift_label=True))
    head = pkg.PositionMixJointHead.from_checkpoint(checkpoint_path=path, target_model=tgt, block_size=16,
                                                    dtype=torch.float32, device="cpu")
    assert head.position_gates.shape == (15, 2) and head.shift_label     # shifted labels: block - 1 positions
    sd = torch.load(path, weights_only=True)["model_state_dict"]
    want = _f64(tgt.lm_head.weight) @ _f64(sd["local_head_model.rank_to_hidden.weight"])
    np.testing.assert_allclose(head.low_rank_lm_head.weight.detach().numpy(), want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("cfg,block,msg", [
    (dict(method="other"), 16, "Only block_prefix_position_mix_joint"),
    (dict(rnn_input="tokens"), 16, "Only block_prefix position-joint"),
    (dict(), 2, "no suffix positions"),
])
def test_position_mix_errors(pkg, tmp_path, cfg, block, msg):
    path = _save(tmp_path, "p.pt", _position_ckpt(torch.zeros(14, 2), torch.zeros(V), **cfg))
    with pytest.raises(ValueError, match=msg):
        pkg.PositionMixJointHead.from_checkpoint(checkpoint_path=path, target_model=_Target(), block_size=block,
                                                 dtype=torch.float32, device="cpu")
    ck = _position_ckpt(torch.zeros(14, 2), torch.zeros(V))
    del ck["model_state_dict"]["baseline_logits"]
    with pytest.raises(ValueError, match="missing baseline_logits"):
        pkg.PositionMixJointHead.from_checkpoint(checkpoint_path=_save(tmp_path, "q.pt", ck),
                                                 target_model=_Target(), block_size=16, dtype=torch.float32,
                                                 device="cpu")
    ck = _position_ckpt(torch.zeros(14, 2), torch.zeros(V))
    ck["model_state_dict"]["local_head_model.rank_to_hidden.weight"] = torch.zeros(H, R)
    with pytest.raises(ValueError, match="Unexpected rank_to_hidden.weight"):
        pkg.PositionMixJointHead.from_checkpoint(checkpoint_path=_save(tmp_path, "r.pt", ck),
                                                 target_model=_Target(), block_size=16, dtype=torch.float32,
                                                 device="cpu")

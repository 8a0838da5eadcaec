"""CPU tests of the C ABI (load + exports + argument checking) and the host-side logic.

No kernel is launched here: every C-ABI call below fails its argument checks
(or only computes a workspace size) before touching the GPU.
"""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

import oracle

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "dels.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(dels_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_header_symbol(pkg):
    lib = pkg._lib.load()
    names = header_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), n
        assert n in pkg._lib.SIGNATURES, n
    assert set(pkg._lib.SIGNATURES) == set(names)


def test_rollout_struct_layout_matches_header(pkg):
    text = open(HEADER).read()
    body = re.search(r"typedef struct dels_rollout \{(.*?)\} dels_rollout;", text, flags=re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        names = decl.split()[-1] if "," not in decl else decl
        if "," in decl:
            first = re.match(r"[\w\s\*]+?\b(\w+)\s*,", decl)
            rest = re.findall(r",\s*\*?(\w+)", decl)
            fields += [first.group(1)] + rest
        else:
            fields.append(names.lstrip("*"))
    assert [f for f, _ in pkg._lib.RolloutParams._fields_] == fields


def test_abi_version_and_strerror(pkg):
    lib = pkg._lib.load()
    assert lib.dels_abi_version() == pkg._lib.ABI_VERSION == 3
    assert lib.dels_strerror(0) == b"success"
    assert lib.dels_strerror(-3) == b"misaligned operand"
    assert lib.dels_strerror(-99) == b"unknown status"


def test_workspace_sizes(pkg):
    lib = pkg._lib.load()
    assert lib.dels_fused_argmax_ws_bytes(16, 512, 151936) >= 256 + 16 * 8
    w = lib.dels_lowrank_argmax_ws_bytes(16, 4096, 512, 151936)
    assert w >= lib.dels_fused_argmax_ws_bytes(16, 512, 151936) + 16 * 512 * 2
    assert w % 256 == 0
    assert lib.dels_rollout_ws_bytes(8, 1024, 512, 151936) >= lib.dels_gru_step_ws_bytes(8, 1024)
    # every layout starts with the 64 KiB control area, the 544 KiB that only
    # the fused decode step writes and the 144 KiB that only the one-launch
    # rollout writes, so one workspace serves every entry point
    reserved = 65536 + 544 * 1024 + 144 * 1024
    assert lib.dels_fused_argmax_ws_bytes(1, 8, 1) == reserved
    assert lib.dels_argmax_rows_ws_bytes(1, 1) == reserved
    for n in (lib.dels_rank_proj_ws_bytes(1, 64, 64), lib.dels_gru_step_ws_bytes(1, 64),
              lib.dels_lowrank_argmax_ws_bytes(1, 64, 64, 100), lib.dels_rollout_ws_bytes(1, 64, 64, 100),
              lib.dels_fused_argmax_fp8_ws_bytes(64, 128, 100), lib.dels_lowrank_argmax_fp8_ws_bytes(1, 64, 128, 100)):
        assert n >= reserved and n % 256 == 0


def test_argument_errors_return_codes(pkg):
    lib = pkg._lib.load()
    # NULL operands
    rc = lib.dels_fused_argmax(None, 512, None, 512, 0, None, 100, 0, None, 0, None, 0, None, 0, 16, 512, 100,
                               None, None, 1, None, 0, None)
    assert rc == -1 and b"rank is NULL" in lib.dels_last_error()
    # unsupported rank dimension
    rc = lib.dels_fused_argmax(None, 0, None, 0, 0, None, 0, 0, None, 0, None, 0, None, 0, 4, 1024, 100,
                               None, None, 1, None, 0, None)
    assert rc == -2
    # misaligned operand (a fake, never-dereferenced address)
    rc = lib.dels_fused_argmax(0x1002, 64, 0x2000, 64, 0, 0x3000, 100, 0, None, 0, 0x4000, 0, 0x4000, 0, 2, 64,
                               100, 0x5000, None, 1, 0x6000, 4096, None)
    assert rc == -3
    # workspace too small
    rc = lib.dels_fused_argmax(0x1000, 64, 0x2000, 64, 0, 0x3000, 100, 0, None, 0, 0x4000, 0, 0x4000, 0, 2, 64,
                               100, 0x5000, None, 1, 0x6000, 16, None)
    assert rc == -4 and b"too small" in lib.dels_last_error()
    # bad base dtype
    rc = lib.dels_fused_argmax(0x1000, 64, 0x2000, 64, 0, 0x3000, 100, 7, None, 0, 0x4000, 0, 0x4000, 0, 2, 64,
                               100, 0x5000, None, 1, 0x6000, 4096, None)
    assert rc == -1
    # GRU: aliasing in/out, batch too large
    rc = lib.dels_gru_step(0x1000, 96, 10, 0x2000, 1, 0x3000, 32, 0x4000, 0, None, 2, 32, 0x3000, 32, 0x5000,
                           1 << 20, None)
    assert rc == -1 and b"alias" in lib.dels_last_error()
    rc = lib.dels_gru_step(0x1000, 96, 10, 0x2000, 1, 0x3000, 32, 0x4000, 0, None, 65, 32, 0x6000, 32, 0x5000,
                           1 << 20, None)
    assert rc == -2
    # rollout: NULL params, steps <= 0
    assert lib.dels_rollout_enqueue(None, None) == -1
    p = pkg._lib.RolloutParams()
    p.steps = 0
    assert lib.dels_rollout_enqueue(ctypes.byref(p), None) == -1
    assert b"steps > 0" in lib.dels_last_error()
    h = ctypes.c_void_p()
    assert lib.dels_graph_create(ctypes.byref(p), ctypes.byref(h)) == -1 and not h.value
    # output rows closer than steps apart, or a negative prefix stride, are refused
    p2 = pkg._lib.RolloutParams()
    p2.steps, p2.batch, p2.r, p2.V, p2.G, p2.act = 4, 2, 64, 100, 64, 0
    p2.ld_out = 3
    assert lib.dels_rollout_enqueue(ctypes.byref(p2), None) == -1 and b"ld_out" in lib.dels_last_error()
    p2.ld_out, p2.ld_prefix = 0, -1
    assert lib.dels_rollout_enqueue(ctypes.byref(p2), None) == -1 and b"ld_prefix" in lib.dels_last_error()
    assert lib.dels_graph_launch(None, None) == -1
    assert lib.dels_graph_destroy(None) == 0
    # unknown weight layout; packing into a too-small buffer
    rc = lib.dels_fused_argmax(0x1000, 64, 0x2000, 64, 7, 0x3000, 100, 0, None, 0, 0x4000, 0, 0x4000, 0, 2, 64,
                               100, 0x5000, None, 1, 0x6000, 1 << 16, None)
    assert rc == -1 and b"layout" in lib.dels_last_error()
    assert lib.dels_packed_bytes(17, 40) == 2 * 2 * 1024
    assert lib.dels_pack_operand(0x1000, 40, 17, 40, 0x8000, 1024, None) == -1
    # Domino step: an unknown middle layer code (DELS_MIDDLE_*) is refused before any operand is read
    for bad in (-1, 7):
        rc = lib.dels_domino_argmax(0x1000, 64, 0x2000, 64, 0x3000, None, 0, 0x4000, 100, 0, 1.0, bad, 2, 64, 100,
                                    0x5000, None, 1, 0x6000, 1 << 20, None)
        assert rc == -1 and b"middle layer" in lib.dels_last_error()
    q = pkg._lib.DominoRolloutParams()
    q.steps, q.batch, q.prefix_len, q.middle = 1, 1, 1, 9
    assert lib.dels_domino_rollout_enqueue(ctypes.byref(q), None) != 0


def test_python_errors_before_the_gpu(pkg):
    with pytest.raises(ValueError, match="no CPU fallback"):
        pkg.fused_argmax(torch.zeros(2, 64, dtype=torch.bfloat16), torch.zeros(10, 64, dtype=torch.bfloat16),
                         torch.zeros(2, 10))
    with pytest.raises(ValueError, match="Unsupported DeLS rank_activation"):
        pkg.lowrank_argmax(torch.zeros(2, 64), None, None, None, act="tanh")


# ------------------------------------------------------------------ schedules and prior

def test_parse_scalar_schedule(pkg):
    p = pkg.parse_scalar_schedule
    assert p("0.3", 4, name="a") == [0.3] * 4
    assert p(0.5, 3, name="a") == [0.5] * 3
    assert p(1, 2, name="a") == [1.0, 1.0]
    assert p("0.1, 0.2,0.3", 3, name="a") == [0.1, 0.2, 0.3]
    assert p([0.1, 0.2], 2, name="a") == [0.1, 0.2]
    assert p("0.1,,0.2,", 2, name="a") == [0.1, 0.2]
    with pytest.raises(ValueError, match="DeLS alpha schedule cannot be empty."):
        p(" , ", 3, name="DeLS alpha")
    with pytest.raises(ValueError, match=r"DeLS beta schedule length must be 1 or 3, got 2\."):
        p("0.1,0.2", 3, name="DeLS beta")


def test_prior_matches_oracle_and_files(pkg, tmp_path):
    counts = torch.tensor([5.0, 0.0, 1.0, 12.0])
    for s in (1.0, 0.5, 0.0):
        got = pkg.unigram_log_prior_from_counts(counts, 6, s).numpy()
        np.testing.assert_allclose(got, oracle.unigram_log_prior(counts.numpy(), 6, s), rtol=0, atol=1e-12)
    ref = oracle.unigram_log_prior(counts.numpy(), 6, 1.0)
    torch.save({"counts": counts}, tmp_path / "a.pt")
    torch.save(counts, tmp_path / "b.pt")
    np.savez(tmp_path / "c.npz", counts=counts.numpy())
    (tmp_path / "d").mkdir()
    np.savez(tmp_path / "d" / "loss_mask_unigram.npz", counts=counts.numpy())
    for name in ("a.pt", "b.pt", "c.npz", "d"):
        t = pkg.load_unigram_log_prior(str(tmp_path / name), vocab_size=6, dtype=torch.float32, device="cpu")
        assert t.shape == (1, 1, 6)
        np.testing.assert_allclose(t.reshape(-1).numpy(), ref.astype(np.float32), rtol=1e-6)
    with pytest.raises(ValueError, match="must contain"):
        (tmp_path / "e").mkdir()
        pkg.load_unigram_log_prior(str(tmp_path / "e"), vocab_size=6, dtype=torch.float32, device="cpu")
    with pytest.raises(ValueError, match="exceeds runtime vocab"):
        pkg.load_unigram_log_prior(str(tmp_path / "a.pt"), vocab_size=2, dtype=torch.float32, device="cpu")
    with pytest.raises(ValueError, match="expected .pt, .npz"):
        pkg.load_unigram_log_prior(str(tmp_path / "x.bin"), vocab_size=6, dtype=torch.float32, device="cpu")


def test_zipf_prior_is_a_normalised_permutation(pkg):
    lp = pkg.synth.zipf_log_prior(1000).numpy()
    assert abs(np.exp(lp).sum() - 1) < 1e-12
    k = np.arange(1, 1001, dtype=np.float64)
    expect = np.sort(np.log(np.round(1e9 * k ** -1.1) + 1) - np.log((np.round(1e9 * k ** -1.1) + 1).sum()))
    np.testing.assert_allclose(np.sort(lp), expect, rtol=1e-12)
    assert not np.all(np.diff(lp) <= 0)     # permuted, not index-monotone


# ------------------------------------------------------------------ runner argument checks

class _Head:
    rank_activation = "identity"


@pytest.mark.parametrize("kwargs,msg", [
    (dict(steps=0), "requires steps > 0, got 0"),
    (dict(alpha_values=[0.1]), r"alpha/beta schedules must match steps: steps=3, alpha=1, beta=3"),
    (dict(beta_values=[0.0, 0.2, 0.0], baseline_logits=None), "requires baseline_logits when any beta is nonzero"),
    (dict(device="cpu"), "no CPU fallback"),
])
def test_runner_argument_checks(pkg, kwargs, msg):
    args = dict(local_head=_Head(), batch_size=1, steps=3, vocab_size=10, alpha_values=[0.1] * 3,
                beta_values=[0.0] * 3, baseline_logits=None, device="cuda")
    args.update(kwargs)
    with pytest.raises(ValueError, match=msg):
        pkg.DeLSGraphRunner(**args)


class _MarkovHead:
    vocab_size = 10
    embedding_weight = None
    lm_head_weight = None


@pytest.mark.parametrize("kwargs,msg", [
    (dict(steps=0, alpha_values=[], beta_values=[]), "requires steps > 0"),
    (dict(alpha_values=[0.1]), "alpha/beta schedules must match steps"),
    (dict(vocab_size=11), "local-head vocab size mismatch"),
    (dict(beta_values=[0.0, 0.2, 0.0], baseline_logits=None), "requires baseline_logits when any beta is nonzero"),
    (dict(device="cpu"), "no CPU fallback"),
])
def test_markov_runner_argument_checks(pkg, kwargs, msg):
    """MarkovDeLSGraphRunner's checks (code/kernel/markov_dels.py:153-173) run before any device use."""
    args = dict(local_head=_MarkovHead(), batch_size=1, steps=3, vocab_size=10, alpha_values=[0.1] * 3,
                beta_values=[0.0] * 3, baseline_logits=None, device="cuda")
    args.update(kwargs)
    with pytest.raises(ValueError, match=msg):
        pkg.MarkovDeLSGraphRunner(**args)


def test_local_head_mirror_eager_methods(pkg):
    class Target:
        class model:
            embed_tokens = torch.nn.Embedding(50, 16)
        lm_head = torch.nn.Linear(16, 50, bias=False)

    head = pkg.DeLSLocalHead(target_model=Target, vocab_size=50, embed_dim=16, gru_hidden_dim=24, low_rank_dim=8,
                             lm_head_mode="low_rank", rank_activation="silu", dtype=torch.float32, device="cpu")
    h = head.init_empty_hidden(3, device="cpu")
    assert h.shape == (1, 3, 24)
    h = head.advance(torch.tensor([[1], [2], [3]]), h)
    logits = head.logits_from_hidden(h)
    assert logits.shape == (3, 1, 50)
    with pytest.raises(ValueError, match="rank_activation='tanh'"):
        pkg.DeLSLocalHead(target_model=Target, vocab_size=50, embed_dim=16, gru_hidden_dim=24, low_rank_dim=8,
                          lm_head_mode="low_rank", rank_activation="tanh", dtype=torch.float32, device="cpu")


def test_golden_fixtures_reproduce_from_oracle():
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(REPO, "tests", "golden",
                                                                              "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    for name, make in mg.CASES.items():
        want = np.load(os.path.join(REPO, "tests", "golden", name))
        got = make()
        assert set(want.files) == set(got), name
        for k in want.files:
            np.testing.assert_array_equal(want[k], got[k], err_msg=f"{name}:{k}")

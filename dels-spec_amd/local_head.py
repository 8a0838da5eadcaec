"""Host-side helpers and the local-head module the DeLS runner consumes.

Mirrors the reference's interface in code/dels.py (paths relative to the
dt-3t/DeLS-Spec repository): ``parse_scalar_schedule`` (93-112),
``load_unigram_log_prior`` (17-90), ``DeLSLocalHead`` (141-345) with its
eager ``init_empty_hidden`` / ``advance`` / ``logits_from_hidden`` methods,
``MarkovDeLSLocalHead`` (348-430) and ``PositionMixJointHead`` (433-621), each
with its ``from_checkpoint`` loader.  The modules are the weight containers
the graph runners read; their eager methods are plain torch, as in the
reference.
"""

from __future__ import annotations

from pathlib import Path
from typing import Iterable, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import checkpoints as ckpt_fmt

_VALID_RANK_ACTIVATIONS = {"identity", "silu"}


def parse_scalar_schedule(values: str | float | Iterable[float], steps: int, *, name: str) -> list[float]:
    """A scalar or comma-separated per-position schedule of length ``steps``.

    A single value is broadcast to every step; any other length than 1 or
    ``steps`` raises ``ValueError`` (code/dels.py:93-112).
    """
    if isinstance(values, str):
        parsed = [float(part.strip()) for part in values.split(",") if part.strip()]
    elif isinstance(values, (float, int)):
        parsed = [float(values)]
    else:
        parsed = [float(v) for v in values]
    if not parsed:
        raise ValueError(f"{name} schedule cannot be empty.")
    if len(parsed) == 1:
        parsed = parsed * steps
    if len(parsed) != steps:
        raise ValueError(f"{name} schedule length must be 1 or {steps}, got {len(parsed)}.")
    return parsed


def unigram_log_prior_from_counts(counts: torch.Tensor, vocab_size: int, smoothing: float = 1.0) -> torch.Tensor:
    """Normalised log unigram probabilities (float64, [vocab_size]) from counts.

    Zero-padded to ``vocab_size``.  ``smoothing > 0``: ``log(c+s) - log(sum(c+s))``;
    ``smoothing == 0``: unseen tokens take the smallest seen log-probability
    (code/dels.py:66-88).
    """
    if smoothing < 0:
        raise ValueError("smoothing must be non-negative.")
    counts = counts.detach().to("cpu", torch.float64).reshape(-1)
    if counts.numel() > vocab_size:
        raise ValueError(
            f"Unigram baseline vocab size {counts.numel()} exceeds runtime vocab size {vocab_size}.")
    if counts.numel() < vocab_size:
        padded = torch.zeros(vocab_size, dtype=torch.float64)
        padded[: counts.numel()] = counts
        counts = padded
    if smoothing == 0.0:
        nonzero = counts > 0
        if not bool(nonzero.any()):
            raise ValueError("Unigram baseline has no positive counts.")
        log_prior = torch.full_like(counts, float("-inf"))
        log_prior[nonzero] = torch.log(counts[nonzero]) - torch.log(counts.sum())
        log_prior[~nonzero] = log_prior[nonzero].min()
        return log_prior
    smoothed = counts + float(smoothing)
    return torch.log(smoothed) - torch.log(smoothed.sum())


def load_unigram_log_prior(path: str, *, vocab_size: int, dtype: torch.dtype, device: torch.device,
                           smoothing: float = 1.0) -> torch.Tensor:
    """Load a finite full-vocab log unigram prior as ``[1, 1, vocab_size]``.

    Accepts a ``.pt`` file (a tensor or a dict with ``"counts"``), an ``.npz``
    with ``counts``, or a directory holding ``loss_mask_unigram.pt`` /
    ``loss_mask_unigram.npz`` (code/dels.py:17-90).  ``.pt`` files are read
    with ``weights_only=True``.
    """
    if smoothing < 0:
        raise ValueError("smoothing must be non-negative.")
    stat_path = Path(path)
    if stat_path.is_dir():
        pt_path = stat_path / "loss_mask_unigram.pt"
        npz_path = stat_path / "loss_mask_unigram.npz"
        if pt_path.exists():
            stat_path = pt_path
        elif npz_path.exists():
            stat_path = npz_path
        else:
            raise ValueError(
                f"Unigram baseline directory {path!r} must contain "
                "loss_mask_unigram.pt or loss_mask_unigram.npz.")
    if stat_path.suffix == ".pt":
        stats = torch.load(stat_path, map_location="cpu", weights_only=True)
        if isinstance(stats, dict) and "counts" in stats:
            counts = stats["counts"]
        elif torch.is_tensor(stats):
            counts = stats
        else:
            raise ValueError(
                f"Unsupported unigram baseline .pt payload in {stat_path}: "
                "expected a tensor or a dict with key 'counts'.")
    elif stat_path.suffix == ".npz":
        import numpy as np

        with np.load(stat_path, allow_pickle=False) as stats:
            if "counts" not in stats.files:
                raise ValueError(f"Unigram baseline npz {stat_path} has no 'counts'.")
            counts = torch.from_numpy(np.array(stats["counts"]))
    else:
        raise ValueError(f"Unsupported unigram baseline path {stat_path}; expected .pt, .npz, or a directory.")
    log_prior = unigram_log_prior_from_counts(counts, vocab_size, smoothing)
    return log_prior.to(device=device, dtype=dtype).view(1, 1, vocab_size)


class DeLSLocalHead(nn.Module):
    """RNN local head: GRU over token embeddings, rank projection, low-rank LM head.

    Same constructor arguments, attributes and eager methods as the
    reference's inference module (code/dels.py:141-206, 307-345), and the
    checkpoint loader ``from_checkpoint`` (code/dels.py:208-305; the formats are
    described in ``checkpoints``).
    """

    def __init__(self, *, target_model: nn.Module, vocab_size: int, embed_dim: int, gru_hidden_dim: int,
                 low_rank_dim: int, lm_head_mode: str, rank_activation: str = "identity",
                 dtype: torch.dtype, device: torch.device, target_lm_head: Optional[nn.Module] = None,
                 embedding_weight: Optional[torch.Tensor] = None):
        super().__init__()
        if rank_activation not in _VALID_RANK_ACTIVATIONS:
            raise ValueError(
                f"rank_activation={rank_activation!r}; must be one of {_VALID_RANK_ACTIVATIONS}")
        if embedding_weight is None:
            self.embed_tokens = target_model.model.embed_tokens
        else:
            expected_shape = (int(vocab_size), int(embed_dim))
            if tuple(embedding_weight.shape) != expected_shape:
                raise ValueError(
                    f"Local embedding shape {tuple(embedding_weight.shape)} does not match config {expected_shape}.")
            if target_model.lm_head.weight.shape[0] != int(vocab_size):
                raise ValueError("Local-head vocabulary does not match the target model.")
            self.embed_tokens = nn.Embedding.from_pretrained(
                embedding_weight.to(device=device, dtype=dtype), freeze=True)
        self.vocab_size = int(vocab_size)
        self.embed_dim = int(embed_dim)
        self.gru_hidden_dim = int(gru_hidden_dim)
        self.low_rank_dim = int(low_rank_dim)
        self.lm_head_mode = lm_head_mode
        self.rank_activation = rank_activation
        self.prefix_gru = nn.GRU(input_size=self.embed_dim, hidden_size=self.gru_hidden_dim, num_layers=1,
                                 batch_first=True, bias=False)
        self.rank_proj = nn.Linear(self.gru_hidden_dim, self.low_rank_dim, bias=False)
        self.low_rank_lm_head = nn.Linear(self.low_rank_dim, self.vocab_size, bias=False)
        self.rank_to_hidden = None
        self.target_lm_head = None
        if lm_head_mode == "target_lm_head":
            if target_lm_head is None:
                raise ValueError("target_lm_head is required for target_lm_head mode.")
            hidden_size = int(target_lm_head.weight.shape[1])
            self.rank_to_hidden = nn.Linear(self.low_rank_dim, hidden_size, bias=False)
            self.target_lm_head = target_lm_head
        self.to(device=device, dtype=dtype)
        self.eval()

    @classmethod
    def from_checkpoint(cls, *, checkpoint_path: str, target_model: nn.Module, dtype: torch.dtype,
                        device: torch.device, merged_lm_head_path: Optional[str] = None) -> "DeLSLocalHead":
        """Build the head from a SpecForge ``local_head.pt`` / ``merged_rnn_local_head.pt``
        (code/dels.py:208-305).

        The config gives the sizes, ``lm_head_mode`` and ``rank_activation``; a
        direct-vocab head brings its own token embedding, otherwise the target's
        is shared (a head trained with an input projection must be converted
        first).  ``merged_lm_head_path`` replaces the low-rank LM head with a
        merged ``[V, r]`` weight; a ``target_lm_head`` head without one is folded
        through the target LM head after loading.
        """
        ckpt = ckpt_fmt.read_checkpoint(checkpoint_path)
        config = ckpt.get("model_config") if isinstance(ckpt, dict) else None
        state = ckpt.get("model_state_dict") if isinstance(ckpt, dict) else None
        if config is None or state is None:
            raise ValueError("Local-head checkpoint must contain model_config and model_state_dict.")
        own_embedding = None
        if ckpt_fmt.direct_vocab(config):
            own_embedding = state.get("embed_tokens.weight")
            if own_embedding is None:
                raise ValueError("Direct-vocab RNN checkpoint has no embed_tokens.weight.")
        elif "embed_down_proj.weight" in state:
            raise ValueError(
                "This RNN checkpoint projects its input embeddings (embed_down_proj); convert it to "
                "merged_rnn_local_head.pt (SpecForge scripts/convert_local_head.py) before inference.")
        head = cls(target_model=target_model, vocab_size=int(config["vocab_size"]),
                   embed_dim=int(config["embed_dim"]), gru_hidden_dim=int(config["gru_hidden_dim"]),
                   low_rank_dim=int(config["low_rank_dim"]), lm_head_mode=config.get("lm_head_mode", "low_rank"),
                   rank_activation=config.get("rank_activation", "identity"), dtype=dtype, device=device,
                   target_lm_head=target_model.lm_head, embedding_weight=own_embedding)
        head.pure_draft_prefix_len = int(config.get("pure_draft_prefix_len", 0 if own_embedding is not None else 1))
        head.shift_label = bool(config.get("shift_label", False))

        own = head.state_dict()

        def rule(name, tensor):
            if name in own and tuple(own[name].shape) == tuple(tensor.shape):
                return ckpt_fmt.LOAD, name, tensor
            frozen = name.startswith(ckpt_fmt.FROZEN_TARGET_PREFIXES)
            if frozen and not (own_embedding is not None and name.startswith("embed_tokens.")):
                return ckpt_fmt.SKIP, name, tensor
            return "reject", name, tensor

        to_load, skipped = ckpt_fmt.map_state(state, own, rule, "local-head")
        if merged_lm_head_path is not None:
            merged = ckpt_fmt.read_checkpoint(merged_lm_head_path)
            weight = merged["weight"] if isinstance(merged, dict) else merged
            to_load["low_rank_lm_head.weight"] = weight.to(dtype=own["low_rank_lm_head.weight"].dtype)
            head.lm_head_mode = "low_rank"
        absent = list(ckpt_fmt.FROZEN_TARGET_PREFIXES)
        absent.append("rank_to_hidden." if head.lm_head_mode == "low_rank" else "low_rank_lm_head.")
        ckpt_fmt.load_mapped(head, to_load, may_be_absent=absent, what="Local-head", skipped=skipped)
        if head.lm_head_mode == "target_lm_head":
            head.fuse_target_lm_head_()
        return head

    @torch.inference_mode()
    def fuse_target_lm_head_(self) -> None:
        """Fold ``target_lm_head . rank_to_hidden`` into ``low_rank_lm_head`` (fp32, cast once)."""
        if self.lm_head_mode != "target_lm_head":
            return
        if self.rank_to_hidden is None or self.target_lm_head is None:
            raise ValueError("Cannot fuse local head without rank_to_hidden/target_lm_head.")
        target_weight = self.target_lm_head.weight.detach().to(torch.float32)
        up_weight = self.rank_to_hidden.weight.detach().to(torch.float32)
        fused = target_weight.matmul(up_weight).to(self.low_rank_lm_head.weight.dtype)
        self.low_rank_lm_head.weight.copy_(fused)
        self.rank_to_hidden = None
        self.target_lm_head = None
        self.lm_head_mode = "low_rank"

    @torch.inference_mode()
    def init_empty_hidden(self, batch_size: int, *, device: torch.device) -> torch.Tensor:
        return torch.zeros(1, batch_size, self.gru_hidden_dim, device=device, dtype=self.rank_proj.weight.dtype)

    @torch.inference_mode()
    def logits_from_hidden(self, hidden: torch.Tensor) -> torch.Tensor:
        rank_state = self.rank_proj(hidden.transpose(0, 1))
        if self.rank_activation == "silu":
            rank_state = F.silu(rank_state)
        return self.low_rank_lm_head(rank_state)

    @torch.inference_mode()
    def advance(self, token_ids: torch.Tensor, hidden: torch.Tensor) -> torch.Tensor:
        token_embeds = self.embed_tokens(token_ids)
        _, hidden = self.prefix_gru(token_embeds, hidden)
        return hidden


class MarkovDeLSLocalHead(nn.Module):
    """Dense Markov local head: the previous token's row of a merged embedding
    ``[V, R]`` is the rank state, scored against a merged LM head ``[V, R]``
    (code/dels.py:348-430).  Consumed by ``MarkovDeLSGraphRunner``."""

    def __init__(self, *, embedding_weight: torch.Tensor, lm_head_weight: torch.Tensor, dtype: torch.dtype,
                 device: torch.device):
        super().__init__()
        if embedding_weight.dim() != 2 or lm_head_weight.dim() != 2:
            raise ValueError("Markov DeLS weights must be rank-2 tensors.")
        if embedding_weight.shape[1] != lm_head_weight.shape[1]:
            raise ValueError(
                "Markov DeLS merged embedding/lm-head rank mismatch: "
                f"embedding={tuple(embedding_weight.shape)}, lm_head={tuple(lm_head_weight.shape)}")
        self.embedding_weight = nn.Parameter(embedding_weight.to(device=device, dtype=dtype), requires_grad=False)
        self.lm_head_weight = nn.Parameter(lm_head_weight.to(device=device, dtype=dtype), requires_grad=False)
        self.vocab_size = int(lm_head_weight.shape[0])
        self.rank = int(lm_head_weight.shape[1])
        self.eval()

    @classmethod
    def from_checkpoint(cls, *, checkpoint_path: str, target_model: nn.Module, dtype: torch.dtype,
                        device: torch.device) -> "MarkovDeLSLocalHead":
        """A merged file (``embedding_weight``/``lm_head_weight``) is used as is; a factored
        one (``down_proj [H, R]``, ``up_proj [R, H]`` in its state dict) is merged through
        the target's embedding and LM head in fp32: ``E_target . down`` and
        ``W_target . up^T`` (code/dels.py:381-426)."""
        ckpt = ckpt_fmt.read_checkpoint(checkpoint_path)
        if not isinstance(ckpt, dict):
            raise ValueError(f"{checkpoint_path}: a Markov checkpoint is a dict.")
        if "embedding_weight" in ckpt and "lm_head_weight" in ckpt:
            return cls(embedding_weight=ckpt["embedding_weight"], lm_head_weight=ckpt["lm_head_weight"], dtype=dtype,
                       device=device)
        config, state = ckpt.get("model_config"), ckpt.get("model_state_dict")
        if config is None or state is None:
            raise ValueError(
                "Markov DeLS checkpoint must be either merged_markov_local_head.pt or "
                "markov_local_head.pt from SpecForge scripts/train_markov_local_head.py.")
        if "down_proj" not in state or "up_proj" not in state:
            raise ValueError("Markov local-head checkpoint must contain down_proj and up_proj.")
        embedding = ckpt_fmt.fold_through_target_head(target_model.model.embed_tokens.weight, state["down_proj"],
                                                      torch.float32)
        lm_head = ckpt_fmt.fold_through_target_head(target_model.lm_head.weight, state["up_proj"].t(), torch.float32)
        rank = int(config.get("rank", state["down_proj"].shape[1]))
        if embedding.shape[1] != rank:
            raise ValueError(f"Unexpected Markov rank: merged={embedding.shape[1]}, config={rank}")
        return cls(embedding_weight=embedding, lm_head_weight=lm_head, dtype=dtype, device=device)

    @torch.inference_mode()
    def logits_from_token(self, token_ids: torch.Tensor) -> torch.Tensor:
        rank_states = F.embedding(token_ids, self.embedding_weight)
        return torch.matmul(rank_states, self.lm_head_weight.t())


class PositionMixJointHead(nn.Module):
    """Block-prefix position-mix joint head (code/dels.py:433-621): a DeLS RNN head
    (the attributes ``DeLSGraphRunner`` reads) plus learned per-position gates
    ``position_gates [suffix_len, 2]`` -- column 0 the alpha, column 1 the beta of
    each suffix position -- and the baseline log-prior it was trained with, kept as
    the persistent buffer ``baseline_logits [1, 1, V]``.  ``alpha_beta_schedules``
    hands the gates to the runner as its alpha/beta schedules."""

    def __init__(self, *, target_model: nn.Module, vocab_size: int, embed_dim: int, gru_hidden_dim: int,
                 low_rank_dim: int, suffix_len: int, shift_label: bool, rank_activation: str,
                 baseline_logits: torch.Tensor, dtype: torch.dtype, device: torch.device):
        super().__init__()
        if rank_activation not in _VALID_RANK_ACTIVATIONS:
            raise ValueError(
                f"rank_activation={rank_activation!r}; must be one of {_VALID_RANK_ACTIVATIONS}")
        self.embed_tokens = target_model.model.embed_tokens
        self.vocab_size = int(vocab_size)
        self.embed_dim = int(embed_dim)
        self.gru_hidden_dim = int(gru_hidden_dim)
        self.low_rank_dim = int(low_rank_dim)
        self.pure_draft_prefix_len = 1
        self.shift_label = bool(shift_label)
        self.rank_activation = rank_activation
        self.rnn_input = "block_prefix"
        self.mix_form = "block_prefix_position"
        self.prefix_gru = nn.GRU(input_size=self.embed_dim, hidden_size=self.gru_hidden_dim, num_layers=1,
                                 batch_first=True, bias=False)
        self.rank_proj = nn.Linear(self.gru_hidden_dim, self.low_rank_dim, bias=False)
        self.low_rank_lm_head = nn.Linear(self.low_rank_dim, self.vocab_size, bias=False)
        self.position_gates = nn.Parameter(torch.zeros(int(suffix_len), 2, dtype=dtype, device=device))
        self.register_buffer("baseline_logits", baseline_logits.to(device=device, dtype=dtype).view(1, 1, -1),
                             persistent=True)
        self.to(device=device, dtype=dtype)
        self.eval()

    @classmethod
    def from_checkpoint(cls, *, checkpoint_path: str, target_model: nn.Module, block_size: int,
                        dtype: torch.dtype, device: torch.device) -> "PositionMixJointHead":
        """Load a SpecForge ``block_prefix_position_mix_joint`` checkpoint (code/dels.py:489-604).

        The local head's tensors sit under ``local_head_model.``; the suffix has
        ``block_size - 2`` positions (``- 1`` when the DFlash labels are shifted);
        a ``rank_to_hidden`` head is folded through the target LM head.
        """
        ckpt = ckpt_fmt.read_checkpoint(checkpoint_path)
        config = ckpt.get("model_config") if isinstance(ckpt, dict) else None
        state = ckpt.get("model_state_dict") if isinstance(ckpt, dict) else None
        if config is None or state is None:
            raise ValueError("Block-prefix position checkpoint must contain model_config and model_state_dict.")
        if config.get("method") != "block_prefix_position_mix_joint":
            raise ValueError("Only block_prefix_position_mix_joint checkpoints are supported.")
        if config.get("rnn_input", "block_prefix") != "block_prefix":
            raise ValueError("Only block_prefix position-joint checkpoints are supported.")
        local = config.get("local_head_config")
        if local is None:
            raise ValueError("Checkpoint is missing local_head_config.")
        if "baseline_logits" not in state:
            raise ValueError("Block-prefix position checkpoint is missing baseline_logits.")
        shift_label = bool(config.get("dflash_shift_label", False))
        first_suffix = 1 if shift_label else 2
        suffix_len = int(block_size) - first_suffix
        if suffix_len <= 0:
            raise ValueError(
                "Block-prefix position checkpoint has no suffix positions: "
                f"block_size={block_size}, suffix_start={first_suffix}.")
        head = cls(target_model=target_model, vocab_size=int(local["vocab_size"]), embed_dim=int(local["embed_dim"]),
                   gru_hidden_dim=int(local["gru_hidden_dim"]), low_rank_dim=int(local["low_rank_dim"]),
                   suffix_len=suffix_len, shift_label=shift_label,
                   rank_activation=local.get("rank_activation", "identity"),
                   baseline_logits=state["baseline_logits"], dtype=dtype, device=device)
        own = head.state_dict()
        prefix = "local_head_model."

        def rule(name, tensor):
            if name.startswith(prefix):
                target = name[len(prefix):]
            elif name in ("position_gates", "baseline_logits"):
                target = name
            else:
                return ckpt_fmt.SKIP, name, tensor                 # training-only state
            if target.startswith(ckpt_fmt.FROZEN_TARGET_PREFIXES):
                return ckpt_fmt.SKIP, target, tensor
            if target == "baseline_logits":
                return ckpt_fmt.LOAD, target, tensor.reshape(own[target].shape)
            if target in own and tuple(own[target].shape) == tuple(tensor.shape):
                return ckpt_fmt.LOAD, target, tensor
            if target == "rank_to_hidden.weight":
                mode = local.get("lm_head_mode", "low_rank")
                if mode != "target_lm_head":
                    raise ValueError(
                        f"Unexpected rank_to_hidden.weight for block-prefix joint local lm_head_mode={mode!r}.")
                folded = ckpt_fmt.fold_through_target_head(target_model.lm_head.weight, tensor, torch.float32)
                return ckpt_fmt.LOAD, "low_rank_lm_head.weight", folded
            return "reject", target, tensor

        to_load, skipped = ckpt_fmt.map_state(state, own, rule, "block-prefix joint")
        ckpt_fmt.load_mapped(head, to_load, may_be_absent=ckpt_fmt.FROZEN_TARGET_PREFIXES,
                             what="Block-prefix position", skipped=skipped)
        return head

    @torch.inference_mode()
    def init_empty_hidden(self, batch_size: int, *, device: torch.device) -> torch.Tensor:
        return torch.zeros(1, batch_size, self.gru_hidden_dim, device=device, dtype=self.rank_proj.weight.dtype)

    @torch.inference_mode()
    def logits_from_hidden(self, hidden: torch.Tensor) -> torch.Tensor:
        rank_state = self.rank_proj(hidden.transpose(0, 1))
        if self.rank_activation == "silu":
            rank_state = F.silu(rank_state)
        return self.low_rank_lm_head(rank_state)

    @torch.inference_mode()
    def alpha_beta_schedules(self) -> tuple[list[float], list[float]]:
        """Per-suffix-position (alpha, beta): the gates' two columns, as Python floats
        (the stored gate values, read in fp32)."""
        gates = self.position_gates.detach().to(device="cpu", dtype=torch.float32)
        return gates[:, 0].tolist(), gates[:, 1].tolist()

    @torch.inference_mode()
    def advance(self, token_ids: torch.Tensor, hidden: torch.Tensor) -> torch.Tensor:
        token_embeds = self.embed_tokens(token_ids)
        _, hidden = self.prefix_gru(token_embeds, hidden)
        return hidden


"""Host-side helpers and the local-head module the DeLS runner consumes.

Mirrors the reference's interface in code/dels.py (paths relative to the
dt-3t/DeLS-Spec repository): ``parse_scalar_schedule`` (93-112),
``load_unigram_log_prior`` (17-90) and ``DeLSLocalHead`` (141-345) with its
eager ``init_empty_hidden`` / ``advance`` / ``logits_from_hidden`` methods.
The module is the weight container the graph runner reads; its eager methods
are plain torch, as in the reference.
"""

from __future__ import annotations

from pathlib import Path
from typing import Iterable, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

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
    reference's inference module (code/dels.py:141-206, 307-345); the
    checkpoint loader is not part of this module.
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

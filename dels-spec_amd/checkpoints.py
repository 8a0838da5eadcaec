"""Local-head checkpoint formats: kind detection and state-dict mapping.

The reference's runtime reads three kinds of SpecForge local-head files
(code/dels.py:115-138 detects them, 208-305, 381-426 and 489-604 load them):

* a DeLS RNN head -- ``{"model_config": {...}, "model_state_dict": {...}}``
  with ``prefix_gru.*``, ``rank_proj.*`` and either ``low_rank_lm_head.*`` or
  ``rank_to_hidden.*`` (folded into the target LM head); the direct-vocab
  variant carries its own ``embed_tokens.weight``;
* a Markov head -- either merged (top-level ``embedding_weight`` and
  ``lm_head_weight``) or factored (``down_proj``/``up_proj`` in the state dict,
  merged with the target's embedding and LM head);
* a block-prefix position-mix joint checkpoint -- a DeLS head under the
  ``local_head_model.`` prefix plus ``position_gates`` and ``baseline_logits``.

Every file is read with ``torch.load(..., weights_only=True)``: tensors and
plain containers only, nothing from the file is executed.  A checkpoint whose
payload needs arbitrary unpickling is refused with a ``ValueError``.

Here a checkpoint is mapped onto a module by one rule table per format: each
state-dict key becomes an action (load it, skip a frozen target tensor, fold
it into the LM head, or reject it), and ``load_mapped`` then loads what was
kept and checks that every tensor the module needs was provided.
"""

from __future__ import annotations

import pickle
from typing import Callable, Iterable, Literal, Optional

import torch
import torch.nn as nn

# Tensors of the target model that checkpoints may carry (frozen copies); they
# are never loaded from a local-head file.
FROZEN_TARGET_PREFIXES = ("embed_tokens.", "target_lm_head.")


def read_checkpoint(path: str):
    """The payload of a ``.pt`` file, loaded without executing anything from it."""
    try:
        return torch.load(path, map_location="cpu", weights_only=True)
    except pickle.UnpicklingError as exc:
        raise ValueError(
            f"{path}: the checkpoint holds objects other than tensors and plain containers, and is "
            f"not loaded (only weights_only=True loading is allowed): {exc}") from exc


def _dict_or_none(x):
    return x if isinstance(x, dict) else None


def detect_local_head_checkpoint_kind(checkpoint_path: str) -> Literal["dels", "markov"]:
    """``"dels"`` or ``"markov"`` for a SpecForge local-head file (code/dels.py:115-138).

    Evidence is taken in this order: a factored Markov state dict
    (``down_proj`` and ``up_proj``), GRU weights (``prefix_gru.*``), a config
    naming a GRU hidden size, a merged Markov payload (top-level
    ``embedding_weight`` and ``lm_head_weight``).
    """
    ckpt = read_checkpoint(checkpoint_path)
    if not isinstance(ckpt, dict):
        raise ValueError(f"{checkpoint_path}: a local-head checkpoint is a dict, got {type(ckpt).__name__}.")
    sd = _dict_or_none(ckpt.get("model_state_dict"))
    cfg = _dict_or_none(ckpt.get("model_config"))
    checks: list[tuple[bool, str]] = [
        (sd is not None and "down_proj" in sd and "up_proj" in sd, "markov"),
        (sd is not None and any(k.startswith("prefix_gru.") for k in sd), "dels"),
        (cfg is not None and "gru_hidden_dim" in cfg, "dels"),
        ("embedding_weight" in ckpt and "lm_head_weight" in ckpt, "markov"),
    ]
    for hit, kind in checks:
        if hit:
            return kind  # type: ignore[return-value]
    raise ValueError(
        "Cannot identify local-head checkpoint type. Expected a SpecForge "
        "local_head.pt, merged_rnn_local_head.pt, markov_local_head.pt, "
        "or merged_markov_local_head.pt.")


# ---- mapping a state dict onto a module ------------------------------------------

LOAD, SKIP = "load", "skip"


def map_state(state_dict: dict, own_state: dict, rule: Callable[[str, torch.Tensor], tuple],
              what: str) -> tuple[dict, list]:
    """Apply ``rule(name, tensor) -> (action, target_name, tensor)`` to every entry.

    ``LOAD`` entries are cast to the module's dtype (and must match its shape),
    ``SKIP`` entries are listed; any other action raises ``ValueError``.
    Returns ``(to_load, skipped)``.
    """
    to_load, skipped = {}, []
    for name, tensor in state_dict.items():
        action, target, value = rule(name, tensor)
        if action == SKIP:
            skipped.append(name)
            continue
        if action != LOAD or target not in own_state or tuple(own_state[target].shape) != tuple(value.shape):
            shape = tuple(tensor.shape) if torch.is_tensor(tensor) else type(tensor).__name__
            raise ValueError(f"Unexpected {what} tensor {name} (as {target}) with shape {shape}.")
        to_load[target] = value.to(dtype=own_state[target].dtype)
    return to_load, skipped


def load_mapped(model: nn.Module, to_load: dict, *, may_be_absent: Iterable[str], what: str,
                skipped: Optional[list] = None) -> None:
    """Load ``to_load`` into ``model``; every other parameter or buffer must match a
    prefix in ``may_be_absent``, and no loaded name may be unknown."""
    missing, unexpected = model.load_state_dict(to_load, strict=False)
    prefixes = tuple(may_be_absent)
    missing = [n for n in missing if not (prefixes and n.startswith(prefixes))]
    if missing or unexpected:
        raise ValueError(f"{what} checkpoint mismatch: missing={missing}, unexpected={list(unexpected)}, "
                         f"skipped={skipped or []}")


def fold_through_target_head(target_lm_head_weight: torch.Tensor, up: torch.Tensor, dtype) -> torch.Tensor:
    """``W_target [V, hidden] . up [hidden, r]`` in fp32, cast once: a low-rank LM head
    that reads the rank state directly (code/dels.py:307-322)."""
    return target_lm_head_weight.detach().to("cpu", torch.float32).matmul(
        up.detach().to("cpu", torch.float32)).to(dtype)


def direct_vocab(config: dict) -> bool:
    """A direct-vocab RNN head (its own token embedding) per the checkpoint config."""
    param = config.get("rnn_parameterization", config.get("local_head_parameterization"))
    return param == "direct_vocab" or config.get("architecture") == "direct_vocab_rnn"

"""The reference's CPU PyTorch path for one draft step, restated with the same torch calls.

TEST INFRASTRUCTURE ONLY -- timed as the CPU baseline and used to report how
often the device path's ids agree with it; never shipped, never called by the
package.  Paths are relative to the dt-3t/DeLS-Spec repository.

* ``eager_step_bf16`` -- what the reference runs without Triton
  (``DeLSGraphRunner._forward_impl``'s fallback, code/kernel/dels.py:437-456,
  and ``spec_generate``'s eager loop, code/dflash.py:516-529): ``F.linear``
  for the rank (and ``F.silu``), ``F.linear`` for the short logits, then
  ``base + alpha * short`` and ``- beta * prior`` as bf16 tensor ops and
  ``torch.argmax``.  Every intermediate is a bf16 tensor, as in the
  reference's runner, whose static buffers hold the local head's bf16 dtype
  (code/kernel/dels.py:252, 278, 295-297); a scalar alpha multiplies in fp32
  and rounds to bf16, which per-row alphas reproduce below.
* ``step_fp32`` -- the same step with every tensor in fp32 (the fused
  kernel's semantics, evaluated unfused by torch).

Pinned in tests/test_oracle_torch_eager.py against the numpy oracle's
``eager_argmax_bf16`` and ``lowrank_argmax``.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F


def _rank(h: torch.Tensor, A: torch.Tensor, act: str) -> torch.Tensor:
    rank = F.linear(h, A, None)                       # code/kernel/dels.py:437
    if act == "silu":
        rank = F.silu(rank)                            # 438-439
    elif act != "identity":
        raise ValueError(f"Unsupported DeLS rank_activation={act!r}.")
    return rank


def eager_logits_bf16(h, A, B, base, prior: Optional[torch.Tensor], alpha, beta, act: str = "identity"):
    """bf16 [M, V] final logits of one draft step on the reference's eager bf16 path.

    ``h`` [M, d], ``A`` [r, d], ``B`` [V, r] bf16; ``base`` [M, V] and ``prior``
    [V] (cast to bf16, the runner's buffer dtype); ``alpha``/``beta`` fp32 [M].
    """
    bf = torch.bfloat16
    short = F.linear(_rank(h.to(bf), A.to(bf), act), B.to(bf), None)          # 448
    a = alpha.to(torch.float32).reshape(-1, 1)
    scaled = (a * short.float()).to(bf)              # python float * bf16 tensor: fp32 product, bf16 result
    logits = base.to(bf) + scaled                    # 449-452
    if prior is not None:
        b = beta.to(torch.float32).reshape(-1, 1)
        pb = (b * prior.to(bf).reshape(1, -1).float()).to(bf)
        with_prior = logits - pb                     # 453-455
        logits = torch.where(b != 0, with_prior, logits)
    return logits


def eager_step_bf16(h, A, B, base, prior: Optional[torch.Tensor], alpha, beta, act: str = "identity"):
    """int64 [M] ids of one draft step on the reference's eager bf16 path (arguments as
    ``eager_logits_bf16``)."""
    return torch.argmax(eager_logits_bf16(h, A, B, base, prior, alpha, beta, act), dim=-1)   # 456


def step_fp32(h, A, B, base, prior: Optional[torch.Tensor], alpha, beta, act: str = "identity"):
    """int64 [M] ids of the same step with fp32 tensors (rank rounded to bf16, as the
    runner's F.linear output is)."""
    f32 = torch.float32
    rank = _rank(h.to(torch.bfloat16), A.to(torch.bfloat16), act).to(f32)
    short = rank @ B.to(f32).t()
    logits = short * alpha.to(f32).reshape(-1, 1) + base.to(f32)
    if prior is not None:
        b = beta.to(f32).reshape(-1, 1)
        logits = torch.where(b != 0, logits - b * prior.to(f32).reshape(1, -1), logits)
    return torch.argmax(logits, dim=-1)

"""``sample()`` of the draft/verify loop (code/dflash.py:31-38) on the gfx950 kernels.

Same call as the reference: ``sample(logits [bsz, seq_len, V], temperature)``
returns ``int64 [bsz, seq_len]``.  Below temperature 1e-5 it is the argmax
over the last dimension (``argmax_rows``: lowest index of the maximum, first
NaN wins, as ``torch.argmax``).  Above, each row is one draw from
``softmax(logits / temperature)``, taken by a Gumbel-max over Philox4x32-10
noise (``sample_rows``) instead of materialising probabilities for
``torch.multinomial``: the same distribution, without writing [rows, V]
probabilities.  The 64-bit Philox key comes from ``seed`` when given, else it
is drawn from ``generator`` (a CPU ``torch.Generator``; torch's default one
when None), so ``torch.manual_seed`` makes runs repeatable as in the reference.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import ops


def draw_seed(generator: Optional[torch.Generator] = None) -> int:
    """A 64-bit Philox key drawn from a CPU generator (torch's default one when None)."""
    hi, lo = torch.randint(0, 2**32, (2,), generator=generator, dtype=torch.int64).tolist()
    return (hi << 32) | lo


def sample(logits: torch.Tensor, temperature: float = 0.0, *, generator: Optional[torch.Generator] = None,
           seed: Optional[int] = None, offset: int = 0) -> torch.Tensor:
    """Token ids ``[bsz, seq_len]`` from logits ``[bsz, seq_len, V]`` (code/dflash.py:31-38)."""
    if logits.dim() != 3:
        raise ValueError(f"logits must be [bsz, seq_len, vocab], got shape {tuple(logits.shape)}")
    bsz, seq_len, vocab_size = logits.shape
    flat = logits.reshape(-1, vocab_size)
    if flat.shape[1] > 1 and flat.stride(1) != 1:
        flat = flat.contiguous()
    if temperature < 1e-5:
        ids, _ = ops.argmax_rows(flat)
    else:
        ids, _ = ops.sample_rows(flat, float(temperature), draw_seed(generator) if seed is None else seed, offset)
    return ids.view(bsz, seq_len)

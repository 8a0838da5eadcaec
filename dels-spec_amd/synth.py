"""Seeded synthetic inputs for the low-rank LM-head argmax workloads.

All tensors are drawn on the CPU from ``torch.Generator`` (so every machine
gets the same values), in fp32, then cast:

* ``h ~ N(0, 1)`` bf16 [M, d]; ``A ~ N(0, 0.02)`` bf16 [r, d] (rank_proj.weight);
  ``B ~ N(0, 0.02)`` bf16 [V, r] (low_rank_lm_head.weight);
* ``base ~ N(0, 3)`` [M, V] in the requested dtype;
* the prior is the normalised log-probability (smoothing 1) of Zipf counts
  ``round(1e9 * k**-1.1)`` for rank k = 1..V, assigned to token ids by a seeded
  permutation;
* alpha/beta: scalars, or per-position schedules of length 16 drawn from
  U[0, 0.6], row m using entry m mod 16.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from .local_head import unigram_log_prior_from_counts

QWEN3_4B = dict(d=2560, r=256, V=151936)
QWEN3_8B = dict(d=4096, r=512, V=151936)


@dataclass
class LowRankInputs:
    h: torch.Tensor
    A: torch.Tensor
    B: torch.Tensor
    base: torch.Tensor
    prior: torch.Tensor
    alpha: torch.Tensor
    beta: torch.Tensor
    act: str = "identity"

    def to(self, device) -> "LowRankInputs":
        f = lambda t: t.to(device)  # noqa: E731
        return LowRankInputs(f(self.h), f(self.A), f(self.B), f(self.base), f(self.prior), f(self.alpha),
                             f(self.beta), self.act)

    @property
    def shape(self) -> dict:
        return dict(M=self.h.shape[0], d=self.h.shape[1], r=self.A.shape[0], V=self.B.shape[0])


def zipf_log_prior(V: int, *, s: float = 1.1, seed: int = 0) -> torch.Tensor:
    """Log unigram prior of permuted Zipf(s) counts, float64 [V]."""
    g = torch.Generator().manual_seed(seed)
    k = torch.arange(1, V + 1, dtype=torch.float64)
    counts = torch.round(1e9 * k.pow(-s))
    perm = torch.randperm(V, generator=g)
    permuted = torch.empty_like(counts)
    permuted[perm] = counts
    return unigram_log_prior_from_counts(permuted, V, smoothing=1.0)


def schedule(M: int, *, per_position: bool, scalar: float = 0.3, seed: int = 0, period: int = 16,
             hi: float = 0.6) -> tuple[torch.Tensor, torch.Tensor]:
    """(alpha, beta) per row as fp32 [M]."""
    if not per_position:
        return torch.full((M,), scalar, dtype=torch.float32), torch.full((M,), scalar, dtype=torch.float32)
    g = torch.Generator().manual_seed(seed + 7)
    a = torch.rand(period, generator=g, dtype=torch.float32) * hi
    b = torch.rand(period, generator=g, dtype=torch.float32) * hi
    idx = torch.arange(M) % period
    return a[idx].contiguous(), b[idx].contiguous()


def lowrank_inputs(M: int, d: int, r: int, V: int, *, base_dtype: torch.dtype = torch.float32,
                   prior_dtype: torch.dtype = torch.float32, per_position: bool = True, scalar: float = 0.3,
                   act: str = "identity", seed: int = 0, base_std: float = 3.0,
                   weight_std: float = 0.02) -> LowRankInputs:
    """One seeded input set of the fused low-rank argmax (CPU tensors)."""
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(M, d, generator=g).to(torch.bfloat16)
    A = (torch.randn(r, d, generator=g) * weight_std).to(torch.bfloat16)
    B = (torch.randn(V, r, generator=g) * weight_std).to(torch.bfloat16)
    base = (torch.randn(M, V, generator=g) * base_std).to(base_dtype)
    prior = zipf_log_prior(V, seed=seed).to(prior_dtype)
    alpha, beta = schedule(M, per_position=per_position, scalar=scalar, seed=seed)
    return LowRankInputs(h, A, B, base, prior, alpha, beta, act)


def config_inputs(name: str, *, seed: int = 0, base_dtype: Optional[torch.dtype] = None) -> LowRankInputs:
    """Input sets of the named workloads.

    ``qwen3_4b_m16``  M=16, d=2560, r=256, fp32 base, alpha = beta = 0.3;
    ``qwen3_8b_m16``  M=16, d=4096, r=512, fp32 base, per-position alpha/beta;
    ``qwen3_8b_m512`` M=512, d=4096, r=512, bf16 base and prior (runtime dtypes),
                      per-position alpha/beta.
    """
    if name == "qwen3_4b_m16":
        return lowrank_inputs(16, per_position=False, base_dtype=base_dtype or torch.float32, seed=seed,
                              **QWEN3_4B)
    if name == "qwen3_8b_m16":
        return lowrank_inputs(16, per_position=True, base_dtype=base_dtype or torch.float32, seed=seed,
                              **QWEN3_8B)
    if name == "qwen3_8b_m512":
        bd = base_dtype or torch.bfloat16
        return lowrank_inputs(512, per_position=True, base_dtype=bd, prior_dtype=bd, seed=seed, **QWEN3_8B)
    raise KeyError(name)


class SyntheticLocalHead(torch.nn.Module):
    """A DeLS local head of the reference's architecture (code/dels.py:186-192:
    embedding, one-layer GRU without bias, rank projection, low-rank LM head)
    with seeded random bf16 weights drawn on the device: the attributes
    DeLSGraphRunner reads.  Weights ~ N(0, std), embeddings ~ N(0, 1)."""

    def __init__(self, V: int, E: int, G: int, r: int, *, act: str = "silu", device="cuda", seed: int = 0,
                 std: float = 0.02):
        super().__init__()
        dev = torch.device(device)
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        kw = dict(device=dev, dtype=torch.bfloat16)
        self.embed_tokens = torch.nn.Embedding(V, E, **kw)
        self.prefix_gru = torch.nn.GRU(E, G, num_layers=1, batch_first=True, bias=False, **kw)
        self.rank_proj = torch.nn.Linear(G, r, bias=False, **kw)
        self.low_rank_lm_head = torch.nn.Linear(r, V, bias=False, **kw)
        self.rank_activation = act
        with torch.no_grad():
            self.embed_tokens.weight.copy_(torch.randn(V, E, generator=g, device=dev))
            self.prefix_gru.weight_ih_l0.copy_(torch.randn(3 * G, E, generator=g, device=dev) * std)
            self.prefix_gru.weight_hh_l0.copy_(torch.randn(3 * G, G, generator=g, device=dev) * std)
            self.rank_proj.weight.copy_(torch.randn(r, G, generator=g, device=dev) * std)
            self.low_rank_lm_head.weight.copy_(torch.randn(V, r, generator=g, device=dev) * std)


@dataclass
class DraftBlockWorkload:
    """The whole-draft-block workload: batch 8, block 16 unshifted (k_draft 15:
    one plain argmax and 14 DeLS steps), a target LM head W [V, d] bf16, a
    local head of hidden size G with rank r, per-step alpha/beta ~ U[0, 0.6]
    and the Zipf log-prior.  Weights live on the device."""

    head: SyntheticLocalHead
    W: torch.Tensor            # [V, d] bf16 ~ N(0, 0.02)
    prior: torch.Tensor        # [V] fp32 log-prior
    alphas: list
    betas: list
    batch: int
    k_draft: int
    d: int
    V: int
    gen: torch.Generator

    def hiddens(self, n: int) -> list:
        """``n`` draft blocks of hidden states [batch, k_draft, d] bf16 ~ N(0, 1)."""
        return [torch.randn(self.batch, self.k_draft, self.d, generator=self.gen, device=self.W.device)
                .to(torch.bfloat16) for _ in range(n)]


def draft_block_workload(device, *, batch: int = 8, k_draft: int = 15, d: int = 4096, V: int = 151936,
                         E: int = 1024, G: int = 1024, r: int = 256, act: str = "silu") -> DraftBlockWorkload:
    """Seeded draft-block workload (defaults: the Qwen3-8B head with the reference
    recipe's local head, E = G = 1024, r = 256, silu)."""
    dev = torch.device(device)
    head = SyntheticLocalHead(V, E, G, r, act=act, device=dev, seed=3)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    W = (torch.randn(V, d, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    prior = zipf_log_prior(V, seed=0).to(torch.float32).to(dev)
    steps = k_draft - 1
    ab = torch.rand(2, steps, generator=g, device=dev) * 0.6
    return DraftBlockWorkload(head, W, prior, ab[0].tolist(), ab[1].tolist(), batch, k_draft, d, V, g)

"""MI355X-native (gfx950) DeLS-Spec draft-token selection path.

Public surface (mirrors the reference's interface for this path):
  * ``DeLSGraphRunner``          -- drop-in hipGraph suffix-rollout runner
  * ``MarkovDeLSGraphRunner``    -- the same for the Markov local head
  * ``DraftCorrectionGraphRunner`` -- the Domino correction rollout (hipGraph)
  * ``DeLSDraftStep``            -- a whole draft block (target LM head, first
    argmax, rollout) as one graph
  * ``DeLSLocalHead``, ``MarkovDeLSLocalHead``, ``PositionMixJointHead`` --
    the local-head modules the runners consume, with their checkpoint
    loaders (``from_checkpoint``), and ``detect_local_head_checkpoint_kind``
  * ``parse_scalar_schedule``, ``load_unigram_log_prior``
  * ``fused_argmax``, ``lowrank_argmax``, ``rank_proj``, ``gru_step`` -- the
    per-step operators, each a thin wrapper over the C ABI in include/dels.h
  * ``pack_operand`` -- repack a weight into the MFMA-16 block layout the
    kernels stream at full HBM bandwidth
  * ``quantize_pack_fp8``, ``fused_argmax_fp8``, ``lowrank_argmax_fp8`` -- the
    fp8 (e4m3 weights, per-channel scales) variant of the same step
  * ``sample`` (and ``argmax_rows``, ``sample_rows``) -- the reference's
    ``sample(logits, temperature)``: argmax, or one softmax draw per row
"""

from .checkpoints import detect_local_head_checkpoint_kind
from .local_head import (DeLSLocalHead, MarkovDeLSLocalHead, PositionMixJointHead, load_unigram_log_prior,
                         parse_scalar_schedule, unigram_log_prior_from_counts)
from .ops import (Fp8Weight, PackedWeight, argmax_rows, fused_argmax, fused_argmax_fp8, gather_argmax, gru_step,
                  lowrank_argmax, lowrank_argmax_fp8, pack_operand, pack_operand_fp8, quantize_e4m3_rows,
                  quantize_pack_fp8, rank_proj, sample_rows, domino_argmax, lm_head, pack_lm_head)
from .sampling import sample
from .draft_step import DeLSDraftStep
from .runner import DeLSGraphRunner
from .markov_runner import MarkovDeLSGraphRunner
from .domino_runner import DraftCorrectionGraphRunner, unwrap_correction_mlp
from . import synth

__all__ = [
    "DeLSGraphRunner",
    "MarkovDeLSGraphRunner",
    "DraftCorrectionGraphRunner",
    "unwrap_correction_mlp",
    "domino_argmax",
    "lm_head",
    "pack_lm_head",
    "gather_argmax",
    "DeLSDraftStep",
    "argmax_rows",
    "sample_rows",
    "sample",
    "DeLSLocalHead",
    "MarkovDeLSLocalHead",
    "PositionMixJointHead",
    "detect_local_head_checkpoint_kind",
    "parse_scalar_schedule",
    "load_unigram_log_prior",
    "unigram_log_prior_from_counts",
    "fused_argmax",
    "lowrank_argmax",
    "rank_proj",
    "gru_step",
    "pack_operand",
    "PackedWeight",
    "Fp8Weight",
    "quantize_e4m3_rows",
    "pack_operand_fp8",
    "quantize_pack_fp8",
    "fused_argmax_fp8",
    "lowrank_argmax_fp8",
    "synth",
]

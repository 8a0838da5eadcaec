"""MarkovDeLSGraphRunner: the Markov DeLS suffix rollout as one native hipGraph.

Drop-in for the reference's ``MarkovDeLSGraphRunner``
(code/kernel/markov_dels.py:139-312; constructed at code/benchmark.py:512-520,
called at code/dflash.py:540-545): same keyword arguments, ``ValueError``
checks and messages, ``__call__(prev_token_ids, base_logits) -> int64[B,
steps]`` returning a fresh tensor, and ``_can_triton_fuse`` (true: the fused
native path is active).  Each step's rank is the previous token's row of the
merged embedding, gathered by the argmax kernel's own rank load, so a step is
one launch; the ``steps`` launches are captured once by the C ABI
(``dels_markov_graph_create``) and replayed per call.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from .ops import _DTYPES, new_workspace, pack_operand


class MarkovDeLSGraphRunner:
    """hipGraph runner for greedy Markov DeLS suffix rollout."""

    def __init__(self, *, local_head, batch_size: int, steps: int, vocab_size: int,
                 alpha_values: list[float], beta_values: list[float],
                 baseline_logits: Optional[torch.Tensor], device: torch.device):
        # Argument checks and messages follow code/kernel/markov_dels.py:153-173, 193-198.
        if steps <= 0:
            raise ValueError(f"MarkovDeLSGraphRunner requires steps > 0, got {steps}.")
        if len(alpha_values) != steps or len(beta_values) != steps:
            raise ValueError(
                "Markov DeLS graph alpha/beta schedules must match steps: "
                f"steps={steps}, alpha={len(alpha_values)}, beta={len(beta_values)}.")
        if int(local_head.vocab_size) != int(vocab_size):
            raise ValueError(
                "Markov DeLS local-head vocab size mismatch: "
                f"local_head={local_head.vocab_size}, vocab={vocab_size}.")
        if any(float(beta) != 0.0 for beta in beta_values) and baseline_logits is None:
            raise ValueError("Markov DeLS graph requires baseline_logits when any beta is nonzero.")
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError("MarkovDeLSGraphRunner needs a GPU device; the DeLS path has no CPU fallback.")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = device
        self.batch_size = int(batch_size)
        self.steps = int(steps)
        self.vocab_size = int(vocab_size)
        self.alpha_values = [float(x) for x in alpha_values]
        self.beta_values = [float(x) for x in beta_values]
        # The reference keeps its buffers in the head's dtype; base logits and the
        # prior do so here too, while the streamed weights are held in bf16.
        dtype = local_head.lm_head_weight.dtype
        if dtype not in _DTYPES:
            raise ValueError(f"Markov DeLS graph runner supports float32, bfloat16 and float16 heads, got {dtype}.")
        self.dtype = dtype
        wdt = torch.bfloat16
        self._can_triton_fuse = True
        with torch.inference_mode():
            self.embedding_weight = local_head.embedding_weight.detach().to(device, wdt).contiguous()
            self.lm_head_weight = local_head.lm_head_weight.detach().to(device, wdt).contiguous()
            self.rank = int(self.lm_head_weight.shape[1])
            if self.rank % 8 != 0:
                raise ValueError(f"Markov DeLS rank must be a multiple of 8, got {self.rank}.")
            baseline_flat = torch.zeros(self.vocab_size, dtype=dtype, device=device)
            if baseline_logits is not None:
                baseline_numel = int(baseline_logits.numel())
                if baseline_numel != self.vocab_size:
                    raise ValueError(
                        "Markov DeLS graph baseline vocab size mismatch: "
                        f"baseline={baseline_numel}, vocab={self.vocab_size}.")
                baseline_flat.copy_(baseline_logits.to(device=device, dtype=dtype).reshape(-1))
            self.baseline_logits = baseline_flat.contiguous()
            self.has_baseline = baseline_logits is not None
            # the LM head is streamed every step: MFMA-16 block layout
            self._lm_w_p = pack_operand(self.lm_head_weight)
            B, S, V = self.batch_size, self.steps, self.vocab_size
            self.static_prev_ids = torch.zeros(B, 1, dtype=torch.long, device=device)
            self.static_base_logits = torch.zeros(B, S, V, dtype=dtype, device=device)
            self.static_out = torch.zeros(B, S, dtype=torch.long, device=device)
            self.static_scores = torch.zeros(B, S, dtype=torch.float32, device=device)
            self._alpha = torch.tensor(self.alpha_values, dtype=torch.float32, device=device)
            self._beta = torch.tensor(self.beta_values, dtype=torch.float32, device=device)
        lib = _lib.load()
        self._ws = new_workspace(device, lib.dels_markov_rollout_ws_bytes(B, self.rank, V))
        self._params = self._rollout_params()
        torch.cuda.synchronize(device)
        handle = ctypes.c_void_p()
        with torch.cuda.device(device):
            _lib.check(lib.dels_markov_graph_create(ctypes.byref(self._params), ctypes.byref(handle)),
                       "dels_markov_graph_create")
        self._graph = handle

    def _rollout_params(self) -> "_lib.MarkovRolloutParams":
        p = _lib.MarkovRolloutParams()
        p.embedding = self.embedding_weight.data_ptr()
        p.ld_embedding = self.embedding_weight.stride(0)
        p.table_rows = self.embedding_weight.shape[0]
        p.lm_w = self._lm_w_p.data.data_ptr()
        p.lm_layout = _lib.LAYOUT_MFMA16
        p.prior = self.baseline_logits.data_ptr() if self.has_baseline else None
        p.prior_dtype = _DTYPES[self.baseline_logits.dtype]
        p.alpha = self._alpha.data_ptr()
        p.beta = self._beta.data_ptr()
        p.batch, p.steps, p.r, p.V = self.batch_size, self.steps, self.rank, self.vocab_size
        p.prev_ids = self.static_prev_ids.data_ptr()
        p.base = self.static_base_logits.data_ptr()
        p.base_dtype = _DTYPES[self.static_base_logits.dtype]
        p.ld_base = self.steps * self.vocab_size
        p.out_ids = self.static_out.data_ptr()
        p.out_scores = self.static_scores.data_ptr()
        p.ws = self._ws.data_ptr()
        p.ws_bytes = self._ws.numel()
        return p

    def replay(self) -> None:
        """Launch the captured rollout on the current stream (no copies)."""
        _lib.check(_lib.load().dels_graph_launch(self._graph, torch.cuda.current_stream(self.device).cuda_stream),
                   "dels_graph_launch")

    def enqueue_eager(self) -> None:
        """Run the rollout without the graph (same kernels, launched one by one)."""
        _lib.check(_lib.load().dels_markov_rollout_enqueue(ctypes.byref(self._params),
                                                           torch.cuda.current_stream(self.device).cuda_stream),
                   "dels_markov_rollout_enqueue")

    @torch.inference_mode()
    def __call__(self, prev_token_ids: torch.Tensor, base_logits: torch.Tensor) -> torch.Tensor:
        self.static_prev_ids.copy_(prev_token_ids)
        self.static_base_logits.copy_(base_logits)
        self.replay()
        return self.static_out.clone()

    def close(self) -> None:
        g = getattr(self, "_graph", None)
        if g is not None and g.value:
            _lib.load().dels_graph_destroy(g)
            self._graph = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

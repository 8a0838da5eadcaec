"""DeLSDraftStep: one whole DeLS draft block on the device, as a single hipGraph.

The graph path of ``spec_generate`` for one block (code/dflash.py:452-486):

    base_logits = target.lm_head(parallel_hiddens)            # [B, k, V] (k = k_draft)
    verify_ids[:, 1] = sample(base_logits[:, :1])             # plain argmax of position 0
    verify_ids[:, 2:k+1] = graph_runner(verify_ids[:, 1:2], base_logits[:, 1:k])

The LM head and the first-position argmax are either (``lm_head="fused"``, the
default wherever the shape allows it: hidden size a multiple of 256, batch * k
<= 8192) one launch of the hand-written ``dels_lm_head`` (W packed once,
streamed from HBM once, the position-0 rows argmaxed inside the GEMM and never
stored), or (``lm_head="library"``) a plain library GEMM (``torch.mm`` ->
hipBLASLt, as ``nn.Linear`` in the reference) followed by ``dels_argmax_rows``.
On the MI355X the hand-written head is the faster one at the bench shape
(batch 8, block 16, d 4096, V 151936: 226 us against 286 us for the library
GEMM).  ``lm_head="auto"`` picks ``fused`` where it applies, else ``library``.
The suffix rollout is ``dels_rollout_enqueue`` over the runner's packed
weights, reading ``base_logits[:, 1:k]`` in place (row stride k * V).  All of
it is captured once into one graph and replayed per block.
The drafter that produces ``parallel_hiddens`` is outside this path.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from .ops import new_workspace, pack_lm_head
from .runner import DeLSGraphRunner


class DeLSDraftStep:
    """One draft block: target LM head, first-position argmax and the DeLS rollout in one graph.

    ``k_draft`` is the block's draft count (block_size - 1 unshifted,
    code/dflash.py:442); the rollout runs ``k_draft - 1`` DeLS steps, so the
    alpha/beta schedules have that length (code/dflash.py:477).
    ``__call__(parallel_hiddens [B, k_draft, d] bf16) -> int64 [B, k_draft]``
    returns verify ids 1 .. k_draft of the block (a fresh tensor).
    """

    def __init__(self, *, local_head, lm_head_weight: torch.Tensor, batch_size: int, k_draft: int,
                 vocab_size: int, alpha_values: list[float], beta_values: list[float],
                 baseline_logits: Optional[torch.Tensor], device: torch.device, lm_head: str = "auto"):
        if lm_head not in ("auto", "library", "fused"):
            raise ValueError(f"lm_head must be 'auto', 'library' or 'fused', got {lm_head!r}")
        if k_draft < 2:
            raise ValueError(f"DeLSDraftStep needs k_draft >= 2 (at least one DeLS step), got {k_draft}.")
        self.runner = DeLSGraphRunner(local_head=local_head, batch_size=batch_size, steps=k_draft - 1,
                                      vocab_size=vocab_size, alpha_values=alpha_values, beta_values=beta_values,
                                      baseline_logits=baseline_logits, device=device)
        device = self.runner.device
        self.device = device
        B, k, V = int(batch_size), int(k_draft), int(vocab_size)
        W = lm_head_weight.detach().to(device)
        if W.dtype != torch.bfloat16 or W.dim() != 2 or int(W.shape[0]) != V:
            raise ValueError("lm_head_weight must be a bfloat16 [vocab_size, hidden] matrix")
        self.lm_head_weight = W.contiguous()
        d = int(W.shape[1])
        lib = _lib.load()
        fused_ok = d % 256 == 0 and B * k <= 8192
        if lm_head == "auto":
            lm_head = "fused" if fused_ok else "library"
        self._fused_head = lm_head == "fused"
        if self._fused_head and not fused_ok:
            raise ValueError("lm_head='fused' needs a hidden size that is a multiple of 256 and batch * k <= 8192")
        self._w_p = pack_lm_head(self.lm_head_weight) if self._fused_head else None
        self.batch_size, self.k_draft, self.vocab_size, self.hidden_size = B, k, V, d
        self.static_hidden = torch.zeros(B, k, d, dtype=torch.bfloat16, device=device)
        self.static_base = torch.empty(B, k, V, dtype=torch.bfloat16, device=device)
        # the block's ids and scores: column 0 from the LM head's argmax, columns 1..k-1
        # from the rollout, each written in place (the rollout reads its prefix ids there)
        self.static_out = torch.zeros(B, k, dtype=torch.int64, device=device)
        self.static_scores = torch.zeros(B, k, dtype=torch.float32, device=device)
        self.static_first, self.static_rest = self.static_out[:, 0], self.static_out[:, 1:]
        self.static_first_score, self.static_rest_scores = self.static_scores[:, 0], self.static_scores[:, 1:]
        self._ws = new_workspace(device, max(lib.dels_rollout_ws_bytes(B, self.runner.gru_hidden_dim,
                                                                        self.runner.rank_dim, V),
                                             lib.dels_argmax_rows_ws_bytes(B, V),
                                             lib.dels_lm_head_ws_bytes(B * k, d, V)))
        self._params = self.runner._rollout_params(self.static_base[:, 1:, :], k * V, self.static_first,
                                                   self.static_rest, self.static_rest_scores, self._ws)
        self._graph = None
        self._capture()

    def _enqueue(self, stream: torch.cuda.Stream) -> None:
        B, k, V, d = self.batch_size, self.k_draft, self.vocab_size, self.hidden_size
        lib = _lib.load()
        if self._fused_head:
            # base logits of positions 1..k-1 and the argmax of position 0 (rows b * k), one launch
            _lib.check(lib.dels_lm_head(self.static_hidden.data_ptr(), d, self._w_p.data.data_ptr(), B * k, d, V,
                                        self.static_base.data_ptr(), V, k, self.static_first.data_ptr(),
                                        self.static_first_score.data_ptr(), k, self._ws.data_ptr(),
                                        self._ws.numel(), stream.cuda_stream), "dels_lm_head")
        else:
            # base logits of the whole block: [B*k, d] . W^T, as nn.Linear
            torch.mm(self.static_hidden.view(B * k, d), self.lm_head_weight.t(),
                     out=self.static_base.view(B * k, V))
            _lib.check(lib.dels_argmax_rows(self.static_base.data_ptr(), k * V, _lib.DTYPE_BF16, B, V,
                                            self.static_first.data_ptr(), self.static_first_score.data_ptr(), k,
                                            self._ws.data_ptr(), self._ws.numel(), stream.cuda_stream),
                       "dels_argmax_rows")
        _lib.check(lib.dels_rollout_enqueue(ctypes.byref(self._params), stream.cuda_stream), "dels_rollout_enqueue")

    def _capture(self) -> None:
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self._enqueue(side)                      # warm-up outside the capture (library plans, workspaces)
            torch.cuda.synchronize(self.device)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                self._enqueue(side)
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self._graph = graph

    def replay(self) -> None:
        """Run the captured block on the current stream (inputs already in ``static_hidden``)."""
        self._graph.replay()

    def enqueue_eager(self) -> None:
        """The same work without the graph, on the current stream."""
        self._enqueue(torch.cuda.current_stream(self.device))

    @torch.inference_mode()
    def __call__(self, parallel_hiddens: torch.Tensor) -> torch.Tensor:
        self.static_hidden.copy_(parallel_hiddens)
        self.replay()
        return self.static_out.clone()

    def close(self) -> None:
        self._graph = None
        self.runner.close()

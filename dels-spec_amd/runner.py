"""DeLSGraphRunner: the block-prefix DeLS suffix rollout as one native hipGraph.

Drop-in for the reference's ``DeLSGraphRunner`` (code/kernel/dels.py:214-478;
constructed at code/benchmark.py:471-480, called at code/dflash.py:479-485):
same keyword arguments, the same ``ValueError`` checks and messages, the same
``__call__(prefix_ids, base_logits) -> int64[B, steps]`` returning a fresh
tensor, and a ``_can_triton_fuse`` attribute (true: the fused native path is
active).  The rollout -- GRU on the prefix token, then per step the rank
projection, the fused low-rank argmax and the GRU step on the chosen token --
is captured once by the C ABI into a hipGraph and replayed per call.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch
import torch.nn.functional as F

from . import _lib
from .ops import _DTYPES, new_workspace, pack_operand

_ACT_CODES = {"identity": _lib.ACT_IDENTITY, "silu": _lib.ACT_SILU}


class DeLSGraphRunner:
    """hipGraph runner for block-prefix DeLS greedy correction."""

    def __init__(self, *, local_head, batch_size: int, steps: int, vocab_size: int,
                 alpha_values: list[float], beta_values: list[float],
                 baseline_logits: Optional[torch.Tensor], device: torch.device):
        # Argument checks and messages follow code/kernel/dels.py:235-243, 257-258, 280-285, 440-443.
        if steps <= 0:
            raise ValueError(f"DeLSGraphRunner requires steps > 0, got {steps}.")
        if len(alpha_values) != steps or len(beta_values) != steps:
            raise ValueError(
                "DeLS graph alpha/beta schedules must match steps: "
                f"steps={steps}, alpha={len(alpha_values)}, beta={len(beta_values)}.")
        if any(float(beta) != 0.0 for beta in beta_values) and baseline_logits is None:
            raise ValueError("DeLS graph requires baseline_logits when any beta is nonzero.")

        self.local_head = local_head
        self.batch_size = int(batch_size)
        self.steps = int(steps)
        self.vocab_size = int(vocab_size)
        self.alpha_values = [float(x) for x in alpha_values]
        self.beta_values = [float(x) for x in beta_values]
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError("DeLSGraphRunner needs a GPU device; the DeLS path has no CPU fallback.")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = device

        # The reference keeps every static buffer in the local head's dtype
        # (code/kernel/dels.py:252).  Here base logits and the prior keep that
        # dtype (the kernels read fp32, bf16 and fp16), while the weights the
        # rollout streams are held in bf16: an fp16 or fp32 head is converted
        # once, so it runs at bf16 weight precision.
        dtype = local_head.rank_proj.weight.dtype
        if dtype not in _DTYPES:
            raise ValueError(f"DeLS graph runner supports float32, bfloat16 and float16 local heads, got {dtype}.")
        self.dtype = dtype
        wdt = torch.bfloat16
        self.rank_dim = int(local_head.low_rank_lm_head.weight.shape[1])
        self._can_triton_fuse = True

        act = local_head.rank_activation
        if act not in _ACT_CODES:
            raise ValueError(f"Unsupported DeLS rank_activation={act!r}.")
        self._act = _ACT_CODES[act]

        gru = local_head.prefix_gru
        if gru.num_layers != 1 or gru.bidirectional:
            raise ValueError("DeLS graph runner supports only a single unidirectional GRU.")
        self.gru_hidden_dim = int(gru.hidden_size)
        with torch.inference_mode():
            self.gru_w_ih = gru.weight_ih_l0.detach().to(device, wdt).contiguous()
            self.gru_w_hh = gru.weight_hh_l0.detach().to(device, wdt).contiguous()
            self.gru_b_ih = gru.bias_ih_l0.detach().to(device, wdt).contiguous() if gru.bias else None
            self.gru_b_hh = gru.bias_hh_l0.detach().to(device, wdt).contiguous() if gru.bias else None
            embed_weight = local_head.embed_tokens.weight.detach().to(device, wdt)
            # One-off input-projection table gi_table[v] = E[v] . W_ih^T + b_ih (code/kernel/dels.py:265-268).
            self._gru_input_proj_table = F.linear(embed_weight, self.gru_w_ih, self.gru_b_ih).contiguous()
            self.rank_weight = local_head.rank_proj.weight.detach().to(device, wdt).contiguous()
            rb = local_head.rank_proj.bias
            self.rank_bias = rb.detach().to(device, wdt).contiguous() if rb is not None else None
            self.lm_head_weight = local_head.low_rank_lm_head.weight.detach().to(device, wdt).contiguous()

            baseline_flat = torch.zeros(self.vocab_size, dtype=dtype, device=device)
            if baseline_logits is not None:
                baseline_numel = int(baseline_logits.numel())
                if baseline_numel != self.vocab_size:
                    raise ValueError(
                        "DeLS graph baseline vocab size mismatch: "
                        f"baseline={baseline_numel}, vocab={self.vocab_size}.")
                baseline_flat.copy_(baseline_logits.to(device=device, dtype=dtype).reshape(-1))
            self.baseline_logits = baseline_flat.contiguous()
            self.has_baseline = baseline_logits is not None

            if int(self.lm_head_weight.shape[0]) != self.vocab_size:
                raise ValueError(
                    "DeLS local-head vocab size does not match the runner: "
                    f"local_head={self.lm_head_weight.shape[0]}, vocab={self.vocab_size}.")
            # Weights the rollout streams every step, repacked once into the MFMA-16 block layout.
            self._packed = self.gru_hidden_dim % 16 == 0
            if self._packed:
                self._w_hh_p = pack_operand(self.gru_w_hh)
                self._rank_w_p = pack_operand(self.rank_weight)
                self._lm_w_p = pack_operand(self.lm_head_weight)

            B, G, r, V, S = self.batch_size, self.gru_hidden_dim, self.rank_dim, self.vocab_size, self.steps
            self.static_prefix_ids = torch.zeros(B, 1, dtype=torch.long, device=device)
            self.static_base_logits = torch.zeros(B, S, V, dtype=dtype, device=device)
            self.static_out = torch.zeros(B, S, dtype=torch.long, device=device)
            self.static_scores = torch.zeros(B, S, dtype=torch.float32, device=device)
            self._h_a = torch.zeros(B, G, dtype=wdt, device=device)
            self._h_b = torch.zeros(B, G, dtype=wdt, device=device)
            self._rank = torch.zeros(B, r, dtype=wdt, device=device)
            self._alpha = torch.tensor(self.alpha_values, dtype=torch.float32, device=device)
            self._beta = torch.tensor(self.beta_values, dtype=torch.float32, device=device)

        lib = _lib.load()
        self._ws = new_workspace(device, lib.dels_rollout_ws_bytes(B, G, r, V))
        p = self._rollout_params(self.static_base_logits, S * V, self.static_prefix_ids, self.static_out,
                                 self.static_scores, self._ws)
        self._params = p
        torch.cuda.synchronize(device)
        handle = ctypes.c_void_p()
        with torch.cuda.device(device):
            _lib.check(lib.dels_graph_create(ctypes.byref(p), ctypes.byref(handle)), "dels_graph_create")
        self._graph = handle

    def _rollout_params(self, base: torch.Tensor, ld_base: int, prefix_ids: torch.Tensor, out_ids: torch.Tensor,
                        out_scores: torch.Tensor, ws: torch.Tensor) -> "_lib.RolloutParams":
        """The C rollout description over these weights, reading ``base`` rows ``ld_base`` elements apart
        (steps * V for a [B, steps, V] tensor) and writing ``out_ids``/``out_scores`` [B, steps].  The
        prefix ids and the outputs may be strided views (rows ``stride(0)`` apart, unit column stride;
        ids and scores with the same row stride)."""
        B, G, r, V, S = self.batch_size, self.gru_hidden_dim, self.rank_dim, self.vocab_size, self.steps
        prior = self.baseline_logits if self.has_baseline else None
        dtype = self.baseline_logits.dtype
        p = _lib.RolloutParams()
        p.gi_table = self._gru_input_proj_table.data_ptr()
        p.ld_gi = self._gru_input_proj_table.stride(0)
        p.table_rows = self._gru_input_proj_table.shape[0]
        p.w_hh = self._w_hh_p.data.data_ptr() if self._packed else self.gru_w_hh.data_ptr()
        p.b_hh = self.gru_b_hh.data_ptr() if self.gru_b_hh is not None else None
        p.rank_w = self._rank_w_p.data.data_ptr() if self._packed else self.rank_weight.data_ptr()
        p.rank_b = self.rank_bias.data_ptr() if self.rank_bias is not None else None
        p.act = self._act
        p.lm_w = self._lm_w_p.data.data_ptr() if self._packed else self.lm_head_weight.data_ptr()
        p.prior = prior.data_ptr() if prior is not None else None
        p.prior_dtype = _DTYPES[dtype]
        p.alpha = self._alpha.data_ptr()
        p.beta = self._beta.data_ptr()
        p.batch, p.steps, p.G, p.r, p.V = B, S, G, r, V
        p.weights_layout = _lib.LAYOUT_MFMA16 if self._packed else _lib.LAYOUT_ROWMAJOR
        if out_scores.stride(0) != out_ids.stride(0) or out_ids.stride(-1) != 1 or out_scores.stride(-1) != 1:
            raise ValueError("out_ids and out_scores need unit column stride and the same row stride")
        p.prefix_ids = prefix_ids.data_ptr()
        p.ld_prefix = int(prefix_ids.stride(0))
        p.base = base.data_ptr()
        p.base_dtype = _DTYPES[base.dtype]
        p.ld_base = int(ld_base)
        p.out_ids = out_ids.data_ptr()
        p.out_scores = out_scores.data_ptr()
        p.ld_out = int(out_ids.stride(0))
        p.h_a = self._h_a.data_ptr()
        p.h_b = self._h_b.data_ptr()
        p.rank = self._rank.data_ptr()
        p.ws = ws.data_ptr()
        p.ws_bytes = ws.numel()
        return p

    def replay(self) -> None:
        """Launch the captured rollout on the current stream (no copies)."""
        _lib.check(_lib.load().dels_graph_launch(self._graph, torch.cuda.current_stream(self.device).cuda_stream),
                   "dels_graph_launch")

    def enqueue_eager(self) -> None:
        """Run the rollout without the graph (same kernels, launched one by one)."""
        _lib.check(_lib.load().dels_rollout_enqueue(ctypes.byref(self._params),
                                                    torch.cuda.current_stream(self.device).cuda_stream),
                   "dels_rollout_enqueue")

    @torch.inference_mode()
    def __call__(self, prefix_ids: torch.Tensor, base_logits: torch.Tensor) -> torch.Tensor:
        self.static_prefix_ids.copy_(prefix_ids)
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

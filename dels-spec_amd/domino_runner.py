"""DraftCorrectionGraphRunner: the Domino correction rollout as one native hipGraph.

Drop-in for the reference's ``DraftCorrectionGraphRunner``
(code/kernel/domino.py:232-520; constructed at code/benchmark.py:527-545,
called at code/dflash.py:604-613): same constructor arguments, the same checks
and messages, ``__call__(prefix_ids, parallel_hiddens, base_logits,
guidance_alpha=None) -> int64[B, steps]`` returning a fresh tensor, and the
``_can_triton_fuse`` attribute (true: the fused native path is active).

The rollout (code/kernel/domino.py:379-436) -- the hidden-state half of the
correction MLP's first layer for all steps at once, the GRU over the prefix
ids, then per step the GRU-state half, the fused middle/fc2/alpha/base argmax
and a GRU step on the chosen id -- is captured once through the C ABI
(``dels_domino_graph_create``) and replayed per call.

Differences from the reference, both from running every layer on the same
kernels: the prefix GRU runs as one table-gather GRU cell per prefix id (the
reference calls ``nn.GRU`` on the prefix embeddings, whose internal precision
the library chooses; every later step of the reference uses the same cell as
here); and the middle layer of the correction MLP is fused whatever it is
among SiLU, Identity, ReLU, GELU (erf or tanh), Tanh and Sigmoid, in fp32 --
the reference fuses SiLU only and runs the others as an unfused eager step
in the model's dtype (code/kernel/domino.py:404-431), so for those its
scores are bf16-rounded where these are not.  Other middle modules are
refused.
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .ops import _DTYPES, new_workspace, pack_operand


def unwrap_correction_mlp(embed_proj: nn.Module) -> tuple[nn.Linear, nn.Module, nn.Linear]:
    """Split ``nn.Sequential(Linear(hidden + G, E), middle..., Linear(E, V))`` into
    ``(fc1, middle, fc2)`` (code/kernel/domino.py:15-51)."""
    if not isinstance(embed_proj, nn.Sequential):
        raise TypeError("Graph runner requires draft_model.embed_proj to be nn.Sequential.")
    layers = list(embed_proj.children())
    if len(layers) < 2:
        raise ValueError("embed_proj must contain at least two layers.")
    if not isinstance(layers[0], nn.Linear):
        raise ValueError("embed_proj first layer must be nn.Linear.")
    if not isinstance(layers[-1], nn.Linear):
        raise ValueError("embed_proj last layer must be nn.Linear.")
    inner = layers[1:-1]
    middle = nn.Sequential(*inner) if inner else nn.Identity()
    return layers[0], middle, layers[-1]


def _is_silu(middle: nn.Module) -> bool:
    return middle_name(middle) == "silu"


def middle_name(middle: nn.Module) -> str | None:
    """The fused kernel's name (``_lib.MIDDLE_CODES``) of the correction MLP's
    middle layer -- a single elementwise module, or a Sequential of one or none
    -- or None when it is not one the kernel fuses."""
    if isinstance(middle, nn.Sequential):
        kids = list(middle.children())
        if not kids:
            return "identity"
        if len(kids) != 1:
            return None
        middle = kids[0]
    if isinstance(middle, nn.SiLU):
        return "silu"
    if isinstance(middle, nn.Identity):
        return "identity"
    if isinstance(middle, nn.ReLU):
        return "relu"
    if isinstance(middle, nn.GELU):
        return {"none": "gelu", "tanh": "gelu_tanh"}.get(middle.approximate)
    if isinstance(middle, nn.Tanh):
        return "tanh"
    if isinstance(middle, nn.Sigmoid):
        return "sigmoid"
    return None


class DraftCorrectionGraphRunner:
    """hipGraph runner for the Domino block draft correction (greedy)."""

    def __init__(self, draft_model: nn.Module, target_model: nn.Module, batch_size: int, steps: int,
                 hidden_dim: int, gru_hidden_dim: int, vocab_size: int, prefix_token_count: int,
                 device: torch.device, guidance_alpha: float = 1.0):
        self.steps = int(steps)
        self.draft_model = draft_model
        self.target_model = target_model
        self.prefix_token_count = int(prefix_token_count)
        self.gru_hidden_dim = int(gru_hidden_dim)
        self.guidance_alpha = float(guidance_alpha)
        self.batch_size = int(batch_size)
        self.hidden_dim = int(hidden_dim)
        self.vocab_size = int(vocab_size)
        if self.steps <= 0:
            raise ValueError(f"DraftCorrectionGraphRunner requires steps > 0, got {steps}.")
        if self.prefix_token_count <= 0:
            raise ValueError("DraftCorrectionGraphRunner requires prefix_token_count > 0.")

        fc1, self.middle, fc2 = unwrap_correction_mlp(draft_model.embed_proj)
        expected_in = self.hidden_dim + self.gru_hidden_dim
        if fc1.in_features != expected_in:
            raise ValueError(
                f"Correction MLP input dim mismatch: got {fc1.in_features}, "
                f"expected {expected_in} = hidden_dim + gru_hidden_dim.")
        self._middle_is_silu = _is_silu(self.middle)
        self._middle = middle_name(self.middle)
        self._can_triton_fuse = self._middle is not None
        if self._middle is None:
            raise ValueError("The native Domino runner fuses a middle layer of SiLU, Identity, ReLU, GELU, "
                             f"Tanh or Sigmoid (embed_proj middle is {self.middle!r}).")
        gru = draft_model.prefix_gru
        if gru.num_layers != 1 or gru.bidirectional:
            raise AssertionError("Domino graph runner supports only a single unidirectional GRU.")
        if int(gru.hidden_size) != self.gru_hidden_dim:
            raise ValueError(f"prefix_gru hidden size {gru.hidden_size} != gru_hidden_dim {self.gru_hidden_dim}.")

        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError("DraftCorrectionGraphRunner needs a GPU device; the Domino path has no CPU fallback.")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = device
        # Static buffers keep the draft model's dtype, as the reference's
        # (code/kernel/domino.py:296); the streamed weights and the hidden
        # states enter the kernels in bf16 (an fp16/fp32 model is converted once).
        dtype = next(draft_model.parameters()).dtype
        if dtype not in _DTYPES:
            raise ValueError(f"Domino graph runner supports float32, bfloat16 and float16 models, got {dtype}.")
        self.dtype = dtype
        wdt = torch.bfloat16
        D, G = self.hidden_dim, self.gru_hidden_dim
        E, V = int(fc1.out_features), int(fc2.out_features)
        if fc2.in_features != E:
            raise ValueError(f"embed_proj last layer takes {fc2.in_features} features, expected {E}.")
        if V != self.vocab_size:
            raise ValueError(f"embed_proj vocab size {V} != vocab_size {self.vocab_size}.")
        if E % 32 != 0 or E > 2048:
            raise ValueError(f"Domino correction width {E} must be a multiple of 32 and at most 2048.")
        self.mlp_hidden_dim = E

        with torch.inference_mode():
            w1 = fc1.weight.detach().to(device, wdt)
            self.w_z = w1[:, :D].contiguous()
            self.w_s = w1[:, D:].contiguous()
            self.fc1_bias = fc1.bias.detach().to(device, wdt).contiguous() if fc1.bias is not None else None
            self.fc2_weight = fc2.weight.detach().to(device, wdt).contiguous()
            self.fc2_bias = fc2.bias.detach().to(device).contiguous() if fc2.bias is not None else None
            self.gru_w_ih = gru.weight_ih_l0.detach().to(device, wdt).contiguous()
            self.gru_w_hh = gru.weight_hh_l0.detach().to(device, wdt).contiguous()
            self.gru_b_ih = gru.bias_ih_l0.detach().to(device, wdt).contiguous() if gru.bias else None
            self.gru_b_hh = gru.bias_hh_l0.detach().to(device, wdt).contiguous() if gru.bias else None
            # gi_table[v] = embed_tokens.weight[v] . W_ih^T + b_ih, once (code/kernel/domino.py:328-333)
            embed_weight = target_model.model.embed_tokens.weight.detach().to(device, wdt)
            self._gru_input_proj_table = F.linear(embed_weight, self.gru_w_ih, self.gru_b_ih).contiguous()

            self._packed = G % 16 == 0 and D % 32 == 0
            if self._packed:
                self._w_hh_p = pack_operand(self.gru_w_hh)
                self._w_z_p = pack_operand(self.w_z)
                self._w_s_p = pack_operand(self.w_s)
            self._fc2_p = pack_operand(self.fc2_weight)

            B, S, P = self.batch_size, self.steps, self.prefix_token_count
            self.static_prefix_ids = torch.zeros(B, P, dtype=torch.long, device=device)
            self.static_parallel_hiddens = torch.zeros(B, S, D, dtype=dtype, device=device)
            self.static_base_logits = torch.zeros(B, S, V, dtype=dtype, device=device)
            self.static_out = torch.zeros(B, S, dtype=torch.long, device=device)
            self.static_scores = torch.zeros(B, S, dtype=torch.float32, device=device)
            self._hiddens = (self.static_parallel_hiddens if dtype == wdt
                             else torch.zeros(B, S, D, dtype=wdt, device=device))
            self._h_a = torch.zeros(B, G, dtype=wdt, device=device)
            self._h_b = torch.zeros(B, G, dtype=wdt, device=device)
            self._z = torch.zeros(B * S, E, dtype=wdt, device=device)
            self._s = torch.zeros(B, E, dtype=wdt, device=device)

        lib = _lib.load()
        self._ws = new_workspace(device, lib.dels_domino_rollout_ws_bytes(B, S, D, G, E, V))
        self._params = self._rollout_params()
        torch.cuda.synchronize(device)
        handle = ctypes.c_void_p()
        with torch.cuda.device(device):
            _lib.check(lib.dels_domino_graph_create(ctypes.byref(self._params), ctypes.byref(handle)),
                       "dels_domino_graph_create")
        self.graph = handle

    def _rollout_params(self) -> "_lib.DominoRolloutParams":
        p = _lib.DominoRolloutParams()
        t = self._gru_input_proj_table
        p.gi_table, p.ld_gi, p.table_rows = t.data_ptr(), t.stride(0), t.shape[0]
        p.w_hh = self._w_hh_p.data.data_ptr() if self._packed else self.gru_w_hh.data_ptr()
        p.b_hh = self.gru_b_hh.data_ptr() if self.gru_b_hh is not None else None
        p.w_z = self._w_z_p.data.data_ptr() if self._packed else self.w_z.data_ptr()
        p.fc1_bias = self.fc1_bias.data_ptr() if self.fc1_bias is not None else None
        p.w_s = self._w_s_p.data.data_ptr() if self._packed else self.w_s.data_ptr()
        p.fc2_w = self._fc2_p.data.data_ptr()
        p.fc2_bias = self.fc2_bias.data_ptr() if self.fc2_bias is not None else None
        p.fc2_bias_dtype = _DTYPES[self.fc2_bias.dtype] if self.fc2_bias is not None else 0
        p.alpha = self.guidance_alpha
        p.batch, p.steps, p.prefix_len = self.batch_size, self.steps, self.prefix_token_count
        p.D, p.G, p.E, p.V = self.hidden_dim, self.gru_hidden_dim, self.mlp_hidden_dim, self.vocab_size
        p.weights_layout = _lib.LAYOUT_MFMA16 if self._packed else _lib.LAYOUT_ROWMAJOR
        p.prefix_ids = self.static_prefix_ids.data_ptr()
        p.hiddens = self._hiddens.data_ptr()
        p.base = self.static_base_logits.data_ptr()
        p.base_dtype = _DTYPES[self.static_base_logits.dtype]
        p.ld_base = 0
        p.out_ids = self.static_out.data_ptr()
        p.out_scores = self.static_scores.data_ptr()
        p.h_a, p.h_b = self._h_a.data_ptr(), self._h_b.data_ptr()
        p.z, p.s = self._z.data_ptr(), self._s.data_ptr()
        p.ws, p.ws_bytes = self._ws.data_ptr(), self._ws.numel()
        p.middle = _lib.MIDDLE_CODES[self._middle]
        return p

    def replay(self) -> None:
        """Launch the captured rollout on the current stream (no copies)."""
        _lib.check(_lib.load().dels_graph_launch(self.graph, torch.cuda.current_stream(self.device).cuda_stream),
                   "dels_graph_launch")

    def enqueue_eager(self) -> None:
        """Run the rollout without the graph (the same kernels, launched one by one)."""
        _lib.check(_lib.load().dels_domino_rollout_enqueue(ctypes.byref(self._params),
                                                           torch.cuda.current_stream(self.device).cuda_stream),
                   "dels_domino_rollout_enqueue")

    @torch.inference_mode()
    def __call__(self, prefix_ids: torch.Tensor, parallel_hiddens: torch.Tensor, base_logits: torch.Tensor,
                 guidance_alpha: float | None = None) -> torch.Tensor:
        if guidance_alpha is not None and float(guidance_alpha) != self.guidance_alpha:
            raise ValueError(
                "DraftCorrectionGraphRunner captures a fixed domino guidance alpha; "
                f"got {float(guidance_alpha)} but runner was built with {self.guidance_alpha}.")
        self.static_prefix_ids.copy_(prefix_ids)
        self.static_parallel_hiddens.copy_(parallel_hiddens)
        if self._hiddens is not self.static_parallel_hiddens:
            self._hiddens.copy_(self.static_parallel_hiddens)
        self.static_base_logits.copy_(base_logits)
        self.replay()
        return self.static_out.clone()

    def close(self) -> None:
        g = getattr(self, "graph", None)
        if g is not None and g.value:
            _lib.load().dels_graph_destroy(g)
            self.graph = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

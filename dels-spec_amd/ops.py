"""Torch-facing operators of the DeLS draft path, backed by the gfx950 kernels.

Each operator validates its tensors, then calls the C ABI on the current HIP
stream.  There is no CPU or eager-PyTorch fallback: a missing library or a
non-GPU tensor raises.

Reference semantics (paths relative to the dt-3t/DeLS-Spec repository):
  * ``fused_argmax``   -- _fused_low_rank_argmax_kernel + _reduce_argmax_kernel,
                          code/kernel/dels.py:15-138, launched at 375-423
  * ``rank_proj``      -- F.linear(h, rank_weight, rank_bias) (+ F.silu),
                          code/kernel/dels.py:437-443
  * ``lowrank_argmax`` -- the two above, one draft step, code/kernel/dels.py:437-446
  * ``gru_step``       -- _gru_cell / _fused_gru_cell_kernel with the input-table
                          gather, code/kernel/dels.py:140-211, 359-373, 432, 461
  * ``gather_argmax``  -- a Markov step: F.embedding + _fused_markov_argmax_kernel +
                          _reduce_argmax_kernel, code/kernel/markov_dels.py:15-138, 216-268
  * ``argmax_rows`` / ``sample_rows`` -- sample() at temperature 0 / above 0,
                          code/dflash.py:31-38
  * ``lm_head``        -- target.lm_head(parallel_hiddens) with sample() of position 0
                          fused, code/dflash.py:468, 475
  * ``domino_argmax``  -- a Domino correction step: _fused_mlp_bias_argmax_kernel +
                          _reduce_argmax_kernel, code/kernel/domino.py:58-173, 438-482
"""

from __future__ import annotations

import threading
from dataclasses import dataclass
from typing import Optional, Sequence, Union

import torch

from . import _lib

_ACTS = {"identity": _lib.ACT_IDENTITY, "silu": _lib.ACT_SILU}
_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16}

Scalars = Union[float, int, Sequence[float], torch.Tensor]


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got device {t.device}); the DeLS path has no CPU fallback")


def _require_bf16_matrix(t: torch.Tensor, name: str, rows: Optional[int] = None,
                         cols: Optional[int] = None) -> None:
    _require_cuda(t, name)
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if rows is not None and t.shape[0] != rows:
        raise ValueError(f"{name} has {t.shape[0]} rows, expected {rows}")
    if cols is not None and t.shape[1] != cols:
        raise ValueError(f"{name} has {t.shape[1]} columns, expected {cols}")
    if t.shape[1] > 1 and t.stride(1) != 1:
        raise ValueError(f"{name} must have unit column stride")


@dataclass
class PackedWeight:
    """A bf16 [rows, cols] weight stored in the MFMA-16 block layout.

    16-row x 32-column blocks of 1 KiB in wave64 lane order (include/dels.h,
    DELS_LAYOUT_MFMA16): every MFMA operand load of the kernels then reads one
    contiguous KiB.  Produced by ``pack_operand``.
    """

    data: torch.Tensor
    rows: int
    cols: int
    kchunk: int = 0        # > 0: the blocks in K-chunk-major order (pack_lm_head)

    @property
    def shape(self) -> tuple[int, int]:
        return (self.rows, self.cols)

    @property
    def device(self) -> torch.device:
        return self.data.device


Weight = Union[torch.Tensor, PackedWeight]


def pack_operand(W: torch.Tensor) -> PackedWeight:
    """Repack a bf16 [rows, cols] GPU matrix into the MFMA-16 block layout."""
    _require_bf16_matrix(W, "W")
    rows, cols = W.shape
    lib = _lib.load()
    nbytes = max(int(lib.dels_packed_bytes(rows, cols)), 16)
    buf = torch.empty(nbytes, dtype=torch.uint8, device=W.device)
    _lib.check(lib.dels_pack_operand(W.data_ptr(), W.stride(0), rows, cols, buf.data_ptr(), buf.numel(),
                                     _stream_ptr(W.device)), "dels_pack_operand")
    return PackedWeight(buf, int(rows), int(cols))


LM_HEAD_KCHUNK = 4     # K blocks per chunk of the LM head's layout (kLmHeadKChunk)


def pack_lm_head(W: torch.Tensor) -> PackedWeight:
    """Repack a bf16 [V, K] LM-head weight (K a multiple of 128) into the LM head kernel's
    layout: MFMA-16 blocks in K-chunk-major order (include/dels.h, dels_pack_lm_head)."""
    _require_bf16_matrix(W, "W")
    rows, cols = W.shape
    lib = _lib.load()
    nbytes = max(int(lib.dels_packed_bytes(rows, cols)), 16)
    buf = torch.empty(nbytes, dtype=torch.uint8, device=W.device)
    _lib.check(lib.dels_pack_lm_head(W.data_ptr(), W.stride(0), rows, cols, buf.data_ptr(), buf.numel(),
                                     _stream_ptr(W.device)), "dels_pack_lm_head")
    return PackedWeight(buf, int(rows), int(cols), LM_HEAD_KCHUNK)


def _weight(w: Weight, name: str, cols: Optional[int] = None, rows: Optional[int] = None):
    """(pointer, leading dimension, layout code, rows, cols) of a weight operand."""
    if isinstance(w, PackedWeight):
        _require_cuda(w.data, name)
        if w.kchunk:
            raise ValueError(f"{name} is packed for the LM head (pack_lm_head); use pack_operand here")
        if cols is not None and w.cols != cols:
            raise ValueError(f"{name} has {w.cols} columns, expected {cols}")
        if rows is not None and w.rows != rows:
            raise ValueError(f"{name} has {w.rows} rows, expected {rows}")
        return w.data.data_ptr(), 0, _lib.LAYOUT_MFMA16, w.rows, w.cols
    _require_bf16_matrix(w, name, rows=rows, cols=cols)
    return w.data_ptr(), w.stride(0), _lib.LAYOUT_ROWMAJOR, int(w.shape[0]), int(w.shape[1])


class _Workspaces:
    """Zero-initialised scratch buffers, one per (device, stream), grown on demand.

    Every entry point lays a workspace out alike (include/dels.h): a control
    area that the kernels return to its previous state, a region only the
    fused decode step writes (tagged words), and data regions that may hold
    anything between calls.  No call needs the buffer cleared, so it is zeroed
    only when it is (re)allocated.  Calls on one stream are ordered and may
    share it; each stream gets its own buffer.
    """

    def __init__(self):
        self._bufs = {}
        self._lock = threading.Lock()

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor:
        key = (device.index, _stream_ptr(device))
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, 1 << 16)
                size = (size + 255) // 256 * 256
                buf = torch.zeros(size, dtype=torch.uint8, device=device)
                self._bufs[key] = buf
            return buf


_WORKSPACES = _Workspaces()


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """The shared zero-initialised workspace for ``device`` and its current stream."""
    return _WORKSPACES.get(device, nbytes)


def new_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A private zero-initialised workspace (e.g. for a captured graph)."""
    size = (max(int(nbytes), 256) + 255) // 256 * 256
    return torch.zeros(size, dtype=torch.uint8, device=device)


def _rows_param(x: Scalars, M: int, device: torch.device, name: str) -> tuple[torch.Tensor, int]:
    """alpha/beta as a device fp32 array and a per-row stride (0 = broadcast)."""
    if isinstance(x, torch.Tensor):
        t = x
        if t.device.type != "cuda":
            t = t.to(device)
        if t.dtype != torch.float32:
            t = t.float()
        t = t.reshape(-1)
        if t.numel() == 1:
            return t.contiguous(), 0
        if t.numel() != M:
            raise ValueError(f"{name} has {t.numel()} entries, expected 1 or {M}")
        return t, t.stride(0)
    if isinstance(x, (float, int)):
        return torch.full((1,), float(x), dtype=torch.float32, device=device), 0
    vals = [float(v) for v in x]
    if len(vals) == 1:
        return torch.tensor(vals, dtype=torch.float32, device=device), 0
    if len(vals) != M:
        raise ValueError(f"{name} has {len(vals)} entries, expected 1 or {M}")
    return torch.tensor(vals, dtype=torch.float32, device=device), 1


def _base_view(base: torch.Tensor, M: int, V: int) -> torch.Tensor:
    _require_cuda(base, "base_logits")
    if base.dtype not in _DTYPES:
        raise TypeError(f"base_logits dtype {base.dtype} not supported (float32, bfloat16, float16)")
    if base.dim() == 3 and base.shape[1] == 1:
        base = base[:, 0, :]
    if base.dim() != 2 or tuple(base.shape) != (M, V):
        raise ValueError(f"base_logits must be [{M}, {V}], got {tuple(base.shape)}")
    if V > 1 and base.stride(1) != 1:
        raise ValueError("base_logits must have unit stride along the vocabulary")
    return base


def _prior_view(prior: Optional[torch.Tensor], V: int) -> Optional[torch.Tensor]:
    if prior is None:
        return None
    _require_cuda(prior, "baseline_logits")
    if prior.dtype not in _DTYPES:
        raise TypeError(f"baseline_logits dtype {prior.dtype} not supported")
    if prior.numel() != V:
        raise ValueError(f"DeLS graph baseline vocab size mismatch: baseline={prior.numel()}, vocab={V}.")
    prior = prior.reshape(-1)
    if not prior.is_contiguous():
        prior = prior.contiguous()
    return prior


def _outputs(out_ids, out_score, M, dev):
    """Output buffers (allocated if not given) and their shared row stride."""
    if out_ids is None:
        out_ids = torch.empty(M, dtype=torch.int64, device=dev)
    if out_score is None:
        out_score = torch.empty(M, dtype=torch.float32, device=dev)
    if out_ids.dtype != torch.int64 or out_score.dtype != torch.float32:
        raise TypeError("out_ids must be int64 and out_score float32")
    if out_ids.numel() != M or out_score.numel() != M:
        raise ValueError(f"output buffers must hold {M} rows")
    ld = out_ids.stride(-1) if M > 1 else 1
    if M > 1 and out_score.stride(-1) != ld:
        raise ValueError("out_ids and out_score must share one row stride")
    return out_ids, out_score, ld


def rank_proj(h: torch.Tensor, rank_weight: Weight, rank_bias: Optional[torch.Tensor] = None,
              act: str = "identity", *, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``rank = act(F.linear(h, rank_weight, rank_bias))`` in bf16 (code/kernel/dels.py:437-443).

    ``rank_weight`` is A [r, d] bf16, row-major or packed (``pack_operand``).
    """
    if act not in _ACTS:
        raise ValueError(f"Unsupported DeLS rank_activation={act!r}.")
    if h.dim() == 1:
        h = h.unsqueeze(0)
    M, d = h.shape
    _require_bf16_matrix(h, "h", cols=d)
    a_ptr, lda, a_lay, r, _ = _weight(rank_weight, "rank_weight", cols=d)
    rank_bias = _bias(rank_bias, r)
    if out is None:
        out = torch.empty(M, r, dtype=torch.bfloat16, device=h.device)
    else:
        _require_bf16_matrix(out, "out", rows=M, cols=r)
    lib = _lib.load()
    nbytes = lib.dels_rank_proj_ws_bytes(M, d, r)
    ws = workspace(h.device, nbytes)
    _lib.check(lib.dels_rank_proj(h.data_ptr(), h.stride(0), a_ptr, lda, a_lay,
                                  rank_bias.data_ptr() if rank_bias is not None else None, _ACTS[act],
                                  M, d, r, out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(),
                                  _stream_ptr(h.device)), "dels_rank_proj")
    return out


def _bias(rank_bias: Optional[torch.Tensor], r: int) -> Optional[torch.Tensor]:
    if rank_bias is None:
        return None
    _require_cuda(rank_bias, "rank_bias")
    if rank_bias.dtype != torch.bfloat16 or rank_bias.numel() != r:
        raise ValueError("rank_bias must be a bfloat16 vector of length r")
    return rank_bias.contiguous()


def fused_argmax(rank: torch.Tensor, lm_head_weight: Weight, base_logits: torch.Tensor,
                 baseline_logits: Optional[torch.Tensor] = None, alpha: Scalars = 1.0, beta: Scalars = 0.0,
                 *, out_ids: Optional[torch.Tensor] = None,
                 out_score: Optional[torch.Tensor] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row argmax of ``rank.B^T * alpha + base - beta * prior`` (code/kernel/dels.py:15-138).

    ``rank`` [M, r] bf16; ``lm_head_weight`` B [V, r] bf16 (row-major or
    packed); ``base_logits`` an [M, V] view (any row stride) in fp32/bf16/fp16;
    ``baseline_logits`` the prior [V] (or None); ``alpha``/``beta`` scalars,
    length-M sequences or device tensors.  Returns ``(ids int64[M], score fp32[M])``.
    """
    if rank.dim() == 1:
        rank = rank.unsqueeze(0)
    M, r = rank.shape
    _require_bf16_matrix(rank, "rank", cols=r)
    b_ptr, ldb, b_lay, V, _ = _weight(lm_head_weight, "lm_head_weight", cols=r)
    base = _base_view(base_logits, M, V)
    prior = _prior_view(baseline_logits, V)
    dev = rank.device
    a, a_s = _rows_param(alpha, M, dev, "alpha")
    b, b_s = _rows_param(beta, M, dev, "beta")
    out_ids, out_score, ld_out = _outputs(out_ids, out_score, M, dev)
    lib = _lib.load()
    ws = workspace(dev, lib.dels_fused_argmax_ws_bytes(M, r, V))
    _lib.check(lib.dels_fused_argmax(
        rank.data_ptr(), rank.stride(0), b_ptr, ldb, b_lay,
        base.data_ptr(), base.stride(0), _DTYPES[base.dtype],
        prior.data_ptr() if prior is not None else None, _DTYPES[prior.dtype] if prior is not None else 0,
        a.data_ptr(), a_s, b.data_ptr(), b_s, M, r, V,
        out_ids.data_ptr(), out_score.data_ptr(), ld_out,
        ws.data_ptr(), ws.numel(), _stream_ptr(dev)), "dels_fused_argmax")
    return out_ids, out_score


def lowrank_argmax(h: torch.Tensor, rank_weight: Weight, lm_head_weight: Weight,
                   base_logits: torch.Tensor, baseline_logits: Optional[torch.Tensor] = None,
                   alpha: Scalars = 1.0, beta: Scalars = 0.0, act: str = "identity",
                   rank_bias: Optional[torch.Tensor] = None, *, out_ids: Optional[torch.Tensor] = None,
                   out_score: Optional[torch.Tensor] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """One DeLS draft step: rank projection of ``h`` then the fused argmax.

    ``h`` [M, d] bf16, ``rank_weight`` A [r, d] and ``lm_head_weight`` B [V, r]
    bf16, each row-major or packed (code/kernel/dels.py:437-446).  Returns
    ``(ids int64[M], score fp32[M])``.
    """
    if act not in _ACTS:
        raise ValueError(f"Unsupported DeLS rank_activation={act!r}.")
    if h.dim() == 1:
        h = h.unsqueeze(0)
    M, d = h.shape
    _require_bf16_matrix(h, "h", cols=d)
    a_ptr, lda, a_lay, r, _ = _weight(rank_weight, "rank_weight", cols=d)
    b_ptr, ldb, b_lay, V, _ = _weight(lm_head_weight, "lm_head_weight", cols=r)
    base = _base_view(base_logits, M, V)
    prior = _prior_view(baseline_logits, V)
    rank_bias = _bias(rank_bias, r)
    dev = h.device
    a, a_s = _rows_param(alpha, M, dev, "alpha")
    b, b_s = _rows_param(beta, M, dev, "beta")
    out_ids, out_score, ld_out = _outputs(out_ids, out_score, M, dev)
    lib = _lib.load()
    ws = workspace(dev, lib.dels_lowrank_argmax_ws_bytes(M, d, r, V))
    _lib.check(lib.dels_lowrank_argmax(
        h.data_ptr(), h.stride(0), a_ptr, lda, a_lay,
        rank_bias.data_ptr() if rank_bias is not None else None, _ACTS[act],
        b_ptr, ldb, b_lay,
        base.data_ptr(), base.stride(0), _DTYPES[base.dtype],
        prior.data_ptr() if prior is not None else None, _DTYPES[prior.dtype] if prior is not None else 0,
        a.data_ptr(), a_s, b.data_ptr(), b_s, M, d, r, V,
        out_ids.data_ptr(), out_score.data_ptr(), ld_out,
        ws.data_ptr(), ws.numel(), _stream_ptr(dev)), "dels_lowrank_argmax")
    return out_ids, out_score




def gather_argmax(tokens: torch.Tensor, embedding: torch.Tensor, lm_head_weight: Weight, base_logits: torch.Tensor,
                  baseline_logits: Optional[torch.Tensor] = None, alpha: Scalars = 1.0, beta: Scalars = 0.0,
                  *, out_ids: Optional[torch.Tensor] = None,
                  out_score: Optional[torch.Tensor] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """One Markov DeLS step: ``fused_argmax`` with the rank gathered from a table,
    ``rank = F.embedding(tokens, embedding)`` (code/kernel/markov_dels.py:216-268).

    ``tokens`` [M] int64 (a strided view is fine; ids are clamped to the table);
    ``embedding`` [rows, r] bf16 row-major; the rest as ``fused_argmax``.
    """
    _require_cuda(tokens, "tokens")
    if tokens.dtype != torch.int64:
        raise TypeError("tokens must be int64")
    if tokens.dim() != 1:
        tokens = tokens.reshape(-1)
    M = tokens.numel()
    _require_bf16_matrix(embedding, "embedding")
    rows, r = embedding.shape
    b_ptr, ldb, b_lay, V, _ = _weight(lm_head_weight, "lm_head_weight", cols=r)
    base = _base_view(base_logits, M, V)
    prior = _prior_view(baseline_logits, V)
    dev = tokens.device
    a, a_s = _rows_param(alpha, M, dev, "alpha")
    b, b_s = _rows_param(beta, M, dev, "beta")
    out_ids, out_score, ld_out = _outputs(out_ids, out_score, M, dev)
    lib = _lib.load()
    ws = workspace(dev, lib.dels_gather_argmax_ws_bytes(M, r, V))
    _lib.check(lib.dels_gather_argmax(
        tokens.data_ptr(), tokens.stride(0), embedding.data_ptr(), embedding.stride(0), rows, b_ptr, ldb, b_lay,
        base.data_ptr(), base.stride(0), _DTYPES[base.dtype],
        prior.data_ptr() if prior is not None else None, _DTYPES[prior.dtype] if prior is not None else 0,
        a.data_ptr(), a_s, b.data_ptr(), b_s, M, r, V,
        out_ids.data_ptr(), out_score.data_ptr(), ld_out,
        ws.data_ptr(), ws.numel(), _stream_ptr(dev)), "dels_gather_argmax")
    return out_ids, out_score


def argmax_rows(logits: torch.Tensor, *, out_ids: Optional[torch.Tensor] = None,
                out_score: Optional[torch.Tensor] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """``sample()`` at temperature 0 (code/dflash.py:31-33): the lowest index of
    each row's maximum over the last dimension.  ``logits`` [M, V] (any row
    stride, unit column stride) fp32/bf16/fp16.  As ``torch.argmax``, the first
    NaN of a row wins (score NaN); an all -inf row gives id 0.  Returns
    ``(ids int64[M], score fp32[M])``."""
    if logits.dim() == 1:
        logits = logits.unsqueeze(0)
    _require_cuda(logits, "logits")
    if logits.dtype not in _DTYPES:
        raise TypeError(f"logits must be float32, bfloat16 or float16, got {logits.dtype}")
    if logits.dim() != 2 or (logits.shape[1] > 1 and logits.stride(1) != 1):
        raise ValueError("logits must be an [M, V] matrix with unit column stride")
    M, V = logits.shape
    out_ids, out_score, ld_out = _outputs(out_ids, out_score, M, logits.device)
    lib = _lib.load()
    ws = workspace(logits.device, lib.dels_argmax_rows_ws_bytes(M, V))
    _lib.check(lib.dels_argmax_rows(logits.data_ptr(), logits.stride(0), _DTYPES[logits.dtype], M, V,
                                    out_ids.data_ptr(), out_score.data_ptr(), ld_out, ws.data_ptr(), ws.numel(),
                                    _stream_ptr(logits.device)), "dels_argmax_rows")
    return out_ids, out_score


def lm_head(hidden: torch.Tensor, weight: Weight, *, out: Optional[torch.Tensor] = None, argmax_period: int = 0,
            out_ids: Optional[torch.Tensor] = None,
            out_score: Optional[torch.Tensor] = None) -> tuple[Optional[torch.Tensor], Optional[torch.Tensor],
                                                             Optional[torch.Tensor]]:
    """``bf16(hidden . W^T)`` (code/dflash.py:468) with ``sample()`` of chosen rows fused
    (code/dflash.py:475).  ``hidden`` [M, K] bf16; ``weight`` [V, K] (from ``pack_lm_head``,
    or a bf16 matrix packed on the fly), K a multiple of 256.  With ``argmax_period`` p > 0
    the rows m = j*p are argmaxed instead of stored (ids/scores [ceil(M/p)]).  ``out``
    ([M, V] bf16, unit column stride) receives the other rows; allocated when None and
    some row is stored.  Returns ``(out, ids, scores)`` (None where absent)."""
    _require_bf16_matrix(hidden, "hidden")
    M, K = hidden.shape
    if not isinstance(weight, PackedWeight):
        weight = pack_lm_head(weight)
    if weight.kchunk != LM_HEAD_KCHUNK:
        raise ValueError("weight must be packed by pack_lm_head")
    _require_cuda(weight.data, "weight")
    if weight.cols != K:
        raise ValueError(f"weight has {weight.cols} columns, expected {K}")
    V = weight.rows
    dev = hidden.device
    p = int(argmax_period)
    stores = p != 1
    if out is None and stores:
        out = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
    if out is not None:
        _require_bf16_matrix(out, "out", rows=M, cols=V)
    nrows = (M + p - 1) // p if p > 0 else 0
    ids = sc = None
    ld_out = 1
    if p > 0:
        ids, sc, ld_out = _outputs(out_ids, out_score, nrows, dev)
    lib = _lib.load()
    ws = workspace(dev, lib.dels_lm_head_ws_bytes(M, K, V))
    _lib.check(lib.dels_lm_head(hidden.data_ptr(), hidden.stride(0), weight.data.data_ptr(), M, K, V,
                                out.data_ptr() if out is not None else None, out.stride(0) if out is not None else V,
                                p, ids.data_ptr() if ids is not None else None,
                                sc.data_ptr() if sc is not None else None, ld_out, ws.data_ptr(), ws.numel(),
                                _stream_ptr(dev)), "dels_lm_head")
    return out, ids, sc


def domino_argmax(z: torch.Tensor, s: torch.Tensor, fc2_weight: Weight, base_logits: torch.Tensor,
                  guidance_alpha: float, fc2_bias: Optional[torch.Tensor] = None, *, middle: str = "silu",
                  out_ids: Optional[torch.Tensor] = None,
                  out_score: Optional[torch.Tensor] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """One Domino correction step (code/kernel/domino.py:58-173, 404-431, 438-482):
    ``argmax_v fma(f(z + s) . fc2[v] (+ fc2_bias[v]), alpha, base[v])`` per row, with
    ``f(z + s)`` kept in fp32; ``f`` is the correction MLP's middle layer, one of
    ``silu`` (the reference's fused case), ``identity``, ``relu``, ``gelu``,
    ``gelu_tanh``, ``tanh``, ``sigmoid``.  ``z``, ``s`` [M, E] bf16 (any row stride);
    ``fc2_weight`` [V, E] (a ``PackedWeight``, or a bf16 matrix packed on the fly);
    ``base_logits`` [M, V].  Returns ``(ids int64[M], score fp32[M])``."""
    if middle not in _lib.MIDDLE_CODES:
        raise ValueError(f"middle must be one of {sorted(_lib.MIDDLE_CODES)}, got {middle!r}")
    _require_bf16_matrix(z, "z")
    M, E = z.shape
    _require_bf16_matrix(s, "s", rows=M, cols=E)
    if not isinstance(fc2_weight, PackedWeight):
        fc2_weight = pack_operand(fc2_weight)
    if fc2_weight.kchunk:
        raise ValueError("fc2_weight is packed for the LM head (pack_lm_head); use pack_operand")
    _require_cuda(fc2_weight.data, "fc2_weight")
    if fc2_weight.cols != E:
        raise ValueError(f"fc2_weight has {fc2_weight.cols} columns, expected {E}")
    V = fc2_weight.rows
    base = _base_view(base_logits, M, V)
    bias = _prior_view(fc2_bias, V) if fc2_bias is not None else None
    dev = z.device
    out_ids, out_score, ld_out = _outputs(out_ids, out_score, M, dev)
    lib = _lib.load()
    ws = workspace(dev, lib.dels_domino_argmax_ws_bytes(M, E, V))
    _lib.check(lib.dels_domino_argmax(
        z.data_ptr(), z.stride(0), s.data_ptr(), s.stride(0), fc2_weight.data.data_ptr(),
        bias.data_ptr() if bias is not None else None, _DTYPES[bias.dtype] if bias is not None else 0,
        base.data_ptr(), base.stride(0), _DTYPES[base.dtype], float(guidance_alpha), _lib.MIDDLE_CODES[middle],
        M, E, V, out_ids.data_ptr(), out_score.data_ptr(), ld_out, ws.data_ptr(), ws.numel(), _stream_ptr(dev)),
        "dels_domino_argmax")
    return out_ids, out_score


def sample_rows(logits: torch.Tensor, temperature: float, seed: int, offset: int = 0, *,
                out_ids: Optional[torch.Tensor] = None,
                out_score: Optional[torch.Tensor] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """One draw per row from ``softmax(logits / temperature)`` (code/dflash.py:31-38).

    A Gumbel-max over Philox4x32-10 noise keyed by ``seed`` (64 bits) at counter
    ``(v // 4, row, offset)``: the ids depend only on ``(seed, offset, row,
    logits)``.  ``temperature < 1e-5`` is ``argmax_rows``, as in the reference.
    ``logits`` [M, V] (unit column stride) fp32/bf16/fp16.  Returns
    ``(ids int64[M], score fp32[M])``, the score being the winning
    ``logits / temperature + gumbel`` value."""
    if logits.dim() == 1:
        logits = logits.unsqueeze(0)
    _require_cuda(logits, "logits")
    if logits.dtype not in _DTYPES:
        raise TypeError(f"logits must be float32, bfloat16 or float16, got {logits.dtype}")
    if logits.dim() != 2 or (logits.shape[1] > 1 and logits.stride(1) != 1):
        raise ValueError("logits must be an [M, V] matrix with unit column stride")
    M, V = logits.shape
    out_ids, out_score, ld_out = _outputs(out_ids, out_score, M, logits.device)
    lib = _lib.load()
    ws = workspace(logits.device, lib.dels_sample_rows_ws_bytes(M, V))
    _lib.check(lib.dels_sample_rows(logits.data_ptr(), logits.stride(0), _DTYPES[logits.dtype], M, V,
                                    float(temperature), int(seed) & (2**64 - 1), int(offset) & (2**64 - 1),
                                    out_ids.data_ptr(), out_score.data_ptr(), ld_out, ws.data_ptr(), ws.numel(),
                                    _stream_ptr(logits.device)), "dels_sample_rows")
    return out_ids, out_score


# ---- fp8 variant (e4m3 weights with per-output-channel scales) -----------------

E4M3_MAX = 448.0
FP8_LAYOUTS = {"k128": _lib.LAYOUT_FP8_K128, "k32": _lib.LAYOUT_FP8_K32}


@dataclass
class Fp8Weight:
    """An e4m3 [rows, cols] weight, packed, with its per-row fp32 scale.

    ``layout`` "k128" is the fp8 argmax's B operand (16 x 128 blocks of 2 KiB,
    include/dels.h DELS_LAYOUT_FP8_K128); "k32" is the rank projection's A
    (16 x 32 blocks of 512 bytes, DELS_LAYOUT_FP8_K32).  ``W ~= q * scale[:, None]``.
    """

    data: torch.Tensor    # packed e4m3 bytes (uint8)
    scale: torch.Tensor   # [rows] fp32
    rows: int
    cols: int
    layout: str


def quantize_e4m3_rows(W: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row absmax e4m3fn quantisation: ``(q uint8 [rows, cols], scale fp32 [rows])``.

    ``scale = absmax / 448`` (1 for an all-zero row) and ``q = e4m3(W / scale)``
    rounded to nearest even (torch's float8_e4m3fn cast); every |W / scale| is
    at most 448, so nothing saturates.  Weight preparation, not the hot path.
    """
    if W.dim() != 2:
        raise ValueError("W must be 2-D")
    w = W.float()
    amax = w.abs().amax(dim=1)
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    q = (w / scale[:, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    return q.contiguous(), scale.contiguous()


def pack_operand_fp8(q: torch.Tensor, scale: torch.Tensor, layout: str) -> Fp8Weight:
    """Pack row-major e4m3 bytes ``q`` [rows, cols] (uint8 or float8_e4m3fn) into ``layout``."""
    if layout not in FP8_LAYOUTS:
        raise ValueError(f"layout must be one of {sorted(FP8_LAYOUTS)}")
    _require_cuda(q, "q")
    _require_cuda(scale, "scale")
    if q.dtype == torch.float8_e4m3fn:
        q = q.view(torch.uint8)
    if q.dtype != torch.uint8 or q.dim() != 2:
        raise ValueError("q must be a 2-D uint8 (e4m3fn bytes) tensor")
    if q.shape[1] > 1 and q.stride(1) != 1:
        raise ValueError("q must have unit column stride")
    rows, cols = q.shape
    if scale.dtype != torch.float32 or scale.numel() != rows:
        raise ValueError("scale must be an fp32 vector with one entry per row")
    lib = _lib.load()
    code = FP8_LAYOUTS[layout]
    nbytes = max(int(lib.dels_packed_fp8_bytes(rows, cols, code)), 16)
    buf = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
    _lib.check(lib.dels_pack_operand_fp8(q.data_ptr(), q.stride(0), rows, cols, code, buf.data_ptr(), buf.numel(),
                                         _stream_ptr(q.device)), "dels_pack_operand_fp8")
    return Fp8Weight(buf, scale.contiguous(), int(rows), int(cols), layout)


def quantize_pack_fp8(W: torch.Tensor, layout: str) -> Fp8Weight:
    """``quantize_e4m3_rows`` then ``pack_operand_fp8``."""
    q, scale = quantize_e4m3_rows(W)
    return pack_operand_fp8(q, scale, layout)


def _fp8_weight(w: Fp8Weight, name: str, layout: str, cols: int) -> Fp8Weight:
    if not isinstance(w, Fp8Weight) or w.layout != layout:
        raise TypeError(f"{name} must be an Fp8Weight in the {layout!r} layout (pack_operand_fp8)")
    if w.cols != cols:
        raise ValueError(f"{name} has {w.cols} columns, expected {cols}")
    _require_cuda(w.data, name)
    return w


def fused_argmax_fp8(rank: torch.Tensor, lm_head_weight: Fp8Weight, base_logits: torch.Tensor,
                     baseline_logits: Optional[torch.Tensor] = None, alpha: Scalars = 1.0, beta: Scalars = 0.0,
                     *, out_ids: Optional[torch.Tensor] = None,
                     out_score: Optional[torch.Tensor] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """``fused_argmax`` with an e4m3 LM head (``Fp8Weight``, layout "k128").

    Each rank row is quantised in the kernel to e4m3 (scale absmax/448); the
    dot is ``fp32(R_q . B_q[v]) * sR[m] * sB[v]``.  r must be 128, 256 or 512.
    """
    if rank.dim() == 1:
        rank = rank.unsqueeze(0)
    M, r = rank.shape
    _require_bf16_matrix(rank, "rank", cols=r)
    B = _fp8_weight(lm_head_weight, "lm_head_weight", "k128", r)
    V = B.rows
    base = _base_view(base_logits, M, V)
    prior = _prior_view(baseline_logits, V)
    dev = rank.device
    a, a_s = _rows_param(alpha, M, dev, "alpha")
    b, b_s = _rows_param(beta, M, dev, "beta")
    out_ids, out_score, ld_out = _outputs(out_ids, out_score, M, dev)
    lib = _lib.load()
    ws = workspace(dev, lib.dels_fused_argmax_fp8_ws_bytes(M, r, V))
    _lib.check(lib.dels_fused_argmax_fp8(
        rank.data_ptr(), rank.stride(0), B.data.data_ptr(), B.scale.data_ptr(),
        base.data_ptr(), base.stride(0), _DTYPES[base.dtype],
        prior.data_ptr() if prior is not None else None, _DTYPES[prior.dtype] if prior is not None else 0,
        a.data_ptr(), a_s, b.data_ptr(), b_s, M, r, V,
        out_ids.data_ptr(), out_score.data_ptr(), ld_out,
        ws.data_ptr(), ws.numel(), _stream_ptr(dev)), "dels_fused_argmax_fp8")
    return out_ids, out_score


def lowrank_argmax_fp8(h: torch.Tensor, rank_weight: Fp8Weight, lm_head_weight: Fp8Weight,
                       base_logits: torch.Tensor, baseline_logits: Optional[torch.Tensor] = None,
                       alpha: Scalars = 1.0, beta: Scalars = 0.0, act: str = "identity",
                       rank_bias: Optional[torch.Tensor] = None, *, out_ids: Optional[torch.Tensor] = None,
                       out_score: Optional[torch.Tensor] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """``lowrank_argmax`` with e4m3 weights: A (layout "k32") and B (layout "k128").

    rank = bf16(act(bf16(fp32(h . A_q^T) * sA + bias))), then ``fused_argmax_fp8``.
    """
    if act not in _ACTS:
        raise ValueError(f"Unsupported DeLS rank_activation={act!r}.")
    if h.dim() == 1:
        h = h.unsqueeze(0)
    M, d = h.shape
    _require_bf16_matrix(h, "h", cols=d)
    A = _fp8_weight(rank_weight, "rank_weight", "k32", d)
    r = A.rows
    B = _fp8_weight(lm_head_weight, "lm_head_weight", "k128", r)
    V = B.rows
    base = _base_view(base_logits, M, V)
    prior = _prior_view(baseline_logits, V)
    rank_bias = _bias(rank_bias, r)
    dev = h.device
    a, a_s = _rows_param(alpha, M, dev, "alpha")
    b, b_s = _rows_param(beta, M, dev, "beta")
    out_ids, out_score, ld_out = _outputs(out_ids, out_score, M, dev)
    lib = _lib.load()
    ws = workspace(dev, lib.dels_lowrank_argmax_fp8_ws_bytes(M, d, r, V))
    _lib.check(lib.dels_lowrank_argmax_fp8(
        h.data_ptr(), h.stride(0), A.data.data_ptr(), A.scale.data_ptr(),
        rank_bias.data_ptr() if rank_bias is not None else None, _ACTS[act],
        B.data.data_ptr(), B.scale.data_ptr(),
        base.data_ptr(), base.stride(0), _DTYPES[base.dtype],
        prior.data_ptr() if prior is not None else None, _DTYPES[prior.dtype] if prior is not None else 0,
        a.data_ptr(), a_s, b.data_ptr(), b_s, M, d, r, V,
        out_ids.data_ptr(), out_score.data_ptr(), ld_out,
        ws.data_ptr(), ws.numel(), _stream_ptr(dev)), "dels_lowrank_argmax_fp8")
    return out_ids, out_score


def gru_step(gi_table: torch.Tensor, tokens: torch.Tensor, h_in: Optional[torch.Tensor],
             w_hh: Weight, b_hh: Optional[torch.Tensor] = None, *,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``h_out = GRUCell(gi_table[tokens], h_in)`` with bf16 state (code/kernel/dels.py:359-373).

    ``gi_table`` [rows, 3G] bf16 is ``F.linear(E, W_ih, b_ih)``; ``tokens`` [B]
    int64 (a strided view is fine); ``h_in`` [B, G] bf16 or None for zeros;
    ``w_hh`` [3G, G] bf16 (row-major contiguous or packed); ``b_hh`` [3G] bf16 or None.
    """
    _require_cuda(tokens, "tokens")
    if tokens.dtype != torch.int64:
        raise TypeError("tokens must be int64")
    tokens = tokens.reshape(-1) if tokens.dim() != 1 else tokens
    nb = tokens.numel()
    G = w_hh.shape[1]
    w_ptr, ldw, w_lay, _, _ = _weight(w_hh, "w_hh", rows=3 * G, cols=G)
    if w_lay == _lib.LAYOUT_ROWMAJOR and ldw != G:
        raise ValueError("w_hh must be contiguous")
    _require_bf16_matrix(gi_table, "gi_table", cols=3 * G)
    if h_in is not None:
        _require_bf16_matrix(h_in, "h_in", rows=nb, cols=G)
    if b_hh is not None:
        if b_hh.dtype != torch.bfloat16 or b_hh.numel() != 3 * G:
            raise ValueError("b_hh must be a bfloat16 vector of length 3G")
        b_hh = b_hh.contiguous()
    dev = tokens.device
    if out is None:
        out = torch.empty(nb, G, dtype=torch.bfloat16, device=dev)
    else:
        _require_bf16_matrix(out, "out", rows=nb, cols=G)
    lib = _lib.load()
    ws = workspace(dev, lib.dels_gru_step_ws_bytes(nb, G))
    _lib.check(lib.dels_gru_step(
        gi_table.data_ptr(), gi_table.stride(0), gi_table.shape[0], tokens.data_ptr(), tokens.stride(0),
        h_in.data_ptr() if h_in is not None else None, h_in.stride(0) if h_in is not None else G,
        w_ptr, w_lay, b_hh.data_ptr() if b_hh is not None else None, nb, G,
        out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), _stream_ptr(dev)), "dels_gru_step")
    return out

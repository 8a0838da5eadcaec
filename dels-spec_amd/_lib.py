"""ctypes binding of the gfx950 C-ABI library (include/dels.h).

The library is built in-tree by ``build.py`` into ``_lib/libdels_mi355x.so``.
There is no fallback: if the library is missing or cannot be loaded, every
operation raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  -- loads torch's HIP runtime first, so the library binds to it

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
# DELS_LIBRARY_PATH names another build of the same library (an instrumented
# one, say); by default the in-tree build is loaded.
LIB_PATH = os.environ.get("DELS_LIBRARY_PATH") or os.path.join(_PKG_DIR, "_lib", "libdels_mi355x.so")

ABI_VERSION = 3
DELS_OK = 0
DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
ACT_IDENTITY, ACT_SILU = 0, 1
LAYOUT_ROWMAJOR, LAYOUT_MFMA16 = 0, 1
LAYOUT_FP8_K128, LAYOUT_FP8_K32 = 2, 3
# the Domino correction MLP's middle layer (DELS_MIDDLE_*): name -> code
MIDDLE_CODES = {"silu": 0, "identity": 1, "relu": 2, "gelu": 3, "gelu_tanh": 4, "tanh": 5, "sigmoid": 6}
NOALLOC_SCRATCH_BYTES = 16 << 20      # DELS_NOALLOC_SCRATCH_BYTES

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_sz = ctypes.c_size_t
_fptr = ctypes.c_void_p


class RolloutParams(ctypes.Structure):
    """Mirror of ``struct dels_rollout`` in include/dels.h."""

    _fields_ = [
        ("gi_table", _ptr), ("ld_gi", _i64), ("table_rows", _i64),
        ("w_hh", _ptr), ("b_hh", _ptr),
        ("rank_w", _ptr), ("rank_b", _ptr), ("act", _int),
        ("lm_w", _ptr),
        ("prior", _ptr), ("prior_dtype", _int),
        ("alpha", _fptr), ("beta", _fptr),
        ("batch", _i64), ("steps", _i64), ("G", _i64), ("r", _i64), ("V", _i64),
        ("weights_layout", _int),
        ("prefix_ids", _ptr),
        ("base", _ptr), ("base_dtype", _int), ("ld_base", _i64),
        ("out_ids", _ptr), ("out_scores", _ptr),
        ("h_a", _ptr), ("h_b", _ptr),
        ("rank", _ptr),
        ("ws", _ptr), ("ws_bytes", _sz),
        ("ld_prefix", _i64), ("ld_out", _i64),
    ]


class DominoRolloutParams(ctypes.Structure):
    """Mirror of ``struct dels_domino_rollout`` in include/dels.h."""

    _fields_ = [
        ("gi_table", _ptr), ("ld_gi", _i64), ("table_rows", _i64),
        ("w_hh", _ptr), ("b_hh", _ptr),
        ("w_z", _ptr), ("fc1_bias", _ptr), ("w_s", _ptr),
        ("fc2_w", _ptr), ("fc2_bias", _ptr), ("fc2_bias_dtype", _int),
        ("alpha", ctypes.c_float),
        ("batch", _i64), ("steps", _i64), ("prefix_len", _i64), ("D", _i64), ("G", _i64), ("E", _i64),
        ("V", _i64),
        ("weights_layout", _int),
        ("prefix_ids", _ptr),
        ("hiddens", _ptr),
        ("base", _ptr), ("base_dtype", _int), ("ld_base", _i64),
        ("out_ids", _ptr), ("out_scores", _ptr),
        ("h_a", _ptr), ("h_b", _ptr),
        ("z", _ptr), ("s", _ptr),
        ("ws", _ptr), ("ws_bytes", _sz),
        ("middle", _int),
    ]


class MarkovRolloutParams(ctypes.Structure):
    """Mirror of ``struct dels_markov_rollout`` in include/dels.h."""

    _fields_ = [
        ("embedding", _ptr), ("ld_embedding", _i64), ("table_rows", _i64),
        ("lm_w", _ptr), ("lm_layout", _int),
        ("prior", _ptr), ("prior_dtype", _int),
        ("alpha", _fptr), ("beta", _fptr),
        ("batch", _i64), ("steps", _i64), ("r", _i64), ("V", _i64),
        ("prev_ids", _ptr),
        ("base", _ptr), ("base_dtype", _int), ("ld_base", _i64),
        ("out_ids", _ptr), ("out_scores", _ptr),
        ("ws", _ptr), ("ws_bytes", _sz),
    ]


# name -> (restype, argtypes); every symbol include/dels.h declares.
SIGNATURES = {
    "dels_abi_version": (_int, []),
    "dels_strerror": (ctypes.c_char_p, [_int]),
    "dels_last_error": (ctypes.c_char_p, []),
    "dels_workspace_init": (_int, [_ptr, _sz, _ptr]),
    "dels_packed_bytes": (_sz, [_i64, _i64]),
    "dels_pack_operand": (_int, [_ptr, _i64, _i64, _i64, _ptr, _sz, _ptr]),
    "dels_rank_proj_ws_bytes": (_sz, [_i64, _i64, _i64]),
    "dels_rank_proj": (_int, [_ptr, _i64, _ptr, _i64, _int, _ptr, _int, _i64, _i64, _i64, _ptr, _i64, _ptr, _sz,
                              _ptr]),
    "dels_fused_argmax_ws_bytes": (_sz, [_i64, _i64, _i64]),
    "dels_fused_argmax": (_int, [_ptr, _i64, _ptr, _i64, _int, _ptr, _i64, _int, _ptr, _int, _fptr, _i64, _fptr, _i64,
                                 _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr, _sz, _ptr]),
    "dels_debug_set_decode_spin_limit": (_int, [_int]),
    "dels_debug_set_rollout_resident": (_int, [_int]),
    "dels_debug_set_resident_spin_limit": (_int, [_int]),
    "dels_lowrank_argmax_ws_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "dels_lowrank_argmax": (_int, [_ptr, _i64, _ptr, _i64, _int, _ptr, _int, _ptr, _i64, _int, _ptr, _i64, _int, _ptr,
                                   _int,
                                   _fptr, _i64, _fptr, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr, _sz,
                                   _ptr]),
    "dels_lowrank_argmax_noalloc": (_int, [_ptr, _i64, _ptr, _i64, _int, _ptr, _int, _ptr, _i64, _int, _ptr, _i64,
                                           _int, _ptr, _int, _fptr, _i64, _fptr, _i64, _i64, _i64, _i64, _i64, _ptr,
                                           _ptr, _i64, _ptr]),
    "dels_gru_step_ws_bytes": (_sz, [_i64, _i64]),
    "dels_gru_step": (_int, [_ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, _int, _ptr, _i64, _i64, _ptr, _i64, _ptr,
                             _sz, _ptr]),
    "dels_rollout_ws_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "dels_rollout_enqueue": (_int, [ctypes.POINTER(RolloutParams), _ptr]),
    "dels_graph_create": (_int, [ctypes.POINTER(RolloutParams), ctypes.POINTER(_ptr)]),
    "dels_graph_launch": (_int, [_ptr, _ptr]),
    "dels_graph_destroy": (_int, [_ptr]),
    "dels_gather_argmax_ws_bytes": (_sz, [_i64, _i64, _i64]),
    "dels_gather_argmax": (_int, [_ptr, _i64, _ptr, _i64, _i64, _ptr, _i64, _int, _ptr, _i64, _int, _ptr, _int, _fptr,
                                  _i64, _fptr, _i64, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr, _sz, _ptr]),
    "dels_markov_rollout_ws_bytes": (_sz, [_i64, _i64, _i64]),
    "dels_markov_rollout_enqueue": (_int, [ctypes.POINTER(MarkovRolloutParams), _ptr]),
    "dels_markov_graph_create": (_int, [ctypes.POINTER(MarkovRolloutParams), ctypes.POINTER(_ptr)]),
    "dels_argmax_rows_ws_bytes": (_sz, [_i64, _i64]),
    "dels_argmax_rows": (_int, [_ptr, _i64, _int, _i64, _i64, _ptr, _ptr, _i64, _ptr, _sz, _ptr]),
    "dels_lm_head_ws_bytes": (_sz, [_i64, _i64, _i64]),
    "dels_pack_lm_head": (_int, [_ptr, _i64, _i64, _i64, _ptr, _sz, _ptr]),
    "dels_lm_head": (_int, [_ptr, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _ptr, _sz, _ptr]),
    "dels_domino_argmax_ws_bytes": (_sz, [_i64, _i64, _i64]),
    "dels_domino_argmax": (_int, [_ptr, _i64, _ptr, _i64, _ptr, _ptr, _int, _ptr, _i64, _int, ctypes.c_float,
                                  _int, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr, _sz, _ptr]),
    "dels_domino_rollout_ws_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64, _i64]),
    "dels_domino_rollout_enqueue": (_int, [ctypes.POINTER(DominoRolloutParams), _ptr]),
    "dels_domino_graph_create": (_int, [ctypes.POINTER(DominoRolloutParams), ctypes.POINTER(_ptr)]),
    "dels_sample_rows_ws_bytes": (_sz, [_i64, _i64]),
    "dels_sample_rows": (_int, [_ptr, _i64, _int, _i64, _i64, ctypes.c_float, ctypes.c_uint64, ctypes.c_uint64, _ptr,
                                _ptr, _i64, _ptr, _sz, _ptr]),
    "dels_packed_fp8_bytes": (_sz, [_i64, _i64, _int]),
    "dels_pack_operand_fp8": (_int, [_ptr, _i64, _i64, _i64, _int, _ptr, _sz, _ptr]),
    "dels_fused_argmax_fp8_ws_bytes": (_sz, [_i64, _i64, _i64]),
    "dels_fused_argmax_fp8": (_int, [_ptr, _i64, _ptr, _fptr, _ptr, _i64, _int, _ptr, _int, _fptr, _i64, _fptr,
                                     _i64, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr, _sz, _ptr]),
    "dels_lowrank_argmax_fp8_ws_bytes": (_sz, [_i64, _i64, _i64, _i64]),
    "dels_lowrank_argmax_fp8": (_int, [_ptr, _i64, _ptr, _fptr, _ptr, _int, _ptr, _fptr, _ptr, _i64, _int, _ptr,
                                       _int, _fptr, _i64, _fptr, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _i64,
                                       _ptr, _sz, _ptr]),
}

_lock = threading.Lock()
_lib = None


class DelsError(RuntimeError):
    """A nonzero status returned by the C ABI."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def load() -> ctypes.CDLL:
    """Load the library once and attach the argument/return types."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"DeLS HIP library not found at {LIB_PATH}; build it with "
                "`python dels-spec_amd/build.py` (or __graft_entry__.build()).")
        lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.dels_abi_version() != ABI_VERSION:
            raise RuntimeError("DeLS HIP library ABI version mismatch")
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    """Raise ``DelsError`` for a nonzero C-ABI status."""
    if status != DELS_OK:
        lib = load()
        name = lib.dels_strerror(status).decode()
        detail = lib.dels_last_error().decode()
        raise DelsError(status, f"{what} failed ({name}): {detail}")

"""ctypes binding of libtrida_hip.so, the C ABI declared in include/trida_hip.h.

The library is the only compute path of this package: there is no CPU or PyTorch fallback, and every
wrapper raises when the library is missing.
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libtrida_hip.so"

TRIDA_OK = 0
TRIDA_ERR_ARG = -1
TRIDA_ERR_NULL = -2
TRIDA_ERR_ALIGN = -3
TRIDA_ERR_WORKSPACE = -4
TRIDA_ERR_LAUNCH = -5

P = C.c_void_p
I64 = C.c_int64
I32 = C.c_int32
F32 = C.c_float

# name -> (restype, argtypes); one line per entry point of include/trida_hip.h
SIGNATURES = {
    "trida_version": (C.c_int, []),
    "trida_last_error": (C.c_char_p, []),
    "trida_greedy_accept_scratch_bytes": (I64, [I64, I64, I64, C.c_int, I64]),
    "trida_greedy_accept": (C.c_int, [P, C.c_int, I64, I64, I64, I64, I64, P, I64, I64, P, P, P, P, P, P, P, I64, I64, P]),
    "trida_greedy_accept_noalloc": (C.c_int, [P, C.c_int, I64, I64, I64, I64, I64, P, I64, I64, P, P, P, P, P, P, I64,
                                              P]),
    "trida_row_argmax_scratch_bytes": (I64, [I64, I64, C.c_int, I64]),
    "trida_row_argmax": (C.c_int, [P, C.c_int, I64, I64, I64, P, P, P, I64, I64, P]),
    "trida_unmask_top": (C.c_int, [P, P, I64, P, P, I64, I64, I64, I64, P]),
    "trida_canvas_advance": (C.c_int, [P, I64, P, P, I64, P, P, P, P, P, P, I64, I64, I64, P]),
    "trida_ban_tokens": (C.c_int, [P, C.c_int, I64, I64, I64, P, I64, P]),
    "trida_gate_tokens": (C.c_int, [P, C.c_int, I64, I64, I64, P, P, I64, P, P]),
    "trida_sample_accept_scratch_bytes": (I64, [I64, I64, I64, I64]),
    "trida_sample_accept": (C.c_int, [P, I64, I64, I64, I64, I64, P, I64, I64, P, I64, I64, P, P, I64, P, P,
                                      F32, I64, F32, I64, P, P, P, P, P, P, I64, P]),
    "trida_truncate_stats": (C.c_int, [P, I64, I64, I64, I64, I64, F32, I64, F32, I64, C.c_int, P, P, P, P, P, P]),
    "trida_sample_rows_scratch_bytes": (I64, [I64, I64]),
    "trida_sample_rows": (C.c_int, [P, I64, I64, I64, F32, I64, P, P, P, P, P, P, I64, P]),
    "trida_truncated_probs": (C.c_int, [P, I64, I64, I64, I64, I64, F32, I64, P, P, P, P, I64, I64, P]),
    "trida_truncated_probs_rows": (C.c_int, [P, I64, I64, I64, I64, I64, F32, I64, P, P, P, P, P, I64, P, I64, I64,
                                             I64, P]),
    "trida_gather_rows": (C.c_int, [P, C.c_int, I64, I64, I64, I64, I64, P, I64, P, I64, I64, P]),
    "trida_wsgemm_shuffle": (C.c_int, [P, I64, I64, I64, C.c_int, P, C.c_int, P, P]),
    "trida_wsgemm_plan": (C.c_int, [I64, I64, C.c_int, P]),
    "trida_wsgemm": (C.c_int, [P, I64, P, I64, I64, I64, C.c_int, P, I64, P]),
    "trida_wsgemm_norm": (C.c_int, [P, I64, P, F32, P, I64, I64, I64, C.c_int, P, I64, P]),
    "trida_residual_ss_chunks": (I64, [I64]),
    "trida_residual_parts": (C.c_int, [P, I64, P, I64, I64, I64, I64, P, P]),
    "trida_ws_frag_elems": (I64, [I64]),
    "trida_wsgemm_argmax_splits": (I64, [I64, I64]),
    "trida_wsgemm_argmax": (C.c_int, [P, I64, P, I64, I64, I64, C.c_int, P, I64, P, P, P]),
    "trida_greedy_accept_splits": (C.c_int, [P, P, I64, I64, I64, P, I64, I64, P, P, P, P, P, P, P]),
    "trida_wsgemm_argmax_conf": (C.c_int, [P, I64, P, I64, I64, I64, C.c_int, P, I64, P, P, P, P]),
    "trida_argmax_conf_splits": (C.c_int, [P, P, P, I64, I64, I64, P, P, I64, P]),
    "trida_gdr_recurrent_gnorm": (C.c_int, [P] * 9 + [I64] * 6 + [C.c_int, I64, C.c_float, P, I64, P, P, P, P]),
    "trida_wsgemm_headnorm_planes": (C.c_int, [I64, I64, I64, P]),
    "trida_wsgemm_headnorm": (C.c_int, [P, P, I64, I64, I64, P, I64, C.c_float, P, P]),
    "trida_ws_frag": (C.c_int, [P, I64, I64, I64, P, P]),
    "trida_wsgemm_ex": (C.c_int, [P, I64, P, F32, P, I64, I64, I64, C.c_int, P, I64, C.c_int, P]),
    "trida_residual_parts_frag": (C.c_int, [P, I64, P, I64, I64, I64, I64, P, P, P]),
    "trida_add_rmsnorm": (C.c_int, [P, P, P, P, I64, I64, I64, I64, I64, F32, C.c_int, P]),
    "trida_add_rmsnorm_parts": (C.c_int, [P, P, I64, I64, P, P, I64, I64, I64, I64, F32, C.c_int, P]),
    "trida_silu_mul": (C.c_int, [P, P, I64, I64, I64, I64, P]),
    "trida_gated_rmsnorm": (C.c_int, [P, P, P, P, I64, I64, I64, I64, F32, P]),
    "trida_gated_rmsnorm_frag": (C.c_int, [P, P, P, P, I64, I64, I64, I64, F32, P]),
    "trida_attn_prep": (C.c_int, [P, I64, P, P, P, P, P, P, P] + [I64] * 7 + [F32, F32, P]),
    "trida_gdn_prep": (C.c_int, [P] * 14 + [I64] * 11 + [P] * 4 + [P]),
    "trida_gdr_recurrent": (C.c_int, [P] * 9 + [I64] * 6 + [C.c_int, I64, F32] + [P, P, P, P, I64] + [P]),
    "trida_gdn_fused_layer": (C.c_int, [P] * 17 + [I64] * 11 + [C.c_int, I64, F32] + [P] * 5 + [I64, P] + [P]),
    "trida_gdr_block_bidir": (C.c_int, [P] * 8 + [I64] * 7 + [F32, P]),
    "trida_gdr_chunk_workspace_bytes": (I64, [I64, I64, I64]),
    "trida_gdr_chunk": (C.c_int, [P] * 9 + [I64] * 7 + [C.c_int, I64, F32, P, I64] + [P, P] + [P]),
    "trida_gdn_snapshot": (C.c_int, [P, P, I64, P, P, I64, P]),
    "trida_gdn_restore": (C.c_int, [P] * 10 + [I64] * 11 + [C.c_int, P, P, P]),
    "trida_attn_canvas_scratch_bytes": (I64, [I64] * 7),
    "trida_attn_set_combine_general": (C.c_int, [C.c_int]),
    "trida_attn_canvas": (C.c_int, [P, P, P, P, P, I64, I64, P] + [I64] * 6 + [C.c_int, I64, F32, I64, I64, P, I64, P]),
    "trida_attn_canvas_frag": (C.c_int, [P, P, P, P, P, I64, I64, P] + [I64] * 6 + [C.c_int, I64, F32, I64, I64, P, I64,
                                                                                   P]),
}

_lock = threading.Lock()
_lib = None


def load() -> C.CDLL:
    """Loads and types the library once per process; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m trida_stack_amd.build` "
                    "(there is no fallback path)")
            lib = C.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Maps a C-ABI status to the exception the caller sees (ValueError for a rejected argument)."""
    if rc == TRIDA_OK:
        return
    msg = load().trida_last_error().decode(errors="replace")
    if rc == TRIDA_ERR_LAUNCH:
        raise RuntimeError(f"{what}: {msg}")
    raise ValueError(f"{what}: {msg} (status {rc})")

"""ctypes binding of the HIP library `_kve.so` (C ABI declared in include/kve.h).

There is no fallback: if the library is missing or fails to load, every entry
point raises. Build it with `python -m kvengine_amd.build`.
"""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_kve.so")

EXPORTS = (
    "kve_last_error",
    "kve_version",
    "kve_attn_workspace_bytes",
    "kve_paged_verify_attn",
    "kve_attn_plan_bytes",
    "kve_attn_plan",
    "kve_kv_write",
    "kve_commit",
    "kve_rollback",
    "kve_lmhead_workspace_bytes",
    "kve_lmhead_argmax",
    "kve_lmhead_argmax_noalloc",
    "kve_accept",
    "kve_rmsnorm",
    "kve_rope_kv_write",
    "kve_silu_mul",
    "kve_pass_prologue",
    "kve_fused_qkv",
    "kve_linear_residual",
    "kve_fused_gate_up",
    "kve_splitk_slices",
    "kve_linear_splitk",
    "kve_residual_norm",
    "kve_kv_slots",
    "kve_qkv_rope",
    "kve_qkv_part_rope",
    "kve_gate_up_silu",
    "kve_linear_rows",
    "kve_linear_rows_slices",
)

DTYPE_F32 = 0
DTYPE_BF16 = 1

_lock = threading.Lock()
_lib = None

P = ctypes.c_void_p
I = ctypes.c_int
I64 = ctypes.c_int64
F = ctypes.c_float
SZ = ctypes.c_size_t

_SIGS = {
    "kve_last_error": (ctypes.c_char_p, []),
    "kve_version": (ctypes.c_char_p, []),
    "kve_attn_workspace_bytes": (SZ, [I, I, I, I, I, I, I, I, I, I]),
    "kve_paged_verify_attn": (I, [P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, I, I, I, I, F, I, P,
                                  P, P, SZ, I, P]),
    "kve_attn_plan_bytes": (SZ, [I, I, I, I, I, I, I, I, I, I]),
    "kve_attn_plan": (I, [P, P, P, P, I, I, I, I, I, I, I, I, I, I, I, I, I, P, SZ, P]),
    "kve_kv_write": (I, [P, P, I64, P, P, P, P, P, P, I, I, I, I, I, I, I, I, I, P]),
    "kve_commit": (I, [P, I, P, P, I, I, P]),
    "kve_rollback": (I, [P, P, I, P, P, I, I, I, P]),
    "kve_lmhead_workspace_bytes": (SZ, [I]),
    "kve_lmhead_argmax": (I, [P, I64, P, I, I, I, I, P, P, P, P, P, SZ, I, P]),
    "kve_lmhead_argmax_noalloc": (I, [P, I64, P, I, I, I, I, P, P, P, P, P]),
    "kve_accept": (I, [P, P, P, I, P, I, I, P, P, P, P]),
    "kve_rmsnorm": (I, [P, P, P, P, P, I, I, F, I, I, P]),
    "kve_rope_kv_write": (I, [P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, I, I, P]),
    "kve_silu_mul": (I, [P, P, I, I, I, P]),
    "kve_pass_prologue": (I, [P, P, I64, I, P, P, I, I, I, P, P, I, I, P, P, P, P]),
    "kve_fused_qkv": (I, [P, P, F, P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, I, I, I, I, P]),
    "kve_linear_residual": (I, [P, P, P, I, I, I, I, P]),
    "kve_fused_gate_up": (I, [P, P, F, P, P, I, I, I, I, I, P]),
    "kve_splitk_slices": (I, [I, I]),
    "kve_linear_splitk": (I, [P, P, P, I, I, I, I, I, P]),
    "kve_residual_norm": (I, [P, I, P, P, F, P, I, I, I, P]),
    "kve_kv_slots": (I, [P, P, P, P, I, I, I, I, I, I, P, P]),
    "kve_qkv_rope": (I, [P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, I, P]),
    "kve_qkv_part_rope": (I, [P, I, P, P, P, P, P, P, P, I, I, I, I, I, P]),
    "kve_gate_up_silu": (I, [P, P, P, I, I, I, I, P]),
    "kve_linear_rows": (I, [P, P, P, I, I, I, I, I, P]),
    "kve_linear_rows_slices": (I, [I, I, I, I]),
}


class KveError(RuntimeError):
    pass


def lib():
    """Load (once) and return the ctypes library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise KveError(f"HIP library not built: {LIB_PATH} (run python -m kvengine_amd.build)")
        import torch  # noqa: F401  (load torch's HIP runtime first: the library shares it)

        handle = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_LOCAL)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().kve_last_error().decode(errors="replace")
        raise KveError(f"{what} failed ({rc}): {msg}")


def exported_symbols() -> list[str]:
    return [n for n in EXPORTS if hasattr(lib(), n)]

"""ctypes binding of libmla_mi355x.so (the C ABI in include/mla_mi355x.h).

There is deliberately no fallback: if the library is missing or fails to load,
every operator raises ``MlaLibraryError``.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmla_mi355x.so")

MLA_OK = 0
MLA_ERR_INVALID_ARGUMENT = 1
MLA_ERR_UNSUPPORTED = 2
MLA_ERR_WORKSPACE_TOO_SMALL = 3
MLA_ERR_HIP = 4

KV_MODES = {"fp8": 0, "mxfp4": 1, "mxfp4k_fp8v": 2, "bf16": 3}

# Every entry point the header declares, with its ctypes signature.
_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
SIGNATURES = {
    "mla_last_error": (ctypes.c_char_p, []),
    "mla_abi_version": (_I, []),
    "mla_device_cu_count": (_I, [ctypes.POINTER(_I)]),
    "mla_workspace_bytes": (_I, [_I, _I, _I, ctypes.POINTER(_L)]),
    "mla_quant_fp8_per_tensor": (_I, [_P, _L, _P, _P, _P, _L, _P]),
    "mla_pack_mxfp4": (_I, [_P, _L, _I, _L, _P, _L, _P, _L, _P]),
    "mla_append_kv": (_I, [_P, _L, _L, _P, _P, _L, _P, _P, _L, _P, _L, _P, _P]),
    "mla_plan": (_I, [_P, _I, _I, _I, _I, _P, _L, _P]),
    "mla_expand_pages": (_I, [_P, _P, _P, _I, _I, _L, _P, _P, _P]),
    "mla_decode": (_I, [_P, _P, _P, _L, _P, _L, _P, _L, _P, _P, _P, _I, _I, _F, _I, _P, _L, _P, _P, _P]),
    "mla_combine": (_I, [_I, _I, _P, _L, _P, _P, _P]),
    "mla_decode_fwd": (_I, [_P, _P, _L, _P, _L, _P, _L, _P, _P, _P, _I, _I, _I, _F, _I, _P, _L, _P, _P, _P]),
    "mla_decode_fwd_a16w8": (_I, [_P, _P, _L, _P, _L, _P, _L, _P, _P, _P, _I, _I, _I, _F, _I, _P, _L, _P, _P, _P]),
    "mla_decode_fwd_rowq": (_I, [_P, _P, _L, _P, _L, _P, _L, _P, _P, _P, _I, _I, _I, _F, _I, _P, _L, _P, _P, _P]),
    "mla_absorb_q": (_I, [_P, _P, _P, _I, _I, _P, _P]),
    "mla_v_up_proj": (_I, [_P, _P, _I, _I, _P, _P, _P, _P, _L, _P]),
    "mla_selftest": (_I, [_I, _P, _P, _P]),
    "mla_decode_fwd_noalloc": (_I, [_P, _P, _L, _P, _L, _P, _L, _P, _P, _P, _I, _I, _I, _F, _I, _P, _P, _P]),
    "mla_noalloc_scratch_bytes": (_L, []),
    "mla_probe_gather": (_I, [_I, _I, _I, _I, _I, _P, _L, _P, _L, _P, _L, _P, _L, _P, _P]),
    "mla_probe_lds": (_I, [_I, _I, _I, _P, _P, _P]),
}


class MlaLibraryError(RuntimeError):
    """The HIP library is missing, failed to load, or an entry point returned an error."""


_lock = threading.Lock()
_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and return the library with all signatures bound."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise MlaLibraryError(
                f"{path} is not built; run `python -m amd_optimization_challenge_amd.build`"
            )
        try:
            lib = ctypes.CDLL(path)
        except OSError as e:  # pragma: no cover - depends on the ROCm runtime
            raise MlaLibraryError(f"failed to load {path}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != MLA_OK:
        msg = load().mla_last_error().decode(errors="replace")
        raise MlaLibraryError(f"{what} failed (status {rc}): {msg}")

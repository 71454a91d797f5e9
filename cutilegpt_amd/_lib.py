"""ctypes binding of libcgpt.so (the gfx950 HIP kernels, C ABI in include/cgpt.h).

torch is imported before the library is opened so that libcgpt.so binds to the
HIP runtime torch already loaded (both name ``libamdhip64.so.7``): one runtime per
process, so torch's device pointers and streams are valid in the kernels.

There is no fallback: if the library is missing or cannot be loaded every
kernel entry point raises ``KernelLibraryError``.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be loaded first, see module docstring)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libcgpt.so")

CGPT_F32 = 0
CGPT_BF16 = 1
CGPT_F16 = 2
EPI_NONE = 0
EPI_BIAS = 1
EPI_BIAS_GELU = 2
EPI_BIAS_RESID = 3
TILE_AUTO = -1
TILE_SKINNY = -2

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# name -> (restype, argtypes); mirrors include/cgpt.h.
SIGNATURES = {
    "cgpt_version": (_I, []),
    "cgpt_status_string": (ctypes.c_char_p, [_I]),
    "cgpt_gelu": (_I, [_P, _P, _I64, _I, _P]),
    "cgpt_add_layernorm": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _F, _I, _I, _I, _I, _P]),
    "cgpt_gemm": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _I, _I, _I, _P]),
    "cgpt_gemm_num_tiles": (_I, []),
    "cgpt_gemm_skinny": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _I, _I,
                              _P, _I64, _P, _I64, _P]),
    "cgpt_gemm_skinny_workspace": (_I, [_I64, _I64, _I64, _I, _P, _P]),
    "cgpt_gemm_skinny_noalloc": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I,
                                      _I, _I, _P]),
    "cgpt_gemm_partials": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P]),
    "cgpt_gemm_partials_plan": (_I, [_I64, _I64, _I64, _I, _P]),
    "cgpt_attention_fwd": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                _I64, _I64, _I64, _F, _I, _I, _P]),
    "cgpt_embedding": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _I, _P, _P]),
    "cgpt_embedding_at": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _I, _I, _P, _P]),
    "cgpt_embedding_layernorm": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                      _I64, _I64, _F, _I, _I, _P, _P]),
    "cgpt_attention_decode": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P,
                                   _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                                   _I64, _I64, _F, _I, _P, _P]),
    "cgpt_attention_decode_partials": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _P,
                                            _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64,
                                            _I64, _I64, _I64, _F, _I, _P, _P]),
    "cgpt_add_layernorm_partials": (_I, [_P, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _I64,
                                         _I64, _F, _I, _I, _I, _I, _P]),
    "cgpt_kv_store": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                           _I64, _I64, _I64, _I64, _I64, _I64, _I, _P]),
    "cgpt_argmax": (_I, [_P, _I64, _I64, _I64, _I, _P, _P, _I64, _P, _P]),
    "cgpt_partials_bias_act": (_I, [_P, _I64, _I64, _I64, _P, _I, _P, _I64, _I64, _I64, _I, _I,
                                    _P]),
}

ABI_VERSION = 1


class KernelLibraryError(RuntimeError):
    """libcgpt.so is missing, stale or failed to load."""


_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Open libcgpt.so once and bind every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise KernelLibraryError(
                f"{LIB_PATH} not found: build the HIP kernels first "
                "(python -m cutilegpt_amd.build, or __graft_entry__.build())")
        try:
            lib = ctypes.CDLL(LIB_PATH)
        except OSError as e:
            raise KernelLibraryError(f"cannot load {LIB_PATH}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as e:
                raise KernelLibraryError(f"{LIB_PATH} does not export {name}") from e
            fn.restype = res
            fn.argtypes = args
        if lib.cgpt_version() != ABI_VERSION:
            raise KernelLibraryError(
                f"{LIB_PATH} has ABI {lib.cgpt_version()}, expected {ABI_VERSION}: rebuild it")
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    """Raise for a non-zero status returned by a cgpt_* entry point."""
    if status == 0:
        return
    msg = load().cgpt_status_string(status).decode()
    if status < 0:
        raise ValueError(f"{what}: {msg} (status {status})")
    raise RuntimeError(f"{what}: HIP error {status}: {msg}")

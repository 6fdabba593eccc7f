"""ctypes binding of libanna_mi.so, the C-ABI HIP library declared in include/anna_mi.h.

The library is loaded after torch so that it shares torch's HIP runtime (both
resolve the soname libamdhip64.so.7).  There is no fallback: if the library is
missing or an entry point fails, a RuntimeError carrying the library's message
is raised.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime first)

LIB_PATH = Path(__file__).resolve().parent / "libanna_mi.so"

BF16, F16, F32 = 0, 1, 2
_DTYPE_CODES = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# name -> argtypes (every entry point returns int status)
PROTOTYPES: dict[str, list] = {
    "anna_mi_int4_linear": [_P, _I, _I64, _I64, _I64, _P, _I64, _I64, _P, _I, _P, _I64, _I64, _P, _P],
    "anna_mi_int4_dequant": [_P, _I64, _I64, _P, _I, _P, _I64, _I64, _I64, _P, _I, _P],
    "anna_mi_int4_quantize": [_P, _I, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _P],
    "anna_mi_autoround_to_int4": [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P],
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"anna_mi HIP library not built ({LIB_PATH} missing); run `python -m anna_amd.build`"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.anna_mi_last_error.restype = ctypes.c_char_p
        lib.anna_mi_last_error.argtypes = []
        lib.anna_mi_abi_version.restype = ctypes.c_int
        for name, argtypes in PROTOTYPES.items():
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = argtypes
        _lib = lib
        return lib


def call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.anna_mi_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {dtype}; expected bfloat16, float16 or float32") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def require_device(*tensors: torch.Tensor) -> None:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"anna_mi ops need ROCm device tensors, got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")

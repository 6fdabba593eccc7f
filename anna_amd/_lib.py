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


class View(ctypes.Structure):
    """anna_mi_view: pointer + 4 element strides."""

    _fields_ = [("ptr", ctypes.c_void_p), ("s0", _I64), ("s1", _I64), ("s2", _I64), ("s3", _I64)]


class DecodeArgs(ctypes.Structure):
    """anna_mi_decode_args (field order and types as in include/anna_mi.h)."""

    _fields_ = [
        ("dtype", _I), ("batch", _I64), ("q_heads", _I64), ("kv_heads", _I64), ("head_dim", _I64),
        ("query", View), ("len1", _I64), ("key_format", _I), ("key", View), ("key_norms", View), ("key_bits", _I),
        ("value_format", _I), ("value", View), ("value_scales", View), ("value_zeros", View), ("value_bits", _I),
        ("value_group_size", _I64), ("rotation", _P), ("rotation_t", _P), ("key_centroids", _P),
        ("value_centroids", _P), ("query_rot", _P), ("len2", _I64), ("residual_key", View), ("residual_value", View),
        ("scaling", _F), ("block_size", _I64), ("gate_layout", _I), ("gate", View), ("out", View),
        ("partial_stats", View), ("partial_values", View), ("partial_capacity", _I64), ("seq_lengths", _P),
        ("rotation_signs", _P),
    ]


class TQDecodeArgs(ctypes.Structure):
    """anna_mi_tq_decode_args."""

    _fields_ = [
        ("batch", _I64), ("q_heads", _I64), ("kv_heads", _I64), ("head_dim", _I64), ("key_bits", _I),
        ("value_bits", _I), ("query", _P), ("gate", _P), ("key_codes", _P), ("key_norms", _P), ("value_codes", _P),
        ("value_norms", _P), ("pool_tokens", _I64), ("residual_key", _P), ("residual_value_t", _P),
        ("residual_capacity", _I64), ("seq_offsets", _P), ("seq_lengths", _P), ("signs", _P), ("key_scale", _F),
        ("value_scale", _F), ("scaling", _F), ("blocks_per_item", _I64), ("num_workgroups", _I64),
        ("partial_stats", _P), ("partial_values", _P), ("item_table", _P), ("out", _P),
    ]


class TQAppendArgs(ctypes.Structure):
    """anna_mi_tq_append_args."""

    _fields_ = [
        ("batch", _I64), ("kv_heads", _I64), ("head_dim", _I64), ("new_key", _P), ("new_value", _P),
        ("key_codes", _P), ("key_norms", _P), ("value_codes", _P), ("value_norms", _P), ("pool_tokens", _I64),
        ("residual_key", _P), ("residual_value_t", _P), ("residual_capacity", _I64), ("seq_offsets", _P),
        ("seq_capacity", _P), ("seq_lengths", _P), ("overflow", _P), ("signs", _P), ("thresholds", _P),
    ]


class TQPackArgs(ctypes.Structure):
    """anna_mi_tq_pack_args."""

    _fields_ = [
        ("kv_heads", _I64), ("head_dim", _I64), ("tokens", _I64), ("keys", _P), ("values", _P),
        ("stride_head", _I64), ("stride_token", _I64), ("key_codes", _P), ("key_norms", _P), ("value_codes", _P),
        ("value_norms", _P), ("pool_tokens", _I64), ("slot_offset", _I64), ("signs", _P), ("thresholds", _P),
    ]


class TQRowsAppendArgs(ctypes.Structure):
    """anna_mi_tq_rows_append_args."""

    _fields_ = [
        ("dtype", _I), ("batch", _I64), ("kv_heads", _I64), ("head_dim", _I64), ("capacity", _I64),
        ("residual_capacity", _I64), ("key_bits", _I), ("value_bits", _I), ("value_group_size", _I64),
        ("new_key", _P), ("new_value", _P), ("key_codes", _P), ("key_norms", _P), ("value_data", _P),
        ("value_scales", _P), ("value_zeros", _P), ("residual_key", _P), ("residual_value", _P),
        ("seq_lengths", _P), ("overflow", _P), ("signs", _P), ("thresholds", _P),
    ]


PROTOTYPES.update({
    "anna_mi_tq_rows_append": [ctypes.POINTER(TQRowsAppendArgs), _P],
    "anna_mi_tq_pack_kv": [ctypes.POINTER(TQPackArgs), _P],
    "anna_mi_tq_decode": [ctypes.POINTER(TQDecodeArgs), _P],
    "anna_mi_tq_append": [ctypes.POINTER(TQAppendArgs), _P],
    "anna_mi_tq_append_decode": [ctypes.POINTER(TQDecodeArgs), ctypes.POINTER(TQAppendArgs), _P],
    "anna_mi_tq_block_values": [_P, _I64, _P, _P],
    "anna_mi_tq_rotation": [_I64, ctypes.c_uint64, _P],
    "anna_mi_tq_codebook": [_I, _I64, _P, _P],
    "anna_mi_tq_hadamard_signs": [_I64, ctypes.c_uint64, _P],
    "anna_mi_tq_hadamard_quantize": [_P, _I, _I64, _I64, _I64, _P, _P, _I, _P, _P, _P],
    "anna_mi_tq_mse_quantize": [_P, _I, _I64, _I64, _I64, _P, _P, _I, _P, _P, _P],
    "anna_mi_tq_mse_dequant": [_P, _P, _I64, _I64, _P, _P, _I, _P, _I, _I64, _P],
    "anna_mi_tq_values_quantize": [_P, _I, _I64, _I64, _I64, _I64, _I64, _I, _I64, _P, _P, _P, _P],
    "anna_mi_tq_values_dequant": [_P, _P, _P, _I, _I64, _I64, _I, _I64, _P, _I, _P],
    "anna_mi_tq_ip_gaussian": [_I64, ctypes.c_uint64, _P],
    "anna_mi_tq_ip_quantize": [_P, _I, _I64, _I64, _I64, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P],
    "anna_mi_tq_ip_dequant": [_P, _P, _P, _P, _I64, _I64, _P, _P, _P, _I, _P, _I, _I64, _P],
    "anna_mi_tq_ip_scores": [_P, _I, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _I64, _P, _P, _P, _I,
                             _F, _P, _P, _P],
    "anna_mi_gqa_decode_splitkv": [ctypes.POINTER(DecodeArgs), _P],
    "anna_mi_gqa_decode_splitkv_noalloc": [ctypes.POINTER(DecodeArgs), _P],
})


class MoeMlpArgs(ctypes.Structure):
    """anna_mi_moe_mlp_args."""

    _fields_ = [
        ("dtype", _I), ("scale_dtype", _I), ("routes", _I64), ("hidden_dim", _I64), ("intermediate_dim", _I64),
        ("compact_hidden", _P), ("compact_weights", _P), ("compact_outputs", _P), ("expert_offsets", _P),
        ("active_experts", _P), ("active_slots", _P), ("active_count", _I64),
        ("gate_qweight", _P), ("gate_qscale", _P), ("gate_qzeros", _P),
        ("up_qweight", _P), ("up_qscale", _P), ("up_qzeros", _P),
        ("down_qweight", _P), ("down_qscale", _P), ("down_qzeros", _P),
        ("hidden_packed_cols", _I64), ("hidden_groups", _I64), ("intermediate_packed_cols", _I64),
        ("intermediate_groups", _I64), ("group_size", _I64), ("activation", _P), ("sweep_chunks", _I),
        ("items", _P), ("items_prefilled", _I),
    ]


PROTOTYPES.update({
    "anna_mi_moe_router": [_P, _I, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _P],
    "anna_mi_moe_dispatch": [_P, _I, _I64, _I64, _I64, _P, _I, _P, _P, _I, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P,
                             _P],
    "anna_mi_moe_route_small": [_P, _I, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "anna_mi_moe_gather": [_P, _I, _I64, _I64, _P, _I, _P, _I64, _I64, _P, _P, _P],
    "anna_mi_moe_scatter": [_P, _I, _I64, _I64, _P, _I64, _P, _P, _P],
    "anna_mi_moe_combine": [_P, _I, _I64, _P, _I64, _I64, _P, _P],
    "anna_mi_moe_grouped_int4_mlp": [ctypes.POINTER(MoeMlpArgs), _P],
    "anna_mi_int4_gemv_tiled": [_P, _I, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I, _P, _I64, _I64, _I64, _I64,
                                _I64, _P, _I, _I64, _P],
    "anna_mi_topk_rows": [_P, _I64, _I64, _I64, _I64, _P, _I, _P, _P],
    "anna_mi_lm_head_int4_topk": [_P, _I, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I, _P, _I64, _I64, _I64, _I64,
                                  _I64, _I64, _P, _P, _P, _P],
})
# entry points that do not return a status code
RAW_PROTOTYPES: dict[str, tuple] = {
    "anna_mi_sizeof_moe_mlp_args": (_I64, []),
    "anna_mi_decode_num_blocks": (_I64, [ctypes.POINTER(DecodeArgs)]),
    "anna_mi_sizeof_decode_args": (_I64, []),
    "anna_mi_gqa_decode_splitkv_noalloc_capacity": (_I64, []),
    "anna_mi_sizeof_tq_decode_args": (_I64, []),
    "anna_mi_sizeof_tq_append_args": (_I64, []),
    "anna_mi_sizeof_tq_pack_args": (_I64, []),
    "anna_mi_sizeof_tq_rows_append_args": (_I64, []),
    "anna_mi_tq_decode_workgroups": (_I64, [_I64, _I64, _P, _I64]),
}

_lock = threading.Lock()


def _check_stamp(lib: ctypes.CDLL) -> None:
    """Refuses a library built from other sources than the csrc/ next to it."""
    from . import build

    if not build.CSRC.is_dir():
        return  # installed without sources: nothing to compare against
    built = lib.anna_mi_source_hash().decode()
    want = build.source_hash()
    if built != want:
        raise RuntimeError(
            f"{LIB_PATH.name} is stale: built from sources {built[:12]}, the tree holds {want[:12]}; "
            "run `python -m anna_amd.build`")
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
        lib.anna_mi_source_hash.restype = ctypes.c_char_p
        lib.anna_mi_source_hash.argtypes = []
        _check_stamp(lib)
        lib.anna_mi_abi_version.restype = ctypes.c_int
        for name, argtypes in PROTOTYPES.items():
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = argtypes
        for name, (restype, argtypes) in RAW_PROTOTYPES.items():
            fn = getattr(lib, name)
            fn.restype = restype
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


def view(t: torch.Tensor | None, dims: tuple[int, ...] = (0, 1, 2, 3)) -> View:
    """View over tensor dims `dims` (index -1 = absent, stride 0)."""
    if t is None:
        return View(None, 0, 0, 0, 0)
    st = [t.stride(d) if d >= 0 else 0 for d in dims] + [0] * (4 - len(dims))
    return View(t.data_ptr(), *st[:4])


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

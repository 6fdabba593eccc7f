"""Op boundary: the reference's ``torch.ops.anna.*`` schemas, backed by libanna_mi.so.

Mirrors src/anna/model/fused_ops.py of the reference (load-once under a lock,
``run_*`` wrappers that raise instead of falling back) and the op schemas of
``TORCH_LIBRARY(anna, m)`` (gated_delta_fused_op.sycl:7621-7914).  The ops are
registered for the ROCm device key (``CUDA`` in PyTorch-ROCm) with Meta kernels
for shape inference; autograd is not supported (inference only, as in the
reference).
"""

from __future__ import annotations

import threading

import torch

from . import _lib

_REG_LOCK = threading.Lock()
_REGISTERED = False
_LIBS: list[torch.library.Library] = []

SCHEMAS = {
    "xpu_int4_gemv": (
        "xpu_int4_gemv(Tensor hidden_states, Tensor qweight, Tensor qscale, Tensor qzeros, "
        "int group_size, int in_features) -> Tensor"
    ),
}


# ---------------------------------------------------------------- int4 linear


def _check_int4_inputs(hidden_states, qweight, qscale, qzeros, group_size, in_features):
    # Same checks, same order of meaning, as validate_xpu_int4_gemv_inputs (sycl:1100-1130),
    # except that bf16/fp16 qscale is accepted besides fp32.
    if hidden_states.dim() != 2:
        raise RuntimeError("xpu_int4_gemv expects hidden_states shaped [rows, in_features]")
    if qweight.dim() != 2:
        raise RuntimeError("qweight must be [out_features, packed_cols]")
    if qscale.dim() != 2:
        raise RuntimeError("qscale must be [group_count, out_features]")
    if qzeros.dim() != 2:
        raise RuntimeError("qzeros must be [group_count, out_features]")
    if group_size <= 0:
        raise RuntimeError("group_size must be positive")
    if in_features <= 0:
        raise RuntimeError("in_features must be positive")
    if hidden_states.size(0) <= 0:
        raise RuntimeError("hidden_states rows must be positive")
    if hidden_states.size(1) != in_features:
        raise RuntimeError("hidden_states last dimension must match in_features")
    if qweight.dtype != torch.int32:
        raise RuntimeError("qweight must be int32")
    if qscale.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        raise RuntimeError("qscale must be float32, bfloat16 or float16")
    if qzeros.dtype != torch.int8:
        raise RuntimeError("qzeros must be int8")
    if not (qweight.is_contiguous() and qscale.is_contiguous() and qzeros.is_contiguous()):
        raise RuntimeError("qweight, qscale and qzeros must be contiguous")
    if qweight.size(1) * 8 < in_features:
        raise RuntimeError("qweight packed columns are smaller than in_features")
    if qscale.size(1) != qweight.size(0):
        raise RuntimeError("qscale output dimension must match qweight")
    if qzeros.shape != qscale.shape:
        raise RuntimeError("qzeros shape must match qscale")
    if qscale.size(0) * group_size < in_features:
        raise RuntimeError("qscale group count is smaller than in_features")
    if hidden_states.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise RuntimeError("xpu_int4_gemv supports float16, bfloat16, and float32 hidden states")


def int4_linear_out(hidden_states, qweight, qscale, qzeros, group_size, in_features, out):
    """y = hidden_states @ dequant(W)^T into ``out`` [rows, N] (hidden_states dtype)."""
    _check_int4_inputs(hidden_states, qweight, qscale, qzeros, group_size, in_features)
    _lib.require_device(hidden_states, qweight, qscale, qzeros, out)
    if hidden_states.stride(1) != 1:
        hidden_states = hidden_states.contiguous()
    rows = hidden_states.size(0)
    n = qweight.size(0)
    if out.shape != (rows, n) or out.dtype != hidden_states.dtype or not out.is_contiguous():
        raise RuntimeError("int4 linear output must be a contiguous [rows, out_features] tensor of the input dtype")
    _lib.call(
        "anna_mi_int4_linear",
        hidden_states.data_ptr(), _lib.dtype_code(hidden_states.dtype), rows, in_features, hidden_states.stride(0),
        qweight.data_ptr(), n, qweight.size(1),
        qscale.data_ptr(), _lib.dtype_code(qscale.dtype), qzeros.data_ptr(), qscale.size(0), group_size,
        out.data_ptr(), _lib.stream_of(hidden_states),
    )
    return out


def _xpu_int4_gemv_impl(hidden_states, qweight, qscale, qzeros, group_size, in_features):
    out = torch.empty((hidden_states.size(0), qweight.size(0)), dtype=hidden_states.dtype, device=hidden_states.device)
    return int4_linear_out(hidden_states, qweight, qscale, qzeros, group_size, in_features, out)


def _xpu_int4_gemv_meta(hidden_states, qweight, qscale, qzeros, group_size, in_features):
    return hidden_states.new_empty((hidden_states.size(0), qweight.size(0)))


def int4_dequant(qweight, qscale, qzeros, group_size, in_features, out_dtype=torch.bfloat16):
    _lib.require_device(qweight, qscale, qzeros)
    n = qweight.size(0)
    out = torch.empty((n, in_features), dtype=out_dtype, device=qweight.device)
    _lib.call(
        "anna_mi_int4_dequant",
        qweight.data_ptr(), n, qweight.size(1), qscale.data_ptr(), _lib.dtype_code(qscale.dtype),
        qzeros.data_ptr(), qscale.size(0), group_size, in_features, out.data_ptr(),
        _lib.dtype_code(out_dtype), _lib.stream_of(qweight),
    )
    return out


def int4_quantize(weight, *, group_size, padded_in_features, rounding="half_even"):
    """Device int4 packer; returns (qweight int32 [N, Kp/8], qscale fp32 [G, N], qzeros int8 [G, N])."""
    _lib.require_device(weight)
    if weight.dim() != 2:
        raise RuntimeError("weight must be [out_features, in_features]")
    weight = weight.contiguous()
    if weight.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        weight = weight.float()
    n, k = weight.shape
    kp = int(padded_in_features)
    g = kp // group_size
    qweight = torch.empty((n, kp // 8), dtype=torch.int32, device=weight.device)
    qscale = torch.empty((g, n), dtype=torch.float32, device=weight.device)
    qzeros = torch.empty((g, n), dtype=torch.int8, device=weight.device)
    mode = {"half_even": 0, "half_away": 1}[rounding]
    _lib.call(
        "anna_mi_int4_quantize",
        weight.data_ptr(), _lib.dtype_code(weight.dtype), n, k, kp, group_size, mode,
        qweight.data_ptr(), qscale.data_ptr(), qzeros.data_ptr(), _lib.stream_of(weight),
    )
    return qweight, qscale, qzeros


def autoround_to_int4(gptq_qweight, gptq_qzeros, scales, *, in_features, out_features, group_size, padded_in_features):
    _lib.require_device(gptq_qweight, gptq_qzeros, scales)
    gptq_qweight = gptq_qweight.contiguous().to(torch.int32)
    gptq_qzeros = gptq_qzeros.contiguous().to(torch.int32)
    scales = scales.contiguous().to(torch.float16)
    g = scales.size(0)
    kp = int(padded_in_features)
    dev = gptq_qweight.device
    qweight = torch.empty((out_features, kp // 8), dtype=torch.int32, device=dev)
    qscale = torch.empty((g, out_features), dtype=torch.float32, device=dev)
    qzeros = torch.empty((g, out_features), dtype=torch.int8, device=dev)
    _lib.call(
        "anna_mi_autoround_to_int4",
        gptq_qweight.data_ptr(), gptq_qzeros.data_ptr(), scales.data_ptr(), in_features, out_features,
        group_size, g, kp, qweight.data_ptr(), qscale.data_ptr(), qzeros.data_ptr(), _lib.stream_of(scales),
    )
    return qweight, qscale, qzeros


# ---------------------------------------------------------------- registration

_IMPLS = {
    "xpu_int4_gemv": (_xpu_int4_gemv_impl, _xpu_int4_gemv_meta),
}


def register_ops() -> None:
    """Define the ``anna::`` schemas and bind them to the HIP library (idempotent)."""
    global _REGISTERED
    if _REGISTERED:
        return
    with _REG_LOCK:
        if _REGISTERED:
            return
        _lib.load()
        lib_def = torch.library.Library("anna", "FRAGMENT")
        for name, schema in SCHEMAS.items():
            lib_def.define(schema)
            impl, meta = _IMPLS[name]
            lib_def.impl(name, impl, "CUDA")
            lib_def.impl(name, meta, "Meta")
        _LIBS.append(lib_def)
        _REGISTERED = True


def maybe_load_gated_delta_library(path=None) -> bool:
    """Reference-compatible loader name (fused_ops.py:414-448): registers the ops."""
    register_ops()
    return True


def _op(name: str):
    register_ops()
    return getattr(torch.ops.anna, name)


def run_xpu_int4_gemv(*, hidden_states, qweight, qscale, qzeros, group_size, in_features):
    return _op("xpu_int4_gemv")(hidden_states, qweight, qscale, qzeros, int(group_size), int(in_features))

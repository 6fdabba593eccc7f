"""Op boundary: the reference's ``torch.ops.anna.*`` schemas, backed by libanna_mi.so.

Mirrors src/anna/model/fused_ops.py of the reference (load-once under a lock,
``run_*`` wrappers that raise instead of falling back) and the op schemas of
``TORCH_LIBRARY(anna, m)`` (gated_delta_fused_op.sycl:7621-7914).  The ops are
registered for the ROCm device key (``CUDA`` in PyTorch-ROCm) with Meta kernels
for shape inference; autograd is not supported (inference only, as in the
reference).
"""

from __future__ import annotations

import ctypes
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
    "gqa_decode_splitkv_fused": (
        "gqa_decode_splitkv_fused(Tensor query, Tensor key, Tensor value, float scaling, int block_size, "
        "Tensor? gate=None) -> Tensor"
    ),
    "gqa_decode_splitkv_fused_out": (
        "gqa_decode_splitkv_fused_out(Tensor query, Tensor key, Tensor value, Tensor(a!) output, "
        "Tensor(b!) partial_stats, Tensor(c!) partial_values, float scaling, int block_size, "
        "Tensor? gate=None) -> Tensor(a!)"
    ),
    "gqa_decode_splitkv_turboquant_fused_out": (
        "gqa_decode_splitkv_turboquant_fused_out(Tensor query, Tensor quantized_key, Tensor value_data, "
        "Tensor value_scales, Tensor value_zeros, Tensor residual_key, Tensor residual_value, Tensor(a!) output, "
        "Tensor(b!) partial_stats, Tensor(c!) partial_values, float scaling, int value_bits, int value_group_size, "
        "int block_size, Tensor? gate=None) -> Tensor(a!)"
    ),
    "xpu_int4_gemv_tiled": (
        "xpu_int4_gemv_tiled(Tensor hidden_states, Tensor qweight, Tensor qscale, Tensor qzeros, int group_size, "
        "int in_features, int out_features) -> Tensor"
    ),
    "lm_head_int4_topk_fused": (
        "lm_head_int4_topk_fused(Tensor hidden_states, Tensor qweight, Tensor qscale, Tensor qzeros, int group_size, "
        "int in_features, int top_k) -> (Tensor, Tensor)"
    ),
    "moe_router_fused": "moe_router_fused(Tensor router_logits, int top_k, bool normalize_topk_prob=True) -> (Tensor, Tensor, Tensor)",
    "moe_dispatch_fused": (
        "moe_dispatch_fused(Tensor hidden_states, Tensor routing_weights, Tensor selected_experts, "
        "Tensor expert_usage) -> (Tensor, Tensor, Tensor, Tensor)"
    ),
    "moe_scatter_fused": "moe_scatter_fused(Tensor compact_outputs, Tensor sorted_token_idx, int num_tokens) -> Tensor",
    "moe_grouped_int4_mlp_fused": (
        "moe_grouped_int4_mlp_fused(Tensor compact_hidden_states, Tensor compact_routing_weights, "
        "Tensor(a!) compact_outputs, Tensor expert_offsets, Tensor active_experts, Tensor active_slots, "
        "Tensor gate_qweight, Tensor gate_qscale, Tensor gate_qzeros, Tensor up_qweight, Tensor up_qscale, "
        "Tensor up_qzeros, Tensor down_qweight, Tensor down_qscale, Tensor down_qzeros, int group_size, "
        "int max_routes_per_expert) -> Tensor(a!)"
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


# ---------------------------------------------------------------- split-KV decode

KEYS_DENSE, KEYS_TQ_MSE = 0, 1
VALUES_DENSE, VALUES_MINMAX, VALUES_TQ_MSE = 0, 1, 2
GATE_NONE, GATE_FLAT, GATE_HEADS = 0, 1, 2


def _check_gate(gate, query):
    """validate_gqa_decode_optional_gate (sycl:1605-1629): dtype, batch and the two layouts."""
    if gate is None:
        return GATE_NONE
    if gate.dtype != query.dtype:
        raise RuntimeError("gate must match query dtype")
    if gate.size(0) != query.size(0):
        raise RuntimeError("gate batch size mismatch")
    num_heads, head_dim = query.size(1), query.size(3)
    if gate.dim() == 3 and gate.size(1) == 1 and gate.size(2) == num_heads * head_dim:
        return GATE_FLAT
    if gate.dim() == 4 and gate.size(1) == num_heads and gate.size(2) == 1 and gate.size(3) == head_dim:
        return GATE_HEADS
    raise RuntimeError("gate must be [batch, 1, heads * head_dim] or [batch, heads, 1, head_dim]")


def _gate_view(gate, query):
    """Accepts the reference's two gate layouts (prepare_gqa_decode_gate, sycl:1631-1669):
    flat [B, 1, Hq*D] or query-aligned [B, Hq, 1, D]."""
    layout = _check_gate(gate, query)
    if layout == GATE_NONE:
        return GATE_NONE, _lib.view(None)
    if layout == GATE_FLAT:
        return GATE_FLAT, _lib.view(gate, (0, 1, 2, -1))
    return GATE_HEADS, _lib.view(gate)


def _splitkv_num_blocks(key_len: int, block_size: int) -> int:
    eb = min(max(int(block_size), 16), int(key_len))
    return (int(key_len) + eb - 1) // eb


def decode_args(*, query, len1, key=None, key_format=KEYS_DENSE, key_norms=None, key_bits=0,
                value=None, value_format=VALUES_DENSE, value_scales=None, value_zeros=None, value_bits=0,
                value_group_size=1, rotation=None, rotation_t=None, key_centroids=None, value_centroids=None,
                query_rot=None, residual_key=None, residual_value=None, scaling, block_size, gate=None, output,
                partial_stats, partial_values, seq_lengths=None, rotation_signs=None):
    """Fills anna_mi_decode_args from tensors (query/out [B, Hq, 1, D], K/V [B, Hkv, L, ...]).
    seq_lengths (optional, device int32 [B]): per-row token counts; len1 and the residual's
    length are then capacities (see include/anna_mi.h).  rotation_signs (optional, device fp32
    [D]): the sign vector of a randomized Hadamard key rotation, so that the query is rotated by
    the fast transform."""
    b, hq, _, d = query.shape
    hkv = (key if key is not None else residual_key).size(1)
    len2 = 0 if residual_key is None else residual_key.size(2)
    gl, gv = _gate_view(gate, query)
    a = _lib.DecodeArgs()
    a.dtype = _lib.dtype_code(query.dtype)
    a.batch, a.q_heads, a.kv_heads, a.head_dim = b, hq, hkv, d
    a.query = _lib.view(query)
    a.len1 = int(len1)
    a.key_format = key_format
    a.key = _lib.view(key)
    a.key_norms = _lib.view(key_norms, (0, 1, 2)) if key_norms is not None else _lib.view(None)
    a.key_bits = key_bits
    a.value_format = value_format
    a.value = _lib.view(value)
    if value_format == VALUES_TQ_MSE:
        a.value_scales = _lib.view(value_scales, (0, 1, 2))
    else:
        a.value_scales = _lib.view(value_scales)
    a.value_zeros = _lib.view(value_zeros)
    a.value_bits = value_bits
    a.value_group_size = int(value_group_size)
    a.rotation = _lib.ptr(rotation)
    a.rotation_t = _lib.ptr(rotation_t)
    a.key_centroids = _lib.ptr(key_centroids)
    a.value_centroids = _lib.ptr(value_centroids)
    a.query_rot = _lib.ptr(query_rot)
    a.len2 = len2
    a.residual_key = _lib.view(residual_key)
    a.residual_value = _lib.view(residual_value)
    a.scaling = float(scaling)
    a.block_size = int(block_size)
    a.gate_layout = gl
    a.gate = gv
    a.out = _lib.view(output)
    a.partial_stats = _lib.view(partial_stats)
    a.partial_values = _lib.view(partial_values)
    a.partial_capacity = min(partial_stats.size(2), partial_values.size(2))
    if seq_lengths is not None:
        if seq_lengths.dtype != torch.int32 or seq_lengths.numel() != b or not seq_lengths.is_contiguous():
            raise RuntimeError("seq_lengths must be a contiguous int32 tensor with one entry per batch row")
        _lib.require_device(seq_lengths)
    a.seq_lengths = _lib.ptr(seq_lengths)
    if rotation_signs is not None:
        _lib.require_device(rotation_signs)
        if rotation_signs.dtype != torch.float32 or rotation_signs.numel() != d:
            raise RuntimeError("rotation_signs must be fp32 [head_dim]")
    a.rotation_signs = _lib.ptr(rotation_signs)
    return a


def decode_num_blocks(args) -> int:
    return int(_lib.load().anna_mi_decode_num_blocks(args))


def run_decode(args, stream_tensor) -> None:
    import ctypes

    _lib.call("anna_mi_gqa_decode_splitkv", ctypes.byref(args), _lib.stream_of(stream_tensor))


def _check_decode_common(query, key, value, block_size, name):
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise RuntimeError("query must be [batch, heads, 1, head_dim]; key/value must be [batch, kv_heads, key_len, head_dim]")
    if query.size(2) != 1:
        raise RuntimeError(f"{name} only supports single-token query")
    if query.size(0) != key.size(0):
        raise RuntimeError("query/key batch size mismatch")
    if key.shape != value.shape:
        raise RuntimeError("key and value must share the same shape")
    if query.size(3) != key.size(3):
        raise RuntimeError("query/key head_dim mismatch")
    if query.size(1) % key.size(1) != 0:
        raise RuntimeError("query heads must be divisible by kv_heads")
    if key.size(2) < 1:
        raise RuntimeError("key_len must be positive")
    if block_size < 16:
        raise RuntimeError(f"{name} block_size must be at least 16")
    if not (query.dtype == key.dtype == value.dtype):
        raise RuntimeError("query, key, and value must share the same dtype")


def _check_workspace(query, key_len, block_size, output, partial_stats, partial_values, name):
    nblk = _splitkv_num_blocks(key_len, block_size)
    b, h, _, d = query.shape
    if output.shape != query.shape or output.dtype != query.dtype:
        raise RuntimeError(f"{name} output must match query shape and dtype")
    if partial_stats.dtype != torch.float32 or partial_values.dtype != torch.float32:
        raise RuntimeError(f"{name} partial_stats/partial_values must be float32")
    if (partial_stats.dim() != 4 or partial_stats.size(0) != b or partial_stats.size(1) != h
            or partial_stats.size(2) < nblk or partial_stats.size(3) != 2):
        raise RuntimeError(f"{name} partial_stats shape/capacity mismatch")
    if (partial_values.dim() != 4 or partial_values.size(0) != b or partial_values.size(1) != h
            or partial_values.size(2) < nblk or partial_values.size(3) != d):
        raise RuntimeError(f"{name} partial_values shape/capacity mismatch")


def _gqa_decode_splitkv_fused_out_impl(query, key, value, output, partial_stats, partial_values, scaling,
                                       block_size, gate=None):
    name = "gqa_decode_splitkv_fused_out"
    _check_decode_common(query, key, value, block_size, name)
    _check_workspace(query, key.size(2), block_size, output, partial_stats, partial_values, name)
    _check_gate(gate, query)
    _lib.require_device(query, key, value, output, partial_stats, partial_values, gate)
    a = decode_args(query=query, len1=key.size(2), key=key, value=value, scaling=scaling, block_size=block_size,
                    gate=gate, output=output, partial_stats=partial_stats, partial_values=partial_values)
    run_decode(a, query)
    return output


def _gqa_decode_splitkv_fused_impl(query, key, value, scaling, block_size, gate=None):
    nblk = _splitkv_num_blocks(key.size(2), block_size)
    b, h, _, d = query.shape
    out = torch.empty_like(query)
    ps = torch.empty((b, h, nblk, 2), dtype=torch.float32, device=query.device)
    pv = torch.empty((b, h, nblk, d), dtype=torch.float32, device=query.device)
    return _gqa_decode_splitkv_fused_out_impl(query, key, value, out, ps, pv, scaling, block_size, gate)


def _check_turboquant_inputs(query, quantized_key, value_data, value_scales, value_zeros, residual_key,
                             residual_value, value_bits, value_group_size, block_size):
    """Shape/dtype checks of validate_gqa_decode_splitkv_turboquant_inputs (sycl:1447-1501).

    Runs before any pointer reaches the library: the C entry point sees only pointers and
    strides, so a short value tensor or a smaller-batch cache must be refused here."""
    def check(cond, msg):
        if not cond:
            raise RuntimeError(msg)

    check(query.dim() == 4, "query must be [batch, heads, 1, head_dim]")
    check(quantized_key.dim() == 4, "quantized_key must be [batch, kv_heads, quantized_len, head_dim]")
    check(value_data.dim() == 4, "value_data must be [batch, kv_heads, quantized_len, packed_dim]")
    check(value_scales.dim() == 4, "value_scales must be [batch, kv_heads, quantized_len, value_groups]")
    check(value_zeros.dim() == 4, "value_zeros must be [batch, kv_heads, quantized_len, value_groups]")
    check(residual_key.dim() == 4, "residual_key must be [batch, kv_heads, residual_len, head_dim]")
    check(residual_value.dim() == 4, "residual_value must be [batch, kv_heads, residual_len, head_dim]")
    check(query.size(2) == 1, "gqa_decode_splitkv_turboquant_fused only supports single-token query")
    check(query.size(0) == quantized_key.size(0), "query/quantized_key batch size mismatch")
    check(query.size(0) == residual_key.size(0), "query/residual_key batch size mismatch")
    check(residual_key.shape == residual_value.shape, "residual_key and residual_value must share the same shape")
    check(quantized_key.size(1) == residual_key.size(1), "quantized and residual KV head count mismatch")
    check(quantized_key.size(1) >= 1, "kv_heads must be positive")
    check(query.size(1) % quantized_key.size(1) == 0, "query heads must be divisible by kv_heads")
    check(query.size(3) == quantized_key.size(3), "query/quantized_key head_dim mismatch")
    check(query.size(3) == residual_key.size(3), "query/residual_key head_dim mismatch")
    check(quantized_key.size(2) >= 1,
          "gqa_decode_splitkv_turboquant_fused requires a non-empty quantized prefix")
    check(value_data.size(0) == quantized_key.size(0), "value_data batch size mismatch")
    check(value_data.size(1) == quantized_key.size(1), "value_data kv head count mismatch")
    check(value_data.size(2) == quantized_key.size(2), "value_data quantized_len mismatch")
    check(value_scales.size(0) == quantized_key.size(0), "value_scales batch size mismatch")
    check(value_scales.size(1) == quantized_key.size(1), "value_scales kv head count mismatch")
    check(value_scales.size(2) == quantized_key.size(2), "value_scales quantized_len mismatch")
    check(value_zeros.shape == value_scales.shape, "value_zeros shape must match value_scales")
    check(value_bits in (2, 3, 4), "TurboQuant value_bits must be 2, 3, or 4")
    check(value_group_size > 0, "TurboQuant value_group_size must be positive")
    d = query.size(3)
    check(d % value_group_size == 0, "TurboQuant value_group_size must evenly divide head_dim")
    check(value_scales.size(3) * value_group_size == d, "TurboQuant value group count/head_dim mismatch")
    per = 4 if value_bits == 2 else 2
    check(value_data.size(3) * per >= d, "TurboQuant packed value width is smaller than head_dim")
    check(block_size >= 16, "gqa_decode_splitkv_turboquant_fused block_size must be at least 16")
    check(value_data.dtype == torch.uint8, "TurboQuant value_data must be uint8")
    check(query.dtype == quantized_key.dtype == residual_key.dtype == residual_value.dtype
          == value_scales.dtype == value_zeros.dtype,
          "query, keys, residual values, value_scales, and value_zeros must share the same dtype")
    check(query.dtype in (torch.float16, torch.bfloat16, torch.float32),
          "gqa_decode_splitkv_turboquant_fused XPU kernel supports float16, bfloat16, and float32 inputs")


def _gqa_decode_splitkv_turboquant_fused_out_impl(query, quantized_key, value_data, value_scales, value_zeros,
                                                  residual_key, residual_value, output, partial_stats,
                                                  partial_values, scaling, value_bits, value_group_size,
                                                  block_size, gate=None):
    # checks of validate_gqa_decode_splitkv_turboquant_inputs (sycl:1447-1501), same order and messages
    name = "gqa_decode_splitkv_turboquant_fused_out"
    _check_turboquant_inputs(query, quantized_key, value_data, value_scales, value_zeros, residual_key,
                             residual_value, value_bits, value_group_size, block_size)
    key_len = quantized_key.size(2) + residual_key.size(2)
    _check_workspace(query, key_len, block_size, output, partial_stats, partial_values, name)
    _check_gate(gate, query)
    _lib.require_device(query, quantized_key, value_data, value_scales, value_zeros, residual_key, residual_value,
                        output, partial_stats, partial_values, gate)
    a = decode_args(query=query, len1=quantized_key.size(2), key=quantized_key, value=value_data,
                    value_format=VALUES_MINMAX, value_scales=value_scales, value_zeros=value_zeros,
                    value_bits=value_bits, value_group_size=value_group_size,
                    residual_key=residual_key if residual_key.size(2) > 0 else None,
                    residual_value=residual_value if residual_key.size(2) > 0 else None,
                    scaling=scaling, block_size=block_size, gate=gate, output=output,
                    partial_stats=partial_stats, partial_values=partial_values)
    run_decode(a, query)
    return output


def _meta_out(query, *args, **kwargs):
    return args[2] if len(args) > 2 else query.new_empty(query.shape)


# ---------------------------------------------------------------- TurboQuant packing


def tq_rotation(head_dim: int, seed: int = 42) -> torch.Tensor:
    """Seeded rotation R (fp32 [D, D], host), generated by the native library: the randomized
    Hadamard H diag(s) / sqrt(D) for power-of-two D, a Haar matrix otherwise."""
    out = torch.empty((head_dim, head_dim), dtype=torch.float32)
    _lib.call("anna_mi_tq_rotation", head_dim, seed, out.data_ptr())
    return out


def tq_codebook(bits: int, head_dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    c = torch.empty(1 << bits, dtype=torch.float32)
    t = torch.empty((1 << bits) - 1, dtype=torch.float32)
    _lib.call("anna_mi_tq_codebook", bits, head_dim, c.data_ptr(), t.data_ptr())
    return c, t


def tq_hadamard_signs(head_dim: int, seed: int = 42) -> torch.Tensor:
    """Sign vector s (fp32 +-1 [D], host) of the randomized Hadamard rotation."""
    out = torch.empty((head_dim,), dtype=torch.float32)
    _lib.call("anna_mi_tq_hadamard_signs", head_dim, seed, out.data_ptr())
    return out


def tq_hadamard_quantize(x2d, signs, thresholds, bits):
    """x [nvec, D] (D a power of two in [64, 1024]) -> (codes uint8 [nvec, D*sb/8], norms fp16 [nvec])."""
    _lib.require_device(x2d, signs, thresholds)
    nvec, d = x2d.shape
    if x2d.stride(1) != 1:
        x2d = x2d.contiguous()
    sb = 2 if bits == 2 else 4
    codes = torch.empty((nvec, d * sb // 8), dtype=torch.uint8, device=x2d.device)
    norms = torch.empty((nvec,), dtype=torch.float16, device=x2d.device)
    _lib.call("anna_mi_tq_hadamard_quantize", x2d.data_ptr(), _lib.dtype_code(x2d.dtype), nvec, d, x2d.stride(0),
              signs.data_ptr(), thresholds.data_ptr(), bits, codes.data_ptr(), norms.data_ptr(), _lib.stream_of(x2d))
    return codes, norms


def tq_mse_quantize(x2d, rotation_t, thresholds, bits):
    """x [nvec, D] -> (codes uint8 [nvec, D*sb/8], norms fp16 [nvec])."""
    _lib.require_device(x2d, rotation_t, thresholds)
    nvec, d = x2d.shape
    if x2d.stride(1) != 1:
        x2d = x2d.contiguous()
    sb = 2 if bits == 2 else 4
    codes = torch.empty((nvec, d * sb // 8), dtype=torch.uint8, device=x2d.device)
    norms = torch.empty((nvec,), dtype=torch.float16, device=x2d.device)
    _lib.call("anna_mi_tq_mse_quantize", x2d.data_ptr(), _lib.dtype_code(x2d.dtype), nvec, d, x2d.stride(0),
              rotation_t.data_ptr(), thresholds.data_ptr(), bits, codes.data_ptr(), norms.data_ptr(),
              _lib.stream_of(x2d))
    return codes, norms


def tq_mse_dequant(codes, norms, rotation, centroids, bits, out_dtype=torch.bfloat16):
    _lib.require_device(codes, norms, rotation, centroids)
    codes, norms = codes.contiguous(), norms.contiguous()
    nvec = codes.size(0)
    d = rotation.size(0)
    out = torch.empty((nvec, d), dtype=out_dtype, device=codes.device)
    _lib.call("anna_mi_tq_mse_dequant", codes.data_ptr(), norms.data_ptr(), nvec, d, rotation.data_ptr(),
              centroids.data_ptr(), bits, out.data_ptr(), _lib.dtype_code(out_dtype), d, _lib.stream_of(codes))
    return out


def tq_values_quantize(values, bits, group_size):
    """values [H, T, D] (last dim contiguous) -> (data uint8 [H,T,P], scales, zeros [H,T,D/group])."""
    _lib.require_device(values)
    h, t, d = values.shape
    if values.stride(2) != 1:
        values = values.contiguous()
    sb = 2 if bits == 2 else 4
    data = torch.empty((h, t, d * sb // 8), dtype=torch.uint8, device=values.device)
    scales = torch.empty((h, t, d // group_size), dtype=values.dtype, device=values.device)
    zeros = torch.empty_like(scales)
    _lib.call("anna_mi_tq_values_quantize", values.data_ptr(), _lib.dtype_code(values.dtype), h, t, d,
              values.stride(0), values.stride(1), bits, group_size, data.data_ptr(), scales.data_ptr(),
              zeros.data_ptr(), _lib.stream_of(values))
    return data, scales, zeros


def tq_values_dequant(data, scales, zeros, bits, group_size, out_dtype):
    _lib.require_device(data, scales, zeros)
    data, scales, zeros = data.contiguous(), scales.contiguous(), zeros.contiguous()
    d = scales.size(-1) * group_size
    rows = data.numel() // data.size(-1)
    out = torch.empty((*data.shape[:-1], d), dtype=out_dtype, device=data.device)
    _lib.call("anna_mi_tq_values_dequant", data.data_ptr(), scales.data_ptr(), zeros.data_ptr(),
              _lib.dtype_code(scales.dtype), rows, d, bits, group_size, out.data_ptr(), _lib.dtype_code(out_dtype),
              _lib.stream_of(data))
    return out




# ---------------------------------------------------------------- TurboQuant inner-product keys
# (the TurboQuantIP quantizer behind turboquant.py:255-332)


def tq_ip_gaussian(head_dim: int, seed: int) -> torch.Tensor:
    """QJL matrix G (fp32 [D, D], host): seeded standard normals from the native library."""
    out = torch.empty((head_dim, head_dim), dtype=torch.float32)
    _lib.call("anna_mi_tq_ip_gaussian", head_dim, seed, out.data_ptr())
    return out


def tq_ip_quantize(x2d, signs, thresholds, centroids, gaussian_t, bits):
    """x [nvec, D] -> (mse_indices uint8 [nvec, D], norms fp32 [nvec], qjl_signs uint8 [nvec, D],
    residual_norms fp32 [nvec])."""
    _lib.require_device(x2d, signs, thresholds, centroids, gaussian_t)
    nvec, d = x2d.shape
    if x2d.stride(1) != 1:
        x2d = x2d.contiguous()
    dev = x2d.device
    idx = torch.empty((nvec, d), dtype=torch.uint8, device=dev)
    qjl = torch.empty((nvec, d), dtype=torch.uint8, device=dev)
    norms = torch.empty((nvec,), dtype=torch.float32, device=dev)
    rn = torch.empty((nvec,), dtype=torch.float32, device=dev)
    _lib.call("anna_mi_tq_ip_quantize", x2d.data_ptr(), _lib.dtype_code(x2d.dtype), nvec, d, max(x2d.stride(0), d),
              signs.data_ptr(), thresholds.data_ptr(), centroids.data_ptr(), gaussian_t.data_ptr(), bits,
              idx.data_ptr(), qjl.data_ptr(), norms.data_ptr(), rn.data_ptr(), _lib.stream_of(x2d))
    return idx, norms, qjl, rn


def tq_ip_dequant(idx, norms, qjl, rn, signs, centroids, gaussian, bits, out_dtype=torch.float32):
    """-> [nvec, D] reconstruction (flattened state of nvec vectors)."""
    _lib.require_device(idx, norms, qjl, rn, signs, centroids, gaussian)
    d = idx.size(-1)
    idx, qjl = idx.reshape(-1, d).contiguous(), qjl.reshape(-1, d).contiguous()
    norms, rn = norms.reshape(-1).float().contiguous(), rn.reshape(-1).float().contiguous()
    nvec = idx.size(0)
    if qjl.size(0) != nvec or norms.numel() != nvec or rn.numel() != nvec:
        raise RuntimeError("TurboQuant key state: mse_indices, qjl_signs, norms and residual_norms disagree")
    out = torch.empty((nvec, d), dtype=out_dtype, device=idx.device)
    _lib.call("anna_mi_tq_ip_dequant", idx.data_ptr(), qjl.data_ptr(), norms.data_ptr(), rn.data_ptr(), nvec, d,
              signs.data_ptr(), centroids.data_ptr(), gaussian.data_ptr(), bits, out.data_ptr(),
              _lib.dtype_code(out_dtype), d, _lib.stream_of(idx))
    return out


def tq_ip_scores(query, idx, norms, qjl, rn, signs, centroids, gaussian_t, bits, scaling):
    """query [Hq, Lq, D], state [Hkv, T, D] / [Hkv, T(, 1)] -> fp32 [Hkv, Hq/Hkv, Lq, T]."""
    _lib.require_device(query, idx, norms, qjl, rn, signs, centroids, gaussian_t)
    hq, lq, d = query.shape
    hkv, t = idx.shape[0], idx.shape[1]
    if query.stride(2) != 1:
        query = query.contiguous()
    idx, qjl = idx.contiguous(), qjl.contiguous()
    norms, rn = norms.reshape(hkv, t).float().contiguous(), rn.reshape(hkv, t).float().contiguous()
    dev = query.device
    out = torch.empty((hkv, hq // hkv, lq, t), dtype=torch.float32, device=dev)
    ws = torch.empty((max(2 * hq * lq * d, 1),), dtype=torch.float32, device=dev)
    _lib.call("anna_mi_tq_ip_scores", query.data_ptr(), _lib.dtype_code(query.dtype), hq, lq, d, query.stride(0),
              query.stride(1), idx.data_ptr(), qjl.data_ptr(), norms.data_ptr(), rn.data_ptr(), hkv, t,
              signs.data_ptr(), centroids.data_ptr(), gaussian_t.data_ptr(), bits, float(scaling), ws.data_ptr(),
              out.data_ptr(), _lib.stream_of(query))
    return out


# ---------------------------------------------------------------- tiled int4 GEMV, LM-head top-k
# (sycl:3272-3343 xpu_int4_gemv_tiled, sycl:2137-2572 lm_head_int4_topk_fused)


def _tiled_layout(qweight, qscale, qzeros, group_size, in_features, *, lm_head):
    """-> (tiles, packed_cols, tile, rows N, group_count, scale stride per group, per row).
    qweight [N/T, Kp/8, T] (or [N, Kp/8] for the LM head); qscale [G, N/T, T], [G, N] or, for the
    LM head, [N, G] (validate_lm_head_int4_topk_inputs, sycl:1045-1086)."""
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int8:
        raise RuntimeError("qweight must be int32 and qzeros int8")
    if qscale.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError("qscale must be float32, float16, or bfloat16")
    if not (qweight.is_contiguous() and qscale.is_contiguous() and qzeros.is_contiguous()):
        raise RuntimeError("qweight, qscale and qzeros must be contiguous")
    if qzeros.shape != qscale.shape:
        raise RuntimeError("qzeros shape must match qscale")
    if group_size <= 0 or group_size % 8 != 0:
        raise RuntimeError("group_size must be a positive multiple of 8")
    if qweight.dim() == 3:
        tiles, pc, tile = qweight.shape
        if tile not in (1, 2, 4, 8):
            raise RuntimeError("output_tile must be 1, 2, 4, or 8")
    elif qweight.dim() == 2 and lm_head:
        (tiles, pc), tile = qweight.shape, 1
    else:
        raise RuntimeError("qweight must be [output_tiles, packed_cols, output_tile]")
    n = tiles * tile
    if pc * 8 < in_features:
        raise RuntimeError("qweight packed columns are smaller than in_features")
    if qscale.dim() == 3 and not lm_head:
        if qscale.shape[1] != tiles or qscale.shape[2] != tile:
            raise RuntimeError("qscale must be [group_count, output_tiles, output_tile] matching qweight")
        g, ssg, ssn = qscale.shape[0], n, 1
    elif qscale.dim() == 2 and qscale.shape[1] == n and qscale.shape[0] * group_size >= in_features:
        g, ssg, ssn = qscale.shape[0], n, 1
    elif lm_head and qscale.dim() == 2 and qscale.shape[0] == n and qscale.shape[1] * group_size >= in_features:
        g, ssg, ssn = qscale.shape[1], 1, qscale.shape[1]
    else:
        raise RuntimeError("qscale must be [group_count, vocab_size] or lm_head top-k layout [vocab_size, group_count]")
    if g * group_size < in_features:
        raise RuntimeError("qscale group count is smaller than in_features")
    return tiles, pc, tile, n, g, ssg, ssn


def int4_gemv_tiled(hidden_states, qweight, qscale, qzeros, group_size, in_features, out_features):
    """y [M, out_features] = x . dequant(W)^T on the tiled layout, in x's dtype."""
    if hidden_states.dim() != 2 or hidden_states.shape[1] != in_features:
        raise RuntimeError("xpu_int4_gemv_tiled expects hidden_states shaped [rows, in_features]")
    _check_same_device("xpu_int4_gemv_tiled", hidden_states, qweight, qscale, qzeros)
    tiles, pc, tile, n, g, ssg, ssn = _tiled_layout(qweight, qscale, qzeros, group_size, in_features, lm_head=False)
    if n < out_features or out_features <= 0:
        raise RuntimeError("qweight output tiles are smaller than out_features")
    x = hidden_states if hidden_states.stride(1) == 1 else hidden_states.contiguous()
    y = torch.empty((x.shape[0], out_features), dtype=x.dtype, device=x.device)
    _lib.call("anna_mi_int4_gemv_tiled", x.data_ptr(), _lib.dtype_code(x.dtype), x.shape[0], in_features, x.stride(0),
              qweight.data_ptr(), tiles, pc, tile, qscale.data_ptr(), _lib.dtype_code(qscale.dtype), qzeros.data_ptr(), g,
              ssg, ssn, int(group_size), int(out_features), y.data_ptr(), 0, out_features, _lib.stream_of(x))
    return y


def lm_head_int4_topk(hidden_states, qweight, qscale, qzeros, group_size, in_features, top_k):
    """(values [..., k] in x's dtype, indices [..., k] int64) of the fp32 int4 logits, descending
    (ties to the lower vocabulary index)."""
    if hidden_states.dim() < 2 or hidden_states.shape[-1] != in_features:
        raise RuntimeError("hidden_states hidden_dim must match in_features")
    _check_same_device("lm_head_int4_topk_fused", hidden_states, qweight, qscale, qzeros)
    tiles, pc, tile, vocab, g, ssg, ssn = _tiled_layout(qweight, qscale, qzeros, group_size, in_features, lm_head=True)
    if not (1 <= top_k <= vocab):
        raise RuntimeError("top_k must be in [1, vocab_size]")
    lead = hidden_states.shape[:-1]
    x = hidden_states.reshape(-1, in_features)
    if x.stride(1) != 1:
        x = x.contiguous()
    rows = x.shape[0]
    logits = torch.empty((rows, vocab), dtype=torch.float32, device=x.device)
    values = torch.empty((rows, top_k), dtype=x.dtype, device=x.device)
    indices = torch.empty((rows, top_k), dtype=torch.int64, device=x.device)
    _lib.call("anna_mi_lm_head_int4_topk", x.data_ptr(), _lib.dtype_code(x.dtype), rows, in_features, x.stride(0),
              qweight.data_ptr(), tiles, pc, tile, qscale.data_ptr(), _lib.dtype_code(qscale.dtype), qzeros.data_ptr(),
              g, ssg, ssn, int(group_size), vocab, int(top_k), logits.data_ptr(), values.data_ptr(), indices.data_ptr(),
              _lib.stream_of(x))
    return values.view(*lead, top_k), indices.view(*lead, top_k)


def _lm_head_topk_meta(hidden_states, qweight, qscale, qzeros, group_size, in_features, top_k):
    lead = hidden_states.shape[:-1]
    return (hidden_states.new_empty((*lead, top_k)), hidden_states.new_empty((*lead, top_k), dtype=torch.int64))


# ---------------------------------------------------------------- MoE (sycl:3716-4324, ops.py:3280-3457)


def _check_same_device(name, *tensors):
    dev = tensors[0].device
    _lib.require_device(tensors[0])
    for t in tensors[1:]:
        if t.device != dev:
            raise RuntimeError(f"{name}: all tensors must be on {dev}")


def moe_router(router_logits, top_k, normalize_topk_prob=True):
    """softmax(fp32) -> top-k -> optional renorm -> usage; returns (weights fp32 [T,k],
    selected int64 [T,k], usage int32 [E]) (moe_router_fused, sycl:3731-3839)."""
    if router_logits.dim() != 2:
        raise RuntimeError("router_logits must be [tokens, num_experts]")
    t, e = router_logits.shape
    if not (0 < top_k <= e):
        raise RuntimeError("top_k must be in [1, num_experts]")
    _lib.require_device(router_logits)
    logits = router_logits if router_logits.stride(1) == 1 else router_logits.contiguous()
    w = torch.empty((t, top_k), dtype=torch.float32, device=logits.device)
    sel = torch.empty((t, top_k), dtype=torch.int64, device=logits.device)
    usage = torch.empty((e,), dtype=torch.int32, device=logits.device)
    _lib.call("anna_mi_moe_router", logits.data_ptr(), _lib.dtype_code(logits.dtype), t, e, logits.stride(0),
              int(top_k), int(bool(normalize_topk_prob)), w.data_ptr(), sel.data_ptr(), usage.data_ptr(),
              _lib.stream_of(logits))
    return w, sel, usage


def moe_route_small(router_logits, top_k, normalize_topk_prob, slots):
    """moe_router followed by the ordering half of moe_dispatch in one launch, for
    tokens * top_k <= 1024 and num_experts <= 512.  Returns (weights fp32 [T,k], selected int64
    [T,k], usage int32 [E], expert_offsets [E+1], sorted_token_idx [R], sorted_route_idx [R],
    route_pos [R], items int32 [4 + 4E]) -- the same values moe_router + moe_dispatch give, plus
    the grouped MLP's list of experts with routes (bank slot slots[e])."""
    if router_logits.dim() != 2:
        raise RuntimeError("router_logits must be [tokens, num_experts]")
    t, e = router_logits.shape
    if not (0 < top_k <= min(e, 64)) or e > 512 or not (0 < t * top_k <= 1024):
        raise RuntimeError("moe_route_small: need 0 < tokens * top_k <= 1024, num_experts <= 512, top_k <= 64")
    if slots.dtype != torch.int64 or slots.numel() != e:
        raise RuntimeError("moe_route_small: slots must be int64 [num_experts]")
    _check_same_device("moe_route_small", router_logits, slots)
    logits = router_logits if router_logits.stride(1) == 1 else router_logits.contiguous()
    dev, r = logits.device, t * top_k
    w = torch.empty((t, top_k), dtype=torch.float32, device=dev)
    sel = torch.empty((t, top_k), dtype=torch.int64, device=dev)
    usage = torch.empty((e,), dtype=torch.int32, device=dev)
    offsets = torch.empty((e + 1,), dtype=torch.int64, device=dev)
    sti = torch.empty((r,), dtype=torch.int64, device=dev)
    sri = torch.empty((r,), dtype=torch.int64, device=dev)
    route_pos = torch.empty((r,), dtype=torch.int64, device=dev)
    items = torch.empty((4 + 4 * e,), dtype=torch.int32, device=dev)
    _lib.call("anna_mi_moe_route_small", logits.data_ptr(), _lib.dtype_code(logits.dtype), t, e, logits.stride(0),
              int(top_k), int(bool(normalize_topk_prob)), w.data_ptr(), sel.data_ptr(), usage.data_ptr(),
              offsets.data_ptr(), sti.data_ptr(), sri.data_ptr(), route_pos.data_ptr(), slots.contiguous().data_ptr(),
              items.data_ptr(), _lib.stream_of(logits))
    return w, sel, usage, offsets, sti, sri, route_pos, items


def _weights_for_gather(routing_weights):
    """Routing weights as the gather reads them: bf16 / fp16 / fp32 as given (the kernel rounds
    them to the hidden dtype, no separate cast launch), other dtypes via fp32."""
    rw = routing_weights
    if rw.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        rw = rw.float()
    return rw.contiguous()


def moe_gather(hidden_states, routing_weights, sorted_route_idx, top_k):
    """The gathering half of moe_dispatch: (compact_hidden [R,H], compact_routing_weights [R,1])
    for routes already ordered by moe_route_small."""
    if hidden_states.dim() != 2 or routing_weights.dim() != 2:
        raise RuntimeError("moe_gather: expected hidden [T,H] and routing_weights [T,k]")
    _check_same_device("moe_gather", hidden_states, routing_weights, sorted_route_idx)
    hs = hidden_states if hidden_states.stride(1) == 1 else hidden_states.contiguous()
    rw = _weights_for_gather(routing_weights)
    r, h = sorted_route_idx.numel(), hs.shape[1]
    compact = torch.empty((r, h), dtype=hs.dtype, device=hs.device)
    cw = torch.empty((r, 1), dtype=hs.dtype, device=hs.device)
    _lib.call("anna_mi_moe_gather", hs.data_ptr(), _lib.dtype_code(hs.dtype), h, hs.stride(0), rw.data_ptr(),
              _lib.dtype_code(rw.dtype), sorted_route_idx.contiguous().data_ptr(), r, int(top_k), compact.data_ptr(), cw.data_ptr(),
              _lib.stream_of(hs))
    return compact, cw


def moe_dispatch(hidden_states, routing_weights, selected_experts, expert_usage, *, route_pos=None, slots=None,
                 items=None):
    """Returns (sorted_token_idx [R], expert_offsets [E+1], compact_hidden [R,H],
    compact_routing_weights [R,1]) with routes ordered by (expert, token, k)
    (moe_dispatch_fused, sycl:3867-3965; order of ops.py:3301-3332).  With slots / items, also
    writes the grouped MLP's list of experts with routes (items_prefilled for the MLP)."""
    if hidden_states.dim() != 2 or routing_weights.dim() != 2 or selected_experts.shape != routing_weights.shape:
        raise RuntimeError("moe_dispatch: expected hidden [T,H], routing_weights/selected_experts [T,k]")
    if selected_experts.dtype != torch.int64 or expert_usage.dtype not in (torch.int32, torch.int64):
        raise RuntimeError("moe_dispatch: selected_experts must be int64 and expert_usage int32/int64")
    _check_same_device("moe_dispatch", hidden_states, routing_weights, selected_experts, expert_usage)
    t, h = hidden_states.shape
    k = routing_weights.shape[1]
    e = expert_usage.shape[0]
    if (slots is None) != (items is None):
        raise RuntimeError("moe_dispatch: slots and items go together")
    if items is not None:
        if slots.dtype != torch.int64 or slots.numel() != e or not slots.is_contiguous():
            raise RuntimeError("moe_dispatch: slots must be contiguous int64 [num_experts]")
        if items.dtype != torch.int32 or items.numel() < 4 + 4 * e or not items.is_contiguous():
            raise RuntimeError("moe_dispatch: items must be contiguous int32 [4 + 4 * num_experts]")
        _check_same_device("moe_dispatch", hidden_states, slots, items)
    hs = hidden_states if hidden_states.stride(1) == 1 else hidden_states.contiguous()
    rw = _weights_for_gather(routing_weights)
    sel = selected_experts.contiguous()
    usage = expert_usage.contiguous()
    dev = hs.device
    sti = torch.empty((t * k,), dtype=torch.int64, device=dev)
    sri = torch.empty((t * k,), dtype=torch.int64, device=dev)
    offsets = torch.empty((e + 1,), dtype=torch.int64, device=dev)
    compact = torch.empty((t * k, h), dtype=hs.dtype, device=dev)
    cw = torch.empty((t * k, 1), dtype=hs.dtype, device=dev)
    _lib.call("anna_mi_moe_dispatch", hs.data_ptr(), _lib.dtype_code(hs.dtype), t, h, hs.stride(0), rw.data_ptr(),
              _lib.dtype_code(rw.dtype), sel.data_ptr(), usage.data_ptr(), int(usage.dtype == torch.int64), e, k,
              sti.data_ptr(), sri.data_ptr(), offsets.data_ptr(), compact.data_ptr(), cw.data_ptr(),
              None if route_pos is None else route_pos.data_ptr(), None if slots is None else slots.data_ptr(),
              None if items is None else items.data_ptr(), _lib.stream_of(hs))
    return sti, offsets, compact, cw


def moe_scatter(compact_outputs, sorted_token_idx, num_tokens):
    """out[t] = sum of the compact rows of token t (fp32 accumulation, moe_scatter_fused)."""
    if compact_outputs.dim() != 2 or sorted_token_idx.dim() != 1 or sorted_token_idx.numel() != compact_outputs.shape[0]:
        raise RuntimeError("moe_scatter: expected compact_outputs [R,H] and sorted_token_idx [R]")
    _check_same_device("moe_scatter", compact_outputs, sorted_token_idx)
    co = compact_outputs.contiguous()
    sti = sorted_token_idx.to(torch.int64).contiguous()
    r, h = co.shape
    acc = torch.empty((num_tokens, h), dtype=torch.float32, device=co.device)
    out = torch.empty((num_tokens, h), dtype=co.dtype, device=co.device)
    _lib.call("anna_mi_moe_scatter", co.data_ptr(), _lib.dtype_code(co.dtype), r, h, sti.data_ptr(), int(num_tokens),
              acc.data_ptr(), out.data_ptr(), _lib.stream_of(co))
    return out


def moe_combine(compact_outputs, route_pos, num_tokens, top_k, out=None):
    """Deterministic scatter through the route positions kept from moe_dispatch
    (route_pos int64 [num_tokens * top_k]: the compact row of token t's k-th route)."""
    if compact_outputs.dim() != 2:
        raise RuntimeError("moe_combine: compact_outputs must be [routes, hidden]")
    if route_pos.dtype != torch.int64 or route_pos.numel() != int(num_tokens) * int(top_k):
        raise RuntimeError("moe_combine: route_pos must be int64 with num_tokens * top_k elements")
    if int(num_tokens) * int(top_k) > compact_outputs.shape[0]:
        raise RuntimeError("moe_combine: fewer compact rows than num_tokens * top_k")
    _check_same_device("moe_combine", compact_outputs, route_pos)
    co = compact_outputs.contiguous()
    route_pos = route_pos.contiguous()
    h = co.shape[1]
    if out is None:
        out = torch.empty((num_tokens, h), dtype=co.dtype, device=co.device)
    _lib.call("anna_mi_moe_combine", co.data_ptr(), _lib.dtype_code(co.dtype), h, route_pos.data_ptr(),
              int(num_tokens), int(top_k), out.data_ptr(), _lib.stream_of(co))
    return out


def moe_mlp_args(compact_hidden_states, compact_routing_weights, compact_outputs, expert_offsets, active_experts,
                 active_slots, gate_qweight, gate_qscale, gate_qzeros, up_qweight, up_qscale, up_qzeros,
                 down_qweight, down_qscale, down_qzeros, group_size, activation,
                 max_routes_per_expert, items=None, items_prefilled=False) -> _lib.MoeMlpArgs:
    a = _lib.MoeMlpArgs()
    a.dtype = _lib.dtype_code(compact_hidden_states.dtype)
    a.scale_dtype = _lib.dtype_code(gate_qscale.dtype)
    a.routes, a.hidden_dim = compact_hidden_states.shape
    a.intermediate_dim = gate_qweight.shape[1]
    a.compact_hidden, a.compact_weights = compact_hidden_states.data_ptr(), compact_routing_weights.data_ptr()
    a.compact_outputs, a.expert_offsets = compact_outputs.data_ptr(), expert_offsets.data_ptr()
    a.active_experts, a.active_slots, a.active_count = active_experts.data_ptr(), active_slots.data_ptr(), active_experts.numel()
    a.gate_qweight, a.gate_qscale, a.gate_qzeros = gate_qweight.data_ptr(), gate_qscale.data_ptr(), gate_qzeros.data_ptr()
    a.up_qweight, a.up_qscale, a.up_qzeros = up_qweight.data_ptr(), up_qscale.data_ptr(), up_qzeros.data_ptr()
    a.down_qweight, a.down_qscale, a.down_qzeros = down_qweight.data_ptr(), down_qscale.data_ptr(), down_qzeros.data_ptr()
    a.hidden_packed_cols, a.hidden_groups = gate_qweight.shape[2], gate_qscale.shape[1]
    a.intermediate_packed_cols, a.intermediate_groups = down_qweight.shape[2], down_qscale.shape[1]
    a.group_size = int(group_size)
    a.activation = activation.data_ptr()
    a.sweep_chunks = min(4, max(1, -(-int(max_routes_per_expert) // 16)))
    a.items = None if items is None else items.data_ptr()
    a.items_prefilled = int(bool(items_prefilled) and items is not None)
    return a


def moe_grouped_int4_mlp_out(compact_hidden_states, compact_routing_weights, compact_outputs, expert_offsets,
                             active_experts, active_slots, gate_qweight, gate_qscale, gate_qzeros, up_qweight,
                             up_qscale, up_qzeros, down_qweight, down_qscale, down_qzeros, group_size,
                             max_routes_per_expert, activation=None, items=None, items_prefilled=False):
    """moe_grouped_int4_mlp_fused (sycl:4078-4324): writes the routes of the active experts
    into compact_outputs and returns it.  items: optional int32 workspace [4 + 4 * active
    experts]; with it the experts that have routes are listed on the device and the launches
    walk only those (callers that pass every expert as active, without a host sync);
    items_prefilled: items already holds that list (from moe_route_small)."""
    bank = (gate_qweight, gate_qscale, gate_qzeros, up_qweight, up_qscale, up_qzeros, down_qweight, down_qscale,
            down_qzeros)
    _check_same_device("moe_grouped_int4_mlp_fused", compact_hidden_states, compact_routing_weights, compact_outputs,
                       expert_offsets, active_experts, active_slots, *bank)
    if compact_hidden_states.dim() != 2 or compact_outputs.shape != compact_hidden_states.shape:
        raise RuntimeError("compact_outputs shape must match compact_hidden_states [routes, hidden_dim]")
    if not compact_outputs.is_contiguous():
        raise RuntimeError("compact_outputs must be contiguous")
    if compact_routing_weights.dtype != compact_hidden_states.dtype or compact_outputs.dtype != compact_hidden_states.dtype:
        raise RuntimeError("compact_routing_weights / compact_outputs dtype must match compact_hidden_states")
    if expert_offsets.dtype != torch.int64 or active_experts.dtype != torch.int64 or active_slots.dtype != torch.int64:
        raise RuntimeError("expert_offsets, active_experts and active_slots must be int64")
    if active_experts.numel() != active_slots.numel() or active_experts.numel() == 0:
        raise RuntimeError("active_experts/active_slots count mismatch or empty")
    if int(max_routes_per_expert) <= 0:
        raise RuntimeError("max_routes_per_expert must be positive")
    for name, t, dt in (("gate_qweight", gate_qweight, torch.int32), ("up_qweight", up_qweight, torch.int32),
                        ("down_qweight", down_qweight, torch.int32), ("gate_qzeros", gate_qzeros, torch.int8),
                        ("up_qzeros", up_qzeros, torch.int8), ("down_qzeros", down_qzeros, torch.int8)):
        if t.dtype != dt or t.dim() != 3:
            raise RuntimeError(f"{name} must be a rank-3 {dt} tensor")
    if not (gate_qscale.dtype == up_qscale.dtype == down_qscale.dtype):
        raise RuntimeError("the bank's qscale tensors must share one dtype")
    if gate_qweight.shape != up_qweight.shape or gate_qscale.shape != up_qscale.shape:
        raise RuntimeError("gate/up bank shape mismatch")
    x = compact_hidden_states.contiguous()
    cw = compact_routing_weights.contiguous()
    bank = tuple(t.contiguous() for t in bank)
    if activation is None:
        activation = torch.empty((x.shape[0], gate_qweight.shape[1]), dtype=torch.float32, device=x.device)
    if items is not None and (items.dtype != torch.int32 or not items.is_contiguous()
                              or items.numel() < 4 + 4 * active_experts.numel() or items.device != x.device):
        raise RuntimeError("items must be a contiguous int32 tensor of >= 4 + 4 * active experts on the device")
    # every tensor whose pointer goes into the args stays bound to a local until the launch
    offsets = expert_offsets.contiguous()
    experts = active_experts.contiguous()
    slots = active_slots.contiguous()
    a = moe_mlp_args(x, cw, compact_outputs, offsets, experts, slots, *bank, group_size, activation,
                     max_routes_per_expert, items, items_prefilled)
    _lib.call("anna_mi_moe_grouped_int4_mlp", ctypes.byref(a), _lib.stream_of(x))
    del offsets, experts, slots, bank, cw, x
    return compact_outputs


def _moe_router_meta(router_logits, top_k, normalize_topk_prob=True):
    t, e = router_logits.shape
    return (router_logits.new_empty((t, top_k), dtype=torch.float32),
            router_logits.new_empty((t, top_k), dtype=torch.int64), router_logits.new_empty((e,), dtype=torch.int32))


def _moe_dispatch_meta(hidden_states, routing_weights, selected_experts, expert_usage):
    r = routing_weights.numel()
    return (selected_experts.new_empty((r,)), selected_experts.new_empty((expert_usage.shape[0] + 1,)),
            hidden_states.new_empty((r, hidden_states.shape[1])), hidden_states.new_empty((r, 1)))


# ---------------------------------------------------------------- registration

_IMPLS = {
    "xpu_int4_gemv": (_xpu_int4_gemv_impl, _xpu_int4_gemv_meta),
    "gqa_decode_splitkv_fused": (_gqa_decode_splitkv_fused_impl, lambda q, *a, **k: q.new_empty(q.shape)),
    "gqa_decode_splitkv_fused_out": (_gqa_decode_splitkv_fused_out_impl, lambda q, k, v, out, *a, **kw: out),
    "gqa_decode_splitkv_turboquant_fused_out": (
        _gqa_decode_splitkv_turboquant_fused_out_impl,
        lambda q, qk, vd, vs, vz, rk, rv, out, *a, **kw: out,
    ),
    "xpu_int4_gemv_tiled": (int4_gemv_tiled, lambda x, qw, qs, qz, g, k, n: x.new_empty((x.shape[0], n))),
    "lm_head_int4_topk_fused": (lm_head_int4_topk, _lm_head_topk_meta),
    "moe_router_fused": (moe_router, _moe_router_meta),
    "moe_dispatch_fused": (moe_dispatch, _moe_dispatch_meta),
    "moe_scatter_fused": (moe_scatter, lambda co, sti, n: co.new_empty((n, co.shape[1]))),
    "moe_grouped_int4_mlp_fused": (moe_grouped_int4_mlp_out, lambda x, w, out, *a, **k: out),
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


def run_gqa_decode_splitkv_fused(*, query, key, value, scaling, block_size, gate=None):
    op = _op("gqa_decode_splitkv_fused")
    if gate is None:
        return op(query, key, value, float(scaling), int(block_size))
    return op(query, key, value, float(scaling), int(block_size), gate)


def run_gqa_decode_splitkv_fused_out(*, query, key, value, output, partial_stats, partial_values, scaling,
                                     block_size, gate=None):
    op = _op("gqa_decode_splitkv_fused_out")
    if gate is None:
        return op(query, key, value, output, partial_stats, partial_values, float(scaling), int(block_size))
    return op(query, key, value, output, partial_stats, partial_values, float(scaling), int(block_size), gate)


def run_gqa_decode_splitkv_turboquant_fused_out(*, query, quantized_key, value_data, value_scales, value_zeros,
                                                residual_key, residual_value, output, partial_stats, partial_values,
                                                scaling, value_bits, value_group_size, block_size, gate=None):
    op = _op("gqa_decode_splitkv_turboquant_fused_out")
    args = (query, quantized_key, value_data, value_scales, value_zeros, residual_key, residual_value, output,
            partial_stats, partial_values, float(scaling), int(value_bits), int(value_group_size), int(block_size))
    return op(*args) if gate is None else op(*args, gate)


def run_moe_router_fused(*, router_logits, top_k, normalize_topk_prob=True):
    return _op("moe_router_fused")(router_logits, int(top_k), bool(normalize_topk_prob))


def run_moe_dispatch_fused(*, hidden_states, routing_weights, selected_experts, expert_usage):
    return _op("moe_dispatch_fused")(hidden_states, routing_weights, selected_experts, expert_usage)


def run_moe_scatter_fused(*, compact_outputs, sorted_token_idx, num_tokens):
    return _op("moe_scatter_fused")(compact_outputs, sorted_token_idx, int(num_tokens))


def run_moe_grouped_int4_mlp_fused(*, compact_hidden_states, compact_routing_weights, compact_outputs, expert_offsets,
                                   active_experts, active_slots, gate_qweight, gate_qscale, gate_qzeros, up_qweight,
                                   up_qscale, up_qzeros, down_qweight, down_qscale, down_qzeros, group_size,
                                   max_routes_per_expert):
    return _op("moe_grouped_int4_mlp_fused")(
        compact_hidden_states, compact_routing_weights, compact_outputs, expert_offsets, active_experts, active_slots,
        gate_qweight, gate_qscale, gate_qzeros, up_qweight, up_qscale, up_qzeros, down_qweight, down_qscale,
        down_qzeros, int(group_size), int(max_routes_per_expert))


def run_xpu_int4_gemv_tiled(*, hidden_states, qweight, qscale, qzeros, group_size, in_features, out_features):
    return _op("xpu_int4_gemv_tiled")(hidden_states, qweight, qscale, qzeros, int(group_size), int(in_features),
                                      int(out_features))


def lm_head_int4_topk_fused_is_available() -> bool:
    register_ops()
    return True


def run_lm_head_int4_topk_fused(*, hidden_states, qweight, qscale, qzeros, group_size, in_features, top_k):
    return _op("lm_head_int4_topk_fused")(hidden_states, qweight, qscale, qzeros, int(group_size), int(in_features),
                                          int(top_k))

"""Drop-in int4 weight-only linear modules for ROCm (MI355X).

Mirrors the public API of the reference's src/anna/model/quantization.py:
``XPUInt4Linear`` (same constructor, buffers, ``from_linear``, ``forward``, LM-head
layout helpers), ``AutoRoundGPTQLinear`` / ``AWQLinear`` / ``DenseLinear`` loader
modules, ``convert_module_linears_to_xpu_int4``, ``replace_linear_modules`` and the
memory estimators.  The class keeps its reference name so engine code that imports
it by name is unchanged; the device gate is ``cuda`` (ROCm) where the reference
tests for ``xpu``.

All arithmetic on quantized weights runs in the HIP library (packing, repacking,
dequant, GEMV/GEMM).  There is no CPU execution path: forward on host tensors
raises.
"""

from __future__ import annotations

import logging
import os
import re
from collections.abc import Callable
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import torch
import torch.nn.functional as F
from torch import nn

from . import fused_ops

_INT4_PER_WORD = 8
_INT4_MATMUL_STRATEGIES = frozenset({"auto", "torch", "dequant", "gemv"})
_LM_HEAD_TILE = 4
_AUTO_ROUND_METHODS = frozenset({"auto-round", "auto_round"})
_AUTO_ROUND_PACKINGS = frozenset({"auto_round:auto_gptq"})
_FLOAT_OVERRIDE_TYPES = frozenset({"fp", "float", "float16", "fp16", "bfloat16", "bf16"})
_REGEX_CHARS = frozenset("\\[](){}?*+^$|")

logger = logging.getLogger(__name__)


@dataclass(slots=True)
class QuantizationConfig:
    """Checkpoint quantization config (fields of the reference's
    qwen3_5_text_config.py:49-96 QuantizationConfig)."""

    quant_method: str | None = None
    bits: int | None = None
    group_size: int | None = None
    zero_point: bool = False
    data_type: str | None = None
    sym: bool | None = None
    packing_format: str | None = None
    autoround_version: str | None = None
    block_name_to_quantize: tuple[str, ...] = ()
    extra_config: dict[str, dict[str, Any]] = field(default_factory=dict)
    modules_to_not_convert: list[str] = field(default_factory=list)
    version: str | None = None

    @property
    def is_enabled(self) -> bool:
        return self.quant_method is not None

    @classmethod
    def from_dict(cls, data: dict[str, Any] | None) -> "QuantizationConfig":
        if not data:
            return cls()
        blocks = data.get("block_name_to_quantize")
        if blocks is None:
            blocks = ()
        elif isinstance(blocks, str):
            blocks = (blocks,)
        else:
            blocks = tuple(str(b) for b in blocks)
        extra = {str(k): dict(v) for k, v in (data.get("extra_config") or {}).items() if isinstance(v, dict)}
        return cls(
            quant_method=data.get("quant_method"),
            bits=data.get("bits"),
            group_size=data.get("group_size"),
            zero_point=bool(data.get("zero_point", False)),
            data_type=data.get("data_type"),
            sym=None if data.get("sym") is None else bool(data.get("sym")),
            packing_format=data.get("packing_format"),
            autoround_version=data.get("autoround_version"),
            block_name_to_quantize=blocks,
            extra_config=extra,
            modules_to_not_convert=list(data.get("modules_to_not_convert", [])),
            version=data.get("version"),
        )


# ---------------------------------------------------------------- packing helpers (integer reshuffles)


def _nibble_shifts(device) -> torch.Tensor:
    return torch.arange(0, 32, 4, device=device, dtype=torch.int32)


def unpack_int4_last_dim(packed: torch.Tensor) -> torch.Tensor:
    """int32 [..., C] -> int32 [..., 8C]; value j of word c is column 8c+j (bits 4j)."""
    vals = (packed.to(torch.int32).unsqueeze(-1) >> _nibble_shifts(packed.device)) & 0xF
    return vals.reshape(*packed.shape[:-1], packed.shape[-1] * _INT4_PER_WORD)


def unpack_int4_first_dim(packed: torch.Tensor) -> torch.Tensor:
    """int32 [R, C] -> int32 [8R, C]; value j of word r is row 8r+j."""
    vals = (packed.to(torch.int32).unsqueeze(-1) >> _nibble_shifts(packed.device)) & 0xF
    return vals.permute(0, 2, 1).reshape(packed.shape[0] * _INT4_PER_WORD, packed.shape[1])


def pack_int4_last_dim(values: torch.Tensor) -> torch.Tensor:
    """int [..., 8C] (0..15) -> int32 [..., C]; inverse of unpack_int4_last_dim."""
    v = values.to(torch.int64).reshape(*values.shape[:-1], values.shape[-1] // 8, 8) & 0xF
    word = (v << _nibble_shifts(values.device).to(torch.int64)).sum(-1)
    return torch.where(word >= 2**31, word - 2**32, word).to(torch.int32)


def _require_rocm(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{what} runs on the MI355X HIP path only; got a tensor on {t.device}")


def _empty_param(shape, dtype=None, *, device=None) -> nn.Parameter:
    return nn.Parameter(torch.empty(*shape, dtype=dtype or torch.float32, device=device), requires_grad=False)


# ---------------------------------------------------------------- loader modules


class DenseLinear(nn.Module):
    def __init__(self, in_features: int, out_features: int, bias: bool = False, *, device=None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.weight = _empty_param((out_features, in_features), device=device)
        if bias:
            self.bias = _empty_param((out_features,), device=device)
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        bias = None if self.bias is None else self.bias.to(dtype=x.dtype)
        return F.linear(x, self.weight.to(dtype=x.dtype), bias)


class AutoRoundGPTQLinear(nn.Module):
    """AutoRound ``auto_round:auto_gptq`` payload (reference quantization.py:279-375).

    Buffers: qweight int32 [ceil(K/8), N] (k packed along the first dim), qzeros int32
    [G, ceil(N/8)] storing zero-1, scales fp16 [G, N].  ``forward`` repacks once into
    the int4 kernel layout on the device and runs the HIP int4 linear.
    """

    def __init__(self, in_features, out_features, *, bits=4, group_size=128, sym=True, bias=False,
                 compute_dtype=torch.bfloat16, device=None):
        super().__init__()
        if bits != 4:
            raise ValueError("AutoRoundGPTQLinear currently only supports 4-bit weights.")
        if group_size <= 0:
            raise ValueError("AutoRoundGPTQLinear requires a positive group_size.")
        self.in_features = in_features
        self.out_features = out_features
        self.bits = bits
        self.group_size = group_size
        self.sym = sym
        self.compute_dtype = compute_dtype
        self.packed_in_features = (in_features + 7) // 8
        self.packed_out_features = (out_features + 7) // 8
        self.group_count = (in_features + group_size - 1) // group_size
        self.register_parameter("weight", None)
        self.register_buffer("qweight", torch.empty((self.packed_in_features, out_features), dtype=torch.int32, device=device))
        self.register_buffer("qzeros", torch.empty((self.group_count, self.packed_out_features), dtype=torch.int32, device=device))
        self.register_buffer("scales", torch.empty((self.group_count, out_features), dtype=torch.float16, device=device))
        if bias:
            self.bias = _empty_param((out_features,), dtype=compute_dtype, device=device)
        else:
            self.register_parameter("bias", None)
        self._converted: XPUInt4Linear | None = None

    def _to_xpu_int4_tensors(self, *, padded_in_features: int):
        if padded_in_features < self.in_features:
            raise ValueError("AutoRound packed weight cannot shrink in_features during conversion.")
        _require_rocm(self.qweight, "AutoRound repacking")
        return fused_ops.autoround_to_int4(
            self.qweight, self.qzeros, self.scales, in_features=self.in_features, out_features=self.out_features,
            group_size=self.group_size, padded_in_features=padded_in_features,
        )

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._converted is None or self._converted.qweight.device != x.device:
            self._converted = XPUInt4Linear.from_linear(self, compute_dtype=self.compute_dtype, device=x.device)
        return self._converted(x.to(self.compute_dtype)).to(x.dtype)


class AWQLinear(nn.Module):
    """AWQ payload (reference quantization.py:378-457); converted to the int4 kernel layout on use."""

    def __init__(self, in_features, out_features, *, bits=4, group_size=128, zero_point=True, bias=False,
                 compute_dtype=torch.float16, device=None):
        super().__init__()
        if bits != 4:
            raise ValueError("The current AWQ implementation only supports 4-bit weights.")
        self.in_features = in_features
        self.out_features = out_features
        self.bits = bits
        self.group_size = group_size
        self.zero_point = zero_point
        self.compute_dtype = compute_dtype
        self.register_parameter("weight", None)
        self.register_buffer("qweight", torch.empty(0, dtype=torch.int32, device=device))
        self.register_buffer("qzeros", torch.empty(0, dtype=torch.int32, device=device))
        self.register_buffer("scales", torch.empty(0, dtype=torch.float16, device=device))
        if bias:
            self.bias = _empty_param((out_features,), dtype=compute_dtype, device=device)
        else:
            self.register_parameter("bias", None)
        self._converted: XPUInt4Linear | None = None

    def _to_xpu_int4_tensors(self, *, padded_in_features: int):
        """Integer reshuffle of the AWQ payload into qweight [N, Kp/8], qscale [G, N], qzeros [G, N]."""
        k, n, g = self.in_features, self.out_features, self.group_size
        q = unpack_int4_last_dim(self.qweight)
        zeros = unpack_int4_last_dim(self.qzeros) if self.qzeros.numel() else None
        if q.shape[0] == k and q.shape[1] >= n:  # [K, N] orientation
            q_nk = q[:, :n].t()
            z_gn = None if zeros is None else zeros[:, :n]
            s_gn = self.scales.float()
        elif q.shape[0] == n and q.shape[1] >= k:  # [N, K] orientation
            q_nk = q[:, :k]
            z_gn = None if zeros is None else zeros[:, :k:g].t()
            s_gn = self.scales.float()
            if s_gn.shape[0] == n:
                s_gn = s_gn.t()
        else:
            raise ValueError(f"Unsupported AWQ packed weight shape {tuple(self.qweight.shape)} for target {(n, k)}")
        groups = (padded_in_features + g - 1) // g
        s_gn = s_gn[:groups].contiguous()
        z_gn = torch.full_like(s_gn, 8, dtype=torch.int8) if z_gn is None else z_gn[:groups].to(torch.int8).contiguous()
        padded = torch.empty((n, padded_in_features), dtype=torch.int32, device=q.device)
        padded[:, :k] = q_nk
        if padded_in_features > k:
            tail = min(groups - 1, k // g)
            padded[:, k:] = z_gn[tail].to(torch.int32).unsqueeze(1)
        return pack_int4_last_dim(padded).contiguous(), s_gn, z_gn

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.weight is not None:
            return F.linear(x.to(self.compute_dtype), self.weight.to(self.compute_dtype),
                            None if self.bias is None else self.bias.to(self.compute_dtype)).to(x.dtype)
        if self._converted is None or self._converted.qweight.device != x.device:
            self._converted = XPUInt4Linear.from_linear(self, compute_dtype=self.compute_dtype, device=x.device)
        return self._converted(x.to(self.compute_dtype)).to(x.dtype)


# ---------------------------------------------------------------- the int4 linear


class XPUInt4Linear(nn.Module):
    """Group-wise int4 weight-only linear (reference quantization.py:460-710).

    Buffers: ``qweight`` int32 [N, Kp/8], ``qscale`` fp32 [G, N], ``qzeros`` int8 [G, N].
    ``forward`` runs the HIP int4 GEMV (M <= 16) or MFMA GEMM (M > 16).
    """

    def __init__(self, in_features: int, out_features: int, *, group_size: int = 128, bias: bool = False,
                 compute_dtype: torch.dtype = torch.bfloat16, device=None, padded_in_features: int | None = None):
        super().__init__()
        if group_size <= 0 or group_size % 32 != 0:
            raise ValueError("XPUInt4Linear requires group_size to be a positive multiple of 32.")
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size
        self.compute_dtype = compute_dtype
        self.padded_in_features = padded_in_features or self._padded_in_features(in_features, group_size)
        groups = self.padded_in_features // group_size
        self.register_buffer("qweight", torch.empty((out_features, self.padded_in_features // 8), dtype=torch.int32, device=device))
        self.register_buffer("qscale", torch.empty((groups, out_features), dtype=torch.float32, device=device))
        self.register_buffer("qzeros", torch.empty((groups, out_features), dtype=torch.int8, device=device))
        if bias:
            self.bias = _empty_param((out_features,), dtype=compute_dtype, device=device)
        else:
            self.register_parameter("bias", None)

    @staticmethod
    def _padded_in_features(in_features: int, group_size: int) -> int:
        kp = -(-in_features // group_size) * group_size
        return -(-kp // 8) * 8

    # ---- LM-head tiled layout (reference quantization.py:491-538)
    def prepare_lm_head_topk_layout(self) -> "XPUInt4Linear":
        tile = _LM_HEAD_TILE
        n_pad = -(-self.out_features // tile) * tile
        cols = self.qweight.shape[1]
        qweight = torch.zeros((n_pad, cols), dtype=self.qweight.dtype, device=self.qweight.device)
        qweight[: self.out_features] = self.qweight
        qweight = qweight.view(n_pad // tile, tile, cols).permute(0, 2, 1).contiguous()
        for name, value in (
            ("lm_head_qweight", qweight),
            ("lm_head_qscale", self.qscale.t().contiguous()),
            ("lm_head_qzeros", self.qzeros.t().contiguous()),
        ):
            if name in self._buffers:
                self._buffers[name] = value
            else:
                self.register_buffer(name, value, persistent=True)
        self.lm_head_output_tile = tile
        return self

    def lm_head_topk_tensors(self):
        bufs = [getattr(self, n, None) for n in ("lm_head_qweight", "lm_head_qscale", "lm_head_qzeros")]
        if any(b is None for b in bufs) or bufs[0].device != self.qweight.device:
            self.prepare_lm_head_topk_layout()
            bufs = [self.lm_head_qweight, self.lm_head_qscale, self.lm_head_qzeros]
        qweight, qscale, qzeros = bufs
        if self.out_features % int(getattr(self, "lm_head_output_tile", _LM_HEAD_TILE)) != 0:
            qweight = self.qweight
        return qweight, qscale, qzeros

    # ---- construction
    @classmethod
    def from_linear(cls, module: nn.Module, *, group_size: int = 128, compute_dtype: torch.dtype = torch.bfloat16,
                    device=None) -> "XPUInt4Linear":
        device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        if isinstance(module, (AutoRoundGPTQLinear, AWQLinear)):
            gsz = int(module.group_size)
            kp = cls._padded_in_features(module.in_features, gsz)
            out = cls(module.in_features, module.out_features, group_size=gsz, bias=module.bias is not None,
                      compute_dtype=compute_dtype or module.compute_dtype, device=device, padded_in_features=kp)
            moved = module.to(device) if module.qweight.device != device else module
            qweight, qscale, qzeros = moved._to_xpu_int4_tensors(padded_in_features=kp)
            with torch.no_grad():
                out.qweight.copy_(qweight)
                out.qscale.copy_(qscale)
                out.qzeros.copy_(qzeros)
                if module.bias is not None:
                    out.bias.copy_(module.bias.detach().to(device=device, dtype=out.bias.dtype))
            return out
        weight, bias = _extract_dense_weight_bias(module)
        n, k = int(weight.shape[0]), int(weight.shape[1])
        kp = cls._padded_in_features(k, group_size)
        out = cls(k, n, group_size=group_size, bias=bias is not None, compute_dtype=compute_dtype, device=device,
                  padded_in_features=kp)
        qweight, qscale, qzeros = cls._quantize_weight(weight.to(device), group_size=group_size, padded_in_features=kp)
        with torch.no_grad():
            out.qweight.copy_(qweight)
            out.qscale.copy_(qscale)
            out.qzeros.copy_(qzeros)
            if bias is not None:
                out.bias.copy_(bias.to(device=device, dtype=out.bias.dtype))
        return out

    @staticmethod
    def _quantize_weight(weight: torch.Tensor, *, group_size: int, padded_in_features: int):
        """Device packer, bit-exact with the reference's torch quantizer (quantization.py:597-624)."""
        _require_rocm(weight, "int4 quantization")
        return fused_ops.int4_quantize(weight, group_size=group_size, padded_in_features=padded_in_features)

    def _dequantize_weight(self) -> torch.Tensor:
        _require_rocm(self.qweight, "int4 dequantization")
        return fused_ops.int4_dequant(self.qweight, self.qscale, self.qzeros, self.group_size, self.in_features,
                                      out_dtype=torch.float32)

    @staticmethod
    def _matmul_strategy() -> str:
        strategy = os.getenv("ANNA_XPU_INT4_MATMUL", "auto").strip().lower()
        if strategy not in _INT4_MATMUL_STRATEGIES:
            logger.warning("Ignoring unsupported ANNA_XPU_INT4_MATMUL=%r; using auto.", strategy)
            return "auto"
        return strategy

    def _forward_dequant(self, x2d: torch.Tensor) -> torch.Tensor:
        w = fused_ops.int4_dequant(self.qweight, self.qscale, self.qzeros, self.group_size, self.in_features,
                                   out_dtype=self.compute_dtype)
        bias = None if self.bias is None else self.bias.to(dtype=self.compute_dtype)
        return F.linear(x2d, w, bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        x2d = x.reshape(-1, x.shape[-1]).to(self.compute_dtype)
        _require_rocm(x2d, "XPUInt4Linear.forward")
        if self._matmul_strategy() == "dequant":
            out = self._forward_dequant(x2d)
        else:
            out = torch.empty((x2d.shape[0], self.out_features), dtype=x2d.dtype, device=x2d.device)
            fused_ops.int4_linear_out(x2d, self.qweight, self.qscale, self.qzeros, self.group_size,
                                      x2d.shape[1], out)
            if self.bias is not None:
                out = out + self.bias.to(dtype=out.dtype)
        return out.reshape(*lead, self.out_features).to(dtype=x.dtype)


@dataclass(slots=True)
class QuantizedModuleSpec:
    module_name: str
    quant_method: str


# ---------------------------------------------------------------- module replacement


def _strip_prefix(name: str) -> str:
    for prefix in ("model.language_model.", "model.visual.", "model."):
        if name.startswith(prefix):
            return name[len(prefix):]
    return name


class _Overrides:
    """Per-module overrides and exclusions of a QuantizationConfig (reference quantization.py:724-865)."""

    def __init__(self, cfg: QuantizationConfig):
        self.excluded = tuple(_strip_prefix(c) for c in cfg.modules_to_not_convert)
        self.exact = dict(cfg.extra_config)
        self.stripped: dict[str, dict] = {}
        self.patterns: list[tuple[re.Pattern, re.Pattern | None, dict]] = []
        for pattern, override in cfg.extra_config.items():
            self.stripped.setdefault(_strip_prefix(pattern), override)
            if any(ch in _REGEX_CHARS for ch in pattern):
                stripped = _strip_prefix(pattern)
                try:
                    full = re.compile(pattern)
                    short = None if stripped == pattern else re.compile(stripped)
                except re.error as exc:
                    raise ValueError(f"Invalid quantization extra_config regex {pattern!r}: {exc}") from exc
                self.patterns.append((full, short, override))
        self.blocks = tuple(b for b in cfg.block_name_to_quantize if b)

    def override_for(self, name: str) -> dict | None:
        short = _strip_prefix(name)
        hit = self.exact.get(name) or self.stripped.get(short)
        if hit is not None:
            return hit
        for full, sh, override in self.patterns:
            if full.fullmatch(name) or (sh is not None and sh.fullmatch(short)):
                return override
        return None

    def skip(self, name: str) -> bool:
        short = _strip_prefix(name)
        if any(short == c or short.startswith(c + ".") for c in self.excluded):
            return True
        override = self.override_for(name)
        if override is None:
            return False
        bits = override.get("bits")
        if bits is not None and int(bits) >= 16:
            return True
        dt = override.get("data_type")
        return dt is not None and str(dt).strip().lower() in _FLOAT_OVERRIDE_TYPES

    def in_blocks(self, name: str) -> bool:
        if not self.blocks:
            raise ValueError("AutoRound quantization_config is missing block_name_to_quantize.")
        return any(name == b or name.startswith(b + ".") for b in self.blocks)


def _set_submodule(model: nn.Module, name: str, replacement: nn.Module) -> None:
    parent_name, _, leaf = name.rpartition(".")
    parent = model.get_submodule(parent_name) if parent_name else model
    setattr(parent, leaf, replacement)


def _extract_dense_weight_bias(module: nn.Module):
    if isinstance(module, XPUInt4Linear):
        w = module._dequantize_weight()
    elif isinstance(module, (DenseLinear, nn.Linear)):
        w = module.weight.detach().to(torch.float32)
    else:
        raise TypeError(f"Unsupported linear module for int4 conversion: {type(module)!r}")
    b = None if module.bias is None else module.bias.detach().to(torch.float32)
    return w, b


def estimate_xpu_int4_linear_bytes(in_features: int, out_features: int, *, group_size: int = 128,
                                   has_bias: bool = False, compute_dtype: torch.dtype = torch.bfloat16) -> int:
    kp = XPUInt4Linear._padded_in_features(in_features, group_size)
    groups = kp // group_size
    bias = out_features * torch.empty((), dtype=compute_dtype).element_size() if has_bias else 0
    return out_features * (kp // 8) * 4 + groups * out_features * (4 + 1) + bias


def estimate_module_xpu_int4_bytes(module: nn.Module, *, group_size: int = 128,
                                   compute_dtype: torch.dtype = torch.bfloat16) -> int:
    total = 0
    for child in module.modules():
        if child is module:
            continue
        if isinstance(child, XPUInt4Linear):
            tensors = [child.qweight, child.qscale, child.qzeros, getattr(child, "lm_head_qscale", None),
                       getattr(child, "lm_head_qzeros", None), child.bias]
            total += sum(t.nelement() * t.element_size() for t in tensors if t is not None)
        elif isinstance(child, (AutoRoundGPTQLinear, AWQLinear, DenseLinear, nn.Linear)):
            total += estimate_xpu_int4_linear_bytes(child.in_features, child.out_features, group_size=group_size,
                                                    has_bias=getattr(child, "bias", None) is not None,
                                                    compute_dtype=compute_dtype)
    return total


def _is_lm_head(name: str) -> bool:
    return name == "lm_head" or name.endswith(".lm_head")


def convert_module_linears_to_xpu_int4(module: nn.Module, *, group_size: int = 128,
                                       compute_dtype: torch.dtype | None = None, device=None,
                                       include_predicate: Callable[[str, nn.Module], bool] | None = None,
                                       cache_dir: str | Path | None = None) -> int:
    """Replace every linear (dense, AutoRound, AWQ) under ``module`` with XPUInt4Linear.

    ``cache_dir`` is accepted and ignored: the reference disables its persistent layout
    cache (quantization.py:927) and pins that in its tests.
    """
    del cache_dir
    names = [n for n, _ in module.named_modules() if n]
    count = 0
    for name in names:
        child = module.get_submodule(name)
        if isinstance(child, XPUInt4Linear):
            continue
        if not isinstance(child, (AutoRoundGPTQLinear, AWQLinear, DenseLinear, nn.Linear)):
            continue
        if include_predicate is not None and not include_predicate(name, child):
            continue
        gsz = int(getattr(child, "group_size", group_size))
        cdt = compute_dtype or getattr(child, "compute_dtype", torch.bfloat16)
        replacement = XPUInt4Linear.from_linear(child, group_size=gsz, compute_dtype=cdt, device=device)
        if _is_lm_head(name):
            replacement.prepare_lm_head_topk_layout()
        _set_submodule(module, name, replacement)
        count += 1
    return count


def replace_linear_modules_with_xpu_int4_placeholders(model: nn.Module, *, group_size: int = 128,
                                                      compute_dtype: torch.dtype = torch.bfloat16, device=None,
                                                      include_predicate=None) -> int:
    todo = []
    for name, mod in list(model.named_modules()):
        if not name or not isinstance(mod, nn.Linear):
            continue
        if include_predicate is not None and not include_predicate(name, mod):
            continue
        todo.append((name, XPUInt4Linear(mod.in_features, mod.out_features, group_size=group_size,
                                         bias=mod.bias is not None, compute_dtype=compute_dtype, device=device)))
    for name, rep in todo:
        if _is_lm_head(name):
            rep.prepare_lm_head_topk_layout()
        _set_submodule(model, name, rep)
    return len(todo)


def replace_linear_modules(model: nn.Module, quantization_config: QuantizationConfig, *,
                           compute_dtype: torch.dtype) -> list[QuantizedModuleSpec]:
    cfg = quantization_config
    if not cfg.is_enabled:
        return []
    method = (cfg.quant_method or "").strip().lower()
    if method in _AUTO_ROUND_METHODS:
        if (cfg.packing_format or "").strip().lower() not in _AUTO_ROUND_PACKINGS:
            raise ValueError(f"Unsupported AutoRound packing format: {cfg.packing_format!r}. "
                             f"Expected one of: {sorted(_AUTO_ROUND_PACKINGS)}")
        if int(cfg.bits or 0) != 4:
            raise ValueError("AutoRound support currently requires 4-bit weights.")
        if (cfg.data_type or "").strip().lower() not in {"int", "int4"}:
            raise ValueError(f"Unsupported AutoRound data_type: {cfg.data_type!r}.")
    rules = _Overrides(cfg)
    pending, specs = [], []
    for name, mod in list(model.named_modules()):
        if not isinstance(mod, nn.Linear) or rules.skip(name):
            continue
        if method in _AUTO_ROUND_METHODS and not rules.in_blocks(name):
            continue
        dev = mod.weight.device
        if method in _AUTO_ROUND_METHODS:
            rep = AutoRoundGPTQLinear(mod.in_features, mod.out_features, bits=int(cfg.bits or 4),
                                      group_size=int(cfg.group_size or 128),
                                      sym=True if cfg.sym is None else bool(cfg.sym), bias=mod.bias is not None,
                                      compute_dtype=compute_dtype, device=dev)
        elif method == "awq":
            rep = AWQLinear(mod.in_features, mod.out_features, bits=cfg.bits or 4, group_size=cfg.group_size or 128,
                            zero_point=cfg.zero_point, bias=mod.bias is not None, compute_dtype=compute_dtype,
                            device=dev)
        else:
            raise ValueError(f"Unsupported quantization method: {cfg.quant_method!r}")
        pending.append((name, rep))
        specs.append(QuantizedModuleSpec(module_name=name, quant_method=method))
    for name, rep in pending:
        _set_submodule(model, name, rep)
    return specs

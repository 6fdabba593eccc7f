"""TurboQuant KV-cache rows for ROCm (MI355X): drop-in for src/anna/model/turboquant.py.

Public surface kept from the reference: ``TurboQuantKVRow`` (append / decode_attention /
materialize / clone / to, length properties), ``TurboQuantTensorRow`` (append /
materialize), ``quantize_turboquant_values`` / ``dequantize_turboquant_values``,
``TurboQuantValueState``, ``VALID_KV_CACHE_QUANT_BITS``, ``turboquant_is_available``,
``get_turboquant_quantizer``, and the inner-product keys: ``TurboQuantKeyState``,
``get_turboquant_ip_quantizer``, ``_quantize_turboquant_keys``, ``dequantize_turboquant_keys``,
``turboquant_key_attention_scores``.

Differences by design:
  * The MSE quantizer (rotation + Lloyd-Max codebook + norm) is this build's own
    (`TurboQuantMSE` below, seed 42 like the reference's call sites, turboquant.py:75-92);
    the third-party `turboquant` package the reference imports is not available, so its
    exact codes cannot be reproduced.
  * ``TurboQuantKVRow`` keeps the reference's key state by default (TurboQuantIP indices,
    norms, QJL signs and residual norms, decoded from their reconstruction in the cache dtype,
    turboquant.py:1098-1111) and its values in the reference's min/max format.
    ``key_quantizer="mse"`` is an opt-in fast mode: TQ-MSE key codes + fp16 norms, scored
    against the rotated query directly, so a key costs D/4 bytes instead of 2*D.
  * Every quantize / dequantize / attention step runs in the HIP library; host tensors
    are rejected.
"""

from __future__ import annotations

import os
from typing import NamedTuple

import torch

from . import fused_ops

VALID_KV_CACHE_QUANT_BITS: frozenset[int] = frozenset((2, 3, 4))
_DECODE_BLOCK_SIZE = max(16, int(os.getenv("ANNA_XPU_TURBOQUANT_DECODE_BLOCK_SIZE", "64")))
_MSE_SEED = 42


class TurboQuantValueState(NamedTuple):
    data: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor
    bits: int
    group_size: int


class TurboQuantKeyState(NamedTuple):
    """TurboQuant inner-product key state (reference turboquant.py:27-31): mse_indices uint8
    [H, T, D], norms fp32 [H, T, 1], qjl_signs uint8 0/1 [H, T, D], residual_norms fp32 [H, T, 1]."""

    mse_indices: torch.Tensor
    norms: torch.Tensor
    qjl_signs: torch.Tensor
    residual_norms: torch.Tensor


def turboquant_is_available() -> bool:
    """The quantizers are native to this library, so TurboQuant is available whenever the
    HIP library loads (the reference checks for the optional `turboquant` package)."""
    try:
        from . import _lib

        _lib.load()
    except RuntimeError:
        return False
    return True


def _require_rocm(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{what} runs on the MI355X HIP path only; got a tensor on {t.device}")


def _resolve_value_group_size(head_dim: int) -> int:
    for candidate in (32, 16, 8, 4, 2, 1):
        if candidate <= head_dim and head_dim % candidate == 0:
            return candidate
    return 1


def quantize_turboquant_values(values: torch.Tensor, *, bits: int, group_size: int) -> TurboQuantValueState:
    """Min/max group quantization + packing (reference turboquant.py:199-230), on the GPU."""
    if values.ndim != 3:
        raise ValueError(f"TurboQuant value quantization expects [heads, tokens, dim], got {tuple(values.shape)}")
    if bits not in {2, 3, 4}:
        raise ValueError(f"Unsupported TurboQuant value bit-width: {bits}. Expected 2, 3, or 4.")
    if group_size <= 0 or values.shape[-1] % group_size != 0:
        raise ValueError(f"TurboQuant value group_size={group_size} must evenly divide head_dim={values.shape[-1]}.")
    _require_rocm(values, "TurboQuant value quantization")
    data, scales, zeros = fused_ops.tq_values_quantize(values, bits, group_size)
    return TurboQuantValueState(data=data, scales=scales, zeros=zeros, bits=bits, group_size=group_size)


def dequantize_turboquant_values(state: TurboQuantValueState, *, device=None, dtype=None) -> torch.Tensor:
    """q * scale + zero (reference turboquant.py:233-252), on the GPU."""
    _require_rocm(state.data, "TurboQuant value dequantization")
    out = fused_ops.tq_values_dequant(state.data, state.scales, state.zeros, state.bits, state.group_size,
                                      out_dtype=torch.float32)
    if device is not None or dtype is not None:
        out = out.to(device=device, dtype=dtype)
    return out


class TurboQuantMSE:
    """Rotation + Lloyd-Max codebook + per-vector norm quantizer (this build's definition).

    quantize(x [n, D]) -> (codes uint8 [n, D*sb/8], norms fp16 [n]);
    dequantize(codes, norms) -> [n, D] = norm * R^T c[codes].
    The rotation is the seeded randomized Hadamard H diag(s) / sqrt(D) when D is a power of
    two in [64, 1024] (kind "hadamard": quantized by an in-register fast transform), a seeded
    Haar matrix otherwise (kind "haar": a dense D x D product).  `rotation` is the dense fp32
    form of either.
    """

    def __init__(self, dim: int, bits: int, device, seed: int = _MSE_SEED):
        self.dim = int(dim)
        self.bits = int(bits)
        self.seed = int(seed)
        self.device = torch.device(device)
        d = self.dim
        self.kind = "hadamard" if d in (64, 128, 256, 512, 1024) else "haar"
        rot = fused_ops.tq_rotation(self.dim, self.seed)
        cent, thr = fused_ops.tq_codebook(self.bits, self.dim)
        self.rotation = rot.to(self.device)
        self.rotation_t = rot.t().contiguous().to(self.device)
        self.centroids = cent.to(self.device)
        self.thresholds = thr.to(self.device)
        self.signs = fused_ops.tq_hadamard_signs(d, self.seed).to(self.device) if self.kind == "hadamard" else None

    def quantize(self, x: torch.Tensor):
        _require_rocm(x, "TurboQuant MSE quantization")
        if self.kind == "hadamard":
            return fused_ops.tq_hadamard_quantize(x.reshape(-1, self.dim), self.signs, self.thresholds, self.bits)
        return fused_ops.tq_mse_quantize(x.reshape(-1, self.dim), self.rotation_t, self.thresholds, self.bits)

    def dequantize(self, codes: torch.Tensor, norms: torch.Tensor, dtype=torch.float32) -> torch.Tensor:
        return fused_ops.tq_mse_dequant(codes.reshape(-1, codes.shape[-1]), norms.reshape(-1), self.rotation,
                                        self.centroids, self.bits, out_dtype=dtype)


_quantizers: dict[tuple[int, int, str], TurboQuantMSE] = {}


def get_turboquant_quantizer(*, head_dim: int, bits: int, device) -> TurboQuantMSE:
    key = (int(head_dim), int(bits), str(torch.device(device)))
    q = _quantizers.get(key)
    if q is None:
        q = TurboQuantMSE(head_dim, bits, device)
        _quantizers[key] = q
    return q


class TurboQuantIP:
    """TurboQuant_prod quantizer (this build's definition of the absent package's TurboQuantIP
    that the reference builds at turboquant.py:84-92; Zandieh et al. 2025, Algorithm 2).

    MSE stage with bits - 1 bits (the Hadamard rotation R and Lloyd-Max codebook of
    `TurboQuantMSE`), then the signs of G (x / |x| - R^T c[idx]) rotated (G a seeded D x D
    standard-normal matrix) and the residual norm.  ``S`` = G R is the reference's projection
    matrix, so its score formula (turboquant.py:311-332) holds with these tensors.

    quantize(x [n, D]) -> (mse_indices uint8 [n, D], norms fp32 [n], qjl_signs uint8 [n, D],
    residual_norms fp32 [n]);  dequantize(...) -> [n, D].  D: a power of two in [64, 1024].
    """

    QJL_SEED_SALT = 0x514A4C

    def __init__(self, dim: int, bits: int, device, seed: int = _MSE_SEED):
        if bits not in VALID_KV_CACHE_QUANT_BITS:
            raise ValueError(f"TurboQuantIP bits must be one of {sorted(VALID_KV_CACHE_QUANT_BITS)}, got {bits}")
        if dim not in (64, 128, 256, 512, 1024):
            raise ValueError(f"TurboQuantIP head_dim must be a power of two in [64, 1024], got {dim}")
        self.dim, self.bits, self.seed = int(dim), int(bits), int(seed)
        self.device = torch.device(device)
        cent, thr = fused_ops.tq_codebook(self.bits - 1, self.dim)
        self.centroids = cent.to(self.device)
        self.thresholds = thr.to(self.device)
        signs = fused_ops.tq_hadamard_signs(self.dim, self.seed)
        self.signs = signs.to(self.device)
        g = fused_ops.tq_ip_gaussian(self.dim, self.seed ^ self.QJL_SEED_SALT)
        self.gaussian = g.to(self.device)
        self.gaussian_t = g.t().contiguous().to(self.device)
        rot = fused_ops.tq_rotation(self.dim, self.seed)
        self.S = (g.double() @ rot.double()).float().to(self.device)

    def quantize(self, x: torch.Tensor):
        _require_rocm(x, "TurboQuant key quantization")
        return fused_ops.tq_ip_quantize(x.reshape(-1, self.dim), self.signs, self.thresholds, self.centroids,
                                        self.gaussian_t, self.bits)

    def dequantize(self, mse_indices, norms, qjl_signs, residual_norms, dtype=torch.float32) -> torch.Tensor:
        _require_rocm(mse_indices, "TurboQuant key dequantization")
        out = fused_ops.tq_ip_dequant(mse_indices, norms, qjl_signs, residual_norms, self.signs, self.centroids,
                                      self.gaussian, self.bits, out_dtype=dtype)
        return out.reshape(*mse_indices.shape[:-1], self.dim)


_ip_quantizers: dict[tuple[int, int, str], TurboQuantIP] = {}


def get_turboquant_ip_quantizer(*, head_dim: int, bits: int, device) -> TurboQuantIP:
    key = (int(head_dim), int(bits), str(torch.device(device)))
    q = _ip_quantizers.get(key)
    if q is None:
        q = TurboQuantIP(head_dim, bits, device)
        _ip_quantizers[key] = q
    return q


def _quantize_turboquant_keys(tensor: torch.Tensor, *, bits: int, device) -> TurboQuantKeyState:
    """Keys [heads, tokens, dim] -> TurboQuantKeyState (reference turboquant.py:255-272)."""
    if tensor.ndim != 3:
        raise ValueError(f"TurboQuant key quantization expects [heads, tokens, dim], got {tuple(tensor.shape)}")
    quantizer = get_turboquant_ip_quantizer(head_dim=int(tensor.shape[-1]), bits=bits, device=device)
    h, t, d = tensor.shape
    idx, norms, qjl, rn = quantizer.quantize(tensor.reshape(-1, d))
    return TurboQuantKeyState(mse_indices=idx.reshape(h, t, d), norms=norms.reshape(h, t, 1),
                              qjl_signs=qjl.reshape(h, t, d), residual_norms=rn.reshape(h, t, 1))


def dequantize_turboquant_keys(state: TurboQuantKeyState, *, bits: int, device, dtype=None) -> torch.Tensor:
    """Reconstructed keys [heads, tokens, dim] (reference turboquant.py:275-287)."""
    head_dim = int(state.mse_indices.shape[-1])
    quantizer = get_turboquant_ip_quantizer(head_dim=head_dim, bits=bits, device=device)
    out_dtype = dtype if dtype in (torch.bfloat16, torch.float16, torch.float32) else torch.float32
    keys = quantizer.dequantize(state.mse_indices, state.norms, state.qjl_signs, state.residual_norms,
                                dtype=out_dtype)
    if dtype is not None and keys.dtype != dtype:
        keys = keys.to(dtype=dtype)
    return keys


def turboquant_key_attention_scores(*, query: torch.Tensor, state: TurboQuantKeyState, bits: int, device,
                                    num_key_value_groups: int, scaling: float) -> torch.Tensor:
    """scaling * (q . k_mse + QJL correction), fp32 [kv_heads, groups, query_len, tokens]
    (reference turboquant.py:290-332), from the codes: the query is rotated and projected once
    per row and the keys are never expanded."""
    if query.ndim != 3:
        raise ValueError(f"TurboQuant key attention expects [query_heads, tokens, dim], got {tuple(query.shape)}")
    num_key_value_heads = int(state.mse_indices.shape[0])
    query_heads, _, head_dim = query.shape
    if query_heads % num_key_value_heads != 0:
        raise ValueError(
            f"Query head count {query_heads} is not compatible with TurboQuant KV heads {num_key_value_heads}.")
    if query_heads != num_key_value_heads * num_key_value_groups:
        raise ValueError(f"Expected {num_key_value_heads * num_key_value_groups} query heads, got {query_heads}.")
    if head_dim != int(state.mse_indices.shape[-1]):
        raise ValueError(
            f"TurboQuant key attention head_dim mismatch: expected {state.mse_indices.shape[-1]}, got {head_dim}.")
    _require_rocm(query, "TurboQuant key attention")
    quantizer = get_turboquant_ip_quantizer(head_dim=head_dim, bits=bits, device=device)
    return fused_ops.tq_ip_scores(query, state.mse_indices, state.norms, state.qjl_signs, state.residual_norms,
                                  quantizer.signs, quantizer.centroids, quantizer.gaussian_t, bits, scaling)


def _next_capacity(current: int, required: int) -> int:
    """Geometric growth, min 16 (reference TurboQuantKVRow._next_decode_capacity)."""
    if required <= current:
        return current
    return max(required, max(16, current * 2))


def _storage_bits(bits: int) -> int:
    return 2 if bits == 2 else 4


# ---------------------------------------------------------------- MSE tensor row


class TurboQuantTensorRow:
    """One K or V stream of a sequence (reference turboquant.py:335-477): the newest
    ``residual_len`` tokens stay in the input dtype, older ones are TQ-MSE packed."""

    def __init__(self, *, bits: int, residual_len: int) -> None:
        self.bits = int(bits)
        self.residual_len = max(1, int(residual_len))
        self.device = None
        self.dtype = None
        self.head_dim = None
        self.num_heads = None
        self._codes: torch.Tensor | None = None  # [H, cap, D*sb/8]
        self._norms: torch.Tensor | None = None  # [H, cap] fp16
        self._qlen = 0
        self._residual: torch.Tensor | None = None
        self._length = 0

    @property
    def length(self) -> int:
        return self._length

    @property
    def quantized_length(self) -> int:
        return self._qlen

    @property
    def initialized(self) -> bool:
        return self.device is not None and self.dtype is not None and self.head_dim is not None

    def _quantizer(self) -> TurboQuantMSE:
        return get_turboquant_quantizer(head_dim=self.head_dim, bits=self.bits, device=self.device)

    def _grow(self, required: int) -> None:
        cap = 0 if self._codes is None else self._codes.shape[1]
        if required <= cap:
            return
        new_cap = _next_capacity(cap, required)
        pb = self.head_dim * _storage_bits(self.bits) // 8
        codes = torch.empty((self.num_heads, new_cap, pb), dtype=torch.uint8, device=self.device)
        norms = torch.empty((self.num_heads, new_cap), dtype=torch.float16, device=self.device)
        if self._qlen > 0:
            codes[:, : self._qlen].copy_(self._codes[:, : self._qlen])
            norms[:, : self._qlen].copy_(self._norms[:, : self._qlen])
        self._codes, self._norms = codes, norms

    def append(self, tensor: torch.Tensor) -> None:
        if tensor.ndim != 3:
            raise ValueError(f"TurboQuantTensorRow expects [heads, tokens, dim], got {tuple(tensor.shape)}")
        if tensor.shape[1] <= 0:
            return
        if not self.initialized:
            _require_rocm(tensor, "TurboQuantTensorRow")
            self.device, self.dtype = tensor.device, tensor.dtype
            self.head_dim, self.num_heads = int(tensor.shape[-1]), int(tensor.shape[0])
            self._residual = tensor.detach().contiguous()
            self._length = int(tensor.shape[1])
        else:
            tensor = tensor.to(device=self.device, dtype=self.dtype)
            if int(tensor.shape[-1]) != self.head_dim:
                raise ValueError(f"TurboQuantTensorRow head_dim mismatch: expected {self.head_dim}, "
                                 f"got {int(tensor.shape[-1])}")
            self._residual = torch.cat((self._residual, tensor.detach()), dim=1).contiguous()
            self._length += int(tensor.shape[1])
        overflow = int(self._residual.shape[1] - self.residual_len)
        if overflow <= 0:
            return
        old = self._residual[:, :overflow, :]
        codes, norms = self._quantizer().quantize(old.reshape(-1, self.head_dim))
        self._grow(self._qlen + overflow)
        self._codes[:, self._qlen : self._qlen + overflow].copy_(codes.view(self.num_heads, overflow, -1))
        self._norms[:, self._qlen : self._qlen + overflow].copy_(norms.view(self.num_heads, overflow))
        self._qlen += overflow
        self._residual = self._residual[:, overflow:, :].contiguous()

    def materialize(self, *, device=None, dtype=None) -> torch.Tensor:
        if not self.initialized:
            raise RuntimeError("TurboQuantTensorRow is not initialized.")
        parts = []
        if self._qlen > 0:
            deq = self._quantizer().dequantize(self._codes[:, : self._qlen].reshape(-1, self._codes.shape[-1]),
                                               self._norms[:, : self._qlen].reshape(-1), dtype=self.dtype)
            parts.append(deq.view(self.num_heads, self._qlen, self.head_dim))
        if self._residual is not None and self._residual.numel() > 0:
            parts.append(self._residual)
        out = torch.cat(parts, dim=1) if parts else torch.empty((0, 0, self.head_dim), device=self.device,
                                                                  dtype=self.dtype)
        if device is not None or dtype is not None:
            out = out.to(device=device, dtype=dtype)
        return out

    def clone(self) -> "TurboQuantTensorRow":
        c = TurboQuantTensorRow(bits=self.bits, residual_len=self.residual_len)
        c.device, c.dtype, c.head_dim, c.num_heads = self.device, self.dtype, self.head_dim, self.num_heads
        c._qlen, c._length = self._qlen, self._length
        c._codes = None if self._codes is None else self._codes.clone()
        c._norms = None if self._norms is None else self._norms.clone()
        c._residual = None if self._residual is None else self._residual.clone()
        return c

    def to(self, *, device=None, dtype=None) -> "TurboQuantTensorRow":
        if not self.initialized:
            return self
        if device is not None:
            self._codes = None if self._codes is None else self._codes.to(device)
            self._norms = None if self._norms is None else self._norms.to(device)
            self.device = torch.device(device)
        if self._residual is not None:
            self._residual = self._residual.to(device=device, dtype=dtype)
        if dtype is not None:
            self.dtype = dtype
        return self


# ---------------------------------------------------------------- K/V row


class TurboQuantKVRow:
    """Compressed K/V cache of one sequence (reference turboquant.py:480-1443).

    Keys: by default (``key_quantizer="ip"``, the reference's semantics) the inner-product key
    state (``TurboQuantKeyState``) plus its dense reconstruction in the cache dtype, which decode
    reads as the reference's XPU path does (turboquant.py:1098-1111); ``key_quantizer="mse"``
    (opt-in fast mode) keeps TQ-MSE codes + fp16 norms and scores them from the codes.
    Values: min/max groups (reference format); the newest ``residual_len`` tokens stay dense.
    ``decode_attention`` runs one split-KV launch over [packed prefix ++ residual] with all
    q-heads of a KV head sharing reads.
    """

    def __init__(self, *, bits: int, residual_len: int, value_group_size: int | None = None,
                 key_quantizer: str = "ip") -> None:
        if key_quantizer not in ("mse", "ip"):
            raise ValueError(f"key_quantizer must be 'mse' or 'ip', got {key_quantizer!r}")
        self.key_quantizer = key_quantizer
        self.bits = int(bits)
        self.residual_len = max(1, int(residual_len))
        self.value_group_size = None if value_group_size is None else max(1, int(value_group_size))
        self.device = None
        self.dtype = None
        self.head_dim = None
        self.num_heads = None
        self._kcodes = self._knorms = None
        self._kqjl = self._krn = self._kdense = None  # inner-product keys: signs, residual norms, reconstruction
        self._vdata = self._vscales = self._vzeros = None
        self._qlen = 0
        self._residual_keys: torch.Tensor | None = None
        self._residual_values: torch.Tensor | None = None
        self._length = 0
        self._ws: dict[str, torch.Tensor] = {}

    # ---- properties (reference turboquant.py:510-530)
    @property
    def initialized(self) -> bool:
        return None not in (self.device, self.dtype, self.head_dim, self.num_heads)

    @property
    def length(self) -> int:
        return self._length

    @property
    def quantized_length(self) -> int:
        return self._qlen

    @property
    def residual_length(self) -> int:
        return 0 if self._residual_keys is None else int(self._residual_keys.shape[1])

    @property
    def quantized_capacity(self) -> int:
        return 0 if self._kcodes is None else int(self._kcodes.shape[1])

    def _quantizer(self) -> TurboQuantMSE:
        return get_turboquant_quantizer(head_dim=self.head_dim, bits=self.bits, device=self.device)

    def _grow(self, required: int) -> None:
        cap = self.quantized_capacity
        if required <= cap:
            return
        new_cap = _next_capacity(cap, required)
        h, d = self.num_heads, self.head_dim
        sb = _storage_bits(self.bits)
        g = self.value_group_size
        ip = self.key_quantizer == "ip"
        kc = torch.empty((h, new_cap, d if ip else d * sb // 8), dtype=torch.uint8, device=self.device)
        kn = torch.empty((h, new_cap), dtype=torch.float32 if ip else torch.float16, device=self.device)
        vd = torch.empty((h, new_cap, d * sb // 8), dtype=torch.uint8, device=self.device)
        vs = torch.empty((h, new_cap, d // g), dtype=self.dtype, device=self.device)
        vz = torch.empty((h, new_cap, d // g), dtype=self.dtype, device=self.device)
        if self._qlen > 0:
            n = self._qlen
            for new, old in ((kc, self._kcodes), (kn, self._knorms), (vd, self._vdata), (vs, self._vscales),
                             (vz, self._vzeros)):
                new[:, :n].copy_(old[:, :n])
        self._kcodes, self._knorms, self._vdata, self._vscales, self._vzeros = kc, kn, vd, vs, vz
        if ip:
            kq = torch.empty((h, new_cap, d), dtype=torch.uint8, device=self.device)
            kr = torch.empty((h, new_cap), dtype=torch.float32, device=self.device)
            kd = torch.empty((h, new_cap, d), dtype=self.dtype, device=self.device)
            if self._qlen > 0:
                n = self._qlen
                for new, old in ((kq, self._kqjl), (kr, self._krn), (kd, self._kdense)):
                    new[:, :n].copy_(old[:, :n])
            self._kqjl, self._krn, self._kdense = kq, kr, kd

    def append(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        if key_states.ndim != 3 or value_states.ndim != 3:
            raise ValueError("TurboQuantKVRow expects key/value tensors shaped [heads, tokens, dim].")
        if key_states.shape != value_states.shape:
            raise ValueError(f"TurboQuantKVRow key/value shape mismatch: {tuple(key_states.shape)} vs "
                             f"{tuple(value_states.shape)}")
        if key_states.shape[1] <= 0:
            return
        if not self.initialized:
            _require_rocm(key_states, "TurboQuantKVRow")
            self.device, self.dtype = key_states.device, key_states.dtype
            self.head_dim, self.num_heads = int(key_states.shape[-1]), int(key_states.shape[0])
            self.value_group_size = self.value_group_size or _resolve_value_group_size(self.head_dim)
            self._residual_keys = key_states.detach().contiguous()
            self._residual_values = value_states.detach().contiguous()
            self._length = int(key_states.shape[1])
        else:
            if int(key_states.shape[0]) != self.num_heads or int(key_states.shape[-1]) != self.head_dim:
                raise ValueError(f"TurboQuantKVRow shape mismatch: expected heads={self.num_heads} "
                                 f"head_dim={self.head_dim}, got {tuple(key_states.shape)}")
            key_states = key_states.to(device=self.device, dtype=self.dtype)
            value_states = value_states.to(device=self.device, dtype=self.dtype)
            self._residual_keys = torch.cat((self._residual_keys, key_states.detach()), dim=1).contiguous()
            self._residual_values = torch.cat((self._residual_values, value_states.detach()), dim=1).contiguous()
            self._length += int(key_states.shape[1])
        overflow = int(self._residual_keys.shape[1] - self.residual_len)
        if overflow <= 0:
            return
        ks = self._residual_keys[:, :overflow]
        vs = self._residual_values[:, :overflow]
        vstate = quantize_turboquant_values(vs, bits=self.bits, group_size=self.value_group_size)
        self._grow(self._qlen + overflow)
        s, e, h = self._qlen, self._qlen + overflow, self.num_heads
        if self.key_quantizer == "ip":
            kst = _quantize_turboquant_keys(ks, bits=self.bits, device=self.device)
            self._kcodes[:, s:e].copy_(kst.mse_indices)
            self._knorms[:, s:e].copy_(kst.norms.view(h, overflow))
            self._kqjl[:, s:e].copy_(kst.qjl_signs)
            self._krn[:, s:e].copy_(kst.residual_norms.view(h, overflow))
            self._kdense[:, s:e].copy_(dequantize_turboquant_keys(kst, bits=self.bits, device=self.device,
                                                                  dtype=self.dtype))
        else:
            codes, norms = self._quantizer().quantize(ks.reshape(-1, self.head_dim))
            self._kcodes[:, s:e].copy_(codes.view(h, overflow, -1))
            self._knorms[:, s:e].copy_(norms.view(h, overflow))
        self._vdata[:, s:e].copy_(vstate.data)
        self._vscales[:, s:e].copy_(vstate.scales)
        self._vzeros[:, s:e].copy_(vstate.zeros)
        self._qlen = e
        self._residual_keys = self._residual_keys[:, overflow:].contiguous()
        self._residual_values = self._residual_values[:, overflow:].contiguous()

    def materialize(self, *, device=None, dtype=None):
        if not self.initialized:
            raise RuntimeError("TurboQuantKVRow is not initialized.")
        kp, vp = [], []
        if self._qlen > 0:
            n, h, d = self._qlen, self.num_heads, self.head_dim
            if self.key_quantizer == "ip":
                kp.append(self._kdense[:, :n])
            else:
                k = self._quantizer().dequantize(self._kcodes[:, :n].reshape(h * n, -1),
                                                 self._knorms[:, :n].reshape(-1), dtype=self.dtype)
                kp.append(k.view(h, n, d))
            vp.append(fused_ops.tq_values_dequant(self._vdata[:, :n], self._vscales[:, :n], self._vzeros[:, :n],
                                                  self.bits, self.value_group_size, self.dtype))
        if self.residual_length > 0:
            kp.append(self._residual_keys)
            vp.append(self._residual_values)
        keys = torch.cat(kp, dim=1)
        values = torch.cat(vp, dim=1)
        if device is not None or dtype is not None:
            keys, values = keys.to(device=device, dtype=dtype), values.to(device=device, dtype=dtype)
        return keys, values

    def _workspace(self, name: str, shape, dtype) -> torch.Tensor:
        t = self._ws.get(name)
        if t is None or t.numel() < torch.Size(shape).numel() or t.dtype != dtype or t.device != self.device:
            numel = torch.Size(shape).numel()
            cap = max(numel, 2 * (0 if t is None else t.numel()))
            t = torch.empty(cap, dtype=dtype, device=self.device)
            self._ws[name] = t
        return t[: torch.Size(shape).numel()].view(shape)

    def decode_attention(self, query: torch.Tensor, *, scaling: float, num_key_value_groups: int,
                         gate: torch.Tensor | None = None) -> torch.Tensor:
        if not self.initialized:
            raise RuntimeError("TurboQuantKVRow is not initialized.")
        if query.ndim != 3 or query.shape[1] != 1:
            raise ValueError(f"TurboQuantKVRow single-token decode expects [query_heads, 1, dim], "
                             f"got {tuple(query.shape)}")
        if int(query.shape[-1]) != self.head_dim:
            raise ValueError(f"TurboQuantKVRow decode head_dim mismatch: expected {self.head_dim}, "
                             f"got {int(query.shape[-1])}")
        hq = int(query.shape[0])
        if hq != self.num_heads * int(num_key_value_groups):
            raise ValueError(f"Expected {self.num_heads * num_key_value_groups} query heads, got {hq}.")
        if gate is not None and (gate.ndim != 3 or tuple(gate.shape) != (hq, 1, self.head_dim)):
            raise ValueError(f"TurboQuantKVRow decode gate expects [query_heads, 1, head_dim], got {tuple(gate.shape)}")
        if self._length <= 0:
            return query.new_zeros((hq, 1, self.head_dim))
        q4 = query.unsqueeze(0)
        out = torch.empty_like(q4)
        qn = self._quantizer()
        n, r = self._qlen, self.residual_length
        res_k = self._residual_keys.unsqueeze(0) if r > 0 else None
        res_v = self._residual_values.unsqueeze(0) if r > 0 else None
        if self.key_quantizer == "ip":
            kargs = dict(key=self._kdense[:, :n].unsqueeze(0) if n > 0 else None, key_format=fused_ops.KEYS_DENSE)
        else:
            kargs = dict(key=self._kcodes[:, :n].unsqueeze(0) if n > 0 else None, key_format=fused_ops.KEYS_TQ_MSE,
                         key_norms=self._knorms[:, :n].unsqueeze(0) if n > 0 else None)
        args = fused_ops.decode_args(
            query=q4, len1=n, **kargs, key_bits=self.bits,
            value=self._vdata[:, :n].unsqueeze(0) if n > 0 else None, value_format=fused_ops.VALUES_MINMAX,
            value_scales=self._vscales[:, :n].unsqueeze(0) if n > 0 else None,
            value_zeros=self._vzeros[:, :n].unsqueeze(0) if n > 0 else None,
            value_bits=self.bits, value_group_size=self.value_group_size,
            rotation=qn.rotation, rotation_t=qn.rotation_t, key_centroids=qn.centroids, rotation_signs=qn.signs,
            query_rot=self._workspace("qrot", (hq, self.head_dim), torch.float32),
            residual_key=res_k, residual_value=res_v, scaling=scaling, block_size=_DECODE_BLOCK_SIZE,
            gate=None if gate is None else gate.unsqueeze(0), output=out,
            partial_stats=self._workspace("ps", (1, hq, 1, 2), torch.float32),
            partial_values=self._workspace("pv", (1, hq, 1, self.head_dim), torch.float32),
        )
        nblk = fused_ops.decode_num_blocks(args)
        ps = self._workspace("ps", (1, hq, nblk, 2), torch.float32)
        pv = self._workspace("pv", (1, hq, nblk, self.head_dim), torch.float32)
        from . import _lib

        args.partial_stats = _lib.view(ps)
        args.partial_values = _lib.view(pv)
        args.partial_capacity = nblk
        fused_ops.run_decode(args, query)
        return out.squeeze(0)

    def clone(self) -> "TurboQuantKVRow":
        c = TurboQuantKVRow(bits=self.bits, residual_len=self.residual_len, value_group_size=self.value_group_size,
                            key_quantizer=self.key_quantizer)
        c.device, c.dtype, c.head_dim, c.num_heads = self.device, self.dtype, self.head_dim, self.num_heads
        c._qlen, c._length = self._qlen, self._length
        for name in ("_kcodes", "_knorms", "_kqjl", "_krn", "_kdense", "_vdata", "_vscales", "_vzeros"):
            t = getattr(self, name)
            setattr(c, name, None if t is None else t[:, : self._qlen].clone())
        c._residual_keys = None if self._residual_keys is None else self._residual_keys.clone()
        c._residual_values = None if self._residual_values is None else self._residual_values.clone()
        return c

    def to(self, *, device=None, dtype=None) -> "TurboQuantKVRow":
        if not self.initialized:
            return self
        for name in ("_kcodes", "_knorms", "_kqjl", "_krn", "_vdata"):
            t = getattr(self, name)
            if t is not None and device is not None:
                setattr(self, name, t.to(device))
        for name in ("_kdense", "_vscales", "_vzeros", "_residual_keys", "_residual_values"):
            t = getattr(self, name)
            if t is not None:
                setattr(self, name, t.to(device=device, dtype=dtype))
        if device is not None:
            self.device = torch.device(device)
        if dtype is not None:
            self.dtype = dtype
        self._ws = {}
        return self

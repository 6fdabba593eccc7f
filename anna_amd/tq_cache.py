"""Batched, variable-length TurboQuant KV cache for decode.

One launch appends a token to every sequence and one call (split + merge launches) decodes every sequence: this
replaces the per-row loops of the reference, the append of
Qwen3DynamicCache._update_turboquant_layer (src/anna/model/ops.py:618-661, calling
TurboQuantKVRow.append, turboquant.py:1027-1140) and the decode of
turboquant_single_token_decode_attention (ops.py:1024-1072, calling
TurboQuantKVRow.decode_attention per row, turboquant.py:1181-1346).

Two forms behind one class.  head_dim 256 with 2-bit codes (the BASELINE shape) takes the
MFMA decode of anna_amd/csrc/tq_decode.hip over TQ-MSE keys and values.  Every
other shape (power-of-two head_dim 64..512, key/value bits 2..4) takes TurboQuantRowsCache:
TQ-MSE keys and min/max values (the reference row's value format, turboquant.py:199-230) in one
region per sequence, one append launch, and the split-KV decode with per-row lengths.

Layout of the 2-bit / 256 form (see anna_amd/csrc/tq_decode.hip): per KV head a pool of token slots, sequence b owning
the slots [offsets[b], offsets[b] + capacity[b]) (capacities rounded up to 32 tokens); keys as
token-major codes, values as 32-token blocked codes; the newest `residual_capacity` tokens of
each sequence stay bf16 in a ring (token j at ring slot j % R), so a sequence of length L has
max(0, L - R) quantized tokens, as in the reference's residual window.  Sequence lengths live
on the device: neither append nor decode needs the host, and both can be captured in a HIP
graph.  The host keeps a mirror of the lengths only to refuse an append past a capacity.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from . import fused_ops
from .turboquant import _resolve_value_group_size, get_turboquant_quantizer

_A16 = 1.123046875  # fp16 LUT magnitude that maps to the centroid a of the 2-bit codebook


def _round32(n: int) -> int:
    return (int(n) + 31) // 32 * 32


class TurboQuantBatchCache:
    """capacities[b]: pool slots (quantized tokens) of sequence b; a sequence holds at most
    capacities[b] + residual_capacity tokens.  Shapes other than head_dim 256 with 2-bit codes
    construct a TurboQuantRowsCache (same methods)."""

    def __new__(cls, *args, head_dim: int = 256, bits: int = 2, **kwargs):
        if cls is TurboQuantBatchCache and (head_dim != 256 or bits != 2):
            cls = TurboQuantRowsCache
        return super().__new__(cls)

    def __init__(self, *, batch: int, kv_heads: int, q_heads: int, capacities, residual_capacity: int = 128,
                 head_dim: int = 256, bits: int = 2, device="cuda", tokens_per_item: int = 0):
        if head_dim != 256 or bits != 2:
            raise ValueError("TurboQuantBatchCache supports head_dim 256 with 2-bit codes")
        if q_heads % kv_heads != 0 or q_heads // kv_heads > 16:
            raise ValueError("q_heads must be G * kv_heads with G <= 16")
        if tokens_per_item % 32 != 0 or tokens_per_item < 0:
            raise ValueError("tokens_per_item must be 0 (automatic) or a positive multiple of 32")
        self.batch, self.kv_heads, self.q_heads, self.head_dim, self.bits = batch, kv_heads, q_heads, head_dim, bits
        self.device = torch.device(device)
        self.capacities = [_round32(c) for c in capacities]
        offs, acc = [], 0
        for c in self.capacities:
            offs.append(acc)
            acc += c
        self.pool_tokens = max(32, acc)
        self.offsets = offs
        self.residual_capacity = _round32(max(1, residual_capacity))
        self.tokens_per_item = tokens_per_item
        dev = self.device
        T, R, D = self.pool_tokens, self.residual_capacity, head_dim
        self.key_codes = torch.zeros((kv_heads, T, D // 4), dtype=torch.uint8, device=dev)
        self.key_norms = torch.zeros((kv_heads, T), dtype=torch.float16, device=dev)
        self.value_codes = torch.zeros((kv_heads, T // 32, 32 * D // 4), dtype=torch.uint8, device=dev)
        self.value_norms = torch.zeros((kv_heads, T), dtype=torch.float16, device=dev)
        self.residual_key = torch.zeros((batch, kv_heads, R, D), dtype=torch.bfloat16, device=dev)
        self.residual_value_t = torch.zeros((batch, kv_heads, D, R), dtype=torch.bfloat16, device=dev)
        self.seq_offsets = torch.tensor(offs, dtype=torch.int32, device=dev)
        self.seq_capacity = torch.tensor(self.capacities, dtype=torch.int32, device=dev)
        self.seq_lengths = torch.zeros((batch,), dtype=torch.int32, device=dev)
        self.overflow = torch.zeros((1,), dtype=torch.int32, device=dev)
        self.lengths = [0] * batch  # host mirror
        self.qn = get_turboquant_quantizer(head_dim=D, bits=bits, device=dev)
        if self.qn.kind != "hadamard":
            raise RuntimeError("the batched cache needs the Hadamard rotation (power-of-two head_dim)")
        self.key_scale = float(self.qn.centroids[2].item()) / _A16
        self.value_scale = self.key_scale
        bpi = tokens_per_item // 32
        caps = torch.tensor(self.capacities, dtype=torch.int64)
        self.num_workgroups = int(_lib.load().anna_mi_tq_decode_workgroups(batch, kv_heads, caps.data_ptr(), bpi))
        nwg = self.num_workgroups
        self.partial_stats = torch.empty((nwg, 16, 2), dtype=torch.float32, device=dev)
        self.partial_values = torch.empty((nwg, 16, D), dtype=torch.float32, device=dev)
        self.item_table = torch.zeros((4 * batch * kv_heads,), dtype=torch.int32, device=dev)  # 4 per (b, h): fused step

    # ---- lengths
    @property
    def quantized_lens(self) -> list[int]:
        return [max(0, n - self.residual_capacity) for n in self.lengths]

    @property
    def residual_lens(self) -> list[int]:
        return [min(n, self.residual_capacity) for n in self.lengths]

    # ---- filling (prefill)
    def load_sequence(self, b: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        """keys/values bf16 [Hkv, L, D]: the sequence's whole history.  Its first
        max(0, L - R) tokens are packed into the pool, the newest min(L, R) go to the ring."""
        h, L, D = keys.shape
        R = self.residual_capacity
        q = max(0, L - R)
        if q > self.capacities[b]:
            raise ValueError(f"sequence {b}: {q} quantized tokens exceed its capacity {self.capacities[b]}")
        off = self.offsets[b]
        if q > 0:
            if keys.dtype != torch.bfloat16 or values.dtype != torch.bfloat16:
                raise ValueError("keys/values must be bf16")
            k, v = keys, values
            if k.stride(2) != 1 or v.stride() != k.stride():  # the pack reads both with one set of strides
                k, v = keys.contiguous(), values.contiguous()
            self._pack(k, v, q, off)
        if L > q:
            slots = torch.arange(q, L, device=self.device) % R
            self.residual_key[b][:, slots] = keys[:, q:]
            self.residual_value_t[b][:, :, slots] = values[:, q:].transpose(1, 2)
        self.seq_lengths[b] = L
        self.lengths[b] = L

    def _pack(self, keys: torch.Tensor, values: torch.Tensor, tokens: int, slot_offset: int) -> None:
        """One launch: the first `tokens` tokens of keys/values [Hkv, L, D] into the pool."""
        a = _lib.TQPackArgs()
        a.kv_heads, a.head_dim, a.tokens = keys.shape[0], self.head_dim, tokens
        a.keys, a.values = keys.data_ptr(), values.data_ptr()
        a.stride_head, a.stride_token = keys.stride(0), keys.stride(1)
        a.key_codes, a.key_norms = self.key_codes.data_ptr(), self.key_norms.data_ptr()
        a.value_codes, a.value_norms = self.value_codes.data_ptr(), self.value_norms.data_ptr()
        a.pool_tokens, a.slot_offset = self.pool_tokens, slot_offset
        a.signs, a.thresholds = self.qn.signs.data_ptr(), self.qn.thresholds.data_ptr()
        _lib.call("anna_mi_tq_pack_kv", ctypes.byref(a), _lib.stream_of(keys))

    # ---- decode step
    def _append_args(self, keys: torch.Tensor, values: torch.Tensor) -> _lib.TQAppendArgs:
        """Checks one token per sequence (keys/values bf16 [B, Hkv, D], contiguous) and builds
        the append arguments."""
        B, H, D = self.batch, self.kv_heads, self.head_dim
        if keys.dtype != torch.bfloat16 or tuple(keys.shape) != (B, H, D) or values.shape != keys.shape:
            raise ValueError("append expects bf16 keys/values of shape [batch, kv_heads, 256]")
        _lib.require_device(keys, values)
        R = self.residual_capacity
        for b, n in enumerate(self.lengths):
            if n >= R and n - R >= self.capacities[b]:
                raise RuntimeError(f"sequence {b} is full: {self.capacities[b]} pool slots + {R} window tokens")
        a = _lib.TQAppendArgs()
        a.batch, a.kv_heads, a.head_dim = B, H, D
        a.new_key, a.new_value = keys.data_ptr(), values.data_ptr()
        a.key_codes, a.key_norms = self.key_codes.data_ptr(), self.key_norms.data_ptr()
        a.value_codes, a.value_norms = self.value_codes.data_ptr(), self.value_norms.data_ptr()
        a.pool_tokens = self.pool_tokens
        a.residual_key, a.residual_value_t = self.residual_key.data_ptr(), self.residual_value_t.data_ptr()
        a.residual_capacity = R
        a.seq_offsets, a.seq_capacity = self.seq_offsets.data_ptr(), self.seq_capacity.data_ptr()
        a.seq_lengths, a.overflow = self.seq_lengths.data_ptr(), self.overflow.data_ptr()
        a.signs, a.thresholds = self.qn.signs.data_ptr(), self.qn.thresholds.data_ptr()
        return a

    def append(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """One token per sequence: keys/values bf16 [B, Hkv, D]."""
        keys, values = keys.contiguous(), values.contiguous()
        a = self._append_args(keys, values)
        _lib.call("anna_mi_tq_append", ctypes.byref(a), _lib.stream_of(keys))
        self.lengths = [n + 1 for n in self.lengths]

    def decode_args(self, query: torch.Tensor, out: torch.Tensor, scaling: float,
                    gate: torch.Tensor | None = None) -> _lib.TQDecodeArgs:
        a = _lib.TQDecodeArgs()
        a.batch, a.q_heads, a.kv_heads, a.head_dim = self.batch, self.q_heads, self.kv_heads, self.head_dim
        a.key_bits = a.value_bits = self.bits
        a.query = query.data_ptr()
        a.gate = None if gate is None else gate.data_ptr()
        a.key_codes, a.key_norms = self.key_codes.data_ptr(), self.key_norms.data_ptr()
        a.value_codes, a.value_norms = self.value_codes.data_ptr(), self.value_norms.data_ptr()
        a.pool_tokens = self.pool_tokens
        a.residual_key, a.residual_value_t = self.residual_key.data_ptr(), self.residual_value_t.data_ptr()
        a.residual_capacity = self.residual_capacity
        a.seq_offsets, a.seq_lengths = self.seq_offsets.data_ptr(), self.seq_lengths.data_ptr()
        a.signs = self.qn.signs.data_ptr()
        a.key_scale, a.value_scale, a.scaling = self.key_scale, self.value_scale, float(scaling)
        a.blocks_per_item = self.tokens_per_item // 32
        a.num_workgroups = self.num_workgroups
        a.partial_stats, a.partial_values = self.partial_stats.data_ptr(), self.partial_values.data_ptr()
        a.item_table = self.item_table.data_ptr()
        a.out = out.data_ptr()
        return a

    def _check_query(self, query: torch.Tensor, gate: torch.Tensor | None) -> torch.Tensor:
        shape = (self.batch, self.q_heads, self.head_dim)
        if query.dtype != torch.bfloat16 or tuple(query.shape) != shape:
            raise ValueError("query must be bf16 [batch, q_heads, 256]")
        if gate is not None and (gate.dtype != torch.bfloat16 or tuple(gate.shape) != shape):
            raise ValueError("gate must be bf16 [batch, q_heads, 256] (the query's shape)")
        _lib.require_device(query, gate)
        return query.contiguous()

    def decode(self, query: torch.Tensor, *, scaling: float, out: torch.Tensor | None = None,
               gate: torch.Tensor | None = None) -> torch.Tensor:
        """query bf16 [B, Hq, D] -> attention output bf16 [B, Hq, D]; gate (optional, bf16, same
        shape as query): out *= sigmoid(gate) (the reference's gated decode, sycl:1605-1669)."""
        query = self._check_query(query, gate)
        gate = None if gate is None else gate.contiguous()
        if out is None:
            out = torch.empty_like(query)
        a = self.decode_args(query, out, scaling, gate)
        _lib.call("anna_mi_tq_decode", ctypes.byref(a), _lib.stream_of(query))
        return out

    def append_decode(self, keys: torch.Tensor, values: torch.Tensor, query: torch.Tensor, *, scaling: float,
                      out: torch.Tensor | None = None, gate: torch.Tensor | None = None) -> torch.Tensor:
        """One decode step in the decode's two launches: append(keys, values) then
        decode(query), same results and cache state, without the append's own launch."""
        query = self._check_query(query, gate)
        gate = None if gate is None else gate.contiguous()
        keys, values = keys.contiguous(), values.contiguous()
        ap = self._append_args(keys, values)
        if out is None:
            out = torch.empty_like(query)
        a = self.decode_args(query, out, scaling, gate)
        _lib.call("anna_mi_tq_append_decode", ctypes.byref(a), ctypes.byref(ap), _lib.stream_of(query))
        self.lengths = [n + 1 for n in self.lengths]
        return out

    def bytes_per_decode(self) -> int:
        """Algorithmic HBM bytes of one decode call: codes + norms of every packed token
        (K and V), the dense window, the query and the output."""
        h, d = self.kv_heads, self.head_dim
        packed = sum(self.quantized_lens) * h * 2 * (d // 4 + 2)
        resid = sum(self.residual_lens) * h * 2 * d * 2
        return packed + resid + 2 * self.batch * self.q_heads * d * 2


class TurboQuantRowsCache(TurboQuantBatchCache):
    """The batched cache for any power-of-two head_dim in [64, 512] and bits 2..4 (keys and
    values).  Per (sequence, KV head) a region of `capacity` packed slots -- keys as Hadamard
    TQ-MSE codes + fp16 norm, values as min/max groups of `value_group_size` -- and a bf16 ring of
    the newest `residual_capacity` tokens (token j at slot j % R).  Lengths live on the device.
    append: one launch (anna_mi_tq_rows_append); decode: the split-KV decode with per-row lengths
    (query rotation, split, merge)."""

    def __init__(self, *, batch: int, kv_heads: int, q_heads: int, capacities, residual_capacity: int = 128,
                 head_dim: int = 256, bits: int = 2, device="cuda", tokens_per_item: int = 0,
                 value_group_size: int | None = None, block_size: int = 64):
        if head_dim not in (64, 128, 256, 512):
            raise ValueError("TurboQuantBatchCache needs a power-of-two head_dim in [64, 512] (the split-KV decode's range)")
        if bits not in (2, 3, 4):
            raise ValueError(f"Unsupported TurboQuant KV bit-width: {bits}. Expected 2, 3, or 4.")
        if q_heads % kv_heads != 0 or q_heads // kv_heads > (8 if head_dim >= 512 else 16):
            raise ValueError("q_heads must be G * kv_heads with G <= 16 (8 at head_dim 512+)")
        self.batch, self.kv_heads, self.q_heads, self.head_dim, self.bits = batch, kv_heads, q_heads, head_dim, bits
        self.device = torch.device(device)
        self.capacities = [int(c) for c in capacities]
        self.capacity = max([1] + self.capacities)
        self.residual_capacity = max(1, int(residual_capacity))
        self.value_group_size = int(value_group_size or _resolve_value_group_size(head_dim))
        if head_dim % self.value_group_size != 0:
            raise ValueError("value_group_size must divide head_dim")
        self.block_size = int(block_size)
        dev, B, H, C, R, D = self.device, batch, kv_heads, self.capacity, self.residual_capacity, head_dim
        pb = D * (2 if bits == 2 else 4) // 8
        self.key_codes = torch.zeros((B, H, C, pb), dtype=torch.uint8, device=dev)
        self.key_norms = torch.zeros((B, H, C), dtype=torch.float16, device=dev)
        self.value_data = torch.zeros((B, H, C, pb), dtype=torch.uint8, device=dev)
        self.value_scales = torch.zeros((B, H, C, D // self.value_group_size), dtype=torch.bfloat16, device=dev)
        self.value_zeros = torch.zeros_like(self.value_scales)
        self.residual_key = torch.zeros((B, H, R, D), dtype=torch.bfloat16, device=dev)
        self.residual_value = torch.zeros_like(self.residual_key)
        self.seq_lengths = torch.zeros((B,), dtype=torch.int32, device=dev)
        self.overflow = torch.zeros((1,), dtype=torch.int32, device=dev)
        self.lengths = [0] * B
        self.qn = get_turboquant_quantizer(head_dim=D, bits=bits, device=dev)
        self.query_rot = torch.empty((B, q_heads, D), dtype=torch.float32, device=dev)
        self._partials(1)

    def _partials(self, n: int) -> None:
        self.partial_stats = torch.empty((self.batch, self.q_heads, n, 2), dtype=torch.float32, device=self.device)
        self.partial_values = torch.empty((self.batch, self.q_heads, n, self.head_dim), dtype=torch.float32,
                                          device=self.device)

    def load_sequence(self, b: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        """keys/values bf16 [Hkv, L, D]: the first max(0, L - R) tokens are quantized into the
        sequence's region, the newest min(L, R) go to the ring."""
        h, L, D = keys.shape
        R = self.residual_capacity
        q = max(0, L - R)
        if q > self.capacities[b]:
            raise ValueError(f"sequence {b}: {q} quantized tokens exceed its capacity {self.capacities[b]}")
        if keys.dtype != torch.bfloat16 or values.dtype != torch.bfloat16:
            raise ValueError("keys/values must be bf16")
        if q > 0:
            codes, norms = self.qn.quantize(keys[:, :q].reshape(-1, D))
            self.key_codes[b, :, :q] = codes.view(h, q, -1)
            self.key_norms[b, :, :q] = norms.view(h, q)
            data, sc, zr = fused_ops.tq_values_quantize(values[:, :q], self.bits, self.value_group_size)
            self.value_data[b, :, :q] = data
            self.value_scales[b, :, :q] = sc
            self.value_zeros[b, :, :q] = zr
        if L > q:
            slots = torch.arange(q, L, device=self.device) % R
            self.residual_key[b][:, slots] = keys[:, q:]
            self.residual_value[b][:, slots] = values[:, q:]
        self.seq_lengths[b] = L
        self.lengths[b] = L

    def append(self, keys: torch.Tensor, values: torch.Tensor) -> None:
        """One token per sequence: keys/values bf16 [B, Hkv, D]."""
        B, H, D, R = self.batch, self.kv_heads, self.head_dim, self.residual_capacity
        if keys.dtype != torch.bfloat16 or tuple(keys.shape) != (B, H, D) or values.shape != keys.shape:
            raise ValueError(f"append expects bf16 keys/values of shape [batch, kv_heads, {D}]")
        _lib.require_device(keys, values)
        for b, n in enumerate(self.lengths):
            if n >= R and n - R >= self.capacities[b]:
                raise RuntimeError(f"sequence {b} is full: {self.capacities[b]} packed slots + {R} window tokens")
        keys, values = keys.contiguous(), values.contiguous()
        a = _lib.TQRowsAppendArgs()
        a.dtype = _lib.dtype_code(torch.bfloat16)
        a.batch, a.kv_heads, a.head_dim, a.capacity, a.residual_capacity = B, H, D, self.capacity, R
        a.key_bits = a.value_bits = self.bits
        a.value_group_size = self.value_group_size
        a.new_key, a.new_value = keys.data_ptr(), values.data_ptr()
        a.key_codes, a.key_norms = self.key_codes.data_ptr(), self.key_norms.data_ptr()
        a.value_data, a.value_scales, a.value_zeros = (self.value_data.data_ptr(), self.value_scales.data_ptr(),
                                                       self.value_zeros.data_ptr())
        a.residual_key, a.residual_value = self.residual_key.data_ptr(), self.residual_value.data_ptr()
        a.seq_lengths, a.overflow = self.seq_lengths.data_ptr(), self.overflow.data_ptr()
        a.signs, a.thresholds = self.qn.signs.data_ptr(), self.qn.thresholds.data_ptr()
        _lib.call("anna_mi_tq_rows_append", ctypes.byref(a), _lib.stream_of(keys))
        self.lengths = [n + 1 for n in self.lengths]

    def decode(self, query: torch.Tensor, *, scaling: float, out: torch.Tensor | None = None,
               gate: torch.Tensor | None = None) -> torch.Tensor:
        """query bf16 [B, Hq, D] -> attention output bf16 [B, Hq, D]; gate (optional, same shape):
        out *= sigmoid(gate)."""
        shape = (self.batch, self.q_heads, self.head_dim)
        if query.dtype != torch.bfloat16 or tuple(query.shape) != shape:
            raise ValueError(f"query must be bf16 [batch, q_heads, {self.head_dim}]")
        if gate is not None and (gate.dtype != torch.bfloat16 or tuple(gate.shape) != shape):
            raise ValueError(f"gate must be bf16 [batch, q_heads, {self.head_dim}] (the query's shape)")
        _lib.require_device(query, gate)
        q4 = query.contiguous().unsqueeze(2)
        if out is None:
            out = torch.empty_like(query)
        o4 = out.unsqueeze(2)
        qn = self.qn
        # Blocks sized so that the call is ~1024 workgroups (about four per CU) on the VALU split
        # kernel (other head dims): one per block, KV head and sequence, each writing G partial
        # rows the merge reads back (64-token blocks at 16K tokens made ~4000 workgroups whose
        # partials were as large as the cache).  The MFMA split kernel (head_dim 64, 128, 256)
        # sizes its own ranges (about 2048 waves with TQ-MSE keys at head_dim <= 128, 1024 at 256)
        # within the partial buffer: room for ~2048 blocks keeps the buffer from lengthening them
        # (D = 128, 4-bit: 27.8 -> 26.8 us).
        wg = 2048 if self.head_dim in (64, 128, 256) else 1024
        per_row = max(1, wg // (self.batch * self.kv_heads))
        bs = max(self.block_size, -(-(self.capacity + self.residual_capacity) // per_row))
        bs = -(-bs // 16) * 16
        args = fused_ops.decode_args(
            query=q4, len1=self.capacity, key=self.key_codes, key_format=fused_ops.KEYS_TQ_MSE,
            key_norms=self.key_norms, key_bits=self.bits, value=self.value_data,
            value_format=fused_ops.VALUES_MINMAX, value_scales=self.value_scales, value_zeros=self.value_zeros,
            value_bits=self.bits, value_group_size=self.value_group_size, rotation=qn.rotation,
            rotation_t=qn.rotation_t, key_centroids=qn.centroids, rotation_signs=qn.signs, query_rot=self.query_rot,
            residual_key=self.residual_key, residual_value=self.residual_value, scaling=scaling,
            block_size=bs, gate=None if gate is None else gate.contiguous().unsqueeze(2), output=o4,
            partial_stats=self.partial_stats, partial_values=self.partial_values, seq_lengths=self.seq_lengths)
        nblk = fused_ops.decode_num_blocks(args)
        if nblk > self.partial_stats.size(2):
            self._partials(nblk)
            args.partial_stats = _lib.view(self.partial_stats)
            args.partial_values = _lib.view(self.partial_values)
            args.partial_capacity = nblk
        fused_ops.run_decode(args, query)
        return out

    def append_decode(self, keys: torch.Tensor, values: torch.Tensor, query: torch.Tensor, *, scaling: float,
                      out: torch.Tensor | None = None, gate: torch.Tensor | None = None) -> torch.Tensor:
        """One decode step in the decode's two launches: append(keys, values) then
        decode(query), same results and cache state, without the append's own launch."""
        query = self._check_query(query, gate)
        gate = None if gate is None else gate.contiguous()
        keys, values = keys.contiguous(), values.contiguous()
        ap = self._append_args(keys, values)
        if out is None:
            out = torch.empty_like(query)
        a = self.decode_args(query, out, scaling, gate)
        _lib.call("anna_mi_tq_append_decode", ctypes.byref(a), ctypes.byref(ap), _lib.stream_of(query))
        self.lengths = [n + 1 for n in self.lengths]
        return out

    def bytes_per_decode(self) -> int:
        """Algorithmic HBM bytes of one decode call: codes, norms, scales and zeros of every packed
        token (K and V), the dense window, the query and the output."""
        h, d = self.kv_heads, self.head_dim
        pb = d * (2 if self.bits == 2 else 4) // 8
        packed = sum(self.quantized_lens) * h * (2 * pb + 2 + 2 * 2 * (d // self.value_group_size))
        resid = sum(self.residual_lens) * h * 2 * d * 2
        return packed + resid + 2 * self.batch * self.q_heads * d * 2

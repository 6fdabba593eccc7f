"""Batched, variable-length TurboQuant KV cache for decode (2-bit TQ-MSE keys and values).

One launch sequence decodes every sequence of the batch: this replaces the per-row Python
loop of the reference (Qwen3DynamicCache.turboquant_single_token_decode_attention,
src/anna/model/ops.py:1024-1072, calling TurboQuantKVRow.decode_attention per row).

Pool layout per KV head (see anna_amd/csrc/tq_decode.hip): sequence b owns the slots
[offsets[b], offsets[b] + capacity[b]) (capacities rounded up to 32 tokens); keys are
token-major codes, values 32-token blocked codes; the newest `residual_capacity` tokens
of each sequence stay bf16 (keys token-major, values dim-major).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib, fused_ops
from .turboquant import get_turboquant_quantizer

_A16 = 1.123046875  # fp16 LUT magnitude that maps to the centroid a of the 2-bit codebook


def _round32(n: int) -> int:
    return (int(n) + 31) // 32 * 32


class TurboQuantBatchCache:
    def __init__(self, *, batch: int, kv_heads: int, q_heads: int, capacities, residual_capacity: int = 128,
                 head_dim: int = 256, bits: int = 2, device="cuda", tokens_per_item: int = 0):
        if head_dim != 256 or bits != 2:
            raise ValueError("TurboQuantBatchCache supports head_dim 256 with 2-bit codes")
        self.batch, self.kv_heads, self.q_heads, self.head_dim, self.bits = batch, kv_heads, q_heads, head_dim, bits
        self.device = torch.device(device)
        self.capacities = [_round32(c) for c in capacities]
        offs, acc = [], 0
        for c in self.capacities:
            offs.append(acc)
            acc += c
        self.pool_tokens = max(32, acc)
        self.offsets = offs
        self.residual_capacity = _round32(residual_capacity)
        self.tokens_per_item = tokens_per_item
        dev = self.device
        T, R, D = self.pool_tokens, self.residual_capacity, head_dim
        self.key_codes = torch.zeros((kv_heads, T, D // 4), dtype=torch.uint8, device=dev)
        self.key_norms = torch.zeros((kv_heads, T), dtype=torch.float16, device=dev)
        self.value_codes = torch.zeros((kv_heads, T // 32, 32 * D // 4), dtype=torch.uint8, device=dev)
        self.value_norms = torch.zeros((kv_heads, T), dtype=torch.float16, device=dev)
        self.residual_key = torch.zeros((batch, kv_heads, R, D), dtype=torch.bfloat16, device=dev)
        self.residual_value_t = torch.zeros((batch, kv_heads, D, R), dtype=torch.bfloat16, device=dev)
        self.quantized_lens = [0] * batch
        self.residual_lens = [0] * batch
        self.qn = get_turboquant_quantizer(head_dim=D, bits=bits, device=dev)
        self.rotation_f16 = self.qn.rotation.to(torch.float16)
        self.rotation_t_f16 = self.qn.rotation_t.to(torch.float16)
        self.key_scale = float(self.qn.centroids[2].item()) / _A16
        self.value_scale = self.key_scale
        self._plan = None

    # ---- filling
    def load_sequence(self, b: int, keys: torch.Tensor, values: torch.Tensor, residual: int) -> None:
        """keys/values [Hkv, L, D] (bf16): the first L - residual tokens are packed, the last
        `residual` tokens stay dense."""
        h, L, D = keys.shape
        q = L - residual
        if q > self.capacities[b] or residual > self.residual_capacity:
            raise ValueError("sequence does not fit its capacity")
        off = self.offsets[b]
        if q > 0:
            kc, kn = self.qn.quantize(keys[:, :q].reshape(-1, D))
            vc, vn = self.qn.quantize(values[:, :q].reshape(-1, D))
            self.key_codes[:, off: off + q].copy_(kc.view(h, q, -1))
            self.key_norms[:, off: off + q].copy_(kn.view(h, q))
            self.value_norms[:, off: off + q].copy_(vn.view(h, q))
            qp = _round32(q)
            nat = torch.zeros((h, qp, D // 4), dtype=torch.uint8, device=self.device)
            nat[:, :q].copy_(vc.view(h, q, -1))
            for hh in range(h):
                blk = self.value_codes[hh, off // 32: (off + qp) // 32]
                _lib.call("anna_mi_tq_block_values", nat[hh].data_ptr(), qp, blk.data_ptr(), _lib.stream_of(nat))
        if residual > 0:
            self.residual_key[b, :, :residual].copy_(keys[:, q:])
            self.residual_value_t[b, :, :, :residual].copy_(values[:, q:].transpose(1, 2))
        self.quantized_lens[b] = q
        self.residual_lens[b] = residual
        self._plan = None

    # ---- decode
    def _make_plan(self):
        B, H = self.batch, self.kv_heads
        if self.tokens_per_item > 0:
            cap = sum(-(-q // self.tokens_per_item) for q in self.quantized_lens) * H + B * H + 1
        else:
            cap = max(256, B * H) + B * H + 1
        items = torch.empty((cap, 4), dtype=torch.int32)
        ranges = torch.empty((B * H, 4), dtype=torch.int32)
        ql = torch.tensor(self.quantized_lens, dtype=torch.int64)
        rl = torch.tensor(self.residual_lens, dtype=torch.int64)
        so = torch.tensor(self.offsets, dtype=torch.int64)
        n = ctypes.c_int64(0)
        _lib.call("anna_mi_tq_decode_plan", B, H, ql.data_ptr(), rl.data_ptr(), so.data_ptr(), self.tokens_per_item,
                  items.data_ptr(), cap, ranges.data_ptr(), ctypes.addressof(n))
        n = n.value
        dev = self.device
        self._plan = dict(
            items=items[:n].to(dev), ranges=ranges.to(dev), n=n,
            ps=torch.empty((max(n, 1), 16, 2), dtype=torch.float32, device=dev),
            pv=torch.empty((max(n, 1), 16, self.head_dim), dtype=torch.float32, device=dev),
            qf=torch.empty((B, H, 4096), dtype=torch.float16, device=dev),
        )
        return self._plan

    def decode_args(self, query: torch.Tensor, out: torch.Tensor, scaling: float) -> _lib.TQDecodeArgs:
        p = self._plan or self._make_plan()
        a = _lib.TQDecodeArgs()
        a.batch, a.q_heads, a.kv_heads, a.head_dim = self.batch, self.q_heads, self.kv_heads, self.head_dim
        a.key_bits = a.value_bits = self.bits
        a.query = query.data_ptr()
        a.key_codes, a.key_norms = self.key_codes.data_ptr(), self.key_norms.data_ptr()
        a.value_codes, a.value_norms = self.value_codes.data_ptr(), self.value_norms.data_ptr()
        a.pool_tokens = self.pool_tokens
        a.residual_key, a.residual_value_t = self.residual_key.data_ptr(), self.residual_value_t.data_ptr()
        a.residual_capacity = self.residual_capacity
        a.rotation_f16, a.rotation_t_f16 = self.rotation_f16.data_ptr(), self.rotation_t_f16.data_ptr()
        a.key_scale, a.value_scale, a.scaling = self.key_scale, self.value_scale, float(scaling)
        a.items, a.num_items, a.bh_items = p["items"].data_ptr(), p["n"], p["ranges"].data_ptr()
        a.query_frag = p["qf"].data_ptr()
        a.partial_stats, a.partial_values = p["ps"].data_ptr(), p["pv"].data_ptr()
        a.out = out.data_ptr()
        return a

    def decode(self, query: torch.Tensor, *, scaling: float, out: torch.Tensor | None = None) -> torch.Tensor:
        """query bf16 [B, Hq, D] -> attention output bf16 [B, Hq, D]."""
        if query.dtype != torch.bfloat16 or tuple(query.shape) != (self.batch, self.q_heads, self.head_dim):
            raise ValueError("query must be bf16 [batch, q_heads, 256]")
        _lib.require_device(query)
        query = query.contiguous()
        if out is None:
            out = torch.empty_like(query)
        a = self.decode_args(query, out, scaling)
        _lib.call("anna_mi_tq_decode", ctypes.byref(a), _lib.stream_of(query))
        return out

    def bytes_per_decode(self) -> int:
        """Algorithmic HBM bytes of one decode call: codes + norms of every packed token
        (K and V), the dense residual window, the query and the output."""
        h, d = self.kv_heads, self.head_dim
        packed = sum(self.quantized_lens) * h * 2 * (d // 4 + 2)
        resid = sum(self.residual_lens) * h * 2 * d * 2
        return packed + resid + 2 * self.batch * self.q_heads * d * 2

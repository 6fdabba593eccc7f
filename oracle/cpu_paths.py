"""Torch restatements of the reference's CPU execution paths -- TEST INFRASTRUCTURE ONLY.

Used only by bench.py's cpu_baseline leg (timed on the host cores) and by tests as a
second checker.  Each function follows the reference code it cites op for op, so the
timing reflects what the reference does on a CPU.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def int4_dequant_f32(qweight: torch.Tensor, qscale: torch.Tensor, qzeros: torch.Tensor, group_size: int,
                     in_features: int) -> torch.Tensor:
    """(q - z) * s in fp32 (quantization.py:626-635), [N, in_features]."""
    n, pc = qweight.shape
    kp = pc * 8
    shifts = torch.arange(0, 32, 4, dtype=torch.int32).view(1, 1, 8)
    unpacked = (torch.bitwise_right_shift(qweight.unsqueeze(-1), shifts) & 0xF).reshape(n, kp).to(torch.float32)
    s = qscale.to(torch.float32).t().contiguous()
    z = qzeros.to(torch.float32).t().contiguous()
    groups = unpacked.reshape(n, kp // group_size, group_size)
    return ((groups - z.unsqueeze(-1)) * s.unsqueeze(-1)).reshape(n, kp)[:, :in_features]


def int4_forward_dequant(x_bf16: torch.Tensor, qweight: torch.Tensor, qscale: torch.Tensor, qzeros: torch.Tensor,
                         group_size: int, in_features: int) -> torch.Tensor:
    """XPUInt4Linear._dequantize_weight + _forward_dequant (quantization.py:626-648):
    unpack all nibbles, (q - z) * s in fp32, cast to bf16, F.linear."""
    w = int4_dequant_f32(qweight, qscale, qzeros, group_size, in_features)
    return F.linear(x_bf16, w.to(torch.bfloat16))


def tq_decode_rows(query: torch.Tensor, keys: list, values: list, scaling: float) -> torch.Tensor:
    """CPU branch of TurboQuantKVRow.decode_attention per row (turboquant.py:1295-1346), as
    called row by row by Qwen3DynamicCache.turboquant_single_token_decode_attention
    (ops.py:1055-1071): bf16 matmul against the (kept, already dequantized) bf16 keys,
    fp32 softmax, bf16 matmul against the values.  query [B, Hq, D]; keys/values per row
    [Hkv, L, D] bf16."""
    outs = []
    for b in range(query.shape[0]):
        k, v = keys[b], values[b]
        hkv, _, d = k.shape
        g = query.shape[1] // hkv
        q = query[b].reshape(hkv, g, 1, d)
        s = torch.matmul(q, k.unsqueeze(1).transpose(-1, -2)) * scaling
        p = torch.softmax(s.to(torch.float32), dim=-1).to(torch.bfloat16)
        outs.append(torch.matmul(p, v.unsqueeze(1)).reshape(hkv * g, d))
    return torch.stack(outs)


def tq_mse_quantize(flat: torch.Tensor, rotation: torch.Tensor, centroids: torch.Tensor):
    """The published TurboQuant-MSE quantizer the reference calls through the third-party
    `TurboQuantMSE.quantize` (turboquant.py:75-82 builds it, TurboQuantTensorRow.append
    turboquant.py:398-405 calls it on the tokens leaving the window): per vector the norm, the
    unit vector rotated by the dense D x D orthogonal matrix (y = u R^T, fp32), and per
    coordinate the index of the nearest codebook centroid.  flat [n, D] -> (int64 indices
    [n, D], norms [n, 1] in flat's dtype)."""
    x = flat.to(torch.float32)
    norms = x.norm(dim=-1, keepdim=True)
    y = (x / norms.clamp_min(1e-12)) @ rotation.t()
    idx = torch.argmin((y.unsqueeze(-1) - centroids).abs(), dim=-1)
    return idx, norms.to(flat.dtype)


def tq_tensor_row_append(tensor: torch.Tensor, residual_len: int, rotation: torch.Tensor,
                         centroids: torch.Tensor):
    """TurboQuantTensorRow.append of a whole [H, T, D] prefill into an empty row
    (turboquant.py:353-405): the oldest T - residual_len tokens are quantized, the newest
    residual_len stay as they are."""
    h, t, d = tensor.shape
    over = max(0, t - residual_len)
    idx, norms = tq_mse_quantize(tensor[:, :over].reshape(-1, d), rotation, centroids)
    return idx.reshape(h, over, d), norms.reshape(h, over, 1), tensor[:, over:].contiguous()


# ---------------------------------------------------------------- MoE (ops.py:3280-3376)


def moe_route(router_logits: torch.Tensor, top_k: int, normalize_topk_prob: bool):
    """_route_tokens CPU branch (ops.py:3290-3297)."""
    w = torch.softmax(router_logits, dim=-1, dtype=torch.float32)
    w, sel = torch.topk(w, top_k, dim=-1)
    if normalize_topk_prob:
        w = w / w.sum(dim=-1, keepdim=True)
    usage = torch.bincount(sel.reshape(-1), minlength=router_logits.shape[-1])
    return w, sel, usage


def moe_sorted_assignments(selected: torch.Tensor, usage: torch.Tensor, num_experts: int):
    """_sorted_routing_assignments (ops.py:3301-3323)."""
    t, k = selected.shape
    flat = selected.reshape(-1)
    tok = torch.arange(t, dtype=torch.long).repeat_interleave(k)
    rte = torch.arange(k, dtype=torch.long).repeat(t)
    order = torch.argsort(flat.to(torch.long) * (t * k) + tok * k + rte)
    offsets = torch.zeros(num_experts + 1, dtype=torch.long)
    offsets[1:] = usage.to(torch.long).cumsum(0)
    return tok.index_select(0, order), rte.index_select(0, order), offsets


def moe_grouped_mlp(compact_hidden: torch.Tensor, compact_weights: torch.Tensor, offsets: torch.Tensor,
                    experts: dict, out_dtype: torch.dtype) -> torch.Tensor:
    """Per-expert SwiGLU MLP times the routing weight, fp64 (the brute-force loop the grouped
    kernel sycl:4078-4324 computes); experts[e] = (Wg, Wu, Wd) dequantized fp32."""
    out = torch.zeros(compact_hidden.shape, dtype=torch.float64)
    x = compact_hidden.to(torch.float64)
    for e, (wg, wu, wd) in experts.items():
        s, t = int(offsets[e]), int(offsets[e + 1])
        if t <= s:
            continue
        g = x[s:t] @ wg.to(torch.float64).t()
        u = x[s:t] @ wu.to(torch.float64).t()
        act = g / (1.0 + torch.exp(-g)) * u
        out[s:t] = (act @ wd.to(torch.float64).t()) * compact_weights[s:t].to(torch.float64)
    return out.to(out_dtype)


def moe_scatter(compact_outputs: torch.Tensor, sorted_token_idx: torch.Tensor, num_tokens: int) -> torch.Tensor:
    """fp32 accumulation of the compact rows per token, then the hidden dtype (sycl:3967-4037)."""
    acc = torch.zeros((num_tokens, compact_outputs.shape[1]), dtype=torch.float32)
    acc.index_add_(0, sorted_token_idx, compact_outputs.to(torch.float32))
    return acc.to(compact_outputs.dtype)

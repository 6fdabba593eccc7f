"""Torch restatements of the reference's CPU execution paths -- TEST INFRASTRUCTURE ONLY.

Used only by bench.py's cpu_baseline leg (timed on the host cores) and by tests as a
second checker.  Each function follows the reference code it cites op for op, so the
timing reflects what the reference does on a CPU.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def int4_forward_dequant(x_bf16: torch.Tensor, qweight: torch.Tensor, qscale: torch.Tensor, qzeros: torch.Tensor,
                         group_size: int, in_features: int) -> torch.Tensor:
    """XPUInt4Linear._dequantize_weight + _forward_dequant (quantization.py:626-648):
    unpack all nibbles, (q - z) * s in fp32, cast to bf16, F.linear."""
    n, pc = qweight.shape
    kp = pc * 8
    shifts = torch.arange(0, 32, 4, dtype=torch.int32).view(1, 1, 8)
    unpacked = (torch.bitwise_right_shift(qweight.unsqueeze(-1), shifts) & 0xF).reshape(n, kp).to(torch.float32)
    s = qscale.to(torch.float32).t().contiguous()
    z = qzeros.to(torch.float32).t().contiguous()
    groups = unpacked.reshape(n, kp // group_size, group_size)
    w = ((groups - z.unsqueeze(-1)) * s.unsqueeze(-1)).reshape(n, kp)[:, :in_features]
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

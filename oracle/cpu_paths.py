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

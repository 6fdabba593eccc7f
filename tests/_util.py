"""Shared helpers of the test suite: tolerance metric and seeded synthetic inputs."""

from __future__ import annotations

import numpy as np

# Float outputs: normwise max relative error against the oracle's reference
# dequant+matmul must stay at or below this (bf16 output rounding is ~4e-3).
BF16_TOL = 1e-2


def rel_err(actual, expected) -> float:
    """max|a - e| / max|e| -- the tolerance metric used for every float output."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    denom = max(float(np.abs(e).max()), 1e-30)
    return float(np.abs(a - e).max()) / denom


def int4_payload(rng: np.random.Generator, n: int, kp: int, group: int, *, scale_dtype: str = "bf16"):
    """Synthetic int4 weight with the distributions of the benchmark configs:
    codes U{0..15}, scales |N(0, 0.02)| + 1e-3, asymmetric zero points U{0..15}."""
    codes = rng.integers(0, 16, size=(n, kp), dtype=np.int64)
    words = (codes.reshape(n, kp // 8, 8) << (4 * np.arange(8))).sum(-1)
    qweight = np.where(words >= 2**31, words - 2**32, words).astype(np.int32)
    g = kp // group
    scales = (np.abs(rng.normal(0.0, 0.02, size=(g, n))) + 1e-3).astype(np.float32)
    if scale_dtype == "bf16":
        from oracle import oracle as orc

        scales = orc.bf16_to_f32(orc.bf16_bits(scales))
    zeros = rng.integers(0, 16, size=(g, n)).astype(np.int8)
    return qweight, scales, zeros


def oracle_tq_quantize(qn, x_bits, dtype):
    """The oracle quantizer matching a TurboQuantMSE's rotation kind (codes, fp16 norm bits)."""
    from oracle import oracle as orc

    x = np.ascontiguousarray(x_bits)
    thr = qn.thresholds.cpu().numpy()
    if qn.kind == "hadamard":
        return orc.tq_hadamard_quantize(x, dtype, qn.signs.cpu().numpy(), thr, qn.bits)
    return orc.tq_mse_quantize(x, dtype, qn.rotation.cpu().numpy(), thr, qn.bits)

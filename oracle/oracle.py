"""Python face of the CPU oracle (anna_oracle.c) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker.  The product (anna_amd/) never does.

Functions take and return numpy arrays.  16-bit floats travel as uint16 bit
patterns (``bf16_bits`` / ``f16_bits``) so that no rounding happens outside the C
code.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB = ORACLE_DIR / "liboracle.so"

BF16, F16, F32 = 0, 1, 2
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        sig = {
            "orc_int4_quantize": [_P, _I64, _I64, _I64, _I64, _I, _P, _P, _P],
            "orc_autoround_to_int4": [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P],
            "orc_int4_dequant": [_P, _P, _I, _P, _I64, _I64, _I64, _I64, _P],
            "orc_int4_linear": [_P, _P, _P, _I, _P, _I64, _I64, _I64, _I64, _I64, _P],
            "orc_tq_values_quantize": [_P, _I, _I64, _I64, _I64, _I, _I64, _P, _P, _P],
            "orc_tq_values_dequant": [_P, _P, _P, _I, _I64, _I64, _I64, _I, _I64, _P],
            "orc_lloyd_max_gaussian": [_I, _P],
            "orc_tq_mse_quantize": [_P, _I, _I64, _I64, _P, _P, _I, _P, _P],
            "orc_tq_mse_dequant": [_P, _P, _I64, _I64, _P, _P, _I, _P],
            "orc_tq_hadamard_signs": [_I64, ctypes.c_uint64, _P],
            "orc_tq_hadamard_rotate": [_P, _P, _I64, _P],
            "orc_tq_hadamard_quantize": [_P, _I, _I64, _I64, _P, _P, _I, _P, _P],
            "orc_tq_ip_quantize": [_P, _I, _I64, _I64, _P, _P, _P, _I, _P, _P, _P, _P, _P],
            "orc_tq_ip_dequant": [_P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P],
            "orc_tq_ip_gaussian": [_I64, ctypes.c_uint64, _P],
        }
        for name, argtypes in sig.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = None
        L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- 16-bit float bit patterns


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_to_f32(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def to_f32(bits: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == BF16:
        return bf16_to_f32(bits)
    if dtype == F16:
        return f16_to_f32(bits)
    return np.asarray(bits, dtype=np.float32)


# ---------------------------------------------------------------- int4 linear (a1-a3)


def int4_quantize(w: np.ndarray, group: int, kp: int, rounding: int = 0):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    g = kp // group
    qw = np.zeros((n, kp // 8), np.int32)
    qs = np.zeros((g, n), np.float32)
    qz = np.zeros((g, n), np.int8)
    lib().orc_int4_quantize(_p(w), n, k, group, kp, rounding, _p(qw), _p(qs), _p(qz))
    return qw, qs, qz


def autoround_to_int4(gq: np.ndarray, gz: np.ndarray, scales_f16_bits: np.ndarray, k: int, n: int, group: int, kp: int):
    gq = np.ascontiguousarray(gq, np.int32)
    gz = np.ascontiguousarray(gz, np.int32)
    sc = np.ascontiguousarray(scales_f16_bits, np.uint16)
    g = sc.shape[0]
    qw = np.zeros((n, kp // 8), np.int32)
    qs = np.zeros((g, n), np.float32)
    qz = np.zeros((g, n), np.int8)
    lib().orc_autoround_to_int4(_p(gq), _p(gz), _p(sc), k, n, group, g, kp, _p(qw), _p(qs), _p(qz))
    return qw, qs, qz


def int4_dequant(qw, qs, qz, k: int, group: int, scale_dtype: int = F32) -> np.ndarray:
    qw = np.ascontiguousarray(qw, np.int32)
    qs = np.ascontiguousarray(qs)
    qz = np.ascontiguousarray(qz, np.int8)
    n, pc = qw.shape
    out = np.zeros((n, k), np.float32)
    lib().orc_int4_dequant(_p(qw), _p(qs), scale_dtype, _p(qz), n, k, pc * 8, group, _p(out))
    return out


def int4_linear(x_bf16_bits: np.ndarray, qw, qs, qz, group: int, scale_dtype: int = F32) -> np.ndarray:
    """Reference CPU path: x_bf16 @ bf16(dequant(W))^T, fp64 accumulation, fp32 result."""
    x = np.ascontiguousarray(x_bf16_bits, np.uint16)
    qw = np.ascontiguousarray(qw, np.int32)
    qs = np.ascontiguousarray(qs)
    qz = np.ascontiguousarray(qz, np.int8)
    m, k = x.shape
    n, pc = qw.shape
    y = np.zeros((m, n), np.float32)
    lib().orc_int4_linear(_p(x), _p(qw), _p(qs), scale_dtype, _p(qz), m, n, k, pc * 8, group, _p(y))
    return y


# ---------------------------------------------------------------- TurboQuant values (a9)


def _storage_bits(bits: int) -> int:
    return 2 if bits == 2 else 4


def tq_values_quantize(values_bits: np.ndarray, dtype: int, bits: int, group: int):
    """values [H, T, D] (16-bit patterns, or fp32 for dtype F32) -> (data, scales, zeros)."""
    v = np.ascontiguousarray(values_bits)
    h, t, d = v.shape
    packed = d * _storage_bits(bits) // 8
    data = np.zeros((h, t, packed), np.uint8)
    sdt = np.float32 if dtype == F32 else np.uint16
    scales = np.zeros((h, t, d // group), sdt)
    zeros = np.zeros((h, t, d // group), sdt)
    lib().orc_tq_values_quantize(_p(v), dtype, h, t, d, bits, group, _p(data), _p(scales), _p(zeros))
    return data, scales, zeros


def tq_values_dequant(data, scales, zeros, dtype: int, bits: int, group: int) -> np.ndarray:
    data = np.ascontiguousarray(data, np.uint8)
    scales = np.ascontiguousarray(scales)
    zeros = np.ascontiguousarray(zeros)
    h, t, _ = data.shape
    d = scales.shape[-1] * group
    out = np.zeros((h, t, d), np.float32)
    lib().orc_tq_values_dequant(_p(data), _p(scales), _p(zeros), dtype, h, t, d, bits, group, _p(out))
    return out


# ---------------------------------------------------------------- TurboQuant-MSE (a10/a11)


def lloyd_max_gaussian(bits: int) -> np.ndarray:
    out = np.zeros(1 << bits, np.float64)
    lib().orc_lloyd_max_gaussian(bits, _p(out))
    return out


def tq_mse_quantize(x_bits: np.ndarray, dtype: int, rotation: np.ndarray, thresholds: np.ndarray, bits: int):
    """x [nvec, D] -> (codes uint8 [nvec, D*sb/8], norms fp16 bits [nvec])."""
    x = np.ascontiguousarray(x_bits)
    nvec, d = x.shape
    P = np.ascontiguousarray(rotation, np.float32)
    thr = np.ascontiguousarray(thresholds, np.float32)
    codes = np.zeros((nvec, d * _storage_bits(bits) // 8), np.uint8)
    norms = np.zeros((nvec,), np.uint16)
    lib().orc_tq_mse_quantize(_p(x), dtype, nvec, d, _p(P), _p(thr), bits, _p(codes), _p(norms))
    return codes, norms


def tq_mse_dequant(codes, norms_f16_bits, rotation, centroids, bits: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.uint8)
    norms = np.ascontiguousarray(norms_f16_bits, np.uint16)
    P = np.ascontiguousarray(rotation, np.float32)
    c = np.ascontiguousarray(centroids, np.float32)
    nvec = codes.shape[0]
    d = P.shape[0]
    out = np.zeros((nvec, d), np.float32)
    lib().orc_tq_mse_dequant(_p(codes), _p(norms), nvec, d, _p(P), _p(c), bits, _p(out))
    return out


def tq_hadamard_signs(d: int, seed: int = 42) -> np.ndarray:
    out = np.zeros(d, np.float32)
    lib().orc_tq_hadamard_signs(d, seed, _p(out))
    return out


def tq_hadamard_rotate(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """y = fl(1/sqrt(D)) * FWHT(s * x) in the fixed fp32 order (one vector)."""
    x = np.ascontiguousarray(x, np.float32)
    s = np.ascontiguousarray(signs, np.float32)
    y = np.zeros_like(x)
    lib().orc_tq_hadamard_rotate(_p(x), _p(s), x.shape[0], _p(y))
    return y


def tq_hadamard_matrix(signs: np.ndarray) -> np.ndarray:
    """The dense fp64 matrix H diag(s) / sqrt(D) (numpy, Sylvester construction)."""
    d = signs.shape[0]
    h = np.array([[1.0]])
    while h.shape[0] < d:
        h = np.block([[h, h], [h, -h]])
    return h * signs.astype(np.float64)[None, :] / np.sqrt(d)


def tq_hadamard_quantize(x_bits: np.ndarray, dtype: int, signs: np.ndarray, thresholds: np.ndarray, bits: int):
    """x [nvec, D] -> (codes, fp16 norm bits) with the Hadamard rotation."""
    x = np.ascontiguousarray(x_bits)
    nvec, d = x.shape
    s = np.ascontiguousarray(signs, np.float32)
    thr = np.ascontiguousarray(thresholds, np.float32)
    codes = np.zeros((nvec, d * _storage_bits(bits) // 8), np.uint8)
    norms = np.zeros((nvec,), np.uint16)
    lib().orc_tq_hadamard_quantize(_p(x), dtype, nvec, d, _p(s), _p(thr), bits, _p(codes), _p(norms))
    return codes, norms


# ---------------------------------------------------------------- TurboQuant inner-product keys (a10)
# This build's TurboQuantIP (the package the reference calls at turboquant.py:84-92, 255-332 is
# absent): PARITY UNPINNED against the reference; pinned by tests/test_oracle_tq_ip.py.


def tq_ip_gaussian(d: int, seed: int) -> np.ndarray:
    out = np.zeros((d, d), np.float32)
    lib().orc_tq_ip_gaussian(d, seed, _p(out))
    return out


def tq_ip_quantize(x_bits: np.ndarray, dtype: int, signs, thresholds, centroids, gaussian, bits: int):
    """x [nvec, D] -> (mse_indices uint8 [nvec, D], norms f32, qjl uint8 [nvec, D], residual norms f32)."""
    x = np.ascontiguousarray(x_bits)
    nvec, d = x.shape
    s = np.ascontiguousarray(signs, np.float32)
    thr = np.ascontiguousarray(thresholds, np.float32)
    c = np.ascontiguousarray(centroids, np.float32)
    g = np.ascontiguousarray(gaussian, np.float32)
    idx = np.zeros((nvec, d), np.uint8)
    qjl = np.zeros((nvec, d), np.uint8)
    norms = np.zeros(nvec, np.float32)
    rn = np.zeros(nvec, np.float32)
    lib().orc_tq_ip_quantize(_p(x), dtype, nvec, d, _p(s), _p(thr), _p(c), bits, _p(g), _p(idx), _p(qjl),
                             _p(norms), _p(rn))
    return idx, norms, qjl, rn


def tq_ip_dequant(idx, norms, qjl, rn, signs, centroids, gaussian) -> np.ndarray:
    idx = np.ascontiguousarray(idx, np.uint8)
    nvec, d = idx.shape
    qjl = np.ascontiguousarray(qjl, np.uint8)
    norms = np.ascontiguousarray(norms, np.float32).reshape(-1)
    rn = np.ascontiguousarray(rn, np.float32).reshape(-1)
    out = np.zeros((nvec, d), np.float32)
    lib().orc_tq_ip_dequant(_p(idx), _p(qjl), _p(norms), _p(rn), nvec, d,
                            _p(np.ascontiguousarray(signs, np.float32)),
                            _p(np.ascontiguousarray(centroids, np.float32)),
                            _p(np.ascontiguousarray(gaussian, np.float32)), _p(out))
    return out


def tq_ip_key_scores(query, idx, norms, qjl, rn, S, signs, centroids, gaussian, groups: int, scaling: float):
    """The reference's turboquant_key_attention_scores (turboquant.py:311-332) in fp64: MSE-only
    keys (dequantize with zero signs and zero residual norms), plus (q S^T)(2 qjl - 1)^T scaled by
    sqrt(pi/2)/D * norms * residual_norms.  query [Hq, Lq, D]; state [Hkv, T, D] / [Hkv, T]."""
    hkv, t, d = idx.shape
    hq, lq, _ = query.shape
    flat = lambda a: a.reshape(hkv * t, -1)
    zero = np.zeros_like(flat(rn)).reshape(-1)
    mse = tq_ip_dequant(flat(idx), flat(norms).reshape(-1), flat(qjl), zero, signs, centroids, gaussian)
    mse = mse.astype(np.float64).reshape(hkv, t, d)
    gq = query.astype(np.float64).reshape(hkv, groups, lq, d)
    mse_scores = np.einsum("hgld,htd->hglt", gq, mse)
    sg = 2.0 * qjl.astype(np.float64) - 1.0
    proj = gq @ S.astype(np.float64).T
    res = (np.sqrt(np.pi / 2.0) / d) * norms.reshape(hkv, t).astype(np.float64) * rn.reshape(hkv, t)
    qjl_scores = np.einsum("hgld,htd->hglt", proj, sg) * res[:, None, None, :]
    return (mse_scores + qjl_scores) * scaling


# ---------------------------------------------------------------- attention (a13) -- textbook, fp64


def gqa_decode(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, gate: np.ndarray | None = None):
    """Single-token GQA decode in fp64: q [Hq, D], k/v [Hkv, L, D] -> [Hq, D].

    Restates the math of grouped_query_attention (reference ops.py:1552-1575) and the
    CPU branch of TurboQuantKVRow.decode_attention (turboquant.py:1295-1346):
    softmax(scale * q k^T) v, times sigmoid(gate) when given.
    """
    q = q.astype(np.float64)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    hq, d = q.shape
    hkv = k.shape[0]
    grp = hq // hkv
    out = np.zeros((hq, d), np.float64)
    for h in range(hq):
        kv = h // grp
        s = (k[kv] @ q[h]) * scale
        s = s - s.max()
        p = np.exp(s)
        p /= p.sum()
        out[h] = p @ v[kv]
    if gate is not None:
        out = out / (1.0 + np.exp(-gate.astype(np.float64)))
    return out

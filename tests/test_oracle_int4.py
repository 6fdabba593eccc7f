"""Pins the int4 part of the CPU oracle (a1-a3) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in oracle/anna_oracle.c (a wrong
nibble shift, a dropped zero point, scale/zero transposed, wrong rounding) fails it.
"""

import numpy as np
import pytest

from oracle import oracle as orc
from tests._util import rel_err


def _pack_first_dim(values: np.ndarray) -> np.ndarray:
    """int [K, N] -> int32 [K/8, N] with k = 8*row + j at bits 4j (GPTQ qweight layout)."""
    k, n = values.shape
    v = values.astype(np.int64).reshape(k // 8, 8, n)
    words = (v << (4 * np.arange(8))[None, :, None]).sum(1)
    return np.where(words >= 2**31, words - 2**32, words).astype(np.int32)


def _pack_last_dim(values: np.ndarray) -> np.ndarray:
    r, c = values.shape
    v = values.astype(np.int64).reshape(r, c // 8, 8)
    words = (v << (4 * np.arange(8))).sum(-1)
    return np.where(words >= 2**31, words - 2**32, words).astype(np.int32)


def test_autoround_known_answer_matches_reference_test():
    # Known-answer input of tests/test_quantization_replace.py:145-176 (reference):
    # weight_int = (arange % 15) + 1, zero point 8 stored as 7, scales 0.125..1.0, group 32.
    k, n, group = 32, 8, 32
    weight_int = (np.arange(k * n).reshape(k, n) % 15) + 1
    gq = _pack_first_dim(weight_int)
    gz = _pack_last_dim(np.full((1, 8), 7))
    scales = np.array([[0.125, 0.25, 0.375, 0.5, 0.625, 0.75, 0.875, 1.0]], np.float32)
    qw, qs, qz = orc.autoround_to_int4(gq, gz, orc.f16_bits(scales), k, n, group, 32)
    assert (qz == 8).all()
    np.testing.assert_array_equal(qs, scales)
    dense = orc.int4_dequant(qw, qs, qz, k, group)
    expected = ((weight_int - 8) * scales[0][None, :]).T
    np.testing.assert_array_equal(dense, expected)
    # the reference test's forward comparison: linspace input, atol 1e-4
    x = np.linspace(-1.0, 1.0, 2 * 32, dtype=np.float32).reshape(2, 32)
    xb = orc.bf16_bits(x)
    y = orc.int4_linear(xb, qw, qs, qz, group)
    y_ref = orc.bf16_to_f32(xb).astype(np.float64) @ expected.T.astype(np.float64)
    np.testing.assert_allclose(y, y_ref, atol=1e-4, rtol=1e-4)


def test_autoround_padding_takes_tail_zero_point():
    k, n, group, kp = 40, 16, 32, 64
    rng = np.random.default_rng(0)
    weight_int = rng.integers(0, 16, size=(48, n))
    gq = _pack_first_dim(weight_int)
    zeros = rng.integers(0, 15, size=(2, n))
    gz = _pack_last_dim(zeros)
    qw, qs, qz = orc.autoround_to_int4(gq, gz, orc.f16_bits(np.ones((2, n), np.float32)), k, n, group, kp)
    np.testing.assert_array_equal(qz, zeros + 1)
    codes = orc.int4_dequant(qw, np.ones((2, n), np.float32), np.zeros((2, n), np.int8), kp, group)
    # real columns copy the GPTQ codes, padded columns carry the tail group's zero point
    np.testing.assert_array_equal(codes[:, :k], weight_int[:k].T)
    np.testing.assert_array_equal(codes[:, k:], np.broadcast_to((zeros[1] + 1)[:, None], (n, kp - k)))


def test_quantize_linspace_matches_reference_error_bounds():
    # tests/test_quantization_replace.py:179-199 (reference): max err < 0.15, mean < 0.05.
    w = np.linspace(-1.0, 1.0, 16 * 32, dtype=np.float32).reshape(16, 32)
    qw, qs, qz = orc.int4_quantize(w, 32, 32)
    x = orc.bf16_bits(np.linspace(-1.0, 1.0, 4 * 32, dtype=np.float32).reshape(4, 32))
    y = orc.bf16_to_f32(orc.bf16_bits(orc.int4_linear(x, qw, qs, qz, 32)))
    ref = orc.bf16_to_f32(orc.bf16_bits(orc.bf16_to_f32(x) @ w.T))
    err = np.abs(y - ref)
    assert err.max() < 0.15 and err.mean() < 0.05


def test_quantize_closed_form_special_cases():
    group = 8
    w = np.zeros((3, 16), np.float32)
    w[1, :8] = [7.0, 0.5, 1.5, -0.5, -7.0, 2.5, -2.5, 0.0]  # scale = 1, exact .5 ties
    w[2, 8:] = [3.0, -3.0, 1.0, 0, 0, 0, 0, 0]
    for rounding, ties in ((0, [15, 8, 10, 8, 1, 10, 6, 8]), (1, [15, 9, 10, 8, 1, 11, 6, 8])):
        qw, qs, qz = orc.int4_quantize(w, group, 16, rounding=rounding)
        codes = orc.int4_dequant(qw, np.ones_like(qs), np.zeros_like(qz), 16, group).astype(int)
        assert (qz == 8).all()
        assert codes[0].tolist() == [8] * 16 and qs[0, 0] == 1.0 and qs[1, 0] == 1.0  # amax == 0
        assert codes[1, :8].tolist() == ties
        assert codes[1, 8:].tolist() == [8] * 8
        # amax element lands on 15 (positive) / 1 (negative)
        assert codes[2, 8] == 15 and codes[2, 9] == 1
        assert qs[1, 2] == np.float32(3.0) / np.float32(7.0)


def test_quantize_matches_independent_numpy_restatement():
    rng = np.random.default_rng(1)
    n, k, group = 24, 200, 32
    kp = 224
    w = rng.normal(0, 1, size=(n, k)).astype(np.float32)
    qw, qs, qz = orc.int4_quantize(w, group, kp)
    wp = np.zeros((n, kp), np.float32)
    wp[:, :k] = w
    grouped = wp.reshape(n, kp // group, group)
    amax = np.abs(grouped).max(-1)
    scale = np.where(amax > 0, amax / np.float32(7.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint((grouped / scale[..., None]).astype(np.float32) + np.float32(8.0)), 0, 15).astype(np.int64)
    np.testing.assert_array_equal(qs, scale.T)
    np.testing.assert_array_equal(qw, _pack_last_dim(q.reshape(n, kp)))
    assert (qw < 0).any(), "nibble 7 >= 8 must give negative int32 words"


def test_dequant_and_linear_match_brute_force():
    rng = np.random.default_rng(2)
    n, kp, group, m = 20, 256, 128, 3
    codes = rng.integers(0, 16, size=(n, kp))
    qw = _pack_last_dim(codes)
    qs = rng.uniform(0.01, 0.1, size=(kp // group, n)).astype(np.float32)
    qz = rng.integers(0, 16, size=(kp // group, n)).astype(np.int8)
    dense = orc.int4_dequant(qw, qs, qz, kp, group)
    gidx = np.arange(kp) // group
    brute = (codes - qz[gidx].T.astype(np.int64)) * qs[gidx].T
    np.testing.assert_array_equal(dense, brute.astype(np.float32))
    # bf16 scales are read as bf16
    qs_b = orc.bf16_bits(qs)
    dense_b = orc.int4_dequant(qw, qs_b, qz, kp, group, scale_dtype=orc.BF16)
    np.testing.assert_array_equal(dense_b, ((codes - qz[gidx].T) * orc.bf16_to_f32(qs_b)[gidx].T).astype(np.float32))
    x = orc.bf16_bits(rng.normal(size=(m, kp)).astype(np.float32))
    y = orc.int4_linear(x, qw, qs, qz, group)
    wb = orc.bf16_to_f32(orc.bf16_bits(dense)).astype(np.float64)
    ref = orc.bf16_to_f32(x).astype(np.float64) @ wb.T
    assert rel_err(y, ref) < 1e-6


@pytest.mark.parametrize("v", [0.0, 1.0, -2.5, 3.14159, 65504.0, 1e-6, 6e-8, 1e-9, 65520.0])
def test_half_and_bf16_conversions_round_to_nearest_even(v):
    L = orc.lib()
    assert L.orc_f32_to_f16(v) == int(np.float16(np.float32(v)).view(np.uint16))
    assert L.orc_f32_to_bf16(v) == int(orc.bf16_bits(np.array([v], np.float32))[0])

"""Pins the TurboQuant part of the CPU oracle (a9-a11) and the native codebook/rotation.

* values: closed form, layout and round-trip bound of quantize_turboquant_values
  (reference turboquant.py:164-252), against an independent numpy restatement;
* codebook: the published Lloyd-Max levels of N(0,1) (Max 1960), independently of the
  oracle's own Lloyd iteration;
* rotation: orthogonal, deterministic per seed, seed-sensitive;
* MSE quantizer: distortion of the 2/3/4-bit quantizer on random unit vectors against
  the values TurboQuant reports (Zandieh et al. 2025), zero-vector special case.
The reference's own MSE/IP quantizer lives in the absent `turboquant` package: parity of
the MSE codes with the reference is unpinned; these checks pin this build's definition.
"""

import numpy as np
import pytest

from anna_amd import fused_ops
from oracle import oracle as orc

# Max (1960), Table I: positive output levels of the N(0,1) Lloyd-Max quantizer.
MAX_1960 = {
    1: [0.7979],
    2: [0.4528, 1.5104],
    3: [0.2451, 0.7560, 1.3440, 2.1520],
    4: [0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6181, 2.0690, 2.7326],
}


def _values_numpy(v: np.ndarray, bits: int, group: int):
    """Independent vectorized restatement (float32 ops, np.rint = half to even)."""
    h, t, d = v.shape
    levels = np.float32((1 << bits) - 1)
    g = v.reshape(h, t, d // group, group)
    vmin, vmax = g.min(-1, keepdims=True), g.max(-1, keepdims=True)
    sc = np.maximum(((vmax - vmin) / levels).astype(np.float32), np.float32(1e-8))
    sc = orc.bf16_to_f32(orc.bf16_bits(sc))
    zr = orc.bf16_to_f32(orc.bf16_bits(vmin))
    q = np.clip(np.rint(((g - zr) / sc).astype(np.float32)), 0, levels).astype(np.uint32).reshape(h, t, d)
    sb = 2 if bits == 2 else 4
    per = 8 // sb
    packed = (q.reshape(h, t, d // per, per) << (sb * np.arange(per))).sum(-1).astype(np.uint8)
    return packed, sc[..., 0], zr[..., 0]


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("group", [32, 16, 8, 2])
def test_values_quantizer_matches_numpy_restatement(bits, group):
    rng = np.random.default_rng(bits * 100 + group)
    v = orc.bf16_to_f32(orc.bf16_bits(rng.normal(size=(2, 9, 64)).astype(np.float32)))
    v[0, 0, :group] = 0.5  # constant group: scale clamps to 1e-8, codes 0
    data, scales, zeros = orc.tq_values_quantize(orc.bf16_bits(v), orc.BF16, bits, group)
    p_np, s_np, z_np = _values_numpy(v, bits, group)
    np.testing.assert_array_equal(data, p_np)
    np.testing.assert_array_equal(orc.bf16_to_f32(scales), s_np)
    np.testing.assert_array_equal(orc.bf16_to_f32(zeros), z_np)
    assert orc.bf16_to_f32(scales)[0, 0, 0] == orc.bf16_to_f32(orc.bf16_bits(np.array([1e-8], np.float32)))[0]
    deq = orc.tq_values_dequant(data, scales, zeros, orc.BF16, bits, group)
    bound = np.repeat(orc.bf16_to_f32(scales), group, axis=-1) * 0.5 + 1e-6
    assert (np.abs(deq - v) <= bound * 1.01 + np.abs(v) * 2 ** -8).all()


def test_values_two_bit_layout_known_answer():
    # one group of 4: min 0, max 3 -> scale 1, codes = values, packed little-end first
    v = np.array([[[0.0, 3.0, 1.0, 2.0]]], np.float32)
    data, scales, zeros = orc.tq_values_quantize(orc.bf16_bits(v), orc.BF16, 2, 4)
    assert data.tolist() == [[[0 | (3 << 2) | (1 << 4) | (2 << 6)]]]
    assert orc.bf16_to_f32(scales).tolist() == [[[1.0]]] and orc.bf16_to_f32(zeros).tolist() == [[[0.0]]]


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_lloyd_max_levels_match_published_table(bits):
    lv = orc.lloyd_max_gaussian(bits)
    np.testing.assert_allclose(lv[len(lv) // 2:], MAX_1960[bits], atol=5e-4)  # table printed to 3-4 decimals
    np.testing.assert_allclose(lv, -lv[::-1], atol=1e-12)


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_native_codebook_is_scaled_lloyd_max(bits):
    d = 256
    cent, thr = (t.numpy() for t in fused_ops.tq_codebook(bits, d))
    ref = orc.lloyd_max_gaussian(bits) / np.sqrt(d)
    # the 2-bit pair is fp16-structured: within 1e-4 relative of Lloyd-Max
    np.testing.assert_allclose(cent, ref, rtol=1e-4 if bits == 2 else 1e-6)
    np.testing.assert_allclose(thr, 0.5 * (cent[1:] + cent[:-1]), rtol=1e-6)
    if bits == 2:
        a16, b16 = np.float16(1.123046875), np.float16(3.74609375)
        assert (a16.view(np.uint16) & 0xFF) == (b16.view(np.uint16) & 0xFF)
        assert abs(cent[3] / cent[2] - float(b16) / float(a16)) < 1e-6


def test_native_rotation_is_orthogonal_and_seeded():
    r = fused_ops.tq_rotation(128, 42).numpy().astype(np.float64)
    np.testing.assert_allclose(r @ r.T, np.eye(128), atol=2e-6)
    np.testing.assert_array_equal(fused_ops.tq_rotation(128, 42).numpy(), r.astype(np.float32))
    assert not np.array_equal(fused_ops.tq_rotation(128, 43).numpy(), r.astype(np.float32))
    # Haar: the diagonal carries no sign bias and entries have variance 1/D
    assert abs(r.var() - 1 / 128) < 1e-4


@pytest.mark.parametrize("bits,expected", [(2, 0.1175), (3, 0.0345), (4, 0.0095)])
def test_mse_distortion_matches_turboquant_paper(bits, expected):
    d = 128
    rng = np.random.default_rng(bits)
    x = rng.normal(size=(400, d)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    r = fused_ops.tq_rotation(d, 42).numpy()
    cent, thr = (t.numpy() for t in fused_ops.tq_codebook(bits, d))
    codes, norms = orc.tq_mse_quantize(x, orc.F32, r, thr, bits)
    xh = orc.tq_mse_dequant(codes, norms, r, cent, bits)
    mse = float(((xh - x) ** 2).sum(1).mean())
    assert abs(mse - expected) / expected < 0.12, mse


def test_mse_quantizer_hand_computed_codes():
    """Identity rotation and hand-chosen thresholds, so every code below is worked out by hand:
    code_i = number of thresholds t_j with x_i >= t_j * |x|, packed 4 per byte (2-bit, element
    i at bits 2i) or 2 per byte (4-bit); the norm is |x| in fp16."""
    eye = np.eye(4, dtype=np.float32)
    thr = np.array([-0.5, 0.0, 0.5], np.float32)
    # |x| = 5: thresholds scale to -2.5, 0, 2.5
    x = np.array([[3.0, 4.0, 0.0, 0.0],    # 3 >= 2.5 -> 3; 4 -> 3; 0 >= 0 -> 2; 0 -> 2
                  [-3.0, 0.0, -4.0, 0.0],  # -3 < -2.5 -> 0; 0 -> 2; -4 -> 0; 0 -> 2
                  [2.5, -2.5, 0.0, 0.0],   # ties: 2.5 >= 2.5 -> 3; -2.5 >= -2.5 -> 1
                  [0.0, 0.0, 0.0, 0.0]],   # zero vector: 0 >= 0 for every threshold -> 3
                 np.float32)
    x[2, 2] = np.sqrt(np.float32(25.0) - np.float32(12.5))  # keep |x| = 5 (3.5355...) -> 3
    codes, norms = orc.tq_mse_quantize(x, orc.F32, eye, thr, 2)
    want = [[3, 3, 2, 2], [0, 2, 0, 2], [3, 1, 3, 2], [3, 3, 3, 3]]
    packed = [c[0] | (c[1] << 2) | (c[2] << 4) | (c[3] << 6) for c in want]
    assert codes[:, 0].tolist() == packed
    assert orc.f16_to_f32(norms).tolist() == [5.0, 5.0, float(np.float16(np.sqrt(np.float32(25.0)))), 0.0]
    # dequant: |x|_fp16 * centroid[code], rotation back by the identity
    cent = np.array([-0.75, -0.25, 0.25, 0.75], np.float32)
    xh = orc.tq_mse_dequant(codes, norms, eye, cent, 2)
    np.testing.assert_array_equal(xh[0], [3.75, 3.75, 1.25, 1.25])
    np.testing.assert_array_equal(xh[1], [-3.75, 1.25, -3.75, 1.25])
    np.testing.assert_array_equal(xh[3], [0.0, 0.0, 0.0, 0.0])


def test_mse_quantizer_hand_computed_four_bit():
    # 4-bit: 15 thresholds -7/16 .. 7/16 (times |x| = 1): code = #{t_j <= x_i}
    eye = np.eye(2, dtype=np.float32)
    thr = (np.arange(-7, 8, dtype=np.float32) / 16).astype(np.float32)
    x = np.array([[0.6, 0.8]], np.float32)  # |x| rounds to 1 in fp32
    codes, norms = orc.tq_mse_quantize(x, orc.F32, eye, thr, 4)
    nrm = np.float32(np.sqrt(np.float32(0.6) * np.float32(0.6) + np.float32(0.8) * np.float32(0.8)))
    c0 = int((x[0, 0] >= thr * nrm).sum())  # 0.6 >= 7/16: all 15
    c1 = int((x[0, 1] >= thr * nrm).sum())
    assert (c0, c1) == (15, 15)
    assert codes.tolist() == [[15 | (15 << 4)]]
    x = np.array([[0.1, -0.995]], np.float32)  # 0.1: t <= 0.1 for t in -7/16..1/16 -> 9; -0.995 -> 0
    codes, _ = orc.tq_mse_quantize(x, orc.F32, eye, thr, 4)
    assert codes.tolist() == [[9 | (0 << 4)]]


# ---------------------------------------------------------------- Hadamard rotation (power-of-two D)


@pytest.mark.parametrize("d", [64, 128, 256, 1024])
def test_hadamard_transform_equals_the_dense_matrix(d):
    """The fixed-order FWHT is the matrix H diag(s) / sqrt(D) (Sylvester H, built independently
    in numpy), to fp32 rounding; the matrix is orthogonal."""
    s = orc.tq_hadamard_signs(d, 42)
    m = orc.tq_hadamard_matrix(s)
    np.testing.assert_allclose(m @ m.T, np.eye(d), atol=1e-12)
    rng = np.random.default_rng(d)
    for _ in range(3):
        x = rng.normal(size=d).astype(np.float32)
        y = orc.tq_hadamard_rotate(x, s)
        np.testing.assert_allclose(y, m @ x.astype(np.float64), rtol=0, atol=2e-6 * np.abs(x).sum() / np.sqrt(d))


@pytest.mark.parametrize("d", [64, 128, 256])
def test_native_rotation_and_signs_match_the_oracle(d):
    s = orc.tq_hadamard_signs(d, 42)
    np.testing.assert_array_equal(fused_ops.tq_hadamard_signs(d, 42).numpy(), s)
    assert 0.3 < (s < 0).mean() < 0.7
    assert not np.array_equal(fused_ops.tq_hadamard_signs(d, 43).numpy(), s)
    np.testing.assert_array_equal(fused_ops.tq_rotation(d, 42).numpy(), orc.tq_hadamard_matrix(s).astype(np.float32))


def test_hadamard_spreads_a_basis_vector_evenly():
    # an outlier channel (a basis vector) lands as +-1/sqrt(D) on every coordinate
    s = orc.tq_hadamard_signs(256, 42)
    for k in (0, 7, 255):
        x = np.zeros(256, np.float32)
        x[k] = 3.0
        np.testing.assert_array_equal(np.abs(orc.tq_hadamard_rotate(x, s)), np.full(256, 3.0 / 16, np.float32))


def test_hadamard_quantizer_hand_computed_codes():
    """D = 4, signs (+1, -1, +1, +1), thresholds (-1/2, 0, 1/2):
    x = e0 -> s x = (1,0,0,0) -> FWHT (1,1,1,1) -> /2 -> 0.5 each, |x| = 1: 0.5 >= 0.5 -> code 3;
    x = (1,1,0,0) -> s x = (1,-1,0,0) -> bit 0: (0,2,0,0) -> bit 1: (0,2,0,2) -> /2 -> (0,1,0,1),
    |x| = sqrt 2: thresholds scale to (-0.707, 0, 0.707): codes (2, 3, 2, 3)."""
    s = np.array([1, -1, 1, 1], np.float32)
    thr = np.array([-0.5, 0.0, 0.5], np.float32)
    x = np.array([[1, 0, 0, 0], [1, 1, 0, 0]], np.float32)
    np.testing.assert_array_equal(orc.tq_hadamard_rotate(x[1], s), [0.0, 1.0, 0.0, 1.0])
    codes, norms = orc.tq_hadamard_quantize(x, orc.F32, s, thr, 2)
    assert codes[:, 0].tolist() == [0xFF, 2 | (3 << 2) | (2 << 4) | (3 << 6)]
    assert orc.f16_to_f32(norms).tolist() == [1.0, float(np.float16(np.sqrt(2.0)))]


@pytest.mark.parametrize("bits", [2, 4])
def test_hadamard_quantizer_agrees_with_the_dense_quantizer(bits):
    """Same rotation as a dense matrix through orc_tq_mse_quantize: codes differ only where y
    lands within fp32 rounding of a threshold (the two round y differently)."""
    d = 256
    s = orc.tq_hadamard_signs(d, 42)
    r = orc.tq_hadamard_matrix(s).astype(np.float32)
    cent, thr = (t.numpy() for t in fused_ops.tq_codebook(bits, d))
    x = np.random.default_rng(bits).normal(size=(64, d)).astype(np.float32)
    c1, n1 = orc.tq_hadamard_quantize(x, orc.F32, s, thr, bits)
    c2, n2 = orc.tq_mse_quantize(x, orc.F32, r, thr, bits)
    assert (c1 == c2).mean() > 0.995
    assert np.abs(orc.f16_to_f32(n1) - orc.f16_to_f32(n2)).max() <= 2 ** -10 * orc.f16_to_f32(n1).max()


@pytest.mark.parametrize("bits,expected", [(2, 0.1175), (3, 0.0345), (4, 0.0095)])
def test_hadamard_mse_distortion_matches_turboquant_paper(bits, expected):
    d = 256
    x = np.random.default_rng(10 + bits).normal(size=(400, d)).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    s = orc.tq_hadamard_signs(d, 42)
    cent, thr = (t.numpy() for t in fused_ops.tq_codebook(bits, d))
    codes, norms = orc.tq_hadamard_quantize(x, orc.F32, s, thr, bits)
    xh = orc.tq_mse_dequant(codes, norms, orc.tq_hadamard_matrix(s).astype(np.float32), cent, bits)
    mse = float(((xh - x) ** 2).sum(1).mean())
    assert abs(mse - expected) / expected < 0.12, mse


def test_cpu_path_tensor_row_append_matches_the_oracle_quantizer():
    """The torch restatement timed as the pack's CPU baseline (nearest centroid after a dense
    rotation) gives the oracle's codes (threshold count at the centroid midpoints) and norms,
    and keeps the newest residual_len tokens as they are."""
    import torch

    from oracle.cpu_paths import tq_tensor_row_append

    d, bits = 64, 2
    rng = np.random.default_rng(7)
    x = rng.normal(size=(2, 40, d)).astype(np.float32)
    r = fused_ops.tq_rotation(d, 42).numpy()
    cent, thr = (t.numpy() for t in fused_ops.tq_codebook(bits, d))
    idx, norms, resid = tq_tensor_row_append(torch.from_numpy(x), 8, torch.from_numpy(r), torch.from_numpy(cent))
    assert idx.shape == (2, 32, d) and norms.shape == (2, 32, 1)
    np.testing.assert_array_equal(resid.numpy(), x[:, 32:])
    codes, _ = orc.tq_mse_quantize(np.ascontiguousarray(x[:, :32].reshape(-1, d)), orc.F32, r, thr, bits)
    unpacked = np.stack([(codes >> (2 * e)) & 3 for e in range(4)], -1).reshape(-1, d)
    np.testing.assert_array_equal(idx.reshape(-1, d).numpy(), unpacked)
    np.testing.assert_allclose(norms.reshape(-1).numpy(), np.linalg.norm(x[:, :32].reshape(-1, d), axis=1),
                               rtol=1e-6)

"""Pins oracle.gqa_decode, the checker of every decode test, with cases the mathematics fixes.

Each case is chosen so that a plausible slip in the oracle fails it: a softmax without the
max shift overflows on the large-score cases, a missing normalization breaks the single-key
and mean cases, a wrong GQA head map (h % Hkv instead of h // G) picks the wrong V in the
head-map case, a transposed product or a dropped scale changes the two-key closed form,
and a gate applied as g instead of sigmoid(g) fails the gate limits.
"""

import numpy as np
import pytest

from oracle import oracle as orc


def rng_case(seed, hq=8, hkv=2, L=17, d=32):
    rng = np.random.default_rng(seed)
    return (rng.normal(size=(hq, d)), rng.normal(size=(hkv, L, d)), rng.normal(size=(hkv, L, d)))


def test_single_key_returns_its_value():
    q, k, v = rng_case(1, L=1)
    out = orc.gqa_decode(q, k, v, 0.37)
    for h in range(8):
        np.testing.assert_allclose(out[h], v[h // 4, 0], rtol=0, atol=1e-12)


def test_identical_keys_give_the_mean_of_values():
    q, k, v = rng_case(2, L=13)
    k[:] = k[:, :1]
    out = orc.gqa_decode(q, k, v, 1.0)
    for h in range(8):
        np.testing.assert_allclose(out[h], v[h // 4].mean(0), atol=1e-12)


def test_zero_scale_gives_the_mean_of_values():
    q, k, v = rng_case(3)
    out = orc.gqa_decode(q, k, v, 0.0)
    np.testing.assert_allclose(out, np.repeat(v.mean(1), 4, axis=0), atol=1e-12)


def test_shifting_every_key_by_one_vector_changes_nothing():
    # q.(k_t + u) = q.k_t + q.u: every score of a head moves by the same constant
    q, k, v = rng_case(4)
    u = np.random.default_rng(40).normal(size=(2, 1, 32)) * 3.0
    a = orc.gqa_decode(q, k, v, 0.5)
    b = orc.gqa_decode(q, k + u, v, 0.5)
    np.testing.assert_allclose(a, b, atol=1e-10)


def test_two_keys_closed_form():
    # softmax of two scores: p0 = 1 / (1 + exp(s1 - s0)), s_t = scale * q.k_t
    q, k, v = rng_case(5, hq=2, hkv=1, L=2, d=16)
    scale = 0.3
    out = orc.gqa_decode(q, k, v, scale)
    for h in range(2):
        s0, s1 = scale * (q[h] @ k[0, 0]), scale * (q[h] @ k[0, 1])
        p0 = 1.0 / (1.0 + np.exp(s1 - s0))
        np.testing.assert_allclose(out[h], p0 * v[0, 0] + (1 - p0) * v[0, 1], atol=1e-12)


def test_large_scores_select_the_best_key_without_overflow():
    q, k, v = rng_case(6, hq=4, hkv=1, L=9, d=8)
    k[0, 5] = q[0] * 50.0  # score ~ 50^2 * |q|^2 >> exp's range
    out = orc.gqa_decode(q[:1], k, v, 1.0)
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out[0], v[0, 5], atol=1e-12)


def test_gqa_head_map_groups_consecutive_heads():
    # Hq/Hkv = 4 with identical keys per kv head: head h must read V of kv head h // 4 only
    hq, hkv, L, d = 8, 2, 5, 4
    q = np.random.default_rng(7).normal(size=(hq, d))
    k = np.ones((hkv, L, d))
    v = np.stack([np.full((L, d), 1.0), np.full((L, d), -3.0)])
    out = orc.gqa_decode(q, k, v, 1.0)
    np.testing.assert_allclose(out[:4], 1.0)
    np.testing.assert_allclose(out[4:], -3.0)


@pytest.mark.parametrize("g,factor", [(60.0, 1.0), (0.0, 0.5), (-60.0, 0.0)])
def test_gate_limits(g, factor):
    q, k, v = rng_case(8)
    plain = orc.gqa_decode(q, k, v, 0.25)
    gated = orc.gqa_decode(q, k, v, 0.25, gate=np.full(q.shape, g))
    np.testing.assert_allclose(gated, plain * factor, atol=1e-12)


def test_gate_is_elementwise_sigmoid():
    q, k, v = rng_case(9)
    g = np.random.default_rng(90).normal(size=q.shape)
    plain = orc.gqa_decode(q, k, v, 0.25)
    np.testing.assert_allclose(orc.gqa_decode(q, k, v, 0.25, gate=g), plain * (1 / (1 + np.exp(-g))), atol=1e-12)


def test_permuting_tokens_changes_nothing():
    # attention is a sum over tokens: a ring-ordered residual window must give the same output
    q, k, v = rng_case(10)
    perm = np.random.default_rng(11).permutation(k.shape[1])
    np.testing.assert_allclose(orc.gqa_decode(q, k, v, 0.4), orc.gqa_decode(q, k[:, perm], v[:, perm], 0.4),
                               atol=1e-12)

"""Batched varlen decode over the 2-bit TQ-MSE pool (the MFMA fast path) against the oracle.

Codes and norms in the pool are bit-exact with the oracle quantizer (values after undoing
the 32-token blocking); the attention output is within normwise max relative error 1e-2
of the oracle's fp64 attention over the oracle-dequantized cache plus the dense window.
"""

import numpy as np
import pytest
import torch

from anna_amd.tq_cache import TurboQuantBatchCache
from oracle import oracle as orc
from tests._util import BF16_TOL, rel_err

pytestmark = pytest.mark.gpu


def bits_of(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def unblock(blocked: np.ndarray, tokens: int) -> np.ndarray:
    """[tokens/32][2048] blocked value codes -> natural [tokens][64] (numpy restatement)."""
    out = np.zeros((tokens, 64), np.uint8)
    for blk in range(tokens // 32):
        for t in range(32):
            kq, half, e = (t % 16) // 4, t // 16, t % 4
            for dim in range(256):
                c = (blocked[blk, kq * 512 + dim * 2 + half] >> (2 * e)) & 3
                out[blk * 32 + t, dim // 4] |= c << (2 * (dim % 4))
    return out


@pytest.mark.parametrize("tokens_per_item", [0, 64, 512])
def test_batched_decode_matches_oracle(gpu, tokens_per_item):
    torch.manual_seed(60)
    hkv, g, d = 2, 8, 256
    lens = [75, 140, 33, 20]
    resid = [5, 0, 32, 20]  # last sequence: residual only
    cache = TurboQuantBatchCache(batch=4, kv_heads=hkv, q_heads=hkv * g, capacities=[l - r for l, r in zip(lens, resid)],
                                 residual_capacity=32, device=gpu, tokens_per_item=tokens_per_item)
    keys = [torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16) for L in lens]
    vals = [torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16) for L in lens]
    for b in range(4):
        cache.load_sequence(b, keys[b], vals[b], resid[b])
    q = torch.randn(4, hkv * g, d, device=gpu).to(torch.bfloat16)
    out = cache.decode(q, scaling=1.0 / 16)
    R = cache.qn.rotation.cpu().numpy()
    cent = cache.qn.centroids.cpu().numpy()
    thr = cache.qn.thresholds.cpu().numpy()
    kc_pool = cache.key_codes.cpu().numpy()
    vc_pool = cache.value_codes.cpu().numpy()
    for b in range(4):
        ql, off = lens[b] - resid[b], cache.offsets[b]
        kk, vv = [], []
        for h in range(hkv):
            parts_k, parts_v = [], []
            if ql > 0:
                kcodes, knorms = orc.tq_mse_quantize(bits_of(keys[b][h, :ql]), orc.BF16, R, thr, 2)
                vcodes, vnorms = orc.tq_mse_quantize(bits_of(vals[b][h, :ql]), orc.BF16, R, thr, 2)
                np.testing.assert_array_equal(kc_pool[h, off:off + ql], kcodes)
                np.testing.assert_array_equal(bits_of(cache.key_norms[h, off:off + ql]), knorms)
                np.testing.assert_array_equal(bits_of(cache.value_norms[h, off:off + ql]), vnorms)
                qp = -(-ql // 32) * 32
                nat = unblock(vc_pool[h, off // 32:(off + qp) // 32], qp)
                np.testing.assert_array_equal(nat[:ql], vcodes)
                parts_k.append(orc.tq_mse_dequant(kcodes, knorms, R, cent, 2))
                parts_v.append(orc.tq_mse_dequant(vcodes, vnorms, R, cent, 2))
            if resid[b] > 0:
                parts_k.append(keys[b][h, ql:].float().cpu().numpy())
                parts_v.append(vals[b][h, ql:].float().cpu().numpy())
            kk.append(np.concatenate(parts_k))
            vv.append(np.concatenate(parts_v))
        ref = orc.gqa_decode(q[b].float().cpu().numpy(), np.stack(kk), np.stack(vv), 1.0 / 16)
        assert rel_err(out[b].float().cpu().numpy(), ref) <= BF16_TOL, b


def np_dequant(codes: np.ndarray, norms_bits: np.ndarray, R: np.ndarray, cent: np.ndarray) -> np.ndarray:
    """x_hat = |x|_fp16 * R^T c[code] for natural 2-bit codes [n, 64] (fp64, vectorized; the
    same map as orc.tq_mse_dequant, which is checked against it on a slice below)."""
    c = np.stack([(codes >> (2 * e)) & 3 for e in range(4)], -1).reshape(codes.shape[0], 256)
    y = cent.astype(np.float64)[c]
    return (y @ R.astype(np.float64)) * orc.f16_to_f32(norms_bits).astype(np.float64)[:, None]


@pytest.mark.parametrize("tokens_per_item", [0, 512, 2048])
def test_batched_decode_config4_sizes(gpu, tokens_per_item):
    """BASELINE config 4 at its own sizes: B=8, Hq=16, Hkv=2, D=256, a full 128-token window on
    every sequence and packed lengths up to 16,384 (two sequences above 4,000).  tokens_per_item
    512 gives 32 items for the longest (b, kv-head) (the combine merges > 16 items, in batches),
    2048 gives 64 blocks per item (each of the 8 split waves runs 4 ping-pong pair iterations).
    Codes are checked bit-exact on sampled tokens of every (b, kv-head); the output against
    fp64 attention over the dequantized pool plus the window."""
    print(f"[case] tq batch config4 tokens_per_item={tokens_per_item}", flush=True)
    torch.manual_seed(4)
    B, HKV, G, D, R = 8, 2, 8, 256, 128
    qlens = [16384, 4100, 1024, 7777, 2048, 1500, 12000, 3001]
    cache = TurboQuantBatchCache(batch=B, kv_heads=HKV, q_heads=HKV * G, capacities=qlens, residual_capacity=R,
                                 device=gpu, tokens_per_item=tokens_per_item)
    keys = [torch.randn(HKV, L + R, D, device=gpu).to(torch.bfloat16) for L in qlens]
    vals = [torch.randn(HKV, L + R, D, device=gpu).to(torch.bfloat16) for L in qlens]
    for b in range(B):
        cache.load_sequence(b, keys[b], vals[b], R)
    q = torch.randn(B, HKV * G, D, device=gpu).to(torch.bfloat16)
    out = cache.decode(q, scaling=1.0 / 16).float().cpu().numpy()
    Rm = cache.qn.rotation.cpu().numpy()
    cent = cache.qn.centroids.cpu().numpy()
    thr = cache.qn.thresholds.cpu().numpy()
    kc_pool = cache.key_codes.cpu().numpy()
    kn_pool = bits_of(cache.key_norms)
    vn_pool = bits_of(cache.value_norms)
    vc_pool = cache.value_codes.cpu().numpy()
    rng = np.random.default_rng(0)
    for b in range(B):
        ql, off = qlens[b], cache.offsets[b]
        qp = -(-ql // 32) * 32
        kk, vv = [], []
        for h in range(HKV):
            vnat = unblock_fast(vc_pool[h, off // 32:(off + qp) // 32], qp)[:ql]
            kcodes, vcodes = kc_pool[h, off:off + ql], vnat
            knorms, vnorms = kn_pool[h, off:off + ql], vn_pool[h, off:off + ql]
            pick = np.sort(rng.choice(ql, size=min(ql, 96), replace=False))
            kb, vb = bits_of(keys[b][h, :ql])[pick], bits_of(vals[b][h, :ql])[pick]
            oc, on = orc.tq_mse_quantize(np.ascontiguousarray(kb), orc.BF16, Rm, thr, 2)
            np.testing.assert_array_equal(kcodes[pick], oc)
            np.testing.assert_array_equal(knorms[pick], on)
            oc, on = orc.tq_mse_quantize(np.ascontiguousarray(vb), orc.BF16, Rm, thr, 2)
            np.testing.assert_array_equal(vcodes[pick], oc)
            np.testing.assert_array_equal(vnorms[pick], on)
            kd = np_dequant(kcodes, knorms, Rm, cent)
            if b == 0 and h == 0:
                np.testing.assert_allclose(kd[:64], orc.tq_mse_dequant(kcodes[:64], knorms[:64], Rm, cent, 2),
                                           rtol=1e-5, atol=1e-6)
            kk.append(np.concatenate([kd, keys[b][h, ql:].float().cpu().numpy()]))
            vv.append(np.concatenate([np_dequant(vcodes, vnorms, Rm, cent), vals[b][h, ql:].float().cpu().numpy()]))
        ref = orc.gqa_decode(q[b].float().cpu().numpy(), np.stack(kk), np.stack(vv), 1.0 / 16)
        assert rel_err(out[b], ref) <= BF16_TOL, b


def unblock_fast(blocked: np.ndarray, tokens: int) -> np.ndarray:
    """Vectorized form of unblock(): blocked [tokens/32][2048] -> natural codes [tokens][64]."""
    nb = tokens // 32
    x = blocked.reshape(nb, 4, 256, 2)  # [blk][kq][dim][half]
    t = np.arange(32)
    kq, half, e = (t % 16) // 4, t // 16, t % 4
    sel = x[:, kq, :, half].transpose(1, 0, 2)  # advanced indices first: [t][blk][dim] -> [blk][t][dim]
    codes = (sel >> (2 * e)[None, :, None].astype(np.uint8)) & 3
    codes = codes.reshape(tokens, 64, 4)
    return (codes[..., 0] | (codes[..., 1] << 2) | (codes[..., 2] << 4) | (codes[..., 3] << 6)).astype(np.uint8)

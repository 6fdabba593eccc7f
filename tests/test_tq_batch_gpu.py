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

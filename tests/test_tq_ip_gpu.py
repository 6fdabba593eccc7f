"""Parity of the HIP TurboQuant inner-product keys (a10: reference turboquant.py:255-332) with
the oracle.

* quantize: mse_indices, qjl_signs, norms and residual norms bit-exact with
  orc_tq_ip_quantize (same fp32 operation order);
* dequantize: fp32 output bit-exact with orc_tq_ip_dequant, bf16 output its rounding;
* attention scores: max relative error 1e-4 against the reference's own score formula
  (turboquant.py:311-332) restated in fp64 with S = G R (fp32 accumulation on the GPU);
* the module API (_quantize_turboquant_keys, dequantize_turboquant_keys,
  turboquant_key_attention_scores) shapes, dtypes and argument checks.
"""

import numpy as np
import pytest
import torch

from anna_amd import fused_ops
from anna_amd.turboquant import (TurboQuantKeyState, _quantize_turboquant_keys, dequantize_turboquant_keys,
                                 get_turboquant_ip_quantizer, turboquant_key_attention_scores)
from oracle import oracle as orc
from tests._util import rel_err

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: orc.BF16, torch.float16: orc.F16, torch.float32: orc.F32}


def _host(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _oracle_state(x: torch.Tensor, q):
    d = x.shape[-1]
    return orc.tq_ip_quantize(_host(x.reshape(-1, d)), DT[x.dtype], q.signs.cpu().numpy(), q.thresholds.cpu().numpy(),
                              q.centroids.cpu().numpy(), q.gaussian.cpu().numpy(), q.bits)


@pytest.mark.parametrize("d,bits,dtype,n", [
    (64, 2, torch.float32, 37),
    (128, 3, torch.bfloat16, 16),
    (256, 4, torch.float16, 21),
    (256, 2, torch.bfloat16, 64),
    (1024, 3, torch.bfloat16, 5),
])
def test_ip_quantize_and_dequant_bit_exact(gpu, d, bits, dtype, n):
    print(f"case ip quantize d={d} bits={bits} {dtype} n={n}", flush=True)
    g = torch.Generator().manual_seed(d * 10 + bits)
    x = (torch.randn(n, d + 8, generator=g) * 2.0).to(dtype)[:, :d].to(gpu)  # strided rows
    x[min(3, n - 1)] = 0
    q = get_turboquant_ip_quantizer(head_dim=d, bits=bits, device=gpu)
    idx, norms, qjl, rn = q.quantize(x)
    torch.cuda.synchronize()
    oi, on, oq, orn = _oracle_state(x, q)
    np.testing.assert_array_equal(idx.cpu().numpy(), oi)
    np.testing.assert_array_equal(qjl.cpu().numpy(), oq)
    np.testing.assert_array_equal(norms.cpu().numpy(), on)
    np.testing.assert_array_equal(rn.cpu().numpy(), orn)
    out = q.dequantize(idx, norms, qjl, rn, dtype=torch.float32)
    want = orc.tq_ip_dequant(oi, on, oq, orn, q.signs.cpu().numpy(), q.centroids.cpu().numpy(),
                             q.gaussian.cpu().numpy())
    np.testing.assert_array_equal(out.cpu().numpy(), want)
    out16 = q.dequantize(idx, norms, qjl, rn, dtype=torch.bfloat16)
    np.testing.assert_array_equal(_host(out16), orc.bf16_bits(want))


@pytest.mark.parametrize("d,bits,hq,hkv,lq,t", [
    (128, 2, 8, 2, 1, 100),
    (256, 3, 16, 2, 3, 64),
    (64, 4, 4, 4, 5, 1),
    (256, 2, 32, 2, 1, 200),
])
def test_ip_scores_match_reference_formula(gpu, d, bits, hq, hkv, lq, t):
    print(f"case ip scores d={d} bits={bits} hq={hq} hkv={hkv} lq={lq} t={t}", flush=True)
    g = torch.Generator().manual_seed(7 * d + t)
    keys = torch.randn(hkv, t, d, generator=g).to(torch.bfloat16).to(gpu)
    query = torch.randn(lq, hq, d, generator=g).to(torch.bfloat16).to(gpu).transpose(0, 1)  # strided heads
    state = _quantize_turboquant_keys(keys, bits=bits, device=gpu)
    assert state.mse_indices.shape == (hkv, t, d) and state.qjl_signs.shape == (hkv, t, d)
    assert state.norms.shape == (hkv, t, 1) and state.residual_norms.shape == (hkv, t, 1)
    scaling = d ** -0.5
    got = turboquant_key_attention_scores(query=query, state=state, bits=bits, device=gpu,
                                          num_key_value_groups=hq // hkv, scaling=scaling)
    assert got.shape == (hkv, hq // hkv, lq, t) and got.dtype == torch.float32
    q = get_turboquant_ip_quantizer(head_dim=d, bits=bits, device=gpu)
    want = orc.tq_ip_key_scores(query.float().cpu().numpy(), state.mse_indices.cpu().numpy(),
                                state.norms.cpu().numpy(), state.qjl_signs.cpu().numpy(),
                                state.residual_norms.cpu().numpy(), q.S.cpu().numpy(), q.signs.cpu().numpy(),
                                q.centroids.cpu().numpy(), q.gaussian.cpu().numpy(), hq // hkv, scaling)
    assert rel_err(got.cpu().numpy(), want) <= 1e-4
    # and the same scores from the expanded keys
    kt = dequantize_turboquant_keys(state, bits=bits, device=gpu, dtype=torch.float32)
    dense = torch.einsum("hgld,htd->hglt", query.float().reshape(hkv, hq // hkv, lq, d), kt) * scaling
    assert rel_err(got.cpu().numpy(), dense.cpu().numpy()) <= 1e-4


def test_ip_key_api_checks(gpu):
    keys = torch.randn(2, 5, 128, device=gpu, dtype=torch.bfloat16)
    state = _quantize_turboquant_keys(keys, bits=3, device=gpu)
    assert isinstance(state, TurboQuantKeyState)
    kt = dequantize_turboquant_keys(state, bits=3, device=gpu, dtype=torch.bfloat16)
    assert kt.shape == (2, 5, 128) and kt.dtype == torch.bfloat16
    # reconstruction error: well below the key norm (3-bit: 2-bit MSE stage + QJL)
    err = (kt.float() - keys.float()).norm(dim=-1) / keys.float().norm(dim=-1)
    assert float(err.max()) < 0.6
    with pytest.raises(ValueError):
        _quantize_turboquant_keys(keys[0], bits=3, device=gpu)
    q = torch.randn(6, 1, 128, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        turboquant_key_attention_scores(query=q, state=state, bits=3, device=gpu, num_key_value_groups=2,
                                        scaling=1.0)
    with pytest.raises(ValueError):
        get_turboquant_ip_quantizer(head_dim=96, bits=3, device=gpu)
    empty = _quantize_turboquant_keys(keys[:, :0], bits=3, device=gpu)
    s = turboquant_key_attention_scores(query=q[:4], state=empty, bits=3, device=gpu, num_key_value_groups=2,
                                        scaling=1.0)
    assert s.shape == (2, 2, 1, 0)


@pytest.mark.parametrize("bits", [2, 3])
def test_kv_row_with_inner_product_keys(gpu, bits):
    """TurboQuantKVRow(key_quantizer="ip"): the reference's key state (turboquant.py:1098-1111)
    bit-exact with the oracle quantizer, its reconstruction as the decode keys, decode attention
    against the oracle over [reconstructed prefix ++ window], clone equal."""
    from anna_amd.turboquant import TurboQuantKVRow

    torch.manual_seed(70 + bits)
    hkv, groups, d, r = 2, 4, 128, 16
    row = TurboQuantKVRow(bits=bits, residual_len=r, key_quantizer="ip")
    ks = [torch.randn(hkv, n, d, device=gpu, dtype=torch.bfloat16) for n in (50, 1, 1, 30)]
    vs = [torch.randn_like(k) for k in ks]
    for k, v in zip(ks, vs):
        row.append(k, v)
    n = row.quantized_length
    assert (row.length, n, row.residual_length) == (82, 66, 16)
    kk = torch.cat(ks, 1)
    q = get_turboquant_ip_quantizer(head_dim=d, bits=bits, device=gpu)
    oi, on, oq, orn = _oracle_state(kk[:, :n].contiguous(), q)
    np.testing.assert_array_equal(row._kcodes[:, :n].reshape(-1, d).cpu().numpy(), oi)
    np.testing.assert_array_equal(row._kqjl[:, :n].reshape(-1, d).cpu().numpy(), oq)
    np.testing.assert_array_equal(row._knorms[:, :n].reshape(-1).cpu().numpy(), on)
    np.testing.assert_array_equal(row._krn[:, :n].reshape(-1).cpu().numpy(), orn)
    kdeq = orc.tq_ip_dequant(oi, on, oq, orn, q.signs.cpu().numpy(), q.centroids.cpu().numpy(),
                             q.gaussian.cpu().numpy())
    np.testing.assert_array_equal(_host(row._kdense[:, :n]).reshape(-1, d), orc.bf16_bits(kdeq))
    query = torch.randn(hkv * groups, 1, d, device=gpu, dtype=torch.bfloat16)
    out = row.decode_attention(query, scaling=d ** -0.5, num_key_value_groups=groups)
    keys, values = row.materialize(dtype=torch.float32)
    ref = orc.gqa_decode(query.float().cpu().numpy()[:, 0], keys.cpu().numpy(), values.cpu().numpy(), d ** -0.5)
    assert rel_err(out.float().cpu().numpy()[:, 0], ref) <= 1e-2
    out2 = row.clone().decode_attention(query, scaling=d ** -0.5, num_key_value_groups=groups)
    assert torch.equal(out, out2)

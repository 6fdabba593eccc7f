"""The batched Qwen3DynamicCache adapter (anna_amd.tq_dynamic, reference ops.py:618-661,
1024-1072) against the per-row path it replaces.

* Rows constructed with the reference's arguments only (bits, residual_len) hold the
  inner-product key state, bit-exact with the oracle quantizer (orc_tq_ip_quantize).
* After the same appends, every adapter row's state (key indices, norms, QJL signs, residual
  norms, reconstruction, value codes/scales/zeros, window) equals a TurboQuantKVRow's bit for bit.
* The batched decode equals the per-row TurboQuantKVRow.decode_attention within 1e-2 (normwise
  max relative error), with and without the gate, with sequences of different lengths; both equal
  the oracle's attention over the materialized cache.
"""

import numpy as np
import pytest
import torch

from anna_amd.tq_dynamic import TurboQuantDynamicCache
from anna_amd.turboquant import TurboQuantKVRow, get_turboquant_ip_quantizer
from oracle import oracle as orc
from tests._util import BF16_TOL, rel_err

pytestmark = pytest.mark.gpu


def _host(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _same_state(a: TurboQuantKVRow, b: TurboQuantKVRow) -> None:
    assert (a.length, a.quantized_length, a.residual_length) == (b.length, b.quantized_length, b.residual_length)
    n = a.quantized_length
    for name in ("_kcodes", "_knorms", "_kqjl", "_krn", "_kdense", "_vdata", "_vscales", "_vzeros"):
        x, y = getattr(a, name), getattr(b, name)
        if x is None or n == 0:
            assert y is None or n == 0, name
            continue
        np.testing.assert_array_equal(_host(x[:, :n]), _host(y[:, :n]), err_msg=name)
    np.testing.assert_array_equal(_host(a._residual_keys), _host(b._residual_keys))
    np.testing.assert_array_equal(_host(a._residual_values), _host(b._residual_values))


def test_reference_row_arguments_give_ip_keys(gpu):
    """TurboQuantKVRow(bits, residual_len) -- the reference's call (ops.py:632-635) -- keeps the
    inner-product key state, bit-exact with the oracle."""
    torch.manual_seed(90)
    hkv, d, r, bits = 2, 128, 8, 4
    row = TurboQuantKVRow(bits=bits, residual_len=r)
    assert row.key_quantizer == "ip"
    k = torch.randn(hkv, 29, d, device=gpu, dtype=torch.bfloat16)
    row.append(k, torch.randn_like(k))
    n = row.quantized_length
    assert n == 21
    q = get_turboquant_ip_quantizer(head_dim=d, bits=bits, device=gpu)
    oi, on, oq, orn = orc.tq_ip_quantize(_host(k[:, :n].reshape(-1, d)), orc.BF16, q.signs.cpu().numpy(),
                                         q.thresholds.cpu().numpy(), q.centroids.cpu().numpy(),
                                         q.gaussian.cpu().numpy(), bits)
    np.testing.assert_array_equal(row._kcodes[:, :n].reshape(-1, d).cpu().numpy(), oi)
    np.testing.assert_array_equal(row._kqjl[:, :n].reshape(-1, d).cpu().numpy(), oq)
    np.testing.assert_array_equal(row._knorms[:, :n].reshape(-1).cpu().numpy(), on)
    np.testing.assert_array_equal(row._krn[:, :n].reshape(-1).cpu().numpy(), orn)
    kdeq = orc.tq_ip_dequant(oi, on, oq, orn, q.signs.cpu().numpy(), q.centroids.cpu().numpy(),
                             q.gaussian.cpu().numpy())
    np.testing.assert_array_equal(_host(row._kdense[:, :n]).reshape(-1, d), orc.bf16_bits(kdeq))


@pytest.mark.parametrize("bits,d,key_quantizer,prefill", [
    (4, 128, "ip", 37),    # the reference's default bits; window full after prefill: batched steps
    (2, 256, "ip", 5),     # windows fill during the steps: per-row steps, then batched ones
    (3, 64, "mse", 20),    # opt-in TQ-MSE keys
])
def test_adapter_matches_per_row_path(gpu, bits, d, key_quantizer, prefill):
    print(f"[case] adapter bits={bits} d={d} keys={key_quantizer} prefill={prefill}", flush=True)
    torch.manual_seed(91 + bits + d)
    B, hkv, groups, r, layer = 3, 2, 4, 16, 1
    dt = torch.bfloat16
    cache = TurboQuantDynamicCache(2, kv_cache_quant_bits=bits, kv_cache_residual_len=r,
                                   turboquant_layers=[layer], key_quantizer=key_quantizer)
    rows = [TurboQuantKVRow(bits=bits, residual_len=r, key_quantizer=key_quantizer) for _ in range(B)]

    k = torch.randn(B, hkv, prefill, d, device=gpu, dtype=dt)
    v = torch.randn_like(k)
    pk, pv, past = cache.update(k, v, layer)
    assert past.tolist() == [0] * B
    for b in range(B):
        rows[b].append(k[b], v[b])
        rk, rv = rows[b].materialize()
        assert torch.equal(pk[b], rk) and torch.equal(pv[b], rv)
    # sequence 1 takes 14 more tokens on its own: lengths now differ
    k1, v1 = torch.randn(hkv, 14, d, device=gpu, dtype=dt), torch.randn(hkv, 14, d, device=gpu, dtype=dt)
    cache.append_row(layer, 1, k1, v1)
    rows[1].append(k1, v1)
    assert cache.layer_lengths[layer] == [prefill, prefill + 14, prefill]

    for step in range(20):
        k = torch.randn(B, hkv, 1, d, device=gpu, dtype=dt)
        v = torch.randn_like(k)
        _, _, past = cache.update(k, v, layer, require_dense_cache=False)
        assert past.tolist() == [rw.length for rw in rows]
        for b in range(B):
            rows[b].append(k[b], v[b])
        q = torch.randn(B, hkv * groups, 1, d, device=gpu, dtype=dt)
        gate = torch.randn_like(q) if step % 2 else None
        out = cache.turboquant_single_token_decode_attention(layer, q, scaling=d ** -0.5,
                                                             num_key_value_groups=groups, gate=gate)
        assert out.shape == q.shape and out.dtype == dt
        for b in range(B):
            ref = rows[b].decode_attention(q[b], scaling=d ** -0.5, num_key_value_groups=groups,
                                           gate=None if gate is None else gate[b])
            assert rel_err(out[b].float().cpu().numpy(), ref.float().cpu().numpy()) <= BF16_TOL
            if step == 19:
                keys, values = cache.turboquant_rows[layer][b].materialize(dtype=torch.float32)
                g = None if gate is None else gate[b, :, 0].float().cpu().numpy()
                oref = orc.gqa_decode(q[b, :, 0].float().cpu().numpy(), keys.cpu().numpy(), values.cpu().numpy(),
                                      d ** -0.5, g)
                assert rel_err(out[b, :, 0].float().cpu().numpy(), oref) <= BF16_TOL
                one = cache.turboquant_rows[layer][b].decode_attention(
                    q[b], scaling=d ** -0.5, num_key_value_groups=groups, gate=None if gate is None else gate[b])
                assert rel_err(one.float().cpu().numpy(), out[b].float().cpu().numpy()) <= 1e-3

    assert cache.get_seq_lengths().tolist() == [rw.length for rw in rows]
    for b in range(B):
        _same_state(cache.turboquant_rows[layer][b].clone(), rows[b])


def test_adapter_argument_checks(gpu):
    cache = TurboQuantDynamicCache(2, kv_cache_quant_bits=4, kv_cache_residual_len=8, turboquant_layers=[0])
    k = torch.randn(2, 2, 3, 64, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        cache.update(k, k, 1)
    cache.update(k, k, 0)
    q = torch.randn(2, 4, 1, 64, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        cache.turboquant_single_token_decode_attention(0, q[:, :, :, :32], scaling=1.0, num_key_value_groups=2)
    with pytest.raises(ValueError):
        cache.turboquant_single_token_decode_attention(0, q, scaling=1.0, num_key_value_groups=3)
    with pytest.raises(ValueError):
        cache.turboquant_single_token_decode_attention(0, q, scaling=1.0, num_key_value_groups=2, gate=q[:1])
    out = cache.turboquant_single_token_decode_attention(0, q, scaling=1.0, num_key_value_groups=2)
    assert torch.isfinite(out.float()).all()
    with pytest.raises(ValueError):
        TurboQuantDynamicCache(1, kv_cache_quant_bits=5)

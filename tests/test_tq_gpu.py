"""Parity of the HIP TurboQuant path (packing, decode attention, KV rows) with the oracle.

Codes, scales, zero points, norms and the residual window are bit-exact; attention
outputs are within normwise max relative error 1e-2 of the oracle's fp64 softmax
attention over the same dequantized cache (reference CPU branch of
TurboQuantKVRow.decode_attention, turboquant.py:1295-1346).
"""

import numpy as np
import pytest
import torch

from anna_amd import fused_ops
from anna_amd.turboquant import (TurboQuantKVRow, TurboQuantTensorRow, dequantize_turboquant_values,
                                 get_turboquant_quantizer, quantize_turboquant_values)
from oracle import oracle as orc
from tests._util import BF16_TOL, oracle_tq_quantize, rel_err

pytestmark = pytest.mark.gpu


def bits_of(t: torch.Tensor) -> np.ndarray:
    """16-bit float tensor -> uint16 bit patterns (numpy)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


DT = {torch.bfloat16: orc.BF16, torch.float16: orc.F16}


# ---------------------------------------------------------------- packing


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("group", [32, 16, 2])
def test_values_quantize_bit_exact(gpu, dtype, bits, group):
    print(f"[case] values bits={bits} group={group} {dtype}", flush=True)
    torch.manual_seed(bits * 10 + group)
    big = torch.randn(2, 40, 96, device=gpu).to(dtype)
    v = big[:, 3:30, :64]  # strided [H, T, D]
    state = quantize_turboquant_values(v, bits=bits, group_size=group)
    data, scales, zeros = orc.tq_values_quantize(bits_of(v), DT[dtype], bits, group)
    np.testing.assert_array_equal(state.data.cpu().numpy(), data)
    np.testing.assert_array_equal(bits_of(state.scales), scales)
    np.testing.assert_array_equal(bits_of(state.zeros), zeros)
    deq = dequantize_turboquant_values(state)
    np.testing.assert_array_equal(f32(deq), orc.tq_values_dequant(data, scales, zeros, DT[dtype], bits, group))


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
@pytest.mark.parametrize("d", [64, 128, 192, 256, 512])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_mse_quantize_bit_exact(gpu, bits, d, dtype):
    """Power-of-two D takes the Hadamard kernel (oracle: orc_tq_hadamard_quantize), D = 192 the
    dense Haar one (oracle: orc_tq_mse_quantize); codes and norms bit-exact either way."""
    print(f"[case] mse bits={bits} D={d} {dtype}", flush=True)
    g = torch.Generator().manual_seed(bits + d)
    x = torch.randn(37, d, generator=g)
    x[:, : max(1, d // 100)] *= 8.0  # outlier channels (benchmark config 3)
    x[5] = 0.0
    x = x.to(dtype)
    qn = get_turboquant_quantizer(head_dim=d, bits=bits, device=gpu)
    codes, norms = qn.quantize(x.to(gpu))
    xin = bits_of(x) if dtype == torch.bfloat16 else x.numpy()
    assert qn.kind == ("haar" if d == 192 else "hadamard")
    ref_codes, ref_norms = oracle_tq_quantize(qn, xin, orc.BF16 if dtype == torch.bfloat16 else orc.F32)
    np.testing.assert_array_equal(codes.cpu().numpy(), ref_codes)
    np.testing.assert_array_equal(bits_of(norms), ref_norms)
    deq = qn.dequantize(codes, norms, dtype=torch.float32)
    ref = orc.tq_mse_dequant(ref_codes, ref_norms, qn.rotation.cpu().numpy(), qn.centroids.cpu().numpy(), bits)
    assert rel_err(f32(deq), ref) < 1e-5


# ---------------------------------------------------------------- decode ops (reference op schemas)


def _oracle_attention(q, k, v, scale, gate=None):
    """q [B, Hq, 1, D], k/v [B, Hkv, L, D] (numpy fp32) -> [B, Hq, 1, D] fp64."""
    out = []
    for b in range(q.shape[0]):
        g = None if gate is None else gate[b, :, 0, :]
        out.append(orc.gqa_decode(q[b, :, 0, :], k[b], v[b], scale, g)[:, None, :])
    return np.stack(out)


def _gate4(gate3, heads, d):
    b = gate3.shape[0]
    return gate3.view(b, 1, heads, d).transpose(1, 2)


def test_splitkv_long_qwen35_shape(gpu):
    # reference test_fused_op_xpu.py:544-560: B=1, Hq=16, Hkv=4, D=256, L=4096, block 256
    torch.manual_seed(19)
    q = torch.randn(1, 16, 1, 256, device=gpu, dtype=torch.bfloat16)
    k = torch.randn(1, 4, 4096, 256, device=gpu, dtype=torch.bfloat16)
    v = torch.randn(1, 4, 4096, 256, device=gpu, dtype=torch.bfloat16)
    out = torch.ops.anna.gqa_decode_splitkv_fused(q, k, v, 256 ** -0.5, 256)
    ref = _oracle_attention(f32(q), f32(k), f32(v), 256 ** -0.5)
    assert rel_err(f32(out), ref) <= BF16_TOL


def test_splitkv_strided_kv_and_gate(gpu):
    # reference test_fused_op_xpu.py:563-597
    torch.manual_seed(20)
    hq, hkv, d, key_len, cap = 8, 2, 64, 257, 512
    q = torch.randn(1, hq, 1, d, device=gpu, dtype=torch.bfloat16)
    ks = torch.randn(1, hkv, cap, d, device=gpu, dtype=torch.bfloat16)
    vs = torch.randn(1, hkv, cap, d, device=gpu, dtype=torch.bfloat16)
    k, v = ks[:, :, :key_len], vs[:, :, :key_len]
    assert not k.is_contiguous()
    gate3 = torch.randn(1, 1, hq * d, device=gpu, dtype=torch.bfloat16)
    gate4 = _gate4(gate3, hq, d)
    out4 = torch.ops.anna.gqa_decode_splitkv_fused(q, k, v, d ** -0.5, 64, gate4)
    out3 = torch.ops.anna.gqa_decode_splitkv_fused(q, k, v, d ** -0.5, 64, gate3)
    ref = _oracle_attention(f32(q), f32(k), f32(v), d ** -0.5, f32(gate4))
    assert rel_err(f32(out4), ref) <= BF16_TOL
    assert rel_err(f32(out3), ref) <= BF16_TOL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_splitkv_out_reuses_workspace_strided_query(gpu, dtype):
    # reference test_fused_op_xpu.py:600-645, plus batch 3 and every activation dtype
    torch.manual_seed(22)
    b, hq, hkv, d, key_len, bs = 3, 8, 2, 64, 193, 64
    blocks = -(-key_len // bs)
    qs = torch.randn(b, hq, 1, 2 * d, device=gpu).to(dtype)
    q = qs[..., ::2]
    k = torch.randn(b, hkv, 256, d, device=gpu).to(dtype)[:, :, :key_len]
    v = torch.randn(b, hkv, 256, d, device=gpu).to(dtype)[:, :, :key_len]
    out = torch.empty_like(q)
    ps = torch.empty(b, hq, blocks + 2, 2, device=gpu)
    pv = torch.empty(b, hq, blocks + 2, d, device=gpu)
    ret = torch.ops.anna.gqa_decode_splitkv_fused_out(q, k, v, out, ps, pv, d ** -0.5, bs)
    assert ret.untyped_storage().data_ptr() == out.untyped_storage().data_ptr()
    ref = _oracle_attention(f32(q), f32(k), f32(v), d ** -0.5)
    assert rel_err(f32(out), ref) <= BF16_TOL
    with pytest.raises(RuntimeError, match="capacity"):
        torch.ops.anna.gqa_decode_splitkv_fused_out(q, k, v, out, ps[:, :, :1], pv[:, :, :1], d ** -0.5, bs)


@pytest.mark.parametrize("value_bits", [2, 3, 4])
def test_splitkv_turboquant_matches_dequantized_reference(gpu, value_bits):
    # reference test_fused_op_xpu.py:647-703: D=64, qlen 77, residual 5, group 16, gate
    torch.manual_seed(24 + value_bits)
    hq, hkv, d, qlen, rlen, bs = 8, 2, 64, 77, 5, 64
    blocks = -(-(qlen + rlen) // bs)
    q = torch.randn(1, hq, 1, 2 * d, device=gpu, dtype=torch.bfloat16)[..., ::2]
    qk = torch.randn(1, hkv, qlen, d, device=gpu, dtype=torch.bfloat16)
    dense_v = torch.randn(hkv, qlen, d, device=gpu, dtype=torch.bfloat16)
    st = quantize_turboquant_values(dense_v, bits=value_bits, group_size=16)
    rk = torch.randn(1, hkv, rlen, d, device=gpu, dtype=torch.bfloat16)
    rv = torch.randn(1, hkv, rlen, d, device=gpu, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    ps = torch.empty(1, hq, blocks + 1, 2, device=gpu)
    pv = torch.empty(1, hq, blocks + 1, d, device=gpu)
    gate4 = _gate4(torch.randn(1, 1, hq * d, device=gpu, dtype=torch.bfloat16), hq, d)
    ret = torch.ops.anna.gqa_decode_splitkv_turboquant_fused_out(
        q, qk, st.data.unsqueeze(0), st.scales.unsqueeze(0), st.zeros.unsqueeze(0), rk, rv, out, ps, pv,
        d ** -0.5, value_bits, st.group_size, bs, gate4)
    assert ret.untyped_storage().data_ptr() == out.untyped_storage().data_ptr()
    vq = orc.tq_values_dequant(st.data.cpu().numpy(), bits_of(st.scales), bits_of(st.zeros), orc.BF16, value_bits, 16)
    kk = np.concatenate([f32(qk), f32(rk)], axis=2)
    vv = np.concatenate([vq[None], f32(rv)], axis=2)
    ref = _oracle_attention(f32(q), kk, vv, d ** -0.5, f32(gate4))
    assert rel_err(f32(out), ref) <= BF16_TOL


@pytest.mark.parametrize("key_stride", [1, 2])
def test_splitkv_turboquant_scalar_and_vector_loads(gpu, key_stride):
    """D=256, batch 2: contiguous keys with group 32 take the kernel's vector loads; keys
    strided in the last dim with group 2 (not a multiple of a lane's 4 dims) take the
    per-element loads.  Both against the oracle on the dequantized cache."""
    torch.manual_seed(40 + key_stride)
    b, hq, hkv, d, qlen, rlen, bits, bs = 2, 8, 2, 256, 203, 9, 4, 64
    group = 32 if key_stride == 1 else 2
    q = torch.randn(b, hq, 1, d, device=gpu, dtype=torch.bfloat16)
    qk = torch.randn(b, hkv, qlen, d * key_stride, device=gpu, dtype=torch.bfloat16)[..., ::key_stride]
    assert qk.stride(-1) == key_stride
    st = quantize_turboquant_values(torch.randn(b * hkv, qlen, d, device=gpu, dtype=torch.bfloat16), bits=bits,
                                    group_size=group)
    rk = torch.randn(b, hkv, rlen, d, device=gpu, dtype=torch.bfloat16)
    rv = torch.randn(b, hkv, rlen, d, device=gpu, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    nb = -(-(qlen + rlen) // bs) + 1
    ps = torch.empty(b, hq, nb, 2, device=gpu)
    pv = torch.empty(b, hq, nb, d, device=gpu)
    torch.ops.anna.gqa_decode_splitkv_turboquant_fused_out(
        q, qk, st.data.view(b, hkv, qlen, -1), st.scales.view(b, hkv, qlen, -1), st.zeros.view(b, hkv, qlen, -1),
        rk, rv, out, ps, pv, d ** -0.5, bits, group, bs, None)
    vq = orc.tq_values_dequant(st.data.cpu().numpy(), bits_of(st.scales), bits_of(st.zeros), orc.BF16, bits,
                               group).reshape(b, hkv, qlen, d)
    kk = np.concatenate([f32(qk), f32(rk)], axis=2)
    vv = np.concatenate([vq, f32(rv)], axis=2)
    ref = _oracle_attention(f32(q), kk, vv, d ** -0.5)
    assert rel_err(f32(out), ref) <= BF16_TOL


@pytest.mark.parametrize("vfmt", ["minmax", "mse"])
def test_splitkv_tq_mse_keys(gpu, vfmt):
    """Packed TQ-MSE keys (scored against R q) with min/max or TQ-MSE values, batch 2."""
    torch.manual_seed(31)
    b, hq, hkv, d, qlen, rlen, bits = 2, 8, 2, 128, 150, 7, 2
    qn = get_turboquant_quantizer(head_dim=d, bits=bits, device=gpu)
    q = torch.randn(b, hq, 1, d, device=gpu, dtype=torch.bfloat16)
    kd = torch.randn(b, hkv, qlen, d, device=gpu, dtype=torch.bfloat16)
    vd = torch.randn(b, hkv, qlen, d, device=gpu, dtype=torch.bfloat16)
    kc, kn = qn.quantize(kd.reshape(-1, d))
    kc, kn = kc.view(b, hkv, qlen, -1), kn.view(b, hkv, qlen)
    kdeq = orc.tq_mse_dequant(kc.reshape(-1, kc.shape[-1]).cpu().numpy(), bits_of(kn.reshape(-1)),
                              qn.rotation.cpu().numpy(), qn.centroids.cpu().numpy(), bits).reshape(b, hkv, qlen, d)
    if vfmt == "mse":
        vc, vn = qn.quantize(vd.reshape(-1, d))
        vc, vn = vc.view(b, hkv, qlen, -1), vn.view(b, hkv, qlen)
        vdeq = orc.tq_mse_dequant(vc.reshape(-1, vc.shape[-1]).cpu().numpy(), bits_of(vn.reshape(-1)),
                                  qn.rotation.cpu().numpy(), qn.centroids.cpu().numpy(), bits).reshape(b, hkv, qlen, d)
        vkw = dict(value=vc, value_format=fused_ops.VALUES_TQ_MSE, value_scales=vn, value_bits=bits,
                   value_centroids=qn.centroids)
    else:
        st = quantize_turboquant_values(vd.reshape(b * hkv, qlen, d), bits=bits, group_size=32)
        vdeq = orc.tq_values_dequant(st.data.cpu().numpy(), bits_of(st.scales), bits_of(st.zeros), orc.BF16, bits,
                                     32).reshape(b, hkv, qlen, d)
        vkw = dict(value=st.data.view(b, hkv, qlen, -1), value_format=fused_ops.VALUES_MINMAX,
                   value_scales=st.scales.view(b, hkv, qlen, -1), value_zeros=st.zeros.view(b, hkv, qlen, -1),
                   value_bits=bits, value_group_size=32)
    rk = torch.randn(b, hkv, rlen, d, device=gpu, dtype=torch.bfloat16)
    rv = torch.randn(b, hkv, rlen, d, device=gpu, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    ps = torch.empty(b, hq, 16, 2, device=gpu)
    pv = torch.empty(b, hq, 16, d, device=gpu)
    args = fused_ops.decode_args(query=q, len1=qlen, key=kc, key_format=fused_ops.KEYS_TQ_MSE, key_norms=kn,
                                 key_bits=bits, rotation=qn.rotation, rotation_t=qn.rotation_t,
                                 key_centroids=qn.centroids, query_rot=torch.empty(b, hq, d, device=gpu),
                                 residual_key=rk, residual_value=rv, scaling=d ** -0.5, block_size=32, output=out,
                                 partial_stats=ps, partial_values=pv, **vkw)
    assert fused_ops.decode_num_blocks(args) == 5 + 1
    fused_ops.run_decode(args, q)
    ref = _oracle_attention(f32(q), np.concatenate([kdeq, f32(rk)], 2), np.concatenate([vdeq, f32(rv)], 2), d ** -0.5)
    assert rel_err(f32(out), ref) <= BF16_TOL


# ---------------------------------------------------------------- rows (module API)


def test_kv_row_lengths_storage_reuse_and_residual(gpu):
    # reference tests/test_model_shapes.py:379-546 row invariants
    torch.manual_seed(40)
    row = TurboQuantKVRow(bits=2, residual_len=4, key_quantizer="mse")
    k = torch.randn(2, 9, 64, device=gpu, dtype=torch.bfloat16)
    v = torch.randn(2, 9, 64, device=gpu, dtype=torch.bfloat16)
    row.append(k, v)
    assert (row.length, row.quantized_length, row.residual_length) == (9, 5, 4)
    cap = row.quantized_capacity
    assert cap >= 5 + 4
    ptr = row._kcodes.data_ptr()
    k2 = torch.randn(2, 3, 64, device=gpu, dtype=torch.bfloat16)
    v2 = torch.randn(2, 3, 64, device=gpu, dtype=torch.bfloat16)
    row.append(k2, v2)
    assert (row.length, row.quantized_length, row.residual_length) == (12, 8, 4)
    assert row._kcodes.data_ptr() == ptr  # capacity reused, no reallocation
    keys, values = row.materialize()
    kk = torch.cat([k, k2], 1)
    vv = torch.cat([v, v2], 1)
    assert torch.equal(keys[:, 8:], kk[:, 8:]) and torch.equal(values[:, 8:], vv[:, 8:])
    # packed prefix is bit-exact with the oracle quantizers
    qn = get_turboquant_quantizer(head_dim=64, bits=2, device=gpu)
    ref_codes, ref_norms = oracle_tq_quantize(qn, bits_of(kk[:, :8].reshape(-1, 64)), orc.BF16)
    np.testing.assert_array_equal(row._kcodes[:, :8].reshape(16, -1).cpu().numpy(), ref_codes)
    np.testing.assert_array_equal(bits_of(row._knorms[:, :8].reshape(-1)), ref_norms)
    data, scales, zeros = orc.tq_values_quantize(bits_of(vv[:, :8]), orc.BF16, 2, 32)
    np.testing.assert_array_equal(row._vdata[:, :8].cpu().numpy(), data)
    np.testing.assert_array_equal(bits_of(row._vscales[:, :8]), scales)


@pytest.mark.parametrize("bits", [2, 4])
def test_kv_row_decode_attention_matches_oracle(gpu, bits):
    torch.manual_seed(41 + bits)
    hkv, groups, d, r = 2, 4, 128, 16
    row = TurboQuantKVRow(bits=bits, residual_len=r, key_quantizer="mse")
    for n in (50, 1, 1, 30):
        row.append(torch.randn(hkv, n, d, device=gpu, dtype=torch.bfloat16),
                   torch.randn(hkv, n, d, device=gpu, dtype=torch.bfloat16))
    q = torch.randn(hkv * groups, 1, d, device=gpu, dtype=torch.bfloat16)
    gate = torch.randn(hkv * groups, 1, d, device=gpu, dtype=torch.bfloat16)
    out = row.decode_attention(q, scaling=d ** -0.5, num_key_value_groups=groups, gate=gate)
    keys, values = row.materialize(dtype=torch.float32)
    ref = orc.gqa_decode(f32(q)[:, 0], f32(keys), f32(values), d ** -0.5, f32(gate)[:, 0])
    assert rel_err(f32(out)[:, 0], ref) <= BF16_TOL
    clone = row.clone()
    out2 = clone.decode_attention(q, scaling=d ** -0.5, num_key_value_groups=groups, gate=gate)
    assert torch.equal(out, out2)


def test_tensor_row_materialize(gpu):
    torch.manual_seed(50)
    row = TurboQuantTensorRow(bits=2, residual_len=3)
    x = torch.randn(2, 11, 64, device=gpu, dtype=torch.bfloat16)
    row.append(x[:, :6])
    row.append(x[:, 6:])
    assert row.length == 11 and row.quantized_length == 8
    mat = row.materialize()
    assert torch.equal(mat[:, 8:], x[:, 8:])
    qn = get_turboquant_quantizer(head_dim=64, bits=2, device=gpu)
    codes, norms = oracle_tq_quantize(qn, bits_of(x[:, :8].reshape(-1, 64)), orc.BF16)
    ref = orc.tq_mse_dequant(codes, norms, qn.rotation.cpu().numpy(), qn.centroids.cpu().numpy(), 2)
    assert rel_err(f32(mat[:, :8]).reshape(-1, 64), ref) <= BF16_TOL


@pytest.mark.parametrize("d,bits,group,dtype,hkv", [
    (64, 2, 32, torch.bfloat16, 2),
    (128, 3, 64, torch.float16, 2),
    (256, 2, 32, torch.bfloat16, 2),
    (256, 2, 64, torch.bfloat16, 1),
    (256, 4, 128, torch.float16, 1),
    (256, 3, 16, torch.bfloat16, 2),
])
def test_splitkv_turboquant_mfma_tiles(gpu, d, bits, group, dtype, hkv):
    """The MFMA split kernel's tile kinds in one call: 32-token tiles wholly in the packed
    segment (raw-code staging when group % 32 == 0, else the chunked loop), the tile that
    straddles the packed/window boundary, window-only tiles and a short last tile; 8 or 16 query
    heads per KV head; both 16-bit activation dtypes."""
    torch.manual_seed(60 + d + bits + group)
    b, hq, qlen, rlen, bs = 2, 16, 517, 43, 64
    q = torch.randn(b, hq, 1, d, device=gpu, dtype=dtype)
    qk = torch.randn(b, hkv, qlen, d, device=gpu, dtype=dtype)
    st = quantize_turboquant_values(torch.randn(b * hkv, qlen, d, device=gpu, dtype=dtype), bits=bits,
                                    group_size=group)
    rk = torch.randn(b, hkv, rlen, d, device=gpu, dtype=dtype)
    rv = torch.randn(b, hkv, rlen, d, device=gpu, dtype=dtype)
    out = torch.empty_like(q)
    nb = -(-(qlen + rlen) // bs)
    ps = torch.empty(b, hq, nb, 2, device=gpu)
    pv = torch.empty(b, hq, nb, d, device=gpu)
    torch.ops.anna.gqa_decode_splitkv_turboquant_fused_out(
        q, qk, st.data.view(b, hkv, qlen, -1), st.scales.view(b, hkv, qlen, -1), st.zeros.view(b, hkv, qlen, -1),
        rk, rv, out, ps, pv, d ** -0.5, bits, group, bs, None)
    odt = orc.BF16 if dtype == torch.bfloat16 else orc.F16
    vq = orc.tq_values_dequant(st.data.cpu().numpy(), bits_of(st.scales), bits_of(st.zeros), odt, bits,
                               group).reshape(b, hkv, qlen, d)
    kk = np.concatenate([f32(qk), f32(rk)], axis=2)
    vv = np.concatenate([vq, f32(rv)], axis=2)
    ref = _oracle_attention(f32(q), kk, vv, d ** -0.5)
    assert rel_err(f32(out), ref) <= BF16_TOL


@pytest.mark.parametrize("value_kind", ["dense", "minmax"])
def test_splitkv_more_blocks_than_one_merge_workgroup(gpu, value_kind):
    """Over 256 blocks (block 16): the merge takes its general kernel; just under, the
    one-pass kernel.  Both against the oracle."""
    torch.manual_seed(71)
    hq, hkv, d, bs = 8, 1, 128, 16
    for qlen in (4101, 4080):
        q = torch.randn(1, hq, 1, d, device=gpu, dtype=torch.bfloat16)
        k = torch.randn(1, hkv, qlen, d, device=gpu, dtype=torch.bfloat16)
        nb = -(-qlen // bs)
        assert (nb > 256) == (qlen == 4101)
        if value_kind == "dense":
            v = torch.randn(1, hkv, qlen, d, device=gpu, dtype=torch.bfloat16)
            out = torch.ops.anna.gqa_decode_splitkv_fused(q, k, v, d ** -0.5, bs)
            vv = f32(v)
        else:
            st = quantize_turboquant_values(torch.randn(hkv, qlen, d, device=gpu, dtype=torch.bfloat16), bits=2,
                                            group_size=32)
            rk = torch.randn(1, hkv, 0, d, device=gpu, dtype=torch.bfloat16)
            out = torch.empty_like(q)
            ps = torch.empty(1, hq, nb, 2, device=gpu)
            pv = torch.empty(1, hq, nb, d, device=gpu)
            torch.ops.anna.gqa_decode_splitkv_turboquant_fused_out(
                q, k, st.data.unsqueeze(0), st.scales.unsqueeze(0), st.zeros.unsqueeze(0), rk, rk, out, ps, pv,
                d ** -0.5, 2, 32, bs, None)
            vv = orc.tq_values_dequant(st.data.cpu().numpy(), bits_of(st.scales), bits_of(st.zeros), orc.BF16, 2,
                                       32)[None]
        ref = _oracle_attention(f32(q), f32(k), vv, d ** -0.5)
        assert rel_err(f32(out), ref) <= BF16_TOL, qlen

"""The allocation-free split-KV decode entry point against the one with a caller workspace.

anna_mi_gqa_decode_splitkv_noalloc keeps its workspace in a static per-GPU device array and
launches the same kernels as anna_mi_gqa_decode_splitkv, so its output must equal that
entry point's bit for bit.  Two calls in a row, the second smaller, check that the shared
array carries nothing from one call into the next; a TQ-MSE-key call also places the
rotated query in the array.  Calls go through the C ABI (ctypes), with the workspace fields
of the argument struct left null.
"""

import ctypes

import pytest
import torch

from anna_amd import _lib, fused_ops
from anna_amd.turboquant import get_turboquant_quantizer, quantize_turboquant_values

pytestmark = pytest.mark.gpu


def _minmax_case(gpu, b, hq, hkv, d, qlen, rlen, bits, group, bs, seed, gate=False):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    q = torch.randn(b, hq, 1, d, device=gpu, generator=g).to(torch.bfloat16)
    qk = torch.randn(b, hkv, qlen, d, device=gpu, generator=g).to(torch.bfloat16)
    st = quantize_turboquant_values(torch.randn(b * hkv, qlen, d, device=gpu, generator=g).to(torch.bfloat16),
                                    bits=bits, group_size=group)
    rk = torch.randn(b, hkv, rlen, d, device=gpu, generator=g).to(torch.bfloat16)
    rv = torch.randn(b, hkv, rlen, d, device=gpu, generator=g).to(torch.bfloat16)
    gt = torch.randn(b, 1, hq * d, device=gpu, generator=g).to(torch.bfloat16) if gate else None
    keep = (q, qk, st, rk, rv, gt)
    kw = dict(query=q, len1=qlen, key=qk, value=st.data.view(b, hkv, qlen, -1), value_format=fused_ops.VALUES_MINMAX,
              value_scales=st.scales.view(b, hkv, qlen, -1), value_zeros=st.zeros.view(b, hkv, qlen, -1),
              value_bits=bits, value_group_size=group, residual_key=rk, residual_value=rv, scaling=d ** -0.5,
              block_size=bs, gate=gt)
    return kw, keep


def _mse_key_case(gpu, b, hq, hkv, d, qlen, rlen, seed):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    qn = get_turboquant_quantizer(head_dim=d, bits=2, device=gpu)
    q = torch.randn(b, hq, 1, d, device=gpu, generator=g).to(torch.bfloat16)
    kc, kn = qn.quantize(torch.randn(b * hkv * qlen, d, device=gpu, generator=g).to(torch.bfloat16))
    vc, vn = qn.quantize(torch.randn(b * hkv * qlen, d, device=gpu, generator=g).to(torch.bfloat16))
    rk = torch.randn(b, hkv, rlen, d, device=gpu, generator=g).to(torch.bfloat16)
    rv = torch.randn(b, hkv, rlen, d, device=gpu, generator=g).to(torch.bfloat16)
    keep = (q, kc, kn, vc, vn, rk, rv, qn)
    kw = dict(query=q, len1=qlen, key=kc.view(b, hkv, qlen, -1), key_format=fused_ops.KEYS_TQ_MSE,
              key_norms=kn.view(b, hkv, qlen), key_bits=2, rotation=qn.rotation, rotation_t=qn.rotation_t,
              key_centroids=qn.centroids, value=vc.view(b, hkv, qlen, -1), value_format=fused_ops.VALUES_TQ_MSE,
              value_scales=vn.view(b, hkv, qlen), value_bits=2, value_centroids=qn.centroids, residual_key=rk,
              residual_value=rv, scaling=d ** -0.5, block_size=32)
    return kw, keep


def _both(gpu, kw):
    """(output of the workspace entry point, output of the allocation-free one)."""
    q = kw["query"]
    b, hq, _, d = q.shape
    out_ws = torch.empty_like(q)
    probe = fused_ops.decode_args(output=out_ws, partial_stats=torch.empty(b, hq, 1, 2, device=gpu),
                                  partial_values=torch.empty(b, hq, 1, d, device=gpu), **kw)
    nblk = fused_ops.decode_num_blocks(probe)
    ps = torch.empty(b, hq, nblk, 2, device=gpu)
    pv = torch.empty(b, hq, nblk, d, device=gpu)
    qrot = torch.empty(b, hq, d, device=gpu) if kw.get("key_format") == fused_ops.KEYS_TQ_MSE else None
    extra = dict(query_rot=qrot) if qrot is not None else {}
    args = fused_ops.decode_args(output=out_ws, partial_stats=ps, partial_values=pv, **kw, **extra)
    _lib.call("anna_mi_gqa_decode_splitkv", ctypes.byref(args), _lib.stream_of(q))
    out_na = torch.full_like(q, float("nan"))
    na = fused_ops.decode_args(output=out_na, partial_stats=ps, partial_values=pv, **kw, **extra)
    na.partial_stats = _lib.View(None, 0, 0, 0, 0)
    na.partial_values = _lib.View(None, 0, 0, 0, 0)
    na.partial_capacity = 0
    na.query_rot = None
    _lib.call("anna_mi_gqa_decode_splitkv_noalloc", ctypes.byref(na), _lib.stream_of(q))
    torch.cuda.synchronize()
    return out_ws, out_na


def test_noalloc_matches_workspace_entry_point_twice(gpu):
    print("[case] no-alloc split-KV decode: B=8 L=4096+128 then B=2 L=300+5", flush=True)
    kw1, keep1 = _minmax_case(gpu, 8, 16, 2, 256, 4096, 128, 2, 32, 64, seed=1, gate=True)
    a, b = _both(gpu, kw1)
    assert torch.equal(a, b)
    kw2, keep2 = _minmax_case(gpu, 2, 8, 2, 128, 300, 5, 4, 16, 32, seed=2)
    a, b = _both(gpu, kw2)
    assert torch.equal(a, b)


def test_noalloc_tq_mse_keys_use_the_scratch_for_the_rotated_query(gpu):
    print("[case] no-alloc split-KV decode: TQ-MSE keys and values, two sizes", flush=True)
    for i, (b, qlen) in enumerate(((4, 700), (1, 64))):
        kw, keep = _mse_key_case(gpu, b, 8, 2, 128, qlen, 9, seed=10 + i)
        x, y = _both(gpu, kw)
        assert torch.equal(x, y)


def test_noalloc_rejects_a_workspace_beyond_the_scratch(gpu):
    cap = _lib.load().anna_mi_gqa_decode_splitkv_noalloc_capacity()
    assert cap == 32 << 20
    kw, keep = _minmax_case(gpu, 1, 16, 2, 256, 64, 1, 2, 32, 16, seed=3)
    kw = dict(kw)
    q = kw["query"]
    args = fused_ops.decode_args(output=torch.empty_like(q), partial_stats=torch.empty(1, 16, 1, 2, device=gpu),
                                 partial_values=torch.empty(1, 16, 1, 256, device=gpu), **kw)
    args.batch = 4096  # 4096 x 16 heads x 5 blocks x 258 x 4 B > 32 MiB: refused before any launch
    with pytest.raises(RuntimeError, match="exceeds the .* static scratch"):
        _lib.call("anna_mi_gqa_decode_splitkv_noalloc", ctypes.byref(args), _lib.stream_of(q))

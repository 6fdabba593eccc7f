"""Tiled int4 GEMV (xpu_int4_gemv_tiled) and the fused int4 LM-head top-k against the CPU
dequant path.  Shapes follow the reference's tests (test_fused_op_xpu.py:260-375): indices
exact, values within the reference's 2e-2; the GEMV within normwise relative error 1e-2."""

import pytest
import torch

from anna_amd import fused_ops
from anna_amd.quantization import XPUInt4Linear
from oracle import cpu_paths as cp
from tests._util import BF16_TOL, rel_err

pytestmark = pytest.mark.gpu


def quantized_linear(k, n, seed, device, group=32, dtype=torch.float16):
    torch.manual_seed(seed)
    dense = torch.nn.Linear(k, n, bias=False, dtype=torch.float32)
    return XPUInt4Linear.from_linear(dense, group_size=group, compute_dtype=dtype, device=device)


def dense_logits(q, x):
    w = cp.int4_dequant_f32(q.qweight.cpu(), q.qscale.cpu(), q.qzeros.cpu(), q.group_size, q.in_features)
    return x.cpu().double() @ w.double().t()


@pytest.mark.parametrize("k,n,seed,layout", [(16, 31, 0, "plain"), (64, 96, 8, "lm_head"), (96, 192, 5, "plain"),
                                             (2048, 1000, 3, "lm_head"),
                                             (128, 20000, 4, "lm_head"),    # rows split over chunks (V >= 8192)
                                             (64, 8193, 6, "plain")])
def test_lm_head_int4_topk_matches_quantized_reference(gpu, k, n, seed, layout):
    q = quantized_linear(k, n, seed, gpu)
    x = torch.randn(2, 3, k, device=gpu, dtype=torch.float16)
    if layout == "lm_head":
        q.prepare_lm_head_topk_layout()
        tensors = (q.lm_head_qweight, q.lm_head_qscale, q.lm_head_qzeros)
    else:
        tensors = (q.qweight, q.qscale, q.qzeros)
    values, indices = torch.ops.anna.lm_head_int4_topk_fused(x, *tensors, q.group_size, q.in_features, 5)
    assert values.shape == (2, 3, 5) and indices.dtype == torch.long
    ref = dense_logits(q, x.reshape(-1, k)).view(2, 3, n)
    rv, ri = torch.topk(ref, 5, dim=-1)
    assert torch.equal(indices.cpu(), ri)
    torch.testing.assert_close(values.cpu().double(), rv, atol=2e-2, rtol=2e-2)
    # the module forward picks the same top-k
    mv, mi = torch.topk(q(x), 5, dim=-1)
    assert torch.equal(indices, mi)


@pytest.mark.parametrize("k,n,seed,layout,rows", [(2048, 1000, 13, "lm_head", 1), (2048, 4096, 14, "lm_head", 4),
                                                  (128, 20000, 15, "lm_head", 1), (200, 300, 16, "plain", 3),
                                                  (64, 8193, 17, "plain", 2)])
def test_lm_head_topk_few_rows(gpu, k, n, seed, layout, rows):
    """One to four rows: the tiled GEMV's LDS-staged form (x and the tiles' scales and zero
    points staged once per workgroup); K = 200 leaves the staged x rows unaligned to 4 words."""
    q = quantized_linear(k, n, seed, gpu, group=32)
    x = torch.randn(rows, k, device=gpu, dtype=torch.float16)
    if layout == "lm_head":
        q.prepare_lm_head_topk_layout()
        tensors = (q.lm_head_qweight, q.lm_head_qscale, q.lm_head_qzeros)
    else:
        tensors = (q.qweight, q.qscale, q.qzeros)
    values, indices = torch.ops.anna.lm_head_int4_topk_fused(x, *tensors, q.group_size, q.in_features, 6)
    ref = dense_logits(q, x)
    rv, ri = torch.topk(ref, 6, dim=-1)
    assert torch.equal(indices.cpu(), ri)
    torch.testing.assert_close(values.cpu().double(), rv, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("tile,sdt,m,k,group", [(1, torch.float32, 1, 256, 64), (2, torch.bfloat16, 3, 256, 64),
                                                (4, torch.float16, 5, 256, 64), (8, torch.float32, 2, 256, 64),
                                                (4, torch.bfloat16, 4, 200, 32), (8, torch.bfloat16, 1, 4096, 128)])
def test_xpu_int4_gemv_tiled_matches_dequant(gpu, tile, sdt, m, k, group):
    q = quantized_linear(k, 200, 11 + tile, gpu, group=group, dtype=torch.bfloat16)
    n, pc = q.qweight.shape
    n_pad = -(-n // tile) * tile
    qw = torch.zeros((n_pad, pc), dtype=torch.int32, device=gpu)
    qw[:n] = q.qweight
    qs = torch.ones((q.qscale.shape[0], n_pad), dtype=sdt, device=gpu)
    qs[:, :n] = q.qscale.to(sdt)
    qz = torch.full((q.qzeros.shape[0], n_pad), 8, dtype=torch.int8, device=gpu)
    qz[:, :n] = q.qzeros
    qw_t = qw.view(n_pad // tile, tile, pc).permute(0, 2, 1).contiguous()
    x = torch.randn(m, k, device=gpu, dtype=torch.bfloat16)
    y = torch.ops.anna.xpu_int4_gemv_tiled(x, qw_t, qs.view(-1, n_pad // tile, tile), qz.view(-1, n_pad // tile, tile),
                                           group, k, n)
    assert y.shape == (m, n) and y.dtype == torch.bfloat16
    w = cp.int4_dequant_f32(q.qweight.cpu(), q.qscale.to(sdt).cpu(), q.qzeros.cpu(), group, k)
    ref = x.cpu().double() @ w.double().t()
    assert rel_err(y.cpu().double().numpy(), ref.numpy()) <= BF16_TOL


def test_lm_head_topk_errors(gpu):
    q = quantized_linear(16, 31, 0, gpu)
    x = torch.randn(1, 16, device=gpu, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="top_k"):
        fused_ops.run_lm_head_int4_topk_fused(hidden_states=x, qweight=q.qweight, qscale=q.qscale, qzeros=q.qzeros,
                                              group_size=32, in_features=16, top_k=40)
    with pytest.raises(RuntimeError, match="in_features"):
        fused_ops.run_lm_head_int4_topk_fused(hidden_states=x, qweight=q.qweight, qscale=q.qscale, qzeros=q.qzeros,
                                              group_size=32, in_features=8, top_k=3)


@pytest.mark.parametrize("v,rows,k", [(31, 1, 5), (5000, 3, 8), (20000, 2, 16), (3000, 1, 32), (40, 2, 32)])
def test_topk_rows_exact_with_ties(gpu, v, rows, k):
    """The row top-k (both kernels: k <= 8 in registers, k > 8 in LDS) against a CPU sort by
    (value descending, index ascending), with many exact ties."""
    from anna_amd import _lib
    print(f"[case] topk_rows V={v} rows={rows} k={k}", flush=True)
    g = torch.Generator().manual_seed(v + k)
    vals = torch.randn(rows, v, generator=g)
    vals[:, ::7] = vals[:, :1]  # every 7th value ties with the first
    dev_vals = vals.to(gpu)
    out_v = torch.empty((rows, k), dtype=torch.float32, device=gpu)
    out_i = torch.empty((rows, k), dtype=torch.int64, device=gpu)
    _lib.call("anna_mi_topk_rows", dev_vals.data_ptr(), rows, v, v, k, out_v.data_ptr(), _lib.dtype_code(torch.float32),
              out_i.data_ptr(), _lib.stream_of(dev_vals))
    for r in range(rows):
        order = sorted(range(v), key=lambda i: (-float(vals[r, i]), i))[:k]
        assert out_i[r].cpu().tolist() == order
        assert torch.equal(out_v[r].cpu(), vals[r, order])


@pytest.mark.parametrize("layout", ["lm_head", "plain"])
def test_lm_head_topk_exact_ties_in_wave_path(gpu, layout):
    """Few long rows take the wave-level top-k (chunk lists and a head tournament across lanes):
    with every weight row duplicated 6144 rows later, each logit ties exactly with its twin, and
    the pairs must come out value-descending, lower index first."""
    torch.manual_seed(99)
    dense = torch.nn.Linear(256, 12288, bias=False, dtype=torch.float32)
    with torch.no_grad():
        dense.weight[6144:] = dense.weight[:6144]
    q = XPUInt4Linear.from_linear(dense, group_size=32, compute_dtype=torch.float16, device=gpu)
    x = torch.randn(2, 256, device=gpu, dtype=torch.float16)
    if layout == "lm_head":
        q.prepare_lm_head_topk_layout()
        tensors = (q.lm_head_qweight, q.lm_head_qscale, q.lm_head_qzeros)
    else:
        tensors = (q.qweight, q.qscale, q.qzeros)
    values, indices = torch.ops.anna.lm_head_int4_topk_fused(x, *tensors, q.group_size, q.in_features, 8)
    ref = dense_logits(q, x)
    for r in range(2):
        order = sorted(range(12288), key=lambda i: (-float(ref[r, i]), i))[:8]
        assert indices[r].cpu().tolist() == order
        got = values[r].float().cpu()
        assert torch.equal(got[0::2], got[1::2])  # twins carry the same value

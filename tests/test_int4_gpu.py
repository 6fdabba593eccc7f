"""Parity of the HIP int4 path against the CPU oracle (through the C ABI / anna:: ops).

Packing, repacking and dequant are integer/exact work: bit-exact.  Linear outputs:
normwise max relative error <= 1e-2 against the oracle's x_bf16 @ bf16(dequant(W))^T
(the reference CPU path, quantization.py:645-648).
"""

import numpy as np
import pytest
import torch

from anna_amd import fused_ops
from anna_amd.quantization import XPUInt4Linear
from oracle import oracle as orc
from tests._util import BF16_TOL, int4_payload, rel_err

pytestmark = pytest.mark.gpu


def _dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _x_tensor(bits_u16, dtype, device):
    t = torch.from_numpy(bits_u16.view(np.int16)).view(torch.bfloat16).to(device)
    return t.to(dtype)


LINEAR_CASES = [
    # (M, K, N, group, scale dtype)
    (1, 2048, 6144, 128, "bf16"),   # benchmark config 1
    (1, 4096, 512, 128, "fp32"),
    (2, 256, 100, 128, "fp32"),     # N tail
    (8, 4096, 384, 128, "bf16"),
    (16, 1024, 64, 128, "fp32"),
    (3, 384, 48, 128, "fp32"),      # K = 3 blocks, odd block count per wave
    (17, 512, 130, 128, "fp32"),    # GEMM path, M and N tails
    (64, 1024, 256, 128, "bf16"),
    (130, 256, 200, 128, "fp32"),
    (5, 96, 40, 32, "fp32"),        # group 32: generic kernel
    (1, 96, 40, 32, "fp32"),        # group 32 on the dot2 GEMV, partial k-slice
    (2, 9216, 72, 128, "bf16"),     # dot2 GEMV with more k-slices than waves
    (1, 4096, 12288, 128, "bf16"),  # benchmark config 2, M = 1
    (1, 512, 102, 128, "bf16"),     # dot2 GEMV, N % 4 != 0: per-row scale / zero loads
    (2, 1024, 37, 128, "fp32"),     # the same with fp32 scales, M = 2
    (1, 1024, 4100, 128, "fp32"),   # dot2 GEMV, fp32 scales as one 16-byte load
    (300, 512, 400, 64, "bf16"),    # tiled GEMM: group 64, M and N tails
    (2048, 4096, 192, 128, "bf16"), # tiled GEMM at the config-2 M and K
    (64, 4096, 6144, 128, "fp32"),  # tiled GEMM, config-2 N = 6144 at M = 64
    (8, 512, 12200, 128, "bf16"),   # MFMA GEMV, three 16-row tiles per wave, N tail
    (4, 1024, 8000, 128, "fp32"),   # MFMA GEMV, two tiles
    (8, 512, 2000, 128, "bf16"),    # MFMA GEMV, one tile
    (48, 4096, 3000, 128, "bf16"),  # MFMA GEMV over three 16-row groups of x (N tail)
    (20, 2048, 4200, 128, "fp32"),  # two row groups, two tiles, four-wave K split
    (40, 8192, 200, 128, "bf16"),   # 16 < M < 64 with K past the row-group GEMV: tiled GEMM
]


@pytest.mark.parametrize("m,k,n,group,sdt", LINEAR_CASES)
def test_int4_linear_matches_oracle(gpu, m, k, n, group, sdt):
    print(f"[case] int4_linear M={m} K={k} N={n} g={group} scale={sdt}", flush=True)
    rng = np.random.default_rng(m * 1000 + k + n)
    qw, qs, qz = int4_payload(rng, n, k, group, scale_dtype=sdt)
    xb = orc.bf16_bits(rng.normal(size=(m, k)).astype(np.float32))
    ref = orc.int4_linear(xb, qw, qs, qz, group)
    qs_t = _dev(qs, gpu).to(torch.bfloat16 if sdt == "bf16" else torch.float32)
    x = _x_tensor(xb, torch.bfloat16, gpu)
    y = torch.ops.anna.xpu_int4_gemv(x, _dev(qw, gpu), qs_t, _dev(qz, gpu), group, k)
    assert y.dtype == torch.bfloat16 and y.shape == (m, n)
    assert rel_err(y.float().cpu().numpy(), ref) <= BF16_TOL


@pytest.mark.parametrize("rg", ["1", "2", "4"])
@pytest.mark.parametrize("m,k,n,sdt", [(1, 4096, 1000, "bf16"), (2, 2048, 998, "fp32"), (1, 8192, 300, "f16"),
                                       (2, 512, 36, "bf16")])
def test_int4_gemv_dot2_row_groups(gpu, monkeypatch, rg, m, k, n, sdt):
    """The M <= 2 GEMV with 1, 2 or 4 row groups per lane (N tails, N % 4 != 0, two passes at K = 8192)."""
    print(f"[case] int4 dot2 RG={rg} M={m} K={k} N={n} scale={sdt}", flush=True)
    monkeypatch.setenv("ANNA_MI_INT4_DOT2_RG", rg)
    rng = np.random.default_rng(m * 7 + k + n)
    qw, qs, qz = int4_payload(rng, n, k, 128, scale_dtype="fp32" if sdt == "fp32" else "bf16")
    xb = orc.bf16_bits(rng.normal(size=(m, k)).astype(np.float32))
    ref = orc.int4_linear(xb, qw, qs, qz, 128)
    sd = {"bf16": torch.bfloat16, "fp32": torch.float32, "f16": torch.float16}[sdt]
    qs_t = _dev(qs, gpu).to(sd)
    x = _x_tensor(xb, torch.bfloat16, gpu)
    y = torch.ops.anna.xpu_int4_gemv(x, _dev(qw, gpu), qs_t, _dev(qz, gpu), 128, k)
    assert rel_err(y.float().cpu().numpy(), ref) <= BF16_TOL


@pytest.mark.parametrize("tile", ["L", "M", "S"])
@pytest.mark.parametrize("m,k,n,group,sdt", [(300, 512, 400, 64, "bf16"), (2048, 1024, 200, 128, "fp32"),
                                             (64, 1024, 96, 128, "bf16"), (257, 256, 1000, 128, "bf16"),
                                             (100, 320, 200, 64, "bf16"),   # odd k-step count (5)
                                             (70, 64, 96, 64, "fp32")])     # a single k-step
def test_int4_gemm_every_tile_shape(gpu, monkeypatch, tile, m, k, n, group, sdt):
    """The tiled GEMM's three tile shapes (chosen by size in production), each forced."""
    print(f"[case] int4 tiled GEMM tile={tile} M={m} K={k} N={n} g={group} scale={sdt}", flush=True)
    monkeypatch.setenv("ANNA_MI_INT4_GEMM_TILE", tile)
    rng = np.random.default_rng(m * 7 + k + n)
    qw, qs, qz = int4_payload(rng, n, k, group, scale_dtype=sdt)
    xb = orc.bf16_bits(rng.normal(size=(m, k)).astype(np.float32))
    ref = orc.int4_linear(xb, qw, qs, qz, group)
    qs_t = _dev(qs, gpu).to(torch.bfloat16 if sdt == "bf16" else torch.float32)
    x = _x_tensor(xb, torch.bfloat16, gpu)
    y = torch.ops.anna.xpu_int4_gemv(x, _dev(qw, gpu), qs_t, _dev(qz, gpu), group, k)
    assert rel_err(y.float().cpu().numpy(), ref) <= BF16_TOL


@pytest.mark.parametrize("m,n", [(256, 6144), (256, 12288), (2048, 6144), (2048, 12288)])
def test_int4_gemm_config2_bench_sizes(gpu, monkeypatch, m, n):
    """BASELINE config 2's large-M points (K = 4096, group 128, bf16 scales) at exactly the grid
    sizes the bench times, with the production tile choice.  The oracle checks 64 random output
    columns over every row and 16 random full rows (<= 0.8 GMAC of fp64 work)."""
    monkeypatch.delenv("ANNA_MI_INT4_GEMM_TILE", raising=False)
    k, group = 4096, 128
    print(f"[case] int4 GEMM config-2 M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(m + n)
    qw, qs, qz = int4_payload(rng, n, k, group, scale_dtype="bf16")
    xb = orc.bf16_bits(rng.normal(size=(m, k)).astype(np.float32))
    x = _x_tensor(xb, torch.bfloat16, gpu)
    y = torch.ops.anna.xpu_int4_gemv(x, _dev(qw, gpu), _dev(qs, gpu).to(torch.bfloat16), _dev(qz, gpu), group, k)
    torch.cuda.synchronize()
    y = y.float().cpu().numpy()
    cols = np.sort(rng.choice(n, size=64, replace=False))
    ref_c = orc.int4_linear(xb, qw[cols], qs[:, cols], qz[:, cols], group)
    assert rel_err(y[:, cols], ref_c) <= BF16_TOL
    rows = np.sort(rng.choice(m, size=16, replace=False))
    ref_r = orc.int4_linear(np.ascontiguousarray(xb[rows]), qw, qs, qz, group)
    assert rel_err(y[rows], ref_r) <= BF16_TOL
    # every column of every row is finite and non-trivial (no unwritten tile)
    assert np.isfinite(y).all() and (np.abs(y).max(axis=0) > 0).all()


@pytest.mark.parametrize("m,k,n,sdt,xdt,stride", [
    (64, 4096, 6144, "bf16", "bf16", 0),     # BASELINE config 2 at M = 64: 128 row blocks x 2 m-blocks
    (33, 1024, 1000, "fp32", "f16", 0),      # one 128-k block per wave, partial m-block and row block
    (17, 2048, 96, "bf16", "bf16", 0),       # one row block, a 1-row second m-block
    (64, 1152, 200, "bf16", "f16", 0),       # 9 blocks over 8 waves: one wave takes two
    (50, 12288, 300, "fp32", "bf16", 0),     # 12 blocks per wave: three passes of four
    (40, 2048, 500, "bf16", "bf16", 2560),   # strided x rows
])
def test_int4_skinny_gemm(gpu, m, k, n, sdt, xdt, stride):
    """The skinny GEMM (16 < M <= 64, group 128, K >= 1024, at most 256 workgroups): 32 rows of x
    per workgroup against 48 rows of W, K split over the waves, W copied into LDS by whole lines,
    "off + q" MFMA fragments with the zero point removed per group."""
    print(f"[case] int4 skinny GEMM M={m} K={k} N={n} scale={sdt} x={xdt} stride={stride}", flush=True)
    group = 128
    rng = np.random.default_rng(m * 31 + k + n)
    qw, qs, qz = int4_payload(rng, n, k, group, scale_dtype=sdt)
    cols = stride or k
    xb = orc.bf16_bits(rng.normal(size=(m, cols)).astype(np.float32))
    ref = orc.int4_linear(np.ascontiguousarray(xb[:, :k]), qw, qs, qz, group)
    tdt = torch.bfloat16 if xdt == "bf16" else torch.float16
    x = _x_tensor(xb, tdt, gpu)[:, :k]
    qs_t = _dev(qs, gpu).to(torch.bfloat16 if sdt == "bf16" else torch.float32)
    out = torch.empty((m, n), dtype=tdt, device=gpu)
    fused_ops.int4_linear_out(x, _dev(qw, gpu), qs_t, _dev(qz, gpu), group, k, out)
    assert rel_err(out.float().cpu().numpy(), ref) <= BF16_TOL


@pytest.mark.parametrize("xdt", [torch.float16, torch.float32])
@pytest.mark.parametrize("m", [1, 4, 128])
def test_int4_linear_other_activation_dtypes(gpu, xdt, m):
    rng = np.random.default_rng(7)
    k, n, group = 1024, 192, 128
    qw, qs, qz = int4_payload(rng, n, k, group, scale_dtype="fp32")
    xb = orc.bf16_bits(rng.normal(size=(m, k)).astype(np.float32))
    ref = orc.int4_linear(xb, qw, qs, qz, group)
    x = _x_tensor(xb, xdt, gpu)
    y = torch.ops.anna.xpu_int4_gemv(x, _dev(qw, gpu), _dev(qs, gpu), _dev(qz, gpu), group, k)
    assert y.dtype == xdt
    assert rel_err(y.float().cpu().numpy(), ref) <= BF16_TOL


def test_int4_linear_strided_rows(gpu):
    rng = np.random.default_rng(8)
    m, k, n, group = 3, 512, 64, 128
    qw, qs, qz = int4_payload(rng, n, k, group, scale_dtype="fp32")
    xb = orc.bf16_bits(rng.normal(size=(m, 2 * k)).astype(np.float32))
    ref = orc.int4_linear(np.ascontiguousarray(xb[:, :k]), qw, qs, qz, group)
    x = _x_tensor(xb, torch.bfloat16, gpu)[:, :k]
    assert not x.is_contiguous()
    out = torch.empty((m, n), dtype=torch.bfloat16, device=gpu)
    fused_ops.int4_linear_out(x, _dev(qw, gpu), _dev(qs, gpu), _dev(qz, gpu), group, k, out)
    assert rel_err(out.float().cpu().numpy(), ref) <= BF16_TOL


@pytest.mark.parametrize("rounding", ["half_even", "half_away"])
def test_int4_quantize_bit_exact(gpu, rounding):
    rng = np.random.default_rng(9)
    n, k, group = 40, 300, 32
    kp = XPUInt4Linear._padded_in_features(k, group)
    w = rng.normal(size=(n, k)).astype(np.float32)
    w[0, :8] = [7.0, 0.5, 1.5, -0.5, -7.0, 2.5, -2.5, 0.0]  # exact ties at scale 1
    w[1] = 0.0
    ref = orc.int4_quantize(w, group, kp, rounding=0 if rounding == "half_even" else 1)
    got = fused_ops.int4_quantize(_dev(w, gpu), group_size=group, padded_in_features=kp, rounding=rounding)
    for a, b in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), b)


def test_int4_quantize_bf16_weight_bit_exact(gpu):
    rng = np.random.default_rng(10)
    n, k, group = 16, 256, 128
    wb = orc.bf16_bits(rng.normal(size=(n, k)).astype(np.float32))
    ref = orc.int4_quantize(orc.bf16_to_f32(wb), group, k)
    got = fused_ops.int4_quantize(_x_tensor(wb, torch.bfloat16, gpu), group_size=group, padded_in_features=k)
    for a, b in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), b)


def test_autoround_repack_bit_exact(gpu):
    rng = np.random.default_rng(11)
    k, n, group, kp = 200, 24, 64, 256
    g = -(-k // group)
    codes = rng.integers(0, 16, size=(-(-k // 8) * 8, n))
    v = codes.reshape(-1, 8, n).astype(np.int64)
    words = (v << (4 * np.arange(8))[None, :, None]).sum(1)
    gq = np.where(words >= 2**31, words - 2**32, words).astype(np.int32)
    zeros = rng.integers(0, 15, size=(g, n))
    zw = (zeros.reshape(g, n // 8, 8).astype(np.int64) << (4 * np.arange(8))).sum(-1)
    gz = np.where(zw >= 2**31, zw - 2**32, zw).astype(np.int32)
    sc = orc.f16_bits(rng.uniform(0.01, 0.1, size=(g, n)).astype(np.float32))
    ref = orc.autoround_to_int4(gq, gz, sc, k, n, group, kp)
    got = fused_ops.autoround_to_int4(_dev(gq, gpu), _dev(gz, gpu), _dev(sc.view(np.int16), gpu).view(torch.float16),
                                      in_features=k, out_features=n, group_size=group, padded_in_features=kp)
    for a, b in zip(got, ref):
        np.testing.assert_array_equal(a.cpu().numpy(), b)


def test_int4_dequant_exact(gpu):
    rng = np.random.default_rng(12)
    n, k, group = 33, 384, 128
    qw, qs, qz = int4_payload(rng, n, k, group, scale_dtype="fp32")
    ref = orc.int4_dequant(qw, qs, qz, k, group)
    got = fused_ops.int4_dequant(_dev(qw, gpu), _dev(qs, gpu), _dev(qz, gpu), group, k, out_dtype=torch.float32)
    np.testing.assert_array_equal(got.cpu().numpy(), ref)


def test_module_from_linear_and_forward(gpu):
    torch.manual_seed(13)
    dense = torch.nn.Linear(1000, 96, bias=True)
    mod = XPUInt4Linear.from_linear(dense, group_size=128, compute_dtype=torch.bfloat16, device=gpu)
    assert mod.padded_in_features == 1024 and mod.qweight.shape == (96, 128)
    w = dense.weight.detach().numpy()
    qw, qs, qz = orc.int4_quantize(w, 128, 1024)
    np.testing.assert_array_equal(mod.qweight.cpu().numpy(), qw)
    np.testing.assert_array_equal(mod.qscale.cpu().numpy(), qs)
    x = torch.randn(2, 3, 1000)
    xb = orc.bf16_bits(x.reshape(6, 1000).numpy())
    ref = orc.int4_linear(xb, qw, qs, qz, 128) + orc.bf16_to_f32(orc.bf16_bits(dense.bias.detach().numpy()))
    y = mod(x.to(gpu).to(torch.bfloat16))
    assert y.shape == (2, 3, 96)
    assert rel_err(y.float().cpu().reshape(6, 96).numpy(), ref) <= BF16_TOL

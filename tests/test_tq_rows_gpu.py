"""The general batched TurboQuant cache (TurboQuantRowsCache: head_dim 64..512, bits 2..4)
against the oracle.

Packed key codes and norms are bit-exact with the oracle's Hadamard quantizer, packed values
bit-exact with the oracle's min/max group quantizer, the ring holds exactly the newest min(L, R)
tokens, and the attention output is within normwise max relative error 1e-2 of the oracle's
fp64 attention over the dequantized prefix plus the dense window (times sigmoid(gate) where
given) -- after loading and after every step of an append + decode loop.
"""

import numpy as np
import pytest
import torch

from anna_amd.tq_cache import TurboQuantBatchCache, TurboQuantRowsCache
from oracle import oracle as orc
from tests._util import BF16_TOL, rel_err

pytestmark = pytest.mark.gpu


def bits_of(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def np_dequant(codes: np.ndarray, norms_bits: np.ndarray, rot: np.ndarray, cent: np.ndarray, bits: int) -> np.ndarray:
    """x_hat = |x|_fp16 * R^T c[code] (fp64); codes [n, D*sb/8] with element i at bits sb*(i % per)
    of byte i / per (sb = 2 for 2-bit codes, else 4)."""
    sb = 2 if bits == 2 else 4
    per = 8 // sb
    n = codes.shape[0]
    c = np.stack([(codes >> (sb * e)) & ((1 << sb) - 1) for e in range(per)], -1).reshape(n, -1)
    return (cent.astype(np.float64)[c] @ rot) * orc.f16_to_f32(norms_bits).astype(np.float64)[:, None]


def check_rows(cache, hist_k, hist_v, q, out, gate=None):
    R, bits, gs = cache.residual_capacity, cache.bits, cache.value_group_size
    signs = cache.qn.signs.cpu().numpy()
    rot = orc.tq_hadamard_matrix(signs)
    cent = cache.qn.centroids.cpu().numpy()
    thr = cache.qn.thresholds.cpu().numpy()
    assert cache.seq_lengths.cpu().tolist() == [k.shape[1] for k in hist_k] == cache.lengths
    kc, kn = cache.key_codes.cpu().numpy(), bits_of(cache.key_norms)
    vd, vs, vz = cache.value_data.cpu().numpy(), bits_of(cache.value_scales), bits_of(cache.value_zeros)
    rk, rv = cache.residual_key.cpu(), cache.residual_value.cpu()
    out = out.float().cpu().numpy()
    for b in range(cache.batch):
        L = hist_k[b].shape[1]
        ql = max(0, L - R)
        if L == 0:
            assert not out[b].any()
            continue
        hk, hv = hist_k[b].cpu(), hist_v[b].cpu()
        kk, vv = [], []
        for h in range(cache.kv_heads):
            parts_k, parts_v = [], []
            if ql > 0:
                oc, on = orc.tq_hadamard_quantize(np.ascontiguousarray(bits_of(hk[h, :ql])), orc.BF16, signs, thr, bits)
                np.testing.assert_array_equal(kc[b, h, :ql], oc)
                np.testing.assert_array_equal(kn[b, h, :ql], on)
                od, os_, oz = orc.tq_values_quantize(np.ascontiguousarray(bits_of(hv[h:h + 1, :ql])), orc.BF16, bits, gs)
                np.testing.assert_array_equal(vd[b, h, :ql], od[0])
                np.testing.assert_array_equal(vs[b, h, :ql], os_[0])
                np.testing.assert_array_equal(vz[b, h, :ql], oz[0])
                parts_k.append(np_dequant(kc[b, h, :ql], kn[b, h, :ql], rot, cent, bits))
                parts_v.append(orc.tq_values_dequant(od, os_, oz, orc.BF16, bits, gs)[0].astype(np.float64))
            slots = np.arange(ql, L) % R
            np.testing.assert_array_equal(bits_of(rk[b, h][slots]), bits_of(hk[h, ql:]))
            np.testing.assert_array_equal(bits_of(rv[b, h][slots]), bits_of(hv[h, ql:]))
            parts_k.append(hk[h, ql:].double().numpy())
            parts_v.append(hv[h, ql:].double().numpy())
            kk.append(np.concatenate(parts_k))
            vv.append(np.concatenate(parts_v))
        g = None if gate is None else gate[b].float().cpu().numpy()
        ref = orc.gqa_decode(q[b].float().cpu().numpy(), np.stack(kk), np.stack(vv), cache.head_dim ** -0.5, g)
        assert rel_err(out[b], ref) <= BF16_TOL, b


@pytest.mark.parametrize("d,bits,gated,hkv,g", [(128, 2, False, 2, 8), (64, 3, True, 2, 8), (256, 3, False, 2, 8),
                                                (256, 4, True, 2, 8), (512, 2, False, 2, 8), (128, 4, False, 16, 2),
                                                (64, 2, True, 11, 1)])
def test_rows_cache_load_append_decode(gpu, d, bits, gated, hkv, g):
    """Three sequences (75 / 20 / 0 tokens, a 32-token window), decoded, then 12 steps of
    append + decode: sequence 0 evicts a token every step, sequence 1 fills its window and
    starts evicting, sequence 2 grows from empty.  Up to 8 KV heads take one wave pair each in
    the append; 11 and 16 heads loop those waves over the heads."""
    print(f"[case] tq rows d={d} bits={bits} gate={gated} hkv={hkv} g={g}", flush=True)
    torch.manual_seed(90 + d + bits + hkv)
    R, steps = 32, 12
    lens = [75, 20, 0]
    cache = TurboQuantBatchCache(batch=3, kv_heads=hkv, q_heads=hkv * g, capacities=[80, 40, 16],
                                 residual_capacity=R, head_dim=d, bits=bits, device=gpu)
    assert isinstance(cache, TurboQuantRowsCache)
    keys = [torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16) for L in lens]
    vals = [torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16) for L in lens]
    for b in range(3):
        cache.load_sequence(b, keys[b], vals[b])
    scale = d ** -0.5
    for step in range(steps + 1):
        if step > 0:
            nk = torch.randn(3, hkv, d, device=gpu).to(torch.bfloat16)
            nv = torch.randn(3, hkv, d, device=gpu).to(torch.bfloat16)
            cache.append(nk, nv)
            keys = [torch.cat([keys[b], nk[b][:, None]], 1) for b in range(3)]
            vals = [torch.cat([vals[b], nv[b][:, None]], 1) for b in range(3)]
        q = torch.randn(3, hkv * g, d, device=gpu).to(torch.bfloat16)
        gate = torch.randn(3, hkv * g, d, device=gpu).to(torch.bfloat16) if gated else None
        out = cache.decode(q, scaling=scale, gate=gate)
        if step in (0, 1, 7, steps):
            check_rows(cache, keys, vals, q, out, gate)
    assert int(cache.overflow.item()) == 0


@pytest.mark.parametrize("d,bits", [(64, 2), (128, 4), (256, 3)])
def test_rows_cache_slots_past_the_lengths_are_never_read_into_the_output(gpu, d, bits):
    """Slots past each row's length hold whatever the memory held before (here NaN in the value
    scales and zeros, the key norms and the window rows past the ring's fill): the decode must
    not let them into the output (a zero probability times NaN is NaN)."""
    print(f"[case] tq rows stale slots d={d} bits={bits}", flush=True)
    torch.manual_seed(700 + d + bits)
    hkv, g, R = 2, 8, 32
    lens = [300, 70, 9]
    cache = TurboQuantBatchCache(batch=3, kv_heads=hkv, q_heads=hkv * g, capacities=[400, 400, 400],
                                 residual_capacity=R, head_dim=d, bits=bits, device=gpu)
    assert isinstance(cache, TurboQuantRowsCache)
    keys = [torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16) for L in lens]
    vals = [torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16) for L in lens]
    for b in range(3):
        cache.load_sequence(b, keys[b], vals[b])
    nan = float("nan")
    for b, L in enumerate(lens):
        ql = max(0, L - R)
        cache.value_scales[b, :, ql:] = nan
        cache.value_zeros[b, :, ql:] = nan
        cache.key_norms[b, :, ql:] = nan
        cache.value_data[b, :, ql:] = 0xFF
        if L < R:
            cache.residual_value[b, :, L:] = nan
            cache.residual_key[b, :, L:] = nan
    q = torch.randn(3, hkv * g, d, device=gpu).to(torch.bfloat16)
    out = cache.decode(q, scaling=d ** -0.5)
    assert torch.isfinite(out.float()).all()
    check_rows(cache, keys, vals, q, out)


def test_rows_cache_full_sequence_refused(gpu):
    print("[case] tq rows full sequence", flush=True)
    cache = TurboQuantBatchCache(batch=1, kv_heads=1, q_heads=2, capacities=[2], residual_capacity=4, head_dim=128,
                                 bits=4, device=gpu)
    kv = torch.randn(1, 1, 128, device=gpu).to(torch.bfloat16)
    for _ in range(6):
        cache.append(kv, kv)
    with pytest.raises(RuntimeError, match="full"):
        cache.append(kv, kv)
    assert cache.lengths == [6] and int(cache.seq_lengths.item()) == 6


def test_rows_cache_graph_replay(gpu):
    """append + decode captured once and replayed: the lengths advance on the device and every
    replay matches the eager result of the same step."""
    print("[case] tq rows graph replay", flush=True)
    torch.manual_seed(97)
    hkv, g, d, R = 2, 4, 128, 16

    def make():
        c = TurboQuantBatchCache(batch=2, kv_heads=hkv, q_heads=hkv * g, capacities=[64, 64], residual_capacity=R,
                                 head_dim=d, bits=3, device=gpu)
        for b, L in enumerate((30, 9)):
            gen = torch.Generator(device=gpu).manual_seed(100 + b)
            k = torch.randn(hkv, L, d, device=gpu, generator=gen).to(torch.bfloat16)
            v = torch.randn(hkv, L, d, device=gpu, generator=gen).to(torch.bfloat16)
            c.load_sequence(b, k, v)
        return c

    eager, graphed = make(), make()
    nk = torch.randn(2, hkv, d, device=gpu).to(torch.bfloat16)
    nv = torch.randn(2, hkv, d, device=gpu).to(torch.bfloat16)
    q = torch.randn(2, hkv * g, d, device=gpu).to(torch.bfloat16)
    out_g = torch.empty_like(q)
    graphed.decode(q, scaling=d ** -0.5, out=out_g)  # sizes the partials outside the capture
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            graphed.append(nk, nv)
            graphed.decode(q, scaling=d ** -0.5, out=out_g)
    torch.cuda.current_stream().wait_stream(stream)
    for step in range(4):
        graph.replay()
        torch.cuda.synchronize()
        graphed.lengths = [n + 1 for n in graphed.lengths]
        eager.append(nk, nv)
        ref = eager.decode(q, scaling=d ** -0.5)
        torch.cuda.synchronize()
        assert graphed.seq_lengths.cpu().tolist() == eager.seq_lengths.cpu().tolist(), step
        assert torch.equal(out_g, ref), step


@pytest.mark.parametrize("d", [64, 256, 512])
def test_rows_cache_hadamard_query_rotation_matches_dense(gpu, d):
    """The query rotation by the fast Walsh-Hadamard transform (the quantizer's sign vector
    passed as rotation_signs) gives the attention of the dense D x D rotation: the same cache
    decoded both ways agrees within the bf16 output tolerance (both rotations are fp32; they
    differ only in summation order)."""
    print(f"[case] tq rows query rotation d={d}", flush=True)
    torch.manual_seed(31 + d)
    hkv, g, R = 2, 4, 16
    cache = TurboQuantBatchCache(batch=2, kv_heads=hkv, q_heads=hkv * g, capacities=[48, 48], residual_capacity=R,
                                 head_dim=d, bits=4, device=gpu)
    for b, L in enumerate((50, 17)):
        cache.load_sequence(b, torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16),
                            torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16))
    q = torch.randn(2, hkv * g, d, device=gpu).to(torch.bfloat16)
    fast = cache.decode(q, scaling=d ** -0.5).float()
    signs = cache.qn.signs
    try:
        cache.qn.signs = None  # no rotation_signs: the dense product
        dense = cache.decode(q, scaling=d ** -0.5).float()
    finally:
        cache.qn.signs = signs
    assert rel_err(fast.cpu().numpy(), dense.cpu().numpy()) <= 1e-2


@pytest.mark.parametrize("d,bits", [(128, 4), (64, 2)])
def test_rows_cache_value_group_16_takes_the_valu_split(gpu, d, bits):
    """Value groups of 16 dims are not whole 32-dim spans, which the MFMA split kernel's raw value
    staging needs: the decode runs on the VALU split kernel instead, and still matches the
    oracle after loading and after appends."""
    print(f"[case] tq rows group 16 d={d} bits={bits}", flush=True)
    torch.manual_seed(1600 + d + bits)
    hkv, g, R = 2, 4, 16
    lens = [90, 23]
    cache = TurboQuantRowsCache(batch=2, kv_heads=hkv, q_heads=hkv * g, capacities=[96, 96], residual_capacity=R,
                                head_dim=d, bits=bits, device=gpu, value_group_size=16)
    keys = [torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16) for L in lens]
    vals = [torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16) for L in lens]
    for b in range(2):
        cache.load_sequence(b, keys[b], vals[b])
    for step in range(3):
        if step > 0:
            nk = torch.randn(2, hkv, d, device=gpu).to(torch.bfloat16)
            nv = torch.randn(2, hkv, d, device=gpu).to(torch.bfloat16)
            cache.append(nk, nv)
            keys = [torch.cat([keys[b], nk[b][:, None]], 1) for b in range(2)]
            vals = [torch.cat([vals[b], nv[b][:, None]], 1) for b in range(2)]
        q = torch.randn(2, hkv * g, d, device=gpu).to(torch.bfloat16)
        out = cache.decode(q, scaling=d ** -0.5)
        check_rows(cache, keys, vals, q, out)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_rows_cache_query_rotation_in_the_split_is_bit_exact(gpu, d):
    """With 16-byte aligned Hadamard signs the MFMA split kernel rotates the query itself; with
    signs that are not (a view one float into a buffer) the separate rotation launch does.  Both
    follow the same operation order, so the decode outputs are identical bit for bit."""
    print(f"[case] tq rows in-split rotation d={d}", flush=True)
    torch.manual_seed(2700 + d)
    hkv, g, R = 2, 8, 32
    cache = TurboQuantRowsCache(batch=2, kv_heads=hkv, q_heads=hkv * g, capacities=[200, 200], residual_capacity=R,
                                head_dim=d, bits=4, device=gpu)
    for b, L in enumerate((190, 57)):
        cache.load_sequence(b, torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16),
                            torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16))
    q = torch.randn(2, hkv * g, d, device=gpu).to(torch.bfloat16)
    in_split = cache.decode(q, scaling=d ** -0.5).clone()
    signs = cache.qn.signs
    buf = torch.empty(d + 1, dtype=signs.dtype, device=gpu)
    buf[1:] = signs
    assert buf[1:].data_ptr() % 16 != 0
    try:
        cache.qn.signs = buf[1:]
        launched = cache.decode(q, scaling=d ** -0.5).clone()
    finally:
        cache.qn.signs = signs
    assert torch.equal(in_split.view(torch.int16), launched.view(torch.int16))

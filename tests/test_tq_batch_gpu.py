"""Batched varlen TQ decode and append (the one-launch MFMA path) against the oracle.

Pool codes and norms are bit-exact with the oracle's Hadamard quantizer (values after undoing
the 32-token blocking), the ring holds exactly the newest min(L, R) tokens, and the attention
output is within normwise max relative error 1e-2 of the oracle's fp64 attention (times
sigmoid(gate) where given) over the dequantized pool plus the dense window.
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
    """[tokens/32][2048] blocked value codes -> natural [tokens][64] (loop restatement)."""
    out = np.zeros((tokens, 64), np.uint8)
    for blk in range(tokens // 32):
        for t in range(32):
            kq, half, e = (t % 16) // 4, t // 16, t % 4
            for dim in range(256):
                c = (blocked[blk, kq * 512 + dim * 2 + half] >> (2 * e)) & 3
                out[blk * 32 + t, dim // 4] |= c << (2 * (dim % 4))
    return out


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


def test_unblock_fast_matches_loop():
    b = np.random.default_rng(0).integers(0, 256, size=(3, 2048), dtype=np.uint8)
    np.testing.assert_array_equal(unblock(b, 96), unblock_fast(b, 96))


def np_dequant(codes: np.ndarray, norms_bits: np.ndarray, rot: np.ndarray, cent: np.ndarray) -> np.ndarray:
    """x_hat = |x|_fp16 * R^T c[code] for natural 2-bit codes [n, 64] (fp64)."""
    c = np.stack([(codes >> (2 * e)) & 3 for e in range(4)], -1).reshape(codes.shape[0], 256)
    return (cent.astype(np.float64)[c] @ rot) * orc.f16_to_f32(norms_bits).astype(np.float64)[:, None]


def check_against_oracle(cache, hist_k, hist_v, q, out, gate=None, sample=None, seed=0):
    """hist_k/hist_v[b]: the dense bf16 history [Hkv, L_b, D] of sequence b (GPU tensors).
    Checks pool codes (all tokens, or `sample` random tokens per (b, h)), the ring, and the
    output against fp64 attention over dequantized pool + ring."""
    R = cache.residual_capacity
    signs = cache.qn.signs.cpu().numpy()
    rot = orc.tq_hadamard_matrix(signs)
    cent = cache.qn.centroids.cpu().numpy()
    thr = cache.qn.thresholds.cpu().numpy()
    kc_pool, vc_pool = cache.key_codes.cpu().numpy(), cache.value_codes.cpu().numpy()
    kn_pool, vn_pool = bits_of(cache.key_norms), bits_of(cache.value_norms)
    ring_k, ring_v = cache.residual_key.cpu(), cache.residual_value_t.cpu()
    assert cache.seq_lengths.cpu().tolist() == [k.shape[1] for k in hist_k] == cache.lengths
    out = out.float().cpu().numpy()
    rng = np.random.default_rng(seed)
    for b in range(cache.batch):
        L = hist_k[b].shape[1]
        ql, off = max(0, L - R), cache.offsets[b]
        if L == 0:
            assert not out[b].any()
            continue
        qp = -(-ql // 32) * 32
        kk, vv = [], []
        hk, hv = hist_k[b].cpu(), hist_v[b].cpu()
        for h in range(cache.kv_heads):
            parts_k, parts_v = [], []
            if ql > 0:
                kcodes, knorms = kc_pool[h, off:off + ql], kn_pool[h, off:off + ql]
                vcodes = unblock_fast(vc_pool[h, off // 32:(off + qp) // 32], qp)[:ql]
                vnorms = vn_pool[h, off:off + ql]
                pick = np.arange(ql) if sample is None else np.sort(rng.choice(ql, size=min(ql, sample), replace=False))
                kb = bits_of(hk[h, :ql])[pick]
                vb = bits_of(hv[h, :ql])[pick]
                oc, on = orc.tq_hadamard_quantize(np.ascontiguousarray(kb), orc.BF16, signs, thr, 2)
                np.testing.assert_array_equal(kcodes[pick], oc)
                np.testing.assert_array_equal(knorms[pick], on)
                oc, on = orc.tq_hadamard_quantize(np.ascontiguousarray(vb), orc.BF16, signs, thr, 2)
                np.testing.assert_array_equal(vcodes[pick], oc)
                np.testing.assert_array_equal(vnorms[pick], on)
                parts_k.append(np_dequant(kcodes, knorms, rot, cent))
                parts_v.append(np_dequant(vcodes, vnorms, rot, cent))
            slots = np.arange(ql, L) % R
            np.testing.assert_array_equal(bits_of(ring_k[b, h][slots]), bits_of(hk[h, ql:]))
            np.testing.assert_array_equal(bits_of(ring_v[b, h][:, slots].t()), bits_of(hv[h, ql:]))
            parts_k.append(hk[h, ql:].float().numpy())
            parts_v.append(hv[h, ql:].float().numpy())
            kk.append(np.concatenate(parts_k))
            vv.append(np.concatenate(parts_v))
        g = None if gate is None else gate[b].float().cpu().numpy()
        ref = orc.gqa_decode(q[b].float().cpu().numpy(), np.stack(kk), np.stack(vv), 1.0 / 16, g)
        assert rel_err(out[b], ref) <= BF16_TOL, b


@pytest.mark.parametrize("tokens_per_item,gated", [(0, False), (64, True), (512, False), (32, True)])
def test_batched_decode_matches_oracle(gpu, tokens_per_item, gated):
    """Four sequences of 75 / 140 / 33 / 20 tokens with a 32-token window (the last one is
    window-only); items of 1 to 16 blocks, a gate on two of the cases."""
    print(f"[case] tq batch small tokens_per_item={tokens_per_item} gate={gated}", flush=True)
    torch.manual_seed(60)
    hkv, g, d, R = 2, 8, 256, 32
    lens = [75, 140, 33, 20]
    cache = TurboQuantBatchCache(batch=4, kv_heads=hkv, q_heads=hkv * g, capacities=[l - R for l in lens],
                                 residual_capacity=R, device=gpu, tokens_per_item=tokens_per_item)
    keys = [torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16) for L in lens]
    vals = [torch.randn(hkv, L, d, device=gpu).to(torch.bfloat16) for L in lens]
    for b in range(4):
        cache.load_sequence(b, keys[b], vals[b])
    q = torch.randn(4, hkv * g, d, device=gpu).to(torch.bfloat16)
    gate = torch.randn(4, hkv * g, d, device=gpu).to(torch.bfloat16) if gated else None
    out = cache.decode(q, scaling=1.0 / 16, gate=gate)
    check_against_oracle(cache, keys, vals, q, out, gate)
    out2 = cache.decode(q, scaling=1.0 / 16, gate=gate)
    assert torch.equal(out, out2)  # the merge order is fixed: the same bits every call


@pytest.mark.parametrize("tokens_per_item", [0, 512, 2048])
def test_batched_decode_config4_sizes(gpu, tokens_per_item):
    """BASELINE config 4 at its own sizes: B=8, Hq=16, Hkv=2, D=256, a full 128-token window on
    every sequence and packed lengths up to 16,384 (two sequences above 4,000).  tokens_per_item
    512 gives 32 items for the longest (b, kv-head) (the merge runs 4 batches of 8 items), 2048
    gives 64 blocks per item (each of the 8 split waves runs 4 ping-pong pair iterations).
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
        cache.load_sequence(b, keys[b], vals[b])
    q = torch.randn(B, HKV * G, D, device=gpu).to(torch.bfloat16)
    out = cache.decode(q, scaling=1.0 / 16)
    check_against_oracle(cache, keys, vals, q, out, sample=96)


def test_append_decode_loop_matches_oracle(gpu):
    """40 decode steps of one append + one decode launch each, from prefilled lengths 0 / 10 /
    40 / 100 with a 32-token window: tokens leave the ring into the pool from the first step on
    (bit-exact codes, blocked values written token by token), an empty sequence decodes to
    zeros, and after 10, 25 and 40 steps the cache and the output match the oracle."""
    print("[case] tq batch append+decode loop", flush=True)
    torch.manual_seed(9)
    B, HKV, G, D, R = 4, 2, 8, 256, 32
    pre = [0, 10, 40, 100]
    cache = TurboQuantBatchCache(batch=B, kv_heads=HKV, q_heads=HKV * G, capacities=[64, 64, 64, 128],
                                 residual_capacity=R, device=gpu)
    hist_k = [torch.randn(HKV, n, D, device=gpu).to(torch.bfloat16) for n in pre]
    hist_v = [torch.randn(HKV, n, D, device=gpu).to(torch.bfloat16) for n in pre]
    for b in range(B):
        cache.load_sequence(b, hist_k[b], hist_v[b])
    q = torch.randn(B, HKV * G, D, device=gpu).to(torch.bfloat16)
    out = cache.decode(q, scaling=1.0 / 16)
    check_against_oracle(cache, hist_k, hist_v, q, out)
    for step in range(1, 41):
        nk = torch.randn(B, HKV, D, device=gpu).to(torch.bfloat16)
        nv = torch.randn(B, HKV, D, device=gpu).to(torch.bfloat16)
        cache.append(nk, nv)
        hist_k = [torch.cat([hist_k[b], nk[b, :, None]], 1) for b in range(B)]
        hist_v = [torch.cat([hist_v[b], nv[b, :, None]], 1) for b in range(B)]
        q = torch.randn(B, HKV * G, D, device=gpu).to(torch.bfloat16)
        out = cache.decode(q, scaling=1.0 / 16)
        if step in (10, 25, 40):
            check_against_oracle(cache, hist_k, hist_v, q, out, seed=step)
    assert int(cache.overflow.item()) == 0


def test_append_decode_graph_replays_match_eager(gpu):
    """One step (append + decode) captured in a HIP graph and replayed 5 times, with eager
    work and synchronizations in between, gives the same bits as the same steps run eagerly
    on a twin cache."""
    print("[case] tq batch graph replay", flush=True)
    torch.manual_seed(12)
    B, HKV, G, D, R = 3, 2, 8, 256, 32
    pre = [5, 31, 70]
    caches = [TurboQuantBatchCache(batch=B, kv_heads=HKV, q_heads=HKV * G, capacities=[64] * B,
                                   residual_capacity=R, device=gpu) for _ in range(2)]
    for b in range(B):
        k = torch.randn(HKV, pre[b], D, device=gpu).to(torch.bfloat16)
        v = torch.randn(HKV, pre[b], D, device=gpu).to(torch.bfloat16)
        for c in caches:
            c.load_sequence(b, k, v)
    nk = torch.empty(B, HKV, D, device=gpu, dtype=torch.bfloat16)
    nv = torch.empty_like(nk)
    q = torch.empty(B, HKV * G, D, device=gpu, dtype=torch.bfloat16)
    out_g = torch.empty_like(q)
    graph_cache, eager_cache = caches
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        graph_cache.append(nk, nv)
        graph_cache.decode(q, scaling=1.0 / 16, out=out_g)
    graph_cache.lengths = list(pre)  # capture ran no kernel: the host mirror rolls back
    for step in range(5):
        nk.copy_(torch.randn(B, HKV, D, device=gpu).to(torch.bfloat16))
        nv.copy_(torch.randn(B, HKV, D, device=gpu).to(torch.bfloat16))
        q.copy_(torch.randn(B, HKV * G, D, device=gpu).to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager_cache.append(nk, nv)
        ref = eager_cache.decode(q, scaling=1.0 / 16)
        torch.cuda.synchronize()
        assert torch.equal(out_g, ref), step
        assert torch.equal(graph_cache.seq_lengths, eager_cache.seq_lengths)
        assert torch.equal(graph_cache.key_codes, eager_cache.key_codes)
        assert torch.equal(graph_cache.value_codes, eager_cache.value_codes)


@pytest.mark.parametrize("gated", [False, True])
def test_fused_append_decode_matches_two_calls_and_oracle(gpu, gated):
    """anna_mi_tq_append_decode (the step's append inside the decode's two launches) against
    append + decode on a twin cache, 40 steps from prefilled lengths 0 / 10 / 40 / 100 with a
    32-token window: the caches stay equal bit for bit (pool codes and norms, ring, lengths),
    the outputs agree (the two tokens the merge scores itself are the only difference in
    arithmetic), and after 1, 10, 25 and 40 steps the fused output matches the oracle."""
    print(f"[case] tq batch fused append+decode gate={gated}", flush=True)
    torch.manual_seed(19 + gated)
    B, HKV, G, D, R = 4, 2, 8, 256, 32
    pre = [0, 10, 40, 100]
    caches = [TurboQuantBatchCache(batch=B, kv_heads=HKV, q_heads=HKV * G, capacities=[64, 64, 64, 128],
                                   residual_capacity=R, device=gpu) for _ in range(2)]
    hist_k = [torch.randn(HKV, n, D, device=gpu).to(torch.bfloat16) for n in pre]
    hist_v = [torch.randn(HKV, n, D, device=gpu).to(torch.bfloat16) for n in pre]
    for c in caches:
        for b in range(B):
            c.load_sequence(b, hist_k[b], hist_v[b])
    fused, split = caches
    for step in range(1, 41):
        nk = torch.randn(B, HKV, D, device=gpu).to(torch.bfloat16)
        nv = torch.randn(B, HKV, D, device=gpu).to(torch.bfloat16)
        q = torch.randn(B, HKV * G, D, device=gpu).to(torch.bfloat16)
        gate = torch.randn(B, HKV * G, D, device=gpu).to(torch.bfloat16) if gated else None
        out_f = fused.append_decode(nk, nv, q, scaling=1.0 / 16, gate=gate)
        split.append(nk, nv)
        out_s = split.decode(q, scaling=1.0 / 16, gate=gate)
        hist_k = [torch.cat([hist_k[b], nk[b, :, None]], 1) for b in range(B)]
        hist_v = [torch.cat([hist_v[b], nv[b, :, None]], 1) for b in range(B)]
        for name in ("key_codes", "key_norms", "value_codes", "value_norms", "residual_key", "residual_value_t",
                     "seq_lengths"):
            assert torch.equal(getattr(fused, name), getattr(split, name)), (step, name)
        assert fused.lengths == split.lengths
        assert rel_err(out_f.float().cpu().numpy(), out_s.float().cpu().numpy().astype(np.float64)) <= BF16_TOL, step
        if step in (1, 10, 25, 40):
            check_against_oracle(fused, hist_k, hist_v, q, out_f, gate=gate, seed=step)
    assert int(fused.overflow.item()) == 0


def test_fused_append_decode_graph_replays_match_eager(gpu):
    """The fused step captured once and replayed 5 times, with eager work in between, gives the
    same bits as the same fused steps run eagerly on a twin cache."""
    print("[case] tq batch fused graph replay", flush=True)
    torch.manual_seed(23)
    B, HKV, G, D, R = 3, 2, 8, 256, 32
    pre = [0, 31, 70]
    caches = [TurboQuantBatchCache(batch=B, kv_heads=HKV, q_heads=HKV * G, capacities=[64] * B,
                                   residual_capacity=R, device=gpu) for _ in range(2)]
    for b in range(B):
        k = torch.randn(HKV, pre[b], D, device=gpu).to(torch.bfloat16)
        v = torch.randn(HKV, pre[b], D, device=gpu).to(torch.bfloat16)
        for c in caches:
            c.load_sequence(b, k, v)
    nk = torch.empty(B, HKV, D, device=gpu, dtype=torch.bfloat16)
    nv = torch.empty_like(nk)
    q = torch.empty(B, HKV * G, D, device=gpu, dtype=torch.bfloat16)
    out_g = torch.empty_like(q)
    graph_cache, eager_cache = caches
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        graph_cache.append_decode(nk, nv, q, scaling=1.0 / 16, out=out_g)
    graph_cache.lengths = list(pre)  # capture ran no kernel: the host mirror rolls back
    for step in range(5):
        nk.copy_(torch.randn(B, HKV, D, device=gpu).to(torch.bfloat16))
        nv.copy_(torch.randn(B, HKV, D, device=gpu).to(torch.bfloat16))
        q.copy_(torch.randn(B, HKV * G, D, device=gpu).to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        graph_cache.lengths = [n + 1 for n in graph_cache.lengths]
        ref = eager_cache.append_decode(nk, nv, q, scaling=1.0 / 16)
        torch.cuda.synchronize()
        assert torch.equal(out_g, ref), step
        for name in ("seq_lengths", "key_codes", "value_codes", "residual_key", "residual_value_t"):
            assert torch.equal(getattr(graph_cache, name), getattr(eager_cache, name)), (step, name)


def test_append_refuses_a_full_sequence(gpu):
    cache = TurboQuantBatchCache(batch=1, kv_heads=1, q_heads=8, capacities=[32], residual_capacity=32, device=gpu)
    k = torch.randn(1, 64, 256, device=gpu).to(torch.bfloat16)
    cache.load_sequence(0, k, k)
    with pytest.raises(RuntimeError, match="sequence 0 is full"):
        cache.append(k[:, :1], k[:, :1])


def test_pack_config3_layout_bit_exact(gpu):
    """K, V bf16 [8192 tokens, 2 kv heads, 256] ~N(0,1) with 1% outlier
    channels x8, read in that token-major layout (head stride 256, token stride 512) by one pack
    launch; every key and value code and norm of the 8064 packed tokens is bit-exact with the
    oracle's Hadamard quantizer (values after undoing the blocking)."""
    print("[case] tq pack config3", flush=True)
    T, H, D, R = 8192, 2, 256, 128
    g = torch.Generator(device=gpu)
    g.manual_seed(33)
    outl = torch.zeros(D, dtype=torch.bool)
    outl[torch.randperm(D, generator=torch.Generator().manual_seed(3))[: D // 100]] = True
    kv = []
    for _ in range(2):
        x = torch.randn((T, H, D), device=gpu, generator=g)
        x[..., outl.to(gpu)] *= 8.0
        kv.append(x.to(torch.bfloat16))
    cache = TurboQuantBatchCache(batch=1, kv_heads=H, q_heads=H * 8, capacities=[T - R], residual_capacity=R,
                                 device=gpu)
    cache._pack(kv[0].transpose(0, 1), kv[1].transpose(0, 1), T - R, 0)  # [H, T, D] views, strides (256, 512, 1)
    signs = cache.qn.signs.cpu().numpy()
    thr = cache.qn.thresholds.cpu().numpy()
    n = T - R
    for h in range(H):
        for which, x in enumerate(kv):
            oc, on = orc.tq_hadamard_quantize(np.ascontiguousarray(bits_of(x[:n, h])), orc.BF16, signs, thr, 2)
            if which == 0:
                np.testing.assert_array_equal(cache.key_codes[h, :n].cpu().numpy(), oc)
                np.testing.assert_array_equal(bits_of(cache.key_norms[h, :n]), on)
            else:
                got = unblock_fast(cache.value_codes[h, : n // 32].cpu().numpy(), n)
                np.testing.assert_array_equal(got, oc)
                np.testing.assert_array_equal(bits_of(cache.value_norms[h, :n]), on)

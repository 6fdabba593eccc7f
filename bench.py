"""Benchmark of the MI355X quantized decode path (one GPU).

Headline (``value``): W4A16 int4 GEMV throughput in GB/s on BASELINE config 2's
M=1, N=12288, K=4096 point (group 128, bf16 scales, asymmetric int8 zero points).
A step is one int4 linear call over one batch; the K timed steps are captured
into a HIP graph that cycles through enough distinct weight copies (> 512 MB) that
the 256 MB Infinity Cache cannot serve them, and are timed with HIP events on the
stream the kernels run on.  The rest of the sweep (and the other path sections)
are reported under ``sections``.

Usage: python bench.py [--gpus 1] [--steps 60] [--warmup 10] [--sections int4,...]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 600 * 2**20  # distinct buffers per timed region (> 2 x 256 MB Infinity Cache)
COPY_BYTES = 256 * 2**20
METRIC = "int4 GEMV/GEMM GB/s & TFLOPs (% roofline); TQ-KV decode attn tokens/s"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


EAGER = False  # --eager: launch the steps directly (for counter collection runs)
REPLAYS = 5  # timed replays of each step graph; the median is reported


def time_graph(fns, steps: int, warmup: int) -> float:
    """Capture `steps` calls (fns[i % len(fns)]) into one HIP graph; return ms per step.
    With --eager the steps are launched one by one on the same stream instead."""
    stream = torch.cuda.Stream()
    if EAGER:
        with torch.cuda.stream(stream):
            for i in range(warmup):
                fns[i % len(fns)]()
            torch.cuda.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for i in range(steps):
                fns[i % len(fns)]()
            end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for f in fns[: min(len(fns), 3)]:  # eager warm-up (loads code objects)
            f()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            fns[i % len(fns)]()
    for _ in range(max(1, warmup // max(1, steps) + 1)):
        graph.replay()
    torch.cuda.synchronize()
    # median of REPLAYS timed replays of the K-step graph (each bracketed by HIP events on the
    # stream the kernels run on)
    times = []
    for _ in range(REPLAYS):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            start.record(stream)
            graph.replay()
            end.record(stream)
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end))
    times.sort()
    ms = times[len(times) // 2]
    return ms / steps


# ---------------------------------------------------------------- int4 linear


def int4_bytes(m, n, k, group, scale_bytes=2):
    g = k // group
    return n * k // 2 + g * n * scale_bytes + g * n + m * k * 2 + m * n * 2


def make_int4_copies(n, k, group, copies, device, gen):
    g = k // group
    out = []
    for _ in range(copies):
        qw = torch.randint(-(2**31), 2**31 - 1, (n, k // 8), dtype=torch.int32, device=device, generator=gen)
        qs = (torch.randn((g, n), device=device, generator=gen) * 0.02).abs_().add_(1e-3).to(torch.bfloat16)
        qz = torch.randint(0, 16, (g, n), dtype=torch.int8, device=device, generator=gen)
        out.append((qw, qs, qz))
    return out


def bench_int4_point(m, n, k, steps, warmup, device, group=128):
    from anna_amd import fused_ops

    gen = torch.Generator(device=device)
    gen.manual_seed(1234 + m + n + k)
    per_copy = int4_bytes(m, n, k, group)
    copies = max(2, math.ceil(ROTATE_BYTES / per_copy))
    ws = make_int4_copies(n, k, group, copies, device, gen)
    x = torch.randn((m, k), device=device, generator=gen).to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=device)

    def mk(w):
        return lambda: fused_ops.int4_linear_out(x, w[0], w[1], w[2], group, k, y)

    ms = time_graph([mk(w) for w in ws], steps, warmup)
    sec = ms / 1e3
    gbs = per_copy / sec / 1e9
    tflops = 2.0 * m * n * k / sec / 1e12
    bound = "hbm" if m <= 64 else "mfma"
    frac = gbs / HBM_PEAK_GBS if bound == "hbm" else tflops / BF16_PEAK_TFLOPS
    del ws
    torch.cuda.empty_cache()
    return {"M": m, "N": n, "K": k, "ms": ms, "us": ms * 1e3, "GB/s": gbs, "TFLOP/s": tflops, "bound": bound,
            "roofline_frac": frac, "bytes": per_copy, "distinct_weight_copies": copies}


def cpu_baseline_int4(m, n, k, group, budget_s):
    from oracle.cpu_paths import int4_forward_dequant

    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(7)
    qw = torch.randint(-(2**31), 2**31 - 1, (n, k // 8), dtype=torch.int32, generator=g)
    qs = (torch.randn((k // group, n), generator=g) * 0.02).abs_().add_(1e-3).to(torch.bfloat16).float()
    qz = torch.randint(0, 16, (k // group, n), dtype=torch.int8, generator=g)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    int4_forward_dequant(x, qw, qs, qz, group, k)  # warm-up
    t0 = time.perf_counter()
    int4_forward_dequant(x, qw, qs, qz, group, k)
    one = time.perf_counter() - t0
    iters = max(3, min(200, int(budget_s / max(one, 1e-6))))
    t0 = time.perf_counter()
    for _ in range(iters):
        int4_forward_dequant(x, qw, qs, qz, group, k)
    sec = (time.perf_counter() - t0) / iters
    return {
        "value": int4_bytes(m, n, k, group) / sec / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{iters} calls of the reference CPU dequant path (XPUInt4Linear._forward_dequant restated in "
                   f"torch) at M={m} N={n} K={k}; {sec * 1e3:.1f} ms/call; CPU: {cpu_model()}, "
                   f"os.cpu_count()={os.cpu_count()}"),
    }


def section_int4(args, device):
    sweep = []
    points = [(1, 6144, 2048)] + [(m, n, 4096) for n in (12288, 6144) for m in (1, 8, 64, 256, 2048)]
    if args.int4_points:
        points = [tuple(int(v) for v in p.split("x")) for p in args.int4_points.split(",")]
    for (m, n, k) in points:
        steps = args.steps if m <= 64 else max(10, args.steps // 4)
        r = bench_int4_point(m, n, k, steps, args.warmup, device)
        log(f"int4 M={m:5d} N={n:6d} K={k}: {r['us']:8.2f} us  {r['GB/s']:8.1f} GB/s  "
            f"{r['TFLOP/s']:7.1f} TFLOP/s  {100 * r['roofline_frac']:5.1f}% of {r['bound']} peak")
        sweep.append(r)
    return sweep


# ---------------------------------------------------------------- TurboQuant


def _clone_cache(c):
    import copy

    n = copy.copy(c)
    for name in ("key_codes", "key_norms", "value_codes", "value_norms", "residual_key", "residual_value_t",
                 "seq_lengths", "item_table", "partial_stats", "partial_values"):
        setattr(n, name, getattr(c, name).clone())
    n.lengths = list(c.lengths)
    return n


def section_tq_decode(args, device):
    """B=8, Hq=16, Hkv=2, D=256, L ~ U[1024, 16384] + 128 bf16 residual."""
    import numpy as np

    from anna_amd.tq_cache import TurboQuantBatchCache

    rng = np.random.default_rng(4)
    lens = [int(v) for v in rng.integers(1024, 16385, size=8)]
    B, HQ, HKV, D, R = 8, 16, 2, 256, 128
    gen = torch.Generator(device=device)
    gen.manual_seed(44)
    base = TurboQuantBatchCache(batch=B, kv_heads=HKV, q_heads=HQ, capacities=lens, residual_capacity=R,
                                device=device, tokens_per_item=args.tq_tokens_per_item)
    dense = []
    for b in range(B):
        k = torch.randn((HKV, lens[b] + R, D), device=device, generator=gen).to(torch.bfloat16)
        v = torch.randn((HKV, lens[b] + R, D), device=device, generator=gen).to(torch.bfloat16)
        base.load_sequence(b, k, v)
        dense.append((k, v))
    q = torch.randn((B, HQ, D), device=device, generator=gen).to(torch.bfloat16)
    out = torch.empty_like(q)
    per_call = base.bytes_per_decode()
    copies = [base] + [_clone_cache(base) for _ in range(max(1, math.ceil(ROTATE_BYTES / per_call)) - 1)]
    fns = [(lambda c=c: c.decode(q, scaling=1.0 / 16, out=out)) for c in copies]
    ms = time_graph(fns, args.steps, args.warmup)
    sec = ms / 1e3
    r = {"B": B, "Hq": HQ, "Hkv": HKV, "D": D, "lens": lens, "residual": R, "bits": 2, "ms": ms, "us": ms * 1e3,
         "tokens/s": B / sec, "GB/s": per_call / sec / 1e9, "bytes": per_call, "roofline_frac": per_call / sec / 1e9 / HBM_PEAK_GBS,
         "distinct_cache_copies": len(copies), "tokens_per_item": args.tq_tokens_per_item}
    log(f"tq decode B=8 mean L={sum(lens) / 8:.0f}: {r['us']:.2f} us/call  {r['tokens/s']:.0f} tokens/s  "
        f"{r['GB/s']:.0f} GB/s  {100 * r['roofline_frac']:.1f}% of HBM peak")
    # a whole decode step: append one token per sequence (the oldest window token of each
    # sequence is quantized into the pool), then decode; on a copy sized for the added tokens
    steps = max(4, args.steps // 4)
    # (the graph is replayed warm-up + REPLAYS times, each replay appending `steps` tokens)
    grow = TurboQuantBatchCache(batch=B, kv_heads=HKV, q_heads=HQ,
                                capacities=[n + (REPLAYS + 3) * steps + 8 for n in lens],
                                residual_capacity=R, device=device)
    for b in range(B):
        grow.load_sequence(b, dense[b][0], dense[b][1])
    nk = torch.randn((B, HKV, D), device=device, generator=gen).to(torch.bfloat16)
    nv = torch.randn((B, HKV, D), device=device, generator=gen).to(torch.bfloat16)

    def step():
        grow.append(nk, nv)
        grow.decode(q, scaling=1.0 / 16, out=out)

    ms_step = time_graph([step], steps, 0)
    r["append_decode_step_us"] = ms_step * 1e3
    log(f"tq append+decode step: {ms_step * 1e3:.2f} us")
    # the same step with the append inside the decode's two launches (anna_mi_tq_append_decode)
    fused = TurboQuantBatchCache(batch=B, kv_heads=HKV, q_heads=HQ,
                                 capacities=[n + (REPLAYS + 3) * steps + 8 for n in lens],
                                 residual_capacity=R, device=device)
    for b in range(B):
        fused.load_sequence(b, dense[b][0], dense[b][1])
    ms_fused = time_graph([lambda: fused.append_decode(nk, nv, q, scaling=1.0 / 16, out=out)], steps, 0)
    r["fused_append_decode_step_us"] = ms_fused * 1e3
    log(f"tq fused append+decode step: {ms_fused * 1e3:.2f} us")
    cpu = None
    if not args.no_cpu:
        from oracle.cpu_paths import tq_decode_rows

        torch.set_num_threads(os.cpu_count() or 1)
        ks = [k.cpu() for k, _ in dense]
        vs = [v.cpu() for _, v in dense]
        qc = q.cpu()
        tq_decode_rows(qc, ks, vs, 1.0 / 16)
        iters = 3
        t0 = time.perf_counter()
        for _ in range(iters):
            tq_decode_rows(qc, ks, vs, 1.0 / 16)
        csec = (time.perf_counter() - t0) / iters
        cpu = {"value": B / csec, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"{iters} calls of the reference CPU decode branch (bf16 matmuls over the kept dequantized "
                         f"cache, fp32 softmax; dequant not timed), same B/L/H/D; {csec * 1e3:.1f} ms/call"}
        log(f"tq decode cpu baseline: {cpu['value']:.1f} tokens/s")
    r["cpu_baseline"] = cpu
    return r


def section_row_decode(args, device):
    """The reference's per-row op (gqa_decode_splitkv_turboquant_fused_out): B=8, Hq=16, Hkv=2,
    D=256, 4096 packed tokens (2-bit min/max values, group 32, dense bf16 keys) + 128 bf16
    residual tokens, block 64."""
    from anna_amd.turboquant import quantize_turboquant_values

    B, HQ, HKV, D, L, R, BITS, GROUP, BS = 8, 16, 2, 256, 4096, 128, 2, 32, 64
    gen = torch.Generator(device=device)
    gen.manual_seed(46)
    q = torch.randn((B, HQ, 1, D), device=device, generator=gen).to(torch.bfloat16)

    def make():
        k = torch.randn((B, HKV, L, D), device=device, generator=gen).to(torch.bfloat16)
        st = quantize_turboquant_values(torch.randn((B * HKV, L, D), device=device, generator=gen).to(torch.bfloat16),
                                        bits=BITS, group_size=GROUP)
        rk = torch.randn((B, HKV, R, D), device=device, generator=gen).to(torch.bfloat16)
        rv = torch.randn((B, HKV, R, D), device=device, generator=gen).to(torch.bfloat16)
        return (k, st.data.view(B, HKV, L, -1), st.scales.view(B, HKV, L, -1), st.zeros.view(B, HKV, L, -1), rk, rv)

    first = make()
    per_call = sum(t.numel() * t.element_size() for t in first)
    caches = [first] + [make() for _ in range(max(1, math.ceil(ROTATE_BYTES / per_call)) - 1)]
    nblk = -(-(L + R) // BS)
    out = torch.empty_like(q)
    ps = torch.empty((B, HQ, nblk, 2), device=device)
    pv = torch.empty((B, HQ, nblk, D), device=device)
    op = torch.ops.anna.gqa_decode_splitkv_turboquant_fused_out
    fns = [(lambda c=c: op(q, *c, out, ps, pv, D ** -0.5, BITS, GROUP, BS, None)) for c in caches]
    ms = time_graph(fns, args.steps, args.warmup)
    sec = ms / 1e3
    r = {"B": B, "Hq": HQ, "Hkv": HKV, "D": D, "L": L, "residual": R, "value_bits": BITS, "group": GROUP,
         "block_size": BS, "ms": ms, "us": ms * 1e3, "tokens/s": B / sec, "bytes": per_call,
         "GB/s": per_call / sec / 1e9, "roofline_frac": per_call / sec / 1e9 / HBM_PEAK_GBS,
         "distinct_cache_copies": len(caches)}
    log(f"row-API decode B=8 L={L}+{R}: {r['us']:.2f} us/call  {r['GB/s']:.0f} GB/s  "
        f"{100 * r['roofline_frac']:.1f}% of HBM peak")
    cpu = None
    if not args.no_cpu:
        from anna_amd.turboquant import TurboQuantValueState, dequantize_turboquant_values
        from oracle.cpu_paths import tq_decode_rows

        k, vd, vs, vz, rk, rv = first
        st = TurboQuantValueState(data=vd.reshape(B * HKV, L, -1), scales=vs.reshape(B * HKV, L, -1),
                                  zeros=vz.reshape(B * HKV, L, -1), bits=BITS, group_size=GROUP)
        vals = dequantize_turboquant_values(st, dtype=torch.bfloat16).view(B, HKV, L, D)
        # the CPU branch decodes against its kept bf16 cache (turboquant.py:1289-1294): keys and
        # dequantized values of the packed prefix followed by the window
        ks = [torch.cat((k[b], rk[b]), dim=1).cpu() for b in range(B)]
        vs_ = [torch.cat((vals[b], rv[b]), dim=1).cpu() for b in range(B)]
        qc = q.squeeze(2).cpu()
        cpu = _time_cpu(lambda: tq_decode_rows(qc, ks, vs_, D ** -0.5), args.cpu_seconds / 4)
        cpu = {"value": B / cpu["sec"], "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"{cpu['iters']} calls of the reference CPU decode branch (turboquant.py:1289-1311: bf16 "
                         f"matmuls over the kept dequantized cache, fp32 softmax), B={B} L={L}+{R}; "
                         f"{cpu['sec'] * 1e3:.1f} ms/call"}
        log(f"row-API decode cpu baseline: {cpu['value']:.1f} tokens/s")
    r["cpu_baseline"] = cpu
    return r


def _time_cpu(fn, budget_s: float, max_iters: int = 50) -> dict:
    """Mean wall time of fn() on the host cores (one untimed warm-up call, then calls until
    budget_s is spent or max_iters are done)."""
    torch.set_num_threads(os.cpu_count() or 1)
    fn()
    iters, t0 = 0, time.perf_counter()
    while iters < max_iters and (iters == 0 or time.perf_counter() - t0 < budget_s):
        fn()
        iters += 1
    return {"sec": (time.perf_counter() - t0) / iters, "iters": iters}


def section_tq_pack(args, device):
    """K, V bf16 [8192, 2, 256] with 1% outlier channels x8 -> 2-bit TQ-MSE
    codes + fp16 norms, last 128 tokens kept bf16."""
    from anna_amd.turboquant import get_turboquant_quantizer

    T, H, D, R = 8192, 2, 256, 128
    gen = torch.Generator(device=device)
    gen.manual_seed(33)
    qn = get_turboquant_quantizer(head_dim=D, bits=2, device=device)
    outl = torch.zeros(D, dtype=torch.bool)
    outl[torch.randperm(D, generator=torch.Generator().manual_seed(3))[: max(1, D // 100)]] = True
    outl = outl.to(device)
    per_copy = 2 * H * T * D * 2
    ncopy = max(2, math.ceil(ROTATE_BYTES / per_copy))  # K/V pairs rotated past the Infinity Cache
    kvs = []
    for _ in range(ncopy):
        pair = []
        for _ in range(2):
            x = torch.randn((H, T, D), device=device, generator=gen)
            x[..., outl] *= 8.0
            pair.append(x.to(torch.bfloat16))
        kvs.append(pair)
    n = (T - R) * H
    from anna_amd.tq_cache import TurboQuantBatchCache

    # the pool of one sequence of T tokens: its first T - R tokens packed by one launch
    # (TurboQuantBatchCache._pack: K and V quantized, values blocked, norms), the rest stays bf16
    dst = TurboQuantBatchCache(batch=1, kv_heads=H, q_heads=H, capacities=[T - R], residual_capacity=R,
                               device=device)

    def pack(kv):
        dst._pack(kv[0], kv[1], T - R, 0)

    ms = time_graph([(lambda kv=kv: pack(kv)) for kv in kvs], max(ncopy, args.steps // 10), 2)
    sec = ms / 1e3
    # algorithmic bytes: the packed tokens of K and V read once (bf16), their codes and fp16
    # norms written (the values already in the blocked layout)
    bytes_ = 2 * n * D * 2 + 2 * n * (D // 4 + 2)
    r = {"T": T, "H": H, "D": D, "residual": R, "ms": ms, "us": ms * 1e3, "GB/s": bytes_ / sec / 1e9, "bytes": bytes_,
         "roofline_frac": bytes_ / sec / 1e9 / HBM_PEAK_GBS, "distinct_input_copies": ncopy,
         "vectors/s": 2 * n / sec, "bound": "hbm (Hadamard rotation: O(D log D) per vector)", "launches": 1,
         "quantizer": qn.kind}
    log(f"tq pack K+V [8192,2,256]: {r['us']:.1f} us  {r['vectors/s'] / 1e6:.2f} M vectors/s  "
        f"{r['GB/s']:.0f} GB/s  {100 * r['roofline_frac']:.1f}% of HBM peak")
    cpu = None
    if not args.no_cpu:
        from oracle.cpu_paths import tq_tensor_row_append

        # the reference's CPU path: TurboQuantTensorRow.append of the prefill for K and for V,
        # through the published quantizer with its dense D x D rotation (a seeded Haar matrix)
        g = torch.Generator().manual_seed(42)
        rot, _ = torch.linalg.qr(torch.randn((D, D), generator=g))
        cent = qn.centroids.float().cpu()
        kc, vc = kvs[0][0].cpu(), kvs[0][1].cpu()
        t = _time_cpu(lambda: (tq_tensor_row_append(kc, R, rot, cent), tq_tensor_row_append(vc, R, rot, cent)),
                      args.cpu_seconds / 4, max_iters=20)
        cpu = {"value": 2 * n / t["sec"], "unit": "vectors/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"{t['iters']} prefills of K and V [{H},{T},{D}] through TurboQuantTensorRow.append's "
                         f"CPU path (turboquant.py:353-405 with the published TurboQuant-MSE quantizer: norm, dense "
                         f"rotation, nearest centroid); {t['sec'] * 1e3:.1f} ms per prefill pair"}
        log(f"tq pack cpu baseline: {cpu['value'] / 1e6:.3f} M vectors/s")
    r["cpu_baseline"] = cpu
    return r


def section_tq_rows(args, device):
    """The batched cache for the shapes other than head_dim 256 / 2-bit (TurboQuantRowsCache):
    B=8, Hq=16, Hkv=2, head_dim 128, 4-bit keys and values (--tq-rows-dim / --tq-rows-bits change
    them), L ~ U[1024, 16384] + 128 bf16 window."""
    import numpy as np

    from anna_amd.tq_cache import TurboQuantRowsCache

    rng = np.random.default_rng(5)
    B, HQ, HKV, D, R, BITS = 8, 16, 2, args.tq_rows_dim, 128, args.tq_rows_bits
    lens = [int(v) for v in rng.integers(1024, 16385, size=B)]
    gen = torch.Generator(device=device)
    gen.manual_seed(55)

    def make():
        c = TurboQuantRowsCache(batch=B, kv_heads=HKV, q_heads=HQ, capacities=lens, residual_capacity=R,
                                head_dim=D, bits=BITS, device=device)
        for b in range(B):
            k = torch.randn((HKV, lens[b] + R, D), device=device, generator=gen).to(torch.bfloat16)
            v = torch.randn((HKV, lens[b] + R, D), device=device, generator=gen).to(torch.bfloat16)
            c.load_sequence(b, k, v)
        return c

    first = make()
    per_call = first.bytes_per_decode()
    caches = [first] + [make() for _ in range(max(1, math.ceil(ROTATE_BYTES / per_call)) - 1)]
    q = torch.randn((B, HQ, D), device=device, generator=gen).to(torch.bfloat16)
    out = torch.empty_like(q)
    for c in caches:  # size the partial buffers outside the captured region
        c.decode(q, scaling=D ** -0.5, out=out)
    ms = time_graph([(lambda c=c: c.decode(q, scaling=D ** -0.5, out=out)) for c in caches], args.steps, args.warmup)
    sec = ms / 1e3
    r = {"B": B, "Hq": HQ, "Hkv": HKV, "D": D, "bits": BITS, "lens": lens, "residual": R, "ms": ms, "us": ms * 1e3,
         "tokens/s": B / sec, "bytes": per_call, "GB/s": per_call / sec / 1e9,
         "roofline_frac": per_call / sec / 1e9 / HBM_PEAK_GBS, "distinct_cache_copies": len(caches),
         "launches": 3}
    log(f"tq rows decode D={D} {BITS}-bit: {r['us']:.2f} us/call  {r['GB/s']:.0f} GB/s  "
        f"{100 * r['roofline_frac']:.1f}% of HBM peak")
    return r


# ---------------------------------------------------------------- MoE (config 5)

MOE_EXPERT_BYTES = 3 * 512 * 2048 // 2 + (2 * 16 * 512 + 4 * 2048) * 3  # int4 + bf16 scales + int8 zeros


def _moe_bank(device, seed):
    from anna_amd.moe import GroupedInt4ExpertBank

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    e, h, i, grp = 128, 2048, 512, 128

    def lin(n, k):
        qw = torch.randint(-(2**31), 2**31 - 1, (e, n, k // 8), dtype=torch.int32, device=device, generator=g)
        qs = (torch.randn((e, k // grp, n), device=device, generator=g) * 0.02).abs_().add_(1e-3).to(torch.bfloat16)
        qz = torch.randint(0, 16, (e, k // grp, n), dtype=torch.int8, device=device, generator=g)
        return qw, qs, qz

    return GroupedInt4ExpertBank(e, h, i, grp, *lin(i, h), *lin(i, h), *lin(h, i), list(range(e)),
                                 {x: x for x in range(e)})


def cpu_baseline_moe(tokens, budget_s):
    """Reference CPU path of the quantized MoE block: _route_tokens, sorted dispatch, a
    Qwen3MLP per hit expert whose projections run XPUInt4Linear._forward_dequant
    (dequantize, bf16 F.linear), index_add_ scatter (ops.py:3280-3376, 3556-3568)."""
    from oracle import cpu_paths as cp

    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(3)
    e, k, h, i, grp = 128, 8, 2048, 512, 128

    def lin(n, kk):
        return (torch.randint(-(2**31), 2**31 - 1, (n, kk // 8), dtype=torch.int32, generator=g),
                (torch.randn((kk // grp, n), generator=g) * 0.02).abs_().add_(1e-3),
                torch.randint(0, 16, (kk // grp, n), dtype=torch.int8, generator=g))

    experts = [(lin(i, h), lin(i, h), lin(h, i)) for _ in range(e)]
    x = torch.randn(tokens, h, generator=g).to(torch.bfloat16)
    logits = torch.randn(tokens, e, generator=g)

    def step():
        w, sel, usage = cp.moe_route(logits, k, True)
        tok, rte, off = cp.moe_sorted_assignments(sel, usage, e)
        compact = x.index_select(0, tok)
        cw = w.to(torch.bfloat16)[tok, rte].unsqueeze(1)
        outs = torch.empty_like(compact)
        for ex in range(e):
            s0, s1 = int(off[ex]), int(off[ex + 1])
            if s1 <= s0:
                continue
            (gq, gs, gz), (uq, us, uz), (dq, ds, dz) = experts[ex]
            xs = compact[s0:s1]
            gate = cp.int4_forward_dequant(xs, gq, gs, gz, grp, h)
            up = cp.int4_forward_dequant(xs, uq, us, uz, grp, h)
            act = torch.nn.functional.silu(gate) * up
            outs[s0:s1] = cp.int4_forward_dequant(act, dq, ds, dz, grp, i) * cw[s0:s1]
        fin = torch.zeros((tokens, h), dtype=torch.bfloat16)
        fin.index_add_(0, tok, outs)
        return fin

    step()
    t0 = time.perf_counter()
    n = 0
    while True:
        step()
        n += 1
        if time.perf_counter() - t0 > budget_s or n >= 20:
            break
    sec = (time.perf_counter() - t0) / n
    return {"value": tokens / sec, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{n} MoE steps of {tokens} tokens through the reference CPU path; {sec * 1e3:.1f} ms/step"}


def section_moe(args, device):
    """128 experts, top-8 of softmax(N(0,1) logits), H=2048, I=512, group 128
    int4 (bf16 scales, int8 zeros), T in {8, 64, 512} bf16 tokens."""
    from anna_amd import fused_ops
    from anna_amd.moe import SparseMoeInt4

    banks = [_moe_bank(device, 100 + c) for c in range(3)]  # 3 x 211 MB: more than 2 x the Infinity Cache
    out = []
    for tokens in (8, 64, 512):
        gen = torch.Generator(device=device)
        gen.manual_seed(tokens)
        x = torch.randn((tokens, 2048), device=device, generator=gen).to(torch.bfloat16)
        logits = torch.randn((tokens, 128), device=device, generator=gen)
        blocks = [SparseMoeInt4(b, num_experts=128, top_k=8) for b in banks]
        w, sel, usage = fused_ops.moe_router(logits, 8, True)
        active = int((usage > 0).sum())
        sti, off, compact, cw = fused_ops.moe_dispatch(x, w.to(torch.bfloat16), sel, usage)
        co = torch.empty_like(compact)
        act = torch.empty((compact.shape[0], 512), dtype=torch.float32, device=device)
        max_routes = int(usage.max())  # host-known, as the reference caller passes it (ops.py:3430-3440)
        mlp = [(lambda b=b: fused_ops.moe_grouped_int4_mlp_out(compact, cw, co, off, blocks[0].active_experts,
                                                               blocks[0].active_slots, *b.tensors(), 128, max_routes,
                                                               activation=act)) for b in banks]
        full = [(lambda blk=blk: blk(x, logits)) for blk in blocks]
        ms_mlp = time_graph(mlp, args.steps, args.warmup)
        ms_full = time_graph(full, args.steps, args.warmup)
        wbytes = active * MOE_EXPERT_BYTES
        io = tokens * 8 * 2048 * 2 * 2
        r = {"tokens": tokens, "routes": tokens * 8, "active_experts": active, "weight_bytes": wbytes,
             "mlp_us": ms_mlp * 1e3, "mlp_GB/s": (wbytes + io) / ms_mlp / 1e6,
             "mlp_roofline_frac": (wbytes + io) / ms_mlp / 1e6 / HBM_PEAK_GBS,
             "step_us": ms_full * 1e3, "step_tokens/s": tokens / ms_full * 1e3,
             "TFLOP/s": tokens * 8 * 2 * (2048 * 1024 + 512 * 2048) / ms_mlp / 1e9}
        log(f"moe T={tokens:4d} active={active:3d}: grouped MLP {r['mlp_us']:.1f} us {r['mlp_GB/s']:.0f} GB/s "
            f"({100 * r['mlp_roofline_frac']:.1f}% HBM); full step {r['step_us']:.1f} us")
        if not args.no_cpu:
            r["cpu_baseline"] = cpu_baseline_moe(tokens, args.cpu_seconds / 2)
            log(f"moe T={tokens} cpu baseline: {r['cpu_baseline']['value']:.1f} tokens/s")
        out.append(r)
    del banks
    torch.cuda.empty_cache()
    return out


def section_lm_head(args, device):
    """The fused int4 LM-head top-k (lm_head_int4_topk_fused, sycl:2137-2572; not a BASELINE config): one token's hidden
    state [1, 2048] against a 151936-row int4 head (group 128) in the reference's top-k layout,
    top 8.  Two weight copies (2 x 163 MB) alternate, more than the Infinity Cache."""
    from anna_amd import fused_ops
    from anna_amd.quantization import XPUInt4Linear

    K, V, TOPK = 2048, 151936, 8
    torch.manual_seed(31)
    dense = torch.nn.Linear(K, V, bias=False, dtype=torch.float32, device=device)
    q = XPUInt4Linear.from_linear(dense, group_size=128, compute_dtype=torch.bfloat16, device=device)
    del dense
    q.prepare_lm_head_topk_layout()
    base = (q.lm_head_qweight, q.lm_head_qscale, q.lm_head_qzeros)
    copies = [base, tuple(t.clone() for t in base)]
    x = torch.randn((1, K), device=device).to(torch.bfloat16)
    fused_ops.register_ops()
    fns = [(lambda c=c: torch.ops.anna.lm_head_int4_topk_fused(x, *c, 128, K, TOPK)) for c in copies]
    ms = time_graph(fns, args.steps, args.warmup)
    wbytes = V * K // 2 + V * (K // 128) * 3
    byts = wbytes + K * 2 + V * 4 * 2  # weights, x, fp32 logits written and read by the top-k
    r = {"K": K, "V": V, "top_k": TOPK, "us": ms * 1e3, "bytes": byts, "GB/s": byts / ms / 1e6,
         "roofline_frac": byts / ms / 1e6 / HBM_PEAK_GBS, "distinct_weight_copies": len(copies)}
    log(f"lm_head top-{TOPK} V={V} K={K}: {r['us']:.1f} us  {r['GB/s']:.0f} GB/s  "
        f"{100 * r['roofline_frac']:.1f}% of HBM peak")
    del copies, q, base
    torch.cuda.empty_cache()
    return r


def calibrate_copy(device, steps: int = 5) -> dict:
    """A plain elementwise kernel of known traffic (reads and writes COPY_BYTES each), run so
    that a counter collection run can scale FETCH_SIZE / WRITE_SIZE to bytes."""
    n = COPY_BYTES // 4
    src = torch.randn(n, device=device)
    dst = torch.empty_like(src)
    for _ in range(steps):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    log(f"calibration copy: {steps} x torch.neg over {COPY_BYTES} bytes (fp32)")
    return {"kernel": "torch.neg fp32 elementwise", "read_bytes": COPY_BYTES, "write_bytes": COPY_BYTES, "calls": steps}


TRAFFIC_FILE = ROOT / "profiles" / "int4_gemv_dot2_m1_n12288_k4096_traffic.txt"


def measured_traffic():
    """HBM bytes per launch of the headline kernel from the committed counter summary
    (FETCH_SIZE + WRITE_SIZE, scaled by the calibration copy); None if absent."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=60)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--sections", default="int4,tq_decode,row_decode,tq_pack,tq_rows,moe,lm_head")
    ap.add_argument("--tq-tokens-per-item", type=int, default=0)
    ap.add_argument("--tq-rows-dim", type=int, default=128, help="head_dim of the tq_rows section (64, 128, 256)")
    ap.add_argument("--tq-rows-bits", type=int, default=4, help="key/value bits of the tq_rows section (2, 3, 4)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--int4-points", default="", help="comma list of MxNxK (default: the BASELINE sweep)")
    ap.add_argument("--eager", action="store_true", help="launch steps one by one (counter collection runs)")
    ap.add_argument("--calibrate-copy", action="store_true", help="also run a known-size copy kernel")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(one GPU's share of the work is what it times); run with --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (no ROCm device visible)", file=sys.stderr)
        return 1
    device = torch.device("cuda", 0)
    from anna_amd import fused_ops

    fused_ops.register_ops()
    sections = {}
    if args.calibrate_copy:
        sections["calibration_copy"] = calibrate_copy(device)
    wanted = set(args.sections.split(","))
    if "int4" in wanted:
        sections["int4_sweep"] = section_int4(args, device)
    if "tq_decode" in wanted:
        sections["tq_decode"] = section_tq_decode(args, device)
    if "row_decode" in wanted:
        sections["row_decode"] = section_row_decode(args, device)
    if "tq_pack" in wanted:
        sections["tq_pack"] = section_tq_pack(args, device)
    if "tq_rows" in wanted:
        sections["tq_rows"] = section_tq_rows(args, device)
    if "moe" in wanted:
        sections["moe"] = section_moe(args, device)
    if "lm_head" in wanted:
        sections["lm_head"] = section_lm_head(args, device)
    if "int4_sweep" not in sections:
        print(json.dumps({"sections": sections}))
        return 0
    head = next((r for r in sections["int4_sweep"] if (r["M"], r["N"], r["K"]) == (1, 12288, 4096)),
                sections["int4_sweep"][0])
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_int4(1, 12288, 4096, 128, args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']:.2f} GB/s on {cpu['cores']} threads")
    line = {
        "metric": METRIC,
        "value": round(head["GB/s"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xbf16 (int4 weights, bf16 activations, fp32 accumulation)",
        "data": "synthetic (seeded codes U{0..15}, bf16 scales |N(0,0.02)|+1e-3, zero points U{0..15}, x ~N(0,1))",
        "config": {"workload": "W4A16 int4 GEMV, M=1 N=12288 K=4096 group=128 (BASELINE config 2, fused gate_up)",
                   "M": 1, "N": 12288, "K": 4096, "group_size": 128, "scale_dtype": "bf16"},
        "roofline": {"bound": "hbm", "achieved": round(head["GB/s"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["GB/s"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "bytes_per_launch": head["bytes"], "kernel": "int4_gemv_dot2"},
        "cpu_baseline": cpu,
        "sections": sections,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())

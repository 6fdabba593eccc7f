"""The MoE CPU restatements (oracle/cpu_paths.py) against brute force and invariants."""

import torch

from oracle import cpu_paths as cp


def test_route_matches_brute_force():
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(23, 16, generator=g).to(torch.bfloat16)
    w, sel, usage = cp.moe_route(logits, 4, True)
    p = torch.softmax(logits.double(), -1)
    for t in range(23):
        order = sorted(range(16), key=lambda e: (-float(p[t, e]), e))[:4]
        assert sel[t].tolist() == order
        top = p[t, order]
        torch.testing.assert_close(w[t].double(), top / top.sum(), rtol=1e-5, atol=1e-6)
    assert usage.sum() == 23 * 4 and usage.tolist() == [int((sel == e).sum()) for e in range(16)]


def test_sorted_assignments_order_and_offsets():
    sel = torch.tensor([[3, 1], [1, 0], [3, 2], [0, 3]])
    usage = torch.bincount(sel.reshape(-1), minlength=5)
    tok, rte, off = cp.moe_sorted_assignments(sel, usage, 5)
    # expert-major, then token, then k
    assert off.tolist() == [0, 2, 4, 5, 8, 8]
    pairs = list(zip(tok.tolist(), rte.tolist()))
    assert pairs == [(1, 1), (3, 0), (0, 1), (1, 0), (2, 1), (0, 0), (2, 0), (3, 1)]


def test_grouped_mlp_matches_per_route_loop():
    g = torch.Generator().manual_seed(9)
    h, i, e = 16, 8, 3
    experts = {k: (torch.randn(i, h, generator=g), torch.randn(i, h, generator=g), torch.randn(h, i, generator=g))
               for k in range(e)}
    x = torch.randn(7, h, generator=g)
    w = torch.rand(7, 1, generator=g)
    off = torch.tensor([0, 3, 3, 7])
    out = cp.moe_grouped_mlp(x, w, off, experts, torch.float64)
    for r in range(7):
        ex = 0 if r < 3 else 2
        wg, wu, wd = (m.double() for m in experts[ex])
        gate = wg @ x[r].double()
        act = torch.nn.functional.silu(gate) * (wu @ x[r].double())
        torch.testing.assert_close(out[r], (wd @ act) * float(w[r]), rtol=1e-12, atol=1e-12)


def test_scatter_sums_rows_per_token():
    co = torch.arange(12, dtype=torch.float32).view(4, 3)
    out = cp.moe_scatter(co, torch.tensor([1, 0, 1, 1]), 3)
    assert out.tolist() == [[3, 4, 5], [15, 18, 21], [0, 0, 0]]

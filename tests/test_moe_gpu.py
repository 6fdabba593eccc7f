"""MoE router / dispatch / grouped int4 MLP / scatter on the GPU against the CPU restatements.

Router indices, usage, dispatch order and offsets are exact; routing weights within 1e-5;
the grouped MLP within normwise relative error 1e-2 of the fp64 brute force over the
dequantized bank (the north-star bf16 tolerance; the reference's own op tests use 2e-2).
"""

import pytest
import torch

from anna_amd import fused_ops
from anna_amd.moe import GroupedInt4ExpertBank, SparseMoeInt4
from oracle import cpu_paths as cp
from tests._util import BF16_TOL, rel_err

pytestmark = pytest.mark.gpu


def make_bank(num_experts, hidden, inter, group, scale_dtype, device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def lin(n, k):
        qw = torch.randint(-(2**31), 2**31 - 1, (num_experts, n, k // 8), dtype=torch.int32, device=device, generator=g)
        qs = (torch.randn((num_experts, k // group, n), device=device, generator=g) * 0.02).abs_().add_(1e-3)
        qz = torch.randint(0, 16, (num_experts, k // group, n), dtype=torch.int8, device=device, generator=g)
        return qw, qs.to(scale_dtype), qz

    gq, gs, gz = lin(inter, hidden)
    uq, us, uz = lin(inter, hidden)
    dq, ds, dz = lin(hidden, inter)
    return GroupedInt4ExpertBank(num_experts, hidden, inter, group, gq, gs, gz, uq, us, uz, dq, ds, dz,
                                 list(range(num_experts)), {e: e for e in range(num_experts)})


def dequant_experts(bank, experts):
    out = {}
    for e in experts:
        s = bank.expert_to_slot[e]
        f = [cp.int4_dequant_f32(q[s].cpu(), sc[s].cpu(), z[s].cpu(), bank.group_size, k)
             for q, sc, z, k in ((bank.gate_qweight, bank.gate_qscale, bank.gate_qzeros, bank.hidden_dim),
                                 (bank.up_qweight, bank.up_qscale, bank.up_qzeros, bank.hidden_dim),
                                 (bank.down_qweight, bank.down_qscale, bank.down_qzeros, bank.intermediate_dim))]
        out[e] = tuple(f)
    return out


@pytest.mark.parametrize("tokens,experts,top_k,dtype,norm", [
    (11, 16, 4, torch.bfloat16, True),  # the reference test's shape (test_fused_op_xpu.py:948-966)
    (11, 16, 4, torch.bfloat16, False),
    (64, 128, 8, torch.float32, True),
    (5, 300, 8, torch.float16, True),
])
def test_router_matches_reference(gpu, tokens, experts, top_k, dtype, norm):
    torch.manual_seed(tokens + experts)
    logits = torch.randn(tokens, experts, device=gpu, dtype=dtype)
    w, sel, usage = torch.ops.anna.moe_router_fused(logits, top_k, norm)
    rw, rsel, rusage = cp.moe_route(logits.cpu(), top_k, norm)
    assert torch.equal(sel.cpu(), rsel)
    assert torch.equal(usage.cpu().long(), rusage.long())
    torch.testing.assert_close(w.cpu(), rw, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_dispatch_matches_cpu_order(gpu, dtype):
    torch.manual_seed(3)
    t, h, e, k = 37, 256, 16, 4
    hidden = torch.randn(t, h, device=gpu, dtype=dtype)
    w, sel, usage = fused_ops.moe_router(torch.randn(t, e, device=gpu), k, True)
    rw = w.to(dtype)
    pos = torch.empty(t * k, dtype=torch.int64, device=gpu)
    sti, off, compact, cw = fused_ops.moe_dispatch(hidden, rw, sel, usage, route_pos=pos)
    tok, rte, roff = cp.moe_sorted_assignments(sel.cpu(), usage.cpu(), e)
    assert torch.equal(sti.cpu(), tok) and torch.equal(off.cpu(), roff)
    assert torch.equal(compact.cpu(), hidden.cpu().index_select(0, tok))
    assert torch.equal(cw.cpu()[:, 0], rw.cpu()[tok, rte])
    # route_pos inverts the order
    assert torch.equal(sti.cpu()[pos.cpu()], torch.arange(t).repeat_interleave(k))
    # the op form returns the same
    sti2, off2, compact2, cw2 = torch.ops.anna.moe_dispatch_fused(hidden, rw, sel, usage.long())
    assert torch.equal(sti2, sti) and torch.equal(off2, off) and torch.equal(compact2, compact)


@pytest.mark.parametrize("hdt,sdt,group,tokens,h,i", [
    (torch.bfloat16, torch.float32, 128, 13, 256, 128),  # reference bank dtype (fp32 scales)
    (torch.bfloat16, torch.bfloat16, 128, 40, 256, 128),  # > 16 routes per expert (chunking)
    (torch.float16, torch.float32, 64, 9, 256, 128),
    (torch.float32, torch.float32, 32, 6, 256, 128),
    # dims multiple of 256, group 128, 16-bit activations and >= 16 routes per active expert: the
    # wide kernels (one sweep of up to 48 routes per expert, K in passes of 256); 100 tokens x 3
    # routes over 8 experts put ~37 routes on an expert (one 48-route sweep), 200 tokens ~75 (a
    # 48-route sweep and a short one); 5 tokens stay on the 16-route kernels
    (torch.bfloat16, torch.bfloat16, 128, 5, 512, 256),
    (torch.bfloat16, torch.float32, 128, 100, 512, 256),
    (torch.float16, torch.bfloat16, 128, 100, 768, 512),
    (torch.bfloat16, torch.bfloat16, 128, 200, 512, 256),
])
def test_grouped_int4_mlp_matches_oracle(gpu, hdt, sdt, group, tokens, h, i):
    print(f"[case] moe grouped MLP {hdt} scales {sdt} group {group} tokens {tokens} h {h} i {i}", flush=True)
    torch.manual_seed(7)
    e, k = 8, 3
    bank = make_bank(e, h, i, group, sdt, gpu, seed=11 + tokens)
    hidden = torch.randn(tokens, h, device=gpu, dtype=hdt)
    w, sel, usage = fused_ops.moe_router(torch.randn(tokens, e, device=gpu), k, True)
    sti, off, compact, cw = fused_ops.moe_dispatch(hidden, w.to(hdt), sel, usage)
    out = torch.full_like(compact, 7.0)
    active = [0, 2, 3, 5, 6, 7]  # experts 1 and 4 inactive: their rows stay untouched
    act_t = torch.tensor(active, dtype=torch.int64, device=gpu)
    res = torch.ops.anna.moe_grouped_int4_mlp_fused(compact, cw, out, off, act_t, act_t, *bank.tensors(), group,
                                                   int(usage.max()))
    assert res.data_ptr() == out.data_ptr()
    offc = off.cpu()
    ref = cp.moe_grouped_mlp(compact.cpu(), cw.cpu(), offc, dequant_experts(bank, active), torch.float64)
    rows = torch.cat([torch.arange(int(offc[x]), int(offc[x + 1])) for x in active])
    got = out.cpu().double()
    assert rel_err(got[rows].numpy(), ref[rows].numpy()) <= BF16_TOL
    inactive = torch.cat([torch.arange(int(offc[x]), int(offc[x + 1])) for x in (1, 4)])
    assert bool((out.cpu()[inactive] == 7.0).all())


@pytest.mark.parametrize("hdt", [torch.bfloat16, torch.float16])
def test_grouped_int4_mlp_skewed_routes(gpu, hdt):
    """Few routes per expert on average (the resident gate/up form: 16 routes per sweep with all
    of K in LDS) but one expert carrying every token (40 routes: three sweeps) against the fp64
    oracle."""
    print(f"[case] moe grouped MLP skewed routes {hdt}", flush=True)
    torch.manual_seed(17)
    e, k, h, i, tokens, group = 16, 2, 512, 256, 40, 128
    bank = make_bank(e, h, i, group, torch.bfloat16, gpu, seed=23)
    hidden = torch.randn(tokens, h, device=gpu, dtype=hdt)
    logits = torch.randn(tokens, e, device=gpu)
    logits[:, 0] += 8.0  # expert 0 is everyone's first choice
    w, sel, usage = fused_ops.moe_router(logits, k, True)
    assert int(usage[0]) == tokens
    sti, off, compact, cw = fused_ops.moe_dispatch(hidden, w.to(hdt), sel, usage)
    out = torch.full_like(compact, 7.0)
    every = torch.arange(e, dtype=torch.int64, device=gpu)
    fused_ops.moe_grouped_int4_mlp_out(compact, cw, out, off, every, every, *bank.tensors(), group, int(usage.max()))
    offc = off.cpu()
    ref = cp.moe_grouped_mlp(compact.cpu(), cw.cpu(), offc, dequant_experts(bank, range(e)), torch.float64)
    assert rel_err(out.cpu().double().numpy(), ref.numpy()) <= BF16_TOL


@pytest.mark.parametrize("tokens,sdt,group", [(6, torch.bfloat16, 128), (40, torch.float32, 128), (9, torch.float32, 64)])
def test_grouped_int4_mlp_item_list_matches_grid(gpu, tokens, sdt, group):
    """The device-listed (persistent) form walks only experts with routes and gives the same
    bits as the one-workgroup-per-expert grid; experts without routes stay untouched."""
    print(f"[case] moe grouped MLP item list tokens={tokens} scales={sdt} group={group}", flush=True)
    torch.manual_seed(3)
    e, k, h, i = 24, 2, 512, 256
    bank = make_bank(e, h, i, group, sdt, gpu, seed=5 + tokens)
    hidden = torch.randn(tokens, h, device=gpu, dtype=torch.bfloat16)
    w, sel, usage = fused_ops.moe_router(torch.randn(tokens, e, device=gpu), k, True)
    sti, off, compact, cw = fused_ops.moe_dispatch(hidden, w.to(torch.bfloat16), sel, usage)
    every = torch.arange(e, dtype=torch.int64, device=gpu)  # empty experts included, as SparseMoeInt4 passes them
    out_grid = torch.full_like(compact, 7.0)
    out_list = torch.full_like(compact, 7.0)
    mx = int(usage.max())
    fused_ops.moe_grouped_int4_mlp_out(compact, cw, out_grid, off, every, every, *bank.tensors(), group, mx)
    items = torch.full((4 + 4 * e,), -1, dtype=torch.int32, device=gpu)
    fused_ops.moe_grouped_int4_mlp_out(compact, cw, out_list, off, every, every, *bank.tensors(), group, mx, items=items)
    assert torch.equal(out_grid, out_list)
    assert int(items[0]) == int((usage > 0).sum())


@pytest.mark.parametrize("tokens,experts,top_k,ldt", [(8, 128, 8, torch.float32), (11, 16, 4, torch.bfloat16),
                                                      (128, 128, 8, torch.float32), (3, 300, 2, torch.float16)])
def test_route_small_matches_router_and_dispatch(gpu, tokens, experts, top_k, ldt):
    """The one-launch router + dispatch order gives exactly the separate ops' outputs, and its
    item list names the experts with routes, in order, with their bank slot and route range."""
    print(f"[case] moe route_small tokens={tokens} experts={experts} k={top_k} logits={ldt}", flush=True)
    torch.manual_seed(tokens + experts)
    logits = torch.randn(tokens, experts, device=gpu).to(ldt)
    if tokens >= 8:
        logits[1] = logits[0]  # identical rows: ties between tokens
    hidden = torch.randn(tokens, 64, device=gpu, dtype=torch.bfloat16)
    slots = torch.randperm(experts, device=gpu).to(torch.int64)
    w, sel, usage = fused_ops.moe_router(logits, top_k, True)
    route_pos = torch.empty((tokens * top_k,), dtype=torch.int64, device=gpu)
    sti, off, compact, cw = fused_ops.moe_dispatch(hidden, w.to(torch.bfloat16), sel, usage, route_pos=route_pos)
    w2, sel2, usage2, off2, sti2, sri2, rp2, items = fused_ops.moe_route_small(logits, top_k, True, slots)
    assert torch.equal(w, w2) and torch.equal(sel, sel2) and torch.equal(usage, usage2)
    assert torch.equal(off, off2) and torch.equal(sti, sti2) and torch.equal(route_pos, rp2)
    compact2, cw2 = fused_ops.moe_gather(hidden, w2, sri2, top_k)
    assert torch.equal(compact, compact2) and torch.equal(cw, cw2)
    offc, uc, sl = off.cpu(), usage.cpu(), slots.cpu()
    have = [e for e in range(experts) if int(uc[e]) > 0]
    it = items.cpu()
    assert int(it[0]) == len(have)
    for j, e in enumerate(have):
        assert [int(v) for v in it[4 + 4 * j: 7 + 4 * j]] == [int(sl[e]), int(offc[e]), int(offc[e + 1])]
    # the dispatch writes the same list when given the slots, and takes the router's fp32
    # weights directly (rounded to bf16 in the gather, as the cast above did)
    items_d = torch.full((4 + 4 * experts,), -1, dtype=torch.int32, device=gpu)
    rp3 = torch.empty_like(route_pos)
    sti3, off3, compact3, cw3 = fused_ops.moe_dispatch(hidden, w, sel, usage, route_pos=rp3, slots=slots, items=items_d)
    assert torch.equal(sti, sti3) and torch.equal(off, off3) and torch.equal(route_pos, rp3)
    assert torch.equal(compact, compact3) and torch.equal(cw, cw3)
    n = 4 + 4 * len(have)
    assert int(items_d[0]) == len(have)
    assert torch.equal(items_d[4:n].reshape(-1, 4)[:, :3].cpu(), it[4:n].reshape(-1, 4)[:, :3])


def test_scatter_and_combine(gpu):
    torch.manual_seed(4)
    t, h, e, k = 29, 384, 12, 3
    w, sel, usage = fused_ops.moe_router(torch.randn(t, e, device=gpu), k, True)
    pos = torch.empty(t * k, dtype=torch.int64, device=gpu)
    sti, off, compact, cw = fused_ops.moe_dispatch(torch.randn(t, h, device=gpu, dtype=torch.bfloat16),
                                                    w.to(torch.bfloat16), sel, usage, route_pos=pos)
    co = torch.randn(t * k, h, device=gpu, dtype=torch.bfloat16)
    ref = cp.moe_scatter(co.cpu(), sti.cpu(), t)
    a = torch.ops.anna.moe_scatter_fused(co, sti, t)
    b = fused_ops.moe_combine(co, pos, t, k)
    torch.testing.assert_close(a.cpu().float(), ref.float(), rtol=8e-3, atol=1e-2)
    torch.testing.assert_close(b.cpu().float(), ref.float(), rtol=8e-3, atol=1e-2)


@pytest.mark.parametrize("tokens", [8, 64])
def test_sparse_moe_block_matches_cpu_chain(gpu, tokens):
    torch.manual_seed(tokens)
    e, k, h, i, group = 16, 4, 256, 128, 128
    bank = make_bank(e, h, i, group, torch.bfloat16, gpu, seed=5)
    block = SparseMoeInt4(bank, num_experts=e, top_k=k)
    hidden = torch.randn(tokens, h, device=gpu, dtype=torch.bfloat16)
    logits = torch.randn(tokens, e, device=gpu, dtype=torch.float32)
    out = block(hidden, logits)
    w, sel, usage = cp.moe_route(logits.cpu(), k, True)
    tok, rte, off = cp.moe_sorted_assignments(sel, usage, e)
    compact = hidden.cpu().index_select(0, tok)
    cw = w.to(torch.bfloat16)[tok, rte].unsqueeze(1)
    co = cp.moe_grouped_mlp(compact, cw, off, dequant_experts(bank, range(e)), torch.float64)
    ref = torch.zeros(tokens, h, dtype=torch.float64).index_add_(0, tok, co)
    assert rel_err(out.cpu().double().numpy(), ref.numpy()) <= BF16_TOL


@pytest.mark.parametrize("tokens", [8, 64, 512])
def test_sparse_moe_block_config5_dims(gpu, tokens):
    """BASELINE config 5 at its own dims: 128 experts, top-8 of softmax(N(0,1) logits),
    H=2048, I=512, group 128, bf16 scales.  T=512 gives ~32 routes per expert (multi-sweep
    experts); T=8 and 64 take the one-launch routing path.  Both the block (device item list)
    and the op with a host-known max_routes_per_expert (the reference caller's form) are
    checked against the fp64 brute force over the dequantized bank."""
    print(f"[case] moe config5 dims tokens={tokens}", flush=True)
    torch.manual_seed(500 + tokens)
    e, k, h, i, group = 128, 8, 2048, 512, 128
    bank = make_bank(e, h, i, group, torch.bfloat16, gpu, seed=77)
    block = SparseMoeInt4(bank, num_experts=e, top_k=k)
    hidden = torch.randn(tokens, h, device=gpu, dtype=torch.bfloat16)
    logits = torch.randn(tokens, e, device=gpu, dtype=torch.float32)
    out = block(hidden, logits)
    w, sel, usage = cp.moe_route(logits.cpu(), k, True)
    tok, rte, off = cp.moe_sorted_assignments(sel, usage, e)
    active = [x for x in range(e) if int(usage[x]) > 0]
    deq = dequant_experts(bank, active)
    compact = hidden.cpu().index_select(0, tok)
    cw = w.to(torch.bfloat16)[tok, rte].unsqueeze(1)
    co = cp.moe_grouped_mlp(compact, cw, off, deq, torch.float64)
    ref = torch.zeros(tokens, h, dtype=torch.float64).index_add_(0, tok, co)
    assert rel_err(out.cpu().double().numpy(), ref.numpy()) <= BF16_TOL
    # the op itself, every active expert listed by the host, max_routes from the usage
    gw, gsel, gusage = fused_ops.moe_router(logits, k, True)
    sti, goff, gcompact, gcw = fused_ops.moe_dispatch(hidden, gw.to(torch.bfloat16), gsel, gusage)
    act_t = torch.tensor(active, dtype=torch.int64, device=gpu)
    res = torch.ops.anna.moe_grouped_int4_mlp_fused(gcompact, gcw, torch.empty_like(gcompact), goff, act_t, act_t,
                                                   *bank.tensors(), group, int(gusage.max()))
    assert rel_err(res.cpu().double().numpy(), co.numpy()) <= BF16_TOL

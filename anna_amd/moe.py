"""Sparse MoE block over a grouped int4 expert bank (MI355X).

Mirrors the quantized expert path of Qwen3SparseMoeBlock (src/anna/model/ops.py:3280-3457,
bank dataclass ops.py:73-89): route (softmax -> top-k -> renorm), dispatch the routes sorted
by (expert, token, k), run the grouped int4 SwiGLU MLP of every expert on its routes, and
combine the routes back per token.  Unlike the reference, which syncs to the host for the
list of hit experts (ops.py:3530, 3541), every expert of the bank is passed as active: the
kernels skip experts without routes, so a step makes no host round trip.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import fused_ops
from .quantization import XPUInt4Linear


@dataclass
class GroupedInt4ExpertBank:
    """Stacked XPUInt4Linear buffers of the experts (reference _GroupedInt4ExpertBank)."""

    capacity: int
    hidden_dim: int
    intermediate_dim: int
    group_size: int
    gate_qweight: torch.Tensor
    gate_qscale: torch.Tensor
    gate_qzeros: torch.Tensor
    up_qweight: torch.Tensor
    up_qscale: torch.Tensor
    up_qzeros: torch.Tensor
    down_qweight: torch.Tensor
    down_qscale: torch.Tensor
    down_qzeros: torch.Tensor
    slot_to_expert: list = field(default_factory=list)
    expert_to_slot: dict = field(default_factory=dict)

    def tensors(self):
        return (self.gate_qweight, self.gate_qscale, self.gate_qzeros, self.up_qweight, self.up_qscale,
                self.up_qzeros, self.down_qweight, self.down_qscale, self.down_qzeros)

    @classmethod
    def from_linears(cls, experts: list[tuple[XPUInt4Linear, XPUInt4Linear, XPUInt4Linear]]) -> "GroupedInt4ExpertBank":
        """Bank of the (gate_proj, up_proj, down_proj) triples, slot i = expert i."""
        if not experts:
            raise RuntimeError("a grouped int4 expert bank needs at least one expert")
        g0, u0, d0 = experts[0]
        h, i = g0.in_features, g0.out_features
        for g, u, d in experts:
            if (g.in_features, g.out_features) != (h, i) or (u.in_features, u.out_features) != (h, i):
                raise RuntimeError("Grouped int4 expert GEMM requires gate_proj/up_proj to share the same shape.")
            if (d.in_features, d.out_features) != (i, h):
                raise RuntimeError("Grouped int4 expert GEMM requires down_proj to invert gate_proj dimensions.")
            if not (g.group_size == u.group_size == d.group_size == g0.group_size):
                raise RuntimeError("Grouped int4 expert GEMM requires a shared int4 group size.")

        def stack(attr, which):
            return torch.stack([getattr(e[which], attr) for e in experts]).contiguous()

        n = len(experts)
        return cls(capacity=n, hidden_dim=h, intermediate_dim=i, group_size=g0.group_size,
                   gate_qweight=stack("qweight", 0), gate_qscale=stack("qscale", 0), gate_qzeros=stack("qzeros", 0),
                   up_qweight=stack("qweight", 1), up_qscale=stack("qscale", 1), up_qzeros=stack("qzeros", 1),
                   down_qweight=stack("qweight", 2), down_qscale=stack("qscale", 2), down_qzeros=stack("qzeros", 2),
                   slot_to_expert=list(range(n)), expert_to_slot={e: e for e in range(n)})


class SparseMoeInt4:
    """Routed experts of one MoE layer on a resident grouped int4 bank."""

    def __init__(self, bank: GroupedInt4ExpertBank, *, num_experts: int, top_k: int, norm_topk_prob: bool = True):
        if bank.capacity < num_experts:
            raise RuntimeError("the bank must hold every expert (resident mode)")
        self.bank, self.num_experts, self.top_k, self.norm_topk_prob = bank, num_experts, top_k, norm_topk_prob
        dev = bank.gate_qweight.device
        self.active_experts = torch.arange(num_experts, dtype=torch.int64, device=dev)
        self.active_slots = torch.tensor([bank.expert_to_slot[e] for e in range(num_experts)], dtype=torch.int64,
                                         device=dev)

    def forward(self, hidden_states: torch.Tensor, router_logits: torch.Tensor) -> torch.Tensor:
        """hidden_states [T, H], router_logits [T, E] -> routed expert output [T, H] (hidden dtype)."""
        t = hidden_states.shape[0]
        # decode-sized batches: router + dispatch order + the MLP's list of experts with routes in
        # one launch (its single workgroup ranks each route against the earlier ones, which pays
        # only while the routes are few)
        small = t * self.top_k <= 128 and self.num_experts <= 512 and self.top_k <= 64
        if small:
            w, sel, usage, offsets, _, sri, route_pos, items = fused_ops.moe_route_small(
                router_logits, self.top_k, self.norm_topk_prob, self.active_slots)
            compact, cw = fused_ops.moe_gather(hidden_states, w, sri, self.top_k)
        else:
            w, sel, usage = fused_ops.moe_router(router_logits, self.top_k, self.norm_topk_prob)
            route_pos = torch.empty((t * self.top_k,), dtype=torch.int64, device=hidden_states.device)
            # every expert is passed as active; the dispatch lists the ones with routes (items)
            items = torch.empty((4 + 4 * self.num_experts,), dtype=torch.int32, device=hidden_states.device)
            _, offsets, compact, cw = fused_ops.moe_dispatch(hidden_states, w, sel, usage, route_pos=route_pos,
                                                              slots=self.active_slots, items=items)
        compact_out = torch.empty_like(compact)
        # Routes per expert are only known on the device; the kernels sweep an expert's routes in
        # as many passes as it needs, so this hint (twice the mean load) only sizes the sweep.
        hint = min(t * self.top_k, 2 * -(-t * self.top_k // self.num_experts) + 8)
        fused_ops.moe_grouped_int4_mlp_out(compact, cw, compact_out, offsets, self.active_experts, self.active_slots,
                                           *self.bank.tensors(), self.bank.group_size, max(1, hint), items=items,
                                           items_prefilled=True)
        return fused_ops.moe_combine(compact_out, route_pos, t, self.top_k)

    __call__ = forward

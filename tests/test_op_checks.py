"""Argument checks of the anna:: ops run on the host, before any pointer reaches the library.

Every case here uses CPU tensors: a check that is missing would let the call go on to the
device check (or, on a GPU, to a kernel reading out of bounds), so each test asserts the
reference's own message (validate_gqa_decode_splitkv_turboquant_inputs sycl:1447-1501,
validate_gqa_decode_optional_gate sycl:1605-1629)."""

import pytest
import torch

from anna_amd import fused_ops

B, HQ, HKV, L, R, D, G = 2, 8, 2, 20, 4, 64, 16


def tq_inputs(**over):
    bf = torch.bfloat16
    t = dict(
        query=torch.zeros(B, HQ, 1, D, dtype=bf),
        quantized_key=torch.zeros(B, HKV, L, D, dtype=bf),
        value_data=torch.zeros(B, HKV, L, D // 4, dtype=torch.uint8),
        value_scales=torch.zeros(B, HKV, L, D // G, dtype=bf),
        value_zeros=torch.zeros(B, HKV, L, D // G, dtype=bf),
        residual_key=torch.zeros(B, HKV, R, D, dtype=bf),
        residual_value=torch.zeros(B, HKV, R, D, dtype=bf),
    )
    nblk = fused_ops._splitkv_num_blocks(L + R, 16)
    t.update(output=torch.zeros(B, HQ, 1, D, dtype=bf), partial_stats=torch.zeros(B, HQ, nblk, 2),
             partial_values=torch.zeros(B, HQ, nblk, D))
    t.update(over)
    return t


def run_tq(t, value_bits=2, group=G, block=16, gate=None):
    return fused_ops._gqa_decode_splitkv_turboquant_fused_out_impl(
        t["query"], t["quantized_key"], t["value_data"], t["value_scales"], t["value_zeros"], t["residual_key"],
        t["residual_value"], t["output"], t["partial_stats"], t["partial_values"], 0.125, value_bits, group, block,
        gate)


def test_valid_inputs_reach_the_device_check():
    with pytest.raises(RuntimeError, match="ROCm device tensors"):
        run_tq(tq_inputs())


@pytest.mark.parametrize("over,msg", [
    (dict(quantized_key=torch.zeros(B + 1, HKV, L, D, dtype=torch.bfloat16)), "query/quantized_key batch size"),
    (dict(residual_key=torch.zeros(B + 1, HKV, R, D, dtype=torch.bfloat16),
          residual_value=torch.zeros(B + 1, HKV, R, D, dtype=torch.bfloat16)), "query/residual_key batch size"),
    (dict(quantized_key=torch.zeros(B, HKV, L, D // 2, dtype=torch.bfloat16)), "query/quantized_key head_dim"),
    (dict(residual_key=torch.zeros(B, HKV, R, D // 2, dtype=torch.bfloat16),
          residual_value=torch.zeros(B, HKV, R, D // 2, dtype=torch.bfloat16)), "query/residual_key head_dim"),
    (dict(value_data=torch.zeros(B - 1, HKV, L, D // 4, dtype=torch.uint8)), "value_data batch size"),
    (dict(value_data=torch.zeros(B, 1, L, D // 4, dtype=torch.uint8)), "value_data kv head count"),
    (dict(value_data=torch.zeros(B, HKV, L - 1, D // 4, dtype=torch.uint8)), "value_data quantized_len"),
    (dict(value_scales=torch.zeros(B - 1, HKV, L, D // G, dtype=torch.bfloat16)), "value_scales batch size"),
    (dict(value_scales=torch.zeros(B, 1, L, D // G, dtype=torch.bfloat16)), "value_scales kv head count"),
    (dict(value_scales=torch.zeros(B, HKV, L - 1, D // G, dtype=torch.bfloat16)), "value_scales quantized_len"),
    (dict(value_zeros=torch.zeros(B, HKV, L - 1, D // G, dtype=torch.bfloat16)), "value_zeros shape must match"),
    (dict(value_data=torch.zeros(B, HKV, L, D // 8, dtype=torch.uint8)), "packed value width"),
    (dict(value_data=torch.zeros(B, HKV, L, D // 4, dtype=torch.int8)), "value_data must be uint8"),
    (dict(value_scales=torch.zeros(B, HKV, L, D // G), value_zeros=torch.zeros(B, HKV, L, D // G)),
     "must share the same dtype"),
    (dict(query=torch.zeros(B, HQ, 2, D, dtype=torch.bfloat16)), "single-token query"),
    (dict(quantized_key=torch.zeros(B, HKV, 0, D, dtype=torch.bfloat16)), "non-empty quantized prefix"),
])
def test_turboquant_shape_checks(over, msg):
    with pytest.raises(RuntimeError, match=msg):
        run_tq(tq_inputs(**over))


@pytest.mark.parametrize("kw,msg", [
    (dict(value_bits=5), "value_bits must be 2, 3, or 4"),
    (dict(group=0), "value_group_size must be positive"),
    (dict(group=24), "evenly divide head_dim"),
    (dict(block=8), "block_size must be at least 16"),
])
def test_turboquant_scalar_checks(kw, msg):
    with pytest.raises(RuntimeError, match=msg):
        run_tq(tq_inputs(), **kw)


def test_workspace_capacity_check():
    t = tq_inputs(partial_stats=torch.zeros(B, HQ, 1, 2))
    with pytest.raises(RuntimeError, match="partial_stats shape/capacity"):
        run_tq(t)


@pytest.mark.parametrize("gate,msg", [
    (torch.zeros(B, 1, HQ * D), "gate must match query dtype"),
    (torch.zeros(B - 1, 1, HQ * D, dtype=torch.bfloat16), "gate batch size mismatch"),
    (torch.zeros(B, 1, HQ * D + 1, dtype=torch.bfloat16), "gate must be"),
])
def test_gate_checks(gate, msg):
    with pytest.raises(RuntimeError, match=msg):
        run_tq(tq_inputs(), gate=gate)
    q = torch.zeros(B, HQ, 1, D, dtype=torch.bfloat16)
    k = torch.zeros(B, HKV, L, D, dtype=torch.bfloat16)
    nblk = fused_ops._splitkv_num_blocks(L, 16)
    with pytest.raises(RuntimeError, match=msg):
        fused_ops._gqa_decode_splitkv_fused_out_impl(q, k, k.clone(), torch.zeros_like(q),
                                                     torch.zeros(B, HQ, nblk, 2), torch.zeros(B, HQ, nblk, D),
                                                     0.125, 16, gate)


def test_moe_combine_checks_route_pos():
    co = torch.zeros(8, 16, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="route_pos must be int64"):
        fused_ops.moe_combine(co, torch.zeros(8, dtype=torch.int32), 4, 2)
    with pytest.raises(RuntimeError, match="route_pos must be int64"):
        fused_ops.moe_combine(co, torch.zeros(6, dtype=torch.int64), 4, 2)
    with pytest.raises(RuntimeError, match="fewer compact rows"):
        fused_ops.moe_combine(co, torch.zeros(10, dtype=torch.int64), 5, 2)

"""The three operators as PyTorch custom ops (torch.library), for graph capture, torch.compile and framework use.

This fills the role of the reference's (empty) framework adapter, framework/CMakeLists.txt:1-9: the operators
registered under the reference's names, with its attributes, over the same C ABI as `ops`:

    torch.ops.moe_mi355x.MoeRoutingTopK(x, w_gate, topK=2) -> (expert_ids, weights)
    torch.ops.moe_mi355x.MoeExpertFFN(x, expert_ids, weights, expert_weights, intermediateSize=0) -> expert_out
    torch.ops.moe_mi355x.MoeCombine(expert_out, expert_ids, weights, topK=2) -> y

The device implementation is registered for GPU tensors only: a CPU tensor finds no kernel (there is no CPU
fallback). The fake (meta) implementations state the InferShape / InferDataType rules of
op_host/moe_ops.cpp:181-226, 364-398, 495-525 so that tracers can propagate shapes without running anything;
argument errors that need the data (ids out of range and the like) are the device implementation's.
Importing this module registers the ops once per process.
"""
from __future__ import annotations

import torch

from . import ops

NAMESPACE = "moe_mi355x"


def _routing_shape(x, w_gate, topK):
    if x.dim() != 2 or w_gate.dim() != 2:
        raise RuntimeError("MoeRoutingTopK: x must be [T, H] and w_gate [H, E]")
    if x.shape[1] != w_gate.shape[0]:
        raise RuntimeError("MoeRoutingTopK: hiddenSize mismatch between x and w_gate")
    k = topK if topK > 0 else 2  # the attr default, op_host/moe_ops.cpp:201-204
    return (x.shape[0], k)


@torch.library.custom_op(f"{NAMESPACE}::MoeRoutingTopK", mutates_args=(), device_types="cuda")
def moe_routing_topk(x: torch.Tensor, w_gate: torch.Tensor, topK: int = 2) -> tuple[torch.Tensor, torch.Tensor]:
    ids, w = ops.MoeRoutingTopK(x, w_gate, topK)
    return ids, w


@moe_routing_topk.register_fake
def _(x, w_gate, topK=2):
    shape = _routing_shape(x, w_gate, topK)
    return x.new_empty(shape, dtype=torch.int32), x.new_empty(shape, dtype=torch.float16)


@torch.library.custom_op(f"{NAMESPACE}::MoeExpertFFN", mutates_args=(), device_types="cuda")
def moe_expert_ffn(x: torch.Tensor, expert_ids: torch.Tensor, weights: torch.Tensor, expert_weights: torch.Tensor,
                   intermediateSize: int = 0) -> torch.Tensor:
    return ops.MoeExpertFFN(x, expert_ids, weights, expert_weights, intermediateSize)


@moe_expert_ffn.register_fake
def _(x, expert_ids, weights, expert_weights, intermediateSize=0):
    if x.dim() != 2 or expert_ids.dim() != 2 or expert_weights.dim() != 3:
        raise RuntimeError("MoeExpertFFN: x [T, H], expert_ids [T, K], expert_weights [E, 3I, H] expected")
    return x.new_empty((x.shape[0], expert_ids.shape[1], x.shape[1]), dtype=torch.float16)


@torch.library.custom_op(f"{NAMESPACE}::MoeCombine", mutates_args=(), device_types="cuda")
def moe_combine(expert_out: torch.Tensor, expert_ids: torch.Tensor | None, weights: torch.Tensor,
                topK: int = 2) -> torch.Tensor:
    return ops.MoeCombine(expert_out, expert_ids, weights, topK)


@moe_combine.register_fake
def _(expert_out, expert_ids, weights, topK=2):
    if expert_out.dim() != 3:
        raise RuntimeError("MoeCombine: expert_out must be [T, K, H]")
    return expert_out.new_empty((expert_out.shape[0], expert_out.shape[2]), dtype=torch.float16)


def moe_layer(x: torch.Tensor, w_gate: torch.Tensor, expert_weights: torch.Tensor, topK: int = 2) -> torch.Tensor:
    """The reference's chain of the three operators (tests/test_moe.cpp:444-463) through the registered ops."""
    op = getattr(torch.ops, NAMESPACE)
    ids, w = op.MoeRoutingTopK(x, w_gate, topK)
    eo = op.MoeExpertFFN(x, ids, w, expert_weights, 0)
    return op.MoeCombine(eo, ids, w, topK)

"""FusedMoE drop-in: the 16-bit / int8 SparseMoeBlock replacement on libi4moe.

Mirrors src/duplex/streaming/fused_moe.py:40-179:
  - FusedMoE(block, chunk=8, q8=False) stacks a block's experts into gate|up
    [E, 2I, H] (gate rows first) and down [E, H, I] (:73-83), optionally as
    per-output-channel symmetric int8 with one scale per output row (:84-97),
    and keeps the sigmoid-gated shared expert of the Talker's block (:60-71);
  - forward(hidden_states) = routed experts + sigmoid(shared_gate(x)) *
    shared_expert(x) (:99-141), run as three launches of libi4moe (router
    logits; routing + gate|up + SiLU for every slot, the shared expert
    included; down + weighted combine) for any number of tokens;
  - fuse_moe_blocks(model, q8) swaps every unquantized SparseMoeBlock
    (:144-179).
Both block forms are accepted: experts as a ModuleList of gate_proj / up_proj /
down_proj Linears (the form fused_moe.py reads), or as the stacked
gate_up_proj [E, 2I, H] / down_proj [E, H, I] parameters of transformers 5.x
(Qwen3OmniMoeTalkerTextExperts, modeling_qwen3_omni_moe.py:2673-2683), whose
router is a module holding weight / top_k / norm_topk_prob.

`chunk` bounds the reference's gathered copies of the selected experts
(fused_moe.py:112-116); the kernels gather nothing (each token's workgroups read
their experts' rows in place), so it is kept for the interface only.  The int8
format is the reference's, computed the same way (the q8 buffers of a block are
identical to the reference's): s = amax_k |W| / 127 in the weights' dtype,
q = clamp(round(W / s), -127, 127).  The kernels apply s to each finished row
dot product in fp32 instead of rounding q * s to 16 bits per weight first.
"""
from __future__ import annotations

import gc

import torch
import torch.nn as nn

from . import ops


def quantize_q8(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel symmetric int8 of a [..., N, K] weight (fused_moe.py:84-94):
    (q int8 [..., N, K], s [..., N, 1] in w's dtype), w ~ q * s."""
    s = w.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8) / 127.0
    q = (w / s).round().clamp_(-127, 127).to(torch.int8)
    return q, s.to(w.dtype)


def _expert_stacks(experts: nn.Module, device) -> tuple[torch.Tensor, torch.Tensor, int]:
    """(gate_up [E, 2I, H], down [E, H, I], I) from either expert container."""
    if hasattr(experts, "gate_up_proj"):  # transformers 5.x stacked parameters
        gu = experts.gate_up_proj.detach().to(device).contiguous()
        dn = experts.down_proj.detach().to(device).contiguous()
        return gu, dn, gu.shape[1] // 2
    e0 = experts[0]
    inter, hidden = e0.gate_proj.weight.shape
    dtype = e0.gate_proj.weight.dtype
    E = len(experts)
    gu = torch.empty(E, 2 * inter, hidden, dtype=dtype, device=device)
    dn = torch.empty(E, hidden, inter, dtype=dtype, device=device)
    for i, e in enumerate(experts):
        gu[i, :inter] = e.gate_proj.weight.detach()
        gu[i, inter:] = e.up_proj.weight.detach()
        dn[i] = e.down_proj.weight.detach()
    return gu, dn, inter


def _is_packed(block: nn.Module) -> bool:
    experts = block.experts
    if hasattr(experts, "gate_up_proj"):
        return False
    gp = getattr(experts[0], "gate_proj", None)
    return gp is None or hasattr(gp, "weight_packed") or not hasattr(gp, "weight")


class FusedMoE(nn.Module):
    """Drop-in replacement for a SparseMoeBlock with 16-bit experts (optionally
    stored as int8), with or without a sigmoid-gated shared expert."""

    def __init__(self, block: nn.Module, chunk: int = 8, q8: bool = False, device=None):
        super().__init__()
        self.chunk = chunk
        self.q8 = q8
        self.workspace = ops.Workspace()
        gate = block.gate
        router_w = gate.weight.detach()
        dev = torch.device(device) if device is not None else router_w.device
        self.gate = gate
        self.top_k = int(getattr(block, "top_k", None) or gate.top_k)
        self.norm_topk_prob = bool(getattr(block, "norm_topk_prob",
                                           getattr(gate, "norm_topk_prob", True)))
        gu, dn, inter = _expert_stacks(block.experts, dev)
        self.num_experts = gu.shape[0]
        self.inter = inter
        self.hidden = gu.shape[2]
        dtype = gu.dtype
        self.register_buffer("router_w", router_w.to(dev, dtype).contiguous(), persistent=False)
        if q8:
            gu_q, gu_s = quantize_q8(gu)
            dn_q, dn_s = quantize_q8(dn)
            del gu, dn
            self.register_buffer("gate_up", gu_q, persistent=False)
            self.register_buffer("down", dn_q, persistent=False)
            self.register_buffer("gate_up_s", gu_s.contiguous(), persistent=False)
            self.register_buffer("down_s", dn_s.contiguous(), persistent=False)
        else:
            self.register_buffer("gate_up", gu, persistent=False)
            self.register_buffer("down", dn, persistent=False)
            self.gate_up_s = self.down_s = None
        # shared expert (the Talker's block; fused_moe.py:60-71): kept 16-bit, as
        # the reference keeps its shared_expert module unquantized
        se = getattr(block, "shared_expert", None)
        seg = getattr(block, "shared_expert_gate", None)
        if se is not None:
            sgu = torch.cat((se.gate_proj.weight.detach(), se.up_proj.weight.detach()), 0)
            self.register_buffer("shared_gate_up", sgu.to(dev, dtype).contiguous(),
                                 persistent=False)
            self.register_buffer("shared_down",
                                 se.down_proj.weight.detach().to(dev, dtype).contiguous(),
                                 persistent=False)
            self.shared_inter = sgu.shape[0] // 2
        else:
            self.shared_gate_up = self.shared_down = None
            self.shared_inter = 0
        if se is not None and seg is not None:
            self.register_buffer("shared_gate_w",
                                 seg.weight.detach().reshape(-1).to(dev, dtype).contiguous(),
                                 persistent=False)
        else:
            self.shared_gate_w = None

    def forward(self, hidden_states: torch.Tensor, residual: torch.Tensor | None = None,
                return_routing: bool = False):
        return ops.dmoe_forward(
            hidden_states, self.gate_up, self.down, self.top_k, router_w=self.router_w,
            norm_topk_prob=self.norm_topk_prob, gate_up_scale=self.gate_up_s,
            down_scale=self.down_s, shared_gate_up=self.shared_gate_up,
            shared_down=self.shared_down, shared_gate_w=self.shared_gate_w, residual=residual,
            return_routing=return_routing, workspace=self.workspace)


def fuse_moe_blocks(model: nn.Module, q8: bool = False, verbose: bool = True) -> int:
    """Replace every unquantized *SparseMoeBlock of `model` with a FusedMoE
    (blocks whose experts hold packed int4 weights are left to
    fuse_packed_moe_blocks).  The original experts are dropped per block, so the
    peak stays at all experts plus one stacked block."""
    sites = []
    for parent in model.modules():
        for name, child in list(parent.named_children()):
            if (type(child).__name__.endswith("SparseMoeBlock") and hasattr(child, "experts")
                    and not _is_packed(child)):
                sites.append((parent, name))
    for parent, name in sites:
        child = getattr(parent, name)
        setattr(parent, name, FusedMoE(child, q8=q8))
        child.experts = None
        del child
        gc.collect()
    if verbose:
        print(f"fused {len(sites)} MoE blocks (libi4moe{', int8' if q8 else ''})")
    return len(sites)

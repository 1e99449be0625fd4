"""FusedPackedMoE drop-in: the int4 SparseMoeBlock replacement on libi4moe.

Mirrors src/duplex/streaming/fused_packed_moe.py:83-319:
  - FusedPackedMoE(block, dtype, device) stacks a transformers block's packed
    experts (weight_packed / weight_scale / weight_shape per Linear) into
    gate|up [E, 2I, H/8] and down [E, H, I/8] with scales cast to `dtype`
    (:68-80, :112-122);
  - forward(hidden_states) routes and runs the experts (:191-263) in four
    launches at T = 1 (router, top-k, gate_up+SiLU, down+combine);
  - fuse_packed_moe_blocks(model, ...) swaps every matching block (:278-319).

Host-resident experts and CPU compute (:86-164, :202-220) exist in the
reference only because its 12 GB card cannot hold the Thinker; on a 288 GB
MI355X every layer stays resident, so those modes are rejected.
Extra constructors build the module from already-stacked CT tensors or from
AutoAWQ tensors.  The module keeps the experts as CT rows (AWQ repacked with
explicit zeros), which the latency-bound decode kernels stream row by row, and
a copy in the library's tile layout for the MFMA kernels of T > 1
(layouts="both", the default); layouts="tile" keeps only the tile copy and
decodes from it (one copy of the weights, slower decode).
"""
from __future__ import annotations

import gc

import torch
import torch.nn as nn

from . import ops
from .weights import QWeight, repack_awq_to_ct, repack_tile


def _stack_ct(linears, dtype, device):
    """Stack packed Linears into CT (packed [E, N, K/8], scale [E, N, NG], N, K)."""
    l0 = linears[0]
    out_f, in_f = (int(v) for v in l0.weight_shape.tolist())
    E = len(linears)
    packed = torch.empty(E, out_f, l0.weight_packed.shape[1], dtype=torch.int32, device=device)
    scale = torch.empty(E, out_f, l0.weight_scale.shape[1], dtype=dtype, device=device)
    for i, lin in enumerate(linears):
        packed[i] = lin.weight_packed.to(device)
        scale[i] = lin.weight_scale.to(device, dtype)
    return packed, scale, out_f, in_f


class _RouterGate(nn.Linear):
    """The block's router Linear H -> E (FusedPackedMoE.gate, as the reference keeps
    block.gate, fused_packed_moe.py:112).  Its weight is the router weight the library
    reads; forward routes inside the library, so this module's own forward (and hooks on
    it) run only when a caller invokes it.  Assigning its weight rebuilds the structs that
    hold raw addresses of it."""

    def __setattr__(self, name, value):
        super().__setattr__(name, value)
        ops.weights_changed()


class FusedPackedMoE(nn.Module):
    """SparseMoeBlock replacement for int4-packed experts."""

    def __setattr__(self, name, value):
        if name == "router_w":  # the router weight is gate.weight
            self.gate.weight = nn.Parameter(value.detach().contiguous(), requires_grad=False)
        else:
            super().__setattr__(name, value)
        ops.weights_changed()

    @property
    def router_w(self) -> torch.Tensor:
        """[E, H] router weight in the activation dtype: gate.weight (assignable)."""
        return self.gate.weight

    def __init__(self, block: nn.Module | None = None, dtype=torch.bfloat16, device="cuda",
                 host_resident: bool = False, cpu_compute: bool = False, group: int = 32,
                 layouts: str = "both"):
        super().__init__()
        if layouts not in ("both", "tile"):
            raise ValueError("layouts is 'both' (CT rows for decode + tiles) or 'tile'")
        self.layouts = layouts
        if host_resident or cpu_compute:
            raise NotImplementedError(
                "host-resident / CPU-computed experts are not provided: every layer is resident "
                "in HBM on MI355X")
        self.workspace = ops.Workspace()
        if block is None:  # filled by a classmethod constructor
            return
        experts = block.experts
        self.num_experts = len(experts)
        self.top_k = int(block.top_k)
        self.norm_topk_prob = bool(getattr(block, "norm_topk_prob", True))
        gw = block.gate.weight.detach().to(device=device, dtype=dtype).contiguous()
        gp, gs, inter, hidden = _stack_ct([e.gate_proj for e in experts], dtype, device)
        up, us, _, _ = _stack_ct([e.up_proj for e in experts], dtype, device)
        dp, ds, hid_out, inter_in = _stack_ct([e.down_proj for e in experts], dtype, device)
        gu = QWeight(torch.cat([gp, up], dim=1), torch.cat([gs, us], dim=1), None, "ct", group,
                     2 * inter, hidden)
        del gp, up, gs, us
        self._install(gu, QWeight(dp, ds, None, "ct", group, hid_out, inter_in), gw)

    def _install(self, gate_up: QWeight, down: QWeight, router_w: torch.Tensor,
                 norm_weight: torch.Tensor | None = None, norm_eps: float = 1e-6,
                 gate_up_tile: QWeight | None = None, down_tile: QWeight | None = None) -> None:
        """gate_up / down in any layout; tile copies are built here unless given."""
        if self.layouts == "tile" or gate_up.layout == "tile":
            gate_up, down = gate_up.to_tile(), down.to_tile()  # tiles cannot become CT rows
            gate_up_tile = down_tile = None
        else:
            if gate_up_tile is None:
                gate_up_tile, down_tile = gate_up.to_tile(), down.to_tile()
            gate_up, down = gate_up.to_ct(), down.to_ct()
        self.gate_up, self.down = gate_up, down
        self.gate_up_tile, self.down_tile = gate_up_tile, down_tile
        self.num_experts = gate_up.E
        self.inter = gate_up.N // 2
        self.hidden = gate_up.K
        self.hid_out, self.inter_in = down.N, down.K
        gate = _RouterGate(gate_up.K, gate_up.E, bias=False, device="meta")
        gate.weight = nn.Parameter(router_w, requires_grad=False)
        self.gate = gate
        self.register_buffer("norm_weight", norm_weight, persistent=False)
        self.norm_eps = float(norm_eps)
        bufs = [("gu_packed", gate_up.packed), ("gu_scale", gate_up.scale),
                ("gu_zeros", gate_up.zeros), ("down_packed", down.packed),
                ("down_scale", down.scale), ("down_zeros", down.zeros)]
        if gate_up_tile is not None:
            bufs += [("gu_tile_packed", gate_up_tile.packed), ("gu_tile_scale", gate_up_tile.scale),
                     ("gu_tile_zeros", gate_up_tile.zeros), ("down_tile_packed", down_tile.packed),
                     ("down_tile_scale", down_tile.scale), ("down_tile_zeros", down_tile.zeros)]
        for name, t in bufs:
            self.register_buffer(name, t, persistent=False)

    @classmethod
    def from_stacked(cls, gate_up: QWeight, down: QWeight, router_w: torch.Tensor, top_k: int,
                     norm_topk_prob: bool = True, norm_weight: torch.Tensor | None = None,
                     norm_eps: float = 1e-6, layouts: str = "both") -> "FusedPackedMoE":
        """From stacked weights in any layout (gate_up = gate rows then up rows).

        norm_weight fuses the decoder's pre-MoE RMSNorm (optional).
        """
        m = cls(layouts=layouts)
        m.top_k, m.norm_topk_prob = int(top_k), bool(norm_topk_prob)
        m._install(gate_up, down, router_w.contiguous(),
                   None if norm_weight is None else norm_weight.contiguous(), norm_eps)
        return m

    @classmethod
    def from_awq(cls, gate: QWeight, up: QWeight, down: QWeight, router_w: torch.Tensor,
                 top_k: int, norm_topk_prob: bool = True, norm_weight: torch.Tensor | None = None,
                 norm_eps: float = 1e-6, layouts: str = "both") -> "FusedPackedMoE":
        """Experts in AutoAWQ packing: gate|up and down repacked (CT + zeros, and tiles)."""
        m = cls(layouts=layouts)
        m.top_k, m.norm_topk_prob = int(top_k), bool(norm_topk_prob)
        gu_t, dn_t = repack_tile([gate, up]), repack_tile([down])
        if layouts == "tile":
            m._install(gu_t, dn_t, router_w.contiguous(),
                       None if norm_weight is None else norm_weight.contiguous(), norm_eps)
        else:
            m._install(repack_awq_to_ct([gate, up]), repack_awq_to_ct([down]),
                       router_w.contiguous(),
                       None if norm_weight is None else norm_weight.contiguous(), norm_eps,
                       gu_t, dn_t)
        return m

    def forward(self, hidden_states: torch.Tensor, residual: torch.Tensor | None = None):
        """MoE(hidden_states) (+ residual); with a fused norm, MoE(RMSNorm(hidden_states))."""
        return ops.moe_forward(hidden_states, self.gate_up, self.down, self.top_k,
                               router_w=self.router_w, norm_topk_prob=self.norm_topk_prob,
                               residual=residual, workspace=self.workspace,
                               norm_w=self.norm_weight, norm_eps=self.norm_eps,
                               gate_up_tile=self.gate_up_tile, down_tile=self.down_tile)

    def stack_entry(self) -> tuple:
        """(gate_up, down, router_w, norm_w, eps, gate_up_tile, down_tile) for ops.moe_stack."""
        return (self.gate_up, self.down, self.router_w, self.norm_weight, self.norm_eps,
                self.gate_up_tile, self.down_tile)

    def route(self, hidden_states: torch.Tensor):
        """(w, sel) exactly as forward() routes: [norm,] router Linear, softmax, top-k, renorm."""
        lg = ops.router_logits(hidden_states.reshape(-1, self.hidden), self.router_w,
                               self.norm_weight, self.norm_eps)
        return ops.route(lg, self.top_k, self.norm_topk_prob)


def fuse_packed_moe_blocks(model: nn.Module, dtype=torch.bfloat16, device="cuda",
                           n_pinned: int | None = None, cpu_compute: bool = False,
                           verbose: bool = True, layouts: str = "both") -> int:
    """Replace every packed *SparseMoeBlock with a FusedPackedMoE (all resident)."""
    if cpu_compute:
        raise NotImplementedError("CPU-computed experts are not provided")
    del n_pinned  # every block is resident in HBM
    sites = []
    for parent in model.modules():
        for name, child in list(parent.named_children()):
            if type(child).__name__.endswith("SparseMoeBlock") and hasattr(child, "experts"):
                gp = getattr(child.experts[0], "gate_proj", None)
                if gp is not None and hasattr(gp, "weight_packed"):
                    sites.append((parent, name))
    for parent, name in sites:
        child = getattr(parent, name)
        setattr(parent, name, FusedPackedMoE(child, dtype, device, layouts=layouts))
        child.experts = None
        del child
        gc.collect()
    if verbose:
        print(f"fused {len(sites)} packed MoE blocks, all HBM-resident")
    return len(sites)

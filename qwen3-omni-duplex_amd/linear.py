"""PackedLinear drop-in: the int4 Linear of the attention projections.

Mirrors TritonPackedLinear and patch_attention_to_triton
(src/duplex/streaming/triton_dequant_gemv.py:125-172): a packed Linear is the
E = 1 case of the expert gather.  The reference launches one kernel per row of
x (:154-155); here all rows go in one launch.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import ops
from .weights import QWeight


class PackedLinear(nn.Module):
    def __init__(self, mod: nn.Module | None = None, device="cuda", group: int = 32,
                 scale_dtype: torch.dtype = torch.float32):
        super().__init__()
        if mod is None:  # filled by from_qweight
            return
        out_f, in_f = (int(v) for v in mod.weight_shape.tolist())
        packed = mod.weight_packed.to(device).unsqueeze(0)
        scale = mod.weight_scale.to(device, scale_dtype).unsqueeze(0)
        b = getattr(mod, "bias", None)
        self._install(QWeight(packed, scale, None, "ct", group, out_f, in_f),
                      None if b is None else b.detach().to(device))

    def _install(self, w: QWeight, bias: torch.Tensor | None) -> None:
        if w.E != 1:
            raise ValueError("a Linear holds one expert")
        self.w = w
        self.out_features, self.in_features = w.N, w.K
        self.register_buffer("packed", w.packed, persistent=False)
        self.register_buffer("scale", w.scale, persistent=False)
        self.register_buffer("zeros", w.zeros, persistent=False)
        self.register_buffer("bias", bias, persistent=False)

    @classmethod
    def from_qweight(cls, w: QWeight, bias: torch.Tensor | None = None,
                     repack: bool = True) -> "PackedLinear":
        """From a CT or AWQ weight; AWQ is repacked to CT+zeros unless repack=False."""
        m = cls()
        m._install(w.to_ct() if repack else w, bias)
        return m

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return ops.linear(x, self.w, self.bias)


def patch_attention(model: nn.Module, device="cuda", verbose: bool = True) -> int:
    """Swap every packed Linear (weight_packed + weight_scale) for a PackedLinear."""
    n = 0
    for parent in model.modules():
        for name, child in list(parent.named_children()):
            if hasattr(child, "weight_packed") and hasattr(child, "weight_scale"):
                setattr(parent, name, PackedLinear(child, device))
                n += 1
    if verbose:
        print(f"moved {n} packed linears onto libi4moe")
    return n

"""PackedLinear drop-in: the int4 Linear of the attention projections.

Mirrors TritonPackedLinear and patch_attention_to_triton
(src/duplex/streaming/triton_dequant_gemv.py:125-172): a packed Linear is the
E = 1 case of the expert gather.  The reference launches one kernel per row of
x (:154-155); here all rows go in one launch, and q/k/v can share one launch
(PackedQKV, patch_attention(fuse_qkv=True)).  Batches of TILE_ROWS rows or more
(prefill) run on MFMA from a tile-layout copy of the weight, which streams each
weight tile once per 64 rows instead of once per row.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import ops
from .weights import QWeight, repack_awq_to_ct


# rows from which a PackedLinear runs on its tile copy; narrow layers (fewer than
# 1024 outputs) keep the per-row GEMV below TILE_ROWS_NARROW rows, where it was
# measured faster (k/v 2048 -> 512 at 32 rows: 5.6 us GEMV, 9.8 us tiles)
TILE_ROWS = 16
TILE_ROWS_NARROW = 64


def _tile_copy(w: QWeight) -> QWeight | None:
    """Tile-layout copy for the MFMA path, or None where the shape has none."""
    if w.N % 128 != 0 or w.K % 128 != 0:
        return None
    return w.to_tile()


class PackedLinear(nn.Module):
    """int4 Linear; tile=True also keeps a tile-layout copy of the weight for
    batches of TILE_ROWS rows or more."""

    def __init__(self, mod: nn.Module | None = None, device="cuda", group: int = 32,
                 scale_dtype: torch.dtype = torch.float32, tile: bool = True):
        super().__init__()
        if mod is None:  # filled by from_qweight
            return
        out_f, in_f = (int(v) for v in mod.weight_shape.tolist())
        packed = mod.weight_packed.to(device).unsqueeze(0)
        scale = mod.weight_scale.to(device, scale_dtype).unsqueeze(0)
        b = getattr(mod, "bias", None)
        self._install(QWeight(packed, scale, None, "ct", group, out_f, in_f),
                      None if b is None else b.detach().to(device), tile)

    def _install(self, w: QWeight, bias: torch.Tensor | None, tile: bool = True) -> None:
        if w.E != 1:
            raise ValueError("a Linear holds one expert")
        self.w = w
        self.w_tile = _tile_copy(w) if tile and w.layout != "awq" else None
        self.out_features, self.in_features = w.N, w.K
        self.register_buffer("packed", w.packed, persistent=False)
        self.register_buffer("scale", w.scale, persistent=False)
        self.register_buffer("zeros", w.zeros, persistent=False)
        self.register_buffer("bias", bias, persistent=False)
        self.workspace = ops.Workspace()  # this module's split-K workspace, kept across calls

    @classmethod
    def from_qweight(cls, w: QWeight, bias: torch.Tensor | None = None,
                     repack: bool = True, tile: bool = True) -> "PackedLinear":
        """From a CT or AWQ weight; AWQ is repacked to CT+zeros unless repack=False
        (the in-place AWQ GEMV, which keeps no tile copy)."""
        m = cls()
        m._install(w.to_ct() if repack else w, bias, tile)
        return m

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        rows = x.numel() // max(x.shape[-1], 1)
        if self.w_tile is not None and rows >= (TILE_ROWS if self.w.N >= 1024
                                                else TILE_ROWS_NARROW):
            return ops.linear(x, self.w_tile, self.bias, workspace=self.workspace)
        return ops.linear(x, self.w, self.bias, workspace=self.workspace)


_SYM_ZEROS = -2004318072  # 0x88888888 as int32: every zero point 8


def concat_rows(parts: list[QWeight]) -> QWeight:
    """One CT weight (E = 1) holding the rows of parts in order, on the device.

    AWQ parts are repacked to CT with explicit zeros; when any part has zero
    points a symmetric part gets explicit 8s, so the result dequantises to the
    parts' rows exactly.
    """
    if all(p.layout == "awq" for p in parts):
        return repack_awq_to_ct(parts)
    cts = [p.to_ct() for p in parts]
    c0 = cts[0]
    for c in cts:
        if c.E != 1 or c.K != c0.K or c.group != c0.group or c.scale.dtype != c0.scale.dtype:
            raise ValueError("row-concatenated parts need E = 1 and equal K, group, scale dtype")
    packed = torch.cat([c.packed for c in cts], dim=1)
    scale = torch.cat([c.scale for c in cts], dim=1)
    zeros = None
    if any(c.zeros is not None for c in cts):
        ng = -(-c0.K // c0.group)
        nzw = -(-ng // 8)
        zeros = torch.cat([c.zeros if c.zeros is not None else
                           torch.full((1, c.N, nzw), _SYM_ZEROS, dtype=torch.int32,
                                      device=c.device) for c in cts], dim=1)
    return QWeight(packed, scale, zeros, "ct", c0.group, sum(c.N for c in cts), c0.K)


def concat_cols_awq(parts: list[QWeight]) -> QWeight:
    """One AWQ weight (E = 1) holding the output columns of parts in order, still in
    AutoAWQ packing ([K][N / 8] words, [groups][N] scales, [groups][N / 8] zero words):
    the in-place GEMV then serves q, k and v in one launch.  A part without zero
    points gets explicit 8s when another has them."""
    p0 = parts[0]
    for p in parts:
        if (p.layout != "awq" or p.E != 1 or p.K != p0.K or p.group != p0.group
                or p.scale.dtype != p0.scale.dtype or p.N % 8):
            raise ValueError("column-concatenated AWQ parts need E = 1, N % 8 == 0 and equal "
                             "K, group, scale dtype")
    packed = torch.cat([p.packed for p in parts], dim=2)
    scale = torch.cat([p.scale for p in parts], dim=2)
    zeros = None
    if any(p.zeros is not None for p in parts):
        ng = -(-p0.K // p0.group)
        zeros = torch.cat([p.zeros if p.zeros is not None else
                           torch.full((1, ng, p.N // 8), _SYM_ZEROS, dtype=torch.int32,
                                      device=p.device) for p in parts], dim=2)
    return QWeight(packed, scale, zeros, "awq", p0.group, sum(p.N for p in parts), p0.K)


class PackedQKV(nn.Module):
    """q, k and v projections of one attention block as one int4 GEMV launch.

    The reference runs q_proj, k_proj and v_proj as three TritonPackedLinear
    calls on the same input (triton_dequant_gemv.py:151-159, once per row of
    the input each); their rows are concatenated here into one weight, so a
    decode step streams all three in a single launch.  forward(x) returns the
    three outputs as views of that launch's result.
    """

    def __init__(self, w: QWeight, sizes: tuple[int, int, int], bias: torch.Tensor | None,
                 tile: bool = True):
        super().__init__()
        self.lin = PackedLinear()
        self.lin._install(w, bias, tile)
        self.sizes = tuple(int(v) for v in sizes)

    @classmethod
    def from_qweights(cls, q: QWeight, k: QWeight, v: QWeight, biases=None,
                      repack: bool = True) -> "PackedQKV":
        """repack=False keeps AWQ parts in AWQ packing (concat_cols_awq, the in-place
        GEMV, no tile copy); otherwise the rows are concatenated in CT (concat_rows)."""
        in_place = not repack and all(p.layout == "awq" for p in (q, k, v))
        w = concat_cols_awq([q, k, v]) if in_place else concat_rows([q, k, v])
        bias = None
        if biases is not None and any(b is not None for b in biases):
            dt = next(b.dtype for b in biases if b is not None)
            bias = torch.cat([b.to(dt) if b is not None else
                              torch.zeros(p.N, dtype=dt, device=p.device)
                              for b, p in zip(biases, (q, k, v))])
        return cls(w, (q.N, k.N, v.N), bias, tile=not in_place)

    def forward(self, x: torch.Tensor):
        y = self.lin(x)
        nq, nk, _ = self.sizes
        return y[..., :nq], y[..., nq:nq + nk], y[..., nq + nk:]


class _SharedQKV:
    """One fused launch serving the q_proj / k_proj / v_proj calls of a block.

    The first of the three calls on an input runs the fused GEMV; the other two
    take their slice of it.  The result is kept for exactly one use of each
    slice on the same input (same storage, version, shape and stream) and
    dropped after the third, so a later input that happens to reuse the memory
    never sees it; any other pattern simply runs the launch again.
    """

    def __init__(self, fused: PackedQKV):
        self.fused = fused
        self.key = None
        self.out = None
        self.served = [False, False, False]

    def take(self, x: torch.Tensor, i: int) -> torch.Tensor:
        key = (x.data_ptr(), x._version, tuple(x.shape), x.dtype,
               torch.cuda.current_stream(x.device).cuda_stream if x.is_cuda else 0)
        if key != self.key or self.served[i]:
            self.out = self.fused(x)
            self.key = key
            self.served = [False, False, False]
        y = self.out[i]
        self.served[i] = True
        if all(self.served):
            self.key, self.out = None, None
        return y


class QKVSlice(nn.Module):
    """Stands in for q_proj, k_proj or v_proj when the three are fused."""

    def __init__(self, shared: _SharedQKV, index: int, out_features: int, in_features: int):
        super().__init__()
        self.shared = shared
        self.index = index
        self.out_features, self.in_features = out_features, in_features

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.shared.take(x, self.index)


def patch_attention(model: nn.Module, device="cuda", verbose: bool = True,
                    fuse_qkv: bool = False) -> int:
    """Swap every packed Linear (weight_packed + weight_scale) for a PackedLinear.

    fuse_qkv: where a module's q_proj, k_proj and v_proj are all packed with the
    same K and group, they become one PackedQKV launch (QKVSlice stand-ins).
    """
    n = 0
    for parent in list(model.modules()):
        packed = {name: child for name, child in parent.named_children()
                  if hasattr(child, "weight_packed") and hasattr(child, "weight_scale")}
        if fuse_qkv and all(k in packed for k in ("q_proj", "k_proj", "v_proj")):
            lins = {k: PackedLinear(packed.pop(k), device) for k in ("q_proj", "k_proj", "v_proj")}
            ws = [lins[k].w for k in ("q_proj", "k_proj", "v_proj")]
            if len({(w.K, w.group, w.scale.dtype) for w in ws}) == 1:
                fused = PackedQKV.from_qweights(*ws, biases=[lins[k].bias for k in
                                                             ("q_proj", "k_proj", "v_proj")])
                shared = _SharedQKV(fused)
                for i, k in enumerate(("q_proj", "k_proj", "v_proj")):
                    setattr(parent, k, QKVSlice(shared, i, ws[i].N, ws[i].K))
            else:
                for k, lin in lins.items():
                    setattr(parent, k, lin)
            n += 3
        for name, child in packed.items():
            setattr(parent, name, PackedLinear(child, device))
            n += 1
    if verbose:
        print(f"moved {n} packed linears onto libi4moe")
    return n

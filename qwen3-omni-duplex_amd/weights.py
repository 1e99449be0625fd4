"""Stacked int4 weights on the device and their C descriptors.

A QWeight is E experts of one logical [N out][K in] matrix in one of the two
packed formats:

  "ct"  compressed-tensors pack-quantized, the reference's checkpoint format
        (src/duplex/quant/dequant.py:23-27; src/duplex/streaming/
        fused_packed_moe.py:7-11,54-65): packed [E, N, K/8] int32, column
        k = 8m + i in nibble i of word m; scale [E, N, ceil(K/G)]; optional
        zeros [E, N, ceil(NG/8)] int32 (group g in nibble g % 8 of word g // 8),
        absent = symmetric with zero point 8.
  "awq" AutoAWQ GEMM packing: qweight [E, K, N/8] int32 with nibble slot i of
        word w holding column 8w + (0, 2, 4, 6, 1, 3, 5, 7)[i]; qzeros
        [E, NG, N/8] packed the same way; scales [E, NG, N].

  "tile" the library's load-time layout for the MoE kernels (no reference
        counterpart): packed [E, N/16, K/128, 16, 16] int32, element
        [e, b, s, r, 4j + t] = CT word 4(4s + t) + j of row 16b + r, so one
        wavefront load of lanes (r, j) reads 1 KB of contiguous memory;
        scale [E, N/16, NG, 16] and zeros [E, N/16, ceil(NG/8), 16] hold the CT
        values of row 16b + r.  Needs N % 16 == 0 and K % 128 == 0.

The dequant-GEMV entry points take "ct" or "awq"; the fused MoE kernels take
"tile", built once on the device with to_tile() / repack_tile() (AWQ can also
be converted to "ct" with explicit zeros by to_ct()).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib


@dataclass
class QWeight:
    packed: torch.Tensor
    scale: torch.Tensor
    zeros: torch.Tensor | None
    layout: str
    group: int
    N: int
    K: int

    def __post_init__(self) -> None:
        if self.layout not in _lib.LAYOUTS:
            raise ValueError(f"unknown layout {self.layout!r}")
        for name in ("packed", "scale", "zeros"):
            t = getattr(self, name)
            if t is None:
                continue
            if t.dim() == 2:
                t = t.unsqueeze(0)
            # Views are used in place, never copied: the descriptor carries the stride
            # between experts (the reference's kernel takes strides too,
            # triton_dequant_gemv.py:105-110), while each expert's rows must be dense.
            if not _dense_per_expert(t):
                raise ValueError(
                    f"{name} {tuple(t.shape)} with strides {t.stride()}: each expert's "
                    "elements must be densely laid out (only the stride between experts may "
                    "differ); pass .contiguous() explicitly to copy")
            setattr(self, name, t)
        if self.packed.dtype != torch.int32:
            raise ValueError("packed weights must be int32")
        if self.zeros is not None and self.zeros.dtype != torch.int32:
            raise ValueError("zeros must be int32")
        E = self.packed.shape[0]
        NG = -(-self.K // self.group)
        if self.layout == "ct":
            want_p = (E, self.N, self.K // 8)
            want_s = (E, self.N, NG)
            want_z = (E, self.N, -(-NG // 8))
        elif self.layout == "tile":
            if self.N % 16 or self.K % 128:
                raise ValueError("the tile layout needs N % 16 == 0 and K % 128 == 0")
            want_p = (E, self.N // 16, self.K // 128, 16, 16)
            want_s = (E, self.N // 16, NG, 16)
            want_z = (E, self.N // 16, -(-NG // 8), 16)
        else:
            want_p = (E, self.K, self.N // 8)
            want_s = (E, NG, self.N)
            want_z = (E, NG, self.N // 8)
        if tuple(self.packed.shape) != want_p:
            raise ValueError(f"{self.layout} packed shape {tuple(self.packed.shape)} != {want_p}")
        if tuple(self.scale.shape) != want_s:
            raise ValueError(f"{self.layout} scale shape {tuple(self.scale.shape)} != {want_s}")
        if self.zeros is not None and tuple(self.zeros.shape) != want_z:
            raise ValueError(f"{self.layout} zeros shape {tuple(self.zeros.shape)} != {want_z}")

    @property
    def E(self) -> int:
        return self.packed.shape[0]

    @property
    def device(self) -> torch.device:
        return self.packed.device

    def c(self) -> _lib.QWeightC:
        """The i4_qweight descriptor, with the tensors' strides between experts."""
        return _lib.QWeightC(
            packed=self.packed.data_ptr(), scale=self.scale.data_ptr(),
            zeros=None if self.zeros is None else self.zeros.data_ptr(),
            packed_estride=_estride(self.packed), scale_estride=_estride(self.scale),
            zeros_estride=0 if self.zeros is None else _estride(self.zeros),
            layout=_lib.LAYOUTS[self.layout], group=self.group,
            scale_dtype=_lib.dtype_code(self.scale.dtype), E=self.E, N=self.N, K=self.K)

    # -- conversions -----------------------------------------------------
    def to_ct(self) -> "QWeight":
        """CT copy with explicit zeros (identity for a CT weight)."""
        if self.layout == "ct":
            return self
        return repack_awq_to_ct([self])

    def to_tile(self) -> "QWeight":
        """Tile-layout copy for the MoE kernels (identity for a tile weight)."""
        if self.layout == "tile":
            return self
        return repack_tile([self])

    @staticmethod
    def ct(packed, scale, group=32, zeros=None, N=None, K=None) -> "QWeight":
        p = packed if packed.dim() == 3 else packed.unsqueeze(0)
        return QWeight(packed, scale, zeros, "ct", group,
                       N if N is not None else p.shape[1], K if K is not None else p.shape[2] * 8)

    @staticmethod
    def awq(qweight, scales, qzeros=None, group=128) -> "QWeight":
        q = qweight if qweight.dim() == 3 else qweight.unsqueeze(0)
        return QWeight(qweight, scales, qzeros, "awq", group, q.shape[2] * 8, q.shape[1])


def _dense_per_expert(t: torch.Tensor) -> bool:
    """True when every expert t[e] is row-major dense and experts do not overlap."""
    want = 1
    for size, stride in zip(reversed(t.shape[1:]), reversed(t.stride()[1:])):
        if size != 1 and stride != want:
            return False
        want *= size
    return t.shape[0] == 1 or t.stride(0) >= want


def _estride(t: torch.Tensor) -> int:
    """Element stride between experts (0: densely stacked, the descriptor's default)."""
    if t.shape[0] == 1:
        return 0
    return int(t.stride(0))


def repack_awq_to_ct(parts: list[QWeight]) -> QWeight:
    """Concatenate AWQ weights along N into one CT(+zeros) weight, on the device.

    parts share E, K, group and scale dtype; the result has N = sum of parts' N
    (the gate|up concatenation of fused_packed_moe.py:122 when parts = [gate, up]).
    """
    p0 = parts[0]
    dev = _lib.require_device(*[p.packed for p in parts])
    E, K, G = p0.E, p0.K, p0.group
    for p in parts:
        if p.layout != "awq" or p.E != E or p.K != K or p.group != G or p.scale.dtype != p0.scale.dtype:
            raise ValueError("repack parts must be AWQ weights with equal E, K, group, scale dtype")
    N = sum(p.N for p in parts)
    NG = -(-K // G)
    packed = torch.empty(E, N, K // 8, dtype=torch.int32, device=dev)
    scale = torch.empty(E, N, NG, dtype=p0.scale.dtype, device=dev)
    zeros = torch.empty(E, N, -(-NG // 8), dtype=torch.int32, device=dev)
    lb = _lib.lib()
    off = 0
    for p in parts:
        if p.zeros is None:
            raise ValueError("AWQ weights carry qzeros")
        cw = p.c()
        _lib.check(lb.i4_repack_awq_to_ct(ctypes.byref(cw), packed.data_ptr(), scale.data_ptr(),
                                          zeros.data_ptr(), N, off, _lib.stream(dev)))
        off += p.N
    return QWeight(packed, scale, zeros, "ct", G, N, K)


def repack_tile(parts: list[QWeight]) -> QWeight:
    """Concatenate CT / AWQ weights along N into one tile-layout weight, on the device.

    parts share E, K, group and scale dtype, and each part's N is a multiple of
    16; the result has N = sum of parts' N (the gate|up concatenation of
    fused_packed_moe.py:122 when parts = [gate, up]).  Zero points are kept
    explicit when any part has them (a symmetric part then gets 8s).
    """
    p0 = parts[0]
    dev = _lib.require_device(*[p.packed for p in parts])
    E, K, G = p0.E, p0.K, p0.group
    for p in parts:
        if (p.layout == "tile" or p.E != E or p.K != K or p.group != G
                or p.scale.dtype != p0.scale.dtype or p.N % 16):
            raise ValueError("repack parts must be CT/AWQ weights with equal E, K, group, scale "
                             "dtype and N % 16 == 0")
    N = sum(p.N for p in parts)
    NG = -(-K // G)
    packed = torch.empty(E, N // 16, K // 128, 16, 16, dtype=torch.int32, device=dev)
    scale = torch.empty(E, N // 16, NG, 16, dtype=p0.scale.dtype, device=dev)
    with_z = any(p.zeros is not None for p in parts)
    zeros = (torch.empty(E, N // 16, -(-NG // 8), 16, dtype=torch.int32, device=dev)
             if with_z else None)
    lb = _lib.lib()
    off = 0
    for p in parts:
        cw = p.c()
        _lib.check(lb.i4_repack_tile(ctypes.byref(cw), packed.data_ptr(), scale.data_ptr(),
                                     None if zeros is None else zeros.data_ptr(), N, off,
                                     _lib.stream(dev)))
        off += p.N
    return QWeight(packed, scale, zeros, "tile", G, N, K)

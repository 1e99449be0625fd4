"""Timed CPU baselines -- TEST/BENCH INFRASTRUCTURE ONLY.

Only bench.py's cpu_baseline leg (and tests) may use this; the product never
does.  Two reference paths are restated in torch on the host:
  - moe_layer: the reference's CPU expert path,
    src/duplex/streaming/fused_packed_moe.py:202-220: route in fp32 (:195-199),
    then per token and selected expert dequantise the packed gate/up/down
    weights to fp32 (:213,217 via _dequant :183-189), matmul -> silu(g) * u ->
    matmul, and sum w_j * y_j (:214-219);
  - gemv: reference_gemv, src/duplex/streaming/triton_dequant_gemv.py:116-122:
    dequantise the selected weight to fp32, then one matmul with x.
The weights are in the workload's AutoAWQ g128 format (qweight [K, N/8] with
nibble order 0,2,4,6,1,3,5,7, qzeros, fp16 scales) instead of the
checkpoint's symmetric group-32 format; only the unpack differs.
"""
from __future__ import annotations

import time

import torch
import torch.nn.functional as F

_SHIFTS = torch.arange(8, dtype=torch.int32) * 4
# column c of a word lives in nibble slot AWQ_SLOT[c]
_AWQ_SLOT = torch.tensor([0, 4, 1, 5, 2, 6, 3, 7])


def awq_unpack(packed: torch.Tensor) -> torch.Tensor:
    """[..., N/8] int32 -> [..., N] int32 nibbles in column order."""
    u = (packed.unsqueeze(-1) >> _SHIFTS) & 0xF       # [..., N/8, 8] slot order
    u = u[..., _AWQ_SLOT]                              # column order
    return u.flatten(-2)


def awq_dequant(qweight, qzeros, scales, group) -> torch.Tensor:
    """AWQ -> dense fp32 [K, N] (value = (q - z) * s)."""
    q = awq_unpack(qweight).float()                    # [K, N]
    z = awq_unpack(qzeros).float()                     # [NG, N]
    s = scales.float()                                 # [NG, N]
    K = q.shape[0]
    g = torch.arange(K) // group
    return (q - z[g]) * s[g]


def moe_layer(x, router_w, gate, up, down, top_k=8, group=128):
    """x [T, H] fp32; gate/up/down = (qweight [E, K, N/8], qzeros, scales). Returns [T, H]."""
    w = F.softmax(x @ router_w.T, dim=1, dtype=torch.float32)
    w, sel = torch.topk(w, top_k, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    outs = []
    for t in range(x.shape[0]):
        y = torch.zeros(x.shape[1])
        for j in range(top_k):
            e = int(sel[t, j])
            g = x[t] @ awq_dequant(gate[0][e], gate[1][e], gate[2][e], group)
            u = x[t] @ awq_dequant(up[0][e], up[1][e], up[2][e], group)
            act = F.silu(g) * u
            y += w[t, j] * (act @ awq_dequant(down[0][e], down[1][e], down[2][e], group))
        outs.append(y)
    return torch.stack(outs)


def gemv(x, qweight, qzeros, scales, group=128):
    """reference_gemv on one AWQ weight: y [N] = dequant(W)^T-form product with x [K], fp32."""
    return x.float() @ awq_dequant(qweight, qzeros, scales, group)


def time_calls(fn, seconds=2.0, min_reps=3):
    """Median seconds of fn(i) over a bounded sample (at least min_reps calls)."""
    times = []
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end or len(times) < min_reps:
        t0 = time.perf_counter()
        fn(i)
        times.append(time.perf_counter() - t0)
        i += 1
    times.sort()
    return times[len(times) // 2], len(times)


def time_layer(x, router_w, gate, up, down, seconds=10.0, top_k=8, group=128, min_reps=3):
    """Median seconds per M=1 layer over a bounded sample (distinct inputs per rep)."""
    times = []
    t_end = time.perf_counter() + seconds
    i = 0
    while time.perf_counter() < t_end or len(times) < min_reps:
        xi = x[i % x.shape[0]: i % x.shape[0] + 1]
        t0 = time.perf_counter()
        moe_layer(xi, router_w, gate, up, down, top_k, group)
        times.append(time.perf_counter() - t0)
        i += 1
    times.sort()
    return times[len(times) // 2], len(times)

#!/usr/bin/env python3
"""Headline benchmark: microseconds per int4 Thinker MoE layer at M = 1.

Workload (one step = one decode token through the 24-layer MoE stack,
Thinker[0:24] with residual adds, src/duplex/streaming/clock.py:168-171; each
layer is h <- h + MoE(RMSNorm(h)), the decoder's pre-MoE norm being fused into
the router kernel -- without it these synthetic weights overflow fp16 within
three layers):
  128 experts, top-8 (softmax, renormalised), hidden 2048, expert FFN 768,
  gate/up/down in AutoAWQ int4 g128 with zero points and fp16 scales
  (scales ~ U[0.002, 0.02], int4 values and zeros ~ U{0..15}), router weight
  fp16 ~ N(0, 0.02), activations fp16 ~ N(0, 1).  Synthetic, seeded,
  generated on the device; the AWQ tensors are repacked once to the CT+zeros
  layout the kernels stream.  Every step feeds a fresh input, so routing (and
  the 8-expert working set of each layer, 19.6 MB) changes from step to step;
  the stack touches ~470 MB of weights per token out of 7.5 GB resident, well
  beyond the 256 MB Infinity Cache.

Printed: one JSON line with value = us per layer (stack time / 24 for the faster of
the two ways to run a token -- one C call enqueueing the stack's 49 launches, or a
hipGraph replay, which also copies the token's input into the captured buffer --
both reported, median and p99 of that mode's per-token times beside them), plus the
roofline of the dominant kernel (the decode experts launch: top-8 routing, gate/up,
SiLU and down of the 8 experts) timed with HIP events on the stream it runs on, and a
CPU baseline (the reference's CPU expert path restated in torch,
oracle/cpu_baseline.py) timed on this host.  Extra fields time the same layer at
M = 32 (router from weights) and M = 512 (Zipf-skewed logits) with their realised
expert histograms, HBM and MFMA fractions; count the rows whose GPU top-8 differs
from the host's exact ranking (routing_agreement); time the dequant-GEMV workloads
(a 2048 -> 768 GEMV, also through the PackedLinear module, and the four attention
projections, individually and back to back), the whole Thinker[0:24] decode step
around the MoE stack (attention with a KV cache at --context positions + MoE per
layer, thinker_decode_step), and the Talker's 16-bit / int8 MoE blocks (talker_moe).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

E, H, I, TOPK, G = 128, 2048, 768, 8, 128
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16
# algorithmic bytes (AWQ g128 + zeros, fp16 scales)
B_GATE_UP_EXPERT = 2 * (H * I // 2 + (H // G) * I * 2 + (H // G) * (I // 8) * 4)  # 1,634,304
B_DOWN_EXPERT = I * H // 2 + (I // G) * H * 2 + (I // G) * (H // 8) * 4            # 817,152
B_ROUTER = E * H * 2
B_LAYER = TOPK * (B_GATE_UP_EXPERT + B_DOWN_EXPERT) + B_ROUTER + 2 * H * 2        # 20,144,128
# the decode experts launch of the stack (k_ct_moe_m1x): 8 experts' gate/up and down
# weights, the normalised input in, the activations out and back in, the 8 slot output
# rows out (their routing-weighted sum and the residual are the next launch's)
B_EXPERTS_LAUNCH = (TOPK * (B_GATE_UP_EXPERT + B_DOWN_EXPERT) + H * 2 + 2 * TOPK * I * 2
                    + TOPK * H * 2)                                                  # 19,673,088
# HBM bytes per decode experts launch measured with rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE (calibrated against a device copy; summary under profiles/)
EXPERTS_TRAFFIC_BYTES = 20_061_560


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_layers(pkg, torch, n_layers, dev, seed=1234, keep_first_awq=False):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)

    def words(*shape):
        return torch.randint(-2**31, 2**31, shape, dtype=torch.int32, device=dev, generator=gen)

    def awq(K, N):
        qw, qz = words(E, K, N // 8), words(E, K // G, N // 8)
        sc = (torch.rand(E, K // G, N, device=dev, generator=gen) * 0.018 + 0.002).half()
        return qw, qz, sc

    mods, first = [], None
    for li in range(n_layers):
        g, u, d = awq(H, I), awq(H, I), awq(I, H)
        wr = (torch.randn(E, H, device=dev, generator=gen) * 0.02).half()
        nw = (torch.rand(H, device=dev, generator=gen) * 0.4 + 0.8).half()
        q = lambda p: pkg.QWeight.awq(p[0], p[2], p[1], group=G)
        mods.append(pkg.FusedPackedMoE.from_awq(q(g), q(u), q(d), wr, top_k=TOPK,
                                                norm_weight=nw, norm_eps=1e-6))
        if keep_first_awq and li == 0:
            first = (g, u, d, wr)
        del g, u, d
    torch.cuda.synchronize()
    return mods, first


def time_stack(torch, step, steps, warmup, per_step=None):
    """Mean ms per step between one pair of HIP events around `steps` steps (and the wall
    clock); with per_step a list, a second pass appends each step's own event time (ms)."""
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        step(warmup + i)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if per_step is not None:
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(steps)]
        for i, (a, b) in enumerate(evs):
            a.record()
            step(warmup + steps + i)
            b.record()
        torch.cuda.synchronize()
        per_step.extend(a.elapsed_time(b) for a, b in evs)
    return e0.elapsed_time(e1) / steps, wall / steps * 1e3


def gpu_backlog(torch, dev, ms=20.0):
    """Queue ~ms of GPU work so the launches behind it are enqueued before they run."""
    a = torch.randn(4096, 4096, device=dev, dtype=torch.float16)
    b = torch.randn(4096, 4096, device=dev, dtype=torch.float16)
    torch.cuda.synchronize()
    t = time.perf_counter()
    c = a @ b
    torch.cuda.synchronize()
    one = max(time.perf_counter() - t, 1e-5)
    for _ in range(max(1, int(ms / 1e3 / one))):
        c = a @ b
    return c


def time_experts(pkg, torch, dev, mods, hs, rounds):
    """HIP-event timing of the dominant kernel, k_ct_moe_m1x: the experts launch of the
    stack's decode layer (top-8 routing, gate/up, SiLU and down of the 8 experts, each slot on
    its own XCD, slot output rows out), on the stream it is launched on.  Each layer has its
    own workspace, so the 24 router launches (i4_moe_route_sum on each layer's own input) can
    run first and the 24 experts launches (i4_moe_experts_x) then run back to back between
    one pair of events; `rounds` such passes behind a queued backlog.  Also returned: router +
    experts interleaved layer by layer, and the router launches alone (each one pair of
    events around all passes).  Returns (experts us, layer us, router us) per launch."""
    from qwen3_omni_duplex_amd import ops

    stream = torch.cuda.current_stream(dev)
    n = len(mods)
    pieces = [ops.StackLayerX(m.stack_entry(), TOPK, torch.float16, workspace=pkg.Workspace())
              for m in mods]
    ypart = torch.empty(TOPK, H, dtype=torch.float16, device=dev)
    ev = lambda: torch.cuda.Event(enable_timing=True)

    def warm():
        for li in range(n):
            pieces[li].route(hs[li], reset_status=True)
            pieces[li].experts(hs[li], ypart)
        torch.cuda.synchronize()
        gpu_backlog(torch, dev)

    def timed(body):
        warm()
        e0, e1 = ev(), ev()
        e0.record(stream)
        for _ in range(rounds):
            body()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (n * rounds)

    def interleaved():
        for li in range(n):
            pieces[li].route(hs[li])
            pieces[li].experts(hs[li], ypart)

    def routers():
        for li in range(n):
            pieces[li].route(hs[li])

    us_layer, us_router = timed(interleaved), timed(routers)
    warm()
    tot = 0.0
    for _ in range(rounds):
        routers()
        e0, e1 = ev(), ev()
        e0.record(stream)
        for li in range(n):
            pieces[li].experts(hs[li], ypart)
        e1.record(stream)
        torch.cuda.synchronize()
        tot += e0.elapsed_time(e1)
    us_experts = tot * 1e3 / (n * rounds)
    for p in pieces:
        if ops.moe_status(p.ws_holder, 1, H, I, E, TOPK) != 0:
            raise RuntimeError("a decode wait of the experts launch gave up")
    return us_experts, us_layer, us_router


def awq_gemv_bytes(K, N):
    """algorithmic bytes of one AWQ g128 GEMV: weights + fp16 scales + zeros + x + fp16 y"""
    return K * N // 2 + (K // G) * N * 2 + (K // G) * (N // 8) * 4 + 2 * K + 2 * N


def graph_times(torch, launches, replays, warm=3):
    """Capture launches() (which enqueues on the current stream) in one hipGraph and replay
    it (`warm` untimed replays first); returns the per-replay times in microseconds, each
    from a pair of HIP events on the replay stream."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        launches()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launches()
    for _ in range(warm):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(replays)]
    for a, b in evs:
        a.record(stream)
        graph.replay()
        b.record(stream)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) * 1e3 for a, b in evs]


def time_decode_step(pkg, torch, dev, mods, ctx, replays):
    """The Thinker[0:24] decode step around the MoE stack (clock.py:164-172): per layer the
    attention half (input RMSNorm, q|k|v int4 GEMV, q/k norm + rotary + KV-cache append,
    GQA attention over ctx cached positions, o_proj + residual) and the MoE block.  Attention
    weights are CT g32 symmetric int4 with fp16 scales (the reference checkpoint's packing),
    32 query / 4 kv heads of 128, generated on the device; cache rows [0, ctx) random.
    Each timed region is one hipGraph of all layers, the position read from device memory."""
    nh, nkv, hd, gs = 32, 4, 128, 32
    gen = torch.Generator(device=dev)
    gen.manual_seed(4321)

    def ct(N, K):
        p = torch.randint(-2**31, 2**31, (1, N, K // 8), dtype=torch.int32, device=dev,
                          generator=gen)
        sc = (torch.rand(1, N, K // gs, device=dev, generator=gen) * 0.018 + 0.002).half()
        return pkg.QWeight(p, sc, None, "ct", gs, N, K)

    def vec(n, lo=0.8, hi=1.2):
        return (torch.rand(n, device=dev, generator=gen) * (hi - lo) + lo).half()

    layers = []
    for m in mods:
        qkv = pkg.PackedQKV.from_qweights(ct(nh * hd, H), ct(nkv * hd, H), ct(nkv * hd, H))
        o = pkg.PackedLinear.from_qweight(ct(H, nh * hd))
        attn = pkg.ThinkerAttention(qkv, o, vec(hd), vec(hd), vec(H), nh, nkv, hd,
                                    max_len=ctx + 64)
        attn.k_cache[:, :ctx] = torch.randn(nkv, ctx, hd, device=dev, generator=gen).half()
        attn.v_cache[:, :ctx] = torch.randn(nkv, ctx, hd, device=dev, generator=gen).half()
        layers.append(pkg.ThinkerDecoderLayer(attn, m))
    dec = pkg.ThinkerDecoder(layers)
    x = torch.randn(1, H, device=dev, generator=gen).half()
    pos = torch.full((1,), ctx, dtype=torch.int32, device=dev)  # read by the kernels
    out = {}
    for name, fn in (("step", lambda: dec.step(x, pos)),
                     ("attention", lambda: [l.attn(x, pos) for l in layers])):
        ts = graph_times(torch, fn, replays)
        us = sum(ts) / len(ts)
        out[name] = {"us_per_token": round(us, 2), "us_per_layer": round(us / len(layers), 3),
                     "us_median": round(pct(ts, 50), 2), "us_p99": round(pct(ts, 99), 2)}
    # eager: one Python call per op (the caller's loop without a graph)
    for _ in range(3):
        dec.step(x, ctx)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n_eager = 20
    for _ in range(n_eager):
        h = dec.step(x, ctx)
    torch.cuda.synchronize()
    out["step_eager"] = {"us_per_token": round((time.perf_counter() - t0) / n_eager * 1e6, 1),
                         "timing": f"wall clock over {n_eager} eager steps"}
    if not torch.isfinite(h.float()).all():
        raise RuntimeError("the decode step produced non-finite values")
    # K and V bytes read by the attention of one layer at this context (fp16 cache)
    kv_bytes = 2 * nkv * (ctx + 1) * hd * 2
    w_bytes = (nh * hd + 2 * nkv * hd) * H // 2 + H * nh * hd // 2
    return {"context": ctx, "layers": len(layers), **out,
            "attention_weight_bytes_per_layer": w_bytes + (nh * hd + 2 * nkv * hd) * (H // gs) * 2
            + H * (nh * hd // gs) * 2, "kv_bytes_per_layer": kv_bytes,
            "timing": "hipGraph of all layers with the position in device memory (one graph "
                      "serves every token), at position ctx with cache rows [0, ctx) filled, "
                      f"mean over {replays} replays"}


def time_talker_moe(pkg, torch, dev, replays, n_layers=20):
    """The Talker's MoE blocks (FusedMoE, src/duplex/streaming/fused_moe.py:40-141) at one
    decode token: hidden 1024, 128 experts, top-6 (renormalised), expert FFN 384, shared
    expert FFN 768 with its sigmoid gate, 20 layers chained with residual adds; experts in
    bf16 and in the reference's int8 mode (per-output-row scales; the shared expert stays
    bf16).  Weights ~ N(0, 0.01), router ~ N(0, 0.05), x ~ N(0, 1), bf16, generated on the
    device.  Each timed region is one hipGraph of the 20 layers (per layer the router launch
    and, for 16-bit experts, one launch of gate|up and down; int8 experts: gate|up and down
    launches)."""
    Ht, Et, Kt, It, Ist = 1024, 128, 6, 384, 768
    dt = torch.bfloat16
    gen = torch.Generator(device=dev)
    gen.manual_seed(2468)

    def rnd(*shape, sd=0.01):
        return (torch.randn(*shape, device=dev, generator=gen) * sd).to(dt)

    x = rnd(1, Ht, sd=1.0)
    base = [dict(gu=rnd(Et, 2 * It, Ht), dn=rnd(Et, Ht, It), rw=rnd(Et, Ht, sd=0.05),
                 sgu=rnd(2 * Ist, Ht), sdn=rnd(Ht, Ist), sgw=rnd(Ht, sd=0.05))
            for _ in range(n_layers)]
    out = {}
    for mode in ("bf16", "int8"):
        layers = []
        for b in base:
            p = dict(b, gus=None, dns=None)
            if mode == "int8":
                p["gu"], p["gus"] = pkg.quantize_q8(b["gu"])
                p["dn"], p["dns"] = pkg.quantize_q8(b["dn"])
            layers.append(p)
        ws = pkg.Workspace()
        res = {}

        def step():
            h = x
            for p in layers:
                h = pkg.dmoe_forward(h, p["gu"], p["dn"], Kt, router_w=p["rw"],
                                     gate_up_scale=p["gus"], down_scale=p["dns"],
                                     shared_gate_up=p["sgu"], shared_down=p["sdn"],
                                     shared_gate_w=p["sgw"], residual=h, workspace=ws)
            res["h"] = h

        ts = graph_times(torch, step, replays, warm=50)
        if not torch.isfinite(res["h"].float()).all():
            raise RuntimeError("the Talker MoE chain produced non-finite values")
        us = sum(ts) / len(ts) / n_layers
        wb = 1 if mode == "int8" else 2
        routed = Kt * 3 * It * Ht * wb + (Kt * (2 * It + Ht) * 2 if mode == "int8" else 0)
        nbytes = (routed + 3 * Ist * Ht * 2 + Et * Ht * 2 + Ht * 2 + 3 * Ht * 2
                  + 2 * (Kt * It + Ist) * 2)
        gbs = nbytes / (us * 1e-6) / 1e9
        out[mode] = {"us_per_layer": round(us, 3), "us_per_token": round(us * n_layers, 2),
                     "us_median_per_token": round(pct(ts, 50), 2),
                     "bytes_per_layer": nbytes, "GBps": round(gbs, 1),
                     "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    return {"layers": n_layers, **out,
            "workload": "Talker MoE block at M=1: hidden 1024, 128 experts, top-6, FFN 384, "
                        "shared expert 768 + sigmoid gate, residual chain",
            "timing": f"hipGraph of {n_layers} layers (router + one expert launch each for "
                      "bf16; router, gate|up, down for int8), "
                      f"mean over {replays} replays"}


def pct(vals, q):
    v = sorted(vals)
    return v[min(len(v) - 1, int(round(q / 100 * (len(v) - 1))))]


def time_gemvs(pkg, torch, dev, replays=20):
    """The dequant-GEMV workloads at decode M = 1, AWQ g128 + zeros, fp16 scales ~ U[0.002,
    0.02], x ~ N(0, 1), fp16 out:
      single:    K=2048 -> N=768, 640 distinct weight copies (526 MB, twice the Infinity
                 Cache) launched back to back;
      attention: q 2048->4096, k/v 2048->512, o 4096->2048, 64 distinct layer sets (628 MB),
                 each projection timed on its own (all 64 copies back to back), the four
                 of a layer back to back, and q/k/v as one launch followed by o.
    Each workload runs on the AWQ tensors as the checkpoint holds them (one launch, split
    along K, the last slice of each column strip summing the strip's partials; q/k/v as one
    launch over their columns side by side, PackedQKV(repack=False)) and on their CT+zeros
    repack (one launch, what PackedLinear installs).
    Times are per GEMV (or per layer of four), mean / median / p99 over graph replays."""
    from qwen3_omni_duplex_amd import _lib

    lb = pkg.lib()
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)

    def awq_copies(K, N, n):
        qw = torch.randint(-2**31, 2**31, (n, K, N // 8), dtype=torch.int32, device=dev,
                           generator=gen)
        qz = torch.randint(-2**31, 2**31, (n, K // G, N // 8), dtype=torch.int32, device=dev,
                           generator=gen)
        sc = (torch.rand(n, K // G, N, device=dev, generator=gen) * 0.018 + 0.002).half()
        return pkg.QWeight.awq(qw, sc, qz, group=G)

    def per_copy(w):
        """i4_qweight descriptors of each copy as an E = 1 Linear weight"""
        c = w.c()
        pes, ses = w.packed[0].numel() * 4, w.scale[0].numel() * 2
        zes = w.zeros[0].numel() * 4
        return [_lib.QWeightC(packed=c.packed + i * pes, scale=c.scale + i * ses,
                              zeros=c.zeros + i * zes, packed_estride=0, scale_estride=0,
                              zeros_estride=0, layout=c.layout, group=c.group,
                              scale_dtype=c.scale_dtype, E=1, N=c.N, K=c.K)
                for i in range(w.E)]

    class Proj:
        def __init__(self, K, N, n):
            self.K, self.N = K, N
            awq = awq_copies(K, N, n)
            ct = awq.to_ct()
            self.desc = {"awq": per_copy(awq), "ct": per_copy(ct)}
            self.keep = (awq, ct)
            self.x = torch.randn(1, K, device=dev, generator=gen).half()
            self.y = torch.empty(1, N, dtype=torch.float16, device=dev)
            nb = lb.i4_linear_workspace_bytes(ctypes.byref(self.desc["awq"][0]), 1)
            # split-K workspace: its status word starts at 0, no other contents needed
            self.ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=dev)

        def launch(self, layout, i):
            d = self.desc[layout][i]
            rc = lb.i4_linear(self.x.data_ptr(), _lib.F16, 1, ctypes.byref(d), None,
                              self.y.data_ptr(), _lib.F16, self.ws.data_ptr(), self.ws.numel(),
                              torch.cuda.current_stream().cuda_stream)
            if rc:
                raise RuntimeError(lb.i4_strerror(rc).decode())

    def stats(times, per, nbytes):
        t = [v / per for v in times]
        mean = sum(t) / len(t)
        return {"us": round(mean, 3), "us_median": round(pct(t, 50), 3),
                "us_p99": round(pct(t, 99), 3), "GBps": round(nbytes / (mean * 1e-6) / 1e9, 1),
                "hbm_frac": round(nbytes / (mean * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                "bytes": nbytes}

    out = {}
    n1 = 640
    single = Proj(2048, 768, n1)
    nbytes = awq_gemv_bytes(2048, 768)
    for layout in ("ct", "awq"):
        ts = graph_times(torch, lambda: [single.launch(layout, i) for i in range(n1)], replays)
        out[f"single_{layout}"] = stats(ts, n1, nbytes)
        log(f"GEMV 2048->768 ({layout}): {out[f'single_{layout}']['us']:.2f} us")
    # the same GEMV through the Python module path (PackedLinear.forward -> ops.linear ->
    # i4_linear, each module with its own kept workspace) on the same copies: eager calls,
    # host dispatch included, and the same calls captured in a hipGraph (what the module
    # path enqueues on the device)
    n_py = n1
    py = {}
    for li, layout in enumerate(("awq", "ct")):
        w = single.keep[li]
        lins = [pkg.PackedLinear.from_qweight(
            pkg.QWeight(w.packed[i:i + 1], w.scale[i:i + 1], w.zeros[i:i + 1], w.layout, w.group,
                        w.N, w.K), repack=False, tile=False) for i in range(n_py)]
        xp = single.x

        def calls(lins=lins, xp=xp):
            for m in lins:
                m(xp)

        for _ in range(3):
            calls()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(5):
            calls()
        e1.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e6 / (5 * n_py)
        g = stats(graph_times(torch, calls, replays), n_py, nbytes)
        py[layout] = {"us_eager": round(e0.elapsed_time(e1) * 1e3 / (5 * n_py), 3),
                      "us_eager_wall": round(wall, 3), "us_graph": g["us"],
                      "us_graph_p99": g["us_p99"]}
        del lins
    py["timing"] = (f"PackedLinear.forward on the {n_py} copies, eager (HIP events and wall "
                    f"clock around 5 passes) and as one hipGraph of the {n_py} calls (mean over "
                    "replays)")
    out["python_linear"] = py
    log("PackedLinear 2048->768: " + ", ".join(
        f"{k} eager {v['us_eager']:.2f} / graph {v['us_graph']:.2f} us"
        for k, v in py.items() if k != "timing"))
    del single
    n2 = 64
    projs = {"q": Proj(2048, 4096, n2), "k": Proj(2048, 512, n2), "v": Proj(2048, 512, n2),
             "o": Proj(4096, 2048, n2)}
    # the q, k, v rows of each layer set in one CT weight (what PackedQKV installs)
    cts = [projs[n].keep[1] for n in ("q", "k", "v")]
    qkv = Proj.__new__(Proj)
    qkv.K, qkv.N = 2048, sum(c.N for c in cts)
    wq = pkg.QWeight(torch.cat([c.packed for c in cts], 1), torch.cat([c.scale for c in cts], 1),
                     torch.cat([c.zeros for c in cts], 1), "ct", G, qkv.N, qkv.K)
    # and in AWQ packing, the q, k, v columns side by side (PackedQKV(repack=False))
    awqs = [projs[n].keep[0] for n in ("q", "k", "v")]
    wqa = pkg.QWeight(torch.cat([a.packed for a in awqs], 2), torch.cat([a.scale for a in awqs], 2),
                      torch.cat([a.zeros for a in awqs], 2), "awq", G, qkv.N, qkv.K)
    qkv.desc = {"ct": per_copy(wq), "awq": per_copy(wqa)}
    qkv.keep = (wq, wqa)
    qkv.x = projs["q"].x
    qkv.y = torch.empty(1, qkv.N, dtype=torch.float16, device=dev)
    nb = lb.i4_linear_workspace_bytes(ctypes.byref(qkv.desc["awq"][0]), 1)
    qkv.ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=dev)
    for layout in ("ct", "awq"):
        att = {}
        for name, p in projs.items():
            ts = graph_times(torch, lambda p=p: [p.launch(layout, i) for i in range(n2)], replays)
            att[name] = stats(ts, n2, awq_gemv_bytes(p.K, p.N))

        def layer_seq():
            for i in range(n2):
                for p in projs.values():
                    p.launch(layout, i)

        ts = graph_times(torch, layer_seq, replays)
        att["qkvo_back_to_back"] = stats(ts, n2, sum(awq_gemv_bytes(p.K, p.N)
                                                    for p in projs.values()))
        # q/k/v as one launch (PackedQKV: CT rows, or AWQ columns side by side), then o
        def fused_seq():
            for i in range(n2):
                qkv.launch(layout, i)
                projs["o"].launch(layout, i)

        ts = graph_times(torch, fused_seq, replays)
        att["qkv_fused_then_o"] = stats(ts, n2, sum(awq_gemv_bytes(p.K, p.N)
                                                    for p in projs.values()))
        out[f"attention_{layout}"] = att
        log(f"attention q/k/v/o ({layout}): " + ", ".join(
            f"{k} {v['us']:.2f}" for k, v in att.items()) + " us")
    # M > 1 (prefill): the same projections on their tile copies (MFMA over 64-row tiles,
    # what PackedLinear runs from TILE_ROWS rows on) and, at M = 32, the per-row GEMV
    pre = {}
    pp = dict(projs, qkv=qkv)  # qkv: the q/k/v rows in one weight (PackedQKV)
    for M in (32, 512):
        xm = torch.randn(M, 4096, device=dev, generator=gen).half()
        ym = torch.empty(M, qkv.N, dtype=torch.float16, device=dev)
        res = {}
        for layout in (("tile", "ct") if M == 32 else ("tile",)):
            for name, p in pp.items():
                if layout == "tile" and "tile" not in p.desc:
                    t = p.keep[0 if name == "qkv" else 1].to_tile()  # from the CT weight
                    p.desc["tile"] = per_copy(t)
                    p.keep = p.keep + (t,)
                nb = max(lb.i4_linear_workspace_bytes(ctypes.byref(p.desc[layout][0]), M), 16)
                wsm = torch.empty(nb, dtype=torch.uint8, device=dev)

                def seq(p=p, layout=layout, wsm=wsm):
                    for i in range(n2):
                        rc = lb.i4_linear(xm.data_ptr(), _lib.F16, M,
                                          ctypes.byref(p.desc[layout][i]), None, ym.data_ptr(),
                                          _lib.F16, wsm.data_ptr(), wsm.numel(),
                                          torch.cuda.current_stream().cuda_stream)
                        if rc:
                            raise RuntimeError(lb.i4_strerror(rc).decode())

                ts = graph_times(torch, seq, max(3, replays // 4))
                st = stats(ts, n2, awq_gemv_bytes(p.K, p.N) + (M - 1) * 2 * (p.K + p.N))
                tf = 2.0 * M * p.N * p.K / (st["us"] * 1e-6) / 1e12
                st.update({"TFLOPs": round(tf, 2), "mfma_frac": round(tf / MFMA_PEAK_TFLOPS, 4)})
                res[f"{name}_{layout}"] = st
        pre[f"M{M}"] = res
        log(f"attention q/k/v/o at M={M}: " + ", ".join(
            f"{k} {v['us']:.2f} us ({v['TFLOPs']:.0f} TF/s)" for k, v in res.items()))
    out["attention_prefill"] = pre
    out["timing"] = ("hipGraph of all copies back to back, HIP events per replay; per-GEMV "
                     "time = replay / copies; bytes = AWQ g128 weights + scales + zeros + x + y")
    return out


def routing_stats(sels, per_expert_bytes, extra_bytes):
    """Realised expert histogram of a list of [T, k] selections: distinct experts hit,
    tokens per hit expert, and the layer's algorithmic bytes (distinct experts' weights)."""
    import torch

    hits, mx, over64, over16, low = [], [], [], [], []
    for sel in sels:
        cnt = torch.bincount(sel.reshape(-1).long().cpu(), minlength=E)
        hits.append(int((cnt > 0).sum()))
        mx.append(int(cnt.max()))
        over64.append(int((cnt > 64).sum()))
        over16.append(int((cnt > 16).sum()))
        low.append(int((cnt <= 2).sum()))
    n = len(sels)
    avg = lambda v: round(sum(v) / n, 2)
    d = avg(hits)
    return {"experts_hit": d, "max_tokens_per_expert": avg(mx), "experts_over_64": avg(over64),
            "experts_over_16": avg(over16), "experts_0_to_2": avg(low),
            "bytes": int(d * per_expert_bytes + extra_bytes)}


def routing_agreement(torch, dev, mods, rows1, rows32):
    """The GPU's top-8 from x against the exact ranking on the host, on the M = 1 decode
    inputs and M = 32 batches of every layer: the router launch of ops.moe_forward (fp16 x
    and the layer's fp16 router weight, no norm) against the float64 product rounded once to
    fp16 and ranked value-descending with ties to the lower id (fused_packed_moe.py:195-197).
    The GPU accumulates in fp32, so a logit within an ulp of a rounding boundary may round
    to its neighbour and swap two near-tied experts.  Returns {M1, M32: rows, differ, rate}."""
    from qwen3_omni_duplex_amd import ops

    ws = ops.Workspace()
    out = {}
    for name, batches in (("M1", rows1), ("M32", rows32)):
        n = bad = 0
        for m in mods:
            wr = m.router_w.detach().double().cpu()
            tiles = dict(gate_up_tile=m.gate_up_tile, down_tile=m.down_tile)
            for x in batches:
                _, sel, _ = ops.moe_forward(x, m.gate_up, m.down, TOPK, router_w=m.router_w,
                                            return_routing=True, workspace=ws, **tiles)
                lg = (x.double().cpu() @ wr.T).half().double()
                ref = torch.sort(lg, dim=1, descending=True, stable=True)[1][:, :TOPK]
                bad += int((sel.long().cpu() != ref).any(dim=1).sum())
                n += x.shape[0]
        out[name] = {"rows": n, "differ": bad, "rate": round(bad / n, 5)}
    out["reference"] = ("float64 x @ router_w.T rounded once to fp16, ranked on the host "
                        "(value descending, ties to the lower id); a row differs if any of its "
                        "8 ids, in order, differs")
    return out


def cpu_model_name() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def cpu_baseline(torch, first, xs, seconds):
    """The reference's CPU paths restated in torch (oracle/cpu_baseline.py), timed on this host
    over bounded samples: the M = 1 MoE layer on all threads (the reported value) and on one
    thread, the M = 32 layer, 64-token slices of the M = 512 layer, and reference_gemv for
    the single 2048 -> 768 GEMV and the four attention projections back to back.  The weights are layer 0's (MoE) and fresh seeded AWQ
    tensors of the workload's shapes (GEMVs); `seconds` bounds the whole leg."""
    from oracle import cpu_baseline as cb

    g, u, d, wr = first
    host = lambda p: tuple(t.detach().cpu() for t in p)
    gate, up, down = host(g), host(u), host(d)
    router = wr.detach().float().cpu()
    x = torch.stack([t.detach().float().cpu().reshape(-1) for t in xs[:64]])
    threads = torch.get_num_threads()
    med, reps = cb.time_layer(x, router, gate, up, down, seconds=0.3 * seconds, top_k=TOPK,
                              group=G)
    torch.set_num_threads(1)
    try:
        med1, reps1 = cb.time_layer(x, router, gate, up, down, seconds=0.12 * seconds, top_k=TOPK,
                                    group=G)
    finally:
        torch.set_num_threads(threads)
    x32 = [x[i:i + 32] for i in (0, 32)]
    med32, reps32 = cb.time_calls(
        lambda i: cb.moe_layer(x32[i % 2], router, gate, up, down, TOPK, G), 0.18 * seconds, 2)
    # M = 512: the reference's CPU path loops over tokens (each dequantises its own 8
    # experts), so a layer costs 512 tokens' worth; timed on 64-token slices of fresh rows
    gen512 = torch.Generator().manual_seed(512)
    x512 = torch.randn(128, H, generator=gen512)
    med512, reps512 = cb.time_calls(
        lambda i: cb.moe_layer(x512[64 * (i % 2):64 * (i % 2) + 64], router, gate, up, down,
                               TOPK, G), 0.2 * seconds, 2)

    gen = torch.Generator().manual_seed(5)

    def awq(K, N):
        return (torch.randint(-2**31, 2**31, (K, N // 8), dtype=torch.int32, generator=gen),
                torch.randint(-2**31, 2**31, (K // G, N // 8), dtype=torch.int32, generator=gen),
                (torch.rand(K // G, N, generator=gen) * 0.018 + 0.002).half())

    c1 = awq(H, I)
    xk = torch.randn(4, 4096, generator=gen).half()
    med_c1, reps_c1 = cb.time_calls(lambda i: cb.gemv(xk[i % 4, :H], *c1, group=G),
                                    0.08 * seconds)
    proj = {"q": awq(2048, 4096), "k": awq(2048, 512), "v": awq(2048, 512), "o": awq(4096, 2048)}

    def attn(i):
        xi = xk[i % 4]
        for name in ("q", "k", "v"):
            cb.gemv(xi[:2048], *proj[name], group=G)
        cb.gemv(xi, *proj["o"], group=G)

    med_c2, reps_c2 = cb.time_calls(attn, 0.12 * seconds)
    model = cpu_model_name()
    return {
        "value": round(med * 1e6, 1), "unit": "us/layer", "cores": threads, "kind": "port",
        "sample": f"{reps} M=1 MoE layers (layer 0 weights, distinct inputs), median; torch fp32 "
                  f"on {threads} threads of {model}",
        "cpu_model": model, "host_threads": os.cpu_count(),
        "one_thread": {"us_per_layer": round(med1 * 1e6, 1), "reps": reps1},
        "configs": {
            "single_gemv_2048x768": {"us": round(med_c1 * 1e6, 1), "reps": reps_c1,
                                     "path": "reference_gemv: fp32 dequant + matmul"},
            "attention_qkvo_back_to_back": {"us": round(med_c2 * 1e6, 1), "reps": reps_c2,
                                            "path": "reference_gemv x 4 (q, k, v, o)"},
            "moe_layer_M32": {"us_per_layer": round(med32 * 1e6, 1), "reps": reps32,
                              "tokens_per_s": round(32 / med32, 1),
                              "path": "CPU expert path, per token (fused_packed_moe.py:202-220)"},
            "moe_layer_M512": {"us_per_layer": round(med512 * 512 / 64 * 1e6, 1),
                               "us_per_token": round(med512 / 64 * 1e6, 1), "reps": reps512,
                               "tokens_per_s": round(64 / med512, 1),
                               "sample": "64-token slices of the 512 (x ~ N(0, 1)), median; "
                                         "the per-token loop makes a layer 8 slices",
                               "path": "CPU expert path, per token (fused_packed_moe.py:202-220)"},
        },
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=24)
    ap.add_argument("--kernel-rounds", type=int, default=8)
    ap.add_argument("--decode-step", action=argparse.BooleanOptionalAction, default=True,
                    help="also time the whole Thinker decode step (attention + MoE per layer)")
    ap.add_argument("--talker", action=argparse.BooleanOptionalAction, default=True,
                    help="also time the Talker's 16-bit / int8 MoE blocks (20 layers, M=1)")
    ap.add_argument("--context", type=int, default=1024,
                    help="cached positions the decode step attends")
    ap.add_argument("--cpu-seconds", type=float, default=20.0,
                    help="bound on the CPU baseline leg (all of its samples together)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--prefill", action=argparse.BooleanOptionalAction, default=True,
                    help="also time the M=32 and M=512 workloads (reported as extra fields)")
    ap.add_argument("--eager", action="store_true", help="time without a hipGraph")
    ap.add_argument("--gemv", action=argparse.BooleanOptionalAction, default=True,
                    help="also time the single and attention-projection dequant-GEMVs")
    ap.add_argument("--replays", type=int, default=20,
                    help="graph replays per timed GEMV / prefill workload")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 10 device copies of 64 MiB (calibrates the FETCH_SIZE / "
                         "WRITE_SIZE counters against a copy of known size) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the single-GPU decode path only: run it with --gpus 1 "
              "(one process, one MI355X); multi-GPU sharding is not part of this build.",
              file=sys.stderr)
        return 2

    import torch

    if args.calibrate_copy:
        src = torch.ones(64 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "device copy", "bytes_read": 64 << 20,
                          "bytes_written": 64 << 20, "dispatches": 10}))
        return 0

    from __graft_entry__ import load_package

    pkg = load_package()
    dev = torch.device("cuda:0")
    log(f"building {args.layers} layers of synthetic AWQ weights on {torch.cuda.get_device_name(0)}")
    mods, first = make_layers(pkg, torch, args.layers, dev, keep_first_awq=not args.no_cpu)
    log("weights resident; generating inputs")
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    P = 64
    xs = [torch.randn(1, H, device=dev, generator=gen).half() for _ in range(P)]
    layers = [m.stack_entry() for m in mods]
    ws = pkg.Workspace()

    # ---- eager: one C call per token (the stack's 2 launches per layer and a last one)
    lb = pkg.lib()
    from qwen3_omni_duplex_amd import _lib, ops

    arr = (_lib.MoeWeightsC * len(layers))(*[ops.moe_weights_c(*layer) for layer in layers])
    nbytes = lb.i4_moe_stack_workspace_bytes(1, H, I, E, TOPK)
    wbuf = ws.get(nbytes, dev)
    out = torch.empty(1, H, dtype=torch.float16, device=dev)
    s_ptr = torch.cuda.current_stream(dev).cuda_stream

    def eager_step(i):
        rc = lb.i4_moe_stack_forward(xs[i % P].data_ptr(), _lib.F16, 1, arr, len(layers), TOPK, 1,
                                     out.data_ptr(), wbuf.data_ptr(), wbuf.numel(), s_ptr)
        if rc:
            raise RuntimeError(lb.i4_strerror(rc).decode())

    # ms of each token through the stack, from each path's own events
    per_eager, per_graph = [], []
    ms_eager, wall_eager = time_stack(torch, eager_step, args.steps, args.warmup, per_eager)
    log(f"eager: {ms_eager:.3f} ms/token ({ms_eager * 1e3 / args.layers:.2f} us/layer)")

    # ---- hipGraph: the 49 launches of one token captured once, replayed per token
    ms_graph = None
    if not args.eager:
        static_x = xs[0].clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            ops.moe_stack(static_x, layers, TOPK, workspace=ws)
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            g_out = ops.moe_stack(static_x, layers, TOPK, workspace=ws)

        def graph_step(i):
            static_x.copy_(xs[i % P])
            graph.replay()

        ms_graph, _ = time_stack(torch, graph_step, args.steps, args.warmup, per_graph)
        # the replay computes what the eager path computes
        graph_step(5)
        eager_step(5)
        torch.cuda.synchronize()
        if not torch.isfinite(out).all():
            raise RuntimeError("the stack produced non-finite values")
        if not torch.equal(g_out, out):
            raise RuntimeError("graph replay differs from the eager stack")
        log(f"graph: {ms_graph:.3f} ms/token ({ms_graph * 1e3 / args.layers:.2f} us/layer)")

    # value: the faster of the two ways to run a token (the graph replay also pays a copy of
    # the token's input into the captured buffer; the eager C call reads it in place)
    if ms_graph is not None and ms_graph <= ms_eager:
        ms, mode = ms_graph, "hipGraph replay of the stack (input copied into its buffer)"
        per_token = per_graph
    else:
        ms, mode = ms_eager, "one i4_moe_stack_forward call per token (49 launches)"
        per_token = per_eager
    us_layer = ms * 1e3 / args.layers

    # ---- dominant kernel: the decode experts launch, HIP events on its stream
    hs = []
    h = xs[1]
    for m in mods:
        hs.append(h)
        h = m(h, residual=h)
    torch.cuda.synchronize()
    k_us, k_layer, k_router = time_experts(pkg, torch, dev, mods, hs, args.kernel_rounds)
    achieved = B_EXPERTS_LAUNCH / (k_us * 1e-6) / 1e9
    log(f"experts kernel: {k_us:.2f} us/launch (24 back to back; layer {k_layer:.2f}, "
        f"router alone {k_router:.2f}) -> {achieved:.0f} GB/s")

    # ---- other workloads of the same layer: M=32 (router from weights) and M=512 prefill
    # with Zipf(1.1)-skewed logits (MFMA tiles for hot experts), rotating over the layers
    prefill = {}
    if args.prefill:
        gen2 = torch.Generator(device=dev)
        gen2.manual_seed(7)
        for T in (32, 512):
            xT = [torch.randn(T, H, device=dev, generator=gen2).half() for _ in range(4)]
            lgT = None
            if T == 512:
                rank = torch.randperm(E, device=dev, generator=gen2).float() + 1
                lgT = [(-1.1 * 2.0 * torch.log(rank)[None, :]
                        - torch.log(-torch.log(torch.rand(T, E, device=dev, generator=gen2))))
                       .half() for _ in range(4)]
            wsT = pkg.Workspace()
            nl = len(mods)
            # layer li takes input li % 4: one replay = every layer once, routing and hence
            # the expert histogram differ from layer to layer
            sels = []
            for li, m in enumerate(mods):
                lg = (ops.router_logits(xT[li % 4], m.router_w) if lgT is None else lgT[li % 4])
                sels.append(ops.route(lg, TOPK)[1])
            rs = routing_stats(sels, B_GATE_UP_EXPERT + B_DOWN_EXPERT,
                               (B_ROUTER if lgT is None else 0) + 2 * 2 * H * T)

            def run_all(T=T, xT=xT, lgT=lgT, wsT=wsT):
                for li, m in enumerate(mods):
                    tiles = dict(gate_up_tile=m.gate_up_tile, down_tile=m.down_tile)
                    x = xT[li % 4]
                    if lgT is None:
                        ops.moe_forward(x, m.gate_up, m.down, TOPK, router_w=m.router_w,
                                        residual=x, workspace=wsT, **tiles)
                    else:
                        ops.moe_forward(x, m.gate_up, m.down, TOPK, logits=lgT[li % 4],
                                        residual=x, workspace=wsT, **tiles)

            ts = [t / nl for t in graph_times(torch, run_all, args.replays)]
            us_T = sum(ts) / len(ts)
            flops = T * TOPK * 3 * 2 * H * I
            tf = flops / (us_T * 1e-6) / 1e12
            gbs = rs["bytes"] / (us_T * 1e-6) / 1e9
            prefill[f"M{T}"] = {
                "us_per_layer": round(us_T, 2), "us_median": round(pct(ts, 50), 2),
                "us_p99": round(pct(ts, 99), 2),
                "tokens_per_s": round(T / (us_T * 1e-6), 1),
                "expert_TFLOPs": round(tf, 2), "mfma_frac": round(tf / MFMA_PEAK_TFLOPS, 4),
                "GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                "routing": ("router weights, x ~ N(0, 1)" if lgT is None else
                            "logits -1.1 tau ln(rank) + Gumbel, tau 2"),
                "realised": rs,
                "timing": f"hipGraph of the {nl} layers (input li % 4), mean over "
                          f"{args.replays} replays"}
            log(f"M={T}: {us_T:.1f} us/layer, {tf:.1f} TFLOP/s, {gbs:.0f} GB/s, "
                f"{rs['experts_hit']} experts hit")

    gen3 = torch.Generator(device=dev)
    gen3.manual_seed(11)
    rows32 = [torch.randn(32, H, device=dev, generator=gen3).half() for _ in range(4)]
    routing = routing_agreement(torch, dev, mods, xs, rows32)
    log(f"routing vs the host's exact top-8: M=1 {routing['M1']['differ']} of "
        f"{routing['M1']['rows']} rows differ, M=32 {routing['M32']['differ']} of "
        f"{routing['M32']['rows']}")

    gemv = time_gemvs(pkg, torch, dev, args.replays) if args.gemv else None

    decode = None
    if args.decode_step:
        decode = time_decode_step(pkg, torch, dev, mods, args.context, args.replays)
        log(f"decode step (context {args.context}): {decode['step']['us_per_token']:.1f} us/token, "
            f"attention {decode['attention']['us_per_layer']:.2f} us/layer")

    talker = None
    if args.talker:
        talker = time_talker_moe(pkg, torch, dev, args.replays)
        log(f"Talker MoE: bf16 {talker['bf16']['us_per_layer']:.2f} us/layer, "
            f"int8 {talker['int8']['us_per_layer']:.2f} us/layer")

    # ---- CPU baseline
    cpu = None
    if not args.no_cpu:
        log(f"CPU baseline: ~{args.cpu_seconds:.0f} s sample")
        cpu = cpu_baseline(torch, first, xs, args.cpu_seconds)
        log(f"CPU: {cpu['value']:.0f} us/layer ({cpu['cores']} threads), "
            f"{cpu['one_thread']['us_per_layer']:.0f} us/layer on one thread")

    res = {
        "metric": "µs per int4 Thinker MoE layer at M=1; achieved HBM GB/s as % of MI355X peak",
        "value": round(us_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x fp16 activations, fp32 accumulation",
        "data": "synthetic (seeded, generated on device)",
        "config": {
            "workload": "Thinker[0:24] int4 MoE stack, decode M=1: 128 experts, top-8, hidden 2048, "
                        "expert FFN 768, AWQ g128 + zeros (fp16 scales) repacked to CT+zeros, "
                        "pre-MoE RMSNorm + residual adds; one step = one token through 24 layers",
            "layers": args.layers, "tokens_per_step": 1,
            "timing": mode,
        },
        "tokens_per_s": round(1e3 / ms, 1),
        "us_per_layer_eager": round(ms_eager * 1e3 / args.layers, 3),
        "us_per_layer_graph": None if ms_graph is None else round(ms_graph * 1e3 / args.layers, 3),
        "us_per_layer_median": round(pct(per_token, 50) * 1e3 / args.layers, 3),
        "us_per_layer_p99": round(pct(per_token, 99) * 1e3 / args.layers, 3),
        "layer_GBps": round(B_LAYER / (us_layer * 1e-6) / 1e9, 1),
        "layer_hbm_frac": round(B_LAYER / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {
            "kernel": "k_ct_moe_m1x (decode top-8 routing + gate/up + SiLU + down of the 8 "
                      "experts, one launch, each slot on its own XCD)",
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": EXPERTS_TRAFFIC_BYTES,
            "bytes_per_launch": B_EXPERTS_LAUNCH, "us_per_launch": round(k_us, 3),
            "timing": "HIP events around the 24 layers' experts launches back to back (their "
                      "router launches run first, each layer with its own workspace)",
            "us_per_layer_launches": round(k_layer, 3), "us_per_router_launch": round(k_router, 3),
        },
        "cpu_baseline": cpu,
        "other_workloads": prefill,
        "routing_agreement": routing,
        "gemv": gemv,
        "thinker_decode_step": decode,
        "talker_moe": talker,
    }
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Functional ops with the reference's signatures, executed by libi4moe.

    dequant_gemv   src/duplex/streaming/triton_dequant_gemv.py:85-113
    reference_gemv is not provided here: it is the checker's job (oracle/)
    unpack4        src/duplex/streaming/fused_packed_moe.py:54-65 (device)
    dequant        FusedPackedMoE._dequant, fused_packed_moe.py:183-189 (device)
    route          fused_packed_moe.py:195-199
    moe_forward    FusedPackedMoE.forward, fused_packed_moe.py:191-263
    moe_stack      Thinker[0:24] MoE stack with residual adds (clock.py:168-171)
    rmsnorm        Qwen3OmniMoeThinkerTextRMSNorm (the decoder's input_layernorm)
    rmsnorm_linear the same norm folded into an int4 Linear (one launch)
    attn_decode    Qwen3OmniMoeThinkerTextAttention.forward between its projections,
                   one decode token with a KV cache (clock.py:164-172)
    dmoe_forward   FusedMoE.forward, src/duplex/streaming/fused_moe.py:99-141 (16-bit or
                   int8 experts, sigmoid-gated shared expert: the Talker's block)

Every op enqueues on torch's current stream of the tensors' device and never
synchronises.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .weights import QWeight


def _gemv_ws(nbytes: int, device: torch.device, workspace: "Workspace | None",
             kind: str = "awq"):
    """The split-K workspace of an AWQ GEMV / linear call (None when the call needs none):
    the caller's Workspace, else one kept per device and stream (the library takes one
    workspace per stream).  Its status word must start at 0, so a workspace is zeroed when
    it is allocated and never again: calls need no initial contents beyond that."""
    if nbytes == 0:
        return None
    if workspace is None:
        key = (device.index, _lib.stream(device), kind)
        workspace = _STREAM_WS.setdefault(key, Workspace())
    return workspace.get(nbytes, device, zeroed=True)


_STREAM_WS: dict = {}


def gemv_status(workspace: "Workspace | None" = None, device: torch.device | None = None) -> int:
    """The status word of an AWQ split-K GEMV workspace (the per-stream one when none is
    given): 0, or the I4_ERR_HANDOFF code once a call on it gave up; synchronises."""
    if workspace is None:
        dev = device or torch.device("cuda", torch.cuda.current_device())
        workspace = _STREAM_WS.get((dev.index, _lib.stream(dev), "awq"))
    if workspace is None or workspace.buf is None:
        return 0
    torch.cuda.synchronize(workspace.buf.device)
    return int(workspace.buf[:4].view(torch.int32).item())


def dequant_gemv(x, packed, scale, sel, group=32, block_r=64, nw_blk=8, *, zeros=None,
                 layout="ct", out_dtype=torch.float32, workspace=None):
    """y[j, r] = sum_c W[sel[j], r, c] * x[j, c], W dequantised from int4 on the fly.

    Same contract as the reference's dequant_gemv: x [K] (shared by every
    selected expert) or [k, K] (one row per expert); packed/scale in the CT
    layout [E, R, K/8] / [E, R, K/group] (or AWQ with layout="awq" and zeros);
    sel [k] expert ids; returns [k, R] float32.  block_r and nw_blk are the
    reference's Triton tile sizes and have no meaning here.
    """
    del block_r, nw_blk
    dev = _lib.require_device(x, packed, scale, sel, zeros)
    xt = _lib.half_code(x.dtype)
    sel32 = sel.to(torch.int32).contiguous()
    k = sel32.numel()
    if layout == "ct":
        w = QWeight(packed, scale, zeros, "ct", group, packed.shape[-2], packed.shape[-1] * 8)
    else:
        w = QWeight(packed, scale, zeros, "awq", group, packed.shape[-1] * 8, packed.shape[-2])
    K = w.K
    if x.dim() == 1:
        if x.numel() != K:
            raise RuntimeError(f"x has {x.numel()} elements, weights have K={K}")
        xc, s_x = x.contiguous(), 0
    else:
        if x.shape[-1] != K or x.shape[0] != k:
            raise RuntimeError(f"x shape {tuple(x.shape)} does not match [k={k}, K={K}]")
        xc = x.contiguous()
        s_x = K
    out = torch.empty(k, w.N, dtype=out_dtype, device=dev)
    lb = _lib.lib()
    cw = w.c()
    ws = _gemv_ws(lb.i4_dq_gemv_workspace_bytes(ctypes.byref(cw), k), dev, workspace)
    _lib.check(lb.i4_dq_gemv(xc.data_ptr(), xt, s_x, ctypes.byref(cw), sel32.data_ptr(), k,
                             out.data_ptr(), _lib.dtype_code(out_dtype),
                             None if ws is None else ws.data_ptr(),
                             0 if ws is None else ws.numel(), _lib.stream(dev)))
    return out


def dequant_gemv_bounded(x: torch.Tensor, w: QWeight, sel: torch.Tensor, max_polls: int,
                         reducers_only: bool, workspace: "Workspace",
                         out_dtype=torch.float32) -> torch.Tensor:
    """i4_dq_gemv_bounded: the AWQ split-K GEMV with a caller bound on its hand-over wait,
    optionally only the reducing workgroups (whose partials then never arrive: the wait
    gives up, NaN out, I4_ERR_HANDOFF in the workspace's status word).  x [k, K]."""
    dev = _lib.require_device(x, w.packed, sel)
    sel32 = sel.to(torch.int32).contiguous()
    k = sel32.numel()
    xc = x.reshape(k, w.K).contiguous()
    out = torch.empty(k, w.N, dtype=out_dtype, device=dev)
    lb = _lib.lib()
    cw = w.c()
    ws = _gemv_ws(lb.i4_dq_gemv_workspace_bytes(ctypes.byref(cw), k), dev, workspace)
    _lib.check(lb.i4_dq_gemv_bounded(xc.data_ptr(), _lib.half_code(x.dtype), w.K,
                                     ctypes.byref(cw), sel32.data_ptr(), k, out.data_ptr(),
                                     _lib.dtype_code(out_dtype), _lib.ptr(ws),
                                     0 if ws is None else ws.numel(), int(max_polls),
                                     int(reducers_only), _lib.stream(dev)))
    return out


def linear(x: torch.Tensor, w: QWeight, bias: torch.Tensor | None = None,
           out_dtype: torch.dtype | None = None,
           workspace: "Workspace | None" = None) -> torch.Tensor:
    """y = x W^T (+ bias) for every row of x in one launch (E = 1 weight).  workspace: kept
    by the caller for the calls that need one (an AWQ weight split along K, a tile weight
    split along K); by default one per device and stream."""
    dev = _lib.require_device(x, w.packed, bias)
    xt = _lib.half_code(x.dtype)
    lead = x.shape[:-1]
    if x.shape[-1] != w.K:
        raise RuntimeError(f"x has K={x.shape[-1]}, weight has K={w.K}")
    flat = x.reshape(-1, w.K).contiguous()
    M = flat.shape[0]
    od = out_dtype or x.dtype
    y = torch.empty(M, w.N, dtype=od, device=dev)
    b = None
    if bias is not None:
        b = bias.to(od).contiguous()
        if b.numel() != w.N:
            raise RuntimeError("bias length != out_features")
    lb = _lib.lib()
    cw = w.c()
    ws = _gemv_ws(lb.i4_linear_workspace_bytes(ctypes.byref(cw), M), dev, workspace, w.layout)
    _lib.check(lb.i4_linear(flat.data_ptr(), xt, M, ctypes.byref(cw), _lib.ptr(b), y.data_ptr(),
                            _lib.dtype_code(od), None if ws is None else ws.data_ptr(),
                            0 if ws is None else ws.numel(), _lib.stream(dev)))
    return y.view(*lead, w.N)


def unpack_nibbles(w: QWeight) -> torch.Tensor:
    """Raw nibbles 0..15 of every expert in logical [E, N, K] order (uint8)."""
    dev = _lib.require_device(w.packed)
    out = torch.empty(w.E, w.N, w.K, dtype=torch.uint8, device=dev)
    cw = w.c()
    _lib.check(_lib.lib().i4_unpack(ctypes.byref(cw), out.data_ptr(), _lib.stream(dev)))
    return out


def unpack4(packed: torch.Tensor, out_cols: int) -> torch.Tensor:
    """The reference's unpack4 on a CT tensor: signed nibble - 8, [..., out_cols]."""
    lead = packed.shape[:-2]
    p = packed.reshape(-1, packed.shape[-2], packed.shape[-1])
    G = 32
    ng = -(-p.shape[-1] * 8 // G)
    dummy_scale = torch.ones(p.shape[0], p.shape[1], ng, dtype=torch.float16, device=p.device)
    w = QWeight(p, dummy_scale, None, "ct", G, p.shape[1], p.shape[2] * 8)
    q = unpack_nibbles(w).to(torch.int32) - 8
    return q[..., :out_cols].reshape(*lead, p.shape[1], out_cols)


def dequant(w: QWeight, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Dense [E, N, K] = (nibble - zero) * scale (FusedPackedMoE._dequant)."""
    dev = _lib.require_device(w.packed)
    out = torch.empty(w.E, w.N, w.K, dtype=out_dtype, device=dev)
    cw = w.c()
    _lib.check(_lib.lib().i4_dequant(ctypes.byref(cw), out.data_ptr(), _lib.dtype_code(out_dtype),
                                     _lib.stream(dev)))
    return out


def router_logits(x: torch.Tensor, router_w: torch.Tensor, norm_w: torch.Tensor | None = None,
                  norm_eps: float = 1e-6, return_xn: bool = False):
    """gate(x): [T, H] x [E, H]^T -> [T, E] in x.dtype, fp32 accumulation.

    With norm_w the router runs on RMSNorm(x) (and return_xn gives it back).
    """
    dev = _lib.require_device(x, router_w, norm_w)
    xt = _lib.half_code(x.dtype)
    if router_w.dtype != x.dtype or (norm_w is not None and norm_w.dtype != x.dtype):
        raise RuntimeError("router and norm weights must have the activation dtype")
    xf = x.reshape(-1, x.shape[-1]).contiguous()
    T, H = xf.shape
    E = router_w.shape[0]
    wr = router_w.contiguous()
    nw = None if norm_w is None else norm_w.contiguous()
    out = torch.empty(T, E, dtype=x.dtype, device=dev)
    # with a norm and T > 1 the library writes xn (its first pass) even if not returned
    xn = torch.empty_like(xf) if (nw is not None and (return_xn or T > 1)) else None
    _lib.check(_lib.lib().i4_router_logits(xf.data_ptr(), xt, T, H, wr.data_ptr(), E,
                                           _lib.ptr(nw), float(norm_eps), _lib.ptr(xn),
                                           out.data_ptr(), _lib.stream(dev)))
    if return_xn:
        return out, (xn if xn is not None else xf)
    return out


def route(logits: torch.Tensor, top_k: int, norm_topk_prob: bool = True,
          w_dtype: torch.dtype | None = None):
    """softmax (fp32) -> top-k -> renorm, from [T, E] logits.

    Returns (w, sel): w [T, top_k] in w_dtype (default logits.dtype, the
    reference's w.to(x.dtype)), sel [T, top_k] int32 in descending-weight
    order; exact ties go to the lower expert id.
    """
    dev = _lib.require_device(logits)
    lt = _lib.dtype_code(logits.dtype)
    lg = logits.reshape(-1, logits.shape[-1]).contiguous()
    T, E = lg.shape
    wd = w_dtype or logits.dtype
    sel = torch.empty(T, top_k, dtype=torch.int32, device=dev)
    w = torch.empty(T, top_k, dtype=wd, device=dev)
    _lib.check(_lib.lib().i4_route_topk(lg.data_ptr(), lt, T, E, top_k, int(norm_topk_prob),
                                        sel.data_ptr(), None, w.data_ptr(),
                                        _lib.dtype_code(wd), _lib.stream(dev)))
    return w, sel


def _decode_layout(*ws: QWeight) -> None:
    for w in ws:
        if w.layout not in ("ct", "tile"):
            raise ValueError(f"the MoE kernels read CT rows or tiles, got {w.layout!r}: "
                             "convert once with QWeight.to_ct() / to_tile()")


def _check_block_dtypes(x_dtype: torch.dtype, H: int, E: int, router_w: torch.Tensor | None,
                        norm_w: torch.Tensor | None) -> None:
    """The kernels read the router and norm weights in the activation dtype, as the
    reference's half-precision gate Linear does (F.linear raises on a mismatch)."""
    if router_w is not None:
        if router_w.dtype != x_dtype:
            raise RuntimeError(f"router weight is {router_w.dtype}, activations are {x_dtype}: "
                               "build the block in the activation dtype")
        if tuple(router_w.shape) != (E, H) or not router_w.is_contiguous():
            raise RuntimeError(f"router weight must be a contiguous [{E}, {H}] tensor, "
                               f"got {tuple(router_w.shape)}")
    if norm_w is not None:
        if norm_w.dtype != x_dtype:
            raise RuntimeError(f"norm weight is {norm_w.dtype}, activations are {x_dtype}")
        if norm_w.numel() != H or not norm_w.is_contiguous():
            raise RuntimeError(f"norm weight must hold {H} contiguous values")


def moe_weights_c(gate_up: QWeight, down: QWeight, router_w: torch.Tensor | None,
                  norm_w: torch.Tensor | None = None, norm_eps: float = 1e-6,
                  gate_up_tile: QWeight | None = None,
                  down_tile: QWeight | None = None) -> _lib.MoeWeightsC:
    """struct i4_moe_weights: decode weights (CT or tile) and optional tile copies (T > 1)."""
    _decode_layout(gate_up, down)
    if (gate_up_tile is None) != (down_tile is None):
        raise ValueError("give both tile copies or neither")
    mw = _lib.MoeWeightsC(gate_up=gate_up.c(), down=down.c(),
                          router_w=None if router_w is None else router_w.data_ptr(),
                          norm_w=None if norm_w is None else norm_w.data_ptr(),
                          norm_eps=float(norm_eps))
    if gate_up_tile is not None:
        if gate_up_tile.layout != "tile" or down_tile.layout != "tile":
            raise ValueError("the tile copies must be in the tile layout")
        mw.gate_up_tile, mw.down_tile = gate_up_tile.c(), down_tile.c()
    return mw


class Workspace:
    """Grow-only device scratch for the MoE entry points (one per module)."""

    def __init__(self) -> None:
        self.buf: torch.Tensor | None = None

    def get(self, nbytes: int, device: torch.device, zeroed: bool = False) -> torch.Tensor:
        """At least nbytes; zeroed: a new buffer is allocated as zeros."""
        if self.buf is None or self.buf.numel() < nbytes or self.buf.device != device:
            make = torch.zeros if zeroed else torch.empty
            self.buf = make(max(nbytes, 1), dtype=torch.uint8, device=device)
        return self.buf


def moe_forward(x: torch.Tensor, gate_up: QWeight, down: QWeight, top_k: int,
                router_w: torch.Tensor | None = None, logits: torch.Tensor | None = None,
                norm_topk_prob: bool = True, residual: torch.Tensor | None = None,
                return_routing: bool = False, workspace: Workspace | None = None,
                norm_w: torch.Tensor | None = None, norm_eps: float = 1e-6,
                gate_up_tile: QWeight | None = None, down_tile: QWeight | None = None,
                _bounded: tuple[int, int] | None = None):
    """One int4 MoE block: out = residual + sum_j w_j down_e(silu(gate_e xn) * up_e xn).

    xn = x, or RMSNorm(x) with weight norm_w (the decoder's post-attention norm).
    gate_up / down (CT or tile) serve one token; more tokens run on tiles: the
    tile copies, or gate_up / down themselves when they are tiles.
    """
    dev = _lib.require_device(x, gate_up.packed, down.packed, router_w, logits, residual, norm_w)
    xt = _lib.half_code(x.dtype)
    shape = x.shape
    xf = x.reshape(-1, shape[-1]).contiguous()
    T, H = xf.shape
    E, I = gate_up.E, down.K
    if router_w is None and logits is None:
        raise RuntimeError("need router_w or logits")
    _check_block_dtypes(x.dtype, H, E, router_w, norm_w)
    lg = None
    if router_w is None:
        lg = logits.reshape(T, E).to(x.dtype).contiguous()
    rs = None if residual is None else residual.reshape(T, H).to(x.dtype).contiguous()
    out = torch.empty(T, H, dtype=x.dtype, device=dev)
    sel = torch.empty(T, top_k, dtype=torch.int32, device=dev) if return_routing else None
    wts = torch.empty(T, top_k, dtype=torch.float32, device=dev) if return_routing else None
    lb = _lib.lib()
    nbytes = lb.i4_moe_workspace_bytes(T, H, I, E, top_k)
    ws = (workspace or Workspace()).get(nbytes, dev)
    mw = moe_weights_c(gate_up, down, router_w, norm_w, norm_eps, gate_up_tile, down_tile)
    if _bounded is not None:
        _lib.check(lb.i4_moe_forward_bounded(
            xf.data_ptr(), xt, T, ctypes.byref(mw), top_k, int(norm_topk_prob), _lib.ptr(lg),
            _lib.ptr(rs), out.data_ptr(), ws.data_ptr(), ws.numel(), int(_bounded[0]),
            int(_bounded[1]), _lib.stream(dev)))
        return out.view(shape)
    _lib.check(lb.i4_moe_forward(xf.data_ptr(), xt, T, ctypes.byref(mw), top_k,
                                 int(norm_topk_prob), _lib.ptr(lg), _lib.ptr(rs), out.data_ptr(),
                                 _lib.ptr(sel), _lib.ptr(wts), ws.data_ptr(), ws.numel(),
                                 _lib.stream(dev)))
    out = out.view(shape)
    if return_routing:
        return out, sel, wts
    return out


def moe_forward_bounded(x: torch.Tensor, gate_up: QWeight, down: QWeight, top_k: int,
                        max_polls: int, down_only: bool = False, rank_only: bool = False,
                        **kw) -> torch.Tensor:
    """moe_forward for 2..64 tokens with the bound of an in-launch wait given
    (i4_moe_forward_bounded): the grouped experts launch's, whose down workgroups
    down_only launches alone; or, with rank_only, the routing launch's, whose ranking waves
    it launches alone.  Either way every wait gives up (NaN out, I4_ERR_HANDOFF in the
    status word).  For testing the bounded waits from the host."""
    mode = 2 if rank_only else (1 if down_only else 0)
    return moe_forward(x, gate_up, down, top_k, _bounded=(max_polls, mode), **kw)


def moe_status(workspace: Workspace, T: int, H: int, I: int, E: int, top_k: int) -> int:
    """The status word the last i4_moe_forward / stack call with this workspace left
    (0, or the I4_ERR_HANDOFF code when a decode wait gave up); synchronises the device."""
    off = _lib.lib().i4_moe_status_offset(T, H, I, E, top_k)
    if workspace.buf is None or workspace.buf.numel() < off + 4:
        raise RuntimeError("the workspace has not served a call of these sizes")
    torch.cuda.synchronize(workspace.buf.device)
    return int(workspace.buf[off:off + 4].view(torch.int32).item())


def moe_down_wait(act: torch.Tensor, down: QWeight, logits: torch.Tensor, top_k: int,
                  norm_topk_prob: bool = True, residual: torch.Tensor | None = None,
                  status: torch.Tensor | None = None, max_polls: int = 1 << 20):
    """The down workgroups of the single-launch decode layer on their own (i4_moe_down_wait):
    rank `logits`, wait (at most max_polls polls) until no value of act [k, I] holds the
    pending pattern 0xFFFF, then out = residual + sum_j w_j down_{sel_j}(act_j) -> [H].
    Returns (out, status); status (int32 [1], device) receives the I4_ERR_HANDOFF code when
    a workgroup gave up (its rows are NaN) and is otherwise left as given (zeroed here
    when not given)."""
    _decode_layout(down)
    dev = _lib.require_device(act, down.packed, logits, residual, status)
    xt = _lib.half_code(act.dtype)
    lg = logits.reshape(-1).to(act.dtype).contiguous()
    rs = None if residual is None else residual.reshape(-1).to(act.dtype).contiguous()
    if status is None:
        status = torch.zeros(1, dtype=torch.int32, device=dev)
    elif status.dtype != torch.int32 or status.numel() < 1:
        raise RuntimeError("status is an int32 device tensor")
    out = torch.empty(down.N, dtype=act.dtype, device=dev)
    cw = down.c()
    _lib.check(_lib.lib().i4_moe_down_wait(act.contiguous().data_ptr(), xt, ctypes.byref(cw),
                                           lg.data_ptr(), lg.numel(), top_k,
                                           int(norm_topk_prob), _lib.ptr(rs), out.data_ptr(),
                                           status.data_ptr(), int(max_polls), _lib.stream(dev)))
    return out, status


def moe_forward_noalloc(x: torch.Tensor, gate_up: QWeight, down: QWeight, top_k: int,
                        router_w: torch.Tensor | None = None, logits: torch.Tensor | None = None,
                        norm_topk_prob: bool = True, residual: torch.Tensor | None = None,
                        norm_w: torch.Tensor | None = None, norm_eps: float = 1e-6,
                        gate_up_tile: QWeight | None = None, down_tile: QWeight | None = None,
                        out: torch.Tensor | None = None,
                        status: torch.Tensor | None = None) -> torch.Tensor:
    """moe_forward through i4_moe_forward_noalloc: the library's static per-GPU scratch
    replaces the workspace (no device allocation by the library; `out` may be given so that
    nothing is allocated here either).  Calls that overlap on one GPU race.  status (int32
    device tensor of one element, optional) receives the call's status word: 0, or the
    I4_ERR_HANDOFF code when a decode wait gave up."""
    dev = _lib.require_device(x, gate_up.packed, down.packed, router_w, logits, residual, norm_w,
                              out, status)
    if status is not None and (status.dtype != torch.int32 or status.numel() < 1):
        raise RuntimeError("status is an int32 device tensor")
    xt = _lib.half_code(x.dtype)
    xf = x.reshape(-1, x.shape[-1])
    if not xf.is_contiguous():
        raise RuntimeError("x must be contiguous")
    T, H = xf.shape
    E = gate_up.E
    if router_w is None and logits is None:
        raise RuntimeError("need router_w or logits")
    _check_block_dtypes(x.dtype, H, E, router_w, norm_w)
    for t, name in ((logits, "logits"), (residual, "residual")):
        if t is not None and (t.dtype != x.dtype or not t.is_contiguous()):
            raise RuntimeError(f"{name} must be contiguous in the activation dtype")
    if out is None:
        out = torch.empty(T, H, dtype=x.dtype, device=dev)
    elif out.dtype != x.dtype or out.numel() != T * H or not out.is_contiguous():
        raise RuntimeError("out must be a contiguous [T, H] tensor in the activation dtype")
    mw = moe_weights_c(gate_up, down, router_w if logits is None else None, norm_w, norm_eps,
                       gate_up_tile, down_tile)
    _lib.check(_lib.lib().i4_moe_forward_noalloc(xf.data_ptr(), xt, T, ctypes.byref(mw), top_k,
                                                 int(norm_topk_prob), _lib.ptr(logits),
                                                 _lib.ptr(residual), out.data_ptr(), None, None,
                                                 _lib.ptr(status), _lib.stream(dev)))
    return out.view(x.shape)


def moe_gate_up(x: torch.Tensor, gate_up: QWeight, sel: torch.Tensor) -> torch.Tensor:
    """Decode gate_up stage: act [k, I] = silu(gate_e x) * up_e x for e = sel (x is [H])."""
    _decode_layout(gate_up)
    dev = _lib.require_device(x, gate_up.packed, sel)
    xt = _lib.half_code(x.dtype)
    xc = x.reshape(-1).contiguous()
    s32 = sel.reshape(-1).to(torch.int32).contiguous()
    act = torch.empty(s32.numel(), gate_up.N // 2, dtype=x.dtype, device=dev)
    cw = gate_up.c()
    _lib.check(_lib.lib().i4_moe_gate_up(xc.data_ptr(), xt, ctypes.byref(cw), s32.data_ptr(),
                                         s32.numel(), act.data_ptr(), _lib.stream(dev)))
    return act


def moe_route_gate_up(x: torch.Tensor, gate_up: QWeight, logits: torch.Tensor, top_k: int,
                      norm_topk_prob: bool = True):
    """Decode routing + gate_up stage in one launch: (act [k, I], sel [k] int32, w [k] fp32)."""
    _decode_layout(gate_up)
    dev = _lib.require_device(x, gate_up.packed, logits)
    xt = _lib.half_code(x.dtype)
    xc = x.reshape(-1).contiguous()
    lg = logits.reshape(-1).to(x.dtype).contiguous()
    act = torch.empty(top_k, gate_up.N // 2, dtype=x.dtype, device=dev)
    sel = torch.empty(top_k, dtype=torch.int32, device=dev)
    w = torch.empty(top_k, dtype=torch.float32, device=dev)
    cw = gate_up.c()
    _lib.check(_lib.lib().i4_moe_route_gate_up(xc.data_ptr(), xt, ctypes.byref(cw), lg.data_ptr(),
                                               lg.numel(), top_k, int(norm_topk_prob),
                                               sel.data_ptr(), w.data_ptr(), act.data_ptr(),
                                               _lib.stream(dev)))
    return act, sel, w


def moe_down_combine(act: torch.Tensor, down: QWeight, sel: torch.Tensor, w: torch.Tensor,
                     residual: torch.Tensor | None = None) -> torch.Tensor:
    """Decode down stage: residual + sum_j w[j] down_{sel[j]}(act[j]) -> [H]."""
    _decode_layout(down)
    dev = _lib.require_device(act, down.packed, sel, w, residual)
    xt = _lib.half_code(act.dtype)
    s32 = sel.reshape(-1).to(torch.int32).contiguous()
    wf = w.reshape(-1).to(torch.float32).contiguous()
    rs = None if residual is None else residual.reshape(-1).to(act.dtype).contiguous()
    out = torch.empty(down.N, dtype=act.dtype, device=dev)
    cw = down.c()
    _lib.check(_lib.lib().i4_moe_down_combine(act.contiguous().data_ptr(), xt, ctypes.byref(cw),
                                              s32.data_ptr(), wf.data_ptr(), s32.numel(),
                                              _lib.ptr(rs), out.data_ptr(), _lib.stream(dev)))
    return out


def moe_stack(x: torch.Tensor, layers: list[tuple], top_k: int,
              norm_topk_prob: bool = True, workspace: Workspace | None = None) -> torch.Tensor:
    """h <- h + moe_l(norm_l(h)) over layers
    [(gate_up, down, router_w[, norm_w[, eps[, gate_up_tile, down_tile]]]), ...]."""
    dev = _lib.require_device(x)
    xt = _lib.half_code(x.dtype)
    shape = x.shape
    xf = x.reshape(-1, shape[-1]).contiguous()
    T, H = xf.shape
    gu0, dn0 = layers[0][0], layers[0][1]
    for layer in layers:
        if len(layer) < 3 or layer[2] is None:
            raise RuntimeError("every layer of the stack routes with its own router weight")
        _check_block_dtypes(x.dtype, H, layer[0].E, layer[2], layer[3] if len(layer) > 3 else None)
    arr = (_lib.MoeWeightsC * len(layers))(*[moe_weights_c(*layer) for layer in layers])
    lb = _lib.lib()
    nbytes = lb.i4_moe_stack_workspace_bytes(T, H, dn0.K, gu0.E, top_k)
    ws = (workspace or Workspace()).get(nbytes, dev)
    out = torch.empty_like(xf)
    _lib.check(lb.i4_moe_stack_forward(xf.data_ptr(), xt, T, arr, len(layers), top_k,
                                       int(norm_topk_prob), out.data_ptr(), ws.data_ptr(),
                                       ws.numel(), _lib.stream(dev)))
    return out.view(shape)


class StackLayerX:
    """The launches of one decode layer of the XCD-local stack path (i4_moe_route_sum,
    i4_moe_experts_x, i4_moe_sum) on one block, given as a moe_stack layer tuple.  The
    workspace is the block's T = 1 MoE workspace; slot outputs go to `ypart` [8, H]."""

    def __init__(self, layer: tuple, top_k: int, dtype: torch.dtype,
                 norm_topk_prob: bool = True, workspace: Workspace | None = None):
        self.mw = moe_weights_c(*layer)
        gu, dn = layer[0], layer[1]
        self.top_k, self.renorm, self.xt = top_k, int(norm_topk_prob), _lib.half_code(dtype)
        self.H = gu.K
        dev = gu.packed.device
        self.dev = dev
        nbytes = _lib.lib().i4_moe_workspace_bytes(1, gu.K, dn.K, gu.E, top_k)
        self.ws_holder = workspace or Workspace()
        self.ws = self.ws_holder.get(nbytes, dev)

    def route(self, res: torch.Tensor, ypart: torch.Tensor | None = None,
              h_out: torch.Tensor | None = None, reset_status: bool = False) -> None:
        _lib.check(_lib.lib().i4_moe_route_sum(
            res.data_ptr(), self.xt, _lib.ptr(ypart), ctypes.byref(self.mw), self.top_k,
            _lib.ptr(h_out), int(reset_status), self.ws.data_ptr(), self.ws.numel(),
            _lib.stream(self.dev)))

    def experts(self, h: torch.Tensor | None, ypart: torch.Tensor, max_polls: int = 1 << 20,
                down_only: bool = False) -> None:
        _lib.check(_lib.lib().i4_moe_experts_x(
            _lib.ptr(h), self.xt, ctypes.byref(self.mw), self.top_k, self.renorm,
            ypart.data_ptr(), int(max_polls), int(down_only), self.ws.data_ptr(),
            self.ws.numel(), _lib.stream(self.dev)))

    def sum(self, res: torch.Tensor, ypart: torch.Tensor, out: torch.Tensor) -> None:
        _lib.check(_lib.lib().i4_moe_sum(
            res.data_ptr(), self.xt, ypart.data_ptr(), ctypes.byref(self.mw), self.top_k,
            out.data_ptr(), self.ws.data_ptr(), self.ws.numel(), _lib.stream(self.dev)))


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Qwen3OmniMoeThinkerTextRMSNorm over the last dim (i4_rmsnorm), in x.dtype."""
    dev = _lib.require_device(x, weight)
    if weight.dtype != x.dtype:
        raise RuntimeError("the norm weight must have the activation dtype")
    xf = x.reshape(-1, x.shape[-1]).contiguous()
    out = torch.empty_like(xf)
    _lib.check(_lib.lib().i4_rmsnorm(xf.data_ptr(), _lib.half_code(x.dtype), xf.shape[0],
                                     xf.shape[1], weight.contiguous().data_ptr(), float(eps),
                                     out.data_ptr(), _lib.stream(dev)))
    return out.view(x.shape)


def attn_decode(qkv: torch.Tensor, n_heads: int, n_kv_heads: int, q_norm_w: torch.Tensor,
                k_norm_w: torch.Tensor, eps: float, inv_freq: torch.Tensor,
                pos: int | torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                workspace: Workspace | None = None) -> torch.Tensor:
    """Decode attention of one token (i4_attn_decode) between the q/k/v and o projections:
    qkv [n_heads + 2 n_kv_heads, head_dim] in, [n_heads * head_dim] out; appends k / v at
    row `pos` of the caches [n_kv_heads, max_len, head_dim] and attends rows [0, pos].
    inv_freq is the host fp32 table of the rotary embedding ([head_dim / 2]).  pos may be an
    int32 device tensor of one element (i4_attn_decode_at): the kernels read it, so a
    captured graph serves every position."""
    dev = _lib.require_device(qkv, q_norm_w, k_norm_w, k_cache, v_cache)
    pos_dev = None
    if isinstance(pos, torch.Tensor):
        if pos.device != dev or pos.dtype != torch.int32 or pos.numel() != 1:
            raise RuntimeError("a device position is one int32 on the tensors' device")
        pos_dev = pos
    xt = _lib.half_code(qkv.dtype)
    nkv, max_len, hd = k_cache.shape
    if k_cache.dtype != qkv.dtype or v_cache.shape != k_cache.shape or v_cache.dtype != qkv.dtype:
        raise RuntimeError("the caches must be [n_kv_heads, max_len, head_dim] in the activation dtype")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise RuntimeError("the caches must be contiguous")
    if qkv.numel() != (n_heads + 2 * n_kv_heads) * hd or nkv != n_kv_heads:
        raise RuntimeError("qkv / cache shapes do not match the head counts")
    tab = inv_freq.detach().to("cpu", torch.float32).contiguous()
    if tab.numel() != hd // 2:
        raise RuntimeError("inv_freq must hold head_dim / 2 values")
    lb = _lib.lib()
    nbytes = lb.i4_attn_decode_workspace_bytes(n_heads, hd, max_len)
    ws = (workspace or Workspace()).get(nbytes, dev)
    out = torch.empty(n_heads * hd, dtype=qkv.dtype, device=dev)
    args = (qkv.contiguous().data_ptr(), xt, n_heads, n_kv_heads, hd,
            q_norm_w.contiguous().data_ptr(), k_norm_w.contiguous().data_ptr(), float(eps),
            tab.data_ptr())
    tail = (k_cache.data_ptr(), v_cache.data_ptr(), max_len, out.data_ptr(), ws.data_ptr(),
            ws.numel(), _lib.stream(dev))
    if pos_dev is None:
        _lib.check(lb.i4_attn_decode(*args, int(pos), *tail))
    else:
        _lib.check(lb.i4_attn_decode_at(*args, pos_dev.data_ptr(), *tail))
    return out


def attn_decode_o(qkv: torch.Tensor, n_heads: int, n_kv_heads: int, q_norm_w: torch.Tensor,
                  k_norm_w: torch.Tensor, eps: float, inv_freq: torch.Tensor,
                  pos: int | torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  o_w: QWeight, residual: torch.Tensor | None = None,
                  workspace: Workspace | None = None) -> torch.Tensor:
    """attn_decode followed by the o projection and the residual add (i4_attn_decode_o):
    returns residual + o_w attn as [o_w.N] in the activation dtype, equal bit for bit to
    linear(attn_decode(...), o_w, bias=residual), in one launch fewer (the o_proj
    workgroups take the merged heads over inside the merge launch).  o_w is a CT weight."""
    dev = _lib.require_device(qkv, q_norm_w, k_norm_w, k_cache, v_cache, o_w.packed, residual)
    pos_dev = None
    if isinstance(pos, torch.Tensor):
        if pos.device != dev or pos.dtype != torch.int32 or pos.numel() != 1:
            raise RuntimeError("a device position is one int32 on the tensors' device")
        pos_dev = pos
    xt = _lib.half_code(qkv.dtype)
    nkv, max_len, hd = k_cache.shape
    if k_cache.dtype != qkv.dtype or v_cache.shape != k_cache.shape or v_cache.dtype != qkv.dtype:
        raise RuntimeError("the caches must be [n_kv_heads, max_len, head_dim] in the activation dtype")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise RuntimeError("the caches must be contiguous")
    if qkv.numel() != (n_heads + 2 * n_kv_heads) * hd or nkv != n_kv_heads:
        raise RuntimeError("qkv / cache shapes do not match the head counts")
    res = None
    if residual is not None:
        if residual.dtype != qkv.dtype or residual.numel() != o_w.N:
            raise RuntimeError("the residual must be [o_w.N] in the activation dtype")
        res = residual.contiguous()
    tab = inv_freq.detach().to("cpu", torch.float32).contiguous()
    if tab.numel() != hd // 2:
        raise RuntimeError("inv_freq must hold head_dim / 2 values")
    lb = _lib.lib()
    ws = (workspace or Workspace()).get(lb.i4_attn_decode_o_workspace_bytes(n_heads, hd, max_len),
                                        dev)
    y = torch.empty(o_w.N, dtype=qkv.dtype, device=dev)
    cw = o_w.c()
    _lib.check(lb.i4_attn_decode_o(
        qkv.contiguous().data_ptr(), xt, n_heads, n_kv_heads, hd,
        q_norm_w.contiguous().data_ptr(), k_norm_w.contiguous().data_ptr(), float(eps),
        tab.data_ptr(), None if pos_dev is None else pos_dev.data_ptr(),
        0 if pos_dev is not None else int(pos), k_cache.data_ptr(), v_cache.data_ptr(), max_len,
        ctypes.byref(cw), _lib.ptr(res), y.data_ptr(), ws.data_ptr(), ws.numel(),
        _lib.stream(dev)))
    return y


def attn_decode_qkv_o(h: torch.Tensor, in_norm_w: torch.Tensor, eps: float, qkv_w: QWeight,
                      n_heads: int, n_kv_heads: int, q_norm_w: torch.Tensor,
                      k_norm_w: torch.Tensor, inv_freq: torch.Tensor, pos: int | torch.Tensor,
                      k_cache: torch.Tensor, v_cache: torch.Tensor, o_w: QWeight,
                      workspace: Workspace | None = None) -> torch.Tensor:
    """The attention half of a decoder layer from its input row (i4_attn_decode_qkv_o):
    h + o_w attn(qkv_w RMSNorm(h)), equal bit for bit to rmsnorm_linear followed by
    attn_decode_o(residual=h).  qkv_w and o_w are CT weights; h is [..., H] holding one
    token.  Where the q|k|v GEMV shape allows, its rows are computed inside the attention
    chunk launch (two launches in all)."""
    dev = _lib.require_device(h, in_norm_w, q_norm_w, k_norm_w, k_cache, v_cache, qkv_w.packed,
                              o_w.packed)
    if h.numel() != h.shape[-1]:
        raise RuntimeError("attn_decode_qkv_o takes one token")
    pos_dev = None
    if isinstance(pos, torch.Tensor):
        if pos.device != dev or pos.dtype != torch.int32 or pos.numel() != 1:
            raise RuntimeError("a device position is one int32 on the tensors' device")
        pos_dev = pos
    xt = _lib.half_code(h.dtype)
    for t, name in ((in_norm_w, "input norm"), (q_norm_w, "q norm"), (k_norm_w, "k norm")):
        if t.dtype != h.dtype:
            raise RuntimeError(f"the {name} weight must have the activation dtype")
    nkv, max_len, hd = k_cache.shape
    if k_cache.dtype != h.dtype or v_cache.shape != k_cache.shape or v_cache.dtype != h.dtype:
        raise RuntimeError("the caches must be [n_kv_heads, max_len, head_dim] in the activation dtype")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()) or nkv != n_kv_heads:
        raise RuntimeError("the caches must be contiguous [n_kv_heads, max_len, head_dim]")
    tab = inv_freq.detach().to("cpu", torch.float32).contiguous()
    if tab.numel() != hd // 2:
        raise RuntimeError("inv_freq must hold head_dim / 2 values")
    hf = h.reshape(-1).contiguous()
    y = torch.empty_like(hf)
    lb = _lib.lib()
    nbytes = lb.i4_attn_decode_qkv_o_workspace_bytes(n_heads, n_kv_heads, hd, max_len)
    # zero-filled when allocated: the q|k|v hand-over tags are odd, so no word of a new
    # buffer can pass for a finished one
    ws = (workspace or Workspace()).get(nbytes, dev, zeroed=True)
    qw, ow = qkv_w.c(), o_w.c()
    _lib.check(lb.i4_attn_decode_qkv_o(
        hf.data_ptr(), xt, in_norm_w.contiguous().data_ptr(), float(eps), ctypes.byref(qw),
        n_heads, n_kv_heads, hd, q_norm_w.contiguous().data_ptr(),
        k_norm_w.contiguous().data_ptr(), tab.data_ptr(),
        None if pos_dev is None else pos_dev.data_ptr(), 0 if pos_dev is not None else int(pos),
        k_cache.data_ptr(), v_cache.data_ptr(), max_len, ctypes.byref(ow), y.data_ptr(),
        ws.data_ptr(), ws.numel(), _lib.stream(dev)))
    return y.view(h.shape)


def attn_status(workspace: Workspace, n_heads: int, head_dim: int, max_len: int) -> int:
    """The status word the last attn_decode_o call with this workspace left (0, or the
    I4_ERR_HANDOFF code when an o_proj wait gave up); synchronises the device."""
    off = _lib.lib().i4_attn_decode_o_status_offset(n_heads, head_dim, max_len)
    if workspace.buf is None or workspace.buf.numel() < off + 4:
        raise RuntimeError("the workspace has not served a call of these sizes")
    torch.cuda.synchronize(workspace.buf.device)
    return int(workspace.buf[off:off + 4].view(torch.int32).item())


def thinker_layer_fits(n_heads: int, n_kv_heads: int, head_dim: int, max_len: int, H: int,
                      I: int, E: int, top_k: int) -> bool:
    """Whether i4_thinker_layer_decode takes a layer of these sizes."""
    return _lib.lib().i4_thinker_layer_workspace_bytes(n_heads, n_kv_heads, head_dim, max_len,
                                                       H, I, E, top_k) > 0


def thinker_layer_decode(h: torch.Tensor, in_norm_w: torch.Tensor, eps: float, qkv_w: QWeight,
                         n_heads: int, n_kv_heads: int, q_norm_w: torch.Tensor,
                         k_norm_w: torch.Tensor, inv_freq: torch.Tensor, pos: int | torch.Tensor,
                         k_cache: torch.Tensor, v_cache: torch.Tensor, o_w: QWeight,
                         gate_up: QWeight, down: QWeight, top_k: int, router_w: torch.Tensor,
                         norm_w: torch.Tensor, norm_eps: float, norm_topk_prob: bool = True,
                         workspace: Workspace | None = None) -> torch.Tensor:
    """One decode token through a Thinker decoder layer (i4_thinker_layer_decode):
    h2 = h + o_proj(attention(RMSNorm(h))), then h2 + MoE(RMSNorm(h2)), in three launches
    (the q|k|v GEMV inside the attention chunk launch, the MoE router in the o_proj
    launch behind the workgroups producing h2, the experts).
    Equal bit for bit to rmsnorm_linear + attn_decode_o + moe_forward(residual=h2).
    qkv_w, o_w and the experts are CT weights; h is [..., H] holding one token."""
    dev = _lib.require_device(h, in_norm_w, q_norm_w, k_norm_w, k_cache, v_cache, o_w.packed,
                              gate_up.packed, down.packed, router_w, norm_w)
    if h.numel() != h.shape[-1]:
        raise RuntimeError("thinker_layer_decode takes one token")
    pos_dev = None
    if isinstance(pos, torch.Tensor):
        if pos.device != dev or pos.dtype != torch.int32 or pos.numel() != 1:
            raise RuntimeError("a device position is one int32 on the tensors' device")
        pos_dev = pos
    xt = _lib.half_code(h.dtype)
    H = h.shape[-1]
    E, I = gate_up.E, down.K
    _check_block_dtypes(h.dtype, H, E, router_w, norm_w)
    for t, name in ((in_norm_w, "input norm"), (q_norm_w, "q norm"), (k_norm_w, "k norm")):
        if t.dtype != h.dtype:
            raise RuntimeError(f"the {name} weight must have the activation dtype")
    nkv, max_len, hd = k_cache.shape
    if k_cache.dtype != h.dtype or v_cache.shape != k_cache.shape or v_cache.dtype != h.dtype:
        raise RuntimeError("the caches must be [n_kv_heads, max_len, head_dim] in the activation dtype")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()) or nkv != n_kv_heads:
        raise RuntimeError("the caches must be contiguous [n_kv_heads, max_len, head_dim]")
    tab = inv_freq.detach().to("cpu", torch.float32).contiguous()
    if tab.numel() != hd // 2:
        raise RuntimeError("inv_freq must hold head_dim / 2 values")
    hf = h.reshape(-1).contiguous()
    out = torch.empty_like(hf)
    lb = _lib.lib()
    nbytes = lb.i4_thinker_layer_workspace_bytes(n_heads, n_kv_heads, hd, max_len, H, I, E, top_k)
    if nbytes == 0:
        raise RuntimeError("unsupported Thinker layer shape")
    ws = (workspace or Workspace()).get(nbytes, dev, zeroed=True)  # see attn_decode_qkv_o
    qw, ow = qkv_w.c(), o_w.c()
    mw = moe_weights_c(gate_up, down, router_w, norm_w, norm_eps)
    _lib.check(lb.i4_thinker_layer_decode(
        hf.data_ptr(), xt, in_norm_w.contiguous().data_ptr(), float(eps), ctypes.byref(qw),
        n_heads, n_kv_heads, hd, q_norm_w.contiguous().data_ptr(),
        k_norm_w.contiguous().data_ptr(), tab.data_ptr(),
        None if pos_dev is None else pos_dev.data_ptr(), 0 if pos_dev is not None else int(pos),
        k_cache.data_ptr(), v_cache.data_ptr(), max_len, ctypes.byref(ow), ctypes.byref(mw),
        top_k, int(norm_topk_prob), out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream(dev)))
    return out.view(h.shape)


_WEIGHTS_GEN = [0]


def weights_changed() -> None:
    """Called when a tensor attribute of a decoder module is assigned: structs holding raw
    addresses of the old tensors are rebuilt before their next use."""
    _WEIGHTS_GEN[0] += 1


def weights_generation() -> int:
    return _WEIGHTS_GEN[0]


def thinker_layer_c(attn, moe) -> _lib.ThinkerLayerC:
    """struct i4_thinker_layer of a ThinkerAttention and its FusedPackedMoE (the struct
    holds raw pointers: the modules' tensors must stay where they are while it is used)."""
    return _lib.ThinkerLayerC(
        in_norm_w=attn.input_norm_w.data_ptr(), q_norm_w=attn.q_norm_w.data_ptr(),
        k_norm_w=attn.k_norm_w.data_ptr(), k_cache=attn.k_cache.data_ptr(),
        v_cache=attn.v_cache.data_ptr(), eps=float(attn.eps), qkv=attn.qkv.lin.w.c(),
        o=attn.o_proj.w.c(),
        moe=moe_weights_c(moe.gate_up, moe.down, moe.router_w, moe.norm_weight, moe.norm_eps))


def thinker_decode_step(h: torch.Tensor, layers_c, n_layers: int, n_heads: int, n_kv_heads: int,
                        head_dim: int, inv_freq: torch.Tensor, pos: int | torch.Tensor,
                        max_len: int, H: int, I: int, E: int, top_k: int,
                        norm_topk_prob: bool = True,
                        workspace: Workspace | None = None) -> torch.Tensor:
    """One decode token through n_layers Thinker decoder layers (i4_thinker_decode_step,
    one library call): layers_c is a ctypes array of thinker_layer_c structs.  Equal bit
    for bit to thinker_layer_decode layer by layer."""
    dev = _lib.require_device(h)
    if h.numel() != H:
        raise RuntimeError(f"thinker_decode_step takes one token of {H} values")
    pos_dev = None
    if isinstance(pos, torch.Tensor):
        if pos.device != dev or pos.dtype != torch.int32 or pos.numel() != 1:
            raise RuntimeError("a device position is one int32 on the tensors' device")
        pos_dev = pos
    tab = inv_freq.detach().to("cpu", torch.float32).contiguous()
    if tab.numel() != head_dim // 2:
        raise RuntimeError("inv_freq must hold head_dim / 2 values")
    hf = h.reshape(-1).contiguous()
    out = torch.empty_like(hf)
    lb = _lib.lib()
    nbytes = lb.i4_thinker_decode_step_workspace_bytes(n_heads, n_kv_heads, head_dim, max_len,
                                                       H, I, E, top_k)
    if nbytes == 0:
        raise RuntimeError("unsupported Thinker layer shape")
    ws = (workspace or Workspace()).get(nbytes, dev, zeroed=True)  # see attn_decode_qkv_o
    _lib.check(lb.i4_thinker_decode_step(
        hf.data_ptr(), _lib.half_code(h.dtype), layers_c, n_layers, n_heads, n_kv_heads,
        head_dim, tab.data_ptr(), None if pos_dev is None else pos_dev.data_ptr(),
        0 if pos_dev is not None else int(pos), max_len, top_k, int(norm_topk_prob),
        out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream(dev)))
    return out.view(h.shape)


def rmsnorm_linear(x: torch.Tensor, norm_w: torch.Tensor, eps: float, w: QWeight,
                   bias: torch.Tensor | None = None, out_dtype: torch.dtype | None = None):
    """y = RMSNorm(x) W^T (+ bias) in one launch (i4_rmsnorm_linear; CT weight, K <= 4096),
    equal bit for bit to linear(rmsnorm(x, norm_w, eps), w, bias)."""
    dev = _lib.require_device(x, norm_w, w.packed, bias)
    if norm_w.dtype != x.dtype:
        raise RuntimeError("the norm weight must have the activation dtype")
    flat = x.reshape(-1, w.K).contiguous()
    M = flat.shape[0]
    od = out_dtype or x.dtype
    y = torch.empty(M, w.N, dtype=od, device=dev)
    b = None if bias is None else bias.to(od).contiguous()
    cw = w.c()
    _lib.check(_lib.lib().i4_rmsnorm_linear(flat.data_ptr(), _lib.half_code(x.dtype), M,
                                            norm_w.contiguous().data_ptr(), float(eps),
                                            ctypes.byref(cw), _lib.ptr(b), y.data_ptr(),
                                            _lib.dtype_code(od), _lib.stream(dev)))
    return y.view(*x.shape[:-1], w.N)


def dweight_c(data: torch.Tensor, scale: torch.Tensor | None = None) -> _lib.DWeightC:
    """struct i4_dweight of a stacked weight [E, N, K] (or one matrix [N, K]):
    16-bit values, or int8 with one scale per output row ([E, N] or [E, N, 1])."""
    if data.dim() == 2:
        data = data.unsqueeze(0)
    if data.dim() != 3 or not data.is_contiguous():
        raise ValueError("a stacked weight is a contiguous [E, N, K] tensor")
    E, N, K = data.shape
    if scale is None:
        if data.dtype not in (torch.float16, torch.bfloat16):
            raise ValueError(f"16-bit weights expected, got {data.dtype} (int8 needs a scale)")
    else:
        if data.dtype != torch.int8:
            raise ValueError(f"scaled weights are int8, got {data.dtype}")
        if scale.numel() != E * N or not scale.is_contiguous():
            raise ValueError("one contiguous scale per output row ([E, N]) expected")
    return _lib.DWeightC(data=data.data_ptr(), scale=_lib.ptr(scale), E=E, N=N, K=K)


def dmoe_workspace_bytes(T: int, E: int, top_k: int, I: int, Is: int) -> int:
    return _lib.lib().i4_dmoe_workspace_bytes(T, E, top_k, I, Is)


def _dmoe_weights(dtype, gate_up, down, rw, gate_up_scale, down_scale, shared_gate_up,
                  shared_down, shared_gate_w, shared_gate_up_scale, shared_down_scale):
    """struct i4_dmoe_weights, and the converted tensors it points into (kept alive by
    the caller until the call is queued)."""
    sgw = None if shared_gate_w is None else shared_gate_w.reshape(-1).to(dtype).contiguous()
    dw = _lib.DmoeWeightsC(gate_up=dweight_c(gate_up, gate_up_scale),
                           down=dweight_c(down, down_scale), router_w=_lib.ptr(rw),
                           shared_gate_w=_lib.ptr(sgw))
    if shared_gate_up is not None:
        dw.shared_gate_up = dweight_c(shared_gate_up, shared_gate_up_scale)
        dw.shared_down = dweight_c(shared_down, shared_down_scale)
    return dw, (rw, sgw)


def dmoe_status(workspace: Workspace, T: int, E: int, top_k: int, I: int, Is: int) -> int:
    """The status word the last dmoe_forward call with this workspace left (0, or the
    I4_ERR_HANDOFF code when a down workgroup of the single-launch decode block gave up
    waiting for its activations); synchronises the device."""
    off = _lib.lib().i4_dmoe_status_offset(T, E, top_k, I, Is)
    if workspace.buf is None or workspace.buf.numel() < off + 4:
        raise RuntimeError("the workspace has not served a call of these sizes")
    torch.cuda.synchronize(workspace.buf.device)
    return int(workspace.buf[off:off + 4].view(torch.int32).item())


def dmoe_down_wait(x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor, top_k: int,
                   logits: torch.Tensor, workspace: Workspace, norm_topk_prob: bool = True,
                   gate_up_scale: torch.Tensor | None = None,
                   down_scale: torch.Tensor | None = None,
                   shared_gate_up: torch.Tensor | None = None,
                   shared_down: torch.Tensor | None = None,
                   shared_gate_w: torch.Tensor | None = None,
                   shared_gate_up_scale: torch.Tensor | None = None,
                   shared_down_scale: torch.Tensor | None = None,
                   residual: torch.Tensor | None = None, max_polls: int = 1 << 20):
    """The down workgroups of dmoe_forward's single-launch decode block on their own
    (i4_dmoe_down_wait), for one token: they rank `logits`, poll the workspace's
    activations as they are (at most max_polls times) and compute the block's output [H];
    a workgroup that gives up writes NaN and leaves I4_ERR_HANDOFF in the status word
    (dmoe_status)."""
    dev = _lib.require_device(x, gate_up, down, logits, shared_gate_up, shared_down,
                              shared_gate_w, residual)
    xt = _lib.half_code(x.dtype)
    xf = x.reshape(-1).contiguous()
    H = xf.numel()
    E, I = gate_up.shape[0], gate_up.shape[1] // 2
    Is = 0 if shared_gate_up is None else shared_gate_up.shape[-2] // 2
    lg = logits.reshape(E).to(x.dtype).contiguous()
    rs = None if residual is None else residual.reshape(H).to(x.dtype).contiguous()
    out = torch.empty(H, dtype=x.dtype, device=dev)
    dw, keep = _dmoe_weights(x.dtype, gate_up, down, None, gate_up_scale, down_scale,
                             shared_gate_up, shared_down, shared_gate_w, shared_gate_up_scale,
                             shared_down_scale)
    lb = _lib.lib()
    ws = workspace.get(lb.i4_dmoe_workspace_bytes(1, E, top_k, I, Is), dev)
    _lib.check(lb.i4_dmoe_down_wait(xf.data_ptr(), xt, ctypes.byref(dw), top_k,
                                    int(norm_topk_prob), lg.data_ptr(), _lib.ptr(rs),
                                    out.data_ptr(), ws.data_ptr(), ws.numel(), int(max_polls),
                                    _lib.stream(dev)))
    del keep
    return out


def dmoe_forward(x: torch.Tensor, gate_up: torch.Tensor, down: torch.Tensor, top_k: int,
                 router_w: torch.Tensor | None = None, logits: torch.Tensor | None = None,
                 norm_topk_prob: bool = True, gate_up_scale: torch.Tensor | None = None,
                 down_scale: torch.Tensor | None = None,
                 shared_gate_up: torch.Tensor | None = None,
                 shared_down: torch.Tensor | None = None,
                 shared_gate_w: torch.Tensor | None = None,
                 shared_gate_up_scale: torch.Tensor | None = None,
                 shared_down_scale: torch.Tensor | None = None,
                 residual: torch.Tensor | None = None, return_routing: bool = False,
                 workspace: Workspace | None = None):
    """MoE block on 16-bit / int8 experts with an optional gated shared expert
    (FusedMoE.forward, src/duplex/streaming/fused_moe.py:99-141):
      out = residual + sum_j w_j down_e(silu(gate_e x) * up_e x)
            + sigmoid(shared_gate_w . x) * down_s(silu(gate_s x) * up_s x)
    gate_up [E, 2I, H] (gate rows first), down [E, H, I]; int8 weights come with
    per-output-row scales in the activation dtype.  Three launches (router
    logits, gate_up + SiLU + routing, down + combine); one token with router_w and 16-bit
    experts runs in two (router logits; gate_up and down in one launch, the down
    workgroups waiting for the activations: dmoe_status reports a wait that gave up)."""
    dev = _lib.require_device(x, gate_up, down, router_w, logits, shared_gate_up, shared_down,
                              shared_gate_w, residual)
    xt = _lib.half_code(x.dtype)
    for s in (gate_up_scale, down_scale, shared_gate_up_scale, shared_down_scale):
        if s is not None and s.dtype != x.dtype:
            raise ValueError(f"int8 scales must be in the activation dtype {x.dtype}, got {s.dtype}")
    for w in (gate_up, down, shared_gate_up, shared_down):
        if w is not None and w.dtype != torch.int8 and w.dtype != x.dtype:
            raise ValueError(f"16-bit weights must be in the activation dtype {x.dtype}")
    if router_w is None and logits is None:
        raise RuntimeError("need router_w or logits")
    if (shared_gate_up is None) != (shared_down is None):
        raise ValueError("give the shared expert's gate|up and down together")
    shape = x.shape
    xf = x.reshape(-1, shape[-1]).contiguous()
    T, H = xf.shape
    E, I = gate_up.shape[0], gate_up.shape[1] // 2
    Is = 0 if shared_gate_up is None else shared_gate_up.shape[-2] // 2
    rw = None if router_w is None else router_w.to(x.dtype).contiguous()
    lg = None if router_w is not None else logits.reshape(T, E).to(x.dtype).contiguous()
    rs = None if residual is None else residual.reshape(T, H).to(x.dtype).contiguous()
    out = torch.empty(T, H, dtype=x.dtype, device=dev)
    sel = torch.empty(T, top_k, dtype=torch.int32, device=dev) if return_routing else None
    wts = torch.empty(T, top_k, dtype=torch.float32, device=dev) if return_routing else None
    dw, keep = _dmoe_weights(x.dtype, gate_up, down, rw, gate_up_scale, down_scale,
                             shared_gate_up, shared_down, shared_gate_w, shared_gate_up_scale,
                             shared_down_scale)
    lb = _lib.lib()
    ws = (workspace or Workspace()).get(lb.i4_dmoe_workspace_bytes(T, E, top_k, I, Is), dev)
    _lib.check(lb.i4_dmoe_forward(xf.data_ptr(), xt, T, ctypes.byref(dw), top_k,
                                  int(norm_topk_prob), _lib.ptr(lg), _lib.ptr(rs),
                                  out.data_ptr(), _lib.ptr(sel), _lib.ptr(wts), ws.data_ptr(),
                                  ws.numel(), _lib.stream(dev)))
    del keep
    out = out.view(shape)
    if return_routing:
        return out, sel, wts
    return out

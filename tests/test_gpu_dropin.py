"""The drop-in boundary at the workload's full size, through the C ABI:

  - fuse_packed_moe_blocks / FusedPackedMoE(block) on a packed SparseMoeBlock stand-in
    (src/duplex/streaming/fused_packed_moe.py:86-122,278-319) at 128 experts x 2048 x 768,
    T = 1 and T = 32, bf16 and fp16, against the oracle;
  - routing end to end on the decode (M = 1) and M = 32 workloads: the oracle ranks its own
    fp16 logits of the same inputs (fused_packed_moe.py:195-199);
  - the 24-layer Thinker[0:24] MoE stack (clock.py:168-171) at 128 experts: bit-equal to the
    module loop, its first and last layers against the oracle on the GPU's own inputs;
  - the bounded wait of the single-launch decode layer, made to give up from the host.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import i4ref
from tests import _gen
from tests.test_gpu_parity import (_awq_moe, check_moe_term, f_, half_name, host, make_x, t_)

pytestmark = pytest.mark.gpu
E, H, I, K8 = 128, 2048, 768, 8


# ---------------------------------------------------------------- packed block stand-in
class _PackedLinear(nn.Module):
    """A compressed-tensors pack-quantized Linear as the reference's loader leaves it
    (weight_packed [N, K/8] int32, weight_scale [N, K/32], weight_shape [N, K])."""

    def __init__(self, packed, scale, N, K):
        super().__init__()
        self.register_buffer("weight_packed", packed)
        self.register_buffer("weight_scale", scale)
        self.register_buffer("weight_shape", torch.tensor([N, K]))


class _Expert(nn.Module):
    def __init__(self, g, u, d):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = g, u, d


class StandInSparseMoeBlock(nn.Module):
    """The attributes fuse_packed_moe_blocks reads from transformers' Thinker block:
    experts (ModuleList of packed gate/up/down), gate (Linear H -> E), top_k, norm_topk_prob."""

    def __init__(self, rng, E, H, I, G=32):
        super().__init__()
        gp, gs, _ = _gen.ct_weight(rng, E, I, H, G, sdt="bf16")
        up, us, _ = _gen.ct_weight(rng, E, I, H, G, sdt="bf16")
        dp, ds, _ = _gen.ct_weight(rng, E, H, I, G, sdt="bf16")
        self.np = (gp, gs, up, us, dp, ds)
        bf = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)  # checkpoint dtype
        self.experts = nn.ModuleList(
            _Expert(_PackedLinear(torch.from_numpy(gp[e]), bf(gs[e]), I, H),
                    _PackedLinear(torch.from_numpy(up[e]), bf(us[e]), I, H),
                    _PackedLinear(torch.from_numpy(dp[e]), bf(ds[e]), H, I)) for e in range(E))
        self.gate = nn.Linear(H, E, bias=False)
        with torch.no_grad():
            self.gate.weight.copy_(torch.from_numpy(rng.standard_normal((E, H)) * 0.02))
        self.top_k, self.norm_topk_prob = K8, True
        self.G = G

    def oracle_weights(self):
        gp, gs, up, us, dp, ds = self.np
        G = self.G
        dgu = lambda e: np.concatenate([i4ref.ct_dequant(gp[e], f_(gs[e]), H, G),
                                        i4ref.ct_dequant(up[e], f_(us[e]), H, G)], axis=0)
        ddn = lambda e: i4ref.ct_dequant(dp[e], f_(ds[e]), I, G)
        return dgu, ddn


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fuse_packed_moe_blocks_replaces_the_block(pkg, dev, dtype):
    """The reference's installer on a model holding a packed block: the block is replaced by a
    FusedPackedMoE that stacks its experts (gate | up concatenated, scales in `dtype`) and whose
    forward matches the oracle at T = 1 (single-launch decode) and T = 32 (grouped MFMA)."""
    packed_block = StandInSparseMoeBlock(np.random.default_rng(101), E, H, I)
    model = nn.Module()
    model.layer = nn.Module()
    model.layer.mlp = packed_block
    model.layer.other = nn.Linear(4, 4)
    n = pkg.fuse_packed_moe_blocks(model, dtype=dtype, device=dev, verbose=False)
    assert n == 1 and isinstance(model.layer.mlp, pkg.FusedPackedMoE)
    assert isinstance(model.layer.other, nn.Linear)
    m = model.layer.mlp
    assert (m.num_experts, m.hidden, m.inter, m.top_k) == (E, H, I, K8)
    assert m.gate_up.layout == "ct" and m.gate_up_tile is not None
    assert m.router_w.dtype == dtype and m.gate_up.scale.dtype == dtype
    # the router stays the block's `gate` Linear (fused_packed_moe.py:112), holding the
    # router weight the library reads; a new gate weight changes the routing
    assert isinstance(m.gate, nn.Linear) and m.gate.weight is m.router_w
    assert torch.equal(m.gate.weight.float().cpu(),
                       packed_block.gate.weight.detach().to(dtype).float())
    xg = t_(make_x(np.random.default_rng(103), (1, H), "bf16" if dtype == torch.bfloat16
                   else "f16"), dev)
    lg_lib = pkg.router_logits(xg, m.router_w).float()
    lg_torch = m.gate(xg.float().to(dtype)).float()
    assert torch.allclose(lg_lib, lg_torch, rtol=2e-2, atol=2e-2)
    saved = m.gate.weight
    sel_before = m.route(xg)[1]
    m.gate.weight = nn.Parameter(torch.flip(saved, dims=[0]), requires_grad=False)
    # expert e's row is now E-1-e's: the same selection (equal logits, which bf16 makes
    # common, may then rank in another order: ties go to the lower id)
    assert torch.equal(m.route(xg)[1].sort().values, (E - 1 - sel_before).sort().values)
    m.gate.weight = saved
    # the stacked gate | up rows are the experts' own words, gate rows first
    gp, _, up, _, dp, _ = packed_block.np
    for e in (0, 77, 127):
        assert np.array_equal(m.gate_up.packed[e, :I].cpu().numpy(), gp[e])
        assert np.array_equal(m.gate_up.packed[e, I:].cpu().numpy(), up[e])
        assert np.array_equal(m.down.packed[e].cpu().numpy(), dp[e])
    dgu, ddn = packed_block.oracle_weights()
    xdt = "bf16" if dtype == torch.bfloat16 else "f16"
    rng = np.random.default_rng(102)
    for T in (1, 32):
        x = t_(make_x(rng, (T, H), xdt), dev)
        out = m(x)
        w, sel = m.route(x)
        lg = host(pkg.router_logits(x, m.router_w))
        sel_ref, w_ref = i4ref.route(lg, K8)
        np.testing.assert_array_equal(sel.cpu().numpy(), sel_ref)
        hn = half_name(xdt)
        moe_ref = i4ref.moe_layer_grouped(host(x), sel_ref, w_ref, dgu, ddn, hn, y_dtype=hn)
        got = host(out)
        assert np.all(np.isfinite(got)) and got.shape == (T, H)
        assert i4ref.rel_err(got, moe_ref) <= 2e-2
        check_moe_term(got, moe_ref, None, hn)
    # the reference's F.linear refuses activations of another dtype; so does the block
    other = torch.float16 if dtype == torch.bfloat16 else torch.bfloat16
    with pytest.raises(RuntimeError, match="activation"):
        m(torch.zeros(1, H, dtype=other, device=dev))


# ---------------------------------------------------------------- routing end to end
def _ulp16(v):
    return 2.0 ** (np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -14))) - 10)


def test_routing_end_to_end_on_the_workload_inputs(pkg, dev):
    """The GPU's experts for the M = 1 and M = 32 workloads against the oracle's top-8 of its
    OWN fp16 logits (the exact product of the same fp16 x and router weight, rounded once):
    no mismatch on any row whose 8th / 9th logits are more than 1 ulp apart (the GPU's fp32
    accumulation may round a logit to its neighbour, so closer rows may legitimately differ);
    the count and rate over all rows are printed, and the rate is at most 5 %."""
    rng = np.random.default_rng(103)
    moe, _, _, wr = _awq_moe(pkg, dev, rng)
    rows = []
    for T, reps in ((1, 96), (32, 4)):
        for _ in range(reps):
            x = make_x(rng, (T, H), "f16")
            _, sel, _ = pkg.moe_forward(t_(x, dev), moe.gate_up, moe.down, K8,
                                        router_w=moe.router_w, return_routing=True,
                                        gate_up_tile=moe.gate_up_tile, down_tile=moe.down_tile)
            lg = i4ref.round_half(f_(x) @ f_(wr).T, "f16")
            rows += [(T, lg[t], sel.cpu().numpy()[t]) for t in range(T)]
    clear = mismatch = clear_mismatch = 0
    for T, lg, got in rows:
        ref = i4ref.topk_sel(lg[None], K8)[0]
        s = np.sort(lg)[::-1]
        is_clear = s[K8 - 1] - s[K8] > _ulp16(s[K8 - 1])
        bad = not np.array_equal(got, ref)
        clear += is_clear
        mismatch += bad
        clear_mismatch += bad and is_clear
    print(f"\nrouting end to end: {len(rows)} rows, {mismatch} differ from the oracle's own "
          f"logits ({mismatch / len(rows):.2%}); {clear} rows with a > 1 ulp top-8 margin, "
          f"{clear_mismatch} of them differ")
    assert clear >= 0.9 * len(rows)
    assert mismatch <= max(2, 0.05 * len(rows)), (mismatch, len(rows))
    # sel is in descending order: a swap inside the top 8 is a mismatch too unless the two
    # logits are within an ulp, which the margin rule does not cover, so allow exactly those
    for T, lg, got in rows:
        ref = i4ref.topk_sel(lg[None], K8)[0]
        s = np.sort(lg)[::-1]
        if s[K8 - 1] - s[K8] > _ulp16(s[K8 - 1]):
            assert set(got) == set(ref)
            for a, b in zip(got, ref):
                assert a == b or abs(lg[a] - lg[b]) <= _ulp16(lg[a])


# ---------------------------------------------------------------- 24-layer stack, 128 experts
def test_stack_24_layers_full_size(pkg, dev):
    """The Thinker[0:24] MoE stack at the workload's size (128 experts, AWQ g128, pre-MoE
    RMSNorm): one stack call equals the loop of 24 module calls bit for bit, and the first
    and last layers match the oracle on the inputs the GPU fed them."""
    n_layers = 24
    gen = torch.Generator(device=dev)
    gen.manual_seed(104)
    G = 128

    def words(*shape):
        return torch.randint(-2**31, 2**31, shape, dtype=torch.int32, device=dev, generator=gen)

    def awq(K, N):
        qw, qz = words(E, K, N // 8), words(E, K // G, N // 8)
        sc = (torch.rand(E, K // G, N, device=dev, generator=gen) * 0.018 + 0.002).half()
        return qw, qz, sc

    mods, keep = [], {}
    for li in range(n_layers):
        g, u, d = awq(H, I), awq(H, I), awq(I, H)
        wr = (torch.randn(E, H, device=dev, generator=gen) * 0.02).half()
        nw = (torch.rand(H, device=dev, generator=gen) * 0.4 + 0.8).half()
        q = lambda p: pkg.QWeight.awq(p[0], p[2], p[1], group=G)
        mods.append(pkg.FusedPackedMoE.from_awq(q(g), q(u), q(d), wr, top_k=K8, norm_weight=nw))
        if li in (0, n_layers - 1):
            keep[li] = (g, u, d, nw)
        del g, u, d
    rng = np.random.default_rng(105)
    x = t_(make_x(rng, (1, H), "f16"), dev)
    stack = pkg.moe_stack(x, [m.stack_entry() for m in mods], K8)
    h, ins = x, []
    for m in mods:
        ins.append(h)
        h = m(h, residual=h)
    assert torch.isfinite(stack).all()
    assert torch.equal(stack, h)
    for li, (g, u, d, nw) in keep.items():
        m = mods[li]
        ex = lambda p, e: [i4ref.awq_dequant(p[0][e].cpu().numpy(), p[1][e].cpu().numpy(),
                                             p[2][e].float().cpu().numpy(), G)]
        dgu = lambda e: np.concatenate(ex(g, e) + ex(u, e), axis=0)
        ddn = lambda e: ex(d, e)[0]
        hin = ins[li]
        lg, xn = pkg.router_logits(hin, m.router_w, m.norm_weight, 1e-6, return_xn=True)
        sel_ref, w_ref = i4ref.route(host(lg), K8)
        w_gpu, sel_gpu = m.route(hin)
        np.testing.assert_array_equal(sel_gpu.cpu().numpy(), sel_ref)
        moe_ref = i4ref.moe_layer_grouped(host(xn), sel_ref, w_ref, dgu, ddn, "f16", y_dtype="f16")
        out_l = host(ins[li + 1] if li + 1 < n_layers else h)
        check_moe_term(out_l, moe_ref, host(hin), "f16")


# ---------------------------------------------------------------- the bounded wait
def test_decode_wait_gives_up_visibly(pkg, dev):
    """The down workgroups of the single-launch decode layer, run alone with their bound on
    the wait lowered from the host: with the activations left pending they give up, write NaN
    rows and report I4_ERR_HANDOFF, and every kernel exits (the stream synchronises); with the
    activations in place they compute the down + combine stage bit for bit."""
    rng = np.random.default_rng(106)
    moe, _, _, _ = _awq_moe(pkg, dev, rng, E=64)
    x = t_(make_x(rng, (1, H), "f16"), dev)
    res = t_(make_x(rng, (1, H), "f16"), dev)
    lg = pkg.router_logits(x, moe.router_w)
    act, sel, w = pkg.moe_route_gate_up(x, moe.gate_up, lg, K8)
    want = pkg.moe_down_combine(act, moe.down, sel, w, residual=res)
    out, status = pkg.moe_down_wait(act, moe.down, lg, K8, residual=res, max_polls=4)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    assert torch.equal(out, want)
    pending = torch.full_like(act, float("nan")).view(torch.int16).fill_(-1).view(act.dtype)
    for polls in (0, 3):
        out, status = pkg.moe_down_wait(pending, moe.down, lg, K8, residual=res, max_polls=polls)
        torch.cuda.synchronize()
        assert int(status.item()) == -10
        assert torch.isnan(out).all()
    lib = pkg.lib()
    assert b"gave up waiting" in lib.i4_strerror(-10)


def test_moe_status_word_reads_ok_after_calls(pkg, dev):
    """The status word of i4_moe_forward / i4_moe_stack_forward is I4_OK after ordinary decode
    and batched calls (it is cleared by the call itself, whatever the workspace held)."""
    rng = np.random.default_rng(107)
    moe, _, _, _ = _awq_moe(pkg, dev, rng, E=32)
    ws = pkg.Workspace()
    for T in (1, 40, 1):
        x = t_(make_x(rng, (T, H), "f16"), dev)
        ws.get(pkg.lib().i4_moe_workspace_bytes(T, H, I, 32, K8), dev).fill_(0xA5)
        pkg.moe_forward(x, moe.gate_up, moe.down, K8, router_w=moe.router_w, workspace=ws,
                        gate_up_tile=moe.gate_up_tile, down_tile=moe.down_tile)
        assert pkg.ops.moe_status(ws, T, H, I, 32, K8) == 0
    x = t_(make_x(rng, (1, H), "f16"), dev)
    ws2 = pkg.Workspace()
    pkg.moe_stack(x, [moe.stack_entry()] * 3, K8, workspace=ws2)
    assert pkg.ops.moe_status(ws2, 1, H, I, 32, K8) == 0


def test_stack_pieces_equal_the_stack(pkg, dev):
    """The XCD-local decode path run launch by launch through the C ABI (i4_moe_route_sum,
    i4_moe_experts_x, i4_moe_sum) equals i4_moe_stack_forward and the module loop bit for
    bit, the layer outputs written by the router launches included."""
    rng = np.random.default_rng(108)
    mods = []
    for _ in range(3):
        m, _, _, _ = _awq_moe(pkg, dev, rng, E=32)
        nw = rng.uniform(0.5, 1.5, H).astype(np.float16)
        m.register_buffer("norm_weight", t_(nw, dev), persistent=False)
        m.norm_eps = 1e-6
        mods.append(m)
    layers = [mods[i % 3].stack_entry() for i in range(5)]
    x = t_(make_x(rng, (1, H), "f16"), dev)
    ws = pkg.Workspace()
    pieces = [pkg.StackLayerX(layer, K8, torch.float16, workspace=ws) for layer in layers]
    ypart = torch.empty(K8, H, dtype=torch.float16, device=dev)
    hbuf = [torch.empty(1, H, dtype=torch.float16, device=dev) for _ in range(2)]
    h, hs = x, []
    for li, p in enumerate(pieces):
        if li == 0:
            p.route(h, reset_status=True)
        else:
            p.route(h, ypart, hbuf[li % 2])
            h = hbuf[li % 2]
            hs.append(h.clone())
        p.experts(h, ypart)
    out = torch.empty_like(x)
    pieces[-1].sum(h, ypart, out)
    stack = pkg.moe_stack(x, layers, K8)
    loop, ref_hs = x, []
    for li in range(5):
        loop = mods[li % 3](loop, residual=loop)
        ref_hs.append(loop)
    torch.cuda.synchronize()
    assert torch.equal(out, stack) and torch.equal(out, loop)
    for got, want in zip(hs, ref_hs[:-1]):
        assert torch.equal(got, want)
    assert pkg.ops.moe_status(ws, 1, H, I, 32, K8) == 0


def test_stack_experts_wait_gives_up_visibly(pkg, dev):
    """The down workgroups of the XCD-local experts launch run alone, with their bound on the
    wait lowered from the host: the activations stay pending, so they give up, write NaN slot
    rows and report I4_ERR_HANDOFF, and every kernel exits.  The next ordinary layer on the
    same workspace (its router launch clears the status word) is correct again."""
    rng = np.random.default_rng(109)
    m, _, _, _ = _awq_moe(pkg, dev, rng, E=64)
    layer = m.stack_entry()
    x = t_(make_x(rng, (1, H), "f16"), dev)
    ws = pkg.Workspace()
    p = pkg.StackLayerX(layer, K8, torch.float16, workspace=ws)
    ypart = torch.zeros(K8, H, dtype=torch.float16, device=dev)
    for polls in (0, 3):
        p.route(x, reset_status=True)  # arms the activations with the pending pattern
        p.experts(x, ypart, max_polls=polls, down_only=True)
        torch.cuda.synchronize()
        assert pkg.ops.moe_status(ws, 1, H, I, 64, K8) == -10
        assert torch.isnan(ypart).all()
    p.route(x, reset_status=True)
    p.experts(x, ypart)
    out = torch.empty_like(x)
    p.sum(x, ypart, out)
    want = m(x, residual=x)
    torch.cuda.synchronize()
    assert pkg.ops.moe_status(ws, 1, H, I, 64, K8) == 0
    assert torch.equal(out, want)


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
def test_decode_layer_against_the_reference_rounding(pkg, dev, xdt):
    """The decode layer (C3: 128 experts, top-8, 2048 / 768, AWQ g128, with the residual)
    against the oracle in the reference's own rounding of the combine (routing weights and
    expert outputs rounded to the activation dtype, 16-bit products, fp32 sum rounded once,
    then the residual add; fused_packed_moe.py:199,262) as well as against the float64
    combine.  The build keeps the weights and the weighted sum in fp32 and rounds once, so
    it sits between the two; its distance from the reference's rounding is within the
    parity bar (2e-2 of max |ref|) and, elementwise, within a few ulps of the largest
    added term; the measured distances are printed."""
    rng = np.random.default_rng(110 + (xdt == "bf16"))
    sdt = "bf16" if xdt == "bf16" else np.float16
    moe, dgu, ddn, _ = _awq_moe(pkg, dev, rng, sdt=sdt)
    tdt = torch.bfloat16 if xdt == "bf16" else torch.float16
    moe.router_w = moe.router_w.to(tdt)
    hn = half_name(xdt)
    worst_rel, worst_ulp = 0.0, 0.0
    for rep in range(4):
        x = make_x(rng, (1, H), xdt)
        res = make_x(rng, (1, H), xdt)
        out, sel, w = pkg.moe_forward(t_(x, dev), moe.gate_up, moe.down, K8,
                                      router_w=moe.router_w, residual=t_(res, dev),
                                      return_routing=True, gate_up_tile=moe.gate_up_tile,
                                      down_tile=moe.down_tile)
        lg = host(pkg.router_logits(t_(x, dev), moe.router_w))
        sel_ref, w_ref = i4ref.route(lg, K8)
        np.testing.assert_array_equal(sel.cpu().numpy(), sel_ref)
        xin, r = f_(x)[0], f_(res)[0]
        ys = []
        for e in sel_ref[0]:
            gu = dgu(int(e)) @ xin
            a = i4ref.round_half(i4ref.silu(gu[:I]) * gu[I:], hn)
            ys.append(i4ref.round_half(ddn(int(e)) @ a, hn))
        ys = np.stack(ys)
        ref_rounding = i4ref.ref_combine(ys, w_ref[0], hn, r)
        exact = r + (w_ref[0][:, None] * ys).sum(0)
        got = host(out)[0]
        rel = i4ref.rel_err(got, ref_rounding)
        scale = np.maximum(np.maximum(np.abs(r), np.abs(exact - r)),
                           np.max(np.abs(w_ref[0][:, None] * ys), axis=0))
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(scale, 2.0 ** -14))) - (10 if hn == "f16" else 7))
        worst_rel = max(worst_rel, rel)
        worst_ulp = max(worst_ulp, float(np.max(np.abs(got - ref_rounding) / ulp)))
        assert rel <= 2e-2, rel
        assert i4ref.rel_err(got, exact) <= 2e-2
    print(f"\n{xdt}: build vs the reference's rounding: max|err|/max|ref| {worst_rel:.2e}, "
          f"{worst_ulp:.1f} ulps of the largest term")
    assert worst_ulp <= 8, worst_ulp

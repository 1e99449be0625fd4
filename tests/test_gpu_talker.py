"""Parity of the Talker MoE kernels (i4_dmoe_forward, called through the C ABI)
and of the FusedMoE drop-in with the CPU oracle (oracle/i4ref.py: route,
dense_moe, q8_quantize).

Bar: routing indices bit-exact against the oracle's routing of the same
logits; int8 weights bit-exact against q8_quantize; floating outputs within
max|got - ref| <= TOL * max|ref| (bf16 1e-2, fp16 2e-3: fp32 accumulation on
the GPU against float64 with the same rounding points; transformers' own bf16
block lands within the same bar, tests/test_talker_ref.py).  Shapes are the
Talker's (hidden 1024, 128 experts, top-6, expert FFN 384, shared expert FFN
768, qwen3-omni-config.json talker_config.text_config) unless a case says
otherwise.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import i4ref

pytestmark = pytest.mark.gpu
TOL = {torch.bfloat16: 1e-2, torch.float16: 2e-3}
NAME = {torch.bfloat16: "bf16", torch.float16: "f16"}
H, E, K, I, IS = 1024, 128, 6, 384, 768


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().double().cpu().numpy()


class _Rows:
    """fp64 view of a device stack [E, N, K] for the oracle: only the experts it
    indexes are copied, int8 rows are dequantised exactly (q * s in fp64)."""

    def __init__(self, t: torch.Tensor, scale: torch.Tensor | None = None):
        self.t, self.scale = t, scale
        self.shape = tuple(t.shape)

    def __getitem__(self, e):
        w = self.t[int(e)].double().cpu()
        if self.scale is not None:
            w = w * self.scale[int(e)].double().cpu().reshape(-1, 1)
        return w.numpy()


def _stacks(dev, dt, seed, E=E, I=I, Is=IS, H=H):
    g = torch.Generator(device=dev).manual_seed(seed)
    r = lambda *s, sd=0.03: (torch.randn(*s, generator=g, device=dev) * sd).to(dt)
    return dict(gu=r(E, 2 * I, H), dn=r(E, H, I), rw=r(E, H, sd=0.05),
                sgu=r(2 * Is, H), sdn=r(H, Is), sgw=r(H, sd=0.05),
                x=r(64, H, sd=1.0), res=r(64, H, sd=1.0))


def _check(pkg, S, dt, T, q8=False, shared=True, gate=True, residual=False, use_logits=False,
           renorm=True, top_k=K):
    x = S["x"][:T].contiguous()
    gu, dn, gus, dns = S["gu"], S["dn"], None, None
    if q8:
        gu, gus = pkg.quantize_q8(S["gu"])
        dn, dns = pkg.quantize_q8(S["dn"])
    logits = pkg.router_logits(x, S["rw"])
    kw = dict(norm_topk_prob=renorm, gate_up_scale=gus, down_scale=dns, return_routing=True)
    if use_logits:
        kw["logits"] = logits
    else:
        kw["router_w"] = S["rw"]
    if shared:
        kw.update(shared_gate_up=S["sgu"], shared_down=S["sdn"],
                  shared_gate_w=S["sgw"] if gate else None)
    if residual:
        kw["residual"] = S["res"][:T]
    out, sel, wts = pkg.dmoe_forward(x, gu, dn, top_k, **kw)
    torch.cuda.synchronize()
    sel_o, w_o = i4ref.route(host(logits), top_k, renorm)
    assert np.array_equal(host(sel).astype(np.int64), sel_o), "routing differs from the oracle"
    np.testing.assert_allclose(host(wts), w_o, rtol=0, atol=2e-6)
    sh = (host(S["sgu"]), host(S["sdn"]), host(S["sgw"]) if gate else None) if shared else None
    ref = i4ref.dense_moe(host(x), sel_o, w_o, _Rows(gu, gus), _Rows(dn, dns), NAME[dt],
                          shared=sh, residual=host(S["res"][:T]) if residual else None,
                          out_dtype=NAME[dt])
    err = i4ref.rel_err(host(out), ref)
    assert err <= TOL[dt], f"rel err {err:.2e} (T={T}, q8={q8})"
    return out


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("q8", [False, True])
@pytest.mark.parametrize("T", [1, 5, 33])
def test_dmoe_matches_oracle(pkg, dev, dt, q8, T):
    print(f"dmoe dt={dt} q8={q8} T={T}", flush=True)
    _check(pkg, _stacks(dev, dt, seed=10 + T), dt, T, q8=q8)


@pytest.mark.parametrize("case", [
    dict(shared=False), dict(gate=False), dict(residual=True), dict(use_logits=True),
    dict(renorm=False), dict(top_k=7), dict(shared=False, top_k=8), dict(q8=True, residual=True),
])
def test_dmoe_variants(pkg, dev, case):
    print(f"dmoe variant {case}", flush=True)
    _check(pkg, _stacks(dev, torch.bfloat16, seed=3), torch.bfloat16, 3, **case)


@pytest.mark.parametrize("case", [
    dict(shared=False), dict(gate=False), dict(residual=True), dict(renorm=False),
    dict(top_k=7), dict(shared=False, top_k=8), dict(q8=True, residual=True),
    dict(dt=torch.float16, q8=True, gate=False),
])
def test_dmoe_single_launch_variants(pkg, dev, case):
    """One token with the router in the block: with 16-bit experts gate|up and down run in
    one launch (the down workgroups rank the logits, make the shared gate and wait for the
    activations), int8 experts in two."""
    print(f"dmoe single launch {case}", flush=True)
    case = dict(case)
    dt = case.pop("dt", torch.bfloat16)
    _check(pkg, _stacks(dev, dt, seed=6), dt, 1, **case)


def test_dmoe_single_launch_equals_two_launches(pkg, dev):
    """The single-launch decode block and the two-launch path over the same logits give the
    same output, routing and weights bit for bit, in bf16 and int8 modes."""
    for dt, q8 in ((torch.bfloat16, False), (torch.bfloat16, True), (torch.float16, False)):
        S = _stacks(dev, dt, seed=7)
        x = S["x"][:1].contiguous()
        gu, dn, gus, dns = S["gu"], S["dn"], None, None
        if q8:
            gu, gus = pkg.quantize_q8(S["gu"])
            dn, dns = pkg.quantize_q8(S["dn"])
        kw = dict(gate_up_scale=gus, down_scale=dns, shared_gate_up=S["sgu"],
                  shared_down=S["sdn"], shared_gate_w=S["sgw"], residual=S["res"][:1],
                  return_routing=True)
        a = pkg.dmoe_forward(x, gu, dn, K, router_w=S["rw"], **kw)
        b = pkg.dmoe_forward(x, gu, dn, K, logits=pkg.router_logits(x, S["rw"]), **kw)
        torch.cuda.synchronize()
        for u, v in zip(a, b):
            assert torch.equal(u, v), f"single launch differs (dt={dt}, q8={q8})"


def test_dmoe_wait_gives_up_visibly(pkg, dev):
    """The down workgroups of the single-launch block run alone with their bound on the wait
    lowered from the host: with the activations left pending they give up, write NaN and
    report I4_ERR_HANDOFF, and every kernel exits; with the activations in place (left by a
    full call on the same workspace) they reproduce that call's output bit for bit; the
    status word reads I4_OK after ordinary calls whatever the workspace held."""
    S = _stacks(dev, torch.bfloat16, seed=8)
    x = S["x"][:1].contiguous()
    kw = dict(shared_gate_up=S["sgu"], shared_down=S["sdn"], shared_gate_w=S["sgw"],
              residual=S["res"][:1])
    ws = pkg.Workspace()
    nb = pkg.ops.dmoe_workspace_bytes(1, E, K, I, IS)
    for T in (1, 3, 1):
        ws.get(pkg.ops.dmoe_workspace_bytes(T, E, K, I, IS), dev).fill_(0xA5)
        pkg.dmoe_forward(S["x"][:T].contiguous(), S["gu"], S["dn"], K, router_w=S["rw"],
                         workspace=ws, shared_gate_up=S["sgu"], shared_down=S["sdn"],
                         shared_gate_w=S["sgw"])
        assert pkg.dmoe_status(ws, T, E, K, I, IS) == 0
    want = pkg.dmoe_forward(x, S["gu"], S["dn"], K, router_w=S["rw"], workspace=ws, **kw)
    lg = pkg.router_logits(x, S["rw"])
    got = pkg.dmoe_down_wait(x, S["gu"], S["dn"], K, lg, ws, max_polls=4, **kw)
    assert pkg.dmoe_status(ws, 1, E, K, I, IS) == 0
    assert torch.equal(got, want.reshape(-1))
    for polls in (0, 3):
        ws.get(nb, dev).fill_(0xFF)  # every activation pending, status word included
        ws.buf[pkg.lib().i4_dmoe_status_offset(1, E, K, I, IS):][:4].zero_()
        out = pkg.dmoe_down_wait(x, S["gu"], S["dn"], K, lg, ws, max_polls=polls, **kw)
        assert pkg.dmoe_status(ws, 1, E, K, I, IS) == -10
        assert torch.isnan(out.float()).all()


def test_dmoe_small_shapes(pkg, dev):
    """H 256, 16 experts (one logit per lane pair), I 48, shared 32: the clamped
    chunk and row paths (fewer chunks than lanes)."""
    S = _stacks(dev, torch.bfloat16, seed=4, E=16, I=48, Is=32, H=256)
    for T in (4, 1):
        _check(pkg, S, torch.bfloat16, T, top_k=4)
        _check(pkg, S, torch.bfloat16, T, top_k=4, q8=True)


def test_dmoe_is_deterministic(pkg, dev):
    S = _stacks(dev, torch.bfloat16, seed=5)
    a = _check(pkg, S, torch.bfloat16, 9)
    b = _check(pkg, S, torch.bfloat16, 9)
    assert torch.equal(a, b)


def test_q8_buffers_match_oracle(pkg, dev):
    S = _stacks(dev, torch.bfloat16, seed=6)
    q, s = pkg.quantize_q8(S["gu"][:4])
    qo, so = i4ref.q8_quantize(host(S["gu"][:4]), "bf16")
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(host(s), so)


# ------------------------------------------------------------- FusedMoE drop-in
def _tf_block(dt, dev, E=32, seed=0):
    from transformers.models.qwen3_omni_moe.configuration_qwen3_omni_moe import (
        Qwen3OmniMoeTalkerTextConfig,
    )
    from transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe import (
        Qwen3OmniMoeTalkerTextSparseMoeBlock,
    )

    cfg = Qwen3OmniMoeTalkerTextConfig(
        hidden_size=H, num_experts=E, num_experts_per_tok=K, moe_intermediate_size=I,
        shared_expert_intermediate_size=IS, norm_topk_prob=True, num_hidden_layers=1)
    cfg._experts_implementation = "eager"
    torch.manual_seed(seed)
    blk = Qwen3OmniMoeTalkerTextSparseMoeBlock(cfg)
    with torch.no_grad():
        for p in blk.parameters():
            p.copy_(torch.randn_like(p) * 0.03)
    return blk.to(dev, dt).eval()


class _MLP(nn.Module):
    def __init__(self, g, u, d):
        super().__init__()
        self.gate_proj = nn.Linear(g.shape[1], g.shape[0], bias=False)
        self.up_proj = nn.Linear(u.shape[1], u.shape[0], bias=False)
        self.down_proj = nn.Linear(d.shape[1], d.shape[0], bias=False)
        with torch.no_grad():
            self.gate_proj.weight.copy_(g)
            self.up_proj.weight.copy_(u)
            self.down_proj.weight.copy_(d)


class _ListSparseMoeBlock(nn.Module):
    """The expert container fused_moe.py reads: a ModuleList of gate/up/down MLPs."""

    def __init__(self, blk):
        super().__init__()
        gu, dn = blk.experts.gate_up_proj.detach(), blk.experts.down_proj.detach()
        self.gate = nn.Linear(H, gu.shape[0], bias=False).to(gu.device, gu.dtype)
        with torch.no_grad():
            self.gate.weight.copy_(blk.gate.weight)
        self.top_k, self.norm_topk_prob = K, True
        self.experts = nn.ModuleList(
            _MLP(gu[e, :I], gu[e, I:], dn[e]).to(gu.device, gu.dtype) for e in range(gu.shape[0]))
        self.shared_expert = blk.shared_expert
        self.shared_expert_gate = blk.shared_expert_gate


def _oracle_block(pkg, fm, x, dt):
    sel, w = i4ref.route(host(pkg.router_logits(x, fm.router_w)), fm.top_k, fm.norm_topk_prob)
    sh = (host(fm.shared_gate_up), host(fm.shared_down), host(fm.shared_gate_w))
    return sel, i4ref.dense_moe(host(x), sel, w, _Rows(fm.gate_up, fm.gate_up_s),
                                _Rows(fm.down, fm.down_s), NAME[dt], shared=sh,
                                out_dtype=NAME[dt])


@pytest.mark.parametrize("q8", [False, True])
def test_fused_moe_replaces_transformers_block(pkg, dev, q8):
    print(f"FusedMoE q8={q8}", flush=True)
    dt = torch.bfloat16
    blk = _tf_block(dt, dev)
    x = (torch.randn(1, 7, H, device=dev) * 0.7).to(dt)
    fm = pkg.FusedMoE(blk, q8=q8)
    if q8:
        q, s = i4ref.q8_quantize(host(blk.experts.gate_up_proj[:3]), "bf16")
        assert np.array_equal(fm.gate_up[:3].cpu().numpy(), q)
        assert np.array_equal(host(fm.gate_up_s[:3]), s)
    out, sel, _ = fm(x, return_routing=True)
    assert out.shape == x.shape and out.dtype == dt
    sel_o, ref = _oracle_block(pkg, fm, x.view(7, H), dt)
    assert np.array_equal(host(sel).astype(np.int64), sel_o)
    assert i4ref.rel_err(host(out.view(7, H)), ref) <= TOL[dt]
    if not q8:
        # and the transformers block itself (bf16 on the GPU) within the same bar, on
        # the tokens where its torch.topk picked the same experts (bf16 logits can
        # tie, and torch.topk fixes no order among ties)
        with torch.no_grad():
            want = blk(x).view(7, H)
            _, _, b_sel = blk.gate(x.view(7, H))
        same = [t for t in range(7)
                if set(host(b_sel[t]).astype(int)) == set(sel_o[t].tolist())]
        assert len(same) >= 5
        assert i4ref.rel_err(host(out.view(7, H)[same]), host(want[same])) <= TOL[dt]


def test_fused_moe_modulelist_and_stacked_forms_agree(pkg, dev):
    dt = torch.bfloat16
    blk = _tf_block(dt, dev, E=16, seed=1)
    a = pkg.FusedMoE(blk)
    b = pkg.FusedMoE(_ListSparseMoeBlock(blk))
    assert torch.equal(a.gate_up, b.gate_up) and torch.equal(a.down, b.down)
    x = (torch.randn(3, H, device=dev) * 0.7).to(dt)
    assert torch.equal(a(x), b(x))


def test_fuse_moe_blocks_swaps_unquantized_blocks(pkg, dev):
    class _PackedLin(nn.Module):
        def __init__(self):
            super().__init__()
            self.weight_packed = torch.zeros(1)

    class _PackedSparseMoeBlock(nn.Module):
        def __init__(self):
            super().__init__()
            e = nn.Module()
            e.gate_proj = _PackedLin()
            self.experts = nn.ModuleList([e])

    model = nn.Module()
    model.a = nn.Module()
    model.a.mlp = _tf_block(torch.bfloat16, dev, E=8, seed=2)
    model.b = nn.Module()
    model.b.mlp = _PackedSparseMoeBlock()
    x = (torch.randn(2, H, device=dev) * 0.7).to(torch.bfloat16)
    want = pkg.FusedMoE(model.a.mlp)(x)
    assert pkg.fuse_moe_blocks(model, verbose=False) == 1
    assert isinstance(model.a.mlp, pkg.FusedMoE)
    assert type(model.b.mlp).__name__ == "_PackedSparseMoeBlock"
    assert torch.equal(model.a.mlp(x), want)


def test_dmoe_rejects_cpu_tensors(pkg):
    x = torch.zeros(1, H, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):
        pkg.dmoe_forward(x, torch.zeros(E, 2 * I, H, dtype=torch.bfloat16),
                         torch.zeros(E, H, I, dtype=torch.bfloat16), K,
                         router_w=torch.zeros(E, H, dtype=torch.bfloat16))


@pytest.mark.parametrize("T,q8", [(64, False), (300, True)])
def test_dmoe_tokens_are_independent(pkg, dev, T, q8):
    """Size-independent property at batch sizes the oracle would take long on: every token
    of a T-token call equals the same token run alone, bit for bit (per-token routing
    through the batched router -- one-token tiles up to 64 tokens, 8-token tiles above --
    gives the single-token router's logits, and each token streams its own experts)."""
    S = _stacks(dev, torch.bfloat16, seed=21)
    gu, dn, gus, dns = S["gu"], S["dn"], None, None
    if q8:
        gu, gus = pkg.quantize_q8(gu)
        dn, dns = pkg.quantize_q8(dn)
    g = torch.Generator(device=dev).manual_seed(22)
    x = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16)
    kw = dict(router_w=S["rw"], gate_up_scale=gus, down_scale=dns, shared_gate_up=S["sgu"],
              shared_down=S["sdn"], shared_gate_w=S["sgw"])
    out = pkg.dmoe_forward(x, gu, dn, K, **kw)
    for t in (0, 1, T // 2, T - 2, T - 1):
        one = pkg.dmoe_forward(x[t:t + 1].contiguous(), gu, dn, K, **kw)
        assert torch.equal(out[t:t + 1], one), f"token {t} of {T}"
    assert torch.isfinite(out.float()).all()

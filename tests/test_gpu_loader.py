"""Checkpoint reader -> HIP kernels: a synthetic compressed-tensors Thinker checkpoint
at the real shapes (hidden 2048, expert FFN 768, group 32 symmetric, bf16 scales and
activations; src/duplex/streaming/clock.py:45-103) loaded onto the device and run
through the MoE block, the 2-layer stack and the attention projections, checked
against the oracle on independently dequantised ground truth."""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from oracle import i4ref
from tests import _ckpt
from tests.test_gpu_parity import TOL, _check_moe, host, make_x, t_

pytestmark = pytest.mark.gpu

E, H, I, G = 16, 2048, 768, 32


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    root = tmp_path_factory.mktemp("thinker_ck")
    truth = _ckpt.write_checkpoint(root, np.random.default_rng(81), n_layers=2, E=E, H=H, I=I,
                                   G=G, top_k=8, shards=2, attention=(4096, 512))
    return root, truth


def _ld(pkg):
    return importlib.import_module(pkg.__name__ + ".loader")


def _dense_fns(t):
    dgu = lambda e: np.concatenate([_ckpt.dense(t["experts"][e]["gate_proj"]),
                                    _ckpt.dense(t["experts"][e]["up_proj"])], axis=0)
    ddn = lambda e: _ckpt.dense(t["experts"][e]["down_proj"])
    return dgu, ddn


@pytest.mark.parametrize("T", [1, 40])
def test_loaded_moe_layer_matches_oracle(pkg, dev, ckpt, T):
    root, truth = ckpt
    ld = _ld(pkg)
    ck = ld.Checkpoint(root)
    rng = np.random.default_rng(82 + T)
    for layer in range(2):
        moe = ld.load_moe_layer(ck, layer, dev, torch.bfloat16)
        assert moe.gate_up.layout == "ct" and moe.gate_up_tile.layout == "tile"
        dgu, ddn = _dense_fns(truth[layer])
        x = make_x(rng, (T, H), "bf16")
        nw = i4ref.f32_to_bf16_bits(truth[layer]["norm"].astype(np.float32))
        _check_moe(pkg, moe, dgu, ddn, x, "bf16", dev, residual=x, norm=(nw, 1e-6))


def test_loaded_stack_equals_module_loop(pkg, dev, ckpt):
    root, _ = ckpt
    ld = _ld(pkg)
    blocks = ld.load_thinker_moe_stack(root, 2, dev, torch.bfloat16)
    x = t_(make_x(np.random.default_rng(84), (1, H), "bf16"), dev)
    stack = pkg.moe_stack(x, [b.stack_entry() for b in blocks], 8)
    h = x
    for b in blocks:
        h = b(h, residual=h)
    assert torch.isfinite(stack.float()).all()
    assert torch.equal(stack, h)


@pytest.mark.parametrize("rows", [1, 40])
def test_loaded_attention_projections(pkg, dev, ckpt, rows):
    root, truth = ckpt
    ld = _ld(pkg)
    ck = ld.Checkpoint(root)
    lin = ld.load_attention(ck, 1, dev)
    fused = ld.load_attention(ck, 1, dev, fuse_qkv=True)
    rng = np.random.default_rng(85 + rows)
    x = make_x(rng, (rows, H), "bf16")
    xt = t_(x, dev)
    qkv = fused["qkv"](xt)
    for i, name in enumerate(("q_proj", "k_proj", "v_proj")):
        W = _ckpt.dense(truth[1]["attn"][name])
        ref = i4ref.bf16_bits_to_f32(x).astype(np.float64) @ W.T
        got = host(lin[name](xt))
        assert i4ref.rel_err(got, ref) <= TOL
        assert i4ref.rel_err(host(qkv[i]), ref) <= TOL
    xo = make_x(rng, (rows, 4096), "bf16")
    W = _ckpt.dense(truth[1]["attn"]["o_proj"])
    ref = i4ref.bf16_bits_to_f32(xo).astype(np.float64) @ W.T
    assert i4ref.rel_err(host(lin["o_proj"](t_(xo, dev))), ref) <= TOL
    assert i4ref.rel_err(host(fused["o"](t_(xo, dev))), ref) <= TOL


def _attn_weights(t):
    return {n[0]: torch.from_numpy(_ckpt.dense(t["attn"][f"{n}_proj"])).float()
            for n in ("q", "k", "v", "o")}


def _bf16_to_torch(a):
    return torch.from_numpy(i4ref.bf16_bits_to_f32(a)).float()


@pytest.mark.parametrize("start", [0, 60])
def test_thinker_attention_decode_matches_reference(pkg, dev, ckpt, start):
    """Decode steps through ThinkerAttention (input RMSNorm, q|k|v GEMV, q/k norm + rotary +
    cache append, GQA attention over the cache, o_proj + residual) against the fp32
    reference on the same inputs; start = 60 crosses the 64-position chunk boundary and
    reads cache rows written by earlier calls."""
    from tests import _thinker_ref

    root, truth = ckpt
    ld = _ld(pkg)
    layer = ld.load_thinker_layer(ld.Checkpoint(root), 1, dev, torch.bfloat16, max_len=256)
    attn = layer.attn
    t = truth[1]
    W = _attn_weights(t)
    rng = np.random.default_rng(90 + start)
    # rows [0, start) of the cache: arbitrary earlier keys / values, shared by both sides
    kv = [i4ref.f32_to_bf16_bits(rng.standard_normal((4, start, 128)).astype(np.float32))
          for _ in range(2)]
    attn.k_cache[:, :start] = t_(kv[0], dev)
    attn.v_cache[:, :start] = t_(kv[1], dev)
    cache = {"k": _bf16_to_torch(kv[0]), "v": _bf16_to_torch(kv[1])}
    for pos in range(start, start + 6):
        h = make_x(rng, (1, H), "bf16")
        got = host(attn(t_(h, dev), pos))[0]
        ref = _thinker_ref.attention_decode(
            _bf16_to_torch(h[0]), W, torch.from_numpy(t["attn"]["q_norm"]),
            torch.from_numpy(t["attn"]["k_norm"]), torch.from_numpy(t["in_norm"]), 1e-6,
            pkg.rope_inv_freq(128, 1e6), pos, cache, 32, 4).numpy()
        assert np.all(np.isfinite(got))
        # the attention's own contribution, checked apart from the residual
        res = i4ref.bf16_bits_to_f32(h[0]).astype(np.float64)
        assert i4ref.rel_err(got - res, ref - res) <= TOL
        # the cache rows the kernel wrote match the reference's (k normed + rotated, v as is)
        kg = attn.k_cache[:, pos].float().cpu().numpy()
        assert i4ref.rel_err(kg, cache["k"][:, pos].numpy()) <= TOL
        vg = attn.v_cache[:, pos].float().cpu().numpy()
        assert i4ref.rel_err(vg, cache["v"][:, pos].numpy()) <= TOL


def test_thinker_attention_long_context(pkg, dev, ckpt):
    """One decode step at position 3000 (47 chunks merged by the combine kernel)."""
    from tests import _thinker_ref

    root, truth = ckpt
    ld = _ld(pkg)
    layer = ld.load_thinker_layer(ld.Checkpoint(root), 0, dev, torch.bfloat16, max_len=4096)
    attn = layer.attn
    t = truth[0]
    rng = np.random.default_rng(95)
    P = 3000
    kv = [i4ref.f32_to_bf16_bits(rng.standard_normal((4, P, 128)).astype(np.float32))
          for _ in range(2)]
    attn.k_cache[:, :P] = t_(kv[0], dev)
    attn.v_cache[:, :P] = t_(kv[1], dev)
    cache = {"k": _bf16_to_torch(kv[0]), "v": _bf16_to_torch(kv[1])}
    h = make_x(rng, (1, H), "bf16")
    got = host(attn(t_(h, dev), P))[0]
    ref = _thinker_ref.attention_decode(
        _bf16_to_torch(h[0]), _attn_weights(t), torch.from_numpy(t["attn"]["q_norm"]),
        torch.from_numpy(t["attn"]["k_norm"]), torch.from_numpy(t["in_norm"]), 1e-6,
        pkg.rope_inv_freq(128, 1e6), P, cache, 32, 4).numpy()
    res = i4ref.bf16_bits_to_f32(h[0]).astype(np.float64)
    assert i4ref.rel_err(got - res, ref - res) <= TOL


def test_thinker_decoder_step_composes(pkg, dev, ckpt):
    """ThinkerDecoder.step = attention then MoE block per layer, bit for bit, and finite over
    several positions (the per-block parity is checked above and in the MoE tests)."""
    root, _ = ckpt
    ld = _ld(pkg)
    dec = ld.load_thinker_decoder(root, 2, dev, torch.bfloat16, max_len=64)
    twin = ld.load_thinker_decoder(root, 2, dev, torch.bfloat16, max_len=64)
    assert dec.fused()  # step runs i4_thinker_decode_step
    rng = np.random.default_rng(96)
    for pos in range(4):
        x = t_(make_x(rng, (1, H), "bf16"), dev)
        out = dec.step(x, pos)
        h = x
        for layer in twin.layers:
            h = layer.attn(h, pos)
            h = layer.moe(h, residual=h)
        assert torch.isfinite(out.float()).all()
        assert torch.equal(out, h)


@pytest.mark.parametrize("xdt,K,M", [("bf16", 2048, 1), ("f16", 4096, 3), ("bf16", 4096, 1)])
def test_rmsnorm_linear_equals_norm_then_linear(pkg, dev, xdt, K, M):
    """The norm folded into the GEMV gives exactly rmsnorm() then linear(), and the norm
    itself matches the oracle's RMSNorm."""
    rng = np.random.default_rng(97 + K + M)
    tdt = torch.bfloat16 if xdt == "bf16" else torch.float16
    p, s, _ = _ckpt_ct(rng, 640, K)
    w = pkg.QWeight(t_(p, dev), t_(s, dev).to(tdt), None, "ct", 32, 640, K)
    x = t_(make_x(rng, (M, K), xdt), dev)
    nw = torch.from_numpy(rng.uniform(0.5, 1.5, K).astype(np.float32)).to(dev, tdt)
    xn = pkg.rmsnorm(x, nw, 1e-6)
    ref_xn = i4ref.rmsnorm(np.asarray(host(x), np.float64), np.asarray(host(nw), np.float64),
                           1e-6, "bf16" if xdt == "bf16" else "f16")
    ulp = np.abs(ref_xn) * (2.0 ** (-7 if xdt == "bf16" else -10)) + 1e-7
    assert np.all(np.abs(np.asarray(host(xn), np.float64) - ref_xn) <= 2 * ulp)
    want = pkg.linear(xn, w)
    got = pkg.rmsnorm_linear(x, nw, 1e-6, w)
    assert torch.equal(got, want)


def _ckpt_ct(rng, N, K, G=32):
    from tests import _gen

    p, s, _ = _gen.ct_weight(rng, 1, N, K, G, sdt=np.float32)
    return p, s, None


@pytest.mark.parametrize("xdt,nh,nkv,pos", [("f16", 8, 8, 0), ("f16", 16, 4, 70), ("bf16", 8, 4, 129),
                                            ("bf16", 4, 2, 5)])
def test_attn_decode_head_layouts(pkg, dev, xdt, nh, nkv, pos):
    """i4_attn_decode alone for 1, 2, 4 query heads per kv head, fp16 and bf16, against the
    fp32 reference; cache rows [0, pos) preset, rows past pos NaN (never written rows must not
    reach the output)."""
    from tests import _thinker_ref

    rng = np.random.default_rng(200 + nh + pos)
    tdt = torch.bfloat16 if xdt == "bf16" else torch.float16
    hd, max_len = 128, 256
    qkv = torch.from_numpy(rng.standard_normal((nh + 2 * nkv) * hd).astype(np.float32)).to(dev, tdt)
    qn = torch.from_numpy(rng.uniform(0.5, 1.5, hd).astype(np.float32)).to(dev, tdt)
    kn = torch.from_numpy(rng.uniform(0.5, 1.5, hd).astype(np.float32)).to(dev, tdt)
    kc = torch.full((nkv, max_len, hd), float("nan"), dtype=tdt, device=dev)
    vc = torch.full((nkv, max_len, hd), float("nan"), dtype=tdt, device=dev)
    kc[:, :pos] = torch.randn(nkv, pos, hd, device=dev).to(tdt)
    vc[:, :pos] = torch.randn(nkv, pos, hd, device=dev).to(tdt)
    inv = pkg.rope_inv_freq(hd, 1e6)
    out = pkg.attn_decode(qkv, nh, nkv, qn, kn, 1e-6, inv, pos, kc, vc)
    # reference: the projections are the identity here, so feed q/k/v through W = I
    x = qkv.float().cpu()
    q, k, v = x[:nh * hd].view(nh, hd), x[nh * hd:(nh + nkv) * hd].view(nkv, hd), x[(nh + nkv) * hd:].view(nkv, hd)
    q = _thinker_ref.rmsnorm(q, qn.float().cpu(), 1e-6)
    k = _thinker_ref.rmsnorm(k, kn.float().cpu(), 1e-6)
    f = pos * inv
    emb = torch.cat((f, f))
    q = q * emb.cos() + _thinker_ref.rotate_half(q) * emb.sin()
    k = k * emb.cos() + _thinker_ref.rotate_half(k) * emb.sin()
    K = torch.cat((kc[:, :pos].float().cpu(), k[:, None]), 1).repeat_interleave(nh // nkv, 0)
    V = torch.cat((vc[:, :pos].float().cpu(), v[:, None]), 1).repeat_interleave(nh // nkv, 0)
    p = torch.softmax(torch.einsum("hd,hsd->hs", q, K) / hd ** 0.5, -1)
    ref = torch.einsum("hs,hsd->hd", p, V).reshape(-1).numpy()
    got = out.float().cpu().numpy()
    assert np.all(np.isfinite(got))
    assert i4ref.rel_err(got, ref) <= TOL
    # this token's k and v landed in row pos
    assert i4ref.rel_err(kc[:, pos].float().cpu().numpy(), k.numpy()) <= TOL
    assert torch.equal(vc[:, pos], v.to(tdt).to(dev))


@pytest.mark.parametrize("xdt,nh,nkv,pos,N,G", [("bf16", 32, 4, 1000, 2048, 32),
                                                 ("f16", 32, 4, 63, 2048, 128),
                                                 ("f16", 16, 4, 70, 1024, 32),
                                                 ("bf16", 8, 8, 0, 2048, 64)])
def test_attn_decode_o_equals_attention_then_o_proj(pkg, dev, xdt, nh, nkv, pos, N, G):
    """i4_attn_decode_o (head merge and o_proj in one launch, the o_proj workgroups taking
    the merged heads over inside it) equals i4_attn_decode followed by i4_linear with the
    residual as bias, bit for bit: the Thinker's 32 / 4 heads at context 1000 and at the
    last row of a chunk, other head layouts and groups, host and device positions; a device
    position past the cache gives NaN."""
    rng = np.random.default_rng(300 + nh + pos)
    tdt = torch.bfloat16 if xdt == "bf16" else torch.float16
    hd, max_len = 128, 1024
    K = nh * hd
    from tests import _gen

    p, sc, z = _gen.ct_weight(rng, 1, N, K, G, zeros=G != 32)
    w = pkg.QWeight(t_(p, dev), t_(sc, dev).to(tdt), None if z is None else t_(z, dev), "ct",
                    G, N, K)
    qkv = torch.from_numpy(rng.standard_normal((nh + 2 * nkv) * hd).astype(np.float32)).to(dev, tdt)
    qn = torch.from_numpy(rng.uniform(0.5, 1.5, hd).astype(np.float32)).to(dev, tdt)
    kn = torch.from_numpy(rng.uniform(0.5, 1.5, hd).astype(np.float32)).to(dev, tdt)
    cache = [torch.randn(nkv, max_len, hd, device=dev).to(tdt) for _ in range(2)]
    res = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(dev, tdt)
    inv = pkg.rope_inv_freq(hd, 1e6)
    kc, vc = cache[0].clone(), cache[1].clone()
    a = pkg.attn_decode(qkv, nh, nkv, qn, kn, 1e-6, inv, pos, kc, vc)
    want = pkg.linear(a.view(1, -1), w, bias=res).view(-1)
    ws = pkg.Workspace()
    for dev_pos in (False, True):
        kc2, vc2 = cache[0].clone(), cache[1].clone()
        pp = torch.full((1,), pos, dtype=torch.int32, device=dev) if dev_pos else pos
        if ws.buf is not None:
            ws.buf.fill_(0xA5)  # the status word is rewritten by every call
        got = pkg.attn_decode_o(qkv, nh, nkv, qn, kn, 1e-6, inv, pp, kc2, vc2, w, res,
                                workspace=ws)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want), dev_pos
        assert torch.equal(kc2, kc) and torch.equal(vc2, vc)
        assert pkg.ops.attn_status(ws, nh, hd, max_len) == 0
    # the o_proj GEMV itself against the oracle's fp32 product on the same attention output
    W = i4ref.ct_dequant(p, w.scale.float().cpu().numpy(), K, G, zeros=z)[0]
    ref = np.asarray(host(a), np.float64) @ W.T.astype(np.float64) + np.asarray(host(res), np.float64)
    assert i4ref.rel_err(np.asarray(host(want), np.float64), ref) <= TOL
    bad = torch.full((1,), max_len, dtype=torch.int32, device=dev)
    kc3 = cache[0].clone()
    got = pkg.attn_decode_o(qkv, nh, nkv, qn, kn, 1e-6, inv, bad, kc3, cache[1].clone(), w, res)
    torch.cuda.synchronize()
    assert torch.isnan(got.float()).all()
    assert torch.equal(kc3, cache[0])


@pytest.mark.parametrize("xdt,H,nh,nkv,G", [("f16", 2048, 32, 4, 32),    # the Thinker's
                                             ("bf16", 2048, 32, 4, 128),
                                             ("bf16", 1024, 16, 8, 32),   # 8 lanes per row
                                             ("f16", 1024, 8, 2, 64)])
def test_attn_decode_qkv_o_equals_norm_linear_then_attn_o(pkg, dev, xdt, H, nh, nkv, G):
    """i4_attn_decode_qkv_o (the input norm + q|k|v GEMV inside the attention chunk launch,
    its rows handed over as tagged words, where the GEMV has 32 lanes per row; three
    launches otherwise) equals i4_rmsnorm_linear + i4_attn_decode_o(residual = h) bit for
    bit, output and caches: consecutive tokens on one workspace (each call must take its
    own rows, not the previous call's), host and device positions, then one hipGraph
    replayed for several tokens with other work between the replays."""
    rng = np.random.default_rng(700 + H + nh + G)
    tdt = torch.bfloat16 if xdt == "bf16" else torch.float16
    hd, max_len = 128, 1024
    N = (nh + 2 * nkv) * hd
    from tests import _gen

    def weight(n, k):
        p, sc, z = _gen.ct_weight(rng, 1, n, k, G, zeros=G == 64)
        return pkg.QWeight(t_(p, dev), t_(sc, dev).to(tdt), None if z is None else t_(z, dev),
                           "ct", G, n, k)

    qw, ow = weight(N, H), weight(H, nh * hd)
    vec = lambda n: torch.from_numpy(rng.uniform(0.5, 1.5, n).astype(np.float32)).to(dev, tdt)
    nw, qn, kn = vec(H), vec(hd), vec(hd)
    inv = pkg.rope_inv_freq(hd, 1e6)
    cache0 = [torch.randn(nkv, max_len, hd, device=dev).to(tdt) for _ in range(2)]
    xs = [torch.from_numpy(rng.standard_normal(H).astype(np.float32)).to(dev, tdt)
          for _ in range(6)]

    def want_of(x, pos, kc, vc):
        qkv = pkg.rmsnorm_linear(x.view(1, -1), nw, 1e-6, qw).view(-1)
        return pkg.attn_decode_o(qkv, nh, nkv, qn, kn, 1e-6, inv, pos, kc, vc, ow, x)

    kc_w, vc_w = cache0[0].clone(), cache0[1].clone()
    kc_g, vc_g = cache0[0].clone(), cache0[1].clone()
    ws = pkg.Workspace()
    positions = (517, 518, 519, 63, 64, 1000)
    for i, pos in enumerate(positions):
        want = want_of(xs[i], pos, kc_w, vc_w)
        pp = torch.full((1,), pos, dtype=torch.int32, device=dev) if i % 2 else pos
        got = pkg.ops.attn_decode_qkv_o(xs[i], nw, 1e-6, qw, nh, nkv, qn, kn, inv, pp, kc_g,
                                        vc_g, ow, workspace=ws)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want), pos
        assert torch.equal(kc_g, kc_w) and torch.equal(vc_g, vc_w)
        assert pkg.ops.attn_status(ws, nh, hd, max_len) == 0
    # a captured graph: every replay runs with the tag its own epoch gives
    h_buf = xs[0].clone()
    pos_buf = torch.zeros(1, dtype=torch.int32, device=dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = pkg.ops.attn_decode_qkv_o(h_buf, nw, 1e-6, qw, nh, nkv, qn, kn, inv, pos_buf,
                                        kc_g, vc_g, ow, workspace=ws)
    for i, pos in enumerate((200, 201, 202, 203)):
        x = xs[(i + 2) % len(xs)] * (1 + i)
        h_buf.copy_(x)
        pos_buf.fill_(pos)
        g.replay()
        want = want_of(x, pos, kc_w, vc_w)
        torch.cuda.synchronize()
        assert torch.equal(out, want), pos
        assert torch.equal(kc_g, kc_w) and torch.equal(vc_g, vc_w)
        _ = (torch.randn(256, 256, device=dev) @ torch.randn(256, 256, device=dev)).sum().item()
    assert pkg.ops.attn_status(ws, nh, hd, max_len) == 0


def _synthetic_layer(pkg, dev, tdt, H, E, I, top_k, nh, nkv, max_len, renorm, seed,
                     qkv_scales=None):
    """A Thinker decoder layer of random CT int4 weights (g32, scales in the activation
    dtype or qkv_scales for q|k|v), router ~ N(0, 0.05), norm weights in [0.8, 1.2), cache
    rows random."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)

    def ct(e, N, K, sdt=tdt):
        p = torch.randint(-2**31, 2**31, (e, N, K // 8), dtype=torch.int32, device=dev,
                          generator=gen)
        sc = (torch.rand(e, N, K // 32, device=dev, generator=gen) * 0.018 + 0.002).to(sdt)
        return pkg.QWeight(p, sc, None, "ct", 32, N, K)

    def vec(n):
        return (torch.rand(n, device=dev, generator=gen) * 0.4 + 0.8).to(tdt)

    hd = 128
    qs = qkv_scales or tdt
    qkv = pkg.PackedQKV.from_qweights(ct(1, nh * hd, H, qs), ct(1, nkv * hd, H, qs),
                                      ct(1, nkv * hd, H, qs))
    o = pkg.PackedLinear.from_qweight(ct(1, H, nh * hd))
    attn = pkg.ThinkerAttention(qkv, o, vec(hd), vec(hd), vec(H), nh, nkv, hd, max_len=max_len)
    attn.k_cache.copy_(torch.randn(nkv, max_len, hd, device=dev, generator=gen).to(tdt))
    attn.v_cache.copy_(torch.randn(nkv, max_len, hd, device=dev, generator=gen).to(tdt))
    wr = (torch.randn(E, H, device=dev, generator=gen) * 0.05).to(tdt)
    moe = pkg.FusedPackedMoE.from_stacked(ct(E, 2 * I, H), ct(E, H, I), wr, top_k,
                                          norm_topk_prob=renorm, norm_weight=vec(H))
    return pkg.ThinkerDecoderLayer(attn, moe)


@pytest.mark.parametrize("xdt,H,E,I,top_k,nh,nkv,renorm", [
    ("f16", 2048, 128, 768, 8, 32, 4, True),     # the Thinker's layer
    ("bf16", 2048, 128, 768, 8, 32, 4, True),
    ("bf16", 1024, 64, 768, 4, 16, 8, False),
    ("f16", 1024, 32, 512, 6, 8, 2, True)])
def test_thinker_layer_decode_equals_attention_then_moe(pkg, dev, xdt, H, E, I, top_k, nh, nkv,
                                                        renorm):
    """i4_thinker_layer_decode (the q|k|v GEMV inside the attention chunk launch, the MoE
    router inside the head merge + o_proj launch, its waves waiting there for the o_proj
    output) equals the attention block followed by the MoE block (i4_rmsnorm_linear +
    i4_attn_decode_o, then i4_moe_forward with residual h2) bit for bit: output, both
    caches and a status word left at 0; host and device positions, the last row of a
    chunk, position 0; a device position past the cache gives NaN and leaves the cache."""
    tdt = torch.bfloat16 if xdt == "bf16" else torch.float16
    max_len = 1024
    assert pkg.thinker_layer_fits(nh, nkv, 128, max_len, H, I, E, top_k)
    layer = _synthetic_layer(pkg, dev, tdt, H, E, I, top_k, nh, nkv, max_len, renorm,
                             seed=500 + H + E + top_k)
    assert layer.fused()
    a = layer.attn
    cache0 = (a.k_cache.clone(), a.v_cache.clone())
    gen = torch.Generator(device=dev)
    gen.manual_seed(77)
    for pos in (1000, 63, 0, 517):
        x = torch.randn(1, H, device=dev, generator=gen).to(tdt)
        for dev_pos in (False, True):
            a.k_cache.copy_(cache0[0])
            a.v_cache.copy_(cache0[1])
            # the three-launch attention (not ThinkerAttention's fused entry), then the MoE
            qkv = pkg.rmsnorm_linear(x, a.input_norm_w, a.eps, a.qkv.lin.w).view(-1)
            h2 = pkg.attn_decode_o(qkv, nh, nkv, a.q_norm_w, a.k_norm_w, a.eps, a.inv_freq,
                                   pos, a.k_cache, a.v_cache, a.o_proj.w,
                                   x.view(-1)).view(x.shape)
            want = layer.moe(h2, residual=h2)
            kc, vc = a.k_cache.clone(), a.v_cache.clone()
            a.k_cache.copy_(cache0[0])
            a.v_cache.copy_(cache0[1])
            pp = torch.full((1,), pos, dtype=torch.int32, device=dev) if dev_pos else pos
            got = layer(x, pp)
            torch.cuda.synchronize()
            assert torch.isfinite(got.float()).all()
            assert torch.equal(got, want), (pos, dev_pos)
            assert torch.equal(a.k_cache, kc) and torch.equal(a.v_cache, vc)
            assert pkg.moe_status(a.workspace, 1, H, I, E, top_k) == 0
    a.k_cache.copy_(cache0[0])
    bad = torch.full((1,), max_len, dtype=torch.int32, device=dev)
    got = layer(x, bad)
    torch.cuda.synchronize()
    assert torch.isnan(got.float()).all()
    assert torch.equal(a.k_cache, cache0[0])
    assert pkg.moe_status(a.workspace, 1, H, I, E, top_k) == 0


@pytest.mark.parametrize("xdt,H,E,I,top_k,nh,nkv,qkv_scales", [
    ("f16", 2048, 128, 768, 8, 32, 4, None),           # the Thinker's layers
    ("bf16", 1024, 32, 512, 6, 8, 2, None),
    ("f16", 2048, 64, 768, 8, 32, 4, torch.float32)])  # fp32 q|k|v scales
def test_thinker_decode_step_equals_layer_by_layer(pkg, dev, xdt, H, E, I, top_k, nh, nkv,
                                                   qkv_scales):
    """i4_thinker_decode_step over three layers (one call, the hidden state between layers
    kept in its workspace) equals i4_thinker_layer_decode layer by layer, bit for bit:
    output, every cache and a status word of 0; host and device positions."""
    tdt = torch.bfloat16 if xdt == "bf16" else torch.float16
    max_len = 512
    layers = [_synthetic_layer(pkg, dev, tdt, H, E, I, top_k, nh, nkv, max_len, True,
                               seed=900 + 7 * i + H, qkv_scales=qkv_scales) for i in range(3)]
    dec = pkg.ThinkerDecoder(layers)
    assert dec.fused()
    caches = [(l.attn.k_cache.clone(), l.attn.v_cache.clone()) for l in layers]

    def restore():
        for l, (k, v) in zip(layers, caches):
            l.attn.k_cache.copy_(k)
            l.attn.v_cache.copy_(v)

    gen = torch.Generator(device=dev)
    gen.manual_seed(31)
    for pos in (300, 127, 0):
        x = torch.randn(1, H, device=dev, generator=gen).to(tdt)
        restore()
        want = dec.unfused(x, pos)
        want_kv = [(l.attn.k_cache.clone(), l.attn.v_cache.clone()) for l in layers]
        for dev_pos in (False, True):
            restore()
            pp = torch.full((1,), pos, dtype=torch.int32, device=dev) if dev_pos else pos
            got = dec.step(x, pp)
            torch.cuda.synchronize()
            assert torch.isfinite(got.float()).all()
            assert torch.equal(got, want), (pos, dev_pos)
            for l, (k, v) in zip(layers, want_kv):
                assert torch.equal(l.attn.k_cache, k) and torch.equal(l.attn.v_cache, v)
            assert pkg.moe_status(dec.workspace, 1, H, I, E, top_k) == 0


def test_decode_step_graph_with_device_position(pkg, dev, ckpt):
    """One hipGraph of the 2-layer decode step, captured with the position in device memory,
    replayed for positions 0..5 with new inputs (and other work between replays): every
    replay equals an eager step at the host position, bit for bit; a position past the cache
    gives NaN and leaves the cache as it was."""
    root, _ = ckpt
    ld = _ld(pkg)
    dec = ld.load_thinker_decoder(root, 2, dev, torch.bfloat16, max_len=128)
    twin = ld.load_thinker_decoder(root, 2, dev, torch.bfloat16, max_len=128)
    rng = np.random.default_rng(98)
    xs = [t_(make_x(rng, (1, H), "bf16"), dev) for _ in range(6)]
    h_buf = xs[0].clone()
    pos_buf = torch.zeros(1, dtype=torch.int32, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        dec.step(h_buf, pos_buf)  # warm the workspaces outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for layer in dec.layers:  # the warm-up wrote row 0: start both decoders clean
        layer.attn.k_cache.zero_()
        layer.attn.v_cache.zero_()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = dec.step(h_buf, pos_buf)
    for p in range(6):
        h_buf.copy_(xs[p])
        pos_buf.fill_(p)
        g.replay()
        want = twin.step(xs[p], p)
        torch.cuda.synchronize()
        assert torch.equal(out, want), p
        _ = (torch.randn(256, 256, device=dev) @ torch.randn(256, 256, device=dev)).sum().item()
    kc = dec.layers[0].attn.k_cache.clone()
    pos_buf.fill_(128)
    g.replay()
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
    assert torch.equal(dec.layers[0].attn.k_cache, kc)


def test_thinker_decoder_matches_transformers_layers(pkg, dev, ckpt):
    """Two Thinker decoder layers read from the checkpoint run five decode steps on the
    GPU (bf16 activations, int4 weights) against transformers' own
    Qwen3OmniMoeThinkerTextDecoderLayer x 2 (5.15, eager, fp32 on the CPU, DynamicCache,
    interleaved mRoPE at text positions) holding the same dequantised weights: the layer-2
    hidden state of every step within TOL.  This pins the composition (input norm,
    attention, residual, post-attention norm, MoE, residual) against the module the clock
    path runs (clock.py:164-172).  The router weights are scaled by 8 on both sides (exact
    in bf16) so that the 8th / 9th expert of a token stay far apart compared with the bf16
    rounding of the logits, and both sides pick the same experts."""
    M = pytest.importorskip("transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe")
    from transformers.cache_utils import DynamicCache
    from transformers.models.qwen3_omni_moe.configuration_qwen3_omni_moe import (
        Qwen3OmniMoeTextConfig,
    )

    root, truth = ckpt
    ld = _ld(pkg)
    dec = ld.load_thinker_decoder(root, 2, dev, torch.bfloat16, max_len=64)
    cfg = Qwen3OmniMoeTextConfig(
        hidden_size=H, num_attention_heads=32, num_key_value_heads=4, head_dim=128,
        rope_scaling={"interleaved": True, "mrope_interleaved": True,
                      "mrope_section": [24, 20, 20], "rope_type": "default", "type": "default"},
        rope_theta=1e6, num_hidden_layers=2, num_experts=E, num_experts_per_tok=8,
        moe_intermediate_size=I, intermediate_size=I, rms_norm_eps=1e-6, norm_topk_prob=True,
        decoder_sparse_step=1, mlp_only_layers=[])
    cfg._attn_implementation = "eager"
    cfg._experts_implementation = "eager"
    f32 = lambda a: torch.from_numpy(np.asarray(a, np.float32))
    layers = []
    with torch.no_grad():
        for li, t in enumerate(truth):
            lay = M.Qwen3OmniMoeThinkerTextDecoderLayer(cfg, li).float().eval()
            lay.input_layernorm.weight.copy_(f32(t["in_norm"]))
            lay.post_attention_layernorm.weight.copy_(f32(t["norm"]))
            for n in "qkvo":
                getattr(lay.self_attn, f"{n}_proj").weight.copy_(
                    f32(_ckpt.dense(t["attn"][f"{n}_proj"])))
            lay.self_attn.q_norm.weight.copy_(f32(t["attn"]["q_norm"]))
            lay.self_attn.k_norm.weight.copy_(f32(t["attn"]["k_norm"]))
            lay.mlp.gate.weight.copy_(f32(t["router"]) * 8)
            dgu, ddn = _dense_fns(t)
            for e in range(E):
                lay.mlp.experts.gate_up_proj[e].copy_(f32(dgu(e)))
                lay.mlp.experts.down_proj[e].copy_(f32(ddn(e)))
            layers.append(lay)
        for layer in dec.layers:
            layer.moe.router_w.mul_(8)
    rot = M.Qwen3OmniMoeThinkerTextRotaryEmbedding(cfg)
    cache = DynamicCache()
    rng = np.random.default_rng(97)
    for pos in range(5):
        x = make_x(rng, (1, H), "bf16")
        got = host(dec.step(t_(x, dev), pos))[0]
        h = torch.from_numpy(i4ref.bf16_bits_to_f32(x)).float().view(1, 1, H)
        with torch.no_grad():
            cos, sin = rot(h, torch.tensor([[pos]]))
            for lay in layers:
                h = lay(h, position_embeddings=(cos, sin), past_key_values=cache, use_cache=True)
        ref = h.view(-1).double().numpy()
        assert np.all(np.isfinite(got))
        assert i4ref.rel_err(got, ref) <= TOL, f"pos {pos}"

"""Pins of the CPU oracle (oracle/i4ref.py) -- runs on CPU.

Every oracle function is checked against at least one of: the known-answer
vectors of tests/golden/known_answers.json (written by an independent
pure-Python script), a closed form or invariant, or a library routine
(torch.topk / torch.softmax / torch's bf16 cast / numpy matmul).  The
mutation tests at the end plant plausible mistakes in the oracle and show
that these checks catch them.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import i4ref
from tests import _gen

GOLD = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())


# ---------------------------------------------------------------- packing
def check_ct_words():
    for case in GOLD["ct_words"]:
        w = np.array([case["word"]], dtype=np.int32)
        assert i4ref.ct_nibbles(w).tolist() == case["nibbles"]
        assert i4ref.ct_pack(np.array(case["nibbles"])).tolist() == [case["word"]]
    rw = np.array(GOLD["random_words"]["words"], dtype=np.int32)
    assert i4ref.ct_nibbles(rw).reshape(-1, 8).tolist() == GOLD["random_words"]["ct_nibbles"]


def check_awq_words():
    for case in GOLD["awq_words"]:
        w = np.array([case["word"]], dtype=np.int32)
        assert i4ref.awq_nibbles(w).tolist() == case["cols"]
        assert i4ref.awq_pack(np.array(case["cols"])).tolist() == [case["word"]]
    rw = np.array(GOLD["random_words"]["words"], dtype=np.int32)
    assert i4ref.awq_nibbles(rw).reshape(-1, 8).tolist() == GOLD["random_words"]["awq_cols"]


def test_ct_known_words():
    check_ct_words()


def test_awq_known_words():
    check_awq_words()
    # the published AutoAWQ example: columns 0..7 -> 0x75316420
    assert int(i4ref.awq_pack(np.arange(8))[0]) == 0x75316420


def test_brute_force_every_value_every_position():
    for pos in range(8):
        for v in range(16):
            q = np.zeros(8, dtype=np.int64)
            q[pos] = v
            w = int(i4ref.ct_pack(q)[0]) & 0xFFFFFFFF
            assert w == v << (4 * pos)
            assert i4ref.ct_nibbles(np.array([w]).astype(np.uint32).view(np.int32))[pos] == v
            wa = int(i4ref.awq_pack(q)[0]) & 0xFFFFFFFF
            assert wa == v << (4 * i4ref.AWQ_SLOT[pos])


def test_round_trips():
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, size=(3, 5, 64))
    assert np.array_equal(i4ref.ct_nibbles(i4ref.ct_pack(q)), q)
    assert np.array_equal(i4ref.awq_nibbles(i4ref.awq_pack(q)), q)
    w = rng.integers(-2**31, 2**31, size=(4, 7), dtype=np.int64).astype(np.int32)
    assert np.array_equal(i4ref.ct_pack(i4ref.ct_nibbles(w)), w)
    assert np.array_equal(i4ref.awq_pack(i4ref.awq_nibbles(w)), w)


def test_unpack4_is_signed_nibble():
    rng = np.random.default_rng(1)
    w = rng.integers(-2**31, 2**31, size=(2, 3, 4), dtype=np.int64).astype(np.int32)
    s = i4ref.unpack4(w, 32)
    assert s.min() >= -8 and s.max() <= 7
    assert np.array_equal(s, i4ref.ct_nibbles(w).astype(np.int32) - 8)
    # out_cols truncates like the reference's [..., :out_cols]
    assert np.array_equal(i4ref.unpack4(w, 20), s[..., :20])


def test_unpack_matches_torch_bit_ops():
    """The reference's own torch expression (fused_packed_moe.py:62-65) on CPU tensors."""
    rng = np.random.default_rng(2)
    w = rng.integers(-2**31, 2**31, size=(3, 16), dtype=np.int64).astype(np.int32)
    t = torch.from_numpy(w)
    shifts = torch.arange(8, dtype=torch.int32) * 4
    u = ((t.unsqueeze(-1) >> shifts) & 0xF).flatten(-2) - 8
    assert np.array_equal(u.numpy(), i4ref.unpack4(w, 128))


# ---------------------------------------------------------------- dequant + gemv
def test_ct_gemv_known_answer():
    g = GOLD["ct_gemv"]
    packed = np.array(g["packed"], dtype=np.int32)[None]
    scale = np.array(g["scale"])[None]
    W = i4ref.ct_dequant(packed, scale, g["K"], g["group"])
    y = i4ref.dq_gemv(np.array(g["x"]), W, [0])[0]
    np.testing.assert_allclose(y, g["y"], rtol=0, atol=1e-12)


def test_awq_gemv_known_answer():
    g = GOLD["awq_gemv"]
    W = i4ref.awq_dequant(np.array(g["qweight"], np.int32)[None], np.array(g["qzeros"], np.int32)[None],
                          np.array(g["scales"])[None], g["group"])
    y = i4ref.dq_gemv(np.array(g["x"]), W, [0])[0]
    np.testing.assert_allclose(y, g["y"], rtol=0, atol=1e-12)


def test_zero_point_8_reduces_to_symmetric():
    rng = np.random.default_rng(3)
    E, N, K, G = 2, 16, 256, 64
    p = rng.integers(-2**31, 2**31, size=(E, N, K // 8), dtype=np.int64).astype(np.int32)
    s = rng.uniform(0.002, 0.02, size=(E, N, K // G))
    z8 = i4ref.ct_pack(np.full((E, N, 8), 8))
    np.testing.assert_array_equal(i4ref.ct_dequant(p, s, K, G, zeros=z8), i4ref.ct_dequant(p, s, K, G))


def test_ct_awq_layout_equivalence():
    """One logical int4 matrix packed both ways dequantises identically; awq_to_ct agrees."""
    rng = np.random.default_rng(4)
    E, N, K, G = 2, 24, 256, 128
    Q = rng.integers(0, 16, size=(E, N, K))
    Z = rng.integers(0, 16, size=(E, N, K // G))
    S = rng.uniform(0.002, 0.02, size=(E, N, K // G)).astype(np.float16)
    qw = i4ref.awq_pack(np.swapaxes(Q, 1, 2))                 # [E, K, N/8]
    qz = i4ref.awq_pack(np.swapaxes(Z, 1, 2))                 # [E, NG, N/8]
    sc = np.swapaxes(S, 1, 2)                                 # [E, NG, N]
    W_awq = i4ref.awq_dequant(qw, qz, sc, G)
    zpad = np.concatenate([Z, np.zeros((E, N, 6), np.int64)], axis=-1)
    W_ct = i4ref.ct_dequant(i4ref.ct_pack(Q), S, K, G, zeros=i4ref.ct_pack(zpad))
    np.testing.assert_array_equal(W_awq, W_ct)
    cp, cs, cz = i4ref.awq_to_ct(qw, qz, sc, G)
    np.testing.assert_array_equal(i4ref.ct_dequant(cp, cs, K, G, zeros=cz), W_awq)
    # direct element check against the definition
    e, n, k = 1, 5, 200
    assert W_awq[e, n, k] == (Q[e, n, k] - Z[e, n, k // G]) * np.float64(S[e, n, k // G])


def test_tile_index_closed_form():
    """Nibble i of tile element [e, b, s, r, 4j + t] is column 128s + 32t + 8j +
    (0, 2, 4, 6, 1, 3, 5, 7)[i] of row 16b + r, checked against CT nibbles taken
    with a direct bit expression (nibble c of CT word m is column 8m + c)."""
    rng = np.random.default_rng(17)
    E, N, K = 2, 32, 256
    p = _gen.words(rng, (E, N, K // 8))
    Q = np.stack([(p.astype(np.int64) >> (4 * c)) & 15 for c in range(8)], axis=-1).reshape(E, N, K)
    sc = np.arange(E * N * 2, dtype=np.float32).reshape(E, N, 2)
    t, ts, tz = i4ref.tile_pack(p, sc, sc.astype(np.int32))
    assert t.shape == (E, N // 16, K // 128, 16, 16) and ts.shape == (E, N // 16, 2, 16)
    order = (0, 2, 4, 6, 1, 3, 5, 7)
    for e, b, s_, r, j, tt in [(0, 0, 0, 0, 0, 0), (1, 1, 1, 15, 3, 3), (0, 1, 0, 7, 2, 1),
                               (1, 0, 1, 3, 1, 2)]:
        word = int(t[e, b, s_, r, 4 * j + tt]) & 0xFFFFFFFF
        for i in range(8):
            col = 128 * s_ + 32 * tt + 8 * j + order[i]
            assert (word >> (4 * i)) & 15 == Q[e, 16 * b + r, col]
    # nibbles i and i + 4 are adjacent columns: one (lo, hi) half pair of the decode
    assert all(order[i + 4] == order[i] + 1 for i in range(4))
    for e, b, g, r in [(0, 0, 0, 0), (1, 1, 1, 15), (0, 1, 0, 9)]:
        assert ts[e, b, g, r] == sc[e, 16 * b + r, g] and tz[e, b, g, r] == int(sc[e, 16 * b + r, g])
    # a lane (r, j) of one 16-byte load holds word j of the four chunks of a superchunk
    lane = t[0, 0, 1, 5, 8:12]
    assert list(i4ref.deinterleave_words(lane)) == [p[0, 5, 4 * (4 + c) + 2] for c in range(4)]
    # the CT nibble order itself would put column 8m + 1 in slot 1, not slot 4
    assert not np.array_equal(t.reshape(-1)[:64], i4ref.deinterleave_words(t.reshape(-1)[:64]))


def test_interleave_round_trip_brute_force():
    """Every value at every nibble slot moves to the slot the AWQ order names."""
    for c in range(8):
        for v in range(16):
            w = np.array([v << (4 * c)], dtype=np.int64).astype(np.uint32).view(np.int32)
            out = int(i4ref.interleave_words(w)[0]) & 0xFFFFFFFF
            assert out == v << (4 * (0, 2, 4, 6, 1, 3, 5, 7).index(c))
            assert i4ref.deinterleave_words(i4ref.interleave_words(w))[0] == w[0]


def test_tile_round_trip_and_dequant():
    rng = np.random.default_rng(5)
    E, N, K, G = 3, 48, 384, 128
    p = _gen.words(rng, (E, N, K // 8))
    sc = rng.uniform(0.002, 0.02, (E, N, K // G)).astype(np.float16)
    z = _gen.words(rng, (E, N, 1))
    t = i4ref.tile_pack(p, sc, z)
    back = i4ref.tile_unpack(*t)
    np.testing.assert_array_equal(back[0], p)
    np.testing.assert_array_equal(back[1], sc)
    np.testing.assert_array_equal(back[2], z)
    assert i4ref.tile_unpack(*i4ref.tile_pack(p, sc))[2] is None


def test_dq_gemv_vs_loops():
    rng = np.random.default_rng(5)
    E, N, K = 3, 5, 64
    W = rng.standard_normal((E, N, K))
    x1 = rng.standard_normal(K)
    x2 = rng.standard_normal((2, K))
    sel = [2, 0]
    y1 = i4ref.dq_gemv(x1, W, sel)
    y2 = i4ref.dq_gemv(x2, W, sel)
    for j, e in enumerate(sel):
        for r in range(N):
            assert abs(y1[j, r] - sum(W[e, r, c] * x1[c] for c in range(K))) < 1e-10
            assert abs(y2[j, r] - sum(W[e, r, c] * x2[j, c] for c in range(K))) < 1e-10


# ---------------------------------------------------------------- routing
def test_route_known_answers():
    for case in GOLD["routing"]:
        sel, w = i4ref.route(np.array([case["logits"]]), case["k"])
        assert sel[0].tolist() == case["sel"]
        np.testing.assert_allclose(w[0], case["w"], rtol=1e-12)


def test_route_matches_torch_on_tie_free_rows():
    torch.manual_seed(6)
    for dt in (torch.float16, torch.bfloat16):
        lg = torch.randn(256, 128).to(dt)
        lgf = lg.float()
        # keep rows whose 8th and 9th largest logits differ
        srt = lgf.sort(dim=-1, descending=True).values
        keep = srt[:, 7] != srt[:, 8]
        p = torch.softmax(lgf, dim=-1, dtype=torch.float32)
        w_t, sel_t = torch.topk(p, 8, dim=-1)
        w_t = w_t / w_t.sum(-1, keepdim=True)
        sel, w = i4ref.route(lgf.double().numpy(), 8)
        assert keep.sum() > 200
        # index sets agree on tie-free rows (order may differ only inside exact ties above the cut)
        for t in np.nonzero(keep.numpy())[0]:
            assert set(sel[t].tolist()) == set(sel_t[t].tolist())
            np.testing.assert_allclose(np.sort(w[t]), np.sort(w_t[t].double().numpy()), rtol=2e-6)


def test_route_ties_go_to_lower_id():
    sel, w = i4ref.route(np.zeros((1, 16)), 5)
    assert sel[0].tolist() == [0, 1, 2, 3, 4]
    np.testing.assert_allclose(w[0], 0.2)


def test_route_without_renorm_is_softmax():
    lg = np.array([[0.0, 1.0, 2.0, 3.0]])
    sel, w = i4ref.route(lg, 2, renorm=False)
    p = np.exp(lg[0] - 3) / np.exp(lg[0] - 3).sum()
    np.testing.assert_allclose(w[0], p[[3, 2]])


def test_bf16_rounding_matches_torch():
    a = np.random.default_rng(7).standard_normal(10000).astype(np.float32) * 100
    a[:4] = [np.inf, -np.inf, 0.0, -0.0]
    bits = i4ref.f32_to_bf16_bits(a)
    tb = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bits, tb)
    np.testing.assert_array_equal(i4ref.round_half(a, "f16"), a.astype(np.float16).astype(np.float64))


# ---------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("dt,tdt", [("f16", torch.float16), ("bf16", torch.bfloat16)])
def test_rmsnorm_matches_torch(dt, tdt):
    """Against torch's own rms_norm followed by the transformers cast-and-scale order."""
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(16, 2048, generator=g) * 30).to(tdt)
    w = (torch.rand(2048, generator=g) + 0.5).to(tdt)
    ref = (w * torch.nn.functional.rms_norm(x.float(), (2048,), eps=1e-6).to(tdt)).float().numpy()
    got = i4ref.rmsnorm(x.float().numpy(), w.float().numpy(), 1e-6, dt)
    ulp = np.abs(ref) * (2.0 ** (-10 if dt == "f16" else -7))
    assert np.all(np.abs(got - ref) <= 2 * ulp + 1e-12)
    assert np.mean(got == ref) > 0.99


def test_rmsnorm_invariants():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((4, 256)) * 7
    ones = np.ones(256)
    y = i4ref.rmsnorm(x, ones, 1e-6, "f16")
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0, rtol=2e-3)
    np.testing.assert_array_equal(i4ref.rmsnorm(4 * x, ones, 0.0, "f16"), i4ref.rmsnorm(x, ones, 0.0, "f16"))


# ---------------------------------------------------------------- MoE layer
def _golden_moe():
    g = GOLD["moe_layer"]
    Wgu = i4ref.ct_dequant(np.array(g["gu_packed"], np.int32), np.array(g["gu_scale"]), g["H"], 32)
    Wdn = i4ref.ct_dequant(np.array(g["dn_packed"], np.int32), np.array(g["dn_scale"]), g["I"], 32)
    return g, Wgu, Wdn


def test_moe_layer_known_answer():
    g, Wgu, Wdn = _golden_moe()
    sel, w = i4ref.route(np.array([g["logits"]]), g["k"])
    assert sel[0].tolist() == g["sel"]
    out = i4ref.moe_layer(np.array([g["x"]]), sel, w, Wgu, Wdn, act_dtype=None)
    np.testing.assert_allclose(out[0], g["out"], rtol=1e-10, atol=1e-12)


def test_moe_grouped_equals_per_token():
    rng = np.random.default_rng(8)
    E, H, I, T, k = 6, 32, 16, 9, 3
    Wgu = rng.standard_normal((E, 2 * I, H)) * 0.1
    Wdn = rng.standard_normal((E, H, I)) * 0.1
    x = rng.standard_normal((T, H))
    sel, w = i4ref.route(rng.standard_normal((T, E)), k)
    a = i4ref.moe_layer(x, sel, w, Wgu, Wdn, "f16", residual=x)
    b = i4ref.moe_layer_grouped(x, sel, w, lambda e: Wgu[e], lambda e: Wdn[e], "f16", residual=x)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dt,eps", [("f16", 2.0 ** -12), ("bf16", 2.0 ** -9)])
def test_moe_expert_output_rounds_before_the_weighted_sum(dt, eps):
    """y_dtype rounds each expert's output y_e to the activation dtype and only then weights
    it (fused_packed_moe.py:262, (y.to(x.dtype) * w).sum(0)).  Two experts whose output is
    1 + eps (below half an ulp above 1 in dt) give exactly sum(w) = 1 with the rounding and
    1 + eps without it; rounding the weighted products instead would not sum to 1."""
    H, I, E = 1, 1, 2
    x = np.array([[1.0]])
    g, u = 3.0, 0.5
    a = float(i4ref.silu(np.array(g))) * u
    Wgu = np.array([[[g], [u]]] * E)                      # gate row, up row
    Wdn = np.array([[[(1.0 + eps) / a]]] * E)
    sel = np.array([[0, 1]])
    w = np.array([[0.3, 0.7]])
    plain = i4ref.moe_layer(x, sel, w, Wgu, Wdn, None)
    np.testing.assert_allclose(plain[0, 0], 1.0 + eps, rtol=1e-14)
    got = i4ref.moe_layer(x, sel, w, Wgu, Wdn, None, y_dtype=dt)
    assert got[0, 0] == pytest.approx(1.0, abs=1e-15)
    wrong = i4ref.round_half(0.3 * (1.0 + eps), dt) + i4ref.round_half(0.7 * (1.0 + eps), dt)
    assert abs(wrong - 1.0) > 1e-6  # the other placement is distinguishable
    grouped = i4ref.moe_layer_grouped(x, sel, w, lambda e: Wgu[e], lambda e: Wdn[e], None,
                                      y_dtype=dt)
    assert grouped[0, 0] == pytest.approx(1.0, abs=1e-15)


def test_moe_grouped_equals_per_token_with_output_rounding():
    rng = np.random.default_rng(18)
    E, H, I, T, k = 6, 32, 16, 9, 3
    Wgu = rng.standard_normal((E, 2 * I, H)) * 0.1
    Wdn = rng.standard_normal((E, H, I)) * 0.1
    x = rng.standard_normal((T, H))
    sel, w = i4ref.route(rng.standard_normal((T, E)), k)
    a = i4ref.moe_layer(x, sel, w, Wgu, Wdn, "bf16", residual=x, y_dtype="bf16")
    b = i4ref.moe_layer_grouped(x, sel, w, lambda e: Wgu[e], lambda e: Wdn[e], "bf16",
                                residual=x, y_dtype="bf16")
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)
    c = i4ref.moe_layer(x, sel, w, Wgu, Wdn, "bf16", residual=x)
    assert 0 < np.max(np.abs(a - c)) <= 2.0 ** -8 * np.max(np.abs(c))


@pytest.mark.parametrize("dt,tdt", [("bf16", torch.bfloat16), ("f16", torch.float16)])
def test_ref_combine_matches_the_reference_expression(dt, tdt):
    """ref_combine equals torch's own evaluation of the reference's combine,
    (y.to(x.dtype) * w.to(x.dtype)[:, None]).sum(dim=0) then + residual in the activation
    dtype (fused_packed_moe.py:199,262 and the decoder layer's residual add), bit for bit
    on many columns; dropping the weights' rounding (a plausible slip) is caught."""
    rng = np.random.default_rng(31)
    for trial in range(6):
        k, H = 8, 4096
        ys = rng.standard_normal((k, H)) * (3.0 if trial % 2 else 0.05)
        w = rng.dirichlet(np.ones(k))
        res = rng.standard_normal(H)
        y32 = torch.from_numpy(ys.astype(np.float32))
        w32 = torch.from_numpy(w.astype(np.float32))
        r16 = torch.from_numpy(res.astype(np.float32)).to(tdt)
        want = r16 + (y32.to(tdt) * w32.to(tdt).unsqueeze(-1)).sum(dim=0)
        want = want.float().double().numpy()
        got = i4ref.ref_combine(y32.double().numpy(), w32.double().numpy(), dt,
                                r16.float().double().numpy())
        np.testing.assert_array_equal(got, want)
        slip = i4ref.round_half(i4ref.round_half(
            (i4ref.round_half(y32.double().numpy(), dt) * w32.double().numpy()[:, None]).sum(0),
            dt) + r16.float().double().numpy(), dt)
        assert not np.array_equal(slip, want)


def test_moe_layer_reference_combine_is_near_the_exact_one():
    """combine="reference" (the reference's own rounding) and the float64 combine of the
    same layer differ by the 16-bit rounding of the products, the sum and the residual add
    only: within a few units in the last place of the larger of the two added terms (the
    residual and the MoE term; where they cancel the output's own ulp is smaller)."""
    rng = np.random.default_rng(32)
    E, H, I, k, T = 6, 64, 32, 4, 5
    Wgu = rng.standard_normal((E, 2 * I, H)) * 0.1
    Wdn = rng.standard_normal((E, H, I)) * 0.1
    x = i4ref.round_half(rng.standard_normal((T, H)), "bf16")
    res = i4ref.round_half(rng.standard_normal((T, H)), "bf16")
    sel = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
    w = rng.dirichlet(np.ones(k), size=T)
    exact = i4ref.moe_layer(x, sel, w, Wgu, Wdn, "bf16", residual=res, out_dtype="bf16",
                            y_dtype="bf16")
    ref = i4ref.moe_layer(x, sel, w, Wgu, Wdn, "bf16", residual=res, y_dtype="bf16",
                          combine="reference")
    scale = np.maximum(np.abs(res), np.abs(exact - res))
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(scale, 2.0 ** -14))) - 7)
    assert np.all(np.abs(ref - exact) <= 4 * ulp)
    assert not np.array_equal(ref, exact)


def test_cpu_baseline_matches_the_oracle():
    """The timed CPU baseline (oracle/cpu_baseline.py, the reference's CPU expert path in torch
    fp32) computes the oracle's MoE layer on seeded AWQ inputs, and its reference_gemv
    restatement the oracle's GEMV: the figure it times is a figure of the right computation."""
    import torch

    from oracle import cpu_baseline as cb

    rng = np.random.default_rng(19)
    E, H, I, G, T, k = 12, 256, 128, 128, 5, 4

    def awq(K, N):
        return (rng.integers(-2**31, 2**31, (E, K, N // 8), dtype=np.int64).astype(np.int32),
                rng.integers(-2**31, 2**31, (E, K // G, N // 8), dtype=np.int64).astype(np.int32),
                rng.uniform(0.002, 0.02, (E, K // G, N)).astype(np.float16))

    g, u, d = awq(H, I), awq(H, I), awq(I, H)
    wr = (rng.standard_normal((E, H)) * 0.3).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = x.astype(np.float64) @ wr.astype(np.float64).T
    srt = np.sort(logits, axis=1)[:, ::-1]
    assert np.min(srt[:, k - 1] - srt[:, k]) > 1e-3  # no near-tie at the top-k cut
    sel, w = i4ref.route(logits, k)
    Wgu = np.concatenate([i4ref.awq_dequant(*g, G), i4ref.awq_dequant(*u, G)], axis=1)
    Wdn = i4ref.awq_dequant(*d, G)
    ref = i4ref.moe_layer(x, sel, w, Wgu, Wdn, None)
    tt = lambda p: tuple(torch.from_numpy(a) for a in p)
    got = cb.moe_layer(torch.from_numpy(x), torch.from_numpy(wr), tt(g), tt(u), tt(d), top_k=k,
                       group=G).numpy()
    assert i4ref.rel_err(got, ref) <= 1e-5
    np.testing.assert_array_equal(cb.awq_unpack(torch.from_numpy(g[0])).numpy(),
                                  i4ref.awq_nibbles(g[0]))
    y = cb.gemv(torch.from_numpy(x[0]), *(torch.from_numpy(a[3]) for a in g), group=G).numpy()
    assert i4ref.rel_err(y, i4ref.dq_gemv(x[0], i4ref.awq_dequant(*g, G), [3])[0]) <= 1e-5


def test_moe_identical_experts_ignore_routing():
    """With every expert equal and renormalised weights, routing cannot matter."""
    rng = np.random.default_rng(9)
    E, H, I, T = 5, 16, 8, 4
    Wg = rng.standard_normal((2 * I, H))
    Wd = rng.standard_normal((H, I))
    Wgu, Wdn = np.stack([Wg] * E), np.stack([Wd] * E)
    x = rng.standard_normal((T, H))
    sel, w = i4ref.route(rng.standard_normal((T, E)), 3)
    out = i4ref.moe_layer(x, sel, w, Wgu, Wdn, None)
    gu = x @ Wg.T
    ref = (i4ref.silu(gu[:, :I]) * gu[:, I:]) @ Wd.T
    np.testing.assert_allclose(out, ref, rtol=1e-10)


# ---------------------------------------------------------------- mutation tests
def test_mutation_wrong_awq_order_is_caught(monkeypatch):
    monkeypatch.setattr(i4ref, "AWQ_ORDER", tuple(range(8)))
    monkeypatch.setattr(i4ref, "AWQ_SLOT", tuple(range(8)))
    with pytest.raises(AssertionError):
        check_awq_words()


def test_mutation_wrong_nibble_shift_is_caught(monkeypatch):
    real = i4ref.ct_nibbles

    def shifted(packed, cols=None):  # nibble i read from bits 4i+1: a plausible off-by-one
        u = np.asarray(packed).astype(np.int64) & 0xFFFFFFFF
        q = ((u[..., None] >> (np.arange(8) * 4 + 1)) & 0xF).astype(np.uint8)
        q = q.reshape(*u.shape[:-1], u.shape[-1] * 8)
        return q if cols is None else q[..., :cols]

    monkeypatch.setattr(i4ref, "ct_nibbles", shifted)
    with pytest.raises(AssertionError):
        check_ct_words()
    monkeypatch.setattr(i4ref, "ct_nibbles", real)


def test_mutation_missing_renorm_or_wrong_tie_rule_is_caught(monkeypatch):
    real = i4ref.route

    def no_renorm(logits, k, renorm=True):
        return real(logits, k, renorm=False)

    monkeypatch.setattr(i4ref, "route", no_renorm)
    with pytest.raises(AssertionError):
        test_route_known_answers()
    monkeypatch.setattr(i4ref, "route", real)

    def high_id_ties(logits, k):
        lg = np.asarray(logits, np.float64)
        E = lg.shape[-1]
        return np.stack([np.lexsort((-np.arange(E), -row))[:k] for row in lg.reshape(-1, E)])

    monkeypatch.setattr(i4ref, "topk_sel", high_id_ties)
    with pytest.raises(AssertionError):
        test_route_known_answers()


def test_mutation_wrong_zero_point_is_caught():
    g = GOLD["ct_gemv"]
    packed = np.array(g["packed"], dtype=np.int32)[None]
    z7 = i4ref.ct_pack(np.full((1, g["N"], 8), 7))
    W = i4ref.ct_dequant(packed, np.array(g["scale"])[None], g["K"], g["group"], zeros=z7)
    y = i4ref.dq_gemv(np.array(g["x"]), W, [0])[0]
    assert np.max(np.abs(y - np.array(g["y"]))) > 1e-3

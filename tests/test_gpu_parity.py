"""Parity of the HIP path (libi4moe, called through its C ABI) with the CPU oracle.

Bar: unpacked nibbles, repacked words and routing indices bit-exact; floating
outputs within max|got - ref| <= 2e-2 * max|ref| (fp32 accumulation on the
GPU, float64 in the oracle), and the MoE blocks' own term (output minus
residual) within 1e-3 (fp16) / 4e-3 (bf16) of its maximum, on top of half an
ulp of the rounded output.  Each expert's output is rounded to the activation
dtype before the weighted sum (the reference's y.to(x.dtype)), in the kernels
and the oracle alike; where the GPU's fp32 value and the oracle's fp64 value
fall on two sides of a rounding boundary the term moves by w_j times one step
of that dtype (relative step up to 2^-10 in fp16, 2^-7 in bf16), which is
what the two bars leave room for.  Inputs are seeded; sizes are the workload's own
(hidden 2048, expert FFN 768, 128 experts, top-8) wherever the oracle finishes
in seconds.
"""
from __future__ import annotations

import ctypes
import zlib

import numpy as np
import pytest
import torch

from oracle import i4ref
from tests import _gen

pytestmark = pytest.mark.gpu
TOL = 2e-2
MOE_TOL = {"f16": 1e-3, "bf16": 4e-3}  # on the MoE term, beyond the output's own rounding


def half_ulp(v, xdt):
    """Half an ulp of fp16 / bf16 values v (the rounding error of the stored output)."""
    m = np.maximum(np.abs(np.asarray(v, np.float64)), 2.0 ** -14)
    return 2.0 ** (np.floor(np.log2(m)) - (11 if xdt == "f16" else 8))


def check_moe_term(got, ref_moe, residual, xdt):
    """got = round(residual + moe): the MoE term within MOE_TOL of max|moe| once the output's
    rounding (half an ulp of got) is allowed for.  Returns the term's relative error."""
    res = 0.0 if residual is None else np.asarray(residual, np.float64)
    err = np.abs(got - (res + ref_moe)) - half_ulp(got, xdt)
    rel = float(max(np.max(err), 0.0) / np.max(np.abs(ref_moe)))
    assert rel <= MOE_TOL[xdt], f"MoE term error {rel:.2e} > {MOE_TOL[xdt]:.0e}"
    return rel


# ---------------------------------------------------------------- helpers
def t_(a, dev):
    """numpy -> device tensor; uint16 arrays are bf16 bit patterns."""
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def f_(a):
    """numpy values as float64 (bf16 bit patterns decoded)."""
    if a.dtype == np.uint16:
        return i4ref.bf16_bits_to_f32(a).astype(np.float64)
    return np.asarray(a, np.float64)


def host(t):
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.float().numpy().astype(np.float64)
    return t.numpy()


def make_x(rng, shape, xdt):
    v = rng.standard_normal(shape).astype(np.float32)
    if xdt == "bf16":
        return i4ref.f32_to_bf16_bits(v)
    return v.astype(np.float16)


def half_name(xdt):
    return "bf16" if xdt == "bf16" else "f16"


def sdt_np(sdt):
    return {"f16": np.float16, "bf16": "bf16", "f32": np.float32}[sdt]


# ---------------------------------------------------------------- unpack / repack
@pytest.mark.parametrize("layout", ["ct", "awq"])
def test_unpack_bit_exact(pkg, dev, layout):
    rng = np.random.default_rng(11)
    E, N, K, G = 3, 40, 256, 32
    if layout == "ct":
        p, s, _ = _gen.ct_weight(rng, E, N, K, G)
        w = pkg.QWeight(t_(p, dev), t_(s, dev), None, "ct", G, N, K)
        ref = i4ref.ct_nibbles(p, K)
    else:
        qw, qz, sc = _gen.awq_weight(rng, E, K, N, G)
        w = pkg.QWeight(t_(qw, dev), t_(sc, dev), t_(qz, dev), "awq", G, N, K)
        ref = np.swapaxes(i4ref.awq_nibbles(qw), 1, 2)
    got = pkg.unpack_nibbles(w).cpu().numpy()
    np.testing.assert_array_equal(got, ref)
    if layout == "ct":  # the reference's signed unpack4
        np.testing.assert_array_equal(pkg.unpack4(w.packed, K).cpu().numpy(), i4ref.unpack4(p, K))


@pytest.mark.parametrize("K,N,G", [(2048, 768, 128), (768, 2048, 128), (256, 64, 32), (512, 48, 64)])
def test_repack_awq_to_ct_bit_exact(pkg, dev, K, N, G):
    rng = np.random.default_rng(12)
    E = 2
    qw, qz, sc = _gen.awq_weight(rng, E, K, N, G)
    w = pkg.QWeight(t_(qw, dev), t_(sc, dev), t_(qz, dev), "awq", G, N, K)
    ct = w.to_ct()
    cp, cs, cz = i4ref.awq_to_ct(qw, qz, sc, G)
    np.testing.assert_array_equal(ct.packed.cpu().numpy(), cp)
    np.testing.assert_array_equal(ct.scale.cpu().numpy(), cs)
    np.testing.assert_array_equal(ct.zeros.cpu().numpy(), cz)


def test_repack_concatenates_gate_up(pkg, dev):
    rng = np.random.default_rng(13)
    E, K, N, G = 2, 256, 64, 128
    parts = [_gen.awq_weight(rng, E, K, N, G) for _ in range(2)]
    ws = [pkg.QWeight(t_(a, dev), t_(c, dev), t_(b, dev), "awq", G, N, K) for a, b, c in parts]
    gu = pkg.repack_awq_to_ct(ws)
    ref = np.concatenate([i4ref.awq_to_ct(a, b, c, G)[0] for a, b, c in parts], axis=1)
    np.testing.assert_array_equal(gu.packed.cpu().numpy(), ref)


def canon_zeros(z, NG):
    """CT zero words with the nibbles past the last group cleared (what a repack writes)."""
    z = np.ascontiguousarray(z).view(np.uint32).copy()
    last = NG - 8 * (z.shape[-1] - 1)
    if last < 8:
        z[..., -1] &= np.uint32((1 << (4 * last)) - 1)
    return z.view(np.int32)


@pytest.mark.parametrize("src,G,zeros", [("ct", 32, False), ("ct", 128, True), ("ct", 64, True),
                                          ("awq", 128, True)])
def test_repack_tile_bit_exact(pkg, dev, src, G, zeros):
    """CT / AWQ -> tile layout on the device equals the oracle's tile_pack of the CT words,
    and the tile weight dequantises to the same values as its source."""
    rng = np.random.default_rng(15)
    E, N, K = 3, 96, 768
    if src == "ct":
        p, s, z = _gen.ct_weight(rng, E, N, K, G, zeros=zeros)
        z = None if z is None else canon_zeros(z, -(-K // G))
        w = pkg.QWeight(t_(p, dev), t_(s, dev), None if z is None else t_(z, dev), "ct", G, N, K)
        cp, cs, cz = p, s, z
    else:
        qw, qz, s = _gen.awq_weight(rng, E, K, N, G)
        w = pkg.QWeight(t_(qw, dev), t_(s, dev), t_(qz, dev), "awq", G, N, K)
        cp, cs, cz = i4ref.awq_to_ct(qw, qz, s, G)
    t = w.to_tile()
    rp, rs, rz = i4ref.tile_pack(cp, cs, cz)
    np.testing.assert_array_equal(t.packed.cpu().numpy(), rp)
    np.testing.assert_array_equal(t.scale.cpu().numpy(), rs)
    if rz is None:
        assert t.zeros is None
    else:
        np.testing.assert_array_equal(t.zeros.cpu().numpy(), rz)
    np.testing.assert_array_equal(host(pkg.dequant(t, torch.float32)),
                                  host(pkg.dequant(w, torch.float32)))


def test_repack_tile_concatenates_gate_up(pkg, dev):
    """gate | up into one tile weight: rows [0, N) from gate, [N, 2N) from up; a symmetric
    part next to one with zeros gets explicit 8s."""
    rng = np.random.default_rng(16)
    E, K, N, G = 2, 256, 64, 128
    g = _gen.ct_weight(rng, E, N, K, G, zeros=True)
    u = _gen.ct_weight(rng, E, N, K, G, zeros=False)
    gz = canon_zeros(g[2], K // G)
    ws = [pkg.QWeight(t_(g[0], dev), t_(g[1], dev), t_(gz, dev), "ct", G, N, K),
          pkg.QWeight(t_(u[0], dev), t_(u[1], dev), None, "ct", G, N, K)]
    gu = pkg.repack_tile(ws)
    u_z = np.full((E, N, 1), 0x88, dtype=np.int32)  # two groups, zero point 8
    rp, rs, rz = i4ref.tile_pack(np.concatenate([g[0], u[0]], axis=1),
                                 np.concatenate([g[1], u[1]], axis=1),
                                 np.concatenate([gz, u_z], axis=1))
    np.testing.assert_array_equal(gu.packed.cpu().numpy(), rp)
    np.testing.assert_array_equal(gu.scale.cpu().numpy(), rs)
    np.testing.assert_array_equal(gu.zeros.cpu().numpy(), rz)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_dequant_matches_oracle(pkg, dev, out_dtype):
    rng = np.random.default_rng(14)
    E, N, K, G = 2, 32, 512, 128
    p, s, z = _gen.ct_weight(rng, E, N, K, G, zeros=True)
    w = pkg.QWeight(t_(p, dev), t_(s, dev), t_(z, dev), "ct", G, N, K)
    got = host(pkg.dequant(w, out_dtype))
    ref = i4ref.ct_dequant(p, f_(s), K, G, zeros=z)
    if out_dtype == torch.float16:
        ref = ref.astype(np.float16)
    np.testing.assert_array_equal(got.astype(np.float64), ref.astype(np.float64))


# ---------------------------------------------------------------- dequant_gemv
GEMV_SHAPES = [
    # name, E, N (rows), K, k (selected), shared x
    ("gate_up", 16, 1536, 2048, 8, True),
    ("down", 16, 2048, 768, 8, False),
    ("q_proj", 1, 4096, 2048, 1, True),
    ("k_proj", 1, 512, 2048, 1, True),
    ("o_proj", 1, 2048, 4096, 1, True),
    ("ragged", 5, 100, 96, 3, True),
    ("long_k", 2, 64, 8192, 2, False),
]
DT_COMBOS = [  # x dtype, scale dtype, zeros, group
    ("f16", "f16", True, 128),
    ("bf16", "bf16", False, 32),
    ("bf16", "f32", False, 32),
    ("f16", "bf16", True, 64),
]


@pytest.mark.parametrize("shape", GEMV_SHAPES, ids=[s[0] for s in GEMV_SHAPES])
@pytest.mark.parametrize("combo", DT_COMBOS, ids=["-".join(map(str, c)) for c in DT_COMBOS])
def test_dq_gemv_ct(pkg, dev, shape, combo):
    name, E, N, K, k, shared = shape
    xdt, sdt, zeros, G = combo
    # K % G != 0 (the ragged shape): the last group is short, ceil(K / G) scales per row
    rng = np.random.default_rng(zlib.crc32(repr((name, combo)).encode()))
    p, s, z = _gen.ct_weight(rng, E, N, K, G, zeros=zeros, sdt=sdt_np(sdt))
    sel = rng.integers(0, E, size=k).astype(np.int32)
    x = make_x(rng, (K,) if shared else (k, K), xdt)
    got = host(pkg.dequant_gemv(t_(x, dev), t_(p, dev), t_(s, dev), t_(sel, dev), group=G,
                                zeros=None if z is None else t_(z, dev)))
    W = i4ref.ct_dequant(p, f_(s), K, G, zeros=z)
    ref = i4ref.dq_gemv(f_(x), W, sel)
    assert got.shape == (k, N) and got.dtype == np.float32
    err = i4ref.rel_err(got, ref)
    assert err <= TOL, err
    assert err <= 1e-4, f"fp32-accumulation result drifted: {err:.2e}"


@pytest.mark.parametrize("K", [768, 96])
def test_dq_gemv_per_channel_scales(pkg, dev, K):
    """One scale per output row (group = K, the per-channel branch of quant/dequant.py:75-76),
    at a K that is not a power of two."""
    rng = np.random.default_rng(K)
    E, N = 3, 80
    p, s, _ = _gen.ct_weight(rng, E, N, K, K)
    assert s.shape == (E, N, 1)
    sel = np.array([2, 0], np.int32)
    x = make_x(rng, (K,), "bf16")
    got = host(pkg.dequant_gemv(t_(x, dev), t_(p, dev), t_(s, dev), t_(sel, dev), group=K))
    W = i4ref.unpack4(p, K) * f_(s)            # (q - 8) * s_row
    assert i4ref.rel_err(got, i4ref.dq_gemv(f_(x), W, sel)) <= 1e-4


def test_dq_gemv_strided_views_run_in_place(pkg, dev):
    """The up half of a stacked gate|up (a view strided between experts) runs in place and gives
    the bits of a contiguous copy; a view with cut rows is refused, not copied."""
    rng = np.random.default_rng(77)
    E, I, K, G = 6, 256, 1024, 128
    p, s, z = _gen.ct_weight(rng, E, 2 * I, K, G, zeros=True)
    pd, sd, zd = t_(p, dev), t_(s, dev), t_(z, dev)
    sel = t_(np.array([4, 1, 5], np.int32), dev)
    x = t_(make_x(rng, (K,), "f16"), dev)
    view = pkg.dequant_gemv(x, pd[:, I:], sd[:, I:], sel, group=G, zeros=zd[:, I:])
    copy = pkg.dequant_gemv(x, pd[:, I:].contiguous(), sd[:, I:].contiguous(), sel, group=G,
                            zeros=zd[:, I:].contiguous())
    assert torch.equal(view, copy)
    with pytest.raises(ValueError, match="densely"):
        pkg.dequant_gemv(x[:512], pd[:, :, :64], sd[:, :, :4], sel, group=G, zeros=zd)


@pytest.mark.parametrize("N,K,xdt,G", [(768, 2048, "f16", 128), (4096, 2048, "f16", 128),
                                       (512, 2048, "bf16", 128), (2048, 4096, "f16", 128),
                                       (64, 256, "bf16", 128), (40, 256, "f16", 128),
                                       (768, 768, "bf16", 32), (96, 8192, "f16", 64),
                                       (256, 768, "f16", 768)])
def test_dq_gemv_awq(pkg, dev, N, K, xdt, G):
    """The AWQ GEMV in place, one launch (split along K into 256-column strips at 2048 ->
    4096, 4096 -> 2048 and 8192 -> 96, K-complete workgroups elsewhere): the workload's
    shapes, column counts that are not a multiple of 32 or of 256 (a partial strip), short
    and long rows, group 32 / 64, and one scale per output row (group = K)."""
    rng = np.random.default_rng(N + K)
    E, k = 2, 2
    qw, qz, sc = _gen.awq_weight(rng, E, K, N, G)
    sel = np.array([1, 0], np.int32)
    x = make_x(rng, (K,), xdt)
    got = host(pkg.dequant_gemv(t_(x, dev), t_(qw, dev), t_(sc, dev), t_(sel, dev), group=G,
                                zeros=t_(qz, dev), layout="awq"))
    W = i4ref.awq_dequant(qw, qz, sc, G)
    ref = i4ref.dq_gemv(f_(x), W, sel)
    err = i4ref.rel_err(got, ref)
    assert err <= 1e-4, err
    assert got.shape == (k, N)


@pytest.mark.parametrize("N,K,G", [(768, 2048, 128), (4096, 2048, 128), (96, 8192, 64)])
def test_dq_gemv_awq_split_k_handover(pkg, dev, N, K, G):
    """Both AWQ kernels through the C ABI: split along K (workspace given) and K-complete
    (no workspace) each match the oracle.  The split launch's partials carry a tag of their
    call, so a workspace of random bytes (status word zeroed) serves, and five calls in a row
    on it give identical outputs (the last slice of a strip adds the partials in a fixed
    order) and leave every tag cleared and the status word 0."""
    from qwen3_omni_duplex_amd import _lib

    lb = pkg.lib()
    rng = np.random.default_rng(7 + N + K)
    E, k = 3, 3
    qw, qz, sc = _gen.awq_weight(rng, E, K, N, G)
    w = pkg.QWeight(t_(qw, dev), t_(sc, dev), t_(qz, dev), "awq", G, N, K)
    sel = np.array([2, 0, 1], np.int32)
    x = make_x(rng, (k, K), "f16")
    ref = i4ref.dq_gemv(f_(x), i4ref.awq_dequant(qw, qz, sc, G), sel)
    xd, seld = t_(x, dev), t_(sel, dev)
    cw = w.c()
    nb = lb.i4_dq_gemv_workspace_bytes(ctypes.byref(cw), k)
    assert nb > 256
    ws = torch.from_numpy(rng.integers(0, 256, nb, dtype=np.uint8)).to(dev)
    ws[:4] = 0
    stream = torch.cuda.current_stream().cuda_stream

    def run(wsp):
        y = torch.empty(k, N, dtype=torch.float32, device=dev)
        rc = lb.i4_dq_gemv(xd.data_ptr(), _lib.F16, K, ctypes.byref(cw), seld.data_ptr(), k,
                           y.data_ptr(), _lib.F32, None if wsp is None else wsp.data_ptr(),
                           0 if wsp is None else wsp.numel(), stream)
        assert rc == 0, lb.i4_strerror(rc)
        return y

    whole = host(run(None))
    assert i4ref.rel_err(whole, ref) <= 1e-4
    outs = []
    for _ in range(5):
        outs.append(run(ws))
        torch.cuda.synchronize()
    for y in outs[1:]:
        assert torch.equal(y, outs[0])
    assert i4ref.rel_err(host(outs[0]), ref) <= 1e-4
    assert pkg.ops.gemv_status(_WsView(ws)) == 0
    # every (value, tag) pair a reducer read has its tag cleared for the next call
    if N % 256 == 0:  # whole strips: every column of slices 0..P-2 was read
        strips = ws[256:].view(torch.int32).view(k, N // 256, -1, 256, 2)
        assert bool((strips[:, :, :-1, :, 1] == 0).all())
    # a workspace one byte short is refused before anything runs
    y = torch.empty(k, N, dtype=torch.float16, device=dev)
    assert lb.i4_dq_gemv(xd.data_ptr(), _lib.F16, K, ctypes.byref(cw), seld.data_ptr(), k,
                         y.data_ptr(), _lib.F16, ws.data_ptr(), nb - 1, stream) == -7


class _WsView:
    """A raw workspace tensor as the ops.Workspace the status readers take."""

    def __init__(self, buf):
        self.buf = buf


@pytest.mark.parametrize("N,K", [(4096, 2048), (2048, 4096)])
def test_dq_gemv_awq_split_k_wait_gives_up_visibly(pkg, dev, N, K):
    """The split launch's reducers run alone (i4_dq_gemv_bounded, reducers_only) with the
    bound on their wait lowered from the host: the partials never arrive, so every reducer
    gives up, writes NaN, clears its strip's tags and stores I4_ERR_HANDOFF in the status
    word; every kernel exits.  The next ordinary calls on the same workspace are correct."""
    G, k = 128, 1
    rng = np.random.default_rng(N + K)
    qw, qz, sc = _gen.awq_weight(rng, 2, K, N, G)
    w = pkg.QWeight(t_(qw, dev), t_(sc, dev), t_(qz, dev), "awq", G, N, K)
    sel = t_(np.array([1], np.int32), dev)
    x = make_x(rng, (k, K), "f16")
    ref = i4ref.dq_gemv(f_(x), i4ref.awq_dequant(qw, qz, sc, G), np.array([1]))
    ws = pkg.Workspace()
    for polls in (0, 3):
        y = pkg.ops.dequant_gemv_bounded(t_(x, dev), w, sel, polls, True, ws)
        torch.cuda.synchronize()
        assert torch.isnan(y).all()
        assert pkg.ops.gemv_status(ws) == -10
    y = pkg.ops.dequant_gemv_bounded(t_(x, dev), w, sel, 1 << 20, False, ws)
    assert i4ref.rel_err(host(y), ref) <= 1e-4
    assert pkg.ops.gemv_status(ws) == -10  # kept until the caller clears it
    ws.buf[:4] = 0
    y2 = pkg.dequant_gemv(t_(x, dev), w.packed, w.scale, sel, group=G, zeros=w.zeros,
                          layout="awq", workspace=ws)
    assert torch.equal(y2, y)
    assert pkg.ops.gemv_status(ws) == 0
    # only a split launch has reducers; a CT weight has no hand-over at all
    wc = w.to_ct()
    with pytest.raises(RuntimeError):
        pkg.ops.dequant_gemv_bounded(t_(x, dev), wc, sel, 3, True, ws)


@pytest.mark.parametrize("M", [1, 5])
@pytest.mark.parametrize("layout", ["ct", "awq"])
def test_linear(pkg, dev, M, layout):
    rng = np.random.default_rng(M)
    N, K, G = 512, 2048, 128
    if layout == "ct":
        p, s, z = _gen.ct_weight(rng, 1, N, K, G, zeros=True)
        w = pkg.QWeight(t_(p, dev), t_(s, dev), t_(z, dev), "ct", G, N, K)
        W = i4ref.ct_dequant(p, f_(s), K, G, zeros=z)[0]
    else:
        qw, qz, sc = _gen.awq_weight(rng, 1, K, N, G)
        w = pkg.QWeight(t_(qw, dev), t_(sc, dev), t_(qz, dev), "awq", G, N, K)
        W = i4ref.awq_dequant(qw, qz, sc, G)[0]
    bias = rng.standard_normal(N).astype(np.float16)
    x = make_x(rng, (M, K), "f16")
    lin = pkg.PackedLinear.from_qweight(w, t_(bias, dev), repack=False)
    got = host(lin(t_(x, dev)))
    ref = f_(x) @ W.T + f_(bias)
    assert i4ref.rel_err(got, ref) <= TOL
    if layout == "awq":  # the repacked CT+zeros copy computes the same thing
        got2 = host(pkg.PackedLinear.from_qweight(w, t_(bias, dev))(t_(x, dev)))
        assert i4ref.rel_err(got2, ref) <= TOL


@pytest.mark.parametrize("M,N", [(16, 512), (64, 512), (100, 512), (512, 512), (512, 4096)])
@pytest.mark.parametrize("fmt", ["awq-g128-f16", "ct-g32-bf16"])
def test_linear_tile_rows(pkg, dev, M, N, fmt):
    """Batches of >= TILE_ROWS rows run on MFMA from the tile copy (64-row tiles, ragged last
    tile; split along K into fp32 partials unless the grid has 256 tiles, as at 512 x 4096):
    the same product as the per-row dequant-GEMV, against the oracle's fp32 matmul."""
    rng = np.random.default_rng(60 + M + N)
    K = 2048
    if fmt == "awq-g128-f16":
        G, xdt = 128, "f16"
        qw, qz, sc = _gen.awq_weight(rng, 1, K, N, G)
        w = pkg.QWeight(t_(qw, dev), t_(sc, dev), t_(qz, dev), "awq", G, N, K)
        W = i4ref.awq_dequant(qw, qz, sc, G)[0]
        bias = rng.standard_normal(N).astype(np.float16)
    else:  # the reference checkpoint's format: CT g32 symmetric, bf16 scales and activations
        G, xdt = 32, "bf16"
        p, sc, _ = _gen.ct_weight(rng, 1, N, K, G, sdt="bf16")
        w = pkg.QWeight(t_(p, dev), t_(sc, dev), None, "ct", G, N, K)
        W = i4ref.ct_dequant(p, f_(sc), K, G)[0]
        bias = i4ref.f32_to_bf16_bits(rng.standard_normal(N).astype(np.float32))
    lin = pkg.PackedLinear.from_qweight(w, t_(bias, dev))
    assert lin.w_tile is not None and lin.w_tile.layout == "tile"
    x = make_x(rng, (M, K), xdt)
    got = host(pkg.ops.linear(t_(x, dev), lin.w_tile, lin.bias))  # the MFMA path at any M
    ref = f_(x) @ W.T + f_(bias)
    assert np.all(np.isfinite(got))
    assert i4ref.rel_err(got, ref) <= TOL
    rows = host(pkg.ops.linear(t_(x, dev), lin.w, lin.bias))  # the per-row GEMV
    assert i4ref.rel_err(got, rows) <= TOL


def test_packed_qkv_matches_three_linears(pkg, dev):
    """q, k, v in one launch equal the three separate launches bit for bit (each row's dot
    product does not depend on its neighbours): AWQ parts, and CT parts with and without
    zero points side by side."""
    rng = np.random.default_rng(41)
    K, G = 2048, 128
    x = t_(make_x(rng, (3, K), "f16"), dev)
    for kind in ("awq", "ct-mixed"):
        parts = []
        for i, N in enumerate((512, 128, 128)):
            if kind == "awq":
                qw, qz, sc = _gen.awq_weight(rng, 1, K, N, G)
                parts.append(pkg.QWeight(t_(qw, dev), t_(sc, dev), t_(qz, dev), "awq", G, N, K))
            else:
                p, sc, z = _gen.ct_weight(rng, 1, N, K, G, zeros=(i != 1))
                parts.append(pkg.QWeight(t_(p, dev), t_(sc, dev), None if z is None else t_(z, dev),
                                         "ct", G, N, K))
        biases = [t_(rng.standard_normal(p.N).astype(np.float16), dev) for p in parts]
        biases[2] = None
        fused = pkg.PackedQKV.from_qweights(*parts, biases=biases)
        got = fused(x)
        for y, w, b in zip(got, parts, biases):
            want = pkg.PackedLinear.from_qweight(w, b)(x)
            assert torch.equal(y, want)
        # the tile path (40 rows): the parts keep their 128-row tiles, but how far K is
        # split depends on the launch's whole grid, so the sums may round differently
        xl = t_(make_x(rng, (40, K), "f16"), dev)
        got = fused(xl)
        for y, w, b in zip(got, parts, biases):
            want = pkg.PackedLinear.from_qweight(w, b)(xl)
            assert i4ref.rel_err(host(y), host(want)) <= 1e-3


def test_packed_qkv_awq_in_place(pkg, dev):
    """q|k|v kept in AWQ packing (PackedQKV(repack=False): the columns side by side, one
    in-place GEMV launch, split along K at these sizes) against the oracle's fp64 product,
    and against the three separate in-place launches (whose k / v run K-complete: the sums
    may round differently, so within 1e-3)."""
    rng = np.random.default_rng(43)
    K, G = 2048, 128
    x = t_(make_x(rng, (1, K), "f16"), dev)
    parts, dense = [], []
    for i, N in enumerate((4096, 512, 512)):
        qw, qz, sc = _gen.awq_weight(rng, 1, K, N, G)
        z = None if i == 2 else qz
        parts.append(pkg.QWeight(t_(qw, dev), t_(sc, dev), None if z is None else t_(z, dev),
                                 "awq", G, N, K))
        dense.append(i4ref.awq_dequant(qw[0], None if z is None else z[0], f_(sc[0]), G))
    fused = pkg.PackedQKV.from_qweights(*parts, repack=False)
    assert fused.lin.w.layout == "awq" and fused.lin.w_tile is None
    got = fused(x)
    xf = np.asarray(host(x), np.float64)[0]
    for y, w, d in zip(got, parts, dense):
        ref = d @ xf
        assert i4ref.rel_err(np.asarray(host(y), np.float64)[0], ref) <= TOL
        alone = pkg.PackedLinear.from_qweight(w, repack=False)(x)
        assert i4ref.rel_err(host(y), host(alone)) <= 1e-3


class _FakePacked(torch.nn.Module):
    """A compressed-tensors pack-quantized Linear as the reference's loader leaves it."""

    def __init__(self, rng, N, K, G=32):
        super().__init__()
        p, sc, _ = _gen.ct_weight(rng, 1, N, K, G, sdt=np.float16)
        self.weight_packed = torch.from_numpy(p[0].copy())
        self.weight_scale = torch.from_numpy(sc[0].copy())
        self.weight_shape = torch.tensor([N, K])
        self.bias = None


def test_patch_attention_fuses_qkv(pkg, dev):
    """patch_attention(fuse_qkv=True) installs one launch for q/k/v; the block's q, k, v and
    o outputs equal the unfused patch's."""
    rng = np.random.default_rng(42)
    K = 512

    def block():
        m = torch.nn.Module()
        m.q_proj, m.k_proj, m.v_proj = _FakePacked(rng, 256, K), _FakePacked(rng, 64, K), \
            _FakePacked(rng, 64, K)
        m.o_proj = _FakePacked(rng, K, 256)
        return m

    a = block()
    b = torch.nn.Module()
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        src = getattr(a, name)
        c = _FakePacked(rng, 1, 32)
        c.weight_packed, c.weight_scale, c.weight_shape = (src.weight_packed.clone(),
                                                           src.weight_scale.clone(),
                                                           src.weight_shape.clone())
        setattr(b, name, c)
    assert pkg.patch_attention(a, device=dev, verbose=False, fuse_qkv=True) == 4
    assert pkg.patch_attention(b, device=dev, verbose=False) == 4
    assert isinstance(a.q_proj, pkg.QKVSlice) and isinstance(b.q_proj, pkg.PackedLinear)
    x = t_(make_x(rng, (2, K), "f16"), dev)
    for name in ("q_proj", "k_proj", "v_proj"):
        assert torch.equal(getattr(a, name)(x), getattr(b, name)(x))
    h = t_(make_x(rng, (2, 256), "f16"), dev)
    assert torch.equal(a.o_proj(h), b.o_proj(h))


def test_bad_expert_id_gives_nan_not_a_fault(pkg, dev):
    rng = np.random.default_rng(15)
    E, N, K, G = 4, 64, 256, 32
    p, s, _ = _gen.ct_weight(rng, E, N, K, G)
    sel = np.array([1, 200, -3, 2], np.int32)
    x = make_x(rng, (K,), "f16")
    got = host(pkg.dequant_gemv(t_(x, dev), t_(p, dev), t_(s, dev), t_(sel, dev), group=G))
    assert np.isnan(got[1]).all() and np.isnan(got[2]).all()
    ref = i4ref.dq_gemv(f_(x), i4ref.ct_dequant(p, f_(s), K, G), [1, 2])
    assert i4ref.rel_err(got[[0, 3]], ref) <= 1e-4


# ---------------------------------------------------------------- routing
@pytest.mark.parametrize("ldt", ["f16", "bf16", "f32"])
def test_route_topk_bit_exact(pkg, dev, ldt):
    rng = np.random.default_rng(16)
    T, E, k = 512, 128, 8
    v = rng.standard_normal((T, E)).astype(np.float32)
    v[:32] = np.round(v[:32] * 4) / 4  # many exact ties, also across the top-k cut
    v[32] = 0.0                        # every logit tied
    if ldt == "bf16":
        lg = i4ref.f32_to_bf16_bits(v)
    elif ldt == "f16":
        lg = v.astype(np.float16)
    else:
        lg = v
    w, sel = pkg.route(t_(lg, dev), k, w_dtype=torch.float32)
    sel_ref, w_ref = i4ref.route(f_(lg), k)
    np.testing.assert_array_equal(sel.cpu().numpy(), sel_ref)
    np.testing.assert_allclose(host(w), w_ref, rtol=1e-5, atol=1e-7)
    wh, _ = pkg.route(t_(lg, dev), k, w_dtype=torch.float16)
    np.testing.assert_allclose(host(wh).astype(np.float64), w_ref, rtol=1e-3, atol=1e-5)


@pytest.mark.parametrize("E,k", [(60, 8), (96, 6), (200, 8), (512, 1), (512, 8)])
def test_route_topk_expert_counts(pkg, dev, E, k):
    """Top-k at expert counts that leave lanes of the wave empty (60, 96: two logits per lane
    with the tail masked) or take eight logits per lane (200, 512), top-1 / 6 / 8, fp16 and
    bf16 logits with exact ties, also across the top-k cut: indices bit-exact with the
    oracle's ranking (value, then lower id), weights to fp32 rounding."""
    rng = np.random.default_rng(300 + E + k)
    T = 96
    v = rng.standard_normal((T, E)).astype(np.float32)
    v[:24] = np.round(v[:24] * 2) / 2  # many exact ties
    v[24] = 0.0                        # every logit tied
    for lg in (v.astype(np.float16), i4ref.f32_to_bf16_bits(v)):
        w, sel = pkg.route(t_(lg, dev), k, w_dtype=torch.float32)
        sel_ref, w_ref = i4ref.route(f_(lg), k)
        np.testing.assert_array_equal(sel.cpu().numpy(), sel_ref)
        np.testing.assert_allclose(host(w), w_ref, rtol=1e-5, atol=1e-7)


def test_route_without_renorm(pkg, dev):
    rng = np.random.default_rng(17)
    lg = rng.standard_normal((8, 128)).astype(np.float16)
    w, sel = pkg.route(t_(lg, dev), 8, norm_topk_prob=False, w_dtype=torch.float32)
    sel_ref, w_ref = i4ref.route(f_(lg), 8, renorm=False)
    np.testing.assert_array_equal(sel.cpu().numpy(), sel_ref)
    np.testing.assert_allclose(host(w), w_ref, rtol=1e-5)


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
@pytest.mark.parametrize("T", [1, 7, 64])
def test_router_logits(pkg, dev, xdt, T):
    rng = np.random.default_rng(T)
    E, H = 128, 2048
    wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    wr = i4ref.f32_to_bf16_bits(wr) if xdt == "bf16" else wr.astype(np.float16)
    x = make_x(rng, (T, H), xdt)
    got = host(pkg.router_logits(t_(x, dev), t_(wr, dev)))
    exact = f_(x) @ f_(wr).T
    ref = i4ref.round_half(exact, half_name(xdt))
    # fp32 accumulation may land on the other side of a rounding boundary: <= 1 ulp
    ulp = np.abs(ref) * (2.0 ** (-10 if xdt == "f16" else -7)) + 1e-6
    assert np.all(np.abs(got - ref) <= ulp)


# ---------------------------------------------------------------- MoE block
def _awq_moe(pkg, dev, rng, E=128, H=2048, I=768, G=128, sdt=np.float16, layouts="both",
             top_k=8):
    g = _gen.awq_weight(rng, E, H, I, G, sdt)
    u = _gen.awq_weight(rng, E, H, I, G, sdt)
    d = _gen.awq_weight(rng, E, I, H, G, sdt)
    wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float16)

    def q(part):
        return pkg.QWeight(t_(part[0], dev), t_(part[2], dev), t_(part[1], dev), "awq", G,
                           part[0].shape[2] * 8, part[0].shape[1])

    moe = pkg.FusedPackedMoE.from_awq(q(g), q(u), q(d), t_(wr, dev), top_k=top_k,
                                      layouts=layouts)
    dgu = lambda e: np.concatenate([i4ref.awq_dequant(g[0][e], g[1][e], f_(g[2][e]), G),
                                    i4ref.awq_dequant(u[0][e], u[1][e], f_(u[2][e]), G)], axis=0)
    ddn = lambda e: i4ref.awq_dequant(d[0][e], d[1][e], f_(d[2][e]), G)
    return moe, dgu, ddn, wr


def _check_moe(pkg, moe, dgu, ddn, x_np, xdt, dev, logits=None, residual=None, norm=None):
    """Run one block on the GPU and check it against the oracle on the same inputs.

    norm = (weight_np, eps): the block normalises x first; routing is checked
    bit-exactly against the oracle's top-k of the GPU's own logits, and the
    GPU's normalised input is checked against the oracle's RMSNorm.
    """
    x = t_(x_np, dev)
    kw = dict(router_w=moe.router_w) if logits is None else dict(logits=t_(logits, dev))
    if norm is not None:
        kw.update(norm_w=t_(norm[0], dev), norm_eps=norm[1])
    out, sel, w = pkg.moe_forward(x, moe.gate_up, moe.down, moe.top_k, return_routing=True,
                                  residual=None if residual is None else t_(residual, dev),
                                  gate_up_tile=moe.gate_up_tile, down_tile=moe.down_tile, **kw)
    xin = f_(x_np)
    if logits is None:
        if norm is None:
            lg = host(pkg.router_logits(x, moe.router_w))
        else:
            lg_t, xn_t = pkg.router_logits(x, moe.router_w, t_(norm[0], dev), norm[1],
                                           return_xn=True)
            lg, xin = host(lg_t), host(xn_t)
            ref_xn = i4ref.rmsnorm(f_(x_np), f_(norm[0]), norm[1], half_name(xdt))
            ulp = np.abs(ref_xn) * (2.0 ** (-10 if xdt == "f16" else -7)) + 1e-7
            assert np.all(np.abs(xin - ref_xn) <= 2 * ulp)
    else:
        lg = f_(logits)
    sel_ref, w_ref = i4ref.route(lg, moe.top_k)
    np.testing.assert_array_equal(sel.cpu().numpy(), sel_ref)          # bit-exact routing
    np.testing.assert_allclose(host(w), w_ref, rtol=1e-5, atol=1e-7)
    hn = half_name(xdt)
    moe_ref = i4ref.moe_layer_grouped(xin, sel_ref, w_ref, dgu, ddn, hn, y_dtype=hn)
    res = None if residual is None else f_(residual)
    ref = moe_ref + (0.0 if res is None else res)
    got = host(out)
    assert np.all(np.isfinite(got))
    err = i4ref.rel_err(got, ref)
    assert err <= TOL, err
    check_moe_term(got, moe_ref, res, hn)
    return got, err


@pytest.mark.parametrize("layouts", ["both", "tile"])
def test_moe_decode_m1(pkg, dev, layouts):
    """One int4 MoE layer at M=1: 128 experts, top-8, hidden 2048, FFN 768, AWQ g128; decode
    on CT rows (layouts="both") or on the tile copy alone (layouts="tile")."""
    rng = np.random.default_rng(21)
    moe, dgu, ddn, _ = _awq_moe(pkg, dev, rng, layouts=layouts)
    assert moe.gate_up.layout == ("ct" if layouts == "both" else "tile")
    for rep in range(3):
        x = make_x(rng, (1, 2048), "f16")
        _, err = _check_moe(pkg, moe, dgu, ddn, x, "f16", dev,
                            residual=make_x(rng, (1, 2048), "f16") if rep == 2 else None)
        assert err <= 1e-3


@pytest.mark.parametrize("layouts", ["both", "tile"])
@pytest.mark.parametrize("xdt", ["f16", "bf16"])
def test_moe_decode_m1_given_logits(pkg, dev, layouts, xdt):
    """A decode block handed its router logits (no router weight: the routed gate_up launch
    ranks them, then down + combine), with and without the residual, against the oracle."""
    rng = np.random.default_rng(26)
    sdt = "bf16" if xdt == "bf16" else np.float16
    moe, dgu, ddn, _ = _awq_moe(pkg, dev, rng, sdt=sdt, layouts=layouts)
    for rep in range(2):
        x = make_x(rng, (1, 2048), xdt)
        lg = rng.standard_normal((1, 128)).astype(np.float32)
        lg = i4ref.f32_to_bf16_bits(lg) if xdt == "bf16" else lg.astype(np.float16)
        _check_moe(pkg, moe, dgu, ddn, x, xdt, dev, logits=lg, residual=x if rep else None)


@pytest.mark.parametrize("layouts", ["both", "tile"])
def test_decode_stages_compose_to_the_block(pkg, dev, layouts):
    """route+gate_up, gate_up(sel) and down+combine reproduce moe_forward at T=1 bit for bit,
    and the stage outputs match the oracle."""
    rng = np.random.default_rng(31)
    moe, dgu, ddn, _ = _awq_moe(pkg, dev, rng, E=64, layouts=layouts)
    x = t_(make_x(rng, (1, 2048), "f16"), dev)
    res = t_(make_x(rng, (1, 2048), "f16"), dev)
    full, sel_f, w_f = pkg.moe_forward(x, moe.gate_up, moe.down, 8, router_w=moe.router_w,
                                       residual=res, return_routing=True)
    lg = pkg.router_logits(x, moe.router_w)
    act, sel, w = pkg.moe_route_gate_up(x, moe.gate_up, lg, 8)
    assert torch.equal(sel, sel_f.reshape(-1)) and torch.equal(w, w_f.reshape(-1))
    act2 = pkg.moe_gate_up(x, moe.gate_up, sel)
    assert torch.equal(act, act2)
    out = pkg.moe_down_combine(act, moe.down, sel, w, residual=res)
    assert torch.equal(out.reshape(1, -1), full)
    # stage values against the oracle
    xs = host(x)[0]
    for j, e in enumerate(sel.cpu().numpy()):
        gu = dgu(int(e)) @ xs
        ref_act = i4ref.round_half(i4ref.silu(gu[:768]) * gu[768:], "f16")
        assert i4ref.rel_err(host(act[j]).astype(np.float64), ref_act) <= 1e-3


@pytest.mark.parametrize("layouts", ["both", "tile"])
def test_moe_decode_reference_format(pkg, dev, layouts):
    """The reference checkpoint's own format: CT g32 symmetric, bf16 scales and activations."""
    rng = np.random.default_rng(22)
    E, H, I, G = 128, 2048, 768, 32
    gp, gs, _ = _gen.ct_weight(rng, E, 2 * I, H, G, sdt="bf16")
    dp, ds, _ = _gen.ct_weight(rng, E, H, I, G, sdt="bf16")
    wr = i4ref.f32_to_bf16_bits((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    gu = pkg.QWeight(t_(gp, dev), t_(gs, dev), None, "ct", G, 2 * I, H)
    dn = pkg.QWeight(t_(dp, dev), t_(ds, dev), None, "ct", G, H, I)
    moe = pkg.FusedPackedMoE.from_stacked(gu, dn, t_(wr, dev), top_k=8, layouts=layouts)
    dgu = lambda e: i4ref.ct_dequant(gp[e], f_(gs[e]), H, G)
    ddn = lambda e: i4ref.ct_dequant(dp[e], f_(ds[e]), I, G)
    for _ in range(2):
        _check_moe(pkg, moe, dgu, ddn, make_x(rng, (1, H), "bf16"), "bf16", dev)


@pytest.mark.parametrize("k", [4, 6])
def test_moe_other_top_k(pkg, dev, k):
    """Top-4 and top-6 of 128 experts: the single-launch decode layer (its down workgroups'
    expert groups past top-k stay idle) and the grouped MFMA path at 32 tokens, routing
    bit-exact, outputs against the oracle."""
    rng = np.random.default_rng(40 + k)
    moe, dgu, ddn, _ = _awq_moe(pkg, dev, rng, top_k=k)
    x1 = make_x(rng, (1, 2048), "f16")
    _check_moe(pkg, moe, dgu, ddn, x1, "f16", dev, residual=x1)
    x = make_x(rng, (32, 2048), "f16")
    _check_moe(pkg, moe, dgu, ddn, x, "f16", dev, residual=x)


def test_moe_entry_size_boundaries(pkg, dev):
    """Experts with exactly 1, 16, 17, 64, 65, 128 and 129 tokens: the edges of the one-m-block
    small entries (<= 16 tokens) and of the 64-token large entries (several per expert, the
    last one ragged), in one grouped call of 129 tokens whose logits put each token's top-8
    on chosen experts (distinct values, no ties)."""
    rng = np.random.default_rng(46)
    E, T, H = 128, 129, 2048
    moe, dgu, ddn, _ = _awq_moe(pkg, dev, rng)
    sizes = {0: 1, 1: 16, 2: 17, 3: 64, 4: 65, 5: 128, 6: 129}
    lg = rng.uniform(-4.0, -1.0, (T, E)).astype(np.float32)
    fill = 7
    for t in range(T):
        chosen = [e for e, n in sizes.items() if t < n]
        while len(chosen) < 8:  # the rest of the top-8 from experts 7..22 in turn
            chosen.append(fill)
            fill = 7 + (fill - 7 + 1) % 16
        lg[t, chosen] = 2.0 + 0.01 * np.arange(8) + rng.uniform(0, 0.001, 8)
    lg = lg.astype(np.float16)
    counts = np.bincount(i4ref.route(lg.astype(np.float64), 8)[0].ravel(), minlength=E)
    assert [counts[e] for e in sizes] == list(sizes.values())
    x = make_x(rng, (T, H), "f16")
    _check_moe(pkg, moe, dgu, ddn, x, "f16", dev, logits=lg, residual=x)


def test_moe_m32(pkg, dev):
    rng = np.random.default_rng(23)
    moe, dgu, ddn, _ = _awq_moe(pkg, dev, rng)
    x = make_x(rng, (32, 2048), "f16")
    _check_moe(pkg, moe, dgu, ddn, x, "f16", dev, residual=x)


@pytest.mark.parametrize("xdt,T,E", [("f16", 2, 128), ("bf16", 64, 128), ("f16", 9, 20)])
def test_moe_fused_routing_edges(pkg, dev, xdt, T, E):
    """Router and top-k as one launch (2..64 tokens, E <= 128, E % 4 == 0) at its
    token-count edges and with E not a multiple of 8, after the block's input RMSNorm:
    routing bit-exact against the oracle's top-k of the GPU's own logits, the normalised
    input against the oracle's RMSNorm, outputs against the oracle."""
    rng = np.random.default_rng(300 + T + E)
    sdt = "bf16" if xdt == "bf16" else np.float16
    moe, dgu, ddn, _ = _awq_moe(pkg, dev, rng, E=E, sdt=sdt)
    if xdt == "bf16":
        moe.router_w = moe.router_w.to(torch.bfloat16)
    nw = rng.uniform(0.5, 1.5, 2048).astype(np.float32)
    nw = i4ref.f32_to_bf16_bits(nw) if xdt == "bf16" else nw.astype(np.float16)
    x = make_x(rng, (T, 2048), xdt)
    _check_moe(pkg, moe, dgu, ddn, x, xdt, dev, residual=x, norm=(nw, 1e-6))


def test_moe_m32_fused_wait_gives_up_visibly(pkg, dev):
    """At T <= 64 both expert projections share one launch whose down workgroups wait for
    the activations of its gate_up workgroups, and router and top-k share one whose ranking
    waves wait for their token's logits.  i4_moe_forward_bounded runs the down workgroups
    (or the ranking waves) alone with the bound lowered from the host: every wait gives up,
    the output is NaN and the status word holds I4_ERR_HANDOFF, and every kernel exits.  The next
    ordinary call on the same workspace is correct (against the oracle) and clears the
    word; the bounded call with its producers present and the full bound equals it bit for
    bit."""
    rng = np.random.default_rng(29)
    moe, dgu, ddn, _ = _awq_moe(pkg, dev, rng)
    T = 32
    x_np = make_x(rng, (T, 2048), "f16")
    x = t_(x_np, dev)
    tiles = dict(gate_up_tile=moe.gate_up_tile, down_tile=moe.down_tile)
    ws = pkg.Workspace()
    E, I = moe.gate_up.E, moe.down.K
    for polls in (0, 3):
        y = pkg.ops.moe_forward_bounded(x, moe.gate_up, moe.down, moe.top_k, polls, True,
                                        router_w=moe.router_w, residual=x, workspace=ws, **tiles)
        torch.cuda.synchronize()
        assert torch.isnan(y.float()).all()
        assert pkg.moe_status(ws, T, 2048, I, E, moe.top_k) == -10
    # the routing launch's ranking waves alone: their waits for the logits give up too
    for polls in (0, 3):
        y = pkg.ops.moe_forward_bounded(x, moe.gate_up, moe.down, moe.top_k, polls,
                                        rank_only=True, router_w=moe.router_w, residual=x,
                                        workspace=ws, **tiles)
        torch.cuda.synchronize()
        assert torch.isnan(y.float()).all()
        assert pkg.moe_status(ws, T, 2048, I, E, moe.top_k) == -10
    got = pkg.moe_forward(x, moe.gate_up, moe.down, moe.top_k, router_w=moe.router_w,
                          residual=x, workspace=ws, **tiles)
    assert pkg.moe_status(ws, T, 2048, I, E, moe.top_k) == 0
    checked, _ = _check_moe(pkg, moe, dgu, ddn, x_np, "f16", dev, residual=x_np)  # vs oracle
    assert np.array_equal(host(got), checked)
    again = pkg.ops.moe_forward_bounded(x, moe.gate_up, moe.down, moe.top_k, 1 << 20, False,
                                        router_w=moe.router_w, residual=x, workspace=ws, **tiles)
    assert torch.equal(again, got)
    assert pkg.moe_status(ws, T, 2048, I, E, moe.top_k) == 0
    # one token runs the decode path, more than 64 the two-list launches: nothing to bound
    for bad_T in (1, 65):
        xb = t_(make_x(rng, (bad_T, 2048), "f16"), dev)
        with pytest.raises(RuntimeError):
            pkg.ops.moe_forward_bounded(xb, moe.gate_up, moe.down, moe.top_k, 3, True,
                                        router_w=moe.router_w, workspace=ws, **tiles)


def test_moe_m512_zipf_logits(pkg, dev):
    rng = np.random.default_rng(24)
    moe, dgu, ddn, _ = _awq_moe(pkg, dev, rng)
    x = make_x(rng, (512, 2048), "f16")
    lg = _gen.zipf_logits(rng, 512, 128).astype(np.float16)
    counts = np.bincount(i4ref.route(lg.astype(np.float64), 8)[0].ravel(), minlength=128)
    assert counts.max() > 64 and (counts <= 2).sum() > 20  # the skew the workload asks for
    _check_moe(pkg, moe, dgu, ddn, x, "f16", dev, logits=lg)


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
def test_moe_mfma_tiles(pkg, dev, xdt):
    """Few experts, many tokens each: every expert takes the MFMA tile path (>= 16 tokens),
    including partial 64-token tiles and ragged m-blocks."""
    rng = np.random.default_rng(32)
    E, H, I, G, T = 12, 2048, 768, 128, 181
    sdt = "bf16" if xdt == "bf16" else np.float16
    moe, dgu, ddn, _ = _awq_moe(pkg, dev, rng, E=E, sdt=sdt)
    if xdt == "bf16":
        moe.router_w = moe.router_w.to(torch.bfloat16)
    x = make_x(rng, (T, H), xdt)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg = i4ref.f32_to_bf16_bits(lg) if xdt == "bf16" else lg.astype(np.float16)
    counts = np.bincount(i4ref.route(f_(lg), 8)[0].ravel(), minlength=E)
    assert counts.min() >= 16  # all MFMA
    _check_moe(pkg, moe, dgu, ddn, x, xdt, dev, logits=lg, residual=x)


@pytest.mark.parametrize("E,T", [(16, 40), (128, 24)])
def test_moe_prefill_reference_format(pkg, dev, E, T):
    """The reference checkpoint's own format (CT g32 symmetric, bf16) at T > 1: per-chunk
    group corrections on the MFMA path, large entries (E = 16: ~20 tokens per expert) and
    small ones (E = 128)."""
    rng = np.random.default_rng(33 + E)
    H, I, G = 2048, 768, 32
    gp, gs, _ = _gen.ct_weight(rng, E, 2 * I, H, G, sdt="bf16")
    dp, ds, _ = _gen.ct_weight(rng, E, H, I, G, sdt="bf16")
    wr = i4ref.f32_to_bf16_bits((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    gu = pkg.QWeight(t_(gp, dev), t_(gs, dev), None, "ct", G, 2 * I, H)
    dn = pkg.QWeight(t_(dp, dev), t_(ds, dev), None, "ct", G, H, I)
    moe = pkg.FusedPackedMoE.from_stacked(gu, dn, t_(wr, dev), top_k=8)
    dgu = lambda e: i4ref.ct_dequant(gp[e], f_(gs[e]), H, G)
    ddn = lambda e: i4ref.ct_dequant(dp[e], f_(ds[e]), I, G)
    x = make_x(rng, (T, H), "bf16")
    _check_moe(pkg, moe, dgu, ddn, x, "bf16", dev, residual=x)


def test_moe_prefill_bf16_small_entries(pkg, dev):
    """bf16 activations with AWQ g128 weights and <= 16 tokens per expert: the small-entry
    MFMA kernel's activation-sum correction."""
    rng = np.random.default_rng(35)
    moe, dgu, ddn, wr = _awq_moe(pkg, dev, rng, sdt="bf16")
    moe.router_w = moe.router_w.to(torch.bfloat16)
    x = make_x(rng, (24, 2048), "bf16")
    _check_moe(pkg, moe, dgu, ddn, x, "bf16", dev)


def test_moe_tokens_are_independent(pkg, dev):
    rng = np.random.default_rng(25)
    moe, _, _, _ = _awq_moe(pkg, dev, rng, E=32)
    x = t_(make_x(rng, (6, 2048), "f16"), dev)
    full = host(moe(x))
    for t in range(6):
        one = host(moe(x[t:t + 1]))
        # decode (CT rows) and grouped (MFMA tiles) sum in different orders: each output may
        # round to a neighbouring fp16 value, beyond which they agree to 1e-3
        err = np.abs(one[0] - full[t]) - 2 * half_ulp(full[t], "f16")
        assert np.max(err) <= 1e-3 * np.max(np.abs(full[t]))


def test_moe_is_deterministic(pkg, dev):
    rng = np.random.default_rng(26)
    moe, _, _, _ = _awq_moe(pkg, dev, rng, E=64)
    for T in (1, 40):
        x = t_(make_x(rng, (T, 2048), "f16"), dev)
        a, b = moe(x), moe(x)
        assert torch.equal(a, b)


def test_stack_matches_layer_loop_and_oracle(pkg, dev):
    """h <- h + moe_l(RMSNorm_l(h)) for 4 layers; each layer checked against the oracle on the
    GPU's own input, and the one-call stack equals the layer-by-layer loop bit for bit."""
    rng = np.random.default_rng(27)
    layers = []
    for _ in range(4):
        m, dgu, ddn, _ = _awq_moe(pkg, dev, rng, E=32)
        nw = rng.uniform(0.5, 1.5, 2048).astype(np.float16)
        m.register_buffer("norm_weight", t_(nw, dev), persistent=False)
        m.norm_eps = 1e-6
        layers.append((m, dgu, ddn, nw))
    x = make_x(rng, (1, 2048), "f16")
    xt = t_(x, dev)
    stack = pkg.moe_stack(xt, [m.stack_entry() for m, _, _, _ in layers], 8)
    h = xt
    for m, dgu, ddn, nw in layers:
        h_np = host(h).astype(np.float16)
        h_next = m(h, residual=h)
        _check_moe(pkg, m, dgu, ddn, h_np, "f16", dev, residual=h_np, norm=(nw, 1e-6))
        h = h_next
    assert torch.isfinite(stack).all()
    assert torch.equal(stack, h)


def _stack_modules(pkg, dev, rng, xdt, norm, n_distinct=3, H=2048, I=768):
    """n_distinct small blocks (32 experts, H x I) in the activation dtype xdt."""
    sdt = "bf16" if xdt == "bf16" else np.float16
    mods = []
    for _ in range(n_distinct):
        m, _, _, _ = _awq_moe(pkg, dev, rng, E=32, H=H, I=I, sdt=sdt)
        tdt = torch.bfloat16 if xdt == "bf16" else torch.float16
        m.router_w = m.router_w.to(tdt)
        if norm:
            nw = torch.from_numpy(rng.uniform(0.5, 1.5, H).astype(np.float32)).to(dev, tdt)
            m.register_buffer("norm_weight", nw, persistent=False)
            m.norm_eps = 1e-6
        mods.append(m)
    return mods


@pytest.mark.parametrize("xdt,norm,n_layers,H,I", [
    ("f16", True, 26, 2048, 768), ("bf16", True, 5, 2048, 768), ("f16", False, 3, 2048, 768),
    ("bf16", False, 1, 2048, 768), ("bf16", True, 4, 1024, 384), ("f16", False, 2, 1024, 384)])
def test_stack_matches_layer_loop_variants(pkg, dev, xdt, norm, n_layers, H, I):
    """The one-call decode stack equals the module-by-module loop bit for bit: an even and an
    odd number of layers (the call alternates its buffers by layer parity), bf16, without
    the RMSNorm, and at hidden size 1024."""
    rng = np.random.default_rng(61 + n_layers)
    mods = _stack_modules(pkg, dev, rng, xdt, norm, H=H, I=I)
    layers = [mods[i % len(mods)] for i in range(n_layers)]
    x = make_x(rng, (1, H), "f16") * (1.0 if norm else 0.1)  # un-normalised layers grow
    xt = t_(i4ref.f32_to_bf16_bits(x.astype(np.float32)) if xdt == "bf16" else x, dev)
    stack = pkg.moe_stack(xt, [m.stack_entry() for m in layers], 8)
    h = xt
    for m in layers:
        h = m(h, residual=h)
    assert torch.isfinite(stack).all()
    assert torch.equal(stack, h)
    ws = pkg.Workspace()
    again = pkg.moe_stack(xt, [m.stack_entry() for m in layers], 8, workspace=ws)
    assert torch.equal(again, stack)
    assert pkg.moe_status(ws, 1, H, I, 32, 8) == 0


@pytest.mark.parametrize("norm,top_k,n_layers", [(True, 8, 4), (False, 4, 3)])
def test_stack_hidden_1024(pkg, dev, norm, top_k, n_layers):
    """A decode stack at hidden 1024 (the router wave of 1024 values) equals the module loop
    bit for bit, with its status word left at 0."""
    rng = np.random.default_rng(140 + n_layers)
    mods = []
    for _ in range(n_layers):
        m, _, _, _ = _awq_moe(pkg, dev, rng, E=16, H=1024, I=768, top_k=top_k)
        if norm:
            nw = rng.uniform(0.5, 1.5, 1024).astype(np.float16)
            m.register_buffer("norm_weight", t_(nw, dev), persistent=False)
            m.norm_eps = 1e-6
        mods.append(m)
    x = make_x(rng, (1, 1024), "f16") * (1.0 if norm else 0.1)
    xt = t_(x, dev)
    ws = pkg.Workspace()
    stack = pkg.moe_stack(xt, [m.stack_entry() for m in mods], top_k, workspace=ws)
    h = xt
    for m in mods:
        h = m(h, residual=h)
    assert torch.isfinite(stack).all()
    assert torch.equal(stack, h)
    assert pkg.moe_status(ws, 1, 1024, 768, 16, top_k) == 0


def test_stack_graph_replays_match_eager(pkg, dev):
    """The decode stack (two launches per layer) captured in a hipGraph gives the eager result
    on every replay, with other work and new inputs between replays."""
    rng = np.random.default_rng(71)
    mods = _stack_modules(pkg, dev, rng, "f16", True)
    entries = [m.stack_entry() for m in mods * 2]
    ws = pkg.Workspace()
    xs = [t_(make_x(rng, (1, 2048), "f16"), dev) for _ in range(3)]
    eager = [pkg.moe_stack(x, entries, 8, workspace=ws).clone() for x in xs]
    static_x = xs[0].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        pkg.moe_stack(static_x, entries, 8, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = pkg.moe_stack(static_x, entries, 8, workspace=ws)
    for r in range(6):
        static_x.copy_(xs[r % 3])
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[r % 3])
        _ = (torch.randn(256, 256, device=dev) @ torch.randn(256, 256, device=dev)).sum().item()


def test_moe_m32_graph_replays_match_eager(pkg, dev):
    """The 32-token block (routing launch whose ranking waves wait for tagged logits, grouping,
    the grouped experts launch, combine) captured in a hipGraph gives the eager result on
    every replay, with other work and new inputs between replays: the tag epoch the
    grouping launch advances makes each replay wait for its own logits."""
    rng = np.random.default_rng(72)
    moe, _, _, _ = _awq_moe(pkg, dev, rng)
    tiles = dict(gate_up_tile=moe.gate_up_tile, down_tile=moe.down_tile)
    ws = pkg.Workspace()
    xs = [t_(make_x(rng, (32, 2048), "f16"), dev) for _ in range(3)]
    run = lambda x: pkg.moe_forward(x, moe.gate_up, moe.down, moe.top_k, router_w=moe.router_w,
                                    residual=x, workspace=ws, **tiles)
    eager = [run(x).clone() for x in xs]
    static_x = xs[0].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(static_x)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = run(static_x)
    for r in range(6):
        static_x.copy_(xs[r % 3])
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[r % 3])
        assert pkg.moe_status(ws, 32, 2048, moe.down.K, moe.gate_up.E, moe.top_k) == 0
        _ = (torch.randn(256, 256, device=dev) @ torch.randn(256, 256, device=dev)).sum().item()


@pytest.mark.parametrize("T", [1, 9])
def test_router_logits_with_norm(pkg, dev, T):
    rng = np.random.default_rng(29 + T)
    E, H = 128, 2048
    wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float16)
    nw = rng.uniform(0.5, 1.5, H).astype(np.float16)
    x = (rng.standard_normal((T, H)) * 40).astype(np.float16)
    lg, xn = pkg.router_logits(t_(x, dev), t_(wr, dev), t_(nw, dev), 1e-6, return_xn=True)
    ref_xn = i4ref.rmsnorm(f_(x), f_(nw), 1e-6, "f16")
    got_xn = host(xn).astype(np.float64)
    assert np.all(np.abs(got_xn - ref_xn) <= 2 * np.abs(ref_xn) * 2.0 ** -10 + 1e-7)
    assert np.mean(got_xn == ref_xn) > 0.99
    ref = i4ref.router_logits(got_xn, f_(wr), "f16")
    got = host(lg).astype(np.float64)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -10 + 1e-6)


@pytest.mark.parametrize("xdt", ["f16", "bf16"])
@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("H", [2048, 1024, 768])
def test_router_tokens_match_single_token_bits(pkg, dev, xdt, norm, H):
    """The multi-token router gives every token the logits and RMSNorm output it gets alone,
    bit for bit (so routing never depends on the batch), including a ragged last tile; the
    single-token router is the one-wavefront-per-expert kernel at H = 2048 (the Thinker) and
    1024 (the Talker), the four-wavefront one otherwise."""
    rng = np.random.default_rng(41)
    E, T = 128, 19
    wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    wr = i4ref.f32_to_bf16_bits(wr) if xdt == "bf16" else wr.astype(np.float16)
    x = t_(make_x(rng, (T, H), xdt), dev)
    w_t = t_(wr, dev)
    nw = t_(rng.uniform(0.5, 1.5, H).astype(np.float16), dev) if norm else None
    if nw is not None and xdt == "bf16":
        nw = nw.to(torch.bfloat16)
    kw = dict(norm_w=nw, norm_eps=1e-6, return_xn=True) if norm else {}
    full = pkg.router_logits(x, w_t, **kw)
    for t in range(T):
        one = pkg.router_logits(x[t:t + 1], w_t, **kw)
        if norm:
            assert torch.equal(one[0][0], full[0][t]) and torch.equal(one[1][0], full[1][t])
        else:
            assert torch.equal(one[0], full[t])


def test_graph_replays_match_eager(pkg, dev):
    rng = np.random.default_rng(28)
    moe, _, _, _ = _awq_moe(pkg, dev, rng, E=32)
    x = t_(make_x(rng, (1, 2048), "f16"), dev)
    eager = moe(x, residual=x).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        moe(x, residual=x)  # warm the workspace outside the capture
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = moe(x, residual=x)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        _ = (torch.randn(256, 256, device=dev) @ torch.randn(256, 256, device=dev)).sum().item()

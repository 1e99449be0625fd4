"""The C ABI: libi4moe.so loads without a GPU, exports every function that
include/i4moe.h declares, and rejects invalid calls on the host before any
launch (no compute call is made here)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "i4moe.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(i4_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_abi():
    names = declared_functions()
    assert "i4_dq_gemv" in names and "i4_moe_forward" in names and len(names) >= 15


def test_every_declared_symbol_is_exported_and_bound(pkg):
    lib = pkg.lib()
    from qwen3_omni_duplex_amd import _lib

    for name in declared_functions():
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(declared_functions())


def test_version_and_errors(pkg):
    lib = pkg.lib()
    assert lib.i4_abi_version() == 9
    codes = {0: b"ok", -1: b"NULL", -2: b"dimension", -3: b"element type", -4: b"aligned",
             -5: b"layout", -6: b"group", -7: b"workspace", -8: b"launch", -9: b"stride",
             -10: b"gave up waiting", -11: b"static buffer"}
    for c, frag in codes.items():
        assert frag in lib.i4_strerror(c)
    assert b"unknown" in lib.i4_strerror(-99)


def _qw(_lib, **kw):
    base = dict(packed=0x10000, scale=0x20000, zeros=None, packed_estride=0, scale_estride=0,
                zeros_estride=0, layout=0, group=32, scale_dtype=1, E=4, N=64, K=256)
    base.update(kw)
    return _lib.QWeightC(**base)


@pytest.mark.parametrize("bad,code", [
    (dict(packed=None), -1),
    (dict(K=100), -2),
    (dict(K=16), -2),
    (dict(group=48), -6),
    (dict(group=16), -6),
    (dict(layout=7), -5),
    (dict(scale_dtype=9), -3),
    (dict(packed=0x10004), -4),
    (dict(packed_estride=10), -9),
    (dict(layout=1, N=60), -2),
])
def test_weight_validation_codes(pkg, bad, code):
    pkg.lib()
    from qwen3_omni_duplex_amd import _lib

    lib = pkg.lib()
    w = _qw(_lib, **bad)
    rc = lib.i4_dq_gemv(0x30000, 1, 0, ctypes.byref(w), 0x40000, 8, 0x50000, 0, None, 0, None)
    assert rc == code


def test_call_validation_codes(pkg):
    from qwen3_omni_duplex_amd import _lib

    lib = pkg.lib()
    w = _qw(_lib)
    # activations must be half precision, aligned, with a sane stride
    assert lib.i4_dq_gemv(0x30000, 0, 0, ctypes.byref(w), 0x40000, 8, 0x50000, 0, None, 0, None) == -3
    assert lib.i4_dq_gemv(0x30002, 1, 0, ctypes.byref(w), 0x40000, 8, 0x50000, 0, None, 0, None) == -4
    assert lib.i4_dq_gemv(0x30000, 1, 100, ctypes.byref(w), 0x40000, 8, 0x50000, 0, None, 0, None) == -9
    assert lib.i4_dq_gemv(0x30000, 1, 0, ctypes.byref(w), None, 8, 0x50000, 0, None, 0, None) == -1
    assert lib.i4_dq_gemv(0x30000, 1, 0, ctypes.byref(w), 0x40000, 0, 0x50000, 0, None, 0, None) == -2
    # AWQ with N % 32 == 0 and more than 2048 rows of lines per CU in a K-complete launch
    # splits K over a workspace of fp32 partials per row of x, 256-column strip and K slice
    # (K = 4096, group 128: 128-row slices, 32 of them); without a workspace, or at smaller
    # shapes, it runs K-complete workgroups; CT needs none; AWQ scales are read 16 bytes
    # at a time
    wa = _qw(_lib, layout=1, N=256, K=4096, group=128)
    # 256-byte header (the status word), then (value, tag) pairs of 8 bytes
    assert lib.i4_dq_gemv_workspace_bytes(ctypes.byref(wa), 8) == 256 + 8 * 1 * 32 * 256 * 8
    # more than 8 rows, or partials beyond 8 MiB, run K-complete: no workspace
    assert lib.i4_dq_gemv_workspace_bytes(ctypes.byref(wa), 9) == 0
    wbig = _qw(_lib, layout=1, N=4096, K=4096, group=128)
    assert lib.i4_dq_gemv_workspace_bytes(ctypes.byref(wbig), 1) == 256 + 16 * 32 * 256 * 8
    assert lib.i4_dq_gemv_workspace_bytes(ctypes.byref(wbig), 8) == 0
    assert lib.i4_dq_gemv_workspace_bytes(ctypes.byref(_qw(_lib, layout=1)), 8) == 0
    assert lib.i4_dq_gemv_workspace_bytes(ctypes.byref(_qw(_lib, layout=1, N=40, K=4096)),
                                          8) == 0
    assert lib.i4_dq_gemv_workspace_bytes(ctypes.byref(w), 8) == 0
    assert lib.i4_dq_gemv(0x30000, 1, 0, ctypes.byref(wa), 0x40000, 8, 0x50000, 0, 0x60000, 16,
                          None) == -7
    assert lib.i4_dq_gemv(0x30000, 1, 0, ctypes.byref(wa), 0x40000, 8, 0x50000, 0, 0x60010,
                          1 << 20, None) == -4
    assert lib.i4_linear_workspace_bytes(
        ctypes.byref(_qw(_lib, layout=1, E=1, N=256, K=4096, group=128)), 1) == 256 + 32 * 256 * 8
    wa_odd = _qw(_lib, layout=1, scale=0x20008)
    assert lib.i4_dq_gemv(0x30000, 1, 0, ctypes.byref(wa_odd), 0x40000, 8, 0x50000, 0, None, 0,
                          None) == -4
    # routing limits
    assert lib.i4_route_topk(0x30000, 1, 1, 128, 0, 1, 0x40000, None, None, 0, None) == -2
    assert lib.i4_route_topk(0x30000, 1, 1, 1024, 8, 1, 0x40000, None, None, 0, None) == -2
    assert lib.i4_route_topk(0x30000, 5, 1, 128, 8, 1, 0x40000, None, None, 0, None) == -3
    assert lib.i4_router_logits(0x30000, 1, 1, 2047, 0x40000, 128, None, 1e-6, None, 0x50000,
                                None) == -2
    # xn output needs a norm weight; norm weight must be aligned
    assert lib.i4_router_logits(0x30000, 1, 1, 2048, 0x40000, 128, None, 1e-6, 0x60000, 0x50000,
                                None) == -1
    assert lib.i4_router_logits(0x30000, 1, 1, 2048, 0x40000, 128, 0x60002, 1e-6, None, 0x50000,
                                None) == -4
    # with a norm and more than one token the normalised rows must have somewhere to go
    assert lib.i4_router_logits(0x30000, 1, 2, 2048, 0x40000, 128, 0x60000, 1e-6, None, 0x50000,
                                None) == -1


def test_moe_validation_codes(pkg):
    from qwen3_omni_duplex_amd import _lib

    lib = pkg.lib()
    gu = _qw(_lib, E=128, N=1536, K=2048, group=128, layout=2)
    dn = _qw(_lib, E=128, N=2048, K=768, group=128, layout=2)
    mw = _lib.MoeWeightsC(gate_up=gu, down=dn, router_w=0x60000)
    ws = lib.i4_moe_workspace_bytes(1, 2048, 768, 128, 8)
    assert ws > 0
    call = lambda **kw: lib.i4_moe_forward(
        kw.get("x", 0x30000), kw.get("xt", 1), kw.get("T", 1), ctypes.byref(kw.get("mw", mw)),
        kw.get("k", 8), 1, None, None, 0x70000, None, None, kw.get("ws", 0x100000),
        kw.get("wsb", ws), None)
    assert call(wsb=ws - 1) == -7
    assert call(ws=0x100010) == -4
    assert call(k=0) == -2
    assert call(T=0) == -2
    assert call(xt=0) == -3
    bad = _lib.MoeWeightsC(gate_up=_qw(_lib, E=128, N=1504, K=2048, group=128, layout=2),
                           down=dn, router_w=0x60000)
    assert call(mw=bad) == -2
    # the tile layout needs N % 16 == 0 and K % 128 == 0
    ragged = _lib.MoeWeightsC(gate_up=_qw(_lib, E=128, N=1528, K=2048, group=128, layout=2),
                              down=dn, router_w=0x60000)
    assert call(mw=ragged) == -2
    # decode reads CT rows or tiles (the same layout for both weights), more tokens need tiles
    # (only validation failures here: a valid call would launch on the fake pointers)
    ct_gu = _qw(_lib, E=128, N=1536, K=2048, group=128, layout=0)
    ct_dn = _qw(_lib, E=128, N=2048, K=768, group=128, layout=0)
    ctw = _lib.MoeWeightsC(gate_up=ct_gu, down=ct_dn, router_w=0x60000)
    assert call(mw=ctw, T=2) == -5
    mixed = _lib.MoeWeightsC(gate_up=ct_gu, down=dn, router_w=0x60000)
    assert call(mw=mixed) == -5
    awq = _lib.MoeWeightsC(gate_up=_qw(_lib, E=128, N=1536, K=2048, group=128, layout=1),
                           down=dn, router_w=0x60000)
    assert call(mw=awq) == -5
    # tile copies: both or neither, in the tile layout, the block's shapes
    half = _lib.MoeWeightsC(gate_up=ct_gu, down=ct_dn, router_w=0x60000, gate_up_tile=gu)
    assert call(mw=half) == -1
    wrong = _lib.MoeWeightsC(gate_up=ct_gu, down=ct_dn, router_w=0x60000, gate_up_tile=ct_gu,
                             down_tile=ct_dn)
    assert call(mw=wrong) == -5
    small = _lib.MoeWeightsC(gate_up=ct_gu, down=ct_dn, router_w=0x60000,
                             gate_up_tile=_qw(_lib, E=64, N=1536, K=2048, group=128, layout=2),
                             down_tile=dn)
    assert call(mw=small) == -2
    # and the dequant-GEMV entry points do not take it
    tw = _qw(_lib, E=8, N=768, K=2048, group=128, layout=2)
    assert lib.i4_dq_gemv(0x30000, 1, 0, ctypes.byref(tw), 0x40000, 8, 0x50000, 0, None, 0,
                          None) == -5
    # repack into tiles: row offsets in whole 16-row blocks, a source in CT or AWQ
    src = _qw(_lib, E=8, N=768, K=2048, group=128)
    assert lib.i4_repack_tile(ctypes.byref(src), 0x40000, 0x50000, None, 1536, 8, None) == -2
    assert lib.i4_repack_tile(ctypes.byref(src), 0x40000, 0x50000, None, 1536, 1024, None) == -2
    assert lib.i4_repack_tile(ctypes.byref(tw), 0x40000, 0x50000, None, 768, 0, None) == -5
    nor = _lib.MoeWeightsC(gate_up=gu, down=dn, router_w=None)
    assert call(mw=nor) == -1
    # a fused norm needs the router weight (it produces the normalised input)
    nrm = _lib.MoeWeightsC(gate_up=gu, down=dn, router_w=None, norm_w=0x80000, norm_eps=1e-6)
    assert lib.i4_moe_forward(0x30000, 1, 1, ctypes.byref(nrm), 8, 1, 0x90000, None, 0x70000,
                              None, None, 0x100000, ws, None) == -1
    assert lib.i4_moe_stack_workspace_bytes(1, 2048, 768, 128, 8) > ws
    # the bounded form takes the fused 2..64-token launch only, checked before any launch
    ws32 = lib.i4_moe_workspace_bytes(32, 2048, 768, 128, 8)
    bnd = lambda **kw: lib.i4_moe_forward_bounded(
        0x30000, 1, kw.get("T", 32), kw.get("mw", ctypes.byref(mw)), 8, 1, kw.get("lg"), None,
        0x70000, 0x100000, kw.get("wsb", ws32), kw.get("polls", 3), kw.get("mode", 1), None)
    assert bnd(mw=None) == -1
    assert bnd(T=1) == -2
    assert bnd(T=65) == -2
    assert bnd(polls=-1) == -2
    assert bnd(mode=3) == -2 and bnd(mode=-1) == -2
    # mode 2 bounds the fused routing launch, which needs the router in the block
    assert bnd(mode=2, lg=0x90000) == -2
    assert bnd(wsb=ws32 - 1) == -7
    g64 = _lib.MoeWeightsC(gate_up=gu, down=_qw(_lib, E=128, N=2048, K=768, group=64, layout=2),
                           router_w=0x60000)
    assert bnd(mw=ctypes.byref(g64)) == -2  # different group sizes: nothing waits


def test_decode_attention_validation_codes(pkg):
    """i4_attn_decode / i4_rmsnorm / i4_rmsnorm_linear reject bad calls before any launch."""
    from qwen3_omni_duplex_amd import _lib

    lib = pkg.lib()
    tab = (ctypes.c_float * 64)(*([1.0] * 64))
    ws = lib.i4_attn_decode_workspace_bytes(32, 128, 4096)
    assert ws > 0 and lib.i4_attn_decode_workspace_bytes(32, 64, 4096) == 0
    call = lambda **kw: lib.i4_attn_decode(
        kw.get("qkv", 0x30000), kw.get("xt", 2), kw.get("nh", 32), kw.get("nkv", 4),
        kw.get("hd", 128), 0x40000, 0x50000, 1e-6, kw.get("tab", tab), kw.get("pos", 5),
        kw.get("kc", 0x100000), 0x200000, kw.get("ml", 4096), 0x60000, kw.get("ws", 0x300000),
        kw.get("wsb", ws), None)
    assert call(qkv=None) == -1
    assert call(tab=None) == -1
    assert call(xt=0) == -3
    assert call(hd=64) == -2            # head_dim is 128
    assert call(nkv=5) == -2            # heads per kv head must divide
    assert call(nh=64, nkv=4) == -2     # at most 8 query heads per kv head
    assert call(pos=4096) == -2         # the row for this token must exist
    assert call(pos=-1) == -2
    assert call(ml=70000) == -2         # merge bound: 1024 chunks of 64
    assert call(kc=0x100008) == -4      # caches 16-byte aligned
    assert call(wsb=ws - 1) == -7
    assert call(ws=0x300010) == -4
    assert lib.i4_rmsnorm(0x30000, 1, 1, 4100, 0x40000, 1e-6, 0x50000, None) == -2
    assert lib.i4_rmsnorm(0x30000, 0, 1, 2048, 0x40000, 1e-6, 0x50000, None) == -3
    assert lib.i4_rmsnorm(0x30008, 1, 1, 2048, 0x40000, 1e-6, 0x50000, None) == -4
    assert lib.i4_rmsnorm(0x30000, 1, 1, 2048, None, 1e-6, 0x50000, None) == -1
    w = _qw(_lib, E=1, N=5120, K=2048)
    assert lib.i4_rmsnorm_linear(0x30000, 1, 1, None, 1e-6, ctypes.byref(w), None, 0x50000, 1,
                                 None) == -1
    wk = _qw(_lib, E=1, N=2048, K=8192)
    assert lib.i4_rmsnorm_linear(0x30000, 1, 1, 0x40000, 1e-6, ctypes.byref(wk), None, 0x50000, 1,
                                 None) == -2
    wt = _qw(_lib, E=1, N=5120, K=2048, group=128, layout=2)
    assert lib.i4_rmsnorm_linear(0x30000, 1, 1, 0x40000, 1e-6, ctypes.byref(wt), None, 0x50000, 1,
                                 None) == -5

    assert lib.i4_attn_decode_at(0x30000, 2, 32, 4, 128, 0x40000, 0x50000, 1e-6, tab, None,
                                 0x100000, 0x200000, 4096, 0x60000, 0x300000, ws, None) == -1
    assert lib.i4_attn_decode_at(0x30000, 2, 32, 4, 128, 0x40000, 0x50000, 1e-6, tab, 0x70002,
                                 0x100000, 0x200000, 4096, 0x60000, 0x300000, ws, None) == -4

    # with o_proj: a CT weight of K = n_heads * head_dim, and a larger workspace (the
    # merged heads live in it after the partials, at a 256-byte boundary)
    wso = lib.i4_attn_decode_o_workspace_bytes(32, 128, 4096)
    # ... the o_proj wait's status word in a 256-byte slot in front of them (the router-fold
    # launch of the decoder layer keeps its output directly behind the merged heads)
    assert lib.i4_attn_decode_o_status_offset(32, 128, 4096) == (ws + 255) & ~255
    assert wso == ((ws + 255) & ~255) + 256 + 32 * 128 * 2
    ow = _qw(_lib, E=1, N=2048, K=4096, group=32)
    callo = lambda **kw: lib.i4_attn_decode_o(
        0x30000, 2, kw.get("nh", 32), 4, 128, 0x40000, 0x50000, 1e-6, tab, kw.get("pd", None),
        5, 0x100000, 0x200000, 4096, kw.get("ow", ctypes.byref(ow)), kw.get("res", 0x80000),
        kw.get("y", 0x90000), 0x300000, kw.get("wsb", wso), None)
    assert callo(ow=None) == -1
    assert callo(y=None) == -1
    assert callo(ow=ctypes.byref(_qw(_lib, E=1, N=2048, K=4096, group=128, layout=1))) == -5
    assert callo(ow=ctypes.byref(_qw(_lib, E=1, N=2048, K=2048, group=32))) == -2  # K != 32*128
    assert callo(ow=ctypes.byref(_qw(_lib, E=2, N=2048, K=4096, group=32))) == -2  # one weight
    assert callo(res=0x80001) == -4
    assert callo(wsb=ws) == -7          # the partials alone do not hold the merged heads
    assert callo(pd=0x70002) == -4

    # from the layer's input row: i4_attn_decode_o's workspace, then the q|k|v row as
    # (value pair, tag) words from a 256-byte boundary
    wsq = lib.i4_attn_decode_qkv_o_workspace_bytes(32, 4, 128, 4096)
    assert wsq == ((wso + 255) & ~255) + 40 * 128 * 4
    assert lib.i4_attn_decode_qkv_o_workspace_bytes(32, 4, 64, 4096) == 0
    qw = _qw(_lib, E=1, N=5120, K=2048, group=32)
    callq = lambda **kw: lib.i4_attn_decode_qkv_o(
        kw.get("h", 0x30000), kw.get("xt", 2), kw.get("nw", 0x40000), 1e-6,
        kw.get("qw", ctypes.byref(qw)), kw.get("nh", 32), 4, 128, 0x50000, 0x51000, tab,
        kw.get("pd", None), kw.get("pos", 5), 0x100000, 0x200000, 4096,
        kw.get("ow", ctypes.byref(ow)), kw.get("y", 0x90000), kw.get("ws", 0x300000),
        kw.get("wsb", wsq), None)
    assert callq(h=None) == -1
    assert callq(qw=None) == -1
    assert callq(y=None) == -1
    assert callq(xt=0) == -3
    assert callq(qw=ctypes.byref(_qw(_lib, E=1, N=5120, K=2048, group=128, layout=1))) == -5
    assert callq(qw=ctypes.byref(_qw(_lib, E=1, N=4096, K=2048, group=32))) == -2  # not 40 heads
    assert callq(qw=ctypes.byref(_qw(_lib, E=1, N=5120, K=1024, group=32))) == -2  # K != o_w.N
    assert callq(nh=16) == -2           # o_w.K != 16 * 128
    assert callq(h=0x30008) == -4
    assert callq(nw=0x40008) == -4
    assert callq(y=0x90001) == -4
    assert callq(wsb=wso) == -7         # the q|k|v row does not fit
    assert callq(ws=0x300080) == -4
    assert callq(pos=4096) == -2
    assert callq(pd=0x70002) == -4


def test_thinker_layer_validation_codes(pkg):
    """i4_thinker_layer_decode rejects bad calls before its first launch (Thinker sizes:
    32 / 4 heads, hidden 2048, 128 experts of FFN 768, top-8), and its workspace query
    returns 0 for sizes the entry does not take."""
    from qwen3_omni_duplex_amd import _lib

    lib = pkg.lib()
    tab = (ctypes.c_float * 64)()
    wsb = lib.i4_thinker_layer_workspace_bytes(32, 4, 128, 4096, 2048, 768, 128, 8)
    # MoE workspace, attention workspace + h2, the q|k|v row as (value pair, tag) words,
    # each from a 256-byte boundary
    parts = (lib.i4_moe_workspace_bytes(1, 2048, 768, 128, 8),
             lib.i4_attn_decode_o_workspace_bytes(32, 128, 4096) + 2048 * 2, 40 * 128 * 4)
    assert wsb == sum((b + 255) & ~255 for b in parts)
    fits = lambda **kw: lib.i4_thinker_layer_workspace_bytes(
        32, 4, kw.get("hd", 128), 4096, kw.get("H", 2048), kw.get("I", 768), 128, kw.get("k", 8))
    assert fits(H=1024) > 0
    assert fits(H=3072) == 0            # the router wave covers H 1024 and 2048
    assert fits(hd=64) == 0
    assert fits(k=9) == 0               # past the single-launch expert kernel
    assert fits(I=4096) == 0
    qw = _qw(_lib, E=1, N=5120, K=2048)
    ow = _qw(_lib, E=1, N=2048, K=4096)
    gu = _qw(_lib, E=128, N=1536, K=2048, group=128)
    dn = _qw(_lib, E=128, N=2048, K=768, group=128)
    mw = _lib.MoeWeightsC(gate_up=gu, down=dn, router_w=0x60000, norm_w=0x61000, norm_eps=1e-6)
    call = lambda **kw: lib.i4_thinker_layer_decode(
        kw.get("h", 0x30000), kw.get("xt", 1), 0x40000, 1e-6, ctypes.byref(kw.get("qw", qw)),
        kw.get("nh", 32), 4, 128, 0x50000, 0x51000, tab, kw.get("pd", None), kw.get("pos", 5),
        0x100000, 0x200000, 4096, ctypes.byref(kw.get("ow", ow)), ctypes.byref(kw.get("mw", mw)),
        kw.get("k", 8), 1, kw.get("out", 0x70000), kw.get("ws", 0x1000000), kw.get("wsb", wsb),
        None)
    assert call(h=None) == -1
    assert call(out=None) == -1
    assert call(xt=0) == -3
    assert call(ow=_qw(_lib, E=1, N=2048, K=4096, group=128, layout=1)) == -5
    assert call(mw=_lib.MoeWeightsC(gate_up=gu, down=dn, router_w=None, norm_w=0x61000)) == -1
    assert call(mw=_lib.MoeWeightsC(gate_up=gu, down=dn, router_w=0x60000, norm_w=None)) == -1
    tile = _lib.MoeWeightsC(gate_up=_qw(_lib, E=128, N=1536, K=2048, group=128, layout=2),
                            down=_qw(_lib, E=128, N=2048, K=768, group=128, layout=2),
                            router_w=0x60000, norm_w=0x61000)
    assert call(mw=tile) == -5
    assert call(k=9) == -2
    assert call(qw=_qw(_lib, E=1, N=5000, K=2048)) == -2    # rows of 32 + 2 x 4 heads
    assert call(ow=_qw(_lib, E=1, N=1024, K=4096)) == -2    # o_proj rows = H
    assert call(nh=16) == -2
    assert call(out=0x70008) == -4
    assert call(wsb=wsb - 1) == -7
    assert call(ws=None) == -7
    assert call(ws=0x1000010) == -4
    assert call(pos=4096) == -2         # the attention's checks come before any launch
    assert call(pd=0x70002) == -4

    # the decode step: the layer's workspace and the hidden state between layers; every
    # layer is checked before the first launch
    wss = lib.i4_thinker_decode_step_workspace_bytes(32, 4, 128, 4096, 2048, 768, 128, 8)
    assert wss == wsb + 2 * 4096 + 8 * 4096
    assert lib.i4_thinker_decode_step_workspace_bytes(32, 4, 128, 4096, 3072, 768, 128, 8) == 0

    def layer(**kw):
        return _lib.ThinkerLayerC(in_norm_w=kw.get("nw", 0x40000), q_norm_w=0x50000,
                                  k_norm_w=0x51000, k_cache=kw.get("kc", 0x100000),
                                  v_cache=0x200000, eps=1e-6, qkv=qw, o=ow,
                                  moe=kw.get("mw", mw))

    def step(ls, **kw):
        arr = (_lib.ThinkerLayerC * len(ls))(*ls)
        return lib.i4_thinker_decode_step(
            kw.get("h", 0x30000), 1, arr, kw.get("n", len(ls)), 32, 4, 128, tab, None,
            kw.get("pos", 5), 4096, 8, 1, 0x70000, 0x1000000, kw.get("wsb", wss), None)

    good = layer()
    assert step([good, good], h=None) == -1
    assert step([good, good], n=0) == -2
    assert step([good, good], wsb=wss - 1) == -7
    assert step([good, good], pos=4096) == -2
    assert step([good, layer(nw=None)]) == -1           # the last layer's checks too
    assert step([good, layer(kc=0x100008)]) == -4
    assert step([good, layer(mw=tile)]) == -5
    other = _lib.MoeWeightsC(gate_up=_qw(_lib, E=64, N=1536, K=2048, group=128),
                             down=_qw(_lib, E=64, N=2048, K=768, group=128),
                             router_w=0x60000, norm_w=0x61000)
    assert step([good, layer(mw=other)]) == -2           # one workspace layout for all


def test_dense_moe_validation_codes(pkg):
    """i4_dmoe_forward rejects bad calls before any launch (Talker shapes: H 1024,
    E 128, I 384, shared I 768, top-6)."""
    from qwen3_omni_duplex_amd import _lib

    lib = pkg.lib()
    ws = lib.i4_dmoe_workspace_bytes(1, 128, 6, 384, 768)
    assert ws > 0 and lib.i4_dmoe_workspace_bytes(0, 128, 6, 384, 768) == 0

    def dw(data, E, N, K, scale=None):
        return _lib.DWeightC(data=data, scale=scale, E=E, N=N, K=K)

    def weights(**kw):
        w = _lib.DmoeWeightsC(
            gate_up=kw.get("gu", dw(0x100000, 128, 768, 1024)),
            down=kw.get("dn", dw(0x200000, 128, 1024, 384)),
            router_w=kw.get("rw", 0x300000),
            shared_gate_up=kw.get("sgu", dw(0x400000, 1, 1536, 1024)),
            shared_down=kw.get("sdn", dw(0x500000, 1, 1024, 768)),
            shared_gate_w=kw.get("sgw", 0x600000))
        return w

    def call(w=None, xt=2, T=1, k=6, x=0x30000, wsb=ws, wsp=0x700000, logits=None):
        w = weights() if w is None else w
        return lib.i4_dmoe_forward(x, xt, T, ctypes.byref(w), k, 1, logits, None, 0x40000, None,
                                   None, wsp, wsb, None)

    assert call(x=None) == -1
    assert call(w=weights(rw=None)) == -1                       # no router and no logits
    assert call(xt=0) == -3
    assert call(T=0) == -2 and call(T=65536) == -2
    assert call(k=8) == -2                                      # 7 slots + the shared expert
    assert call(w=weights(gu=dw(0x100000, 128, 768, 1000))) == -2   # H % 16
    assert call(w=weights(gu=dw(0x100000, 128, 768, 4096))) == -2   # H <= 2048
    assert call(w=weights(dn=dw(0x200000, 128, 1024, 380))) == -2   # down K = I
    assert call(w=weights(dn=dw(0x200000, 64, 1024, 384))) == -2    # same E
    assert call(w=weights(gu=dw(0x100008, 128, 768, 1024))) == -4   # 16-byte rows
    assert call(w=weights(gu=dw(0x100000, 128, 768, 1024, scale=0x800000))) == -3  # mixed
    assert call(w=weights(sgu=dw(0x400000, 2, 1536, 1024))) == -2   # one shared expert
    assert call(w=weights(sgu=dw(0, 1, 1536, 1024))) == -1          # shared down, no gate|up
    assert call(w=weights(sgu=dw(0x400000, 1, 4096, 1024),
                          sdn=dw(0x500000, 1, 1024, 2048))) == -2   # 16-bit shared I <= 1024
    assert call(wsb=ws - 1) == -7
    assert call(wsp=0x700008) == -4

    # the single-launch block's down stage on its own: one token, given logits
    def wait(w=None, xt=2, k=6, logits=0x50000, polls=16, wsb=ws):
        w = weights() if w is None else w
        return lib.i4_dmoe_down_wait(0x30000, xt, ctypes.byref(w), k, 1, logits, None, 0x40000,
                                     0x700000, wsb, polls, None)

    assert wait(xt=0) == -3
    assert wait(logits=None) == -2                              # ranks the given logits
    assert wait(polls=-1) == -2
    assert wait(k=8) == -2
    assert wait(wsb=ws - 1) == -7
    big = weights(dn=dw(0x200000, 128, 1024, 1024), gu=dw(0x100000, 128, 2048, 1024))
    assert wait(w=big, wsb=1 << 30) == -2                       # 6 x 1024 + 768 > 4096 staged
    q8 = weights(gu=dw(0x100000, 128, 768, 1024, scale=0x800000),
                 dn=dw(0x200000, 128, 1024, 384, scale=0x900000))
    assert wait(w=q8) == -3                                     # int8 experts: three launches


def test_dense_moe_status_word_lies_inside_the_workspace(pkg):
    lib = pkg.lib()
    for T, E, k, I, Is in ((1, 128, 6, 384, 768), (5, 128, 6, 384, 0), (1, 16, 4, 48, 32)):
        off = lib.i4_dmoe_status_offset(T, E, k, I, Is)
        assert off % 4 == 0 and 0 < off and off + 4 <= lib.i4_dmoe_workspace_bytes(T, E, k, I, Is)
    assert lib.i4_dmoe_status_offset(0, 128, 6, 384, 768) == 0


def test_status_word_lies_inside_the_workspace(pkg):
    lib = pkg.lib()
    for T, H, I, E, k in ((1, 2048, 768, 128, 8), (32, 2048, 768, 128, 8), (512, 1024, 384, 64, 6)):
        off = lib.i4_moe_status_offset(T, H, I, E, k)
        assert off % 4 == 0 and 0 < off and off + 4 <= lib.i4_moe_workspace_bytes(T, H, I, E, k)
    assert lib.i4_moe_status_offset(0, 2048, 768, 128, 8) == 0


def test_whole_row_group_is_per_channel(pkg):
    """A group at least as long as the row is one scale per output row (the reference's
    per-channel branch, quant/dequant.py:75-76): accepted, where other non-powers of two are
    refused."""
    from qwen3_omni_duplex_amd import _lib

    lib = pkg.lib()
    for group, K, code in ((768, 768, -1), (1000, 768, -1), (96, 768, -6), (48, 256, -6)):
        w = _qw(_lib, group=group, K=K)
        # sel = NULL: a valid weight gets as far as the pointer check
        rc = lib.i4_dq_gemv(0x30000, 1, 0, ctypes.byref(w), None, 8, 0x50000, 0, None, 0, None)
        assert rc == code, (group, K, rc)


def test_down_wait_validation_codes(pkg):
    from qwen3_omni_duplex_amd import _lib

    lib = pkg.lib()
    dn = _qw(_lib, E=128, N=2048, K=768, group=128)
    args = dict(act=0x30000, xt=1, lg=0x40000, E_r=128, k=8, renorm=1, res=None, out=0x50000,
                status=0x60000, polls=16)

    def call(**kw):
        a = dict(args, **kw)
        return lib.i4_moe_down_wait(a["act"], a["xt"], ctypes.byref(dn), a["lg"], a["E_r"], a["k"],
                                    a["renorm"], a["res"], a["out"], a["status"], a["polls"], None)

    assert call(status=None) == -1
    assert call(act=None) == -1
    assert call(xt=0) == -3
    assert call(k=9) == -2            # the single-launch layer covers top-k <= 8
    assert call(E_r=129) == -2
    assert call(polls=-1) == -2
    assert call(out=0x50008) == -4
    tile = _qw(_lib, E=128, N=2048, K=768, group=128, layout=2)
    assert lib.i4_moe_down_wait(0x30000, 1, ctypes.byref(tile), 0x40000, 128, 8, 1, None, 0x50000,
                                0x60000, 16, None) == -5

"""CPU oracle for the int4 clock path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker: the product (libi4moe) never calls it
and has no CPU fallback.

A numpy restatement of the reference's algorithm for the quantized clock path
(thecodacus/qwen3-omni-duplex); every function cites the reference lines it
follows.  Integer work (nibble packing, unpacking, routing indices) is exact;
floating-point work is done in float64, with the reference's half-precision
rounding points applied where the reference has them.

Pinning (tests/test_oracle.py): every function below is checked against the
known-answer vectors in tests/golden/ (written by an independent pure-Python
script), against closed forms (z = 8 reduction, CT <-> AWQ layout
equivalence, round trips) and against library routines (numpy matmul,
torch.topk / torch.softmax on tie-free rows).  No function is unpinned.
"""
from __future__ import annotations

import numpy as np

PACK = 8                            # nibbles per int32 (fused_packed_moe.py:33-34)
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)  # nibble slot i holds column AWQ_ORDER[i]
AWQ_SLOT = tuple(AWQ_ORDER.index(c) for c in range(8))  # column c -> nibble slot


# ---------------------------------------------------------------------------
# half-precision helpers (bf16 has no numpy dtype: carried as uint16 bits)
def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet)."""
    u = np.asarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = np.isnan(np.asarray(a, dtype=np.float32))
    return np.where(nan, np.uint16(0x7FC0), rounded.astype(np.uint16)).astype(np.uint16)


def round_half(a: np.ndarray, dtype: str) -> np.ndarray:
    """Round to fp16 / bf16 and return the rounded values as float64."""
    if dtype == "f16":
        return np.asarray(a, dtype=np.float64).astype(np.float16).astype(np.float64)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(a, dtype=np.float32))).astype(np.float64)
    if dtype == "f32":
        return np.asarray(a, dtype=np.float32).astype(np.float64)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# CT layout: src/duplex/streaming/fused_packed_moe.py:54-65 (unpack4),
# src/duplex/streaming/triton_dequant_gemv.py:12-14,63, quant/dequant.py:23-27
def ct_nibbles(packed: np.ndarray, cols: int | None = None) -> np.ndarray:
    """[..., C] int32 -> [..., C*8] uint8 raw nibbles; column 8m+i = (word m >> 4i) & 15."""
    u = np.asarray(packed).astype(np.int64) & 0xFFFFFFFF
    shifts = np.arange(PACK, dtype=np.int64) * 4
    q = ((u[..., None] >> shifts) & 0xF).astype(np.uint8)
    q = q.reshape(*u.shape[:-1], u.shape[-1] * PACK)
    return q if cols is None else q[..., :cols]


def unpack4(packed: np.ndarray, out_cols: int) -> np.ndarray:
    """The reference's signed unpack: nibble - 8 (fused_packed_moe.py:65)."""
    return ct_nibbles(packed, out_cols).astype(np.int32) - 8


def ct_pack(q: np.ndarray) -> np.ndarray:
    """[..., K] values 0..15 -> [..., K/8] int32 (inverse of ct_nibbles)."""
    q = np.asarray(q).astype(np.int64)
    if q.shape[-1] % PACK:
        raise ValueError("K must be a multiple of 8")
    q = q.reshape(*q.shape[:-1], q.shape[-1] // PACK, PACK)
    word = np.zeros(q.shape[:-1], dtype=np.int64)
    for i in range(PACK):
        word |= (q[..., i] & 0xF) << (4 * i)
    return word.astype(np.uint32).view(np.int32)


# ---------------------------------------------------------------------------
# AWQ layout (AutoAWQ GEMM packing; no counterpart in the reference, which
# ships only CT checkpoints -- pinned by known answers and CT equivalence)
def awq_pack(q: np.ndarray) -> np.ndarray:
    """[..., N] values 0..15 -> [..., N/8] int32, slot i <- column 8w + AWQ_ORDER[i]."""
    q = np.asarray(q).astype(np.int64)
    q = q.reshape(*q.shape[:-1], q.shape[-1] // PACK, PACK)
    word = np.zeros(q.shape[:-1], dtype=np.int64)
    for i in range(PACK):
        word |= (q[..., AWQ_ORDER[i]] & 0xF) << (4 * i)
    return word.astype(np.uint32).view(np.int32)


def awq_nibbles(packed: np.ndarray) -> np.ndarray:
    """[..., N/8] int32 -> [..., N] uint8 in column order."""
    u = np.asarray(packed).astype(np.int64) & 0xFFFFFFFF
    slots = np.array(AWQ_SLOT, dtype=np.int64) * 4
    q = ((u[..., None] >> slots) & 0xF).astype(np.uint8)
    return q.reshape(*u.shape[:-1], u.shape[-1] * PACK)


# ---------------------------------------------------------------------------
# dequantisation: FusedPackedMoE._dequant (fused_packed_moe.py:183-189) and
# dequantize_weight (quant/dequant.py:67-74): value = (q - z) * s per group,
# z = 8 for the reference's symmetric format.
def ct_dequant(packed, scale, K, group, zeros=None) -> np.ndarray:
    """CT [..., N, K/8] (+ scale [..., N, NG], zeros [..., N, ceil(NG/8)]) -> float64 [..., N, K]."""
    q = ct_nibbles(packed, K).astype(np.float64)
    g = np.arange(K) // group
    s = np.asarray(scale, dtype=np.float64)[..., g]
    if zeros is None:
        z = 8.0
    else:
        zn = ct_nibbles(zeros).astype(np.float64)      # [..., N, NZW*8]
        z = zn[..., g]
    return (q - z) * s


def awq_dequant(qweight, qzeros, scales, group) -> np.ndarray:
    """AWQ qweight [..., K, N/8] -> float64 [..., N, K] (the logical y = W x form)."""
    q = awq_nibbles(qweight).astype(np.float64)          # [..., K, N]
    K = q.shape[-2]
    g = np.arange(K) // group
    z = awq_nibbles(qzeros).astype(np.float64)[..., g, :] if qzeros is not None else 8.0
    s = np.asarray(scales, dtype=np.float64)[..., g, :]
    w = (q - z) * s                                       # [..., K, N]
    return np.swapaxes(w, -1, -2)


def awq_to_ct(qweight, qzeros, scales, group):
    """AWQ -> CT + explicit zeros, the library's load-time repack.

    Returns (packed [E, N, K/8], scale [E, N, NG], zeros [E, N, ceil(NG/8)]).
    """
    q = np.swapaxes(awq_nibbles(qweight), -1, -2)         # [..., N, K]
    zn = np.swapaxes(awq_nibbles(qzeros), -1, -2)         # [..., N, NG]
    NG = zn.shape[-1]
    pad = (-NG) % 8
    if pad:
        zn = np.concatenate([zn, np.zeros(zn.shape[:-1] + (pad,), np.uint8)], axis=-1)
    return ct_pack(q), np.swapaxes(np.asarray(scales), -1, -2).copy(), ct_pack(zn)


# ---------------------------------------------------------------------------
# The library's tile layout (I4_LAYOUT_TILE in include/i4moe.h).  No reference
# counterpart: a permutation of the CT words, pinned by its closed form
# (test_tile_index_closed_form) and its round trip.
TILE_NIBBLE_ORDER = AWQ_ORDER  # tile word nibble slot i holds column 8m + order[i]


def interleave_words(words, order=TILE_NIBBLE_ORDER) -> np.ndarray:
    """CT words (nibble i = column 8m + i) -> words whose slot i holds column 8m + order[i]."""
    w = np.asarray(words).astype(np.int64) & 0xFFFFFFFF
    out = np.zeros_like(w)
    for i, c in enumerate(order):
        out |= ((w >> (4 * c)) & 0xF) << (4 * i)
    return out.astype(np.uint32).view(np.int32)


def deinterleave_words(words, order=TILE_NIBBLE_ORDER) -> np.ndarray:
    """Inverse of interleave_words."""
    w = np.asarray(words).astype(np.int64) & 0xFFFFFFFF
    out = np.zeros_like(w)
    for i, c in enumerate(order):
        out |= ((w >> (4 * i)) & 0xF) << (4 * c)
    return out.astype(np.uint32).view(np.int32)


def tile_pack(packed, scale, zeros=None):
    """CT (packed [E, N, K/8], scale [E, N, NG], zeros [E, N, NZW] or None) -> tile.

    packed -> [E, N/16, K/128, 16, 16]: element [e, b, s, r, 4j + t] is CT word
    4 (4s + t) + j of row 16b + r with its nibbles interleaved (slot i holds
    column 8m + (0, 2, 4, 6, 1, 3, 5, 7)[i]); scale -> [E, N/16, NG, 16]; zeros
    -> [E, N/16, NZW, 16] (element [e, b, g, r] = CT element [e, 16b + r, g],
    zero words unchanged).
    """
    p = np.asarray(packed)
    E, N, KW = p.shape
    SC = KW // 16
    t = interleave_words(p).reshape(E, N // 16, 16, SC, 4, 4)   # [e, b, r, s, t, j]
    t = t.transpose(0, 1, 3, 2, 5, 4).reshape(E, N // 16, SC, 16, 16)

    def rows(a):
        a = np.asarray(a)
        return a.reshape(E, N // 16, 16, a.shape[-1]).transpose(0, 1, 3, 2).copy()

    return t.copy(), rows(scale), None if zeros is None else rows(zeros)


def tile_unpack(packed, scale, zeros=None):
    """Inverse of tile_pack: tile -> CT."""
    p = np.asarray(packed)
    E, NB, SC = p.shape[:3]
    c = p.reshape(E, NB, SC, 16, 4, 4).transpose(0, 1, 3, 2, 5, 4).reshape(E, NB * 16, SC * 16)
    c = deinterleave_words(c)

    def rows(a):
        a = np.asarray(a)
        return a.transpose(0, 1, 3, 2).reshape(E, NB * 16, a.shape[2]).copy()

    return c.copy(), rows(scale), None if zeros is None else rows(zeros)


# ---------------------------------------------------------------------------
# GEMV: _dq_gemv_kernel / dequant_gemv / reference_gemv
# (triton_dequant_gemv.py:43-82, 85-113, 116-122)
def dq_gemv(x, W, sel) -> np.ndarray:
    """out[j, r] = sum_c W[sel[j], r, c] * x[j or shared, c] in float64.

    x: [K] (shared, s_x = 0) or [k, K] (per expert, s_x = K); W dense [E, N, K].
    """
    x = np.asarray(x, dtype=np.float64)
    Wd = np.asarray(W, dtype=np.float64)[np.asarray(sel)]
    if x.ndim == 1:
        return np.einsum("jrc,c->jr", Wd, x)
    return np.einsum("jrc,jc->jr", Wd, x)


# ---------------------------------------------------------------------------
# routing: FusedPackedMoE.forward (fused_packed_moe.py:195-199)
#   w = softmax(logits, dtype=float); w, sel = topk(w, k); w /= w.sum(); w.to(dtype)
def topk_sel(logits: np.ndarray, k: int) -> np.ndarray:
    """Top-k expert ids per row, value descending, ties -> lower id."""
    lg = np.asarray(logits, dtype=np.float64)
    E = lg.shape[-1]
    # lexsort: last key is primary -> (-value, index)
    idx = np.arange(E)
    out = np.empty(lg.shape[:-1] + (k,), dtype=np.int64)
    flat = lg.reshape(-1, E)
    of = out.reshape(-1, k)
    for t in range(flat.shape[0]):
        order = np.lexsort((idx, -flat[t]))
        of[t] = order[:k]
    return out


def route(logits: np.ndarray, k: int, renorm: bool = True):
    """(sel int64 [T, k], w float64 [T, k]); logits are the half-precision values."""
    lg = np.asarray(logits, dtype=np.float64)
    sel = topk_sel(lg, k)
    m = lg.max(axis=-1, keepdims=True)
    p = np.exp(lg - m)
    p = p / p.sum(axis=-1, keepdims=True)
    w = np.take_along_axis(p, sel, axis=-1)
    if renorm:
        w = w / w.sum(axis=-1, keepdims=True)
    return sel, w


def router_logits(x, router_w, dtype: str) -> np.ndarray:
    """gate(x) (fused_packed_moe.py:112,195): fp64 product rounded to the activation dtype."""
    return round_half(np.asarray(x, np.float64) @ np.asarray(router_w, np.float64).T, dtype)


# ---------------------------------------------------------------------------
# pre-MoE RMSNorm of the Thinker decoder layer (post_attention_layernorm; the
# caller in front of FusedPackedMoE).  transformers 5.15
# Qwen3OmniMoeThinkerTextRMSNorm.forward (modeling_qwen3_omni_moe.py:1388-1393):
#   h = x.float(); h = h * rsqrt(mean(h^2) + eps); return weight * h.to(dtype)
def rmsnorm(x, weight, eps: float, dtype: str) -> np.ndarray:
    xf = np.asarray(x, np.float64)
    var = np.mean(xf * xf, axis=-1, keepdims=True)
    xn = round_half(xf / np.sqrt(var + eps), dtype)
    return round_half(xn * np.asarray(weight, np.float64), dtype)


# ---------------------------------------------------------------------------
# MoE block: Triton branch of FusedPackedMoE.forward (fused_packed_moe.py:222-263)
# with the CPU branch's fp32-everywhere arithmetic (:202-220); act is rounded to
# the activation dtype between the projections exactly as :257 does.
def silu(v: np.ndarray) -> np.ndarray:
    return v / (1.0 + np.exp(-v))


def ref_combine(ys, w, dtype: str, residual=None) -> np.ndarray:
    """The reference's own combine of one token (fused_packed_moe.py:199,262): the routing
    weights rounded to the activation dtype (w.to(x.dtype)), each expert output rounded
    (y.to(x.dtype)), their products rounded to the dtype (a 16-bit tensor multiply), the k
    products summed in fp32 in slot order and rounded once (torch's 16-bit sum accumulates
    in fp32); the decoder layer then adds the residual in the dtype.
    ys [k, H], w [k] -> [H] (values of the dtype, as float64)."""
    wr = round_half(np.asarray(w, np.float64), dtype)
    prods = round_half(round_half(np.asarray(ys, np.float64), dtype) * wr[:, None], dtype)
    acc = np.zeros(prods.shape[1], np.float32)
    for p in prods:
        acc = (acc + p.astype(np.float32)).astype(np.float32)
    out = round_half(acc.astype(np.float64), dtype)
    if residual is not None:
        out = round_half(out + np.asarray(residual, np.float64), dtype)
    return out


def moe_layer(x, sel, w, Wgu, Wdn, act_dtype: str | None, residual=None,
              out_dtype: str | None = None, y_dtype: str | None = None,
              combine: str = "exact") -> np.ndarray:
    """x [T, H]; sel/w [T, k]; Wgu dense [E, 2I, H] (gate rows first); Wdn dense [E, H, I].

    y_dtype rounds each expert's output before the routing-weighted sum, the
    reference's y.to(x.dtype) (fused_packed_moe.py:262); with combine="exact" the sum
    itself stays float64.  combine="reference" models the reference's own rounding of
    the combine instead (ref_combine, in act_dtype), residual included."""
    x = np.asarray(x, np.float64)
    T = x.shape[0]
    I = Wgu.shape[1] // 2
    H = Wdn.shape[1]
    out = np.zeros((T, H), np.float64)
    for t in range(T):
        ys = []
        for j in range(sel.shape[1]):
            e = int(sel[t, j])
            gu = Wgu[e] @ x[t]
            a = silu(gu[:I]) * gu[I:]
            if act_dtype is not None:
                a = round_half(a, act_dtype)
            y = Wdn[e] @ a
            if y_dtype is not None:
                y = round_half(y, y_dtype)
            ys.append(y)
            out[t] += w[t, j] * y
        if combine == "reference":
            res_t = None if residual is None else np.asarray(residual, np.float64)[t]
            out[t] = ref_combine(np.stack(ys), w[t], act_dtype, res_t)
    if combine == "reference":
        return out
    if residual is not None:
        out = out + np.asarray(residual, np.float64)
    if out_dtype is not None:
        out = round_half(out, out_dtype)
    return out


def moe_layer_grouped(x, sel, w, dense_gu, dense_dn, act_dtype, residual=None,
                      y_dtype: str | None = None):
    """Same as moe_layer, computed per expert over all its tokens (for large T).

    dense_gu(e) / dense_dn(e) return expert e's dense matrices on demand so only
    the selected experts are ever dequantised.
    """
    x = np.asarray(x, np.float64)
    T, k = sel.shape
    H = x.shape[1]
    out = np.zeros((T, H), np.float64)
    for e in np.unique(sel):
        tt, jj = np.nonzero(sel == e)
        Wg = dense_gu(int(e))
        I = Wg.shape[0] // 2
        gu = x[tt] @ Wg.T                      # [n, 2I]
        a = silu(gu[:, :I]) * gu[:, I:]
        if act_dtype is not None:
            a = round_half(a, act_dtype)
        y = a @ dense_dn(int(e)).T             # [n, H]
        if y_dtype is not None:
            y = round_half(y, y_dtype)
        np.add.at(out, tt, w[tt, jj][:, None] * y)
    if residual is not None:
        out = out + np.asarray(residual, np.float64)
    return out


# ---------------------------------------------------------------------------
# Talker MoE block: FusedMoE (src/duplex/streaming/fused_moe.py:40-141), the
# stand-in for transformers' Qwen3OmniMoeTalkerTextSparseMoeBlock
# (modeling_qwen3_omni_moe.py:2712-2733, transformers 5.15).
def q8_quantize(W, dtype: str):
    """Per-output-channel symmetric int8 of fused_moe.py:84-94, with the 16-bit
    arithmetic of the reference's tensors: every op computes in fp32 and rounds
    to `dtype` (the weights' dtype).
        s = (amax_k |W| clamped at 1e-8) / 127;  q = clamp(round(W / s), -127, 127)
    W [..., N, K] holds values exactly representable in `dtype`.
    Returns (q int8 [..., N, K], s float64 [..., N, 1])."""
    W32 = np.asarray(W, np.float32)
    floor = np.float32(round_half(np.array([1e-8], np.float32), dtype)[0])
    amax = np.maximum(np.abs(W32).max(axis=-1, keepdims=True), floor)
    s = round_half(amax / np.float32(127.0), dtype).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        r = round_half(W32 / s, dtype)                  # the 16-bit quotient
    # an all-zero fp16 row has s = 0 (1e-8 underflows in fp16): its 0 / 0 quotients
    # convert to q = 0, as torch's NaN -> int8 conversion gives
    r = np.where(np.isnan(r), 0.0, r)
    q = np.clip(np.round(r), -127, 127).astype(np.int8)  # round half to even
    return q, s.astype(np.float64)


def sigmoid(v):
    return 1.0 / (1.0 + np.exp(-np.asarray(v, np.float64)))


def dense_moe(x, sel, w, Wgu, Wdn, act_dtype: str | None, shared=None, residual=None,
              out_dtype: str | None = None) -> np.ndarray:
    """FusedMoE.forward after routing (fused_moe.py:110-141), fp64.

    x [T, H]; sel / w [T, k]; Wgu [E, 2I, H] (gate rows first); Wdn [E, H, I].
    shared = (Wsgu [2Is, H], Wsdn [H, Is], gate_w [H] or None) adds
    sigmoid(gate_w . x) * down_s(silu(gate_s x) * up_s x) (fused_moe.py:136-140).
    act_dtype rounds each activation (routed and shared), the shared gate's logit
    and its sigmoid to the activation dtype, where the reference's 16-bit
    tensors round them (:127, :139)."""
    x = np.asarray(x, np.float64)
    out = moe_layer(x, sel, w, Wgu, Wdn, act_dtype)
    if shared is not None:
        Wsgu, Wsdn, gate_w = shared
        Is = Wsgu.shape[0] // 2
        gu = x @ np.asarray(Wsgu, np.float64).T                 # [T, 2Is]
        a = silu(gu[:, :Is]) * gu[:, Is:]
        if act_dtype is not None:
            a = round_half(a, act_dtype)
        y = a @ np.asarray(Wsdn, np.float64).T                  # [T, H]
        if gate_w is None:
            g = np.ones((x.shape[0], 1))
        else:
            z = x @ np.asarray(gate_w, np.float64).reshape(-1, 1)
            if act_dtype is not None:
                z = round_half(z, act_dtype)
            g = sigmoid(z)
            if act_dtype is not None:
                g = round_half(g, act_dtype)
        out = out + g * y
    if residual is not None:
        out = out + np.asarray(residual, np.float64)
    if out_dtype is not None:
        out = round_half(out, out_dtype)
    return out


def rel_err(got, ref) -> float:
    """max |got - ref| / max |ref| -- the tolerance measure of the parity bar."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(got - ref)) / (den if den > 0 else 1.0))

"""Write tests/golden/known_answers.json -- known-answer vectors for the oracle.

The reference ships no tests, fixtures or golden vectors for this path, so
these vectors are derived here from first principles, with an implementation
deliberately independent of oracle/i4ref.py: bit-by-bit loops over Python ints,
exact rational arithmetic (fractions.Fraction) and math.exp, no numpy.

  - CT packing: column 8m+i of a row is nibble i of word m
    (src/duplex/streaming/fused_packed_moe.py:55-60, triton_dequant_gemv.py:12-14).
  - AWQ packing: nibble slot i of a word holds column (0,2,4,6,1,3,5,7)[i]
    (AutoAWQ GEMM format); [0..7] packs to 0x75316420.
  - value = (q - z) * s per group; z = 8 for the symmetric CT checkpoint
    (quant/dequant.py:23-27,73; fused_packed_moe.py:65,183-189).
  - routing: softmax, top-k (ties to the lower id), renormalise
    (fused_packed_moe.py:195-199).

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
import random
from fractions import Fraction
from pathlib import Path

OUT = Path(__file__).with_name("known_answers.json")
AWQ_ORDER = [0, 2, 4, 6, 1, 3, 5, 7]


def to_i32(u: int) -> int:
    return u - (1 << 32) if u & 0x80000000 else u


def ct_word(vals):
    w = 0
    for i, v in enumerate(vals):
        w += v * 16 ** i
    return to_i32(w)


def awq_word(cols):
    w = 0
    for slot in range(8):
        w += cols[AWQ_ORDER[slot]] * 16 ** slot
    return to_i32(w)


def ct_unpack_word(word):
    u = word & 0xFFFFFFFF
    out = []
    for _ in range(8):
        out.append(u % 16)
        u //= 16
    return out


def awq_unpack_word(word):
    u = word & 0xFFFFFFFF
    slots = []
    for _ in range(8):
        slots.append(u % 16)
        u //= 16
    cols = [0] * 8
    for slot in range(8):
        cols[AWQ_ORDER[slot]] = slots[slot]
    return cols


def main() -> None:
    rng = random.Random(20261201)
    ka = {}

    # 1. packing known answers
    ka["ct_words"] = [
        {"nibbles": list(range(8)), "word": ct_word(list(range(8)))},
        {"nibbles": [15, 0, 0, 0, 0, 0, 0, 8], "word": ct_word([15, 0, 0, 0, 0, 0, 0, 8])},
        {"nibbles": [8] * 8, "word": ct_word([8] * 8)},
    ]
    assert ka["ct_words"][0]["word"] == 0x76543210
    ka["awq_words"] = [
        {"cols": list(range(8)), "word": awq_word(list(range(8)))},
        {"cols": list(range(8, 16)), "word": awq_word(list(range(8, 16)))},
    ]
    assert ka["awq_words"][0]["word"] == 0x75316420
    words = [to_i32(rng.getrandbits(32)) for _ in range(64)]
    ka["random_words"] = {
        "words": words,
        "ct_nibbles": [ct_unpack_word(w) for w in words],
        "awq_cols": [awq_unpack_word(w) for w in words],
    }

    # 2. a CT g32 GEMV with exact rational answer: N=3 rows, K=64, symmetric
    K, N, G = 64, 3, 32
    q = [[rng.randrange(16) for _ in range(K)] for _ in range(N)]
    s = [[Fraction(rng.randrange(1, 64), 1024) for _ in range(K // G)] for _ in range(N)]
    x = [Fraction(rng.randrange(-64, 64), 32) for _ in range(K)]
    y = [sum((q[n][k] - 8) * s[n][k // G] * x[k] for k in range(K)) for n in range(N)]
    packed = [[ct_word(q[n][8 * m:8 * m + 8]) for m in range(K // 8)] for n in range(N)]
    ka["ct_gemv"] = {
        "K": K, "N": N, "group": G, "packed": packed,
        "scale": [[float(v) for v in row] for row in s],
        "x": [float(v) for v in x], "y": [float(v) for v in y],
    }

    # 3. AWQ g32 with zero points: the same logical matrix, explicit z
    z = [[rng.randrange(16) for _ in range(N + 5)] for _ in range(K // G)]  # [NG][N8] cols
    Nw = 8  # one AWQ word of columns; use N=8 columns
    qa = [[rng.randrange(16) for _ in range(Nw)] for _ in range(K)]        # [K][N]
    sa = [[Fraction(rng.randrange(1, 64), 1024) for _ in range(Nw)] for _ in range(K // G)]
    za = [[z[g][n] for n in range(Nw)] for g in range(K // G)]
    ya = [sum((qa[k][n] - za[k // G][n]) * sa[k // G][n] * x[k] for k in range(K))
          for n in range(Nw)]
    ka["awq_gemv"] = {
        "K": K, "N": Nw, "group": G,
        "qweight": [[awq_word(qa[k])] for k in range(K)],
        "qzeros": [[awq_word(za[g])] for g in range(K // G)],
        "scales": [[float(v) for v in row] for row in sa],
        "x": [float(v) for v in x], "y": [float(v) for v in ya],
    }

    # 4. routing known answers (ties resolved to the lower expert id)
    def route(logits, k):
        order = sorted(range(len(logits)), key=lambda e: (-logits[e], e))[:k]
        m = max(logits)
        ex = [math.exp(v - m) for v in logits]
        tot = sum(ex)
        p = [ex[e] / tot for e in order]
        ps = sum(p)
        return order, [v / ps for v in p]

    cases = [
        ([0.5, 2.0, 2.0, -1.0, 1.0, 2.0, 0.0, 3.0], 3),
        ([1.0] * 8, 4),
        ([-3.0, -1.0, -2.0, -1.0, 5.0, 5.0, 0.25, 0.25], 4),
    ]
    for _ in range(4):
        E = 16
        lg = [rng.randrange(-8, 8) / 4.0 for _ in range(E)]  # many exact ties
        cases.append((lg, 5))
    ka["routing"] = []
    for lg, k in cases:
        sel, w = route(lg, k)
        ka["routing"].append({"logits": lg, "k": k, "sel": sel, "w": w})

    # 5. a tiny symmetric CT MoE layer, pure-Python float arithmetic
    E, H, I, k = 4, 32, 32, 2
    qg = [[[rng.randrange(16) for _ in range(H)] for _ in range(2 * I)] for _ in range(E)]
    qd = [[[rng.randrange(16) for _ in range(I)] for _ in range(H)] for _ in range(E)]
    sg = [[rng.randrange(1, 32) / 256 for _ in range(2 * I)] for _ in range(E)]
    sd = [[rng.randrange(1, 32) / 256 for _ in range(H)] for _ in range(E)]
    xm = [rng.randrange(-32, 32) / 16 for _ in range(H)]
    lgm = [rng.randrange(-16, 16) / 8 for _ in range(E)]
    selm, wm = route(lgm, k)
    outm = [0.0] * H
    for j, e in enumerate(selm):
        gu = [sum((qg[e][r][c] - 8) * sg[e][r] * xm[c] for c in range(H)) for r in range(2 * I)]
        act = [gu[r] / (1 + math.exp(-gu[r])) * gu[I + r] for r in range(I)]
        for n in range(H):
            outm[n] += wm[j] * sum((qd[e][n][c] - 8) * sd[e][n] * act[c] for c in range(I))
    ka["moe_layer"] = {
        "E": E, "H": H, "I": I, "k": k, "group": 32,
        "gu_packed": [[[ct_word(qg[e][r][8 * m:8 * m + 8]) for m in range(H // 8)]
                       for r in range(2 * I)] for e in range(E)],
        "gu_scale": [[[v] for v in sg[e]] for e in range(E)],
        "dn_packed": [[[ct_word(qd[e][r][8 * m:8 * m + 8]) for m in range(I // 8)]
                       for r in range(H)] for e in range(E)],
        "dn_scale": [[[v] for v in sd[e]] for e in range(E)],
        "x": xm, "logits": lgm, "sel": selm, "w": wm, "out": outm,
    }

    OUT.write_text(json.dumps(ka, indent=1))
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()

"""Seeded synthetic inputs shared by the GPU tests (numpy on the host).

Distributions follow the workload definitions: int4 values and zero points
uniform 0..15 (random int32 words), scales uniform [0.002, 0.02], router
weight N(0, 0.02), activations N(0, 1).
"""
from __future__ import annotations

import numpy as np


def words(rng, shape):
    return rng.integers(-2**31, 2**31, size=shape, dtype=np.int64).astype(np.int32)


def scales(rng, shape, dtype=np.float16):
    s = rng.uniform(0.002, 0.02, size=shape)
    if dtype == "bf16":
        from oracle import i4ref

        return i4ref.f32_to_bf16_bits(s.astype(np.float32))  # uint16 bits
    return s.astype(dtype)


def ct_weight(rng, E, N, K, G, zeros=False, sdt=np.float16):
    NG = -(-K // G)
    p = words(rng, (E, N, K // 8))
    s = scales(rng, (E, N, NG), sdt)
    z = words(rng, (E, N, -(-NG // 8))) if zeros else None
    return p, s, z


def awq_weight(rng, E, K, N, G, sdt=np.float16):
    NG = -(-K // G)
    return words(rng, (E, K, N // 8)), words(rng, (E, NG, N // 8)), scales(rng, (E, NG, N), sdt)


def zipf_logits(rng, T, E, s=1.1, tau=2.0):
    """Skewed router logits: logit[t, e] = -s * tau * ln(rank(e)) + Gumbel(0, 1)."""
    rank = rng.permutation(E) + 1
    g = rng.gumbel(size=(T, E))
    return (-s * tau * np.log(rank))[None, :] + g

"""Pins the Talker MoE functions of the oracle (oracle/i4ref.py: q8_quantize,
dense_moe) -- runs on CPU.

  - dense_moe (with route) equals transformers' own
    Qwen3OmniMoeTalkerTextSparseMoeBlock run in float64 (the block FusedMoE,
    src/duplex/streaming/fused_moe.py:40, replaces), shared expert and its
    sigmoid gate included, to 1e-12;
  - the same block run in bfloat16 lands within the tolerance the GPU tests use
    of dense_moe with the bf16 rounding points: the reference's own 16-bit
    arithmetic is as far from the fp64 oracle as the kernels are allowed to be;
  - q8_quantize equals torch's bf16 / fp16 evaluation of fused_moe.py:84-94's
    formula bit for bit, and meets the invariants of symmetric per-row int8;
  - planted mistakes (no shared gate, a floor for the rounding, an fp64 scale)
    fail these checks.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import i4ref

M = pytest.importorskip("transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe")

# max |got - ref| / max |ref| allowed between a 16-bit computation of the block
# and the fp64 oracle with the same rounding points (the GPU parity bar)
TOL = {"bf16": 1e-2, "f16": 2e-3}


def _block(H=64, E=16, k=4, I=32, Is=48, renorm=True, seed=0, dtype=torch.float64):
    from transformers.models.qwen3_omni_moe.configuration_qwen3_omni_moe import (
        Qwen3OmniMoeTalkerTextConfig,
    )

    cfg = Qwen3OmniMoeTalkerTextConfig(
        hidden_size=H, num_experts=E, num_experts_per_tok=k, moe_intermediate_size=I,
        shared_expert_intermediate_size=Is, norm_topk_prob=renorm, num_hidden_layers=1)
    cfg._experts_implementation = "eager"
    torch.manual_seed(seed)
    blk = M.Qwen3OmniMoeTalkerTextSparseMoeBlock(cfg).to(dtype).eval()
    with torch.no_grad():
        for p in blk.parameters():
            p.copy_(torch.randn_like(p) * 0.2)
    return blk


def _weights(blk):
    f = lambda t: t.detach().double().numpy()
    se = blk.shared_expert
    sgu = np.concatenate((f(se.gate_proj.weight), f(se.up_proj.weight)), 0)
    return dict(router=f(blk.gate.weight), gu=f(blk.experts.gate_up_proj),
                dn=f(blk.experts.down_proj),
                shared=(sgu, f(se.down_proj.weight), f(blk.shared_expert_gate.weight).ravel()))


@pytest.mark.parametrize("renorm", [True, False])
def test_dense_moe_matches_transformers_block_fp64(renorm):
    blk = _block(renorm=renorm)
    W = _weights(blk)
    x = torch.randn(7, 64, dtype=torch.float64)
    with torch.no_grad():
        want = blk(x.view(1, 7, 64)).view(7, 64).numpy()
        _, b_w, b_sel = blk.gate(x)
    xn = x.numpy()
    sel, w = i4ref.route(xn @ W["router"].T, 4, renorm)
    # the block's softmax runs in fp32 (dtype=torch.float) even in a float64 module
    assert np.array_equal(sel, b_sel.numpy())
    np.testing.assert_allclose(w, b_w.numpy(), rtol=0, atol=1e-6)
    got = i4ref.dense_moe(xn, sel, b_w.numpy(), W["gu"], W["dn"], None, shared=W["shared"])
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)
    got = i4ref.dense_moe(xn, sel, w, W["gu"], W["dn"], None, shared=W["shared"])
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-5)


def test_bf16_block_is_within_tolerance_of_oracle():
    """transformers' block in bf16 (its own rounding everywhere) against the oracle
    with the kernels' rounding points, on the routing the bf16 block chose."""
    blk = _block(dtype=torch.bfloat16, H=256, E=32, k=6, I=64, Is=128)
    W = _weights(blk)
    x = (torch.randn(5, 256) * 0.5).to(torch.bfloat16)
    with torch.no_grad():
        want = blk(x.view(1, 5, 256)).view(5, 256).double().numpy()
        _, wts, sel = blk.gate(x)
    xn = x.double().numpy()
    got = i4ref.dense_moe(xn, sel.numpy(), wts.double().numpy(), W["gu"], W["dn"], "bf16",
                          shared=W["shared"], out_dtype="bf16")
    assert i4ref.rel_err(got, want) < TOL["bf16"]


def _torch_q8(w: torch.Tensor):
    s = w.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8) / 127.0
    return (w / s).round().clamp(-127, 127).to(torch.int8), s


@pytest.mark.parametrize("dtype,tdt", [("bf16", torch.bfloat16), ("f16", torch.float16)])
def test_q8_quantize_matches_torch_16bit_arithmetic(dtype, tdt):
    g = torch.Generator().manual_seed(1)
    w = (torch.randn(3, 40, 96, generator=g) * 0.05).to(tdt)
    w[0, 3] = 0                                            # an all-zero row
    w[1, 5, :] = torch.linspace(-1, 1, 96).to(tdt)          # exact halves among the quotients
    q_t, s_t = _torch_q8(w)
    q, s = i4ref.q8_quantize(w.float().numpy(), dtype)
    assert np.array_equal(q, q_t.numpy())
    assert np.array_equal(s, s_t.double().numpy())


def test_q8_quantize_invariants():
    rng = np.random.default_rng(2)
    w = i4ref.round_half(rng.standard_normal((64, 128)) * 0.03, "bf16")
    q, s = i4ref.q8_quantize(w, "bf16")
    assert q.dtype == np.int8 and np.abs(q.astype(int)).max() <= 127
    # the row maximum maps to +-127 up to the 16-bit rounding of the scale
    assert np.all(np.abs(q.astype(int)).max(axis=1) >= 126)
    # symmetric: negating the weights negates q and keeps s
    qn, sn = i4ref.q8_quantize(-w, "bf16")
    assert np.array_equal(qn, -q) and np.array_equal(sn, s)
    # reconstruction error: half a step, plus the 16-bit rounding of W / s
    err = np.abs(q * s - w)
    assert np.all(err <= s * (0.5 + 128 * 2.0 ** -8) + 1e-12)


def test_mutation_shared_gate_dropped_is_caught():
    blk = _block()
    W = _weights(blk)
    x = torch.randn(3, 64, dtype=torch.float64)
    with torch.no_grad():
        want = blk(x.view(1, 3, 64)).view(3, 64).numpy()
    xn = x.numpy()
    sel, w = i4ref.route(xn @ W["router"].T, 4, True)
    sgu, sdn, _ = W["shared"]
    bad = i4ref.dense_moe(xn, sel, w, W["gu"], W["dn"], None, shared=(sgu, sdn, None))
    assert not np.allclose(bad, want, atol=1e-6)


def test_mutation_q8_rounding_is_caught(monkeypatch):
    w = (torch.randn(8, 64) * 0.05).to(torch.bfloat16)
    q_t, s_t = _torch_q8(w)
    monkeypatch.setattr(i4ref.np, "round", np.floor)
    q, _ = i4ref.q8_quantize(w.float().numpy(), "bf16")
    assert not np.array_equal(q, q_t.numpy())
    monkeypatch.undo()
    # scale kept in full precision instead of the weights' dtype
    q, s = i4ref.q8_quantize(w.float().numpy(), "f32")
    assert not (np.array_equal(q, q_t.numpy()) and np.array_equal(s, s_t.double().numpy()))

"""Pins the fp32 attention reference (tests/_thinker_ref.py) to transformers' own
Qwen3OmniMoeThinkerTextAttention + RMSNorm (the installed transformers, fp32 on the CPU)
over several decode steps with a DynamicCache, including the interleaved multimodal
rotary embedding at text positions (equal along its three axes)."""
from __future__ import annotations

import pytest
import torch

from tests import _thinker_ref as ref

M = pytest.importorskip("transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe")


def _module(hidden=64, nh=4, nkv=2, hd=16, theta=1e6, seed=0):
    from transformers.models.qwen3_omni_moe.configuration_qwen3_omni_moe import (
        Qwen3OmniMoeTextConfig,
    )

    cfg = Qwen3OmniMoeTextConfig(
        hidden_size=hidden, num_attention_heads=nh, num_key_value_heads=nkv, head_dim=hd,
        rope_scaling={"interleaved": True, "mrope_interleaved": True, "mrope_section": [3, 3, 2],
                      "rope_type": "default", "type": "default"},
        rope_theta=theta, num_hidden_layers=1, num_experts=4, num_experts_per_tok=2,
        moe_intermediate_size=32, intermediate_size=64, rms_norm_eps=1e-6)
    cfg._attn_implementation = "eager"
    torch.manual_seed(seed)
    att = M.Qwen3OmniMoeThinkerTextAttention(cfg, 0).float().eval()
    norm = M.Qwen3OmniMoeThinkerTextRMSNorm(hidden, eps=1e-6)
    with torch.no_grad():
        for p in list(att.parameters()) + list(norm.parameters()):
            p.copy_(torch.randn_like(p) * (0.2 if p.dim() == 2 else 1.0) + (1.0 if p.dim() == 1 else 0))
    rot = M.Qwen3OmniMoeThinkerTextRotaryEmbedding(cfg)
    return cfg, att, norm, rot


@pytest.mark.parametrize("nh,nkv", [(4, 2), (8, 1)])
def test_reference_matches_transformers_attention(nh, nkv):
    from transformers.cache_utils import DynamicCache

    cfg, att, norm, rot = _module(nh=nh, nkv=nkv)
    cache = DynamicCache()
    rcache = {"k": torch.zeros(nkv, 0, 16), "v": torch.zeros(nkv, 0, 16)}
    W = {n: getattr(att, f"{n}_proj").weight.detach() for n in ("q", "k", "v", "o")}
    inv_freq = rot.inv_freq
    for pos in range(5):
        h = torch.randn(64)
        with torch.no_grad():
            x = norm(h.view(1, 1, -1))
            cos, sin = rot(x, torch.tensor([[pos]]))
            out, _ = att(x, (cos, sin), None, past_key_values=cache)
            want = h + out.view(-1)
        got = ref.attention_decode(h, W, att.q_norm.weight.detach(), att.k_norm.weight.detach(),
                                   norm.weight.detach(), 1e-6, inv_freq, pos, rcache, nh, nkv)
        torch.testing.assert_close(got, want, rtol=2e-5, atol=2e-5)


def test_rotary_table_matches_transformers():
    """rope_inv_freq (the host table the HIP kernel gets) equals transformers' inv_freq, and
    at text positions the interleaved mRoPE angle is pos * inv_freq."""
    from __graft_entry__ import load_package

    pkg = load_package()
    cfg, att, norm, rot = _module(hd=128, nh=2, nkv=1, hidden=128)
    tab = pkg.rope_inv_freq(128, 1e6)
    assert torch.equal(tab, rot.inv_freq)
    x = torch.zeros(1, 1, 128)
    for pos in (0, 7, 4095, 60000):
        cos, sin = rot(x, torch.tensor([[pos]]))
        f = pos * tab
        torch.testing.assert_close(cos.view(-1), torch.cat((f, f)).cos(), rtol=0, atol=1e-6)
        torch.testing.assert_close(sin.view(-1), torch.cat((f, f)).sin(), rtol=0, atol=1e-6)

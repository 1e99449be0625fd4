"""fp32 torch reference of one decode token through a Thinker attention block.

Restates Qwen3OmniMoeThinkerTextDecoderLayer's attention half
(transformers modeling_qwen3_omni_moe.py:1539-1551 and the attention module at
:1473-1514, transformers 5.15) in plain fp32 on the CPU, with dense weights:

    x = RMSNorm(h) * input_norm_w
    q, k, v = x Wq^T, x Wk^T, x Wv^T                  (per head: [n, head_dim])
    q, k = RMSNorm_head(q) * q_norm_w, RMSNorm_head(k) * k_norm_w
    q, k = q cos + rotate_half(q) sin, ...            (angle = pos * inv_freq, cat twice)
    cache <- k, v at row pos; softmax(q K^T / sqrt(head_dim)) V over rows [0, pos]
    h + out Wo^T

test_thinker_ref.py checks it against transformers' own module on the CPU.
"""
from __future__ import annotations

import torch


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def attention_decode(h, W, q_norm_w, k_norm_w, in_norm_w, eps, inv_freq, pos, cache,
                     n_heads, n_kv_heads):
    """h [H] fp32; W = {"q", "k", "v", "o"} dense fp32 [out, in]; cache = {"k": [n_kv, S, d],
    "v": ...} fp32 tensors grown in place by one row (pos == rows already cached).
    Returns h + attention output [H]."""
    d = W["q"].shape[0] // n_heads
    x = rmsnorm(h, in_norm_w, eps)
    q = (W["q"] @ x).view(n_heads, d)
    k = (W["k"] @ x).view(n_kv_heads, d)
    v = (W["v"] @ x).view(n_kv_heads, d)
    q, k = rmsnorm(q, q_norm_w, eps), rmsnorm(k, k_norm_w, eps)
    f = pos * inv_freq.float()
    emb = torch.cat((f, f))
    cos, sin = emb.cos(), emb.sin()
    q = q * cos + rotate_half(q) * sin
    k = k * cos + rotate_half(k) * sin
    if cache["k"].shape[1] != pos:
        raise ValueError("the reference cache must hold exactly pos rows")
    cache["k"] = torch.cat((cache["k"], k[:, None]), dim=1)
    cache["v"] = torch.cat((cache["v"], v[:, None]), dim=1)
    g = n_heads // n_kv_heads
    K = cache["k"].repeat_interleave(g, dim=0)       # [n_heads, S, d]
    V = cache["v"].repeat_interleave(g, dim=0)
    s = torch.einsum("hd,hsd->hs", q, K) / d ** 0.5
    p = torch.softmax(s, dim=-1)
    out = torch.einsum("hs,hsd->hd", p, V).reshape(-1)
    return h + W["o"] @ out

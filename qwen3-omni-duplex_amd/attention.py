"""Thinker decode step around the int4 path: attention block, decoder layer, stack.

The clock path runs Thinker[0:24] one token per frame (src/duplex/streaming/
clock.py:164-172: `th(inputs_embeds=emb, past_key_values=th_kv, use_cache=True)`),
i.e. transformers' Qwen3OmniMoeThinkerTextDecoderLayer.forward
(modeling_qwen3_omni_moe.py:1539-1565 in transformers 5.15) per layer:

    h = h + o_proj(attention(input_layernorm(h)))            ThinkerAttention
    h = h + moe(post_attention_layernorm(h))                  FusedPackedMoE (norm fused)

with the projections on the library's int4 GEMVs (q|k|v with the input norm inside the
attention chunk launch, o with the residual added in the launch that merges the attention
heads), and q/k norm, rotary embedding, KV-cache append and GQA attention in
i4_attn_decode_qkv_o.  The KV cache is preallocated
([n_kv_heads, max_len, head_dim] per layer, the activation dtype) instead of
transformers' growing DynamicCache.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib, ops
from .linear import PackedLinear, PackedQKV
from .moe import FusedPackedMoE


def rope_inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """inv_freq of the default rotary embedding, computed as transformers does
    (compute_default_rope_parameters: 1 / theta ** (arange(0, d, 2) / d) in fp32)."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))


class ThinkerAttention(nn.Module):
    """One decode token of the attention half of a Thinker layer, residual included."""

    def __init__(self, qkv: PackedQKV, o_proj: PackedLinear, q_norm_w: torch.Tensor,
                 k_norm_w: torch.Tensor, input_norm_w: torch.Tensor, n_heads: int,
                 n_kv_heads: int, head_dim: int = 128, eps: float = 1e-6,
                 rope_theta: float = 1_000_000.0, max_len: int = 4096):
        super().__init__()
        if qkv.lin.w.layout != "ct":
            raise ValueError("the q|k|v weight must be in the CT layout: the input norm runs "
                             "inside its GEMV (build PackedQKV with repack=True)")
        self.qkv, self.o_proj = qkv, o_proj
        self.n_heads, self.n_kv_heads, self.head_dim = int(n_heads), int(n_kv_heads), int(head_dim)
        self.eps = float(eps)
        if qkv.sizes != (n_heads * head_dim, n_kv_heads * head_dim, n_kv_heads * head_dim):
            raise ValueError(f"q|k|v rows {qkv.sizes} do not match {n_heads}/{n_kv_heads} heads")
        dt = input_norm_w.dtype
        self.register_buffer("q_norm_w", q_norm_w.to(dt).contiguous(), persistent=False)
        self.register_buffer("k_norm_w", k_norm_w.to(dt).contiguous(), persistent=False)
        self.register_buffer("input_norm_w", input_norm_w.contiguous(), persistent=False)
        self.inv_freq = rope_inv_freq(head_dim, rope_theta)  # host table
        shape = (n_kv_heads, max_len, head_dim)
        dev = input_norm_w.device
        self.register_buffer("_k_cache", torch.zeros(shape, dtype=dt, device=dev), persistent=False)
        self.register_buffer("_v_cache", torch.zeros(shape, dtype=dt, device=dev), persistent=False)
        self.max_len = int(max_len)
        self.workspace = ops.Workspace()

    # The caches are written in place by the kernels and their addresses are held by the
    # decoder's layer structs, so they cannot be replaced: fill them in place
    # (k_cache.copy_(...)) or clear them with reset_cache().
    @property
    def k_cache(self) -> torch.Tensor:
        return self._k_cache

    @property
    def v_cache(self) -> torch.Tensor:
        return self._v_cache

    def reset_cache(self) -> None:
        """Empty the KV cache in place (a new conversation)."""
        self._k_cache.zero_()
        self._v_cache.zero_()

    def __setattr__(self, name, value):
        super().__setattr__(name, value)
        ops.weights_changed()

    def forward(self, h: torch.Tensor, pos: int | torch.Tensor) -> torch.Tensor:
        """h [1, H] (one token at cache position pos) -> h + o_proj(attn(norm(h))).

        pos is an int, or an int32 device tensor of one element that the kernels read (a
        decode step captured in a hipGraph then serves every token; a position outside the
        cache gives NaN and leaves the cache untouched)."""
        if h.numel() != h.shape[-1]:
            raise ValueError("ThinkerAttention decodes one token")
        if not isinstance(pos, torch.Tensor) and not 0 <= pos < self.max_len:
            raise ValueError(f"position {pos} outside the cache (max_len {self.max_len})")
        if self.o_proj.w.layout == "ct":
            # input_layernorm + q|k|v inside the attention chunk launch, then the head
            # merge and o_proj (+ the residual) in one more
            return ops.attn_decode_qkv_o(h, self.input_norm_w, self.eps, self.qkv.lin.w,
                                         self.n_heads, self.n_kv_heads, self.q_norm_w,
                                         self.k_norm_w, self.inv_freq, pos, self.k_cache,
                                         self.v_cache, self.o_proj.w, self.workspace)
        # input_layernorm folded into the q|k|v launch
        qkv = ops.rmsnorm_linear(h, self.input_norm_w, self.eps, self.qkv.lin.w)
        a = ops.attn_decode(qkv, self.n_heads, self.n_kv_heads, self.q_norm_w, self.k_norm_w,
                            self.eps, self.inv_freq, pos, self.k_cache, self.v_cache,
                            self.workspace)
        # one token: the residual enters the o_proj launch as its bias
        return ops.linear(a.view(1, -1), self.o_proj.w, bias=h.reshape(-1)).view(h.shape)


class ThinkerDecoderLayer(nn.Module):
    """Qwen3OmniMoeThinkerTextDecoderLayer.forward for one decode token."""

    def __init__(self, attn: ThinkerAttention, moe: FusedPackedMoE):
        super().__init__()
        if moe.norm_weight is None:
            raise ValueError("the MoE block must carry its post_attention_layernorm")
        self.attn, self.moe = attn, moe
        self._fused: bool | None = None

    def fused(self) -> bool:
        """Whether forward runs as one i4_thinker_layer_decode call: CT projections and
        experts of the single-launch expert kernel, with the router in the block."""
        a, m = self.attn, self.moe
        if self._fused is None:
            self._fused = bool(
                a.qkv.lin.w.layout == "ct" and a.o_proj.w.layout == "ct"
                and m.gate_up.layout == "ct" and m.router_w is not None
                and ops.thinker_layer_fits(a.n_heads, a.n_kv_heads, a.head_dim, a.max_len,
                                           m.hidden, m.down.K, m.gate_up.E, m.top_k))
        return self._fused

    def forward(self, h: torch.Tensor, pos: int | torch.Tensor) -> torch.Tensor:
        if h.numel() == h.shape[-1] and self.fused():
            a, m = self.attn, self.moe
            if not isinstance(pos, torch.Tensor) and not 0 <= pos < a.max_len:
                raise ValueError(f"position {pos} outside the cache (max_len {a.max_len})")
            return ops.thinker_layer_decode(
                h, a.input_norm_w, a.eps, a.qkv.lin.w, a.n_heads, a.n_kv_heads, a.q_norm_w,
                a.k_norm_w, a.inv_freq, pos, a.k_cache, a.v_cache, a.o_proj.w, m.gate_up,
                m.down, m.top_k, m.router_w, m.norm_weight, m.norm_eps, m.norm_topk_prob,
                a.workspace)
        return self.unfused(h, pos)

    def unfused(self, h: torch.Tensor, pos: int | torch.Tensor) -> torch.Tensor:
        """The attention block, then the MoE block (each its own entry points)."""
        h = self.attn(h, pos)
        return self.moe(h, residual=h)


class ThinkerDecoder(nn.Module):
    """Thinker[0:n] decode: step(h, pos) runs every layer on one token and returns the
    hidden state after the last layer (the clock path's layer-24 tap, clock.py:168)."""

    def __init__(self, layers: list[ThinkerDecoderLayer]):
        super().__init__()
        self.layers = nn.ModuleList(layers)
        self.workspace = ops.Workspace()
        self._fused: bool | None = None
        self._layers_c, self._layers_refs, self._layers_gen = None, None, -1

    def _apply(self, fn, *args, **kwargs):
        # moved tensors: the layer structs hold their old addresses
        self._fused, self._layers_c = None, None
        return super()._apply(fn, *args, **kwargs)

    def _structs(self):
        """The layer structs (raw addresses of the layers' tensors), rebuilt when any tensor of
        a ThinkerAttention or FusedPackedMoE was assigned since they were made; the tensors
        they point at are kept referenced with them."""
        gen = ops.weights_generation()
        if self._layers_c is None or self._layers_gen != gen:
            arr = _lib.ThinkerLayerC * len(self.layers)
            self._layers_c = arr(*[ops.thinker_layer_c(l.attn, l.moe) for l in self.layers])
            self._layers_refs = [(l.attn._k_cache, l.attn._v_cache, l.attn.input_norm_w,
                                  l.attn.q_norm_w, l.attn.k_norm_w, l.attn.qkv.lin.w,
                                  l.attn.o_proj.w, l.moe.gate_up, l.moe.down, l.moe.router_w,
                                  l.moe.norm_weight) for l in self.layers]
            self._layers_gen = gen
        return self._layers_c

    def fused(self) -> bool:
        """Whether step runs as one i4_thinker_decode_step call: every layer takes
        i4_thinker_layer_decode and all share their sizes, dtype and routing."""
        if self._fused is None:
            ls = list(self.layers)

            def sizes(l):
                a, m = l.attn, l.moe
                return (a.n_heads, a.n_kv_heads, a.head_dim, a.max_len, m.hidden, m.down.K,
                        m.gate_up.E, m.top_k, m.norm_topk_prob, a.input_norm_w.dtype,
                        tuple(a.inv_freq.tolist()))

            self._fused = bool(ls) and all(l.fused() for l in ls) and all(
                sizes(l) == sizes(ls[0]) for l in ls)
        return self._fused

    def step(self, h: torch.Tensor, pos: int | torch.Tensor) -> torch.Tensor:
        if h.numel() == h.shape[-1] and self.fused():
            a0, m0 = self.layers[0].attn, self.layers[0].moe
            if not isinstance(pos, torch.Tensor) and not 0 <= pos < a0.max_len:
                raise ValueError(f"position {pos} outside the cache (max_len {a0.max_len})")
            return ops.thinker_decode_step(
                h, self._structs(), len(self.layers), a0.n_heads, a0.n_kv_heads, a0.head_dim,
                a0.inv_freq, pos, a0.max_len, m0.hidden, m0.down.K, m0.gate_up.E, m0.top_k,
                m0.norm_topk_prob, self.workspace)
        return self.unfused(h, pos)

    def unfused(self, h: torch.Tensor, pos: int | torch.Tensor) -> torch.Tensor:
        """Layer by layer (each its own i4_thinker_layer_decode or module calls)."""
        for layer in self.layers:
            h = layer(h, pos)
        return h

    forward = step

"""Thinker checkpoint reader: compressed-tensors int4 triplets into stacked buffers.

Mirrors the reference's two readers of the quantized Thinker checkpoint,
src/duplex/streaming/clock.py:45-103 (load_thinker_prefix) and
src/duplex/loader.py:31-55 (_assign): the shards of model.safetensors.index.json
hold, per packed Linear, the compressed-tensors pack-quantized triplet

    <name>.weight_packed  int32 [out, ceil(in / 8)], column 8m + i in nibble i of word m
    <name>.weight_scale   [out, ceil(in / group)]
    <name>.weight_shape   int [2] = (out, in)

(src/duplex/quant/dequant.py:23-27), symmetric with zero point 8.  The
reference attaches the triplets to a transformers module tree and stacks the
experts afterwards (fused_packed_moe.py:68-80, gate|up concatenated at :122);
here each layer's experts are read tensor by tensor from the memory-mapped
shards straight into the stacked [E, N, K/8] buffers on the device, so no
module tree, no per-expert Linear and no host copy of a whole shard exists.
Dense tensors (the router `mlp.gate.weight`, the RMSNorm weights) are cast to
the activation dtype, scales to `dtype` as in the reference
(clock.py:88-89, loader.py:42).

Checkpoint tensor names (Qwen3-Omni, transformers 4.57 layout):
    thinker.model.layers.{l}.mlp.experts.{e}.{gate,up,down}_proj.weight_*
    thinker.model.layers.{l}.mlp.gate.weight                   router [E, H]
    thinker.model.layers.{l}.post_attention_layernorm.weight   pre-MoE RMSNorm [H]
    thinker.model.layers.{l}.self_attn.{q,k,v,o}_proj.weight_*
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

from .attention import ThinkerAttention, ThinkerDecoder, ThinkerDecoderLayer
from .linear import PackedLinear, PackedQKV
from .moe import FusedPackedMoE
from .weights import QWeight

PREFIX = "thinker.model.layers"
TRIPLET = ("weight_packed", "weight_scale", "weight_shape")


class Checkpoint:
    """A safetensors checkpoint directory: config.json plus one model.safetensors or
    shards listed in model.safetensors.index.json.  Tensors are read one at a time
    from memory-mapped shards."""

    def __init__(self, root: str | Path):
        from safetensors import safe_open

        self._safe_open = safe_open
        self.root = Path(root)
        self.config = json.loads((self.root / "config.json").read_text())
        index = self.root / "model.safetensors.index.json"
        if index.exists():
            self.weight_map = json.loads(index.read_text())["weight_map"]
        else:
            single = self.root / "model.safetensors"
            if not single.exists():
                raise FileNotFoundError(f"{self.root}: no model.safetensors(.index.json)")
            with safe_open(str(single), framework="pt") as f:
                self.weight_map = {k: single.name for k in f.keys()}
        self._handles: dict[str, object] = {}

    # -- config ------------------------------------------------------------
    def text_config(self) -> dict:
        """The Thinker's text config (thinker_config.text_config, or the top level)."""
        c = self.config
        c = c.get("thinker_config", c)
        return c.get("text_config", c)

    def group_size(self, default: int = 32) -> int:
        """Quantisation group along the input dim from quantization_config
        (config_groups.*.weights.group_size), else `default`."""
        for c in (self.config, self.config.get("thinker_config", {})):
            q = c.get("quantization_config") or {}
            for grp in (q.get("config_groups") or {}).values():
                w = grp.get("weights") or {}
                if w.get("group_size"):
                    return int(w["group_size"])
        return default

    # -- tensors -----------------------------------------------------------
    def has(self, name: str) -> bool:
        return name in self.weight_map

    def tensor(self, name: str) -> torch.Tensor:
        shard = self.weight_map.get(name)
        if shard is None:
            raise KeyError(f"{name} is not in the checkpoint")
        h = self._handles.get(shard)
        if h is None:
            h = self._safe_open(str(self.root / shard), framework="pt")
            self._handles[shard] = h
        return h.get_tensor(name)

    def triplet(self, name: str) -> tuple[torch.Tensor, torch.Tensor, int, int]:
        """(packed, scale, out_features, in_features) of packed Linear `name`, checked
        against its weight_shape."""
        packed, scale, shape = (self.tensor(f"{name}.{t}") for t in TRIPLET)
        out_f, in_f = (int(v) for v in shape.reshape(-1).tolist())
        if packed.dtype != torch.int32 or tuple(packed.shape) != (out_f, -(-in_f // 8)):
            raise ValueError(f"{name}.weight_packed: {packed.dtype} {tuple(packed.shape)} does not "
                             f"pack a [{out_f}, {in_f}] int4 weight")
        if scale.dim() != 2 or scale.shape[0] != out_f:
            raise ValueError(f"{name}.weight_scale: shape {tuple(scale.shape)}")
        if self.has(f"{name}.weight_zero_point"):
            raise NotImplementedError(f"{name}: asymmetric (zero-point) checkpoints are not read")
        return packed, scale, out_f, in_f


def _group_of(ckpt: Checkpoint, in_f: int, n_groups: int) -> int:
    g = ckpt.group_size()
    if -(-in_f // g) != n_groups:
        raise ValueError(f"{n_groups} scale groups do not cover {in_f} inputs at group size {g}")
    return g


def stack_experts(ckpt: Checkpoint, layer: int, proj: str, E: int, device,
                  scale_dtype=torch.bfloat16, out: tuple | None = None,
                  row_offset: int = 0) -> QWeight:
    """Expert `proj` ("gate_proj" / "up_proj" / "down_proj") of every expert of a layer,
    stacked as CT: packed [E, N, K/8], scale [E, N, NG] (fused_packed_moe.py:68-80).
    With out = (packed, scale) of a wider stack, the rows land at
    [row_offset, row_offset + N) of each expert (the gate|up concatenation, :122)."""
    base = f"{PREFIX}.{layer}.mlp.experts"
    p0, s0, N, K = ckpt.triplet(f"{base}.0.{proj}")
    G = _group_of(ckpt, K, s0.shape[1])
    if out is None:
        packed = torch.empty(E, N, p0.shape[1], dtype=torch.int32, device=device)
        scale = torch.empty(E, N, s0.shape[1], dtype=scale_dtype, device=device)
    else:
        packed, scale = out
    for e in range(E):
        p, s, n, k = (p0, s0, N, K) if e == 0 else ckpt.triplet(f"{base}.{e}.{proj}")
        if (n, k) != (N, K) or s.shape != s0.shape:
            raise ValueError(f"{base}.{e}.{proj}: shape ({n}, {k}) differs from expert 0 ({N}, {K})")
        packed[e, row_offset:row_offset + N].copy_(p)
        scale[e, row_offset:row_offset + N].copy_(s)
    return QWeight(packed, scale, None, "ct", G, packed.shape[1], K)


def read_moe_layer(ckpt: Checkpoint, layer: int, device="cuda", dtype=torch.bfloat16,
                   scale_dtype=None) -> dict:
    """The packed MoE block of one Thinker layer as stacked CT tensors on `device`:
    {"gate_up", "down": QWeight, "router_w", "norm_w": dtype, "norm_eps", "top_k",
    "norm_topk_prob"}.  gate_up rows [0, I) are gate_proj, [I, 2I) up_proj."""
    tc = ckpt.text_config()
    E = int(tc["num_experts"])
    scale_dtype = scale_dtype or dtype
    base = f"{PREFIX}.{layer}.mlp.experts.0"
    pg, sg, I, H = ckpt.triplet(f"{base}.gate_proj")
    gu_packed = torch.empty(E, 2 * I, pg.shape[1], dtype=torch.int32, device=device)
    gu_scale = torch.empty(E, 2 * I, sg.shape[1], dtype=scale_dtype, device=device)
    stack_experts(ckpt, layer, "gate_proj", E, device, scale_dtype, (gu_packed, gu_scale), 0)
    up = stack_experts(ckpt, layer, "up_proj", E, device, scale_dtype, (gu_packed, gu_scale), I)
    gate_up = QWeight(gu_packed, gu_scale, None, "ct", up.group, 2 * I, H)
    down = stack_experts(ckpt, layer, "down_proj", E, device, scale_dtype)
    if down.N != H or down.K != I:
        raise ValueError(f"layer {layer}: down_proj is [{down.N}, {down.K}], not [{H}, {I}]")
    router = ckpt.tensor(f"{PREFIX}.{layer}.mlp.gate.weight")
    if tuple(router.shape) != (E, H):
        raise ValueError(f"layer {layer}: router weight {tuple(router.shape)} != ({E}, {H})")
    norm_name = f"{PREFIX}.{layer}.post_attention_layernorm.weight"
    norm = ckpt.tensor(norm_name).to(device, dtype) if ckpt.has(norm_name) else None
    return {"gate_up": gate_up, "down": down, "router_w": router.to(device, dtype).contiguous(),
            "norm_w": norm, "norm_eps": float(tc.get("rms_norm_eps", 1e-6)),
            "top_k": int(tc["num_experts_per_tok"]),
            "norm_topk_prob": bool(tc.get("norm_topk_prob", True))}


def load_moe_layer(ckpt: Checkpoint, layer: int, device="cuda", dtype=torch.bfloat16,
                   layouts: str = "both", fuse_norm: bool = True) -> FusedPackedMoE:
    """A FusedPackedMoE for Thinker layer `layer` (CT rows for decode and, with
    layouts="both", the tile copy for batches).  fuse_norm folds the layer's
    post_attention_layernorm into the block (it then takes the un-normalised
    residual stream, as ops.moe_stack does)."""
    d = read_moe_layer(ckpt, layer, device, dtype)
    return FusedPackedMoE.from_stacked(d["gate_up"], d["down"], d["router_w"], d["top_k"],
                                       d["norm_topk_prob"],
                                       d["norm_w"] if fuse_norm else None, d["norm_eps"],
                                       layouts=layouts)


def load_thinker_moe_stack(root: str | Path, n_layers: int = 24, device="cuda",
                           dtype=torch.bfloat16, layouts: str = "both") -> list[FusedPackedMoE]:
    """The MoE blocks of Thinker[0:n_layers] (clock.py:45-103 reads the same prefix),
    each with its pre-MoE RMSNorm fused, ready for ops.moe_stack via stack_entry()."""
    ckpt = Checkpoint(root)
    tc = ckpt.text_config()
    step = int(tc.get("decoder_sparse_step", 1))
    dense = set(tc.get("mlp_only_layers", []) or [])
    for layer in range(n_layers):  # transformers' MoE-layer rule, checked before any read
        if layer in dense or (layer + 1) % step != 0:
            raise ValueError(f"layer {layer} has a dense MLP; only MoE stacks are read")
    return [load_moe_layer(ckpt, layer, device, dtype, layouts) for layer in range(n_layers)]


def load_attention(ckpt: Checkpoint, layer: int, device="cuda", fuse_qkv: bool = False,
                   scale_dtype=torch.float32, tile: bool = True) -> dict:
    """The packed q/k/v/o projections of one layer as PackedLinear modules
    (TritonPackedLinear keeps fp32 scales, triton_dequant_gemv.py:141-144);
    fuse_qkv returns {"qkv": PackedQKV, "o": PackedLinear}."""
    base = f"{PREFIX}.{layer}.self_attn"
    ws = {}
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        p, s, out_f, in_f = ckpt.triplet(f"{base}.{name}")
        G = _group_of(ckpt, in_f, s.shape[1])
        ws[name] = QWeight(p.to(device).unsqueeze(0), s.to(device, scale_dtype).unsqueeze(0),
                           None, "ct", G, out_f, in_f)
    if fuse_qkv:
        return {"qkv": PackedQKV.from_qweights(ws["q_proj"], ws["k_proj"], ws["v_proj"]),
                "o": PackedLinear.from_qweight(ws["o_proj"], tile=tile)}
    return {k: PackedLinear.from_qweight(w, tile=tile) for k, w in ws.items()}


def rope_theta(tc: dict) -> float:
    """rope_theta of a text config (top level, or inside rope_parameters / rope_scaling)."""
    for src in (tc, tc.get("rope_parameters") or {}, tc.get("rope_scaling") or {}):
        if "rope_theta" in src:
            return float(src["rope_theta"])
    return 10000.0


def load_thinker_layer(ckpt: Checkpoint, layer: int, device="cuda", dtype=torch.bfloat16,
                       max_len: int = 4096, layouts: str = "both") -> ThinkerDecoderLayer:
    """One Thinker decoder layer for decode: attention (input_layernorm, q|k|v in one
    launch, q_norm / k_norm, rotary, KV cache of max_len positions, o_proj) and the MoE
    block with its post_attention_layernorm (clock.py:45-103 loads the same tensors)."""
    tc = ckpt.text_config()
    base = f"{PREFIX}.{layer}"
    nh, nkv = int(tc["num_attention_heads"]), int(tc["num_key_value_heads"])
    hd = int(tc.get("head_dim") or tc["hidden_size"] // nh)
    proj = load_attention(ckpt, layer, device, fuse_qkv=True)
    attn = ThinkerAttention(
        proj["qkv"], proj["o"],
        ckpt.tensor(f"{base}.self_attn.q_norm.weight").to(device, dtype),
        ckpt.tensor(f"{base}.self_attn.k_norm.weight").to(device, dtype),
        ckpt.tensor(f"{base}.input_layernorm.weight").to(device, dtype),
        nh, nkv, hd, float(tc.get("rms_norm_eps", 1e-6)), rope_theta(tc), max_len)
    return ThinkerDecoderLayer(attn, load_moe_layer(ckpt, layer, device, dtype, layouts))


def load_thinker_decoder(root: str | Path, n_layers: int = 24, device="cuda",
                         dtype=torch.bfloat16, max_len: int = 4096) -> ThinkerDecoder:
    """Thinker[0:n_layers] for one-token decode steps (the clock path's prefix)."""
    ckpt = Checkpoint(root)
    return ThinkerDecoder([load_thinker_layer(ckpt, layer, device, dtype, max_len)
                           for layer in range(n_layers)])

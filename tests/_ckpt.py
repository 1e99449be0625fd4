"""Synthetic Qwen3-Omni Thinker checkpoints in the compressed-tensors format.

Writes the layout the reference reads (src/duplex/streaming/clock.py:45-103,
src/duplex/loader.py:31-55, src/duplex/quant/dequant.py:23-27): config.json
with thinker_config.text_config and a quantization_config, safetensors shards
listed in model.safetensors.index.json, and per packed Linear the triplet
weight_packed (int32 [out, in/8], column 8m + i in nibble i of word m),
weight_scale (bf16 [out, in/group]) and weight_shape (int64 [out, in]).
Returns the ground truth (raw nibbles and scales) the tests dequantise
independently.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

from oracle import i4ref


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)


def _linear(rng, out_f, in_f, G):
    q = rng.integers(0, 16, size=(out_f, in_f), dtype=np.int64).astype(np.uint8)
    s = i4ref.bf16_bits_to_f32(i4ref.f32_to_bf16_bits(
        rng.uniform(0.002, 0.02, size=(out_f, -(-in_f // G))).astype(np.float32)))
    tensors = {"weight_packed": torch.from_numpy(i4ref.ct_pack(q)),
               "weight_scale": _bf16(s),
               "weight_shape": torch.tensor([out_f, in_f], dtype=torch.int64)}
    return q, s, tensors


def write_checkpoint(root: Path, rng, n_layers=2, E=4, H=256, I=128, G=32, top_k=2,
                     shards=2, attention=None, single_file=False, group_in_config=True,
                     head_dim=128):
    """attention = (q_out, kv_out) adds self_attn.{q,k,v,o}_proj and q_norm / k_norm
    ([head_dim]) to every layer."""
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    truth, blobs = [], [dict() for _ in range(shards)]
    for layer in range(n_layers):
        t = {"experts": [], "attn": {}}
        blob = blobs[layer % shards]
        base = f"thinker.model.layers.{layer}"
        for e in range(E):
            ex = {}
            for proj, (o, i) in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
                q, s, tens = _linear(rng, o, i, G)
                ex[proj] = (q, s)
                for k, v in tens.items():
                    blob[f"{base}.mlp.experts.{e}.{proj}.{k}"] = v
            t["experts"].append(ex)
        router = i4ref.bf16_bits_to_f32(i4ref.f32_to_bf16_bits(
            (rng.standard_normal((E, H)) * 0.02).astype(np.float32)))
        norm = i4ref.bf16_bits_to_f32(i4ref.f32_to_bf16_bits(
            rng.uniform(0.5, 1.5, H).astype(np.float32)))
        blob[f"{base}.mlp.gate.weight"] = _bf16(router)
        blob[f"{base}.post_attention_layernorm.weight"] = _bf16(norm)
        in_norm = i4ref.bf16_bits_to_f32(i4ref.f32_to_bf16_bits(
            rng.uniform(0.5, 1.5, H).astype(np.float32)))
        blob[f"{base}.input_layernorm.weight"] = _bf16(in_norm)
        t["router"], t["norm"], t["in_norm"] = router, norm, in_norm
        if attention is not None:
            q_out, kv_out = attention
            for proj, (o, i) in (("q_proj", (q_out, H)), ("k_proj", (kv_out, H)),
                                 ("v_proj", (kv_out, H)), ("o_proj", (H, q_out))):
                q, s, tens = _linear(rng, o, i, G)
                t["attn"][proj] = (q, s)
                for k, v in tens.items():
                    blob[f"{base}.self_attn.{proj}.{k}"] = v
            for nm in ("q_norm", "k_norm"):
                w = i4ref.bf16_bits_to_f32(i4ref.f32_to_bf16_bits(
                    rng.uniform(0.5, 1.5, head_dim).astype(np.float32)))
                blob[f"{base}.self_attn.{nm}.weight"] = _bf16(w)
                t["attn"][nm] = w
        truth.append(t)
    from safetensors.torch import save_file

    weight_map = {}
    if single_file:
        merged = {k: v for b in blobs for k, v in b.items()}
        save_file(merged, str(root / "model.safetensors"))
    else:
        for i, b in enumerate(blobs):
            name = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
            save_file(b, str(root / name))
            weight_map.update({k: name for k in b})
        (root / "model.safetensors.index.json").write_text(
            json.dumps({"metadata": {}, "weight_map": weight_map}))
    cfg = {"thinker_config": {"text_config": {
        "num_experts": E, "num_experts_per_tok": top_k, "hidden_size": H,
        "moe_intermediate_size": I, "norm_topk_prob": True, "rms_norm_eps": 1e-6,
        "decoder_sparse_step": 1, "mlp_only_layers": [], "num_hidden_layers": n_layers,
        "head_dim": head_dim, "rope_theta": 1000000.0,
        "num_attention_heads": (attention[0] // head_dim) if attention else 1,
        "num_key_value_heads": (attention[1] // head_dim) if attention else 1}}}
    if group_in_config:
        cfg["quantization_config"] = {"format": "pack-quantized", "config_groups": {"group_0": {
            "weights": {"num_bits": 4, "group_size": G, "symmetric": True,
                        "strategy": "group"}}}}
    (root / "config.json").write_text(json.dumps(cfg))
    return truth


def dense(qs) -> np.ndarray:
    """(nibbles [N, K], scales [N, NG]) -> float64 [N, K] = (q - 8) * s per group, by
    explicit group loops (independent of the oracle's vectorised dequant)."""
    q, s = qs
    N, K = q.shape
    G = -(-K // s.shape[1])
    out = np.empty((N, K), np.float64)
    for g in range(s.shape[1]):
        sl = slice(g * G, min(K, (g + 1) * G))
        out[:, sl] = (q[:, sl].astype(np.float64) - 8.0) * s[:, g:g + 1].astype(np.float64)
    return out

"""MI355X (gfx950) int4 clock-path kernels for Qwen3-Omni Thinker layers 0-23.

Drop-in replacements for thecodacus/qwen3-omni-duplex's quantized compute:
  dequant_gemv           <- src/duplex/streaming/triton_dequant_gemv.py:85
  PackedLinear           <- TritonPackedLinear (:125), patch_attention (:162)
  FusedPackedMoE         <- src/duplex/streaming/fused_packed_moe.py:83
  fuse_packed_moe_blocks <- fused_packed_moe.py:278
  loader                 <- src/duplex/streaming/clock.py:45 (load_thinker_prefix),
                            src/duplex/loader.py:31 (packed triplets from safetensors)
  ThinkerDecoder         <- the Thinker[0:24] decode step the clock path runs
                            (clock.py:164-172): attention with KV cache + MoE per layer
  FusedMoE               <- src/duplex/streaming/fused_moe.py:40 (16-bit / int8
                            experts + gated shared expert: the Talker's block)
  fuse_moe_blocks        <- fused_moe.py:144
all executed by the hand-written HIP kernels of libi4moe.so (C ABI in
include/i4moe.h).  There is no fallback: without the built library every op
raises.
"""
from . import _lib
from .linear import (TILE_ROWS, PackedLinear, PackedQKV, QKVSlice, concat_cols_awq, concat_rows,
                     patch_attention)
from .attention import ThinkerAttention, ThinkerDecoder, ThinkerDecoderLayer, rope_inv_freq
from .loader import (Checkpoint, load_attention, load_moe_layer, load_thinker_decoder,
                     load_thinker_layer, load_thinker_moe_stack, read_moe_layer)
from .fused_moe import FusedMoE, fuse_moe_blocks, quantize_q8
from .moe import FusedPackedMoE, fuse_packed_moe_blocks
from .ops import (dequant, dequant_gemv, linear, moe_down_combine, moe_down_wait, moe_forward,
                  moe_forward_noalloc, moe_gate_up, moe_route_gate_up, moe_stack, moe_status,
                  route, router_logits, unpack4, unpack_nibbles, Workspace, rmsnorm,
                  rmsnorm_linear, attn_decode, attn_decode_o, attn_decode_qkv_o,
                  thinker_layer_decode,
                  thinker_layer_fits, thinker_layer_c, thinker_decode_step, dmoe_forward,
                  dmoe_status, dmoe_down_wait, StackLayerX)
from .weights import QWeight, repack_awq_to_ct, repack_tile

lib = _lib.lib

__all__ = [
    "QWeight", "repack_awq_to_ct", "repack_tile", "dequant_gemv", "linear", "unpack4", "unpack_nibbles",
    "dequant", "router_logits", "route", "moe_forward", "moe_gate_up", "moe_route_gate_up",
    "moe_down_combine", "moe_down_wait", "moe_status", "moe_forward_noalloc",
    "moe_stack", "Workspace",
    "FusedPackedMoE", "fuse_packed_moe_blocks", "PackedLinear", "PackedQKV", "QKVSlice",
    "concat_rows", "concat_cols_awq", "patch_attention", "TILE_ROWS", "lib",
    "Checkpoint", "read_moe_layer", "load_moe_layer", "load_thinker_moe_stack", "load_attention",
    "load_thinker_layer", "load_thinker_decoder", "rmsnorm", "rmsnorm_linear", "attn_decode",
    "attn_decode_o", "attn_decode_qkv_o", "thinker_layer_decode", "thinker_layer_fits",
    "thinker_layer_c",
    "thinker_decode_step",
    "ThinkerAttention", "ThinkerDecoderLayer", "ThinkerDecoder", "rope_inv_freq",
    "FusedMoE", "fuse_moe_blocks", "quantize_q8", "dmoe_forward", "dmoe_status",
    "dmoe_down_wait", "StackLayerX",
]

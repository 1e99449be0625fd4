"""The checkpoint reader on the host (no GPU): compressed-tensors triplets from
safetensors shards into stacked CT buffers (src/duplex/streaming/clock.py:45-103,
fused_packed_moe.py:68-80,122), checked against independently dequantised ground
truth."""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from oracle import i4ref
from tests import _ckpt


@pytest.fixture(scope="module")
def ckpt_dir(tmp_path_factory):
    root = tmp_path_factory.mktemp("thinker")
    truth = _ckpt.write_checkpoint(root, np.random.default_rng(51), n_layers=3, E=4, H=256,
                                   I=128, G=32, shards=2, attention=(256, 64))
    return root, truth


def _loader(pkg):
    import importlib

    return importlib.import_module(pkg.__name__ + ".loader")


def test_moe_layer_matches_ground_truth(pkg, ckpt_dir):
    root, truth = ckpt_dir
    ld = _loader(pkg)
    ck = ld.Checkpoint(root)
    for layer in range(3):
        d = ld.read_moe_layer(ck, layer, device="cpu", dtype=torch.bfloat16)
        gu, dn = d["gate_up"], d["down"]
        assert (gu.E, gu.N, gu.K, gu.group, gu.layout) == (4, 256, 256, 32, "ct")
        assert (dn.E, dn.N, dn.K) == (4, 256, 128)
        assert gu.scale.dtype == torch.bfloat16 and gu.zeros is None
        w_gu = i4ref.ct_dequant(gu.packed.numpy(), gu.scale.float().numpy(), 256, 32)
        w_dn = i4ref.ct_dequant(dn.packed.numpy(), dn.scale.float().numpy(), 128, 32)
        for e, ex in enumerate(truth[layer]["experts"]):
            # rows [0, I) gate_proj, [I, 2I) up_proj (fused_packed_moe.py:122)
            np.testing.assert_array_equal(w_gu[e, :128], _ckpt.dense(ex["gate_proj"]))
            np.testing.assert_array_equal(w_gu[e, 128:], _ckpt.dense(ex["up_proj"]))
            np.testing.assert_array_equal(w_dn[e], _ckpt.dense(ex["down_proj"]))
            # the reference's own unpack of the same words (signed nibble - 8)
            np.testing.assert_array_equal(i4ref.unpack4(dn.packed[e].numpy(), 128),
                                          ex["down_proj"][0].astype(np.int32) - 8)
        np.testing.assert_array_equal(d["router_w"].float().numpy(), truth[layer]["router"])
        np.testing.assert_array_equal(d["norm_w"].float().numpy(), truth[layer]["norm"])
        assert d["top_k"] == 2 and d["norm_topk_prob"] and d["norm_eps"] == 1e-6


def test_single_file_checkpoint_and_group_inference(pkg, tmp_path):
    ld = _loader(pkg)
    truth = _ckpt.write_checkpoint(tmp_path, np.random.default_rng(52), n_layers=1, E=2, H=128,
                                   I=64, G=64, single_file=True, group_in_config=True)
    ck = ld.Checkpoint(tmp_path)
    assert ck.group_size() == 64
    d = ld.read_moe_layer(ck, 0, device="cpu")
    w = i4ref.ct_dequant(d["down"].packed.numpy(), d["down"].scale.float().numpy(), 64, 64)
    np.testing.assert_array_equal(w[1], _ckpt.dense(truth[0]["experts"][1]["down_proj"]))


def test_attention_triplets(pkg, ckpt_dir):
    root, truth = ckpt_dir
    ld = _loader(pkg)
    ck = ld.Checkpoint(root)
    for name, (out_f, in_f) in (("q_proj", (256, 256)), ("k_proj", (64, 256)),
                                ("o_proj", (256, 256))):
        p, s, n, k = ck.triplet(f"thinker.model.layers.1.self_attn.{name}")
        assert (n, k) == (out_f, in_f)
        w = i4ref.ct_dequant(p.numpy(), s.float().numpy(), k, 32)
        np.testing.assert_array_equal(w, _ckpt.dense(truth[1]["attn"][name]))


def test_reader_rejects_bad_checkpoints(pkg, tmp_path):
    ld = _loader(pkg)
    with pytest.raises(FileNotFoundError):
        (tmp_path / "config.json").write_text("{}")
        ld.Checkpoint(tmp_path)
    root = tmp_path / "ck"
    _ckpt.write_checkpoint(root, np.random.default_rng(53), n_layers=1, E=2, H=128, I=64,
                           single_file=True)
    ck = ld.Checkpoint(root)
    with pytest.raises(KeyError):
        ck.tensor("thinker.model.layers.7.mlp.gate.weight")
    # a weight_shape that does not match the packed words
    from safetensors.torch import load_file, save_file

    blob = load_file(str(root / "model.safetensors"))
    key = "thinker.model.layers.0.mlp.experts.1.up_proj.weight_shape"
    blob[key] = torch.tensor([64, 256], dtype=torch.int64)
    save_file(blob, str(root / "model.safetensors"))
    with pytest.raises(ValueError):
        ld.read_moe_layer(ld.Checkpoint(root), 0, device="cpu")
    # asymmetric (zero-point) triplets are refused, not misread
    blob[key] = torch.tensor([64, 128], dtype=torch.int64)
    blob["thinker.model.layers.0.mlp.experts.0.gate_proj.weight_zero_point"] = torch.zeros(
        64, 4, dtype=torch.int32)
    save_file(blob, str(root / "model.safetensors"))
    with pytest.raises(NotImplementedError):
        ld.read_moe_layer(ld.Checkpoint(root), 0, device="cpu")
    # a group size that does not match the scale columns
    cfg = json.loads((root / "config.json").read_text())
    cfg["quantization_config"]["config_groups"]["group_0"]["weights"]["group_size"] = 64
    (root / "config.json").write_text(json.dumps(cfg))
    del blob["thinker.model.layers.0.mlp.experts.0.gate_proj.weight_zero_point"]
    save_file(blob, str(root / "model.safetensors"))
    with pytest.raises(ValueError):
        ld.read_moe_layer(ld.Checkpoint(root), 0, device="cpu")


def test_dense_layers_are_refused(pkg, tmp_path):
    ld = _loader(pkg)
    _ckpt.write_checkpoint(tmp_path, np.random.default_rng(54), n_layers=2, E=2, H=128, I=64,
                           single_file=True)
    cfg = json.loads((tmp_path / "config.json").read_text())
    cfg["thinker_config"]["text_config"]["mlp_only_layers"] = [1]
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError):
        ld.load_thinker_moe_stack(tmp_path, 2, device="cpu")

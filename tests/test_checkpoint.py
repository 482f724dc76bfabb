"""Checkpoint loader on the CPU: safetensors shards, fused static Linear
components, the SOFT embedding and the static KV metadata.  The KV metadata
cases restate the reference's test_hif8_kv_runtime.py:203-249."""

import json

import pytest
import torch

from _checkpoint import ATTN, EMBED, GATE_UP, KV_SCALES, MLP, QKV, VOCAB, HIDDEN, write_checkpoint
from hif8_rocm import checkpoint as ckpt


@pytest.fixture
def tiny(tmp_path):
    tensors = write_checkpoint(tmp_path / "ckpt")
    return tmp_path / "ckpt", tensors


def test_fused_static_linear_concatenates_components(tiny):
    root, tensors = tiny
    c = ckpt.Hif8Checkpoint.open(root)
    layer = c.static_linear([f"{ATTN}.{n}" for n in QKV], "cpu")
    want_w = torch.cat([tensors[f"{ATTN}.{n}.weight"] for n in QKV])
    want_s = torch.cat([tensors[f"{ATTN}.{n}.weight_scale"] for n in QKV]).reshape(-1)
    assert layer.weight.dtype == torch.uint8 and tuple(layer.weight.shape) == (sum(QKV.values()), HIDDEN)
    assert torch.equal(layer.weight, want_w)
    assert torch.equal(layer.weight_scale, want_s)
    assert tuple(layer.input_scale.shape) == (1,) and float(layer.input_scale) == pytest.approx(0.01)
    assert layer.quant_method.quant_type == "W8A8HIF8_STATIC"
    mlp = c.static_linear([f"{MLP}.{n}" for n in GATE_UP], "cpu")
    assert tuple(mlp.weight.shape) == (sum(GATE_UP.values()), HIDDEN)


def test_single_file_checkpoint_without_index(tmp_path):
    tensors = write_checkpoint(tmp_path, single_file=True)
    c = ckpt.Hif8Checkpoint.open(tmp_path)
    assert set(c.weight_map) == set(tensors)
    assert torch.equal(c.tensor("model.norm.weight"), tensors["model.norm.weight"])


def test_fused_components_must_share_the_input_scale(tmp_path):
    write_checkpoint(tmp_path, qkv_input_scales=(0.01, 0.01, 0.02))
    c = ckpt.Hif8Checkpoint.open(tmp_path)
    with pytest.raises(ValueError, match="different input scales"):
        c.static_linear([f"{ATTN}.{n}" for n in QKV], "cpu")
    layer = c.static_linear([f"{ATTN}.q_proj"], "cpu")
    assert tuple(layer.weight.shape) == (QKV["q_proj"], HIDDEN)


def test_quant_types_are_checked(tiny):
    root, _ = tiny
    c = ckpt.Hif8Checkpoint.open(root)
    with pytest.raises(ValueError, match="expected W8A8HIF8_STATIC"):
        c.static_linear([EMBED], "cpu")
    with pytest.raises(ValueError, match="expected W8A8HIF8_SOFT"):
        c.embedding(f"{ATTN}.q_proj", "cpu")
    with pytest.raises(KeyError, match="not in the checkpoint"):
        c.tensor("model.layers.9.mlp.down_proj.weight")
    emb = c.embedding(EMBED, "cpu")
    assert tuple(emb.weight.shape) == (VOCAB, HIDDEN) and tuple(emb.weight_scale.shape) == (VOCAB,)


def test_unknown_quant_type_is_rejected(tiny):
    root, _ = tiny
    desc = json.loads((root / "quant_model_description.json").read_text())
    desc["model.norm.weight"] = "W4A4_MXFP4"
    (root / "quant_model_description.json").write_text(json.dumps(desc))
    with pytest.raises(ValueError, match="unsupported quant types"):
        ckpt.Hif8Checkpoint.open(root)


def test_missing_files_are_reported(tmp_path):
    with pytest.raises(FileNotFoundError, match="model.safetensors"):
        ckpt.Hif8Checkpoint.open(tmp_path)
    write_checkpoint(tmp_path)
    (tmp_path / "quant_model_description.json").unlink()
    with pytest.raises(FileNotFoundError, match="quant_model_description.json"):
        ckpt.Hif8Checkpoint.open(tmp_path)


def test_static_kv_metadata_is_loaded_and_validated(tmp_path):
    meta = {"format": "W8A8HIF8_STATIC",
            "kv_cache": {"mode": "static_per_layer_per_head",
                         "layers": {"3": {"key_scales": [0.1, 0.2], "value_scales": [0.3, 0.4]}}}}
    (tmp_path / "hif8_metadata.json").write_text(json.dumps(meta))
    assert ckpt.load_static_kv_scales(tmp_path) == {3: ((0.1, 0.2), (0.3, 0.4))}
    meta["kv_cache"]["layers"]["3"]["key_scales"][0] = 0.0
    (tmp_path / "hif8_metadata.json").write_text(json.dumps(meta))
    with pytest.raises(ValueError, match="invalid key_scales"):
        ckpt.load_static_kv_scales(tmp_path)


def test_static_checkpoint_never_silently_uses_dynamic_kv(tmp_path):
    (tmp_path / "hif8_metadata.json").write_text(json.dumps({"format": "W8A8HIF8_STATIC"}))
    with pytest.raises(ValueError, match="missing kv_cache metadata"):
        ckpt.load_static_kv_scales(tmp_path)


def test_legacy_checkpoint_without_static_metadata_keeps_dynamic_fallback(tmp_path):
    assert ckpt.load_static_kv_scales(tmp_path) is None
    (tmp_path / "hif8_metadata.json").write_text(json.dumps({"format": "W8A8HIF8_SOFT"}))
    assert ckpt.load_static_kv_scales(tmp_path) is None


@pytest.mark.parametrize("layers,match", [
    ({}, "layers is empty"),
    ({"03": dict(KV_SCALES)}, "invalid static KV layer index"),
    ({"-1": dict(KV_SCALES)}, "invalid static KV layer index"),
    ({"x": dict(KV_SCALES)}, "invalid static KV layer index"),
    ({"2": {"value_scales": [1.0]}}, "has no key_scales"),
    ({"2": {"key_scales": [1.0], "value_scales": [float("inf")]}}, "invalid value_scales"),
    ({"2": {"key_scales": [1.0, 2.0], "value_scales": [1.0]}}, "different K/V head counts"),
])
def test_malformed_kv_metadata_is_rejected(tmp_path, layers, match):
    meta = {"format": "W8A8HIF8_STATIC", "kv_cache": {"mode": "static_per_layer_per_head", "layers": layers}}
    (tmp_path / "hif8_metadata.json").write_text(json.dumps(meta))
    with pytest.raises(ValueError, match=match):
        ckpt.load_static_kv_scales(tmp_path)


def test_unsupported_kv_mode_is_rejected(tmp_path):
    meta = {"format": "W8A8HIF8_STATIC", "kv_cache": {"mode": "dynamic_per_token", "layers": {}}}
    (tmp_path / "hif8_metadata.json").write_text(json.dumps(meta))
    with pytest.raises(ValueError, match="unsupported HIF8 kv_cache metadata"):
        ckpt.load_static_kv_scales(tmp_path)


def test_kv_scales_of_one_layer_as_tensors(tiny):
    root, _ = tiny
    c = ckpt.Hif8Checkpoint.open(root)
    k, v = c.kv_scales(3, "cpu")
    assert k.dtype == torch.float32 and k.tolist() == KV_SCALES["key_scales"]
    assert v.tolist() == KV_SCALES["value_scales"]
    with pytest.raises(KeyError, match="layer 4"):
        c.kv_scales(4, "cpu")

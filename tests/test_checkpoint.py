"""MLX-LM checkpoint metadata, selection and conversion guards (CPU), after
the tests of eredu/src/backend/mlx/runtime/checkpoint/quantization.rs:545-620."""
import json
import os

import pytest
import torch

from eredu_amd import EreduError
from eredu_amd import checkpoint as C


def test_affine_config_uses_mlx_spelling():
    assert C.WeightQuantization().to_json() == {"group_size": 64, "bits": 4, "mode": "affine"}


def test_mxfp4_metadata_is_fixed_and_round_trips():
    v = {"group_size": 32, "bits": 4, "mode": "mxfp4"}
    assert C.WeightQuantization.from_json(v).to_json() == v
    for bad in ({"group_size": 64, "bits": 4, "mode": "mxfp4"}, {"group_size": 32, "bits": 8, "mode": "mxfp4"}):
        with pytest.raises(EreduError):
            C.WeightQuantization.from_json(bad)


def test_omitted_quantization_mode_defaults_to_affine():
    assert C.WeightQuantization.from_json({"group_size": 64, "bits": 4}) == C.WeightQuantization(64, 4, "affine")


def test_affine_config_accepts_mlx_widths():
    for gs, bits in ((32, 3), (32, 5), (32, 6), (16, 2), (128, 8)):
        C.WeightQuantization(gs, bits).validate()
    for gs, bits in ((32, 7), (48, 4), (0, 4)):
        with pytest.raises(EreduError):
            C.WeightQuantization(gs, bits).validate()


def test_on_load_resolution_reuses_matching_metadata_and_rejects_mismatch():
    q4, q8 = C.WeightQuantization(), C.WeightQuantization(64, 8)
    assert C.should_quantize_on_load("test", None, q4)
    assert not C.should_quantize_on_load("test", q4, q4)
    with pytest.raises(EreduError, match="already quantized.*implicit dequantization"):
        C.should_quantize_on_load("test", q4, q8)
    mx = C.WeightQuantization(32, 4, "mxfp4")
    assert not C.should_quantize_on_load("test", mx, mx)


def test_selection_is_model_agnostic_and_filterable():
    tensor, vector = torch.zeros(128, 64), torch.zeros(8192)
    opts = C.CheckpointQuantizationOptions()
    assert opts.selects("anything.proj.weight", tensor)
    assert opts.selects("anything.proj_weight", tensor)
    assert not opts.selects("anything.norm.weight", vector)
    assert not opts.selects("anything.proj.bias", tensor)
    assert not opts.selects("anything.proj.weight", torch.zeros(128, 64, dtype=torch.int32))
    assert not opts.selects("anything.proj.weight", torch.zeros(128, 96))  # 96 % 64
    opts.exclude.append("proj")
    assert not opts.selects("anything.proj.weight", tensor)
    opts = C.CheckpointQuantizationOptions(include=["mlp"], minimum_elements=4096)
    assert opts.selects("layers.0.mlp.up.weight", torch.zeros(64, 64))
    assert not opts.selects("layers.0.mlp.up.weight", torch.zeros(32, 64))
    assert not opts.selects("layers.0.attn.q.weight", torch.zeros(64, 64))


def test_canonical_weight_names():
    assert C.canonical_weight_name("a.b.weight") == "a.b.weight"
    assert C.canonical_weight_name("a.b_weight") == "a.b.weight"
    assert C.canonical_weight_name("a.b.bias") is None


def test_metadata_reading():
    assert C.checkpoint_quantization_metadata(None) is None
    assert C.checkpoint_quantization_metadata({"model_type": "x"}) is None
    q = C.checkpoint_quantization_metadata({"quantization": None,
                                            "quantization_config": {"group_size": 32, "bits": 8, "mode": "affine"}})
    assert q == C.WeightQuantization(32, 8)
    with pytest.raises(EreduError, match="not MLX affine/MXFP4"):
        C.checkpoint_quantization_metadata({"quantization_config": {"quant_method": "gptq", "bits": 4}})
    with pytest.raises(EreduError, match="JSON object"):
        C.checkpoint_quantization_metadata([1, 2])


def _write_config(d, obj):
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(obj, f)


def test_checkpoint_conversion_rejects_prequantized_inputs(tmp_path):
    src = tmp_path / "source"
    src.mkdir()
    _write_config(src, {"quantization": {"group_size": 64, "bits": 4, "mode": "affine"}})
    opts = C.CheckpointQuantizationOptions(quantization=C.WeightQuantization(32, 4, "mxfp4"))
    with pytest.raises(EreduError, match="implicit transcoding"):
        C.quantize_checkpoint(str(src), str(tmp_path / "out"), opts)
    with pytest.raises(EreduError, match="reuse it"):
        C.quantize_checkpoint(str(src), str(tmp_path / "out"))
    assert not (tmp_path / "out").exists()
    with pytest.raises(EreduError, match="not a directory"):
        C.quantize_checkpoint(str(tmp_path / "missing"), str(tmp_path / "out"))
    with pytest.raises(EreduError, match="shard_size_bytes"):
        C.quantize_checkpoint(str(src), str(tmp_path / "out"), C.CheckpointQuantizationOptions(shard_size_bytes=0))


def test_safetensors_files_follow_the_index(tmp_path):
    assert C.safetensors_files(str(tmp_path)) == [str(tmp_path / "model.safetensors")]
    with open(tmp_path / "model.safetensors.index.json", "w") as f:
        json.dump({"weight_map": {"a": "model-00002-of-00002.safetensors", "b": "model-00001-of-00002.safetensors",
                                  "c": "model-00002-of-00002.safetensors"}}, f)
    assert C.safetensors_files(str(tmp_path)) == [str(tmp_path / "model-00001-of-00002.safetensors"),
                                                  str(tmp_path / "model-00002-of-00002.safetensors")]


def test_loader_refuses_quantized_tensors_without_metadata(tmp_path):
    from safetensors.torch import save_file

    save_file({"p.weight": torch.zeros(4, 8, dtype=torch.int32), "p.scales": torch.zeros(4, 1)},
              str(tmp_path / "model.safetensors"))
    with pytest.raises(EreduError, match="no affine or MXFP4 quantization metadata"):
        C.load_quantized_checkpoint(str(tmp_path))


def test_gguf_blocks_cannot_be_produced_by_dense_quantization():
    """quantization.rs:226-233: GgufIQuant has no dense quantizer (raised before any device work)."""
    import torch

    with pytest.raises(EreduError, match="cannot be produced by dense quantization"):
        C.quantize_tensor(torch.ones(2, 256), C.WeightQuantization.GgufIQuant(12))

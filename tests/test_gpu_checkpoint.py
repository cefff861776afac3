"""MLX-LM checkpoint conversion and loading on the GPU, after
saved_checkpoint_matches_direct_tensor_quantization
(eredu/src/backend/mlx/runtime/checkpoint/quantization.rs:693-781): the
saved codes/scales/biases equal direct tensor quantization and the oracle's
MLX quantizer restatement bit for bit; a loaded checkpoint's linears match
quantized_matmul on the same tensors bit for bit and the fp64 oracle within
the matmul rule (1e-2 RMS + 1/2 bf16 ulp)."""
import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import load_file, save_file

from eredu_amd import EreduError, quantized_matmul
from eredu_amd import checkpoint as C
from oracle import oracle as orc
from tests.fixtures import host_bits16

pytestmark = pytest.mark.gpu


def test_saved_checkpoint_matches_direct_tensor_quantization(cuda, tmp_path):
    src, out = tmp_path / "source", tmp_path / "output"
    src.mkdir()
    with open(src / "config.json", "w") as f:
        f.write('{"model_type":"test"}')
    weight = ((torch.arange(8 * 64, dtype=torch.float32) - 255.5) / 64.0).reshape(8, 64)
    norm = torch.ones(64)
    save_file({"model.proj.weight": weight, "model.norm.weight": norm}, str(src / "model.safetensors"))
    save_file({"auxiliary.weight": norm}, str(src / "auxiliary.safetensors"))
    opts = C.CheckpointQuantizationOptions(shard_size_bytes=300)  # proj's three arrays (320 B), then norm
    report = C.quantize_checkpoint(str(src), str(out), opts)
    assert report == {"quantized_tensors": 1, "copied_tensors": 1, "shards": 2, "total_size": 256 + 32 + 32 + 256}
    saved = {}
    for file in C.safetensors_files(str(out)):
        saved.update(load_file(file))
    wq, s, b = C.quantize_tensor(weight, opts.quantization)
    assert saved["model.proj.weight"].dtype == torch.uint32
    assert torch.equal(saved["model.proj.weight"], wq.cpu())
    assert torch.equal(saved["model.proj.scales"], s.cpu()) and torch.equal(saved["model.proj.biases"], b.cpu())
    assert torch.equal(saved["model.norm.weight"], norm)
    # the oracle's restatement of MLX's quantizer, f32 parameters
    ow, os_, ob = orc.quantize_affine(weight.numpy(), 64, 4, orc.F32)
    assert np.array_equal(saved["model.proj.weight"].view(torch.int32).numpy().view(np.uint32), ow)
    assert np.array_equal(saved["model.proj.scales"].numpy(), os_) and np.array_equal(saved["model.proj.biases"].numpy(), ob)
    config = json.load(open(out / "config.json"))
    assert config["quantization"] == config["quantization_config"] == {"group_size": 64, "bits": 4, "mode": "affine"}
    assert config["model_type"] == "test"
    assert (out / "auxiliary.safetensors").exists()
    index = json.load(open(out / "model.safetensors.index.json"))
    assert index["metadata"]["total_size"] == report["total_size"]
    wm = index["weight_map"]
    assert sorted(wm) == sorted(saved)
    assert set(wm.values()) == {"model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors"}
    assert wm["model.norm.weight"] != wm["model.proj.weight"] == wm["model.proj.scales"] == wm["model.proj.biases"]


def test_rank_three_expert_bank(cuda):
    experts = torch.full((3, 8, 64), 0.25)
    wq, s, b = C.quantize_tensor(experts, C.WeightQuantization(32, 4))
    assert tuple(wq.shape) == (3, 8, 8) and tuple(s.shape) == (3, 8, 2) and tuple(b.shape) == (3, 8, 2)


def test_mxfp4_checkpoint_round_trip(cuda, tmp_path):
    """An MXFP4 checkpoint: weight + uint8 scales, no biases, both metadata
    keys; loaded layers run the MXFP4 matmul (quantization.rs:226-233)."""
    from eredu_amd import QuantizationMode, quantized_matmul_with_mode

    src, out = tmp_path / "source", tmp_path / "out"
    src.mkdir()
    g = torch.Generator().manual_seed(4)
    dense = {"m.proj.weight": (0.05 * torch.randn(256, 512, generator=g)).to(torch.bfloat16),
             "m.norm.weight": torch.ones(512, dtype=torch.bfloat16)}
    save_file(dense, str(src / "model.safetensors"))
    mx = C.WeightQuantization(32, 4, "mxfp4")
    C.quantize_checkpoint(str(src), str(out), C.CheckpointQuantizationOptions(quantization=mx))
    saved = load_file(str(out / "model.safetensors"))
    assert sorted(saved) == ["m.norm.weight", "m.proj.scales", "m.proj.weight"]
    assert saved["m.proj.scales"].dtype == torch.uint8 and tuple(saved["m.proj.scales"].shape) == (256, 16)
    with open(out / "config.json") as f:
        assert json.load(f)["quantization"] == {"group_size": 32, "bits": 4, "mode": "mxfp4"}
    linears, rest, quant = C.load_quantized_checkpoint(str(out))
    assert quant == mx and list(rest) == ["m.norm.weight"]
    lin = linears["m.proj"]
    assert lin.mode is QuantizationMode.MxFp4 and lin.biases is None
    x = torch.randn(3, 512, generator=g).to(torch.bfloat16).cuda()
    wq, s, b = C.quantize_tensor(dense["m.proj.weight"], mx)
    assert b is None
    y2 = quantized_matmul_with_mode(x, wq.view(torch.int32), s, None, True, 32, 4, QuantizationMode.MxFp4)
    assert torch.equal(lin(x).view(torch.int16), y2.view(torch.int16))



@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 32)])
def test_loaded_checkpoint_runs_the_quantized_path(cuda, tmp_path, bits, gs):
    src, out = tmp_path / "source", tmp_path / "output"
    src.mkdir()
    g = torch.Generator().manual_seed(bits)
    dense = {f"layers.{i}.mlp.{p}.weight": (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16)
             for i in range(2) for p, N, K in (("up", 512, 256), ("down", 256, 512))}
    dense["layers.0.norm.weight"] = torch.ones(256, dtype=torch.bfloat16)
    save_file(dense, str(src / "model.safetensors"))
    C.quantize_checkpoint(str(src), str(out), C.CheckpointQuantizationOptions(quantization=C.WeightQuantization(gs, bits)))
    linears, rest, quant = C.load_quantized_checkpoint(str(out))
    assert quant == C.WeightQuantization(gs, bits)
    assert sorted(linears) == sorted(k[: -len(".weight")] for k in dense if ".mlp." in k)
    assert list(rest) == ["layers.0.norm.weight"]
    for name, lin in linears.items():
        K = lin.input_dims
        x = (torch.randn(3, K, generator=g)).to(torch.bfloat16).cuda()
        y = lin(x)
        wq, s, b = C.quantize_tensor(dense[name + ".weight"], C.WeightQuantization(gs, bits))
        y2 = quantized_matmul(x, wq.view(torch.int32), s, b, transpose=True, group_size=gs, bits=bits)
        assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
        xb = host_bits16(x)
        y_ref = orc.quantized_matmul_f64(xb, orc.BF16, wq.view(torch.int32).cpu().numpy().view(np.uint32),
                                         host_bits16(s), host_bits16(b), orc.BF16, True, gs, bits, lin.output_dims, K)
        ok, worst, _ = orc.matmul_within_tolerance(y.float().cpu().numpy(), y_ref, out_is_bf16=True)
        assert ok, f"{name}: max|err|/RMS = {worst:.3e}"

"""MLX-LM quantized SafeTensors checkpoints: the on-disk form of the affine
contract (eredu/src/backend/mlx/runtime/checkpoint/quantization.rs).

A dense ``name.weight`` matrix becomes the packed ``name.weight`` (uint32
codes) plus ``name.scales`` and ``name.biases``; ``config.json`` carries the
settings under both ``quantization`` and ``quantization_config``.  This
module mirrors the reference's metadata rules, tensor selection and
``quantize_checkpoint`` (tensor-by-tensor conversion, shards of at most
``shard_size_bytes``, a ``model.safetensors.index.json`` when there is more
than one), quantizing on the GPU with ``eq_quantize``; and loads such a
checkpoint into device-resident ``QuantizedLinear`` layers.
"""
from __future__ import annotations

import dataclasses
import json
import os
import shutil
from typing import Dict, List, Optional, Tuple

import torch

from ._native import EreduError
from .quantization import QuantizationMode, QuantizedLinear, quantize_with_mode

_INDEX = "model.safetensors.index.json"


@dataclasses.dataclass(frozen=True)
class WeightQuantization:
    """Stored weight encoding (eredu-checkpoint/src/lib.rs:69-123,140-250):
    affine (group_size 16 or a positive multiple of 32; bits 2, 3, 4, 5, 6
    or 8), MXFP4 (fixed group 32, 4 bits, no biases), or checkpoint-native
    GGML blocks (``mode`` "gguf" with ``ggml_type`` and ``endian``; group_size
    and bits then hold the block geometry, values and bytes per block, as
    WeightQuantization::GgufIQuant reports them)."""

    group_size: int = 64
    bits: int = 4
    mode: str = "affine"
    ggml_type: Optional[int] = None
    endian: int = 0

    @staticmethod
    def Affine(group_size: int = 64, bits: int = 4) -> "WeightQuantization":
        q = WeightQuantization(group_size, bits, "affine")
        q.validate()
        return q

    @staticmethod
    def MxFp4() -> "WeightQuantization":
        return WeightQuantization(32, 4, "mxfp4")

    @staticmethod
    def GgufIQuant(ggml_type: int, endian: int = 0) -> "WeightQuantization":
        """Native GGML blocks of ``ggml_type`` in a file of byte order ``endian``."""
        from .gguf import ggml_type_from_code

        ty = ggml_type_from_code(int(ggml_type))
        values, nbytes = ty.block_and_bytes()
        return WeightQuantization(values, nbytes, "gguf", int(ty), int(endian))

    def gguf_iquant(self):
        """(ggml_type, endian) for native GGML blocks, else None (lib.rs:190-196)."""
        return (self.ggml_type, self.endian) if self.mode == "gguf" else None

    def validate(self) -> None:
        if self.mode == "gguf":
            from .gguf import ggml_type_from_code

            if self.ggml_type is None:
                raise EreduError("native GGUF quantization needs a GGML type")
            ggml_type_from_code(self.ggml_type).block_and_bytes()
            return
        if self.mode == "mxfp4":
            if (self.group_size, self.bits) != (32, 4):
                raise EreduError(f"mxfp4 metadata must be group_size 32, bits 4, got {self.group_size}, {self.bits}")
            return
        if self.mode != "affine":
            raise EreduError(f"unknown quantization mode {self.mode!r}")
        if self.group_size != 16 and (self.group_size <= 0 or self.group_size % 32 != 0):
            raise EreduError(f"group_size must be 16 or a positive multiple of 32, got {self.group_size}")
        if self.bits not in (2, 3, 4, 5, 6, 8):
            raise EreduError(f"bits must be one of 2, 3, 4, 5, 6, or 8, got {self.bits}")

    @property
    def has_biases(self) -> bool:
        return self.mode == "affine"

    def to_json(self) -> dict:
        """MLX spelling: {"group_size", "bits", "mode"} (affine and MXFP4 only)."""
        if self.mode == "gguf":
            raise EreduError("native GGUF quantization has no MLX checkpoint metadata")
        return {"group_size": self.group_size, "bits": self.bits, "mode": self.mode}

    @staticmethod
    def from_json(value: dict) -> "WeightQuantization":
        """An omitted mode means affine (lib.rs:207-214)."""
        if not isinstance(value, dict) or "group_size" not in value or "bits" not in value:
            raise EreduError(f"invalid quantization metadata {value!r}")
        mode = str(value.get("mode", "affine"))
        if mode not in ("affine", "mxfp4"):
            raise EreduError(f"unknown quantization mode {mode!r}")
        q = WeightQuantization(int(value["group_size"]), int(value["bits"]), mode)
        q.validate()
        return q


def checkpoint_quantization_metadata(config: Optional[dict]) -> Optional[WeightQuantization]:
    """The stored encoding of a checkpoint's config.json (quantization.rs:315-342):
    the first non-null of ``quantization`` / ``quantization_config``; it must
    name a ``mode`` (other prequantized formats are refused)."""
    if config is None:
        return None
    if not isinstance(config, dict):
        raise EreduError("config.json must contain a JSON object")
    for key in ("quantization", "quantization_config"):
        value = config.get(key)
        if value is None:
            continue
        if isinstance(value, dict) and "mode" in value:
            try:
                return WeightQuantization.from_json(value)
            except EreduError as e:
                raise EreduError(f"invalid {key} metadata: {e}") from e
        raise EreduError(f"checkpoint contains prequantized {key} metadata that is not MLX affine/MXFP4; "
                         f"implicit transcoding is unsupported")
    return None


def should_quantize_on_load(architecture: str, existing: Optional[WeightQuantization],
                            requested: WeightQuantization) -> bool:
    """True for a dense checkpoint that must be quantized, False when it is
    already stored as requested (quantization.rs:26-39)."""
    requested.validate()
    if existing is None:
        return True
    if existing == requested:
        return False
    raise EreduError(f"{architecture} checkpoint is already quantized as {existing}, requested {requested}; "
                     f"implicit dequantization and requantization is unsupported")


def canonical_weight_name(name: str) -> Optional[str]:
    """``x.weight`` as is, ``x_weight`` as ``x.weight``, else None (quantization.rs:125-131)."""
    if name.endswith(".weight"):
        return name
    if name.endswith("_weight"):
        return name[: -len("_weight")] + ".weight"
    return None


@dataclasses.dataclass
class CheckpointQuantizationOptions:
    """Tensor selection and output sharding (quantization.rs:73-121)."""

    quantization: WeightQuantization = dataclasses.field(default_factory=WeightQuantization)
    shard_size_bytes: int = 512 * 1024 * 1024
    include: List[str] = dataclasses.field(default_factory=list)
    exclude: List[str] = dataclasses.field(default_factory=list)
    minimum_elements: int = 0

    def selects(self, name: str, tensor: torch.Tensor) -> bool:
        gs = self.quantization.group_size
        return (canonical_weight_name(name) is not None and tensor.dim() == 2 and tensor.dtype.is_floating_point
                and tensor.shape[1] % gs == 0 and tensor.shape[1] % 32 == 0
                and tensor.numel() >= self.minimum_elements
                and (not self.include or any(s in name for s in self.include))
                and not any(s in name for s in self.exclude))

    def validate(self) -> None:
        self.quantization.validate()
        if self.shard_size_bytes <= 0:
            raise EreduError("shard_size_bytes must be greater than zero")


def safetensors_files(model_dir: str) -> List[str]:
    """The index's files (sorted, unique) or ``model.safetensors``
    (eredu/src/backend/mlx/runtime/checkpoint/load.rs:771-788)."""
    index = os.path.join(model_dir, _INDEX)
    if os.path.exists(index):
        with open(index) as f:
            weight_map = json.load(f)["weight_map"]
        return sorted({os.path.join(model_dir, v) for v in weight_map.values()})
    return [os.path.join(model_dir, "model.safetensors")]


def quantize_tensor(weight: torch.Tensor, quantization: WeightQuantization
                    ) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Packed uint32 codes, scales and biases of one floating-point weight of
    rank >= 2, grouped along its last axis (leading dimensions, an expert
    bank's included, kept; quantization.rs:169-224), on the GPU with
    eq_quantize: affine (bits 2, 3, 4, 5, 6 or 8, group size 16 or a multiple
    of 32) or MXFP4 (uint8 E8M0 scales, biases None; quantization.rs:226-233)."""
    quantization.validate()
    if weight.dim() < 2 or not weight.dtype.is_floating_point:
        raise EreduError(f"expected a floating-point weight with at least two dimensions, got shape "
                         f"{tuple(weight.shape)} and dtype {weight.dtype}")
    cols = weight.shape[-1]
    if cols % quantization.group_size != 0 or cols % 32 != 0:
        raise EreduError(f"input dimension {cols} must be divisible by group_size {quantization.group_size} and 32")
    if quantization.mode not in ("affine", "mxfp4"):
        raise EreduError("checkpoint-native GGML blocks cannot be produced by dense quantization")
    mode = QuantizationMode.MxFp4 if quantization.mode == "mxfp4" else QuantizationMode.Affine
    dev = weight if weight.is_cuda else weight.cuda()
    if dev.dtype == torch.float64:
        raise EreduError("float64 weights are not supported (f32, f16 or bf16)")
    wq, s, b = quantize_with_mode(dev, quantization.group_size, quantization.bits, mode)
    return wq.view(torch.uint32), s, b


def _config(model_dir: str) -> Optional[dict]:
    path = os.path.join(model_dir, "config.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


def quantize_checkpoint(source_dir: str, output_dir: str,
                        options: Optional[CheckpointQuantizationOptions] = None) -> Dict[str, int]:
    """Quantizes a SafeTensors model directory tensor by tensor into a new
    MLX-LM checkpoint (quantization.rs:273-510): selected matrices become
    weight/scales/biases, other tensors are copied, non-weight files are
    copied, config.json gains both quantization keys.  The output directory
    must not exist; it is removed again if conversion fails.  Returns the
    report (quantized_tensors, copied_tensors, shards, total_size)."""
    from safetensors import safe_open
    from safetensors.torch import save_file

    options = options or CheckpointQuantizationOptions()
    options.validate()
    if not os.path.isdir(source_dir):
        raise EreduError(f"source is not a directory: {source_dir}")
    existing = checkpoint_quantization_metadata(_config(source_dir))
    if existing is not None:
        if existing == options.quantization:
            raise EreduError(f"checkpoint already uses {existing}; reuse it instead of quantizing it again")
        raise EreduError(f"checkpoint is already quantized as {existing}, requested {options.quantization}; "
                         f"implicit transcoding is unsupported")
    try:
        os.mkdir(output_dir)
    except OSError as e:
        raise EreduError(f"could not create empty output directory {output_dir}: {e}") from e
    try:
        weight_files = safetensors_files(source_dir)
        for entry in sorted(os.listdir(source_dir)):
            path = os.path.join(source_dir, entry)
            if (os.path.isfile(path) and entry not in ("config.json", _INDEX)
                    and os.path.abspath(path) not in {os.path.abspath(p) for p in weight_files}):
                shutil.copy(path, os.path.join(output_dir, entry))
        config = _config(source_dir) or {}
        if not isinstance(config, dict):
            raise EreduError("config.json must contain a JSON object")
        config["quantization"] = options.quantization.to_json()
        config["quantization_config"] = options.quantization.to_json()
        if "moshi_name" in config:
            config["moshi_name"] = "model.safetensors"
        with open(os.path.join(output_dir, "config.json"), "w") as f:
            json.dump(config, f, indent=2)

        pending: Dict[str, torch.Tensor] = {}
        pending_bytes = 0
        shards: List[str] = []
        locations: Dict[str, int] = {}
        report = {"quantized_tensors": 0, "copied_tensors": 0, "shards": 0, "total_size": 0}

        def flush():
            nonlocal pending, pending_bytes
            path = os.path.join(output_dir, f".quantized-{len(shards):05d}.safetensors")
            save_file({k: v.contiguous().cpu() for k, v in pending.items()}, path)
            for k in pending:
                locations[k] = len(shards)
            shards.append(path)
            pending, pending_bytes = {}, 0

        for file in weight_files:
            with safe_open(file, "pt") as f:
                for name in f.keys():
                    tensor = f.get_tensor(name)
                    if options.selects(name, tensor):
                        report["quantized_tensors"] += 1
                        wname = canonical_weight_name(name)
                        wq, s, b = quantize_tensor(tensor, options.quantization)
                        prefix = wname[: -len(".weight")]
                        arrays = [(wname, wq), (prefix + ".scales", s)]
                        if b is not None and options.quantization.has_biases:
                            arrays.append((prefix + ".biases", b))
                    else:
                        report["copied_tensors"] += 1
                        arrays = [(name, tensor)]
                    incoming = sum(a.numel() * a.element_size() for _, a in arrays)
                    if pending and pending_bytes + incoming > options.shard_size_bytes:
                        flush()
                    for k, a in arrays:
                        report["total_size"] += a.numel() * a.element_size()
                        pending[k] = a
                        pending_bytes += a.numel() * a.element_size()
        if pending:
            flush()
        if not shards:
            raise EreduError("checkpoint contains no tensors")
        if len(shards) == 1:
            os.replace(shards[0], os.path.join(output_dir, "model.safetensors"))
        else:
            names = [f"model-{i + 1:05d}-of-{len(shards):05d}.safetensors" for i in range(len(shards))]
            for tmp, final in zip(shards, names):
                os.replace(tmp, os.path.join(output_dir, final))
            index = {"metadata": {"total_size": report["total_size"]},
                     "weight_map": {k: names[i] for k, i in sorted(locations.items())}}
            with open(os.path.join(output_dir, _INDEX), "w") as f:
                json.dump(index, f, indent=2)
        report["shards"] = len(shards)
        return report
    except BaseException:
        shutil.rmtree(output_dir, ignore_errors=True)
        raise


def load_quantized_checkpoint(model_dir: str, device: str = "cuda"
                              ) -> Tuple[Dict[str, QuantizedLinear], Dict[str, torch.Tensor],
                                         Optional[WeightQuantization]]:
    """Loads an MLX-LM checkpoint onto the GPU: every ``p.weight`` with a
    ``p.scales`` sibling becomes ``QuantizedLinear`` (key ``p``; codes,
    scales, biases resident in HBM), every other tensor is returned as is.
    The encoding (affine or MXFP4) comes from config.json; quantized tensors
    without such metadata are refused."""
    from safetensors import safe_open

    quant = checkpoint_quantization_metadata(_config(model_dir))
    tensors: Dict[str, torch.Tensor] = {}
    for file in safetensors_files(model_dir):
        with safe_open(file, "pt") as f:
            for name in f.keys():
                tensors[name] = f.get_tensor(name)
    linears: Dict[str, QuantizedLinear] = {}
    for name in sorted(tensors):
        if not name.endswith(".scales"):
            continue
        prefix = name[: -len(".scales")]
        if prefix + ".weight" not in tensors:
            raise EreduError(f"{name} has no {prefix}.weight")
        if quant is None or quant.mode not in ("affine", "mxfp4"):
            raise EreduError(f"{prefix} is quantized but config.json has no affine or MXFP4 quantization metadata")
        w = tensors.pop(prefix + ".weight")
        s = tensors.pop(name)
        b = tensors.pop(prefix + ".biases", None)
        if w.dtype not in (torch.uint32, torch.int32) or w.dim() != 2:
            raise EreduError(f"{prefix}.weight must be 2-D packed uint32 codes, got {w.dtype} {tuple(w.shape)}")
        K = w.shape[1] * 32 // quant.bits
        if tuple(s.shape) != (w.shape[0], K // quant.group_size) or (b is not None and b.shape != s.shape):
            raise EreduError(f"{prefix}: scales/biases {tuple(s.shape)} do not match weight {tuple(w.shape)} "
                             f"at group_size {quant.group_size}, bits {quant.bits}")
        mode = QuantizationMode.MxFp4 if quant.mode == "mxfp4" else QuantizationMode.Affine
        if mode is QuantizationMode.MxFp4 and (b is not None or s.dtype != torch.uint8):
            raise EreduError(f"{prefix}: MXFP4 layers carry uint8 scales and no biases")
        bias = tensors.pop(prefix + ".bias", None)
        linears[prefix] = QuantizedLinear(w.view(torch.int32).to(device), s.to(device),
                                          None if b is None else b.to(device), quant.group_size, quant.bits,
                                          None if bias is None else bias.to(device), mode)
    return linears, tensors, quant

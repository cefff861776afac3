"""Streaming GGUF load (gguf_file.stream_convert_affine) on the GPU: a file
of Q4_0 / Q8_0 / Q4_K tensors (synthetic blocks) and a dense F32 tensor, in
both byte orders, read through 4 KiB pinned staging buffers (tensors split
across pieces and buffers alternating); every converted triple equal bit
for bit to the oracle's convert_affine restatement of the same blocks."""
import io

import numpy as np
import pytest
import torch

from eredu_amd import EreduError
from eredu_amd import gguf_file as F
from oracle import oracle as orc
from tests.fixtures import host_bits16, synthetic_blocks

pytestmark = pytest.mark.gpu

SHAPES = [("blk.0.attn_q.weight", F.Q4_0, 256, 96), ("blk.0.ffn_up.weight", F.Q8_0, 512, 40),
          ("blk.0.ffn_down.weight", F.Q4_K, 512, 24)]


def swap_headers(ty, raw):
    """f16 d (and Q4_K dmin) stored big-endian."""
    _, nbytes = F.BLOCK_GEOMETRY[ty]
    b = raw.reshape(-1, nbytes).copy()
    for h in ([0, 2] if ty == F.Q4_K else [0]):
        b[:, [h, h + 1]] = b[:, [h + 1, h]]
    return b.reshape(-1)


@pytest.mark.parametrize("endian", ["little", "big"])
def test_stream_convert_matches_the_oracle(cuda, tmp_path, endian):
    print(f"[case] stream GGUF endian={endian}", flush=True)
    tensors, raws = [], {}
    for i, (name, ty, cols, rows) in enumerate(SHAPES):
        block, _ = F.BLOCK_GEOMETRY[ty]
        raw = synthetic_blocks(ty, rows * cols // block, seed=i + 1)
        raws[name] = raw
        stored = swap_headers(ty, raw) if endian == "big" else raw
        tensors.append((name, [cols, rows], ty, stored.tobytes()))
    dense = np.arange(12, dtype=np.float32).reshape(3, 4)
    if endian == "little":
        tensors.append(("output_norm.weight", [4, 3], F.F32, dense.tobytes()))
    path = tmp_path / "model.gguf"
    with open(path, "wb") as f:
        F.write_gguf(f, {"general.architecture": F.MetadataValue(8, "llama")}, tensors, endian=endian,
                     alignment=64)
    out = F.stream_convert_affine(str(path), staging_bytes=4096)
    assert set(out) == {t[0] for t in tensors}
    for name, ty, cols, rows in SHAPES:
        a = out[name]
        w, s, b = orc.gguf_convert_affine(ty, raws[name])
        assert list(a.weight_shape) == [rows, cols * a.bits // 32]
        assert np.array_equal(a.weights.cpu().numpy().view(np.uint32).reshape(-1), w.reshape(-1)), name
        assert np.array_equal(host_bits16(a.scales).reshape(-1), s.reshape(-1)), name
        assert np.array_equal(host_bits16(a.biases).reshape(-1), b.reshape(-1)), name
    if endian == "little":
        assert torch.equal(out["output_norm.weight"].cpu(), torch.from_numpy(dense))


def test_selected_names_and_missing(cuda, tmp_path):
    raw = synthetic_blocks(F.Q4_0, 8, seed=3)
    path = tmp_path / "m.gguf"
    with open(path, "wb") as f:
        F.write_gguf(f, {}, [("a.weight", [64, 4], F.Q4_0, raw.tobytes()),
                             ("b.weight", [64, 4], F.Q4_0, raw.tobytes())])
    out = F.stream_convert_affine(str(path), names=["b.weight"])
    assert list(out) == ["b.weight"]
    with pytest.raises(EreduError, match="not present"):
        F.stream_convert_affine(str(path), names=["c.weight"])

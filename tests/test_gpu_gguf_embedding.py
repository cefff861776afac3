"""Native GGUF embedding on the device (eq_gguf_embedding): rows picked by
device token ids and decoded by the native definition, bit-exact against the
oracle's native dense decode of the same rows (f32, and bf16 as its
round-to-nearest-even image); ids outside the table raise the reference's
error in the mirror and give +0 rows through the C ABI."""
import numpy as np
import pytest
import torch

from eredu_amd import EreduError, _native
from eredu_amd import gguf as G
from oracle import oracle as orc
from tests.fixtures import dev_u8, host_bits16, synthetic_blocks
from tests.test_gpu_gguf import desc_for

pytestmark = pytest.mark.gpu

T = G.GgmlType
NATIVE = [T.Q4K, T.Q5K, T.Q6K, T.Q5_1, T.Q8_0, T.IQ4NL, T.IQ4XS]
ALL = NATIVE + [T.Q4_0, T.Q4_1, T.Q5_0, T.Q2K, T.Q3K]


def expected_rows(ty, raw, cols, ids, big=False):
    """The oracle's native decode of exactly the picked rows."""
    vals, nbytes = ty.block_and_bytes()
    row_bytes = cols // vals * nbytes
    picked = np.concatenate([raw[i * row_bytes:(i + 1) * row_bytes] for i in ids]) if len(ids) else raw[:0]
    return orc.gguf_dequant_f32(int(ty), picked, 1, big_endian=big).reshape(len(ids), cols)


def same_f32(got, ref):
    return np.all((got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref)))


@pytest.mark.parametrize("ty", ALL)
@pytest.mark.parametrize("endian", [G.Endian.Little, G.Endian.Big])
def test_embedding_bit_exact(cuda, ty, endian):
    rows, cols = 97, 768
    print(f"[case] embedding {ty.name} {endian.name} {rows}x{cols}", flush=True)
    vals, _ = ty.block_and_bytes()
    raw = synthetic_blocks(int(ty), rows * cols // vals, seed=int(ty) + 30)
    ids = np.array([5, 0, 96, 5, 41, 17, 96, 3], dtype=np.int32)  # repeats, both ends
    ref = expected_rows(ty, raw, cols, ids, endian == G.Endian.Big)
    desc = desc_for(ty, rows, cols)
    out = G.embedding(torch.from_numpy(ids).cuda(), desc, dev_u8(raw), endian)
    assert out.dtype == torch.float32 and list(out.shape) == [len(ids), cols]
    assert same_f32(out.cpu().numpy(), ref)
    out16 = G.embedding(torch.from_numpy(ids).cuda(), desc, dev_u8(raw), endian, torch.bfloat16)
    nan16 = lambda v: ((v & 0x7F80) == 0x7F80) & ((v & 0x7F) != 0)  # noqa: E731
    got16, ref16 = host_bits16(out16).reshape(-1), orc.f32_to_bf16_bits(ref).reshape(-1)
    assert np.all((got16 == ref16) | (nan16(got16) & nan16(ref16)))


def test_embedding_nd_indices_and_native_tensor(cuda):
    """NativeTensor.embedding: indices of any shape give shape + [cols]."""
    rows, cols = 64, 512
    raw = synthetic_blocks(int(T.Q4K), rows * cols // 256, seed=3)
    nt = G.NativeTensor("token_embd.weight", [rows, cols], T.Q4K, G.Endian.Little, dev_u8(raw))
    ids = torch.tensor([[1, 2, 63], [0, 0, 7]], dtype=torch.int64, device="cuda")
    out = nt.embedding(ids)
    assert list(out.shape) == [2, 3, cols]
    ref = expected_rows(T.Q4K, raw, cols, ids.cpu().numpy().reshape(-1)).reshape(2, 3, cols)
    assert same_f32(out.cpu().numpy(), ref)
    dense = nt.dequantize(torch.float32)  # the same rows of the whole-tensor native decode
    assert torch.equal(out.view(-1, cols).view(torch.int32), dense[ids.view(-1)].view(torch.int32))


def test_embedding_llama_vocab_row_and_unaligned_rows(cuda):
    """A decode-sized call (one token) on a 32000 x 4096 Q6_K table, and Q8_0
    rows of 102 bytes (not 16-byte multiples: byte copies)."""
    rows, cols = 32000, 4096
    print("[case] embedding Q6_K 32000x4096, 1 token", flush=True)
    raw = synthetic_blocks(int(T.Q6K), rows * cols // 256, seed=9)
    for tok in (31999, 12345):
        out = G.embedding(torch.tensor([tok], device="cuda"), desc_for(T.Q6K, rows, cols), dev_u8(raw))
        assert same_f32(out.cpu().numpy(), expected_rows(T.Q6K, raw, cols, [tok]))
    rows, cols = 40, 96
    raw = synthetic_blocks(int(T.Q8_0), rows * cols // 32, seed=10)
    ids = np.arange(39, -1, -3, dtype=np.int32)
    out = G.embedding(torch.from_numpy(ids).cuda(), desc_for(T.Q8_0, rows, cols), dev_u8(raw))
    assert same_f32(out.cpu().numpy(), expected_rows(T.Q8_0, raw, cols, ids))


def test_embedding_out_of_range(cuda):
    rows, cols = 16, 256
    raw = synthetic_blocks(int(T.Q8_0), rows * cols // 32, seed=11)
    desc = desc_for(T.Q8_0, rows, cols)
    with pytest.raises(EreduError, match=r"native embedding index 16 is outside 0\.\.16"):
        G.embedding(torch.tensor([3, 16, 2], device="cuda"), desc, dev_u8(raw))
    with pytest.raises(EreduError, match=r"index -1 is outside"):
        G.embedding(torch.tensor([-1], device="cuda"), desc, dev_u8(raw))
    # through the C ABI the ids are not read on the host: such a row is +0
    ids = torch.tensor([3, 16, -5, 2], dtype=torch.int32, device="cuda")
    out = torch.full((4, cols), float("nan"), device="cuda")
    d = dev_u8(raw)
    _native.check(_native.lib().eq_gguf_embedding(out.data_ptr(), d.data_ptr(), d.numel(), int(T.Q8_0), rows, cols,
                                                  ids.data_ptr(), 4, 0, _native.EQ_DTYPE_F32,
                                                  torch.cuda.current_stream().cuda_stream))
    got = out.cpu().numpy()
    assert np.all(got[1:3].view(np.uint32) == 0)
    assert same_f32(got[[0, 3]], expected_rows(T.Q8_0, raw, cols, [3, 2]))


def test_embedding_empty_and_rejects(cuda):
    raw = synthetic_blocks(int(T.Q4K), 4, seed=1)
    desc = desc_for(T.Q4K, 4, 256)
    out = G.embedding(torch.zeros(0, dtype=torch.int32, device="cuda"), desc, dev_u8(raw))
    assert list(out.shape) == [0, 256]
    with pytest.raises(EreduError, match="bfloat16 or float32"):
        G.embedding(torch.tensor([0], device="cuda"), desc, dev_u8(raw), dtype=torch.float16)

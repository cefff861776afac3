"""The device quantizer (C ABI eq_quantize) against the oracle's restatement
of MLX's affine quantize (bit-exact codes, scales and biases: the same f32
operations in the same order), and the reference's own round-trip test
(safemlx/src/ops/quantization.rs:457-486: rows 0..511 of arange, group 128,
bits 2/4/8, max |w - dequantize(quantize(w))| <= 127 / 2^bits)."""
import numpy as np
import pytest
import torch

from eredu_amd import dequantize, quantize, quantize_with_mode
from oracle import oracle as orc
from tests.fixtures import host_bits16

pytestmark = pytest.mark.gpu

DT = {orc.BF16: torch.bfloat16, orc.F16: torch.float16, orc.F32: torch.float32}


@pytest.mark.parametrize("dtype", [orc.BF16, orc.F16, orc.F32])
@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantize_matches_oracle(cuda, dtype, bits, gs):
    print(f"[case] quantize dtype={dtype} bits={bits} gs={gs}", flush=True)
    rng = np.random.default_rng(bits * 1000 + gs + dtype)
    rows, cols = 37, 512
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[3, :gs] = 0.0            # a constant group (scale clamps to 1e-7)
    w[5, :gs] = -1.0 * np.arange(gs) / gs  # all negative: the min is the edge
    wt = torch.from_numpy(w).to(DT[dtype]).cuda()
    w_in = wt.float().cpu().numpy()  # the values the device sees
    wq, s, b = quantize_with_mode(wt, gs, bits)
    torch.cuda.synchronize()
    rq, rs, rb = orc.quantize_affine(w_in, gs, bits, dtype)
    assert np.array_equal(wq.cpu().numpy().view(np.uint32), rq)
    if dtype == orc.F32:
        assert np.array_equal(s.cpu().numpy(), rs) and np.array_equal(b.cpu().numpy(), rb)
    else:
        assert np.array_equal(host_bits16(s), rs) and np.array_equal(host_bits16(b), rb)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_reference_round_trip(cuda, bits):
    x = (torch.ones((128, 1)) * torch.arange(512, dtype=torch.float32)[None, :]).cuda()
    wq, s, b = quantize(x, 128, bits)
    assert tuple(wq.shape) == (128, 512 * bits // 32)
    assert tuple(s.shape) == (128, 4) and tuple(b.shape) == (128, 4)
    x_hat = dequantize(wq, s, b, 128, bits)
    assert float((x - x_hat).abs().max()) <= 127.0 / (1 << bits)


def test_quantize_leading_dims_and_defaults(cuda):
    w = (torch.randn((2, 3, 256)) * 0.02).to(torch.bfloat16).cuda()
    wq, s, b = quantize(w)
    assert tuple(wq.shape) == (2, 3, 32) and tuple(s.shape) == (2, 3, 4) and s.dtype == torch.bfloat16
    wq2, s2, b2 = quantize(w.reshape(6, 256))
    assert torch.equal(wq.reshape(6, 32), wq2) and torch.equal(s.reshape(6, 4), s2)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_unaligned_buffers_take_the_scalar_kernels(cuda, bits):
    """Input / output pointers off 16-byte alignment run the one-value-per-step
    kernels; their results equal the vector kernels' bit for bit."""
    from eredu_amd import _native as n

    rows, cols, gs = 9, 256, 64
    rng = np.random.default_rng(bits)
    w = torch.from_numpy((rng.standard_normal(rows * cols) * 0.02).astype(np.float32)).to(torch.bfloat16)
    buf = torch.empty(rows * cols + 1, dtype=torch.bfloat16, device="cuda")
    buf[1:] = w.cuda()
    w_off = buf[1:].view(rows, cols)  # 2 bytes past a 16-byte boundary
    assert w_off.data_ptr() % 16 != 0
    q0, s0, b0 = quantize_with_mode(w.cuda().view(rows, cols), gs, bits)
    q1, s1, b1 = quantize_with_mode(w_off, gs, bits)
    assert torch.equal(q0, q1) and torch.equal(s0.view(torch.int16), s1.view(torch.int16))
    assert torch.equal(b0.view(torch.int16), b1.view(torch.int16))
    out = torch.empty(rows * cols + 1, dtype=torch.bfloat16, device="cuda")
    d0 = dequantize(q0, s0, b0, group_size=gs, bits=bits)
    n.check(n.lib().eq_dequantize(out.data_ptr() + 2, q0.data_ptr(), s0.data_ptr(), b0.data_ptr(), rows, cols, gs,
                                  bits, b"affine", n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, 0))
    torch.cuda.synchronize()
    assert torch.equal(out[1:].view(rows, cols).view(torch.int16), d0.view(torch.int16))

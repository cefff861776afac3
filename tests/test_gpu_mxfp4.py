"""MXFP4 mode ("mxfp4": E2M1 codes packed 8 per u32, one E8M0 scale byte per
32 values, no biases; safemlx/src/ops/quantization.rs:16-46) on the device,
against the oracle's MXFP4 functions.

* quantize: bit-exact codes and scale bytes (ties, zero / NaN / infinity
  groups, f32 subnormals, every activation dtype).
* dequantize: bit-exact f32 and bf16 values (scale bytes 0 and 255 included).
* the reference's own test (quantization.rs:488-549): arange(-64, 64) / 16 as
  [2, 64] -> weights [2, 8], scales [2, 2], no biases, max round-trip error
  <= 1, quantized_matmul of ones [3, 64] within 1e-3 of x @ dequantized^T;
  and its gather test (quantization.rs:700-730: zero codes, scale 127 -> 0).
* matmul (both transposes, the decode kernel, f16 / f32 activations), gather
  and batched calls: the matmul rule against mxfp4_matmul_f64,
  |y - y_ref| <= 1e-2 RMS(y_ref) (+ 1/2 bf16 ulp of y_ref for bf16 outputs).
* GGUF type 39: the golden block of eredu-gguf/tests/mxfp4.rs:5-60 and random
  blocks against mxfp4_convert_ggml (bit-exact).
"""
import math

import numpy as np
import pytest
import torch

from eredu_amd import (EreduError, QuantizationMode, dequantize_with_mode, gather_qmm_with_mode,
                       quantize_with_mode, quantized_matmul_batched, quantized_matmul_with_mode)
from eredu_amd import gguf as G
from oracle import oracle as orc
from tests.fixtures import dev_bf16, dev_param, dev_u8, dev_words, host_f32, synthetic_x

pytestmark = pytest.mark.gpu

MX = QuantizationMode.MxFp4
DT = {orc.BF16: torch.bfloat16, orc.F16: torch.float16, orc.F32: torch.float32}


def special_weights(rows, cols, seed):
    rng = np.random.default_rng(seed)
    mags = np.array([1e-3, 0.02, 1.0, 30.0, 0.5, 7.0])
    w = (rng.standard_normal((rows, cols)) * mags[np.arange(rows) % len(mags)][:, None]).astype(np.float32)
    w[0, :32] = 0.0                                          # an all-zero group
    w[1, 32:64] = -0.0
    w[2, :8] = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0]  # ties at scale 1 (amax 6)
    w[2, 8:32] = 0.0
    w[3, 40] = np.inf
    w[4, 70] = np.nan
    w[5, 100] = -np.inf
    w[6, :32] = 12.0                                         # a power of two times 6: scale 2, codes 6
    return w


@pytest.mark.parametrize("dtype", [orc.BF16, orc.F16, orc.F32])
def test_quantize_matches_oracle(cuda, dtype):
    print(f"[case] mxfp4 quantize dtype={dtype}", flush=True)
    rows, cols = 37, 512
    w = special_weights(rows, cols, 5 + dtype)
    if dtype == orc.F32:
        w[7, :32] = np.float32(1e-40) * np.arange(32)          # subnormals
        w[8, :32] = np.float32(3e38)                           # near the top of f32
    wt = torch.from_numpy(w).to(DT[dtype]).cuda()
    w_in = wt.float().cpu().numpy()  # the values the device sees
    wq, s, b = quantize_with_mode(wt, 32, 4, MX)
    torch.cuda.synchronize()
    assert b is None and s.dtype == torch.uint8
    assert tuple(wq.shape) == (rows, cols // 8) and tuple(s.shape) == (rows, cols // 32)
    rq, rs = orc.mxfp4_quantize(w_in)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(wq.cpu().numpy().view(np.uint32), rq)


def test_quantize_leading_dims(cuda):
    w = (torch.randn((2, 3, 128)) * 0.1).to(torch.bfloat16).cuda()
    wq, s, b = quantize_with_mode(w, 32, 4, MX)
    assert tuple(wq.shape) == (2, 3, 16) and tuple(s.shape) == (2, 3, 4) and b is None
    wq2, s2, _ = quantize_with_mode(w.reshape(6, 128), 32, 4, MX)
    assert torch.equal(wq.reshape(6, 16), wq2) and torch.equal(s.reshape(6, 4), s2)


@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16, torch.float16])
def test_dequantize_matches_oracle(cuda, out):
    rng = np.random.default_rng(3)
    rows, cols = 19, 256
    wq = rng.integers(0, 2 ** 32, size=(rows, cols // 8), dtype=np.uint32)
    sc = rng.integers(110, 140, size=(rows, cols // 32)).astype(np.uint8)
    sc[0, 0], sc[1, 1], sc[2, 2], sc[3, 3] = 0, 1, 254 if out == torch.float32 else 140, 255
    ref = orc.mxfp4_dequant_f64(wq, sc, rows, cols)
    y = dequantize_with_mode(dev_words(wq), dev_u8(sc), None, 32, 4, MX, dtype=out)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy().astype(np.float64)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    if out == torch.float32:
        with np.errstate(over="ignore"):  # 6 * 2^127 overflows to inf, as on the device
            exp = ref.astype(np.float32).astype(np.float64)
    else:
        exp = torch.from_numpy(ref).to(out).double().numpy()
    assert np.array_equal(got[~nan], exp[~nan])


@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16, torch.float16])
def test_dequantize_unaligned_output_takes_the_scalar_kernel(cuda, out):
    """An output 2 bytes past a 16-byte boundary runs the per-word kernel;
    its values equal the 16-byte-store kernel's bit for bit."""
    from eredu_amd import _native as n

    rows, cols = 7, 128
    wq, sc = random_mx(rows, cols, 31)
    w, s = dev_words(wq), dev_u8(sc)
    ref = dequantize_with_mode(w, s, None, 32, 4, MX, dtype=out)
    code = {torch.float32: n.EQ_DTYPE_F32, torch.bfloat16: n.EQ_DTYPE_BF16, torch.float16: n.EQ_DTYPE_F16}[out]
    buf = torch.zeros(rows * cols + 8, dtype=out, device="cuda")
    shifted = buf[1:1 + rows * cols]
    n.check(n.lib().eq_dequantize(shifted.data_ptr(), w.data_ptr(), s.data_ptr(), None, rows, cols, 32, 4, b"mxfp4",
                                  n.EQ_DTYPE_U8, code, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    got, exp = shifted.view(rows, cols), ref
    assert torch.equal(torch.isnan(got), torch.isnan(exp))
    ok = ~torch.isnan(exp)
    assert torch.equal(got[ok], exp[ok])


def test_dequantize_default_dtype_is_bf16(cuda):
    wq = torch.zeros((2, 4), dtype=torch.int32, device="cuda")
    sc = torch.full((2, 1), 127, dtype=torch.uint8, device="cuda")
    assert dequantize_with_mode(wq, sc, None, 32, 4, MX).dtype == torch.bfloat16


def test_reference_round_trip_and_matmul(cuda):
    weight = (torch.arange(-64, 64, dtype=torch.float32) / 16.0).reshape(2, 64).cuda()
    wq, s, b = quantize_with_mode(weight, 32, 4, MX)
    assert tuple(wq.shape) == (2, 8) and tuple(s.shape) == (2, 2) and b is None
    restored = dequantize_with_mode(wq, s, None, 32, 4, MX, dtype=torch.float32)
    assert float((weight - restored).abs().max()) <= 1.0
    x = torch.ones((3, 64), dtype=torch.float32, device="cuda")
    actual = quantized_matmul_with_mode(x, wq, s, None, True, 32, 4, MX)
    expected = x @ restored.T
    assert float((actual - expected).abs().max()) < 1e-3


def test_reference_gather_zero_codes(cuda):
    x = torch.ones((1, 1, 32), dtype=torch.float32, device="cuda")
    w = torch.zeros((1, 1, 4), dtype=torch.int32, device="cuda")
    s = torch.tensor([127], dtype=torch.uint8, device="cuda").reshape(1, 1, 1)
    idx = torch.tensor([0], dtype=torch.int32, device="cuda")
    y = gather_qmm_with_mode(x, w, s, None, idx, idx, True, 32, 4, True, MX)
    assert tuple(y.shape) == (1, 1, 1) and float(y.reshape(-1)[0]) == 0.0


def random_mx(rows, cols, seed):
    rng = np.random.default_rng(seed)
    wq = rng.integers(0, 2 ** 32, size=(rows, cols // 8), dtype=np.uint32)
    sc = rng.integers(120, 128, size=(rows, cols // 32)).astype(np.uint8)
    return wq, sc


def x_of(M, K, xdt, seed):
    xb = synthetic_x(M, K, seed)
    if xdt == orc.BF16:
        return xb, dev_bf16(xb)
    xf = orc.bf16_bits_to_f32(xb)
    host = xf.astype(np.float16).view(np.uint16) if xdt == orc.F16 else xf
    return host, dev_param(host, xdt)


MATMUL_CASES = [
    # (M, N, K, x dtype, transpose)
    (1, 4096, 4096, orc.BF16, True),     # the decode kernel
    (4, 1024, 2048, orc.BF16, True),     # decode kernel, four activation rows
    (5, 1000, 2048, orc.BF16, True),     # decode kernel, two passes (N % 128 != 0)
    (16, 512, 1024, orc.BF16, True),     # the MFMA qmm from M = 5 on
    (1, 300, 14336, orc.BF16, True),     # a long row: the decode kernel's single-row LDS case
    (37, 256, 512, orc.BF16, True),      # the MFMA qmm (N % 128 == 0, K % 64 == 0)
    (300, 1024, 2048, orc.BF16, True),   # MFMA qmm, K split over workgroups
    (130, 384, 4160, orc.BF16, True),    # MFMA qmm, ragged row tile, odd chunk count
    (37, 200, 512, orc.BF16, True),      # the general kernel (N % 128 != 0)
    (7, 258, 1024, orc.F32, True),
    (3, 130, 160, orc.F16, True),
    (1, 4096, 1024, orc.BF16, False),    # split-K VALU kernel (M <= 8, bf16)
    (8, 512, 2048, orc.BF16, False),
    (12, 256, 512, orc.BF16, False),     # 8-row launches plus the rest (M > 8)
    (9, 512, 256, orc.F32, False),       # the general kernel (f32 x)
    (4, 96, 64, orc.F16, False),
]


@pytest.mark.parametrize("M,N,K,xdt,transpose", MATMUL_CASES)
def test_matmul_matches_oracle(cuda, M, N, K, xdt, transpose):
    print(f"[case] mxfp4 matmul M={M} N={N} K={K} xdt={xdt} transpose={transpose}", flush=True)
    rows, cols = (N, K) if transpose else (K, N)
    wq, sc = random_mx(rows, cols, M * 7 + N + K)
    xh, xd = x_of(M, K, xdt, M + N)
    y = quantized_matmul_with_mode(xd, dev_words(wq), dev_u8(sc), None, transpose, 32, 4, MX)
    torch.cuda.synchronize()
    assert y.dtype == DT[xdt] and tuple(y.shape) == (M, N)
    ref = orc.mxfp4_matmul_f64(xh, xdt, wq, sc, transpose, N, K)
    ok, worst, rms = orc.matmul_within_tolerance(host_f32(y), ref, out_is_bf16=(xdt != orc.F32))
    assert ok, f"worst {worst:.3e} of RMS {rms:.3e}"


@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("sorted_hint", [False, True])
def test_gather_matches_oracle(cuda, transpose, sorted_hint):
    E, N, K, M, B = 4, 256, 512, 2, 6
    rows, cols = (N, K) if transpose else (K, N)
    banks = [random_mx(rows, cols, 50 + e) for e in range(E)]
    wq = np.stack([b[0] for b in banks])
    sc = np.stack([b[1] for b in banks])
    xb = synthetic_x(B * M, K, 9).reshape(B, M, K)
    lhs = np.arange(B, dtype=np.int32)
    rhs = np.array([0, 0, 1, 2, 3, 7] if sorted_hint else [3, 0, 2, 2, 1, 7], dtype=np.int32)  # 7: out of range
    y = gather_qmm_with_mode(dev_bf16(xb), dev_words(wq), dev_u8(sc), None, torch.from_numpy(lhs).cuda(),
                             torch.from_numpy(rhs).cuda(), transpose, 32, 4, sorted_hint, MX)
    torch.cuda.synchronize()
    got = host_f32(y)
    for b in range(B):
        if rhs[b] >= E:
            assert np.all(got[b] == 0.0)
            continue
        ref = orc.mxfp4_matmul_f64(xb[lhs[b]], orc.BF16, wq[rhs[b]], sc[rhs[b]], transpose, N, K)
        assert orc.matmul_within_tolerance(got[b], ref, True)[0], b


@pytest.mark.parametrize("B,E,sorted_hint", [(6, 4, False), (40, 4, True), (160, 8, True)])
def test_routed_decode_matches_oracle(cuda, B, E, sorted_hint):
    """One activation row per route (moe.rs:121-139): the per-route kernel, and
    for many sorted routes the grouped MFMA qmm (an out-of-range expert gives a
    zero row either way)."""
    print(f"[case] mxfp4 routed decode B={B} E={E} sorted={sorted_hint}", flush=True)
    N, K = 512, 1024
    banks = [random_mx(N, K, 60 + e) for e in range(E)]
    wq = np.stack([b[0] for b in banks])
    sc = np.stack([b[1] for b in banks])
    xb = synthetic_x(B, K, 19).reshape(B, 1, K)
    rng = np.random.default_rng(B)
    rhs = rng.integers(0, E, size=B).astype(np.int32)
    rhs[-1] = E + 3
    if sorted_hint:
        rhs = np.sort(rhs)
    lhs = np.arange(B, dtype=np.int32)
    y = gather_qmm_with_mode(dev_bf16(xb), dev_words(wq), dev_u8(sc), None, torch.from_numpy(lhs).cuda(),
                             torch.from_numpy(rhs).cuda(), True, 32, 4, sorted_hint, MX)
    torch.cuda.synchronize()
    got = host_f32(y)
    for b in range(B):
        if rhs[b] >= E:
            assert np.all(got[b] == 0.0), b
            continue
        ref = orc.mxfp4_matmul_f64(xb[b], orc.BF16, wq[rhs[b]], sc[rhs[b]], True, N, K)
        assert orc.matmul_within_tolerance(got[b], ref, True)[0], b


def test_batched_equals_single_calls(cuda):
    M = 3
    probs = []
    for i, (N, K) in enumerate([(512, 1024), (128, 1024), (256, 1024)]):
        wq, sc = random_mx(N, K, 80 + i)
        probs.append((dev_bf16(synthetic_x(M, K, 90 + i)), dev_words(wq), dev_u8(sc), None))
    outs = quantized_matmul_batched(probs, True, 32, 4, MX)
    for (x, w, s, _), y in zip(probs, outs):
        y1 = quantized_matmul_with_mode(x, w, s, None, True, 32, 4, MX)
        assert torch.equal(y.view(torch.int16), y1.view(torch.int16))


def test_mirror_rejects_bad_arguments(cuda):
    w = torch.zeros((4, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(EreduError, match="group_size=32 and bits=4"):
        quantize_with_mode(w, 64, 4, MX)
    with pytest.raises(EreduError, match="group_size=32 and bits=4"):
        quantize_with_mode(w, 32, 8, MX)
    wq, s, _ = quantize_with_mode(w, 32, 4, MX)
    x = torch.ones((1, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(EreduError, match="no biases"):
        quantized_matmul_with_mode(x, wq, s, torch.zeros_like(s, dtype=torch.float32), True, 32, 4, MX)
    with pytest.raises(EreduError, match="uint8"):
        quantized_matmul_with_mode(x, wq, s.float(), None, True, 32, 4, MX)


def test_gguf_golden_block(cuda):
    block = np.zeros(17, dtype=np.uint8)
    block[0] = 130
    for i in range(16):
        block[1 + i] = i | ((15 - i) << 4)
    for endian in (G.Endian.Little, G.Endian.Big):
        desc = G.TensorDescriptor("experts.weight", [32], G.GgmlType.MXFP4, 17)
        t = G.convert(desc, dev_u8(block), endian)
        assert isinstance(t, G.MxFp4Tensor)
        assert t.weight_shape == [4] and t.scale_shape == [1]
        assert t.scales.cpu().tolist() == [130]
        assert [int(v) for v in t.weights.cpu().numpy().view(np.uint32)] == [0x76543210, 0xFEDCBA98, 0x89ABCDEF,
                                                                             0x01234567]


def test_gguf_random_blocks(cuda):
    rng = np.random.default_rng(17)
    dims = [96, 5, 3]  # GGML order: MLX shape [3, 5, 96]
    rows, cols = 15, 96
    raw = rng.integers(0, 256, size=rows * cols // 32 * 17, dtype=np.uint8)
    raw[0::17] = rng.integers(100, 150, size=rows * cols // 32)  # finite scales
    desc = G.TensorDescriptor("blk.0.ffn_up_exps.weight", dims, G.GgmlType.MXFP4, raw.size)
    t = G.convert(desc, dev_u8(raw))
    assert t.weight_shape == [3, 5, 12] and t.scale_shape == [3, 5, 3]
    rw, rs = orc.mxfp4_convert_ggml(raw, rows, cols)
    assert np.array_equal(t.weights.reshape(rows, -1).cpu().numpy().view(np.uint32), rw)
    assert np.array_equal(t.scales.reshape(rows, -1).cpu().numpy(), rs)
    deq = t.dequantize(torch.float32)
    assert tuple(deq.shape) == (3, 5, 96)
    assert np.array_equal(deq.reshape(rows, cols).cpu().numpy().astype(np.float64),
                          orc.mxfp4_dequant_f64(rw, rs, rows, cols))
    with pytest.raises(EreduError, match="divisible by 32"):
        G.convert(G.TensorDescriptor("bad", [48], G.GgmlType.MXFP4, 17), dev_u8(raw[:17]))
    assert math.isfinite(float(deq.abs().max()))


def test_streamed_gguf_mxfp4_layer(cuda, tmp_path):
    """A type-39 tensor in a GGUF file streams to an MxFp4Tensor (both byte
    orders: single bytes), and a QuantizedLinear over it computes the MXFP4
    matmul (safemlx/src/ops/gguf.rs:498-525 hands MLX the same pair)."""
    from eredu_amd import QuantizedLinear
    from eredu_amd import gguf_file as F

    N, K = 256, 512
    rng = np.random.default_rng(23)
    raw = rng.integers(0, 256, size=N * K // 32 * 17, dtype=np.uint8)
    raw[0::17] = rng.integers(118, 128, size=N * K // 32)
    for endian in ("little", "big"):
        path = tmp_path / f"mx_{endian}.gguf"
        with open(path, "wb") as f:
            F.write_gguf(f, {}, [("blk.0.ffn_gate_exps.weight", [K, N], 39, raw.tobytes())], endian=endian)
        t = F.stream_convert(str(path), staging_bytes=4096)["blk.0.ffn_gate_exps.weight"]
        assert isinstance(t, G.MxFp4Tensor) and t.weight_shape == [N, K // 8] and t.scale_shape == [N, K // 32]
        rw, rs = orc.mxfp4_convert_ggml(raw, N, K)
        assert np.array_equal(t.weights.cpu().numpy().view(np.uint32), rw)
        layer = QuantizedLinear(t.weights, t.scales, None, 32, 4, mode=MX)
        xb = synthetic_x(3, K, 29)
        y = layer(dev_bf16(xb))
        ref = orc.mxfp4_matmul_f64(xb, orc.BF16, rw, rs, True, N, K)
        assert orc.matmul_within_tolerance(host_f32(y), ref, True)[0]
    with pytest.raises(EreduError, match="no device conversion"):
        F.stream_convert_affine(str(tmp_path / "mx_little.gguf"))


def test_quantized_embedding_mxfp4(cuda):
    """QuantizedEmbedding over an MXFP4 table (safemlx/src/nn/quantized.rs:
    359-435 with mode MxFp4): forward = the ids' rows dequantized (bf16,
    bit-exact against the oracle), as_linear = the MXFP4 matmul."""
    from eredu_amd import QuantizedEmbedding

    vocab, dim = 300, 256
    wq, sc = random_mx(vocab, dim, 71)
    emb = QuantizedEmbedding(dev_words(wq), dev_u8(sc), None, 32, 4, MX)
    ids = torch.tensor([[0, 299, 17], [17, 5, 128]], device="cuda")
    out = emb(ids)
    assert tuple(out.shape) == (2, 3, dim) and out.dtype == torch.bfloat16
    ref = orc.mxfp4_dequant_f64(wq, sc, vocab, dim)[ids.cpu().numpy().reshape(-1)]
    exp = torch.from_numpy(ref).to(torch.bfloat16).reshape(2, 3, dim)
    assert torch.equal(out.cpu().view(torch.int16), exp.view(torch.int16))
    xb = synthetic_x(2, dim, 72)
    y = emb.as_linear(dev_bf16(xb))
    yref = orc.mxfp4_matmul_f64(xb, orc.BF16, wq, sc, True, vocab, dim)
    assert orc.matmul_within_tolerance(host_f32(y), yref, True)[0]


def test_reference_mxfp4_modules_have_no_quantization_biases(cuda):
    """safemlx/src/nn/quantized.rs:906-939: an MXFP4 QuantizedLinear (64 -> 8,
    with a dense bias) and QuantizedEmbedding (16 x 64) built unloaded run
    and carry no quantization biases."""
    from eredu_amd import QuantizedEmbedding, QuantizedLinear

    linear = QuantizedLinear.unloaded_with_mode(64, 8, 32, 4, MX, bias=True)
    assert linear.biases is None and linear.bias is not None and linear.scales.dtype == torch.uint8
    out = linear(torch.ones((2, 64), dtype=torch.float32, device="cuda"))
    assert tuple(out.shape) == (2, 8)
    emb = QuantizedEmbedding.unloaded_with_mode(16, 64, 32, 4, MX)
    assert emb.biases is None
    tokens = torch.tensor([[0, 3], [7, 15]], dtype=torch.int32, device="cuda")
    assert tuple(emb(tokens).shape) == (2, 2, 64)

"""Pins the CPU oracle (oracle/eq_oracle.c, oracle/oracle.py) before it is
trusted as the checker of the HIP kernels.  CPU only.

What pins what:
* f16/bf16 rounding     -- numpy float16 and torch bfloat16 (independent RNE implementations).
* GGUF convert          -- the reference's golden vectors (mlx-v0.32.0.oracle rows 2, 8, 12),
                           byte-exact, and the boundary blocks of eredu-gguf/tests/oracle.rs:235-266.
* affine dequant        -- the fixture's MLX f16 dequantized column (exact after f16 rounding).
* native Q4_K / Q8_0    -- exact closed form in f64, the native-vs-affine tests of
                           native_quantization.rs:3867-3890,4042-4070, zero blocks decode to 0.
* quantized matmul      -- an independent pure-Python brute force on tiny shapes, special
                           cases (zero codes, one-hot x, transpose=false vs true), and the
                           reference test's contract (|y_q - x.dequant(w)| < 1e-3 at
                           M=32, N=K=128, g64 b4; ops/quantization.rs:562-604).
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests.fixtures import golden_rows, synthetic_blocks

ROWS = golden_rows()


# ----------------------------------------------------------------- floats

def test_f16_to_f32_all_patterns():
    L = orc.lib()
    pats = np.arange(65536, dtype=np.uint16)
    ref = pats.view(np.float16).astype(np.float32)
    got = np.array([L.or_f16_to_f32(int(p)) for p in pats], dtype=np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(1)
    # random bit patterns across the whole range, f16 halfway points and subnormal territory
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[~np.isnan(vals)]
    halfway = (np.arange(0, 65535, 7, dtype=np.uint16).view(np.float16).astype(np.float64))
    halfway = (halfway[:-1] + halfway[1:]) / 2
    halfway = halfway[np.isfinite(halfway)].astype(np.float32)
    tiny = (rng.random(50_000) * 2.0 ** -14).astype(np.float32) * rng.choice([-1, 1], 50_000)
    x = np.concatenate([vals, halfway, tiny, np.array([65504, 65520, 65519.99, -65520, 1e30, 0.0, -0.0], np.float32)])
    got = orc.f32_to_f16_bits_c(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_bf16_matches_torch():
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2**32, size=500_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16_bits(x), ref)
    L = orc.lib()
    assert all(L.or_f32_to_bf16(float(v)) == int(r) for v, r in zip(x[:2000], ref[:2000]))


# ------------------------------------------------------------ GGUF convert

@pytest.mark.parametrize("code", [orc.Q4_0, orc.Q8_0, orc.Q4_K])
def test_convert_affine_matches_golden_byte_for_byte(code):
    row = ROWS[code]
    raw = np.frombuffer(row["raw"], dtype=np.uint8)
    w, s, b = orc.gguf_convert_affine(code, raw)
    assert w.tobytes() == row["weight"], "weights"
    assert s.tobytes() == row["scales"], "scales"
    assert b.tobytes() == row["biases"], "biases"
    bits, gs = orc.AFFINE_CONFIG[code]
    values, _ = orc.BLOCK_GEOMETRY[code]
    assert row["weight_name"] == f"oracle.weight:[2, {values * bits // 32}]"
    assert row["scales_name"] == f"oracle.scales:[2, {values // gs}]"


@pytest.mark.parametrize("code", [orc.Q4_0, orc.Q8_0, orc.Q4_K])
def test_affine_dequant_matches_golden_f16_exactly(code):
    row = ROWS[code]
    raw = np.frombuffer(row["raw"], dtype=np.uint8)
    f32 = orc.gguf_dequant_f32(code, raw, definition=0)
    expected = np.frombuffer(row["dequantized"], dtype=np.uint16).view(np.float16).astype(np.float32)
    assert f32.size == expected.size
    # the reference test allows 4 f16 ulps (oracle.rs:105-110); the restatement is exact
    assert np.array_equal(f32.astype(np.float16).astype(np.float32), expected)


def test_boundary_blocks_extreme_codes():
    # eredu-gguf/tests/oracle.rs:235-266: all-0xff quants, f16 one as the scale
    one = np.float16(1.0).view(np.uint16)
    q40 = np.full(18, 0xFF, np.uint8)
    q40[0:2] = np.frombuffer(one.tobytes(), np.uint8)
    w, _, _ = orc.gguf_convert_affine(orc.Q4_0, q40)
    assert (w == 0xFFFFFFFF).all()
    q80 = np.full(34, 0xFF, np.uint8)
    q80[0:2] = np.frombuffer(one.tobytes(), np.uint8)
    w, _, _ = orc.gguf_convert_affine(orc.Q8_0, q80)
    assert (w == 0x7F7F7F7F).all()
    assert orc.gguf_dequant_f32(orc.Q4_0, q40).size == 32
    assert orc.gguf_dequant_f32(orc.Q8_0, q80).size == 32


@pytest.mark.parametrize("code", [orc.Q8_0, orc.Q4_K])
def test_zero_blocks_decode_to_zero(code):
    # eredu-gguf/tests/iquant.rs:143-156
    _, nbytes = orc.BLOCK_GEOMETRY[code]
    z = np.zeros(nbytes, np.uint8)
    for definition in (0, 1):
        assert (orc.gguf_dequant_f32(code, z, definition) == 0).all()


def _q4k_sample_block():
    # safemlx/src/native_quantization.rs:3780-3791 sample_block
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    b[4:16] = [(i * 17 + 3) & 0xFF for i in range(12)]
    b[16:] = [(i * 29 + 11) & 0xFF for i in range(128)]
    return b


def _q8_0_sample_block():
    # native_quantization.rs:3804-3811
    b = np.zeros(34, np.uint8)
    b[0:2] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
    b[2:] = [((np.int8(i).astype(np.int32) * 11 - 97) & 0xFF) for i in range(32)]
    return b


def test_native_matches_affine_on_reference_sample_blocks():
    # native_quantization.rs:3867-3890 and :4042-4070: |native - affine| <= 1e-6
    for code, blk in ((orc.Q4_K, _q4k_sample_block()), (orc.Q8_0, np.tile(_q8_0_sample_block(), 2))):
        nat = orc.gguf_dequant_f32(code, blk, definition=1)
        aff = orc.gguf_dequant_f32(code, blk, definition=0)
        assert np.max(np.abs(nat - aff)) <= 1e-6


def _q4k_closed_form_f64(raw):
    """Exact w = d*sc*q - dmin*m (products exact; f64 holds the difference exactly
    for the magnitudes drawn here), then one rounding to f32."""
    out = []
    for blk in raw.reshape(-1, 144):
        d = float(blk[0:2].view(np.float16)[0])
        dm = float(blk[2:4].view(np.float16)[0])
        s = [int(v) for v in blk[4:16]]
        for g in range(8):
            if g < 4:
                sc, m = s[g] & 63, s[g + 4] & 63
            else:
                sc = (s[g + 4] & 15) | ((s[g - 4] >> 6) << 4)
                m = (s[g + 4] >> 4) | ((s[g] >> 6) << 4)
            for i in range(32):
                p = int(blk[16 + (g // 2) * 32 + i])
                q = (p & 15) if g % 2 == 0 else (p >> 4)
                out.append(d * sc * q - dm * m)
    return np.array(out, dtype=np.float64).astype(np.float32)


def test_native_q4k_closed_form():
    raw = synthetic_blocks(orc.Q4_K, 24, seed=5)
    assert np.array_equal(orc.gguf_dequant_f32(orc.Q4_K, raw, definition=1), _q4k_closed_form_f64(raw))


def test_native_q8_0_closed_form():
    raw = synthetic_blocks(orc.Q8_0, 64, seed=6).reshape(-1, 34)
    d = raw[:, 0:2].copy().view(np.float16).astype(np.float64)
    q = raw[:, 2:].view(np.int8).astype(np.float64)
    expect = (d * q).astype(np.float32).reshape(-1)
    assert np.array_equal(orc.gguf_dequant_f32(orc.Q8_0, raw.reshape(-1), definition=1), expect)


def test_q4k_affine_route_closed_form():
    # scale = f16(d*sc), bias = f16(-dmin*m), w = f32(scale)*q + f32(bias) in f32
    raw = synthetic_blocks(orc.Q4_K, 16, seed=7)
    w, s, b = orc.gguf_convert_affine(orc.Q4_K, raw)
    q = orc.unpack_codes(w.reshape(-1, 32), 256, 4).reshape(-1, 8, 32).astype(np.float32)
    sf = s.view(np.float16).astype(np.float32).reshape(-1, 8, 1)
    bf = b.view(np.float16).astype(np.float32).reshape(-1, 8, 1)
    expect = (sf * q + bf).reshape(-1)  # numpy: one f32 multiply, one f32 add
    assert np.array_equal(orc.gguf_dequant_f32(orc.Q4_K, raw, definition=0), expect)
    # and the affine/native routes differ somewhere under the config-4 distribution (F4)
    raw = synthetic_blocks(orc.Q4_K, 2048, seed=8)
    a = orc.gguf_dequant_bf16(orc.Q4_K, raw, 0)
    n = orc.gguf_dequant_bf16(orc.Q4_K, raw, 1)
    assert (a != n).mean() > 0.01


def test_big_endian_fields_are_swapped():
    raw = synthetic_blocks(orc.Q4_K, 4, seed=9).reshape(-1, 144)
    be = raw.copy()
    be[:, [0, 1, 2, 3]] = raw[:, [1, 0, 3, 2]]
    le_out = orc.gguf_convert_affine(orc.Q4_K, raw.reshape(-1))
    be_out = orc.gguf_convert_affine(orc.Q4_K, be.reshape(-1), big_endian=True)
    for a, b in zip(le_out, be_out):
        assert np.array_equal(a, b)


# ------------------------------------------------------------ affine matmul

def _brute_qmm(x, w, s, b, gs, bits, N, K):
    """Pure-Python brute force: y[m][n] = sum_k x*(s*q + b), codes via Python ints."""
    M = x.shape[0]
    y = [[0.0] * N for _ in range(M)]
    for n in range(N):
        words = [int(v) for v in w[n]]
        bitstream = sum(v << (32 * i) for i, v in enumerate(words))
        for m in range(M):
            acc = 0.0
            for k in range(K):
                q = (bitstream >> (k * bits)) & ((1 << bits) - 1)
                acc += float(x[m][k]) * (float(s[n][k // gs]) * q + float(b[n][k // gs]))
            y[m][n] = acc
    return np.array(y)


@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 64), (4, 32), (2, 32), (8, 128)])
def test_matmul_oracle_against_brute_force(bits, gs):
    rng = np.random.default_rng(bits * 100 + gs)
    N, K, M = 6, 2 * gs, 3
    w = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = rng.normal(0, 0.05, size=(N, K // gs)).astype(np.float32)
    b = rng.normal(0, 0.05, size=(N, K // gs)).astype(np.float32)
    x = rng.normal(size=(M, K)).astype(np.float32)
    y = orc.quantized_matmul_f64(x, orc.F32, w, s, b, orc.F32, True, gs, bits, N, K)
    yb = _brute_qmm(x, w, s, b, gs, bits, N, K)
    assert np.allclose(y, yb, rtol=1e-12, atol=1e-12)
    y32 = orc.qmm_t_f32(x, orc.F32, w, s, b, orc.F32, M, N, K, gs, bits)
    # f32 accumulation: |error| <= K * eps32 * sum_k |x_k w_k|
    W = orc.affine_dequant_f64(w, s, b, orc.F32, N, K, gs, bits)
    bound = K * 2.0 ** -24 * (np.abs(x.astype(np.float64)) @ np.abs(W).T)
    assert np.all(np.abs(y32 - yb) <= bound)


def test_matmul_oracle_special_cases():
    rng = np.random.default_rng(11)
    N, K, gs, bits = 8, 128, 64, 4
    s = rng.normal(0, 0.05, size=(N, K // gs)).astype(np.float32)
    b = rng.normal(0, 0.05, size=(N, K // gs)).astype(np.float32)
    x = rng.normal(size=(2, K)).astype(np.float32)
    # all-zero codes: y = sum_g b_g * sum_{k in g} x_k
    w0 = np.zeros((N, K * bits // 32), np.uint32)
    y = orc.quantized_matmul_f64(x, orc.F32, w0, s, b, orc.F32, True, gs, bits, N, K)
    xs = x.astype(np.float64).reshape(2, K // gs, gs).sum(-1)
    assert np.allclose(y, xs @ b.astype(np.float64).T, rtol=1e-12)
    # one-hot x selects a dequantized column
    w = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    W = orc.affine_dequant_f64(w, s, b, orc.F32, N, K, gs, bits)
    e = np.zeros((1, K), np.float32)
    e[0, 77] = 1.0
    assert np.array_equal(orc.quantized_matmul_f64(e, orc.F32, w, s, b, orc.F32, True, gs, bits, N, K)[0], W[:, 77])
    # transpose=false on the transposed pack equals transpose=true
    Wt_codes = orc.unpack_codes(w, K, bits).T  # [K, N] codes
    Ntp = N  # pack along N: needs N % gs == 0 -> use gs=8? keep gs dividing N
    gs_t = 8
    st = rng.normal(0, 0.05, size=(K, Ntp // gs_t)).astype(np.float32)
    bt = rng.normal(0, 0.05, size=(K, Ntp // gs_t)).astype(np.float32)
    packed = np.zeros((K, Ntp * bits // 32), np.uint32)
    for c in range(Ntp):
        packed[:, c * bits // 32] |= (Wt_codes[:, c].astype(np.uint32) << np.uint32((c * bits) % 32))
    y_n = orc.quantized_matmul_f64(x, orc.F32, packed, st, bt, orc.F32, False, gs_t, bits, Ntp, K)
    # same weights expressed in [N, K] layout with per-element scales
    Wn = orc.affine_dequant_f64(packed, st, bt, orc.F32, K, Ntp, gs_t, bits)  # [K, N]
    assert np.allclose(y_n, x.astype(np.float64) @ Wn, rtol=1e-12)
    assert np.allclose(Wn.T, Wt_codes.T * np.repeat(st, gs_t, axis=1).T + np.repeat(bt, gs_t, axis=1).T)


def test_reference_quantized_matmul_contract():
    # safemlx/src/ops/quantization.rs:562-604: M=32, N=K=128, g64 b4, x,w ~ N(0,1)/sqrt(K)
    rng = np.random.default_rng(0)
    M, N, K, gs, bits = 32, 128, 128, 64, 4
    scale = 1.0 / math.sqrt(K)
    x = (rng.normal(size=(M, K)) * scale).astype(np.float32)
    W = (rng.normal(size=(N, K)) * scale).astype(np.float32)
    wq, s, b = orc.quantize_affine(W, gs, bits, orc.F32)
    w_hat = orc.affine_dequant_f32(wq, s, b, orc.F32, N, K, gs, bits)
    y_q = orc.qmm_t_f32(x, orc.F32, wq, s, b, orc.F32, M, N, K, gs, bits)
    assert np.max(np.abs(y_q - x @ w_hat.T)) < 1e-3


def test_quantize_dequantize_bound():
    # safemlx/src/ops/quantization.rs:457-486: x = outer(ones[128], arange(512)), gs 128
    x = np.outer(np.ones(128), np.arange(512)).astype(np.float32)
    for bits in (2, 4, 8):
        wq, s, b = orc.quantize_affine(x, 128, bits, orc.F32)
        assert wq.shape == (128, 512 * bits // 32) and s.shape == (128, 4)
        xh = orc.affine_dequant_f32(wq, s, b, orc.F32, 128, 512, 128, bits)
        assert np.max(np.abs(x - xh)) <= 127.0 / (1 << bits)


def test_tolerance_rule_rejects_planted_errors():
    # a dropped group, a sign flip and a transposed operand must all fail the parity rule
    rng = np.random.default_rng(3)
    N, K, gs, bits = 64, 256, 64, 4
    w = rng.integers(0, 2**32, size=(N, K * bits // 32), dtype=np.uint64).astype(np.uint32)
    s = orc.f32_to_bf16_bits(rng.normal(0, 0.01, size=(N, K // gs)).astype(np.float32))
    b = orc.f32_to_bf16_bits(rng.normal(0, 0.05, size=(N, K // gs)).astype(np.float32))
    x = orc.f32_to_bf16_bits(rng.normal(size=(2, K)).astype(np.float32))
    y = orc.quantized_matmul_f64(x, orc.BF16, w, s, b, orc.BF16, True, gs, bits, N, K)
    ok, _, _ = orc.matmul_within_tolerance(y, y, out_is_bf16=True)
    assert ok
    s_drop = s.copy()
    s_drop[:, 1] = 0
    b_drop = b.copy()
    b_drop[:, 1] = 0
    y_drop = orc.quantized_matmul_f64(x, orc.BF16, w, s_drop, b_drop, orc.BF16, True, gs, bits, N, K)
    assert not orc.matmul_within_tolerance(y_drop, y, True)[0]
    assert not orc.matmul_within_tolerance(-y, y, True)[0]
    x_rev = x[:, ::-1].copy()
    y_rev = orc.quantized_matmul_f64(x_rev, orc.BF16, w, s, b, orc.BF16, True, gs, bits, N, K)
    assert not orc.matmul_within_tolerance(y_rev, y, True)[0]


def _pack_bitstream(codes: np.ndarray, bits: int) -> np.ndarray:
    """Rows of codes as one Python integer each, code i at bit i * bits
    (eredu-gguf/src/convert.rs:413-427: LSB-first, a code may straddle two
    words), cut into 32-bit words."""
    rows, cols = codes.shape
    words = cols * bits // 32
    out = np.zeros((rows, words), dtype=np.uint32)
    for r in range(rows):
        stream = 0
        for i, c in enumerate(codes[r]):
            stream |= int(c) << (i * bits)
        for j in range(words):
            out[r, j] = (stream >> (32 * j)) & 0xFFFFFFFF
    return out


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_unpack_matches_the_reference_bit_stream(bits):
    """Both oracle unpackers (numpy and C) read the reference packer's bit
    stream back, including 3-, 5- and 6-bit codes that straddle words."""
    rng = np.random.default_rng(bits)
    rows, cols = 3, 96
    codes = rng.integers(0, 1 << bits, size=(rows, cols), dtype=np.uint32)
    codes[0, :] = (1 << bits) - 1  # all ones: every straddling bit is set
    w = _pack_bitstream(codes, bits)
    assert np.array_equal(orc.unpack_codes(w, cols, bits), codes)
    ones = np.ones((rows, cols // 16), dtype=np.float32)
    zeros = np.zeros_like(ones)
    assert np.array_equal(orc.affine_dequant_f32(w, ones, zeros, orc.F32, rows, cols, 16, bits),
                          codes.astype(np.float32))


@pytest.mark.parametrize("bits", [3, 5, 6])
@pytest.mark.parametrize("gs", [16, 32])
def test_quantize_odd_widths_round_trip(bits, gs):
    """The oracle quantizer at 3/5/6 bits packs a stream the reference's
    packer would produce from its codes, and meets the round-trip bound."""
    rng = np.random.default_rng(bits * 100 + gs)
    rows, cols = 5, 96
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    wq, s, b = orc.quantize_affine(w, gs, bits, orc.F32)
    assert wq.shape == (rows, cols * bits // 32)
    codes = orc.unpack_codes(wq, cols, bits)
    assert np.array_equal(_pack_bitstream(codes, bits), wq)
    w_hat = orc.affine_dequant_f32(wq, s, b, orc.F32, rows, cols, gs, bits)
    # MLX's edge rule: the group's larger-magnitude extreme is the bias and
    # dequantizes exactly; the opposite extreme may clamp, so the bound is one
    # step rather than half of one
    g = w.reshape(rows, cols // gs, gs)
    mn, mx = g.min(axis=2), g.max(axis=2)
    edge = np.where(np.abs(mn) > np.abs(mx), mn, mx)
    assert np.array_equal(b, edge)
    at_edge = g == edge[:, :, None]
    assert np.array_equal(w_hat.reshape(g.shape)[at_edge], g[at_edge])
    step = np.repeat(np.abs(s), gs, axis=1)
    assert np.all(np.abs(w_hat - w) <= step * (1 + 1e-5))

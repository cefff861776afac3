"""Pins of the oracle's MXFP4 functions (CPU).

* e2m1_decode: the table against the E2M1 bit fields (OCP Microscaling
  Formats v1.0: sign, 2 exponent bits with bias 1, 1 mantissa bit, exponent
  0 subnormal), decoded here field by field.
* e8m0_decode: the reference's decode test (eredu/src/backend/mlx/nn/fp8.rs:
  1670-1678: bytes 127, 128, 126 -> 1, 2, 0.5), 2^(e - 127) by repeated
  doubling, 255 -> NaN.
* mxfp4_convert_ggml: the golden block of eredu-gguf/tests/mxfp4.rs:5-60
  (scale 130, code bytes index | (15 - index) << 4 -> words 0x76543210,
  0xfedcba98, 0x89abcdef, 0x01234567), and per-nibble bookkeeping on random
  blocks.
* mxfp4_quantize: brute force on small groups (every exponent tried, every
  grid value tried, written as loops), ties to even, saturation never
  needed, the reference's round-trip bound (safemlx/src/ops/quantization.rs:
  488-549: arange(-64, 64) / 16 as [2, 64] -> weights [2, 8], scales [2, 2],
  max error <= 1), and dequantize(quantize(dequantize(q))) == dequantize(q)
  (idempotence up to the sign of zero).
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc


def test_e2m1_table_from_bit_fields():
    for code in range(16):
        sign = -1.0 if code & 8 else 1.0
        exp, man = (code >> 1) & 3, code & 1
        mag = (man / 2.0) if exp == 0 else (1.0 + man / 2.0) * 2.0 ** (exp - 1)
        got = float(orc.e2m1_decode(np.array([code]))[0])
        assert got == sign * mag, code


def test_e8m0_decode():
    assert list(orc.e8m0_decode(np.array([127, 128, 126]))) == [1.0, 2.0, 0.5]
    v = 1.0
    for e in range(127, 255):
        assert orc.e8m0_decode(np.array([e]))[0] == v
        v *= 2.0
    v = 1.0
    for e in range(127, -1, -1):
        assert orc.e8m0_decode(np.array([e]))[0] == v
        v /= 2.0
    assert math.isnan(orc.e8m0_decode(np.array([255]))[0])


def test_convert_golden_block():
    block = np.zeros(17, dtype=np.uint8)
    block[0] = 130
    for i in range(16):
        block[1 + i] = i | ((15 - i) << 4)
    assert list(block[1:]) == [0xF0, 0xE1, 0xD2, 0xC3, 0xB4, 0xA5, 0x96, 0x87, 0x78, 0x69, 0x5A, 0x4B, 0x3C,
                               0x2D, 0x1E, 0x0F]
    w, s = orc.mxfp4_convert_ggml(block, 1, 32)
    assert w.shape == (1, 4) and s.shape == (1, 1)
    assert list(s.reshape(-1)) == [130]
    assert [int(v) for v in w.reshape(-1)] == [0x76543210, 0xFEDCBA98, 0x89ABCDEF, 0x01234567]


def test_convert_random_blocks_nibble_by_nibble():
    rng = np.random.default_rng(7)
    rows, cols = 3, 96
    raw = rng.integers(0, 256, size=rows * cols // 32 * 17, dtype=np.uint8)
    w, s = orc.mxfp4_convert_ggml(raw, rows, cols)
    blocks = raw.reshape(-1, 17)
    codes = orc.unpack_codes(w, cols, 4).reshape(-1, 32)
    for b in range(blocks.shape[0]):
        assert s.reshape(-1)[b] == blocks[b, 0]
        for j in range(16):
            assert codes[b, j] == blocks[b, 1 + j] & 15
            assert codes[b, 16 + j] == blocks[b, 1 + j] >> 4


def _brute_group(vals):
    """Loops over exponents and grid values (float64)."""
    if not all(math.isfinite(v) for v in vals):
        return 255, [8 if v < 0 else 0 for v in vals]
    amax = max(abs(v) for v in vals)
    if amax == 0:
        return 0, [8 if v < 0 else 0 for v in vals]
    e = -127
    while amax > 6.0 * 2.0 ** e:
        e += 1
    grid = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    codes = []
    for v in vals:
        a = abs(v) / 2.0 ** e
        best = None
        for m, gv in enumerate(grid):
            d = abs(a - gv)
            if best is None or d < best[0] or (d == best[0] and m % 2 == 0 and best[1] % 2 == 1):
                best = (d, m)
        codes.append(best[1] | (8 if v < 0 else 0))
    return e + 127, codes


def test_quantize_matches_brute_force():
    rng = np.random.default_rng(3)
    rows = 6
    w = (rng.standard_normal((rows, 64)) * np.array([1e-3, 0.02, 1.0, 30.0, 1e-30, 1e30])[:, None]).astype(np.float32)
    w[0, :32] = 0.0
    w[1, 5] = -0.0
    w[2, :8] = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0], dtype=np.float32)  # ties at scale 1
    w[2, 8] = -6.0
    w[3, 40] = np.inf
    w[4, 3] = np.nan
    wq, sq = orc.mxfp4_quantize(w)
    codes = orc.unpack_codes(wq, 64, 4)
    for r in range(rows):
        for g in range(2):
            sb, c = _brute_group([float(v) for v in w[r, 32 * g:32 * g + 32]])
            assert sq[r, g] == sb, (r, g)
            assert list(codes[r, 32 * g:32 * g + 32]) == c, (r, g)
    # the ties: 0.25 -> 0, 0.75 -> 1, 1.25 -> 1, 1.75 -> 2, 2.5 -> 2, 3.5 -> 4, 5 -> 4, 6 -> 6
    assert sq[2, 0] == 127
    assert list(orc.e2m1_decode(codes[2, :8])) == [0.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0, 6.0]


def test_reference_round_trip_bound_and_idempotence():
    w = (np.arange(-64, 64, dtype=np.float32) / 16.0).reshape(2, 64)
    wq, sq = orc.mxfp4_quantize(w)
    assert wq.shape == (2, 8) and sq.shape == (2, 2)
    restored = orc.mxfp4_dequant_f64(wq, sq, 2, 64)
    assert np.abs(w - restored).max() <= 1.0
    wq2, sq2 = orc.mxfp4_quantize(restored.astype(np.float32))
    # idempotent up to the sign of zero (a -0 code dequantizes to -0.0, which is not < 0)
    assert np.array_equal(sq, sq2)
    assert np.array_equal(orc.mxfp4_dequant_f64(wq2, sq2, 2, 64), restored)
    # y = ones [3, 64] @ restored^T (the reference's matmul check, here on the oracle's own closed form)
    y = orc.mxfp4_matmul_f64(np.ones((3, 64), dtype=np.float32), orc.F32, wq, sq, True, 2, 64)
    assert np.allclose(y, np.ones((3, 64)) @ restored.T)


@pytest.mark.parametrize("transpose", [True, False])
def test_matmul_matches_dense_product(transpose):
    rng = np.random.default_rng(11)
    rows, cols = 8, 96
    wq, sq = orc.mxfp4_quantize(rng.standard_normal((rows, cols)).astype(np.float32))
    dense = orc.mxfp4_dequant_f64(wq, sq, rows, cols)
    if transpose:
        x = rng.standard_normal((5, cols)).astype(np.float32)
        y = orc.mxfp4_matmul_f64(x, orc.F32, wq, sq, True, rows, cols)
        ref = np.array([[sum(float(x[i, k]) * dense[n, k] for k in range(cols)) for n in range(rows)]
                        for i in range(5)])
    else:
        x = rng.standard_normal((5, rows)).astype(np.float32)
        y = orc.mxfp4_matmul_f64(x, orc.F32, wq, sq, False, cols, rows)
        ref = np.array([[sum(float(x[i, k]) * dense[k, n] for k in range(rows)) for n in range(cols)]
                        for i in range(5)])
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12)

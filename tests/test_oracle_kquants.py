"""Pins the C oracle's conversion of the GGML block types beyond Q4_0 / Q8_0 /
Q4_K: Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K and Q6_K (eredu-gguf/src/convert.rs:
362-373, 439-564).  CPU only.

What pins what:
* weights / scales / biases -- the reference's golden rows 3, 10, 11, 13, 14
  of mlx-v0.32.0.oracle, byte for byte (eredu-gguf/tests/oracle.rs:26-128).
* affine dequant            -- the rows' MLX f16 "dequantized" column: exact
  after f16 rounding for Q4_1 / Q2_K / Q3_K / Q5_K, within the reference
  test's tolerance for Q6_K, and exactly equal (all five rows) to f16
  arithmetic that rounds the multiply and the add separately, which is what
  MLX's f16 kernel does.
* Q5_0 / Q5_1               -- golden rows 6 / 7 (f16 dequant, exact) and the
  reference's repack tests (eredu-gguf/tests/oracle.rs:130-234).
* all seven types           -- an independent closed form written from ggml's
  published block decoders (dequantize_row_q4_1 / q5_0 / q5_1 / q2_K / q3_K /
  q5_K / q6_K of ggml-quants.c: signed codes and per-group factors laid out
  the way ggml describes them, not the way convert.rs re-packs them): equal in
  f32 for the 32-value types, within the f16 rounding of the affine scale and
  bias for the super-block types.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.fixtures import KQUANT_HEADERS, golden_rows, synthetic_blocks

ROWS = golden_rows()
NEW = (orc.Q4_1, orc.Q5_0, orc.Q5_1, orc.Q2_K, orc.Q3_K, orc.Q5_K, orc.Q6_K)
GOLDEN_AFFINE = (orc.Q4_1, orc.Q2_K, orc.Q3_K, orc.Q5_K, orc.Q6_K)


def _f16(raw, off):
    return raw[:, off:off + 2].copy().view(np.float16).astype(np.float64)[:, 0]


# ---------------------------------------------------------------- golden rows

@pytest.mark.parametrize("code", GOLDEN_AFFINE)
def test_convert_affine_matches_golden_byte_for_byte(code):
    row = ROWS[code]
    w, s, b = orc.gguf_convert_affine(code, np.frombuffer(row["raw"], dtype=np.uint8))
    assert w.tobytes() == row["weight"], "weights"
    assert s.tobytes() == row["scales"], "scales"
    assert b.tobytes() == row["biases"], "biases"
    bits, gs = orc.AFFINE_CONFIG[code]
    values, _ = orc.BLOCK_GEOMETRY[code]
    assert row["weight_name"] == f"oracle.weight:[2, {values * bits // 32}]"
    assert row["scales_name"] == f"oracle.scales:[2, {values // gs}]"


@pytest.mark.parametrize("code", GOLDEN_AFFINE)
def test_affine_dequant_matches_golden(code):
    row = ROWS[code]
    raw = np.frombuffer(row["raw"], dtype=np.uint8)
    expected = np.frombuffer(row["dequantized"], dtype=np.uint16).view(np.float16)
    got = orc.gguf_dequant_f32(code, raw, definition=0).astype(np.float16).astype(np.float32)
    e32 = expected.astype(np.float32)
    # eredu-gguf/tests/oracle.rs:103-113: four f16 ulps at the fixture's magnitudes
    assert (np.abs(got - e32) <= np.maximum(4.0, np.abs(e32) * 0.002)).all()
    if code != orc.Q6_K:
        assert np.array_equal(got, e32)
    # MLX's f16 kernel: f16(f16(scale * code) + bias), each step rounded
    w, s, b = orc.gguf_convert_affine(code, raw)
    bits, gs = orc.AFFINE_CONFIG[code]
    values, _ = orc.BLOCK_GEOMETRY[code]
    q = orc.unpack_codes(w.reshape(2, -1), values, bits).reshape(-1).astype(np.float16)
    sc = np.repeat(s.view(np.float16), gs)
    bi = np.repeat(b.view(np.float16), gs)
    assert np.array_equal((sc * q).astype(np.float16) + bi, expected)


@pytest.mark.parametrize("code", [orc.Q5_0, orc.Q5_1])
def test_q5_dequant_matches_golden_f16_exactly(code):
    # oracle.rs:54-75: legacy Q5 rows hold only the f16 dequantized weight
    row = ROWS[code]
    raw = np.frombuffer(row["raw"], dtype=np.uint8)
    expected = np.frombuffer(row["weight"], dtype=np.uint16).view(np.float16).astype(np.float32)
    assert row["weight_name"] == "oracle.weight:[2, 32]"
    got = orc.gguf_dequant_f32(code, raw, definition=0)
    assert np.array_equal(got.astype(np.float16).astype(np.float32), expected)


# --------------------------------------------------- reference repack tests

def _q5_block(code, scale, bias, codes):
    """oracle.rs:130-148 q5_block: codes (32 values < 32) into one Q5_0/Q5_1 block."""
    q50 = code == orc.Q5_0
    blk = np.zeros(22 if q50 else 24, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(scale).tobytes(), np.uint8)
    if not q50:
        blk[2:4] = np.frombuffer(np.float16(bias).tobytes(), np.uint8)
    qh_off, qs_off = (2, 6) if q50 else (4, 8)
    qh = 0
    for j in range(16):
        qh |= (codes[j] >> 4) << j
        qh |= (codes[j + 16] >> 4) << (j + 16)
        blk[qs_off + j] = (codes[j] & 15) | ((codes[j + 16] & 15) << 4)
    blk[qh_off:qh_off + 4] = np.frombuffer(np.uint32(qh).tobytes(), np.uint8)
    return blk


@pytest.mark.parametrize("code,scales,biases", [(orc.Q5_0, (0.5, -1.25), (0.0, 0.0)),
                                                (orc.Q5_1, (0.25, 1.75), (1.5, -0.75))])
def test_q5_repacking_preserves_values_and_gguf_bit_order(code, scales, biases):
    # oracle.rs:185-234 assert_q5_repacked
    codes = [[i for i in range(32)], [(i * 13 + 7) & 31 for i in range(32)]]
    raw = np.concatenate([_q5_block(code, scales[i], biases[i], codes[i]) for i in range(2)])
    w, s, b = orc.gguf_convert_affine(code, raw)
    assert w.size == 10 and s.size == 2 and b.size == 2
    assert orc.unpack_codes(w.reshape(1, 10), 64, 5).reshape(-1).tolist() == codes[0] + codes[1]
    got = orc.gguf_dequant_f32(code, raw, definition=0)
    for blk in range(2):
        d, m = float(np.float16(scales[blk])), float(np.float16(biases[blk]))
        for i, c in enumerate(codes[blk]):
            want = np.float32(d * (c - 16)) if code == orc.Q5_0 else np.float32(np.float32(d * c) + np.float32(m))
            assert got[blk * 32 + i] == want, (blk, i)


# ------------------------------------------------ ggml closed forms (f64)

def _q4_1_closed(raw):
    raw = raw.reshape(-1, 20)
    d, m = _f16(raw, 0), _f16(raw, 2)
    q = np.concatenate([raw[:, 4:20] & 15, raw[:, 4:20] >> 4], axis=1).astype(np.float64)
    return d[:, None] * q + m[:, None]


def _q5_closed(raw, q50):
    raw = raw.reshape(-1, 22 if q50 else 24)
    d = _f16(raw, 0)
    qh_off, qs_off = (2, 6) if q50 else (4, 8)
    qh = raw[:, qh_off:qh_off + 4].copy().view("<u4")[:, 0].astype(np.int64)
    bit = (qh[:, None] >> np.arange(32)) & 1
    qs = raw[:, qs_off:qs_off + 16].astype(np.int64)
    q = np.concatenate([qs & 15, qs >> 4], axis=1) | (bit << 4)
    if q50:
        return d[:, None] * (q - 16)
    return d[:, None] * q + _f16(raw, 2)[:, None]


def _scale_min_k4(s, j):
    """ggml get_scale_min_k4 over a [n, 12] byte array."""
    s = s.astype(np.int64)
    if j < 4:
        return s[:, j] & 63, s[:, j + 4] & 63
    return (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4), (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)


def _q2k_closed(raw):
    """dequantize_row_q2_K: per 128-value half, 4 shifts x 2 runs of 16; returns
    (y, |dl|, |ml|) per value."""
    raw = raw.reshape(-1, 84)
    n = raw.shape[0]
    d, dm = _f16(raw, 80), _f16(raw, 82)
    y, dl_all, ml_all = (np.zeros((n, 256)) for _ in range(3))
    for half in range(2):
        q = raw[:, 16 + 32 * half:16 + 32 * half + 32].astype(np.int64)
        for j in range(4):
            for t in range(2):
                sc = raw[:, half * 8 + 2 * j + t].astype(np.int64)
                dl, ml = d * (sc & 15), dm * (sc >> 4)
                v0 = half * 128 + j * 32 + t * 16
                y[:, v0:v0 + 16] = dl[:, None] * ((q[:, 16 * t:16 * t + 16] >> (2 * j)) & 3) - ml[:, None]
                dl_all[:, v0:v0 + 16], ml_all[:, v0:v0 + 16] = np.abs(dl)[:, None], np.abs(ml)[:, None]
    return y, dl_all, ml_all


def _q3k_closed(raw):
    """dequantize_row_q3_K with its 12-byte scale unpack through u32 words
    (kmask1 = 0x03030303, kmask2 = 0x0f0f0f0f)."""
    raw = raw.reshape(-1, 110)
    n = raw.shape[0]
    d = _f16(raw, 108)
    aux = raw[:, 96:108].copy().view("<u4").astype(np.int64)
    k1, k2 = 0x03030303, 0x0F0F0F0F
    tmp = aux[:, 2]
    words = [(aux[:, 0] & k2) | (((tmp >> 0) & k1) << 4), (aux[:, 1] & k2) | (((tmp >> 2) & k1) << 4),
             ((aux[:, 0] >> 4) & k2) | (((tmp >> 4) & k1) << 4), ((aux[:, 1] >> 4) & k2) | (((tmp >> 6) & k1) << 4)]
    scales = np.stack([(w >> (8 * k)) & 0xFF for w in words for k in range(4)], axis=1) - 32
    hm = raw[:, 0:32].astype(np.int64)
    y, dl_all = np.zeros((n, 256)), np.zeros((n, 256))
    for half in range(2):
        q = raw[:, 32 + 32 * half:32 + 32 * half + 32].astype(np.int64)
        for j in range(4):
            mbit = 1 << (half * 4 + j)
            for t in range(2):
                dl = d * scales[:, half * 8 + 2 * j + t]
                low = (q[:, 16 * t:16 * t + 16] >> (2 * j)) & 3
                sub = np.where(hm[:, 16 * t:16 * t + 16] & mbit, 0, 4)
                v0 = half * 128 + j * 32 + t * 16
                y[:, v0:v0 + 16] = dl[:, None] * (low - sub)
                dl_all[:, v0:v0 + 16] = np.abs(dl)[:, None]
    return y, dl_all, np.zeros_like(dl_all)


def _q5k_closed(raw):
    """dequantize_row_q5_K: 4 chunks of 64, high bits u1 = 1 << 2j, u2 = 2 << 2j."""
    raw = raw.reshape(-1, 176)
    n = raw.shape[0]
    d, dm = _f16(raw, 0), _f16(raw, 2)
    qh = raw[:, 16:48].astype(np.int64)
    y, dl_all, ml_all = (np.zeros((n, 256)) for _ in range(3))
    for j in range(4):
        ql = raw[:, 48 + 32 * j:48 + 32 * j + 32].astype(np.int64)
        for t in range(2):
            sc, m = _scale_min_k4(raw[:, 4:16], 2 * j + t)
            dl, ml = d * sc, dm * m
            lo = (ql & 15) if t == 0 else (ql >> 4)
            hi = np.where(qh & (1 << (2 * j + t)), 16, 0)
            v0 = 64 * j + 32 * t
            y[:, v0:v0 + 32] = dl[:, None] * (lo + hi) - ml[:, None]
            dl_all[:, v0:v0 + 32], ml_all[:, v0:v0 + 32] = np.abs(dl)[:, None], np.abs(ml)[:, None]
    return y, dl_all, ml_all


def _q6k_closed(raw):
    """dequantize_row_q6_K: per half, y[l + 32 k] from ql/qh with scale is + 2k."""
    raw = raw.reshape(-1, 210)
    n = raw.shape[0]
    d = _f16(raw, 208)
    y, dl_all = np.zeros((n, 256)), np.zeros((n, 256))
    for half in range(2):
        ql = raw[:, 64 * half:64 * half + 64].astype(np.int64)
        qh = raw[:, 128 + 32 * half:128 + 32 * half + 32].astype(np.int64)
        sc = raw[:, 192 + 8 * half:200 + 8 * half].view(np.int8).astype(np.int64)
        qs = [(ql[:, 0:32] & 15) | ((qh & 3) << 4), (ql[:, 32:64] & 15) | (((qh >> 2) & 3) << 4),
              (ql[:, 0:32] >> 4) | (((qh >> 4) & 3) << 4), (ql[:, 32:64] >> 4) | (((qh >> 6) & 3) << 4)]
        for k in range(4):
            for l16 in range(2):
                dl = d * sc[:, l16 + 2 * k]
                v0 = half * 128 + 32 * k + 16 * l16
                y[:, v0:v0 + 16] = dl[:, None] * (qs[k][:, 16 * l16:16 * l16 + 16] - 32)
                dl_all[:, v0:v0 + 16] = np.abs(dl)[:, None]
    return y, dl_all, np.zeros_like(dl_all)


@pytest.mark.parametrize("code", [orc.Q4_1, orc.Q5_0, orc.Q5_1])
def test_32_value_types_equal_the_ggml_closed_form(code):
    # scale = d and bias = m (or -16 d, exact) are f16 already: one rounding, to f32
    raw = synthetic_blocks(code, 64, seed=20 + code)
    closed = _q4_1_closed(raw) if code == orc.Q4_1 else _q5_closed(raw, code == orc.Q5_0)
    got = orc.gguf_dequant_f32(code, raw, definition=0)
    assert np.array_equal(got, closed.astype(np.float32).reshape(-1))


@pytest.mark.parametrize("code,fn", [(orc.Q2_K, _q2k_closed), (orc.Q3_K, _q3k_closed),
                                     (orc.Q5_K, _q5k_closed), (orc.Q6_K, _q6k_closed)])
def test_superblock_types_match_the_ggml_closed_form(code, fn):
    raw = synthetic_blocks(code, 48, seed=30 + code)
    y, dl, ml = fn(raw)
    bits, _ = orc.AFFINE_CONFIG[code]
    got = orc.gguf_dequant_f32(code, raw, definition=0).reshape(y.shape).astype(np.float64)
    # the affine form rounds scale and bias to f16 (2^-11 relative each) and the
    # result to f32; a wrong code, group or scale is off by >= one |dl|
    bound = (dl * (1 << bits) + ml) * 2.0 ** -10 + np.abs(y) * 2.0 ** -23 + 2.0 ** -24
    assert (np.abs(got - y) <= bound).all()


def test_closed_form_bound_rejects_planted_errors():
    """The superblock bound above fails a code off by one, a scale of the
    neighbouring group or a dropped bias (mistakes planted in the oracle's
    output, on the CPU)."""
    raw = synthetic_blocks(orc.Q6_K, 8, seed=44)
    y, dl, ml = _q6k_closed(raw)
    got = orc.gguf_dequant_f32(orc.Q6_K, raw).reshape(y.shape).astype(np.float64)
    bound = (dl * 64 + ml) * 2.0 ** -10 + np.abs(y) * 2.0 ** -23 + 2.0 ** -24
    assert (np.abs(got - y) <= bound).all()
    off_by_one = got.copy()
    off_by_one[3, 17] += dl[3, 17]
    swapped = got.copy()
    swapped[:, 0:16], swapped[:, 16:32] = got[:, 16:32].copy(), got[:, 0:16].copy()
    for bad in (off_by_one, swapped):
        assert not (np.abs(bad - y) <= bound).all()
    raw2 = synthetic_blocks(orc.Q2_K, 8, seed=45)
    y2, dl2, ml2 = _q2k_closed(raw2)
    w, s, b = orc.gguf_convert_affine(orc.Q2_K, raw2)
    no_bias = orc.affine_dequant_f32(w.reshape(8, -1), s.reshape(8, -1), np.zeros_like(b).reshape(8, -1),
                                     orc.F16, 8, 256, 16, 2).astype(np.float64)
    assert not (np.abs(no_bias - y2) <= (dl2 * 4 + ml2) * 2.0 ** -10 + 2.0 ** -24).all()


# ---------------------------------------------------- endianness, zeros, native

def _to_big_endian(code, raw):
    """The same blocks with every multi-byte field byte-swapped: the f16 fields
    and, for Q5_0 / Q5_1, the u32 high-bit word (convert.rs:406-408, 553)."""
    nbytes, pos, signed = KQUANT_HEADERS[code]
    be = raw.reshape(-1, nbytes).copy()
    for off in pos + signed:
        be[:, [off, off + 1]] = be[:, [off + 1, off]]
    if code in (orc.Q5_0, orc.Q5_1):
        off = 2 if code == orc.Q5_0 else 4
        be[:, off:off + 4] = be[:, off:off + 4][:, ::-1]
    return be.reshape(-1)


@pytest.mark.parametrize("code", NEW)
def test_big_endian_fields_are_swapped(code):
    raw = synthetic_blocks(code, 6, seed=50 + code)
    le = orc.gguf_convert_affine(code, raw)
    be = orc.gguf_convert_affine(code, _to_big_endian(code, raw), big_endian=True)
    for a, b in zip(le, be):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("code", NEW)
def test_zero_blocks_decode_to_zero(code):
    _, nbytes = orc.BLOCK_GEOMETRY[code]
    z = np.zeros(3 * nbytes, np.uint8)
    for definition in (0, 1):
        assert (orc.gguf_dequant_f32(code, z, definition) == 0).all()


def test_q5_1_native_decoder_equals_the_affine_route():
    # native_quantization.rs:3499-3509: d * q + m with d, m unrounded f16 --
    # the affine scale and bias exactly
    raw = synthetic_blocks(orc.Q5_1, 128, seed=60)
    assert np.array_equal(orc.gguf_dequant_f32(orc.Q5_1, raw, 1), orc.gguf_dequant_f32(orc.Q5_1, raw, 0))

"""Pins the C oracle's IQ4_NL / IQ4_XS decoders (eredu-gguf/src/iquant.rs:
271-301) against the reference's llama.cpp differential vectors
(llama-c0bc8591-iq.oracle rows 20 and 23, f16 outputs, exact), its zero-block
and byte-order tests (eredu-gguf/tests/iquant.rs:130-180), and a closed form
of the 6-bit IQ4_XS group scales written from the field layout.  CPU only."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.fixtures import golden_iq_rows, synthetic_blocks

ROWS = golden_iq_rows()
LEVELS = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.float64)


@pytest.mark.parametrize("code", [orc.IQ4_NL, orc.IQ4_XS])
def test_matches_llama_cpp_vectors_exactly(code):
    raw, expected = ROWS[code]
    got = orc.gguf_dequant_f32(code, np.frombuffer(raw, np.uint8))
    with np.errstate(over="ignore"):
        assert np.array_equal(got.astype(np.float16).view(np.uint16), expected)


@pytest.mark.parametrize("code", [orc.IQ4_NL, orc.IQ4_XS])
def test_zero_blocks_decode_to_zero(code):
    _, nbytes = orc.BLOCK_GEOMETRY[code]
    for definition in (0, 1):
        assert (orc.gguf_dequant_f32(code, np.zeros(2 * nbytes, np.uint8), definition) == 0).all()


def test_byte_order_of_the_multibyte_fields():
    # iquant.rs:158-166: an IQ4_NL block of 0xff codes with d = -0.75
    little = np.full(18, 0xFF, np.uint8)
    little[:2] = np.frombuffer(np.float16(-0.75).tobytes(), np.uint8)
    big = little.copy()
    big[:2] = big[:2][::-1]
    assert np.array_equal(orc.gguf_dequant_f32(orc.IQ4_NL, little),
                          orc.gguf_dequant_f32(orc.IQ4_NL, big, big_endian=True))
    # IQ4_XS: d and the u16 of high scale bits both swap
    raw = synthetic_blocks(orc.IQ4_XS, 4, seed=1).reshape(-1, 136)
    be = raw.copy()
    be[:, [0, 1, 2, 3]] = raw[:, [1, 0, 3, 2]]
    assert np.array_equal(orc.gguf_dequant_f32(orc.IQ4_XS, raw.reshape(-1)),
                          orc.gguf_dequant_f32(orc.IQ4_XS, be.reshape(-1), big_endian=True))


def _closed_form(code, raw):
    """Group factor times level, in f64, from the field layout: IQ4_XS's
    6-bit scale = low nibble (scales_low[ib / 2] >> 4 (ib % 2)) plus the 2-bit
    high part (scales_high >> 2 ib) << 4, offset 32."""
    values, nbytes = orc.BLOCK_GEOMETRY[code]
    blocks = raw.reshape(-1, nbytes)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    if code == orc.IQ4_NL:
        q = np.concatenate([blocks[:, 2:18] & 15, blocks[:, 2:18] >> 4], axis=1)
        return (d[:, None] * LEVELS[q]).reshape(-1)
    sh = blocks[:, 2:4].copy().view("<u2")[:, 0].astype(np.int64)
    out = np.zeros((blocks.shape[0], 256))
    for ib in range(8):
        ls = ((blocks[:, 4 + ib // 2].astype(np.int64) >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
        qs = blocks[:, 8 + 16 * ib:24 + 16 * ib]
        q = np.concatenate([qs & 15, qs >> 4], axis=1)
        out[:, 32 * ib:32 * ib + 32] = (d * (ls - 32))[:, None] * LEVELS[q]
    return out.reshape(-1)


@pytest.mark.parametrize("code", [orc.IQ4_NL, orc.IQ4_XS])
def test_closed_form_on_random_blocks(code):
    raw = synthetic_blocks(code, 64, seed=code)
    got = orc.gguf_dequant_f32(code, raw)
    assert np.array_equal(got, _closed_form(code, raw).astype(np.float32))  # every product exact in f32

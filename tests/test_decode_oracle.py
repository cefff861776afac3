"""Pins of the decode-step oracle (oracle/decode_oracle.py) on the CPU: closed
forms, invariants and special cases chosen so that a dropped term, a wrong
sign or a swapped index fails one of them."""
import numpy as np
import pytest

from oracle import decode_oracle as D
from oracle import oracle as O


def test_llama3_freqs_regimes():
    f = D.llama3_rope_freqs(128, 500000.0)
    assert f.dtype == np.float32 and f.shape == (64,)
    assert f[0] == np.float32(1.0)  # wavelength 2 pi: high-frequency band, unscaled
    last = np.float32(500000.0) ** np.float32(126 / 128)
    assert np.isclose(f[63], 8.0 * last, rtol=1e-6)  # low-frequency band: scaled by the factor
    assert np.all(np.diff(f.astype(np.float64)) > 0)
    plain = D.llama3_rope_freqs(128, 500000.0, factor=1.0)
    ref = np.float32(500000.0) ** (np.arange(64, dtype=np.float32) * np.float32(2 / 128))
    assert np.allclose(plain, ref, rtol=1e-6)
    # the medium band joins both ends: the smooth interpolation at the
    # band edges equals the unscaled / scaled frequency
    wl = ref.astype(np.float64) * 2 * np.pi
    med = (wl > 2048) & (wl < 8192)
    assert med.any()
    ratio = f[med].astype(np.float64) / ref[med].astype(np.float64)
    assert np.all((ratio > 1.0) & (ratio < 8.0))


def test_rope_sign_pairing_and_invariants():
    freqs = D.llama3_rope_freqs(128, 10000.0, factor=1.0)
    e0 = np.zeros((1, 128))
    e0[0, 0] = 1.0
    pos = 3
    out = D.rope(e0, pos, freqs)
    a = pos / 1.0
    assert np.isclose(out[0, 0], np.cos(a)) and np.isclose(out[0, 64], np.sin(a))
    assert np.allclose(np.delete(out[0], [0, 64]), 0)
    rng = np.random.default_rng(0)
    q, k = rng.standard_normal((2, 128)), rng.standard_normal((2, 128))
    assert np.allclose(np.linalg.norm(D.rope(q, 17, freqs), axis=1), np.linalg.norm(q, axis=1))
    # relative position: <R(p)q, R(t)k> = <R(p - t)q, k>
    lhs = np.sum(D.rope(q, 29, freqs) * D.rope(k, 11, freqs), axis=1)
    rhs = np.sum(D.rope(q, 18, freqs) * k, axis=1)
    assert np.allclose(lhs, rhs, rtol=1e-5, atol=1e-5)  # angles are f32, as in the reference


def _bits(x):
    return O.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


def test_attention_special_cases():
    rng = np.random.default_rng(1)
    freqs = D.llama3_rope_freqs(128, 500000.0)
    nh, nkv, seq = 4, 2, 8
    q = _bits(rng.standard_normal(nh * 128))
    kn = _bits(rng.standard_normal(nkv * 128))
    vn = _bits(rng.standard_normal(nkv * 128))
    kc = _bits(rng.standard_normal((nkv, seq, 128)))
    vc = _bits(rng.standard_normal((nkv, seq, 128)))
    # one position: the output is the new value, per KV head h // 2
    out, kc2, vc2 = D.attention_decode(q, kn, vn, kc, vc, freqs, 0, nh, nkv, 1 / np.sqrt(128))
    v = D.bits_to_f64(vn).reshape(nkv, 128)
    for h in range(nh):
        assert np.allclose(out[h], v[h // 2])
    assert np.array_equal(vc2[:, 0], vn.reshape(nkv, 128))
    assert np.array_equal(kc2[:, 1:], kc[:, 1:])  # only row pos written
    rot = D.rope(D.bits_to_f64(kn).reshape(nkv, 128), 0, freqs)
    assert np.array_equal(kc2[:, 0], _bits(rot))  # position 0 rotates by zero
    assert np.array_equal(kc2[:, 0], kn.reshape(nkv, 128))
    # equal keys everywhere: uniform weights, the mean of the values
    same = np.broadcast_to(kc[:, :1], kc.shape).copy()
    kn_same = np.zeros(nkv * 128, dtype=np.uint16)  # rotated zero stays zero; make all keys zero
    zero_cache = np.zeros_like(same)
    out, _, _ = D.attention_decode(q, kn_same, vn, zero_cache, vc, freqs, seq - 1, nh, nkv, 0.1)
    vv = D.bits_to_f64(vc).copy()
    vv[:, seq - 1] = D.bits_to_f64(vn).reshape(nkv, 128)
    for h in range(nh):
        assert np.allclose(out[h], vv[h // 2].mean(axis=0))


def test_rms_norm_closed_forms():
    w = _bits(np.linspace(0.5, 1.5, 64))
    c = 0.75
    xbits = _bits(np.full(64, c))
    _, out = D.rms_norm_bf16(xbits, w, 1e-5)
    expect = D.bf16(D.bits_to_f64(w) * c / np.sqrt(c * c + 1e-5))
    assert np.array_equal(D.bits_to_f64(out), expect)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 64))
    a = D.rms_norm(x, 1.0, 0.0)
    b = D.rms_norm(4.0 * x, 1.0, 0.0)
    assert np.allclose(a, b)
    assert np.allclose(np.mean(a * a, axis=1), 1.0)
    # the residual is added (and rounded) before the norm
    r = _bits(rng.standard_normal(64))
    hid, _ = D.rms_norm_bf16(xbits, w, 1e-5, r)
    assert np.array_equal(D.bits_to_f64(hid), D.bf16(c + D.bits_to_f64(r)))


def test_silu_mul_special_cases():
    g = _bits([0.0, 20.0, -20.0, 1.0])
    u = _bits([3.0, 2.0, 5.0, 1.0])
    out = D.bits_to_f64(D.silu_mul_bf16(g, u))
    assert out[0] == 0.0
    assert out[1] == 40.0
    assert abs(out[2]) < 1e-6
    assert np.isclose(out[3], 1.0 / (1.0 + np.exp(-1.0)), rtol=1e-2)

"""CPU oracle for the quantized-linear path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg import this module, and only as the checker or the timed CPU baseline.
The product (``eredu_amd``) never imports it and has no CPU fallback.

Two layers:

* ``eq_oracle.c`` (built by ``oracle/Makefile`` into ``oracle/_build``): the
  byte-level restatement of ``eredu-gguf/src/convert.rs`` and the native
  decoders of ``safemlx/src/native_quantization.rs``, f16/bf16 rounding, an
  input quantizer and the restated MLX CPU ``_qmm_t`` loop (CPU baseline).
* numpy: the fp64 closed form of ``quantized_matmul`` (the matmul oracle),
  ``gather_qmm_f64`` (index broadcasting around it; pinned in
  tests/test_oracle_gather.py by a closed form: expert e dequantizing to the
  constant e + 1 gives y[b] = (rhs[b] + 1) * sum(x[lhs[b]]), which a swapped,
  mis-broadcast or dropped index fails) and bf16 helpers.

Parity status per function is listed in the header of ``eq_oracle.c``; every
function here that is not a thin wrapper names what pins it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libeq_oracle.so")

F32, F16, BF16 = 0, 1, 2
Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 2, 3, 6, 7, 8
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 10, 11, 12, 13, 14
BLOCK_GEOMETRY = {Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24), Q8_0: (32, 34),
                  Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176),
                  Q6_K: (256, 210)}  # format.rs:368-400
AFFINE_CONFIG = {Q4_0: (4, 32), Q4_1: (4, 32), Q5_0: (5, 32), Q5_1: (5, 32), Q8_0: (8, 32),
                 Q2_K: (2, 16), Q3_K: (3, 16), Q4_K: (4, 32), Q5_K: (5, 32), Q6_K: (6, 16)}  # convert.rs:142-152
GGUF_TYPES = tuple(BLOCK_GEOMETRY)
IQ4_NL, IQ4_XS = 20, 23
BLOCK_GEOMETRY.update({IQ4_NL: (32, 18), IQ4_XS: (256, 136)})  # format.rs:368-400 (no affine form)

_lib = None


def build() -> str:
    """Compile eq_oracle.c with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH) or os.path.getmtime(LIB_PATH) < os.path.getmtime(
            os.path.join(HERE, "eq_oracle.c")
        ):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_bf16.argtypes = [ctypes.c_float]
        L.or_f32_to_bf16.restype = ctypes.c_uint16
        L.or_gguf_convert_affine.argtypes = [i32, i32, vp, i64, vp, vp, vp]
        L.or_gguf_dequant_f32.argtypes = [i32, i32, i32, vp, i64, vp]
        L.or_affine_dequant_f32.argtypes = [vp, vp, vp, i32, i64, i64, i32, i32, vp]
        L.or_quantize_affine.argtypes = [vp, i64, i64, i32, i32, i32, vp, vp, vp]
        L.or_qmm_t_f32.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, i32, i32, i32, i32, i32]
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------ floats

def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (NaN kept quiet).
    Pinned against torch's bfloat16 conversion in tests/test_oracle.py."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x7FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def scalar_to_f32(a: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == F16:
        return f16_bits_to_f32(a)
    if dtype == BF16:
        return bf16_bits_to_f32(a)
    return np.asarray(a, dtype=np.float32)


def scalar_to_f64(a: np.ndarray, dtype: int) -> np.ndarray:
    return scalar_to_f32(a, dtype).astype(np.float64)  # exact widening


def f32_to_f16_bits_c(x: np.ndarray) -> np.ndarray:
    L = lib()
    flat = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([L.or_f32_to_f16(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(x))


# ------------------------------------------------------------------ GGUF

def gguf_convert_affine(ggml_type: int, raw: np.ndarray, big_endian: bool = False):
    """Blocks -> (u32 codes, f16 scale bits, f16 bias bits), eredu-gguf/src/convert.rs:318-465.
    Returned flat in block order; reshape to [rows, ...] at the caller."""
    values, nbytes = BLOCK_GEOMETRY[ggml_type]
    bits, gs = AFFINE_CONFIG[ggml_type]
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    assert raw.size % nbytes == 0
    nblocks = raw.size // nbytes
    w = np.zeros(nblocks * values * bits // 32, dtype=np.uint32)
    s = np.zeros(nblocks * values // gs, dtype=np.uint16)
    b = np.zeros_like(s)
    rc = lib().or_gguf_convert_affine(ggml_type, int(big_endian), _p(raw), nblocks, _p(w), _p(s), _p(b))
    assert rc == 0
    return w, s, b


def gguf_dequant_f32(ggml_type: int, raw: np.ndarray, definition: int = 0, big_endian: bool = False) -> np.ndarray:
    """Dense f32 dequant; definition 0 = affine route (convert.rs:81-101),
    1 = native decoder (native_quantization.rs:3445-3469, 3499-3509,
    3539-3542) where the type has one, else the affine route."""
    values, nbytes = BLOCK_GEOMETRY[ggml_type]
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    nblocks = raw.size // nbytes
    out = np.zeros(nblocks * values, dtype=np.float32)
    rc = lib().or_gguf_dequant_f32(ggml_type, int(big_endian), definition, _p(raw), nblocks, _p(out))
    assert rc == 0
    return out


def gguf_dequant_bf16(ggml_type: int, raw: np.ndarray, definition: int = 0, big_endian: bool = False) -> np.ndarray:
    return f32_to_bf16_bits(gguf_dequant_f32(ggml_type, raw, definition, big_endian))


# ------------------------------------------------------------------ affine

def unpack_codes(w: np.ndarray, cols: int, bits: int) -> np.ndarray:
    """LSB-first codes of each row of packed u32 words (convert.rs:87-99)."""
    w = np.ascontiguousarray(w, dtype=np.uint32)
    rows = w.shape[0]
    if 32 % bits == 0:  # codes never straddle words
        pack = 32 // bits
        shifts = (np.arange(pack, dtype=np.uint32) * bits).astype(np.uint32)
        codes = (w[:, :, None] >> shifts) & np.uint32((1 << bits) - 1)
        return codes.reshape(rows, -1)[:, :cols]
    bitstream = np.unpackbits(w.view(np.uint8).reshape(rows, -1), axis=1, bitorder="little")
    bitstream = bitstream[:, : cols * bits].reshape(rows, cols, bits).astype(np.uint32)
    return (bitstream << np.arange(bits, dtype=np.uint32)).sum(axis=2).astype(np.uint32)


def affine_dequant_f32(w, scales, biases, scale_dtype, rows, cols, gs, bits) -> np.ndarray:
    """f32 s*q + b with one multiply and one add (convert.rs:81-101)."""
    out = np.zeros((rows, cols), dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    scales = np.ascontiguousarray(scales)
    biases = None if biases is None else np.ascontiguousarray(biases)
    lib().or_affine_dequant_f32(_p(w), _p(scales), _p(biases), scale_dtype, rows, cols, gs, bits, _p(out))
    return out


def affine_dequant_f64(w, scales, biases, scale_dtype, rows, cols, gs, bits) -> np.ndarray:
    """Exact dequantized weights in f64 (s and b are at most f32-precise and the
    codes at most 8 bits, so s*q + b is exact in f64 up to one final rounding)."""
    q = unpack_codes(np.asarray(w).reshape(rows, -1), cols, bits).reshape(rows, cols // gs, gs)
    s = scalar_to_f64(np.asarray(scales).reshape(rows, cols // gs), scale_dtype)
    out = q * s[:, :, None]
    if biases is not None:
        b = scalar_to_f64(np.asarray(biases).reshape(rows, cols // gs), scale_dtype)
        out += b[:, :, None]
    return out.reshape(rows, cols)


def quantized_matmul_f64(x, x_dtype, w, scales, biases, scale_dtype, transpose, group_size, bits, N, K):
    """fp64 closed form of quantized_matmul (safemlx/src/ops/quantization.rs:190-226):
    transpose=True : W is [N, K] packed along K; y = x @ W^T.
    transpose=False: W is [K, N] packed along N; y = x @ W.
    ``x`` is [..., K] as stored bits (f16/bf16) or f32 values."""
    x64 = scalar_to_f64(np.asarray(x), x_dtype).reshape(-1, K)
    if transpose:
        W = affine_dequant_f64(w, scales, biases, scale_dtype, N, K, group_size, bits)
        return x64 @ W.T
    W = affine_dequant_f64(w, scales, biases, scale_dtype, K, N, group_size, bits)
    return x64 @ W


def gather_qmm_f64(x, x_dtype, w, scales, biases, scale_dtype, lhs, rhs, transpose, group_size, bits, N, K):
    """fp64 gather_qmm (MLX's gather_qmm under safemlx::ops::gather_qmm_with_mode,
    safemlx/src/ops/quantization.rs:298-379): x [Bx, M, K] (stored bits or
    f32), w / scales / biases [Bw, ...]; lhs and rhs (integer arrays, or None
    for arange over x's / w's batches) broadcast together to the output batch
    shape; y[b] = quantized_matmul(x[lhs[b]], w[rhs[b]]).  Returns f64
    [*batch, M, N]; a batch with an index out of range is all zeros (the
    device path's rule; MLX leaves it undefined)."""
    x = np.asarray(x)
    Bx, Bw = x.shape[0], np.asarray(w).shape[0]
    lhs = np.arange(Bx) if lhs is None else np.asarray(lhs)
    rhs = np.arange(Bw) if rhs is None else np.asarray(rhs)
    shape = np.broadcast_shapes(lhs.shape, rhs.shape)
    li = np.broadcast_to(lhs, shape).reshape(-1)
    ri = np.broadcast_to(rhs, shape).reshape(-1)
    M = x.shape[1]
    y = np.zeros((li.size, M, N))
    for b, (i, e) in enumerate(zip(li, ri)):
        if not (0 <= i < Bx and 0 <= e < Bw):
            continue
        y[b] = quantized_matmul_f64(x[i], x_dtype, w[e], scales[e], None if biases is None else biases[e],
                                    scale_dtype, transpose, group_size, bits, N, K)
    return y.reshape(*shape, M, N)


def qmm_t_f32(x, x_dtype, w, scales, biases, scale_dtype, M, N, K, gs, bits, threads=1) -> np.ndarray:
    """Restated MLX CPU _qmm_t (f32 accumulate); the timed CPU baseline."""
    y = np.zeros((M, N), dtype=np.float32)
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w, dtype=np.uint32)
    scales = np.ascontiguousarray(scales)
    biases = None if biases is None else np.ascontiguousarray(biases)
    rc = lib().or_qmm_t_f32(_p(y), _p(x), _p(w), _p(scales), _p(biases), M, N, K, gs, bits,
                            x_dtype, scale_dtype, threads)
    assert rc == 0
    return y


def quantize_affine(wf32: np.ndarray, group_size: int, bits: int, scale_dtype: int):
    """Input generator (role of MLX quantize); parity unpinned, see eq_oracle.c."""
    wf32 = np.ascontiguousarray(wf32, dtype=np.float32)
    rows, cols = wf32.shape
    wq = np.zeros((rows, cols * bits // 32), dtype=np.uint32)
    sdt = np.float32 if scale_dtype == F32 else np.uint16
    s = np.zeros((rows, cols // group_size), dtype=sdt)
    b = np.zeros_like(s)
    lib().or_quantize_affine(_p(wf32), rows, cols, group_size, bits, scale_dtype, _p(wq), _p(s), _p(b))
    return wq, s, b


# ------------------------------------------------------------------ MXFP4

# E2M1 magnitudes of codes 0..7 (OCP Microscaling Formats v1.0, sec. 5.3.3:
# 1 sign, 2 exponent bits with bias 1, 1 mantissa bit, exponent 0 subnormal);
# code bit 3 is the sign.  Pinned in tests/test_oracle_mxfp4.py by decoding
# the bit fields.
E2M1_MAGNITUDES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def e2m1_decode(codes: np.ndarray) -> np.ndarray:
    c = np.asarray(codes, dtype=np.uint32)
    return np.where(c & 8, -1.0, 1.0) * E2M1_MAGNITUDES[c & 7]


def e8m0_decode(e: np.ndarray) -> np.ndarray:
    """2^(e - 127); 255 is NaN (OCP MX v1.0 sec. 5.4).  Pinned by the
    reference's decode test (eredu/src/backend/mlx/nn/fp8.rs:1670-1678:
    127, 128, 126 -> 1, 2, 0.5) and np.ldexp."""
    e = np.asarray(e, dtype=np.int64)
    out = np.ldexp(1.0, e - 127)
    return np.where(e == 255, np.nan, out)


def mxfp4_convert_ggml(raw: np.ndarray, rows: int, cols: int):
    """GGML type-39 blocks -> (u32 weights [rows, cols/8], u8 scales [rows,
    cols/32]) as eredu-gguf/src/convert.rs:247-276: each 17-byte block is the
    scale byte and 16 code bytes, low nibbles values 0..15, high nibbles
    16..31, packed 8 codes per word LSB-first.  Pinned by the golden vector of
    eredu-gguf/tests/mxfp4.rs:5-60."""
    blocks = np.asarray(raw, dtype=np.uint8).reshape(-1, 17)
    assert blocks.shape[0] == rows * (cols // 32)
    q = blocks[:, 1:].astype(np.uint32)
    values = np.concatenate([q & 15, q >> 4], axis=1)  # [blocks, 32]
    words = (values.reshape(-1, 4, 8) << (np.arange(8, dtype=np.uint32) * 4)).sum(axis=2).astype(np.uint32)
    return words.reshape(rows, cols // 8), blocks[:, 0].reshape(rows, cols // 32).copy()


def mxfp4_dequant_f64(w, scales, rows, cols) -> np.ndarray:
    """2^(e - 127) * e2m1(q) per value (exact in f64 and in f32 for e >= 1)."""
    q = unpack_codes(np.asarray(w).reshape(rows, -1), cols, 4).reshape(rows, cols // 32, 32)
    s = e8m0_decode(np.asarray(scales).reshape(rows, cols // 32))
    return (e2m1_decode(q) * s[:, :, None]).reshape(rows, cols)


def mxfp4_quantize(wf32: np.ndarray):
    """(u32 codes, u8 scales) of w [rows, cols] in groups of 32 along the last
    axis: the scale is the smallest power of two 2^e, e in [-127, 127], with
    amax / 2^e <= 6, so nothing saturates (this is not the OCP MX v1.0
    sec. 6.3 rule, which takes 2^(floor(log2 amax) - 2) and clamps to 6:
    at amax = 7 that rule gives scale 1, this one 2); every value is w / 2^e rounded to the
    nearest E2M1 value, ties to the even code, sign bit set for w < 0; a
    group with a NaN or an infinity gets scale byte 255 (NaN) and magnitude
    codes 0, an all-zero group byte 0.  Found by
    search over exponents and over the 8 magnitudes (no closed form is
    shared with the device code).  MLX's own mxfp4 quantizer is not in this
    image: parity of this rule with MLX is unpinned."""
    w = np.ascontiguousarray(wf32, dtype=np.float32).astype(np.float64)
    rows, cols = w.shape
    g = w.reshape(rows, cols // 32, 32)
    amax = np.abs(g).max(axis=2)
    bad = ~np.isfinite(g).all(axis=2)
    exps = np.arange(-127, 128)
    fits = amax[:, :, None] <= 6.0 * np.ldexp(1.0, exps)[None, None, :]
    e = exps[np.argmax(fits, axis=2)]  # the first (smallest) exponent that fits
    e = np.where(amax > 0, e, -127)
    sbyte = np.where(bad, 255, e + 127).astype(np.uint8)
    a = np.abs(np.where(bad[:, :, None], 0.0, g)) / np.ldexp(1.0, e)[:, :, None]
    dist = np.abs(a[..., None] - E2M1_MAGNITUDES)  # [rows, groups, 32, 8]
    best = dist.min(axis=3, keepdims=True)
    cand = dist == best
    # ties: the even code (codes 0..7 alternate even/odd mantissa bits)
    even = cand & (np.arange(8) % 2 == 0)
    m = np.where(even.any(axis=3), np.argmax(even, axis=3), np.argmax(cand, axis=3)).astype(np.uint32)
    # the sign bit follows w < 0 (so small negatives become -0, NaN and -0.0 stay +)
    codes = (m | np.where(g < 0, 8, 0).astype(np.uint32)).reshape(rows, cols)
    words = (codes.reshape(rows, -1, 8) << (np.arange(8, dtype=np.uint32) * 4)).sum(axis=2).astype(np.uint32)
    return words, sbyte


def mxfp4_matmul_f64(x, x_dtype, w, scales, transpose, N, K):
    """fp64 closed form of the MXFP4 quantized_matmul
    (safemlx/src/ops/quantization.rs:190-226, mode "mxfp4")."""
    x64 = scalar_to_f64(np.asarray(x), x_dtype).reshape(-1, K)
    if transpose:
        return x64 @ mxfp4_dequant_f64(w, scales, N, K).T
    return x64 @ mxfp4_dequant_f64(w, scales, K, N)


# ------------------------------------------------------------------ parity rule

def bf16_half_ulp(y: np.ndarray) -> np.ndarray:
    """Half a bf16 ulp at |y| (the output-rounding allowance)."""
    a = np.abs(np.asarray(y, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 0.5 * 2.0 ** (e - 7)


def matmul_within_tolerance(y, y_ref, out_is_bf16: bool, rel: float = 1e-2):
    """|y - y_ref| <= rel*RMS(y_ref) (+ half a bf16 ulp when y is bf16)."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    rms = float(np.sqrt(np.mean(y_ref ** 2))) if y_ref.size else 0.0
    bound = rel * rms + (bf16_half_ulp(y_ref) if out_is_bf16 else 0.0)
    err = np.abs(y - y_ref)
    ok = bool(np.all(err <= bound))
    worst = float(np.max(err / max(rms, 1e-30))) if err.size else 0.0
    return ok, worst, rms

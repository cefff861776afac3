"""CPU oracle of the Llama decode step around the quantized projections --
TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and ``__graft_entry__.smoke()`` import this module, as the
checker of ``eq_rms_norm``, ``eq_rope_attention_decode``, ``eq_silu_mul``,
``eq_embedding``, ``eq_argmax`` and of a whole decode step.  numpy, with the
reference's bf16 roundings at the op boundaries it has them and f64 inside
an op (the GPU accumulates in f32; tests compare within a stated tolerance).

What pins each function (tests/test_decode_oracle.py):
* ``llama3_rope_freqs``: i = 0 gives 1 (wavelength 2*pi, below the
  high-frequency cut, unscaled); the last pair is base^((d-2)/d) * factor
  (wavelength past the low-frequency cut); factor 1 gives base^(2i/d)
  everywhere; the medium band is continuous with both ends.
* ``rope``: e_0 at angle a maps to cos a at 0 and sin a at d/2 (the sign and
  the half-split pairing); norms are preserved; <R(p)q, R(t)k> depends on
  p - t only.
* ``attention_decode``: one position returns v; equal keys return the mean
  of the values; head h reads KV head h // group.
* ``rms_norm``: a constant row c gives weight * c / sqrt(c^2 + eps); scaling
  the row leaves the output unchanged (eps = 0).
* ``silu_mul``: silu(0) = 0, silu(x) -> x for large x, silu(-x) -> 0.
* ``decode_step``: composed of the above and ``oracle.quantized_matmul_f64``.
"""
from __future__ import annotations

import numpy as np

from . import oracle as O


def bf16(x) -> np.ndarray:
    """Round to bf16 (RNE), returned as f64 values."""
    return O.bf16_bits_to_f32(O.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))).astype(np.float64)


def bits_to_f64(b: np.ndarray) -> np.ndarray:
    return O.bf16_bits_to_f32(np.asarray(b, dtype=np.uint16)).astype(np.float64)


def llama3_rope_freqs(dims: int, base: float, factor: float = 8.0, low_freq_factor: float = 1.0,
                      high_freq_factor: float = 4.0, original_max_position_embeddings: int = 8192) -> np.ndarray:
    """Llama3Rope's `freqs` (eredu/src/backend/mlx/nn/rope.rs:105-186), in f32
    like the reference's arrays: freqs_i = base^(2i/dims), then wavelengths
    2*pi*freqs past orig/low scaled by `factor`, those between orig/high and
    orig/low interpolated."""
    f32 = np.float32
    half = dims // 2
    exps = np.arange(half, dtype=f32) * f32(2.0 / dims)
    freqs = np.power(f32(base), exps).astype(f32)
    old = f32(original_max_position_embeddings)
    low_wl, high_wl = old / f32(low_freq_factor), old / f32(high_freq_factor)
    wl = freqs * f32(2.0 * np.pi)
    freqs = np.where(wl > low_wl, freqs * f32(factor), freqs).astype(f32)
    medium = (wl > high_wl) & (wl < low_wl)
    smooth = ((f32(1.0) / wl) * old - f32(low_freq_factor)) / f32(high_freq_factor - low_freq_factor)
    denom = (f32(1.0) - smooth) / f32(factor) + smooth
    freqs = np.where(medium, freqs / denom, freqs).astype(f32)
    return freqs


def rope(x: np.ndarray, pos: int, freqs: np.ndarray) -> np.ndarray:
    """Half-split rotation of rows of x (f64 [heads, d]) at position pos, angle
    pos / freqs[i] (rope.rs:196-216): out1 = x1 cos - x2 sin, out2 = x2 cos + x1 sin."""
    d = x.shape[-1]
    h = d // 2
    a = np.float64(np.float32(pos) / freqs.astype(np.float32))
    c, s = np.cos(a), np.sin(a)
    x1, x2 = x[..., :h], x[..., h:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """weight * x / sqrt(mean(x^2) + eps) per row (fast::rms_norm), f64."""
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return weight * (x / np.sqrt(ms + eps))


def rms_norm_bf16(x_bits, weight_bits, eps, residual_bits=None):
    """eq_rms_norm: hidden (+ residual, rounded to bf16), then the norm rounded
    to bf16.  Returns (hidden_bits, out_bits)."""
    x = bits_to_f64(x_bits)
    if residual_bits is not None:
        x = bf16(x + bits_to_f64(residual_bits))
    out = bf16(rms_norm(x, bits_to_f64(weight_bits), eps))
    return O.f32_to_bf16_bits(x.astype(np.float32)), O.f32_to_bf16_bits(out.astype(np.float32))


def attention_decode(q_bits, k_new_bits, v_new_bits, k_cache_bits, v_cache_bits, freqs, pos, n_heads, n_kv_heads,
                     scale):
    """eq_rope_attention_decode: rotate q and the new key at pos, store the
    rotated key (bf16) and value at row pos of the caches (copies returned),
    softmax(scale q.k) . v over rows 0..pos per head, KV head h // group.
    Returns (out f64 [n_heads, d], k_cache_bits, v_cache_bits)."""
    d = 128
    group = n_heads // n_kv_heads
    q = rope(bits_to_f64(q_bits).reshape(n_heads, d), pos, freqs)
    kn = rope(bits_to_f64(k_new_bits).reshape(n_kv_heads, d), pos, freqs)
    kc = np.array(k_cache_bits, dtype=np.uint16, copy=True)
    vc = np.array(v_cache_bits, dtype=np.uint16, copy=True)
    kc[:, pos, :] = O.f32_to_bf16_bits(kn.astype(np.float32))
    vc[:, pos, :] = np.asarray(v_new_bits, dtype=np.uint16).reshape(n_kv_heads, d)
    K = bits_to_f64(kc[:, : pos + 1, :])
    V = bits_to_f64(vc[:, : pos + 1, :])
    out = np.empty((n_heads, d))
    for h in range(n_heads):
        g = h // group
        s = scale * (K[g] @ q[h])
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V[g]
    return out, kc, vc


def silu_mul_bf16(gate_bits, up_bits) -> np.ndarray:
    """silu(gate) * up with bf16 rounding after sigmoid, after x * sigmoid and
    after the product (layers.rs:21, llama.rs:414-422).  Returns bf16 bits."""
    g = bits_to_f64(gate_bits)
    u = bits_to_f64(up_bits)
    sg = bf16(1.0 / (1.0 + np.exp(-g)))
    sl = bf16(g * sg)
    return O.f32_to_bf16_bits((sl * u).astype(np.float32))


def linear_bf16(x_bits, lin) -> np.ndarray:
    """A quantized projection (transpose = true, bf16 scales) rounded to bf16."""
    w, s, b, bits, gs = lin["w"], lin["s"], lin["b"], lin["bits"], lin["gs"]
    N = w.shape[0]
    K = w.shape[1] * 32 // bits
    y = O.quantized_matmul_f64(np.asarray(x_bits, dtype=np.uint16).reshape(1, K), O.BF16, w, s, b, O.BF16, True,
                               gs, bits, N, K)
    return O.f32_to_bf16_bits(y.astype(np.float32)).reshape(N)


def decode_step(model: dict, token: int, pos: int, k_caches, v_caches):
    """One batch-1 decode step of a Llama-shaped model (Model::forward with
    one token, llama.rs:477-495, 557-574, 649-658), every op rounded to bf16
    at its output.  model: dims, eps, freqs, embed bits [V, H], final_norm,
    layers [{in_norm, post_norm, q, k, v, o, gate, up, down}], lm_head.
    Caches (bits [n_kv, max_seq, 128] per layer) are updated in place.
    Returns (logits f64 [V], hidden bits after the last layer)."""
    H, nh, nkv, eps = model["hidden"], model["n_heads"], model["n_kv_heads"], model["eps"]
    scale = 1.0 / np.sqrt(128.0)
    x = np.asarray(model["embed"][token], dtype=np.uint16).copy()
    resid = None
    for li, L in enumerate(model["layers"]):
        x, h = rms_norm_bf16(x, L["in_norm"], eps, resid)
        q, k, v = linear_bf16(h, L["q"]), linear_bf16(h, L["k"]), linear_bf16(h, L["v"])
        att, kc, vc = attention_decode(q, k, v, k_caches[li], v_caches[li], model["freqs"], pos, nh, nkv, scale)
        k_caches[li][...] = kc
        v_caches[li][...] = vc
        att_bits = O.f32_to_bf16_bits(att.reshape(-1).astype(np.float32))
        o = linear_bf16(att_bits, L["o"])
        x, h2 = rms_norm_bf16(x, L["post_norm"], eps, o)
        act = silu_mul_bf16(linear_bf16(h2, L["gate"]), linear_bf16(h2, L["up"]))
        resid = linear_bf16(act, L["down"])
    x, hf = rms_norm_bf16(x, model["final_norm"], eps, resid)
    lm = model["lm_head"]
    N = lm["w"].shape[0]
    logits = O.quantized_matmul_f64(hf.reshape(1, H), O.BF16, lm["w"], lm["s"], lm["b"], O.BF16, True, lm["gs"],
                                    lm["bits"], N, H).reshape(N)
    return logits, x

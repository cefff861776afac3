"""Batch-1 decode step of a Llama-shaped model on the HIP kernels.

Mirrors the caller structure of the reference's decoder
(eredu-architectures/src/llama.rs): ``Decoder::embed`` (:576-582), per layer
``TransformerBlock::forward`` (:477-495) -- input RMSNorm, q/k/v projections,
RoPE + KV-cache update + attention (``Attention::attend``, :296-330), output
projection, residual add, post-attention RMSNorm, SwiGLU MLP (``Mlp``,
:414-433), residual add -- then the final norm and ``Model::logits``
(:649-658), and greedy selection of the next token.

All seven projections per layer and the LM head go through the quantized
matmul C ABI (q/k/v and gate/up as one grouped launch each, results
bit-identical to separate calls); the rest through the decode entry points of
``include/eredu_hip.h``.  Every buffer is allocated once, so a step can be
captured in a HIP graph; the token id lives in device memory and the step
reads it (embedding) and overwrites it (argmax).  The position is either an
argument of the step that a capture records (``step(pos)``: one graph replays
one position), or lives in device memory too (``step_device()``: attention
reads it when it runs and the step ends by advancing it, so one captured
graph decodes successive tokens, as the reference's token loop advances its
cache offset every token, eredu/src/runtime/generation/streaming.rs:1038-1050).
There is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _native
from ._native import check

HEAD_DIM = 128


def llama3_rope_freqs(dims: int, base: float, factor: float = 8.0, low_freq_factor: float = 1.0,
                      high_freq_factor: float = 4.0, original_max_position_embeddings: int = 8192) -> np.ndarray:
    """The rotary frequencies of Llama3Rope::new (eredu/src/backend/mlx/nn/rope.rs:105-186),
    in f32 like the reference's arrays: base^(2i/dims), long wavelengths
    (past orig / low_freq_factor) scaled by ``factor``, the band between
    orig / high_freq_factor and orig / low_freq_factor interpolated.
    ``factor = 1`` gives plain RoPE frequencies."""
    f32 = np.float32
    exps = np.arange(dims // 2, dtype=f32) * f32(2.0 / dims)
    freqs = np.power(f32(base), exps).astype(f32)
    old = f32(original_max_position_embeddings)
    low_wl, high_wl = old / f32(low_freq_factor), old / f32(high_freq_factor)
    wl = freqs * f32(2.0 * math.pi)
    freqs = np.where(wl > low_wl, freqs * f32(factor), freqs).astype(f32)
    medium = (wl > high_wl) & (wl < low_wl)
    smooth = ((f32(1.0) / wl) * old - f32(low_freq_factor)) / f32(high_freq_factor - low_freq_factor)
    freqs = np.where(medium, freqs / ((f32(1.0) - smooth) / f32(factor) + smooth), freqs).astype(f32)
    return freqs


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _bf16(t: torch.Tensor, what: str) -> None:
    if t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous():
        raise _native.EreduError(f"{what} must be a contiguous bf16 CUDA tensor")


def rms_norm(hidden: torch.Tensor, weight: torch.Tensor, eps: float,
             residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``hidden += residual`` (in place, when given), then RMSNorm(hidden) * weight
    (C ABI: eq_rms_norm)."""
    for t, n in ((hidden, "hidden"), (weight, "weight")):
        _bf16(t, n)
    if residual is not None:
        _bf16(residual, "residual")
    dim = hidden.shape[-1]
    out = torch.empty_like(hidden)
    check(_native.lib().eq_rms_norm(out.data_ptr(), hidden.data_ptr(),
                                    residual.data_ptr() if residual is not None else None, weight.data_ptr(),
                                    hidden.numel() // dim, dim, float(eps), _native.EQ_DTYPE_BF16, _stream()))
    return out


def rope_attention_decode(q, k_new, v_new, k_cache, v_cache, freqs: torch.Tensor, pos: int, n_heads: int,
                          n_kv_heads: int, scale: float) -> torch.Tensor:
    """RoPE of q and k_new at ``pos``, cache update, grouped-query attention over
    positions 0..pos (C ABI: eq_rope_attention_decode).  Caches are
    [n_kv_heads, max_seq, 128] bf16 and are written at row ``pos``."""
    for t, n in ((q, "q"), (k_new, "k_new"), (v_new, "v_new"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _bf16(t, n)
    if freqs.dtype != torch.float32 or not freqs.is_cuda:
        raise _native.EreduError("freqs must be a float32 CUDA tensor")
    out = torch.empty((n_heads * HEAD_DIM,), dtype=torch.bfloat16, device=q.device)
    check(_native.lib().eq_rope_attention_decode(
        out.data_ptr(), q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        freqs.data_ptr(), int(pos), k_cache.shape[1], n_heads, n_kv_heads, HEAD_DIM, float(scale),
        _native.EQ_DTYPE_BF16, _stream()))
    return out


def rope_attention_decode_at(q, k_new, v_new, k_cache, v_cache, freqs: torch.Tensor, pos: torch.Tensor,
                             n_heads: int, n_kv_heads: int, scale: float) -> torch.Tensor:
    """rope_attention_decode at the position held by the int32 device tensor
    ``pos`` (read when the kernel runs; C ABI: eq_rope_attention_decode_at)."""
    for t, n in ((q, "q"), (k_new, "k_new"), (v_new, "v_new"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _bf16(t, n)
    if freqs.dtype != torch.float32 or not freqs.is_cuda:
        raise _native.EreduError("freqs must be a float32 CUDA tensor")
    if pos.dtype != torch.int32 or not pos.is_cuda:
        raise _native.EreduError("pos must be an int32 CUDA tensor")
    out = torch.empty((n_heads * HEAD_DIM,), dtype=torch.bfloat16, device=q.device)
    check(_native.lib().eq_rope_attention_decode_at(
        out.data_ptr(), q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        freqs.data_ptr(), pos.data_ptr(), k_cache.shape[1], n_heads, n_kv_heads, HEAD_DIM, float(scale),
        _native.EQ_DTYPE_BF16, _stream()))
    return out


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up with the reference's bf16 roundings (C ABI: eq_silu_mul)."""
    _bf16(gate, "gate")
    _bf16(up, "up")
    out = torch.empty_like(gate)
    check(_native.lib().eq_silu_mul(out.data_ptr(), gate.data_ptr(), up.data_ptr(), gate.numel(),
                                    _native.EQ_DTYPE_BF16, _stream()))
    return out


def embedding(table: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
    """Rows of a bf16 table by int32 device token ids (C ABI: eq_embedding)."""
    _bf16(table, "table")
    if tokens.dtype != torch.int32 or not tokens.is_cuda:
        raise _native.EreduError("tokens must be an int32 CUDA tensor")
    out = torch.empty((tokens.numel(), table.shape[1]), dtype=torch.bfloat16, device=table.device)
    check(_native.lib().eq_embedding(out.data_ptr(), table.data_ptr(), tokens.data_ptr(), tokens.numel(),
                                     table.shape[0], table.shape[1], _native.EQ_DTYPE_BF16, _stream()))
    return out


def argmax(logits: torch.Tensor) -> torch.Tensor:
    """First index of the largest value per row, int32 (C ABI: eq_argmax)."""
    _bf16(logits, "logits")
    n = logits.shape[-1]
    out = torch.empty((logits.numel() // n,), dtype=torch.int32, device=logits.device)
    check(_native.lib().eq_argmax(out.data_ptr(), logits.data_ptr(), logits.numel() // n, n,
                                  _native.EQ_DTYPE_BF16, _stream()))
    return out


@dataclass
class QLinear:
    """A packed projection W [N, K] (transpose = true): codes int32/uint32
    [N, K * bits / 32], bf16 scales and biases [N, K / group_size]."""

    w: torch.Tensor
    scales: torch.Tensor
    biases: Optional[torch.Tensor]
    bits: int = 4
    group_size: int = 64

    @property
    def N(self) -> int:
        return self.w.shape[0]

    @property
    def K(self) -> int:
        return self.w.shape[1] * 32 // self.bits


def interleave_gate_up(gate: QLinear, up: QLinear) -> QLinear:
    """The gate and up projections as one packed matrix [2F, K] in
    eq_quantized_matmul_swiglu's layout: rows 16t .. 16t + 7 are gate rows
    8t .. 8t + 7, rows 16t + 8 .. 16t + 15 up rows 8t .. 8t + 7 (codes, scales
    and biases moved row by row; a copy on the device)."""
    if (gate.N != up.N or gate.K != up.K or gate.bits != up.bits or gate.group_size != up.group_size or
            (gate.biases is None) != (up.biases is None) or gate.N % 8 != 0):
        raise _native.EreduError("gate and up must share shape, bits, group size and bias presence, N % 8 == 0")

    def il(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        F = a.shape[0]
        return torch.stack((a.reshape(F // 8, 8, -1), b.reshape(F // 8, 8, -1)), dim=1).reshape(2 * F, -1).contiguous()

    return QLinear(il(gate.w, up.w), il(gate.scales, up.scales),
                   il(gate.biases, up.biases) if gate.biases is not None else None, gate.bits, gate.group_size)


def gate_up_swiglu(x: torch.Tensor, gate_up: QLinear, prologue=None) -> torch.Tensor:
    """silu(x . Wg^T) * (x . Wu^T) for one bf16 row x [K], gate_up from
    interleave_gate_up (C ABI: eq_quantized_matmul_swiglu); prologue: an
    _native.ActivationPrologue (RMS_NORM) or None."""
    _bf16(x, "x")
    F = gate_up.N // 2
    out = torch.empty((F,), dtype=torch.bfloat16, device=x.device)
    n = _native
    check(n.lib().eq_quantized_matmul_swiglu(
        out.data_ptr(), x.data_ptr(), gate_up.w.data_ptr(), gate_up.scales.data_ptr(),
        gate_up.biases.data_ptr() if gate_up.biases is not None else None, F, gate_up.K, gate_up.group_size,
        gate_up.bits, b"affine", n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16,
        ctypes.byref(prologue) if prologue is not None else None, _stream()))
    return out


@dataclass
class DecoderLayer:
    in_norm: torch.Tensor
    post_norm: torch.Tensor
    q: QLinear
    k: QLinear
    v: QLinear
    o: QLinear
    gate: QLinear
    up: QLinear
    down: QLinear


class LlamaDecoder:
    """Batch-1 greedy decode of a Llama-shaped model.  ``step(pos)`` embeds the
    token in ``self.token``, runs every layer with the cache row ``pos`` as the
    new position, and writes the argmax of the logits back into ``self.token``.
    ``step_device()`` does the same at the position held in ``self.position``
    (int32 device memory, set with ``set_position``) and then advances it by
    one, so that replays of one captured graph decode successive tokens.  Both
    enqueue on the current stream and allocate nothing.

    ``fused`` (default: when the shapes allow it) folds each residual add +
    RMSNorm into the launch of the projections that consume it
    (eq_quantized_matmul_batched_prologue), and SiLU-mul into the gate/up
    launch (eq_quantized_matmul_swiglu, on an interleaved copy of each
    layer's gate and up matrices made at construction; into the down
    projection's launch instead when K is not a whole number of the decode
    kernel's code blocks): 6 launches per layer instead of 9.  The hidden
    state then alternates between two buffers (every workgroup of a launch
    reads the old one)."""

    def __init__(self, layers: Sequence[DecoderLayer], embed: torch.Tensor, final_norm: torch.Tensor,
                 lm_head: QLinear, *, n_heads: int, n_kv_heads: int, eps: float, freqs: np.ndarray, max_seq: int,
                 k_caches: Optional[List[torch.Tensor]] = None, v_caches: Optional[List[torch.Tensor]] = None,
                 fused: Optional[bool] = None):
        dev = embed.device
        self.layers = list(layers)
        self.embed, self.final_norm, self.lm_head = embed, final_norm, lm_head
        self.n_heads, self.n_kv_heads, self.eps, self.max_seq = n_heads, n_kv_heads, float(eps), max_seq
        self.hidden = embed.shape[1]
        self.vocab = embed.shape[0]
        self.scale = 1.0 / math.sqrt(HEAD_DIM)
        self.freqs = torch.from_numpy(np.ascontiguousarray(freqs, dtype=np.float32)).to(dev)
        L0 = self.layers[0]
        self.ffn = L0.gate.N
        H, bf = self.hidden, torch.bfloat16
        if n_heads * HEAD_DIM != L0.q.N or n_kv_heads * HEAD_DIM != L0.k.N or L0.q.K != H:
            raise _native.EreduError("projection shapes do not match the head geometry")
        cache_shape = (n_kv_heads, max_seq, HEAD_DIM)
        self.k_caches = k_caches if k_caches is not None else [torch.zeros(cache_shape, dtype=bf, device=dev)
                                                                for _ in self.layers]
        self.v_caches = v_caches if v_caches is not None else [torch.zeros(cache_shape, dtype=bf, device=dev)
                                                                for _ in self.layers]
        e = lambda n: torch.empty((n,), dtype=bf, device=dev)
        self.x, self.h = e(H), e(H)
        self.q, self.k, self.v = e(L0.q.N), e(L0.k.N), e(L0.v.N)
        self.att, self.o = e(L0.q.N), e(H)
        self.gate, self.up, self.act, self.down = e(self.ffn), e(self.ffn), e(self.ffn), e(H)
        self.logits = e(lm_head.N)
        self.token = torch.zeros((1,), dtype=torch.int32, device=dev)
        self.position = torch.zeros((1,), dtype=torch.int32, device=dev)
        lins = [getattr(Lr, p) for Lr in self.layers for p in ("q", "k", "v", "o", "gate", "up", "down")]
        can_fuse = (H <= 4096 and H % 64 == 0 and self.ffn % 64 == 0 and lm_head.N % 16 == 0 and
                    all(l.group_size == 64 and l.bits in (4, 8) and l.N % 16 == 0 and l.scales.dtype == torch.bfloat16
                        for l in lins + [lm_head]))
        self.fused = can_fuse if fused is None else bool(fused)
        if self.fused and not can_fuse:
            raise _native.EreduError("fused decode needs hidden <= 4096, group size 64, 4/8-bit codes, bf16 scales")
        self.x2 = e(H)  # the hidden state's second buffer (fused mode)
        self.swiglu = False  # (fused mode: SiLU-mul in the gate/up launch)
        # grouped problems (pointers fixed for the decoder's lifetime)
        n = _native
        self._qkv, self._gu = [], []
        for Lr in self.layers:
            qkv = (n.QmmProblem * 3)()
            for i, (lin, y) in enumerate(((Lr.q, self.q), (Lr.k, self.k), (Lr.v, self.v))):
                qkv[i] = self._problem(lin, self.h, y)
            gu = (n.QmmProblem * 2)()
            for i, (lin, y) in enumerate(((Lr.gate, self.gate), (Lr.up, self.up))):
                gu[i] = self._problem(lin, self.h, y)
            self._qkv.append(qkv)
            self._gu.append(gu)
        if self.fused:
            # layer 0 reads the embedding row in x; afterwards q/k/v read x2
            # (writing x) and gate/up read x (writing x2)
            self._fqkv, self._fgu, self._fdown, self._pro_in, self._pro_post = [], [], [], [], []
            for li, Lr in enumerate(self.layers):
                src = self.x if li == 0 else self.x2
                qkv = (n.QmmProblem * 3)()
                for i, (lin, y) in enumerate(((Lr.q, self.q), (Lr.k, self.k), (Lr.v, self.v))):
                    qkv[i] = self._problem(lin, src, y)
                gu = (n.QmmProblem * 2)()
                for i, (lin, y) in enumerate(((Lr.gate, self.gate), (Lr.up, self.up))):
                    gu[i] = self._problem(lin, self.x, y)
                down = (n.QmmProblem * 1)()
                down[0] = self._problem(Lr.down, self.gate, self.down)
                pin = n.ActivationPrologue(n.EQ_PROLOGUE_RMS_NORM, self.down.data_ptr() if li else None,
                                           Lr.in_norm.data_ptr(), self.x.data_ptr() if li else None, self.eps)
                ppost = n.ActivationPrologue(n.EQ_PROLOGUE_RMS_NORM, self.o.data_ptr(), Lr.post_norm.data_ptr(),
                                             self.x2.data_ptr(), self.eps)
                self._fqkv.append(qkv)
                self._fgu.append(gu)
                self._fdown.append(down)
                self._pro_in.append(pin)
                self._pro_post.append(ppost)
            self._pro_silu = n.ActivationPrologue(n.EQ_PROLOGUE_SILU_MUL, self.up.data_ptr(), None, None, 0.0)
            # SwiGLU in the gate/up launch: K a whole number of code blocks
            # (512 values at 4 bits, 256 at 8) and F % 8 == 0
            self.swiglu = all(Lr.gate.K % (512 if Lr.gate.bits == 4 else 256) == 0 and Lr.gate.N % 8 == 0 and
                              Lr.gate.bits == Lr.up.bits and (Lr.gate.biases is None) == (Lr.up.biases is None)
                              for Lr in self.layers)
            self._gu_il = [interleave_gate_up(Lr.gate, Lr.up) for Lr in self.layers] if self.swiglu else []
            self._flm = (n.QmmProblem * 1)()
            self._flm[0] = self._problem(lm_head, self.x2, self.logits)
            self._pro_final = n.ActivationPrologue(n.EQ_PROLOGUE_RMS_NORM, self.down.data_ptr(),
                                                   final_norm.data_ptr(), None, self.eps)

    @staticmethod
    def _problem(lin: QLinear, x: torch.Tensor, y: torch.Tensor):
        return _native.QmmProblem(y.data_ptr(), x.data_ptr(), lin.w.data_ptr(), lin.scales.data_ptr(),
                                  lin.biases.data_ptr() if lin.biases is not None else None, lin.N, lin.K)

    def _group(self, probs, count: int, lin: QLinear, st: int) -> None:
        n = _native
        check(n.lib().eq_quantized_matmul_batched(probs, count, 1, True, lin.group_size, lin.bits, b"affine",
                                                  n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, st))

    def _linear(self, lin: QLinear, x: torch.Tensor, y: torch.Tensor, st: int) -> None:
        n = _native
        check(n.lib().eq_quantized_matmul(
            y.data_ptr(), x.data_ptr(), lin.w.data_ptr(), lin.scales.data_ptr(),
            lin.biases.data_ptr() if lin.biases is not None else None, 1, lin.N, lin.K, True, lin.group_size,
            lin.bits, b"affine", n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, st))

    def launches_per_step(self, device_position: bool = False) -> int:
        # embedding; per layer 2 norms, 4 projection launches, attention (2
        # kernels), silu_mul; final norm, LM head, argmax, and the position
        # advance of step_device (fused: the norms and silu_mul ride in the
        # projections' launches)
        per_layer = 6 if self.fused else 9
        tail = (2 if self.fused else 3) + (1 if device_position else 0)
        return 1 + len(self.layers) * per_layer + tail

    def _pro(self, probs, count: int, lin: QLinear, pro, st: int) -> None:
        n = _native
        check(n.lib().eq_quantized_matmul_batched_prologue(probs, count, 1, True, lin.group_size, lin.bits, b"affine",
                                                           n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, ctypes.byref(pro), st))

    def _attend(self, li: int, pos: Optional[int], st: int) -> None:
        """Layer li's attention at ``pos``, or at the device position when None."""
        n, L = _native, _native.lib()
        if pos is None:
            check(L.eq_rope_attention_decode_at(
                self.att.data_ptr(), self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                self.k_caches[li].data_ptr(), self.v_caches[li].data_ptr(), self.freqs.data_ptr(),
                self.position.data_ptr(), self.max_seq, self.n_heads, self.n_kv_heads, HEAD_DIM, self.scale,
                n.EQ_DTYPE_BF16, st))
        else:
            check(L.eq_rope_attention_decode(
                self.att.data_ptr(), self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                self.k_caches[li].data_ptr(), self.v_caches[li].data_ptr(), self.freqs.data_ptr(), pos, self.max_seq,
                self.n_heads, self.n_kv_heads, HEAD_DIM, self.scale, n.EQ_DTYPE_BF16, st))

    def set_position(self, pos: int) -> None:
        """Writes the device position that ``step_device`` decodes next (a copy
        on the current stream; not inside a capture)."""
        if not 0 <= pos < self.max_seq:
            raise _native.EreduError(f"position {pos} outside the cache of {self.max_seq}")
        self.position.fill_(int(pos))

    def step_device(self) -> None:
        """One step at the device position, then position += 1 (one launch).  A
        position that reaches max_seq makes attention write no cache row and
        return zeros; the caller stops before that, as it would with step()."""
        st = _stream()
        if self.fused:
            self._step_fused(None, st)
        else:
            self._step_unfused(None, st)
        check(_native.lib().eq_advance_position(self.position.data_ptr(), st))

    def _step_fused(self, pos: Optional[int], st: int) -> None:
        n, L = _native, _native.lib()
        bf = n.EQ_DTYPE_BF16
        check(L.eq_embedding(self.x.data_ptr(), self.embed.data_ptr(), self.token.data_ptr(), 1, self.vocab,
                             self.hidden, bf, st))
        for li, Lr in enumerate(self.layers):
            self._pro(self._fqkv[li], 3, Lr.q, self._pro_in[li], st)
            self._attend(li, pos, st)
            self._linear(Lr.o, self.att, self.o, st)
            if self.swiglu:
                gu = self._gu_il[li]
                check(L.eq_quantized_matmul_swiglu(
                    self.act.data_ptr(), self.x.data_ptr(), gu.w.data_ptr(), gu.scales.data_ptr(),
                    gu.biases.data_ptr() if gu.biases is not None else None, self.ffn, gu.K, gu.group_size, gu.bits,
                    b"affine", bf, bf, ctypes.byref(self._pro_post[li]), st))
                self._linear(Lr.down, self.act, self.down, st)
            else:
                self._pro(self._fgu[li], 2, Lr.gate, self._pro_post[li], st)
                self._pro(self._fdown[li], 1, Lr.down, self._pro_silu, st)
        self._pro(self._flm, 1, self.lm_head, self._pro_final, st)
        check(L.eq_argmax(self.token.data_ptr(), self.logits.data_ptr(), 1, self.lm_head.N, bf, st))

    def step(self, pos: int) -> None:
        if not 0 <= pos < self.max_seq:
            raise _native.EreduError(f"position {pos} outside the cache of {self.max_seq}")
        st = _stream()
        if self.fused:
            self._step_fused(pos, st)
        else:
            self._step_unfused(pos, st)

    def _step_unfused(self, pos: Optional[int], st: int) -> None:
        n, L = _native, _native.lib()
        bf = n.EQ_DTYPE_BF16
        H, F = self.hidden, self.ffn
        check(L.eq_embedding(self.x.data_ptr(), self.embed.data_ptr(), self.token.data_ptr(), 1, self.vocab, H, bf,
                             st))
        resid = None
        for li, Lr in enumerate(self.layers):
            check(L.eq_rms_norm(self.h.data_ptr(), self.x.data_ptr(), resid, Lr.in_norm.data_ptr(), 1, H, self.eps,
                                bf, st))
            self._group(self._qkv[li], 3, Lr.q, st)
            self._attend(li, pos, st)
            self._linear(Lr.o, self.att, self.o, st)
            check(L.eq_rms_norm(self.h.data_ptr(), self.x.data_ptr(), self.o.data_ptr(), Lr.post_norm.data_ptr(), 1,
                                H, self.eps, bf, st))
            self._group(self._gu[li], 2, Lr.gate, st)
            check(L.eq_silu_mul(self.act.data_ptr(), self.gate.data_ptr(), self.up.data_ptr(), F, bf, st))
            self._linear(Lr.down, self.act, self.down, st)
            resid = self.down.data_ptr()
        check(L.eq_rms_norm(self.h.data_ptr(), self.x.data_ptr(), resid, self.final_norm.data_ptr(), 1, H, self.eps,
                            bf, st))
        self._linear(self.lm_head, self.h, self.logits, st)
        check(L.eq_argmax(self.token.data_ptr(), self.logits.data_ptr(), 1, self.lm_head.N, bf, st))

    def bytes_per_step(self, pos: int) -> int:
        """Algorithmic bytes of one step: packed projections (codes, scales,
        biases, input and output vectors), the KV rows read and written,
        norms, the embedding row and the logits."""
        def lin_bytes(l: QLinear) -> int:
            nb = 2 if l.biases is not None else 1
            return l.N * l.K * l.bits // 8 + nb * 2 * l.N * (l.K // l.group_size) + 2 * l.K + 2 * l.N

        total = sum(lin_bytes(getattr(Lr, p)) for Lr in self.layers
                    for p in ("q", "k", "v", "o", "gate", "up", "down"))
        total += lin_bytes(self.lm_head)
        kv = 2 * self.n_kv_heads * HEAD_DIM * 2  # one row of K and of V
        total += len(self.layers) * (kv * (pos + 1) + kv)  # rows 0..pos read, row pos written
        total += len(self.layers) * 2 * self.hidden * 2 + self.hidden * 2  # norm weights
        total += self.hidden * 2  # embedding row
        return total

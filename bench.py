"""Benchmark of the quantized-linear hot path on one MI355X.

Headline workload (BASELINE.json configs[1] at M = 1): one step is the
decode-time projections of a Llama-3-8B-shaped stack -- q, k, v, o, gate, up,
down (N x K = 4096x4096, 1024x4096, 1024x4096, 4096x4096, 14336x4096,
14336x4096, 4096x14336) for each of 32 layers: 224 quantized matmuls at M = 1
with 4-bit, group-64 weights and bf16 activations/scales/biases.  Every layer
has its own weights (3.93 GB in HBM), so the 256 MB Infinity Cache cannot
serve repeats.  The projections are issued the way a decode step can issue
them -- one grouped launch (eq_quantized_matmul_batched) for each set that
shares an input: {q, k, v}, {o}, {gate, up}, {down}, i.e. 128 launches per
step -- captured once as a HIP graph and replayed; inputs are resident in HBM
before the timed region starts.

value = algorithmic bytes of the step / step time, in GB/s
(bytes per linear: N*K/2 packed codes + 4*N*K/64 scale+bias + 2*M*K + 2*M*N).

Also reported (not the headline): the same step with one launch per
projection (the drop-in eq_quantized_matmul path) and with all seven
projections of a layer in one launch, M = 8, per-shape qmv, prefill qmm
TFLOP/s, GGUF dequant/convert GB/s, the MXFP4
mode (decode, prefill, routed experts, codec, GGUF type 39), the roofline
record of the dominant kernel (qmv_lds_kernel) and the CPU baseline (the
restated MLX CPU qmm loop of oracle/, timed on this host).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
LAYERS = 32
HIDDEN, FFN, KV = 4096, 14336, 1024
LAYER_SHAPES = [  # (name, N, K)
    ("q", HIDDEN, HIDDEN), ("k", KV, HIDDEN), ("v", KV, HIDDEN), ("o", HIDDEN, HIDDEN),
    ("gate", FFN, HIDDEN), ("up", FFN, HIDDEN), ("down", HIDDEN, FFN),
]
DECODE_GROUPS = [["q", "k", "v"], ["o"], ["gate", "up"], ["down"]]  # sets sharing an input
ALL7 = [["q", "k", "v", "o", "gate", "up", "down"]]
GS, BITS = 64, 4
# Every timed buffer set rotates at least this many distinct bytes, so that the
# 256 MB Infinity Cache cannot serve a repeat from cache.
ROTATE_BYTES = 300_000_000


def rotation(bytes_per_copy, minimum=2):
    """Copies of a buffer set needed to rotate ROTATE_BYTES."""
    return max(minimum, -(-ROTATE_BYTES // int(bytes_per_copy)))


def qmv_bytes(M, N, K, bits=BITS, gs=GS):
    return N * K * bits // 8 + 2 * 2 * N * (K // gs) + 2 * M * K + 2 * M * N


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Linear:
    """One layer's packed weight on the GPU (random codes; bf16 scales/biases of
    the magnitude a N(0, 0.02) weight quantizes to)."""

    def __init__(self, N, K, gen, bits=BITS, gs=GS):
        import torch

        self.N, self.K = N, K
        self.w = torch.randint(-(2**31), 2**31 - 1, (N, K * bits // 32), dtype=torch.int32, device="cuda",
                               generator=gen)
        self.s = (torch.rand((N, K // gs), device="cuda", generator=gen) * 0.004 + 0.004).to(torch.bfloat16)
        self.b = (-7.5 * self.s.float()).to(torch.bfloat16)


class Timer:
    """Replays a captured HIP graph on its own stream and times each replay
    with HIP events recorded on that same stream; a replay's time is the
    median over the timed replays (the mean is kept in ``last_mean_ms``)."""

    def __init__(self, fn):
        import torch

        self.stream = torch.cuda.Stream()
        self.graph = torch.cuda.CUDAGraph()
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self.stream):
            fn(self.stream.cuda_stream)  # warm once outside capture
            torch.cuda.synchronize()
            with torch.cuda.graph(self.graph, stream=self.stream):
                fn(self.stream.cuda_stream)
        torch.cuda.synchronize()

    def ms_per_replay(self, steps, warmup):
        import torch

        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                self.graph.replay()
            torch.cuda.synchronize()
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
            ev[0].record(self.stream)
            for i in range(steps):
                self.graph.replay()
                ev[i + 1].record(self.stream)
        torch.cuda.synchronize()
        times = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
        self.last_mean_ms = ev[0].elapsed_time(ev[-1]) / steps
        return float(np.median(times))


def _lib():
    from eredu_amd import _native

    return _native


def _dtype_code(t):
    import torch

    n = _lib()
    return n.EQ_DTYPE_F16 if t.dtype == torch.float16 else n.EQ_DTYPE_BF16


def run_one(lin, x, y, stream, bits=BITS, gs=GS):
    """One eq_quantized_matmul; activation and scale types from the tensors
    (bf16 or f16)."""
    n = _lib()
    n.check(n.lib().eq_quantized_matmul(
        y.data_ptr(), x.data_ptr(), lin.w.data_ptr(), lin.s.data_ptr(), lin.b.data_ptr(), x.shape[0], lin.N, lin.K,
        True, gs, bits, b"affine", _dtype_code(x), _dtype_code(lin.s), stream))


def run_group(lins, xs, ys, stream, bits=BITS, gs=GS):
    n = _lib()
    arr = (n.QmmProblem * len(lins))()
    for i, (lin, x, y) in enumerate(zip(lins, xs, ys)):
        arr[i] = n.QmmProblem(y.data_ptr(), x.data_ptr(), lin.w.data_ptr(), lin.s.data_ptr(), lin.b.data_ptr(),
                              lin.N, lin.K)
    n.check(n.lib().eq_quantized_matmul_batched(arr, len(lins), xs[0].shape[0], True, gs, bits, b"affine",
                                                _dtype_code(xs[0]), _dtype_code(lins[0].s), stream))


def decode_step_fn(layers, M, groups, act_dtype=None):
    """Step of all layers' projections at batch M; groups=None issues one launch per
    projection, else one grouped launch per listed set.  Returns (fn, launches)."""
    import torch

    dt = torch.bfloat16 if act_dtype is None else act_dtype
    xs = {K: torch.randn((M, K), device="cuda").to(dt) for K in (HIDDEN, FFN)}
    ys = {name: torch.empty((M, N), device="cuda", dtype=dt) for name, N, K in LAYER_SHAPES}
    Ks = {name: K for name, N, K in LAYER_SHAPES}

    def step(stream):
        for layer in layers:
            if groups is None:
                for name, _, K in LAYER_SHAPES:
                    run_one(layer[name], xs[K], ys[name], stream)
            else:
                for g in groups:
                    run_group([layer[n] for n in g], [xs[Ks[n]] for n in g], [ys[n] for n in g], stream)

    launches = len(layers) * (len(LAYER_SHAPES) if groups is None else len(groups))
    return step, launches


def bench_decode(layers, M, groups, steps, warmup, act_dtype=None):
    step, launches = decode_step_fn(layers, M, groups, act_dtype)
    ms = Timer(step).ms_per_replay(steps, warmup)
    nbytes = len(layers) * sum(qmv_bytes(M, N, K) for _, N, K in LAYER_SHAPES)
    return ms, nbytes, launches


def bench_per_shape(layers, M, steps, warmup):
    """One eq_quantized_matmul launch per call, per distinct Llama shape; the
    layers' weights rotate, topped up with more copies of a shape whose 32
    layers hold less than ROTATE_BYTES (k/v)."""
    import torch

    out = {}
    gen = torch.Generator(device="cuda").manual_seed(7)
    for name, N, K in LAYER_SHAPES:
        if name in ("v", "up", "o"):
            continue  # same shapes as k, gate, q
        lins = [layer[name] for layer in layers]
        extra = rotation(qmv_bytes(M, N, K), len(lins)) - len(lins)
        lins += [Linear(N, K, gen) for _ in range(extra)]
        x = torch.randn((M, K), device="cuda").to(torch.bfloat16)
        y = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
        t = Timer(lambda st: [run_one(lin, x, y, st) for lin in lins])
        us = t.ms_per_replay(max(steps // 2, 10), warmup) * 1e3 / len(lins)
        gbs = qmv_bytes(M, N, K) / (us * 1e-6) / 1e9
        out[f"{N}x{K}"] = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                           "copies": len(lins)}
        del lins
        torch.cuda.empty_cache()
    return out


def bench_qmm(steps, warmup, bits_list=(4, 8), Ms=(128, 512, 2048)):
    """Prefill qmm TFLOP/s at the Llama shapes; the weights rotate
    over at least ROTATE_BYTES (and at least 4 copies)."""
    import torch

    gen = torch.Generator(device="cuda").manual_seed(1)
    out = {}
    for bits in bits_list:
        for (name, N, K) in [("q/o", HIDDEN, HIDDEN), ("k/v", KV, HIDDEN), ("gate/up", FFN, HIDDEN),
                             ("down", HIDDEN, FFN)]:
            lins = [Linear(N, K, gen, bits=bits) for _ in range(rotation(qmv_bytes(0, N, K, bits), 4))]
            for M in Ms:
                x = torch.randn((M, K), device="cuda").to(torch.bfloat16)
                y = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
                t = Timer(lambda st: [run_one(l, x, y, st, bits=bits) for l in lins])
                ms = t.ms_per_replay(max(steps // 4, 5), warmup) / len(lins)
                tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
                out[f"b{bits} M{M} {N}x{K}"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tflops, 1),
                                                "frac_mfma": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4)}
            del lins
            torch.cuda.empty_cache()
    return out


class F16View:
    """A layer's packed codes with its scales and biases as f16 (an f16 model's
    parameters), for the f16-activation figures."""

    def __init__(self, lin):
        import torch

        self.N, self.K, self.w = lin.N, lin.K, lin.w
        self.s, self.b = lin.s.to(torch.float16), lin.b.to(torch.float16)


def bench_f16(layers, steps, warmup):
    """f16 activations with f16 scales/biases on the same kernels as bf16: the
    grouped decode step at M = 1 and 8 over the 32 layers' codes,
    and prefill qmm at M = 512 for the four shapes (configs[2], 4-bit g64)."""
    import torch

    out = {}
    f16layers = [{name: F16View(L[name]) for name, _, _ in LAYER_SHAPES} for L in layers]
    for M in (1, 8):
        ms, nb, launches = bench_decode(f16layers, M, DECODE_GROUPS, max(steps // 2, 5), warmup, torch.float16)
        out[f"decode_M{M}_grouped"] = {"ms": round(ms, 4), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                                       "launches": launches}
    del f16layers
    torch.cuda.empty_cache()
    gen = torch.Generator(device="cuda").manual_seed(5)
    M = 512
    for (name, N, K) in [("q/o", HIDDEN, HIDDEN), ("k/v", KV, HIDDEN), ("gate/up", FFN, HIDDEN), ("down", HIDDEN, FFN)]:
        lins = [F16View(Linear(N, K, gen)) for _ in range(rotation(qmv_bytes(0, N, K), 4))]
        x = torch.randn((M, K), device="cuda").to(torch.float16)
        y = torch.empty((M, N), device="cuda", dtype=torch.float16)
        t = Timer(lambda st: [run_one(l, x, y, st) for l in lins])
        ms = t.ms_per_replay(max(steps // 4, 5), warmup) / len(lins)
        tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        out[f"qmm M{M} {N}x{K}"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tflops, 1),
                                    "frac_mfma": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4)}
        del lins
        torch.cuda.empty_cache()
    return out


def bench_qmm_widths(steps, warmup, M=512):
    """Prefill TFLOP/s at the other code widths and group size 16 (the widths
    GGUF k-quants convert to and MLX-LM admits): 2/3/5/6-bit codes go through
    the byte re-pack and the 8-bit matrix-core kernel, 4/8-bit g16 straight to
    it; q/o and gate/up shapes at M = 512, weights rotating as in bench_qmm."""
    import torch

    gen = torch.Generator(device="cuda").manual_seed(2)
    out = {}
    for bits, gs in ((2, 16), (3, 16), (5, 32), (6, 16), (4, 16), (8, 16)):
        for (name, N, K) in [("q/o", HIDDEN, HIDDEN), ("gate/up", FFN, HIDDEN)]:
            lins = [Linear(N, K, gen, bits=bits, gs=gs) for _ in range(rotation(qmv_bytes(0, N, K, bits, gs), 4))]
            x = torch.randn((M, K), device="cuda").to(torch.bfloat16)
            y = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
            t = Timer(lambda st: [run_one(l, x, y, st, bits=bits, gs=gs) for l in lins])
            ms = t.ms_per_replay(max(steps // 4, 5), warmup) / len(lins)
            tflops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
            out[f"b{bits} g{gs} M{M} {N}x{K}"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tflops, 1),
                                                  "frac_mfma": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4)}
            del lins
            torch.cuda.empty_cache()
    return out


def lin_m(n, ty, y, x, raws, nraw, M, rows, cols):
    """One eq_gguf_linear per payload copy: y [M, rows] = x [M, cols] . W^T."""
    def lin(st):
        for r in raws:
            n.check(n.lib().eq_gguf_linear(y.data_ptr(), x.data_ptr(), r.data_ptr(), nraw, int(ty), M, rows, cols, 0,
                                           n.EQ_DTYPE_BF16, st))
    return lin


def bench_gguf(steps, warmup):
    """GGUF 4096x14336 dequant (bf16) and convert (affine) GB/s,
    for every block type with an affine form (Q4_0 / Q8_0 / Q4_K first, the
    configs' types), and dequant for IQ4_NL / IQ4_XS; the native linear at
    M = 1 (GB/s) and M = 512 (TFLOP/s, the matrix-core prefill) for the
    natively executed types."""
    import torch

    from eredu_amd import gguf as G

    n = _lib()
    rows, cols = 4096, 14336
    out = {}
    T = G.GgmlType
    for ty in (T.Q4_0, T.Q8_0, T.Q4K, T.Q4_1, T.Q5_0, T.Q5_1, T.Q2K, T.Q3K, T.Q5K, T.Q6K, T.IQ4NL, T.IQ4XS):
        vals, nbytes = ty.block_and_bytes()
        nraw = rows * cols // vals * nbytes
        affine = G.affine_config(ty) is not None  # (the IQ4 types have none: dequant and linear only)
        bits, gs = G.affine_config(ty) if affine else (4, 32)
        conv_bytes = rows * cols * bits // 8 + 2 * 2 * rows * (cols // gs)
        # each copy is a distinct input and its own output, rotating >= ROTATE_BYTES
        copies = rotation(nraw + rows * cols * 2)
        raws = [torch.randint(0, 256, (nraw,), dtype=torch.uint8, device="cuda") for _ in range(rotation(nraw))]
        dense = [torch.empty((rows, cols), dtype=torch.bfloat16, device="cuda") for _ in range(copies)]
        cc = rotation(nraw + conv_bytes) if affine else 0
        aw = [torch.empty((rows, cols * bits // 32), dtype=torch.int32, device="cuda") for _ in range(cc)]
        asb = [torch.empty((rows, cols // gs), dtype=torch.float16, device="cuda") for _ in range(cc)]
        abb = [torch.empty((rows, cols // gs), dtype=torch.float16, device="cuda") for _ in range(cc)]

        def deq(st):
            for i in range(copies):
                n.check(n.lib().eq_gguf_dequantize(dense[i].data_ptr(), raws[i].data_ptr(), nraw, int(ty), rows, cols,
                                                   0, n.EQ_DEQUANT_AFFINE, n.EQ_DTYPE_BF16, st))

        def conv(st):
            for i in range(cc):
                n.check(n.lib().eq_gguf_convert_affine(aw[i].data_ptr(), asb[i].data_ptr(), abb[i].data_ptr(),
                                                       raws[i].data_ptr(), nraw, int(ty), rows, cols, 0, st))

        legs = [("dequant_bf16", deq, rows * cols * 2, copies)]
        if affine:
            legs.append((f"convert_affine_g{gs}", conv, conv_bytes, cc))
        for label, fn, out_bytes, k in legs:
            ms = Timer(fn).ms_per_replay(max(steps // 4, 5), warmup) / k
            gbs = (nraw + out_bytes) / (ms * 1e-3) / 1e9
            out[f"{ty.name} {label}"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                         "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "copies": k}
        del dense, aw, asb, abb
        if ty.has_device_linear():
            # batch-1 linear straight from the blocks: y [1, 4096] = x [1, 14336] . W^T
            x = torch.randn((1, cols), device="cuda").to(torch.bfloat16)
            y = torch.empty((1, rows), dtype=torch.bfloat16, device="cuda")
            ms = Timer(lin_m(n, ty, y, x, raws, nraw, 1, rows, cols)).ms_per_replay(max(steps // 4, 5), warmup)
            ms /= len(raws)
            gbs = (nraw + cols * 2 + rows * 2) / (ms * 1e-3) / 1e9
            out[f"{ty.name} linear_M1"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                           "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "copies": len(raws)}
            # prefill: 512 activation rows, through the matrix cores (blocks re-packed per call)
            M = 512
            x = torch.randn((M, cols), device="cuda").to(torch.bfloat16)
            y = torch.empty((M, rows), dtype=torch.bfloat16, device="cuda")
            ms = Timer(lin_m(n, ty, y, x, raws, nraw, M, rows, cols)).ms_per_replay(max(steps // 4, 5), warmup)
            ms /= len(raws)
            tf = 2.0 * M * rows * cols / (ms * 1e-3) / 1e12
            out[f"{ty.name} linear_M{M}"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1),
                                             "frac_mfma": round(tf / BF16_MFMA_PEAK_TFLOPS, 4), "copies": len(raws)}
            del x, y
        del raws
        torch.cuda.empty_cache()
    return out


def bench_gguf_embedding(steps, warmup):
    """Native GGUF embedding (eq_gguf_embedding): rows of a 128256 x 4096
    token table (Llama-3's vocabulary) in Q6_K and Q4_K blocks, f32 out, for
    1 token (decode) and 512 tokens (prefill); tables rotate >= 300 MB.
    GB/s over the picked rows' blocks read plus the f32 rows written."""
    import torch

    from eredu_amd.gguf import GgmlType as T

    n = _lib()
    out = {}
    rows, cols = 128256, 4096
    for ty in (T.Q6K, T.Q4K):
        vals, nbytes = ty.block_and_bytes()
        nraw = rows * cols // vals * nbytes
        row_bytes = cols // vals * nbytes
        tables = [torch.randint(0, 256, (nraw,), dtype=torch.uint8, device="cuda") for _ in range(rotation(nraw))]
        for label, count in (("1_token", 1), ("512_tokens", 512)):
            ids = torch.randint(0, rows, (count,), device="cuda", dtype=torch.int32)
            y = torch.empty((count, cols), dtype=torch.float32, device="cuda")

            def call(st):
                for t in tables:
                    n.check(n.lib().eq_gguf_embedding(y.data_ptr(), t.data_ptr(), nraw, int(ty), rows, cols,
                                                      ids.data_ptr(), count, 0, n.EQ_DTYPE_F32, st))

            ms = Timer(call).ms_per_replay(max(steps // 4, 5), warmup) / len(tables)
            gbs = count * (row_bytes + cols * 4) / (ms * 1e-3) / 1e9
            out[f"{ty.name} {label}"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "copies": len(tables)}
        del tables
        torch.cuda.empty_cache()
    return out


def bench_gguf_grouped(steps, warmup):
    """Native GGUF mixture-of-experts linear (eq_gguf_grouped_linear): an
    expert bank of 8 x 14336 x 4096 (Mixtral's gate projection shape) in
    Q4_K and Q6_K blocks; decode = 2 routes (top-2 of one token), prefill =
    1024 routes (512 tokens x top-2, sorted ids).  Banks rotate >= 300 MB."""
    import torch

    n = _lib()
    out = {}
    from eredu_amd.gguf import GgmlType as T
    experts, N, K = 8, 14336, 4096
    for ty in (T.Q4K, T.Q6K):
        vals, nbytes = ty.block_and_bytes()
        nraw = experts * N * K // vals * nbytes
        banks = [torch.randint(0, 256, (nraw,), dtype=torch.uint8, device="cuda") for _ in range(rotation(nraw))]
        for label, routes in (("decode_2routes", 2), ("prefill_1024routes", 1024)):
            ids = torch.sort(torch.randint(0, experts, (routes,), device="cuda", dtype=torch.int32)).values
            x = torch.randn((routes, K), device="cuda").to(torch.bfloat16)
            y = torch.empty((routes, N), dtype=torch.bfloat16, device="cuda")

            def call(st):
                for bnk in banks:
                    n.check(n.lib().eq_gguf_grouped_linear(y.data_ptr(), x.data_ptr(), bnk.data_ptr(), nraw, int(ty),
                                                           experts, N, K, ids.data_ptr(), routes, 0,
                                                           n.EQ_DTYPE_BF16, True, st))

            ms = Timer(call).ms_per_replay(max(steps // 4, 5), warmup) / len(banks)
            tf = 2.0 * routes * N * K / (ms * 1e-3) / 1e12
            out[f"{ty.name} {label}"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 2), "copies": len(banks)}
        del banks
        torch.cuda.empty_cache()
    return out


def bench_qmm_n(steps, warmup):
    """transpose = false at M = 1 (x . W, W [K, N] packed along N; the
    safemlx default layout): N x K = 4096 x 4096 and 14336 x 4096, weight
    copies rotating >= ROTATE_BYTES per replay; and the values product of the quantized KV
    attention at one decode position (32 query heads over 8 KV heads, 1024
    cached tokens, D = 128: gather_qmm batches through quantized_matmul's
    broadcasting)."""
    import torch

    n = _lib()
    out = {}
    for N, K in ((4096, 4096), (14336, 4096)):
        copies = rotation(qmv_bytes(1, N, K))
        ws = [torch.randint(-2**31, 2**31 - 1, (K, N * BITS // 32), dtype=torch.int32, device="cuda")
              for _ in range(copies)]
        s = (0.01 * torch.rand((K, N // GS), device="cuda")).to(torch.bfloat16)
        b = (-0.08 * torch.rand((K, N // GS), device="cuda")).to(torch.bfloat16)
        x = torch.randn((1, K), device="cuda").to(torch.bfloat16)
        y = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")

        def fn(st):
            for w in ws:
                n.check(n.lib().eq_quantized_matmul(y.data_ptr(), x.data_ptr(), w.data_ptr(), s.data_ptr(),
                                                    b.data_ptr(), 1, N, K, False, GS, BITS, b"affine",
                                                    n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, st))

        ms = Timer(fn).ms_per_replay(max(steps // 4, 20), warmup) / copies
        gbs = qmv_bytes(1, N, K) / (ms * 1e-3) / 1e9
        out[f"x.W_{N}x{K}"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                               "copies": copies}
        del ws
    # values product of the quantized KV attention: probs [1, 8, 4, 1, T] . values [1, 8, 1, T, D]
    n_kv, n_rep, T, D = 8, 4, 1024, 128
    vw = torch.randint(-2**31, 2**31 - 1, (n_kv, T, D * BITS // 32), dtype=torch.int32, device="cuda")
    vs = (0.01 * torch.rand((n_kv, T, D // GS), device="cuda")).to(torch.bfloat16)
    vb = (-0.08 * torch.rand((n_kv, T, D // GS), device="cuda")).to(torch.bfloat16)
    probs = torch.softmax(torch.randn((n_kv * n_rep, 1, T), device="cuda"), -1).to(torch.bfloat16)
    yv = torch.empty((n_kv * n_rep, 1, D), dtype=torch.bfloat16, device="cuda")
    lhs = torch.arange(n_kv * n_rep, dtype=torch.int32, device="cuda")
    rhs = torch.arange(n_kv, dtype=torch.int32, device="cuda").repeat_interleave(n_rep)

    def fv(st):
        n.check(n.lib().eq_gather_qmm(yv.data_ptr(), probs.data_ptr(), vw.data_ptr(), vs.data_ptr(), vb.data_ptr(),
                                      lhs.data_ptr(), rhs.data_ptr(), n_kv * n_rep, n_kv * n_rep, n_kv, 1, D, T,
                                      False, GS, BITS, b"affine", n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, True, st))

    ms = Timer(fv).ms_per_replay(max(steps // 4, 20), warmup)
    out[f"kv_values_{n_kv}x{T}x{D}_rep{n_rep}"] = {"us": round(ms * 1e3, 2),
                                                   "MB_values": round(n_kv * T * D * (BITS / 8 + 4 / GS) / 1e6, 3)}
    return out


def bench_gather(steps, warmup):
    """Routed-expert decode through gather_qmm (the eredu MoE call, x [routes,
    1, K], lhs = arange, rhs = expert of each route): a Mixtral-8x7B-shaped
    bank of 8 experts, 4-bit g64 bf16, 2 routes per token, for the gate/up
    shape (14336 x 4096) and the down shape (4096 x 14336); a replay runs 4
    tokens over disjoint expert pairs.  Bytes per call = the two selected
    experts' codes + scales + biases + x + y."""
    import torch

    n = _lib()
    E, routes, gs, bits = 8, 2, GS, BITS
    out = {}
    for label, N, K in (("gate_up_14336x4096", 14336, 4096), ("down_4096x14336", 4096, 14336)):
        w = torch.randint(-2**31, 2**31 - 1, (E, N, K * bits // 32), dtype=torch.int32, device="cuda")
        s = (0.01 * torch.rand((E, N, K // gs), device="cuda")).to(torch.bfloat16)
        b = (-0.08 * torch.rand((E, N, K // gs), device="cuda")).to(torch.bfloat16)
        x = torch.randn((routes, 1, K), device="cuda").to(torch.bfloat16)
        y = torch.empty((routes, 1, N), dtype=torch.bfloat16, device="cuda")
        lhs = torch.arange(routes, dtype=torch.int32, device="cuda")
        # four tokens' routes per replay, each pair on experts not read by the others
        rhs = [torch.tensor([2 * i + 1, 2 * i], dtype=torch.int32, device="cuda") for i in range(E // 2)]

        def fn(st):
            for r in rhs:
                n.check(n.lib().eq_gather_qmm(y.data_ptr(), x.data_ptr(), w.data_ptr(), s.data_ptr(), b.data_ptr(),
                                              lhs.data_ptr(), r.data_ptr(), routes, routes, E, 1, N, K, True, gs,
                                              bits, b"affine", n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, True, st))

        ms = Timer(fn).ms_per_replay(max(steps // 4, 20), warmup) / len(rhs)
        nbytes = routes * (N * K * bits // 8 + 2 * N * (K // gs) * 2) + routes * (K + N) * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[label] = {"us": round(ms * 1e3, 2), "MB": round(nbytes / 1e6, 2), "GB/s": round(gbs, 1),
                      "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        del w, s, b
        torch.cuda.empty_cache()
    # prefill: many routes over sorted experts -- grouped MFMA GEMM (sorted hint)
    # against the per-route kernel (no hint); TFLOP/s = 2 routes N K / time
    for label, E, routes, N, K in (("prefill_mixtral_8x_1024routes_14336x4096", 8, 1024, 14336, 4096),
                                   ("prefill_qwen3moe_128x_4096routes_768x2048", 128, 4096, 768, 2048)):
        w = torch.randint(-2**31, 2**31 - 1, (E, N, K * bits // 32), dtype=torch.int32, device="cuda")
        s = (0.01 * torch.rand((E, N, K // gs), device="cuda")).to(torch.bfloat16)
        b = (-0.08 * torch.rand((E, N, K // gs), device="cuda")).to(torch.bfloat16)
        x = torch.randn((routes, 1, K), device="cuda").to(torch.bfloat16)
        y = torch.empty((routes, 1, N), dtype=torch.bfloat16, device="cuda")
        lhs = torch.arange(routes, dtype=torch.int32, device="cuda")
        g = torch.Generator(device="cuda").manual_seed(5)
        rhs = torch.sort(torch.randint(0, E, (routes,), device="cuda", generator=g, dtype=torch.int32)).values
        res = {}
        for hint in (True, False):
            def fg(st, hint=hint):
                n.check(n.lib().eq_gather_qmm(y.data_ptr(), x.data_ptr(), w.data_ptr(), s.data_ptr(), b.data_ptr(),
                                              lhs.data_ptr(), rhs.data_ptr(), routes, routes, E, 1, N, K, True, gs,
                                              bits, b"affine", n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, hint, st))

            ms = Timer(fg).ms_per_replay(max(steps // 4, 10), warmup)
            tf = 2.0 * routes * N * K / (ms * 1e-3) / 1e12
            res["grouped" if hint else "per_route"] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1)}
        out[label] = res
        del w, s, b
        torch.cuda.empty_cache()
    return out


def bench_affine_codec(steps, warmup):
    """Affine dequantize (eq_dequantize: codes + scales + biases -> bf16) and
    quantize (eq_quantize: bf16 -> codes + scales + biases) of a 4096 x 14336
    matrix, 4-bit g64 bf16; GB/s of bytes read + written; each copy is a
    distinct input and output, rotating >= ROTATE_BYTES."""
    import torch

    n = _lib()
    rows, cols = 4096, 14336
    packed = rows * cols * BITS // 8 + 2 * 2 * rows * (cols // GS)
    copies = rotation(packed + rows * cols * 2)
    gen = torch.Generator(device="cuda").manual_seed(3)
    lins = [Linear(rows, cols, gen) for _ in range(copies)]
    dense = [torch.randn((rows, cols), device="cuda", generator=gen).to(torch.bfloat16) * 0.02 for _ in range(copies)]
    outs = [torch.empty((rows, cols), dtype=torch.bfloat16, device="cuda") for _ in range(copies)]
    res = {}

    def deq(st):
        for lin, o in zip(lins, outs):
            n.check(n.lib().eq_dequantize(o.data_ptr(), lin.w.data_ptr(), lin.s.data_ptr(), lin.b.data_ptr(), rows,
                                          cols, GS, BITS, b"affine", n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, st))

    def quant(st):
        for d, lin in zip(dense, lins):  # (written into the copies' own packed buffers)
            n.check(n.lib().eq_quantize(lin.w.data_ptr(), lin.s.data_ptr(), lin.b.data_ptr(), d.data_ptr(), rows, cols,
                                        GS, BITS, b"affine", n.EQ_DTYPE_BF16, st))

    for label, fn in (("dequantize_bf16", deq), ("quantize_bf16", quant)):
        ms = Timer(fn).ms_per_replay(max(steps // 4, 5), warmup) / copies
        gbs = (packed + rows * cols * 2) / (ms * 1e-3) / 1e9
        res[label] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                      "copies": copies}
    return res


def bench_mxfp4(steps, warmup):
    """MXFP4 mode (E2M1 codes, one E8M0 scale byte per 32 values, no biases):
    decode (M = 1) and prefill (M = 512) quantized_matmul, the routed-expert
    decode of a Mixtral-shaped bank (2 routes per token), transpose = false
    at M = 1, dequantize / quantize, and GGUF type-39 conversion.  Weight
    copies rotate >= ROTATE_BYTES per replay (the prefill leg: 4 copies).
    Bytes per linear: N*K/2 codes + N*K/32 scale bytes + 2*M*K + 2*M*N."""
    import torch

    n = _lib()
    u8 = n.EQ_DTYPE_U8
    out = {}

    def mx_bytes(M, N, K):
        return N * K // 2 + N * K // 32 + 2 * M * K + 2 * M * N

    def mx_weights(rows, cols, count):
        ws = [torch.randint(-2**31, 2**31 - 1, (rows, cols // 8), dtype=torch.int32, device="cuda")
              for _ in range(count)]
        ss = [torch.randint(118, 128, (rows, cols // 32), dtype=torch.uint8, device="cuda") for _ in range(count)]
        return ws, ss

    for label, M, N, K, transpose in (("decode_M1_4096x4096", 1, 4096, 4096, True),
                                      ("decode_M1_14336x4096", 1, 14336, 4096, True),
                                      ("decode_M1_4096x14336", 1, 4096, 14336, True),
                                      ("prefill_M512_4096x4096", 512, 4096, 4096, True),
                                      ("prefill_M512_14336x4096", 512, 14336, 4096, True),
                                      ("xW_M1_4096x4096", 1, 4096, 4096, False)):
        rows, cols = (N, K) if transpose else (K, N)
        copies = rotation(mx_bytes(M, N, K)) if M == 1 else 4
        ws, ss = mx_weights(rows, cols, copies)
        x = torch.randn((M, K), device="cuda").to(torch.bfloat16)
        y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")

        def fn(st):
            for w, sc in zip(ws, ss):
                n.check(n.lib().eq_quantized_matmul(y.data_ptr(), x.data_ptr(), w.data_ptr(), sc.data_ptr(), None, M,
                                                    N, K, transpose, 32, 4, b"mxfp4", n.EQ_DTYPE_BF16, u8, st))

        ms = Timer(fn).ms_per_replay(max(steps // 4, 10), warmup) / copies
        rec = {"us": round(ms * 1e3, 2), "copies": copies}
        if M == 1:
            gbs = mx_bytes(M, N, K) / (ms * 1e-3) / 1e9
            rec.update({"GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)})
        else:
            tf = 2.0 * M * N * K / (ms * 1e-3) / 1e12
            rec.update({"TFLOP/s": round(tf, 1), "frac_mfma": round(tf / BF16_MFMA_PEAK_TFLOPS, 4)})
        out[label] = rec
        del ws, ss
        torch.cuda.empty_cache()

    # routed experts: 8 experts, 2 routes per token, 4 tokens per replay on disjoint pairs
    E, routes = 8, 2
    for label, N, K in (("routed_gate_up_14336x4096", 14336, 4096), ("routed_down_4096x14336", 4096, 14336)):
        w = torch.randint(-2**31, 2**31 - 1, (E, N, K // 8), dtype=torch.int32, device="cuda")
        sc = torch.randint(118, 128, (E, N, K // 32), dtype=torch.uint8, device="cuda")
        x = torch.randn((routes, 1, K), device="cuda").to(torch.bfloat16)
        y = torch.empty((routes, 1, N), dtype=torch.bfloat16, device="cuda")
        lhs = torch.arange(routes, dtype=torch.int32, device="cuda")
        rhs = [torch.tensor([2 * i + 1, 2 * i], dtype=torch.int32, device="cuda") for i in range(E // 2)]

        def fr(st):
            for r in rhs:
                n.check(n.lib().eq_gather_qmm(y.data_ptr(), x.data_ptr(), w.data_ptr(), sc.data_ptr(), None,
                                              lhs.data_ptr(), r.data_ptr(), routes, routes, E, 1, N, K, True, 32, 4,
                                              b"mxfp4", n.EQ_DTYPE_BF16, u8, True, st))

        ms = Timer(fr).ms_per_replay(max(steps // 4, 20), warmup) / len(rhs)
        nbytes = routes * (N * K // 2 + N * K // 32) + routes * (K + N) * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[label] = {"us": round(ms * 1e3, 2), "MB": round(nbytes / 1e6, 2), "GB/s": round(gbs, 1),
                      "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        del w, sc
        torch.cuda.empty_cache()

    # codec: 4096 x 14336 dequantize (-> bf16), quantize (bf16 ->), GGUF type-39 blocks -> MLX pair
    rows, cols = 4096, 14336
    packed = rows * cols // 2 + rows * cols // 32
    copies = rotation(packed + rows * cols * 2)
    ws, ss = mx_weights(rows, cols, copies)
    dense = [torch.randn((rows, cols), device="cuda").to(torch.bfloat16) for _ in range(copies)]
    nraw = rows * cols // 32 * 17
    cc = rotation(nraw + packed)
    raws = [torch.randint(0, 256, (nraw,), dtype=torch.uint8, device="cuda") for _ in range(cc)]
    cw, cs = mx_weights(rows, cols, cc)

    def deq(st):
        for w, sc, o in zip(ws, ss, dense):
            n.check(n.lib().eq_dequantize(o.data_ptr(), w.data_ptr(), sc.data_ptr(), None, rows, cols, 32, 4,
                                          b"mxfp4", u8, n.EQ_DTYPE_BF16, st))

    def quant(st):
        for d, w, sc in zip(dense, ws, ss):
            n.check(n.lib().eq_quantize(w.data_ptr(), sc.data_ptr(), None, d.data_ptr(), rows, cols, 32, 4,
                                        b"mxfp4", n.EQ_DTYPE_BF16, st))

    def conv(st):
        for r, w, sc in zip(raws, cw, cs):
            n.check(n.lib().eq_gguf_convert_mxfp4(w.data_ptr(), sc.data_ptr(), r.data_ptr(), nraw, rows, cols, st))

    for label, fn, nb, k in (("dequantize_bf16", deq, packed + rows * cols * 2, copies),
                             ("quantize_bf16", quant, packed + rows * cols * 2, copies),
                             ("gguf_convert_type39", conv, nraw + packed, cc)):
        ms = Timer(fn).ms_per_replay(max(steps // 4, 5), warmup) / k
        gbs = nb / (ms * 1e-3) / 1e9
        out[label] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                      "copies": k}
    return out


def bench_gguf_stream():
    """GGUF file -> HBM affine triples (gguf_file.stream_convert_affine): a
    file of 8 Q4_K tensors of 4096 x 14336 (264 MB, synthetic blocks) in the
    page cache, streamed through 64 MiB pinned buffers with conversion on
    the GPU; beside it the same file read whole, copied in one transfer and
    converted tensor by tensor (no overlap).  GB/s of file bytes, host clock
    around each call (PCIe-inclusive; not a kernel figure)."""
    import tempfile

    import torch

    from eredu_amd import gguf as G
    from eredu_amd import gguf_file as F

    rows, cols, count = 4096, 14336, 8
    nbytes = rows * cols // 256 * 144
    tensors = []
    for i in range(count):
        raw = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda").cpu().numpy()
        tensors.append((f"blk.{i}.ffn_down.weight", [cols, rows], F.Q4_K, raw.tobytes()))
    fd, path = tempfile.mkstemp(suffix=".gguf")
    try:
        with os.fdopen(fd, "wb") as f:
            F.write_gguf(f, {}, tensors)
        total = sum(len(t[3]) for t in tensors)
        del tensors
        F.stream_convert_affine(path, staging_bytes=64 << 20)  # warm: page cache, pinned pools
        best = 1e9
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = F.stream_convert_affine(path, staging_bytes=64 << 20)
            best = min(best, time.perf_counter() - t0)
            del out
        reader = F.GgufReader(path)
        host = torch.empty(os.path.getsize(path), dtype=torch.uint8, pin_memory=True)
        seq = 1e9
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            with open(path, "rb") as f:
                f.readinto(memoryview(host.numpy()))
            dev = host.cuda(non_blocking=True)
            for t in reader.tensors:
                d = G.TensorDescriptor(t.name, list(t.dimensions), G.GgmlType(t.ggml_type), t.byte_len)
                G.convert_affine(d, dev[t.data_offset:t.data_offset + t.byte_len])
            torch.cuda.synchronize()
            seq = min(seq, time.perf_counter() - t0)
        reader.close()
        return {"file_MB": round(total / 1e6, 1), "stream_ms": round(best * 1e3, 2),
                "stream_GB/s": round(total / best / 1e9, 2), "sequential_ms": round(seq * 1e3, 2),
                "sequential_GB/s": round(total / seq / 1e9, 2)}
    finally:
        os.unlink(path)


VOCAB, N_HEADS, N_KV_HEADS, CACHE_TOKENS = 128256, 32, 8, 1024


def build_decoder(layers, gen, fused=None):
    """the Llama-3-8B-shaped stack around the 32 layers' packed
    projections -- bf16 embeddings and norms, a 4-bit LM head, a bf16 KV cache
    of CACHE_TOKENS random N(0, 1) rows per layer, Llama-3 RoPE (theta 5e5,
    llama3 scaling) -- for the batch-1 decode step of eredu_amd.decode."""
    import torch

    from eredu_amd import decode as E

    def q(l):
        return E.QLinear(l.w, l.s, l.b, BITS, GS)

    bf = torch.bfloat16
    norm = lambda: (1.0 + 0.1 * torch.randn((HIDDEN,), device="cuda", generator=gen)).to(bf)
    dec_layers = [E.DecoderLayer(norm(), norm(), *(q(L[p]) for p in ("q", "k", "v", "o", "gate", "up", "down")))
                  for L in layers]
    embed = torch.empty((VOCAB, HIDDEN), dtype=bf, device="cuda")
    for r0 in range(0, VOCAB, 8192):
        embed[r0:r0 + 8192] = torch.randn((min(8192, VOCAB - r0), HIDDEN), device="cuda", generator=gen).to(bf)
    lm = Linear(VOCAB, HIDDEN, gen)
    # room past the 1024 cached rows for the positions that the device-position
    # graph's replays advance through
    max_seq = CACHE_TOKENS + 256
    caches = [[torch.randn((N_KV_HEADS, max_seq, 128), device="cuda", generator=gen).to(bf) for _ in layers]
              for _ in range(2)]
    freqs = E.llama3_rope_freqs(128, 500000.0, 8.0, 1.0, 4.0, 8192)
    return E.LlamaDecoder(dec_layers, embed, norm(), q(lm), n_heads=N_HEADS, n_kv_heads=N_KV_HEADS, eps=1e-5,
                          freqs=freqs, max_seq=max_seq, k_caches=caches[0], v_caches=caches[1], fused=fused)


def bench_decode_step(layers, steps, warmup, gen):
    """Full batch-1 decode step: tok/s of one HIP graph that
    decodes successive tokens (the position in device memory, advanced by
    each replay, from the 1024 cached tokens on), and the step's algorithmic
    bytes against 8 TB/s.  Also the step at a position fixed by the capture
    (one graph per position) for comparison."""
    from eredu_amd import decode as E

    dec = build_decoder(layers, gen)
    # the same model with the norms and SiLU-mul as launches of their own
    other = E.LlamaDecoder(dec.layers, dec.embed, dec.final_norm, dec.lm_head, n_heads=N_HEADS, n_kv_heads=N_KV_HEADS,
                           eps=1e-5, freqs=dec.freqs.cpu().numpy(), max_seq=dec.max_seq, k_caches=dec.k_caches,
                           v_caches=dec.v_caches, fused=not dec.fused)
    pos = CACHE_TOKENS
    ms_host = Timer(lambda st: dec.step(pos)).ms_per_replay(steps, warmup)

    def device_ms(d):
        d.set_position(pos)  # the Timer's eager call decodes pos, the replays pos + 1, pos + 2, ...
        return Timer(lambda st: d.step_device()).ms_per_replay(steps, warmup)

    ms_a, ms_b = device_ms(dec), device_ms(other)
    if ms_b < ms_a:
        dec, other, ms_a, ms_b = other, dec, ms_b, ms_a
    ms = ms_a
    mean_pos = pos + warmup + (steps + 1) // 2  # mean position of the timed replays
    nbytes = dec.bytes_per_step(mean_pos)
    gbs = nbytes / (ms * 1e-3) / 1e9
    roof = HBM_PEAK_GBS * 1e9 / nbytes
    out = {"ms": round(ms, 4), "tok/s": round(1e3 / ms, 1), "bytes_per_token": nbytes, "GB/s": round(gbs, 1),
           "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "roofline_tok/s": round(roof, 1),
           "launches": dec.launches_per_step(device_position=True), "fused_prologues": dec.fused,
           "position": f"device memory, advanced by each replay of one graph; timed replays at positions "
                       f"{pos + warmup + 1}..{pos + warmup + steps}",
           "other_variant_ms": round(ms_b, 4),
           "other_variant_launches": other.launches_per_step(device_position=True),
           "host_position_ms": round(ms_host, 4), "host_position_launches": dec.launches_per_step(),
           "workload": "batch 1, 32 layers, H 4096, 32 q / 8 kv heads x 128, FFN 14336, vocab 128256, 4-bit g64 "
                       "linears incl. LM head, bf16 embeddings/norms, 1024-token bf16 KV cache, greedy argmax"}
    del dec, other
    return out


def bench_decode_variants(layers, args):
    """The decode step issued other ways: one launch per projection (the drop-in
    path), all seven projections per launch, and the grouped step at M = 8."""
    out = {}
    steps = max(args.steps // 2, 5)
    for key, M, groups, what in (("decode_M1_per_projection", 1, None, "one launch per projection (drop-in path)"),
                                 ("decode_M1_all7_per_launch", 1, ALL7, "seven projections per launch"),
                                 ("decode_M8_grouped", 8, DECODE_GROUPS, "grouped launches")):
        log(f"[bench] decode step M={M}, {what}")
        ms, nb, launches = bench_decode(layers, M, groups, steps, args.warmup)
        out[key] = {"ms": round(ms, 4), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1), "launches": launches}
    return out


def host_cpu():
    """The host CPU as lscpu names it (model, sockets, cores, threads)."""
    import subprocess

    info = {}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in txt.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core", "CPU(s)"):
                info[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    info["affinity_cpus"] = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None
    return info


def cpu_baseline(layer, budget_s=20.0):
    """The restated MLX CPU quantized matmul (oracle/eq_oracle.c or_qmm_t_f32), on the
    same packed inputs of one layer's 7 projections at M = 1, single-threaded and
    with one thread per host core (at most 16, the box's CPU share)."""
    import torch

    from oracle import oracle as orc

    host = []
    for name, N, K in LAYER_SHAPES:
        lin = layer[name]
        host.append((N, K, lin.w.cpu().numpy().view(np.uint32), lin.s.view(torch.int16).cpu().numpy().view(np.uint16),
                     lin.b.view(torch.int16).cpu().numpy().view(np.uint16)))
    x = {K: np.ascontiguousarray(orc.f32_to_bf16_bits(np.random.default_rng(0).standard_normal((1, K), dtype=np.float32)))
         for K in (HIDDEN, FFN)}
    # one thread per host core the process may use, at most 16: the GPU box's
    # CPU share for one GPU (its nproc reports the whole host)
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = max(1, min(16, avail))
    res = {}
    for nthreads in sorted({1, threads}):
        reps, t0 = 0, time.perf_counter()
        while True:
            for N, K, w, s, b in host:
                orc.qmm_t_f32(x[K], orc.BF16, w, s, b, orc.BF16, 1, N, K, GS, BITS, threads=nthreads)
            reps += 1
            el = time.perf_counter() - t0
            if el > budget_s / 2 or reps >= 200:
                break
        nbytes = reps * sum(qmv_bytes(1, N, K) for N, K, *_ in host)
        res[nthreads] = (nbytes / el / 1e9, reps, el)
    return res, threads


def cpu_baseline_prefill(threads, budget_s=8.0, M=512, N=256, K=HIDDEN):
    """The restated MLX CPU _qmm_t loop (or_qmm_t_f32, f32 accumulate) at the
    prefill point M = 512 of the 4096 x 4096 projection, on a bounded sample:
    N = 256 of its 4096 output features (the loop's cost is linear in N), 4-bit
    group 64, single-threaded and on `threads` threads.  TFLOP/s = 2 M N K / s."""
    from oracle import oracle as orc

    rng = np.random.default_rng(1)
    w = rng.integers(0, 2**32, (N, K * BITS // 32), dtype=np.uint32)
    s = orc.f32_to_bf16_bits(rng.random((N, K // GS), dtype=np.float32) * 0.004 + 0.004)
    b = orc.f32_to_bf16_bits(-7.5 * orc.bf16_bits_to_f32(s))
    x = orc.f32_to_bf16_bits(rng.standard_normal((M, K), dtype=np.float32))
    res = {}
    for nthreads in sorted({1, threads}):
        reps, t0 = 0, time.perf_counter()
        while True:
            orc.qmm_t_f32(x, orc.BF16, w, s, b, orc.BF16, M, N, K, GS, BITS, threads=nthreads)
            reps += 1
            el = time.perf_counter() - t0
            if el > budget_s / 2 or reps >= 100:
                break
        res[nthreads] = {"TFLOP/s": round(2.0 * M * N * K * reps / el / 1e12, 6), "passes": reps,
                         "seconds": round(el, 2)}
    return {"unit": "TFLOP/s", "kind": "port", "threads": threads,
            "value": res[threads]["TFLOP/s"], "single_thread_TFLOP/s": res[1]["TFLOP/s"],
            "sample": f"M={M} x N={N} (of 4096) x K={K}, 4-bit group 64, bf16 x/scales/biases: restated MLX CPU "
                      f"_qmm_t loop (oracle/eq_oracle.c or_qmm_t_f32)", "runs": res}


def cpu_baseline_gguf(budget_s=6.0, rows=4096, cols=14336):
    """eredu-gguf's convert_affine (convert.rs:318-465) as the oracle restates it
    (oracle/eq_oracle.c or_gguf_convert_affine), single-threaded like the
    reference's scalar loop, on uniform random blocks of a 4096 x 14336
    tensor (the GPU leg's input); GB/s counts blocks in + codes/scales/biases
    out, as the GPU leg does."""
    from oracle import oracle as orc

    rng = np.random.default_rng(2)
    out = {}
    geo = {"Q4_0": (2, 32, 18, 4, 32), "Q8_0": (8, 32, 34, 8, 32), "Q4_K": (12, 256, 144, 4, 32)}
    for name, (code, vals, nbytes, bits, gs) in geo.items():
        nraw = rows * cols // vals * nbytes
        raw = rng.integers(0, 256, nraw, dtype=np.uint8)
        moved = nraw + rows * cols * bits // 8 + 2 * 2 * rows * (cols // gs)
        reps, t0 = 0, time.perf_counter()
        while True:
            orc.gguf_convert_affine(code, raw)
            reps += 1
            el = time.perf_counter() - t0
            if el > budget_s / 3 or reps >= 50:
                break
        out[name] = {"GB/s": round(moved * reps / el / 1e9, 4), "passes": reps, "seconds": round(el, 2)}
    return {"unit": "GB/s", "kind": "port", "threads": 1, "convert_affine": out,
            "sample": f"{rows} x {cols} tensors of uniform random blocks, one thread"}


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "qmv_lds_decode_M1_grouped.md")


def profiled_traffic():
    """HBM bytes per launch of the headline kernel from the committed PMC summary
    (FETCH_SIZE and WRITE_SIZE runs of this same command, scaled by a copy-kernel
    calibration); None if the summary is absent."""
    try:
        for line in open(TRAFFIC_PROFILE):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--quick", action="store_true", help="decode steps only (no qmm / gguf / per-shape sweeps)")
    ap.add_argument("--headline-only", action="store_true",
                    help="the headline step only (the run a kernel-trace profile of the roofline kernel uses)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the prefill qmm sweep, one JSON object of its figures (for kernel-trace profiles)")
    ap.add_argument("--prefill-m", type=int, default=None,
                    help="with --prefill-only: this M only, 4- and 8-bit at the four shapes, no other widths "
                         "(for counter profiles of one prefill size)")
    ap.add_argument("--gguf-only", action="store_true",
                    help="only the GGUF dequant/convert sweep, one JSON object of its figures")
    ap.add_argument("--gather-only", action="store_true",
                    help="only the gather_qmm and transpose = false figures, one JSON object")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the full decode step of configs[4], one JSON object of its figures")
    ap.add_argument("--mxfp4-only", action="store_true",
                    help="only the MXFP4-mode figures, one JSON object")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: this build runs on a single GPU "
              f"only (one GPU's share of a sharded projection is the same kernel at a smaller N or K)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    _lib().lib()
    torch.cuda.set_device(0)
    if args.prefill_only or args.gguf_only or args.gather_only or args.mxfp4_only:
        out = {}
        if args.mxfp4_only:
            log("[bench] mxfp4 mode")
            out["mxfp4"] = bench_mxfp4(args.steps, args.warmup)
        if args.prefill_only:
            log("[bench] qmm prefill")
            if args.prefill_m:
                out["qmm"] = bench_qmm(args.steps, args.warmup, Ms=(args.prefill_m,))
            else:
                out["qmm"] = bench_qmm(args.steps, args.warmup)
                log("[bench] qmm prefill, other widths")
                out["qmm_widths"] = bench_qmm_widths(args.steps, args.warmup)
        if args.gguf_only:
            log("[bench] gguf")
            out["gguf"] = bench_gguf(args.steps, args.warmup)
            log("[bench] gguf mixture-of-experts linear")
            out["gguf_grouped"] = bench_gguf_grouped(args.steps, args.warmup)
            log("[bench] gguf native embedding")
            out["gguf_embedding"] = bench_gguf_embedding(args.steps, args.warmup)
            log("[bench] gguf streaming load")
            out["gguf_stream"] = bench_gguf_stream()
            log("[bench] affine dequantize / quantize")
            out["affine_codec"] = bench_affine_codec(args.steps, args.warmup)
        if args.gather_only:
            log("[bench] gather_qmm routed-expert decode")
            out["gather_qmm"] = bench_gather(args.steps, args.warmup)
            log("[bench] transpose = false (qmm_n)")
            out["qmm_n"] = bench_qmm_n(args.steps, args.warmup)
        print(json.dumps(out), flush=True)
        return
    gen = torch.Generator(device="cuda").manual_seed(0)
    log("[bench] allocating 32 layers of 4-bit weights")
    layers = [{name: Linear(N, K, gen) for name, N, K in LAYER_SHAPES} for _ in range(LAYERS)]
    torch.cuda.synchronize()
    if args.decode_only:
        log("[bench] full decode step (configs[4])")
        print(json.dumps({"decode_step": bench_decode_step(layers, args.steps, args.warmup, gen)}), flush=True)
        return

    log("[bench] decode step M=1, grouped launches")
    ms, nbytes, launches = bench_decode(layers, 1, DECODE_GROUPS, args.steps, args.warmup)
    value = nbytes / (ms * 1e-3) / 1e9
    detail = {"decode_M1_grouped": {"ms": round(ms, 4), "GB/s": round(value, 1), "launches": launches}}
    if args.headline_only:
        args.quick = args.no_cpu = True
    else:
        detail.update(bench_decode_variants(layers, args))
    step = None
    if not args.quick:
        log("[bench] full decode step (configs[4])")
        step = bench_decode_step(layers, args.steps, args.warmup, gen)
        detail["decode_step_config5"] = step
        log("[bench] per-shape qmv")
        detail["qmv_M1_per_shape"] = bench_per_shape(layers, 1, args.steps, args.warmup)
        detail["qmv_M8_per_shape"] = bench_per_shape(layers, 8, args.steps, args.warmup)
        log("[bench] f16 activations")
        detail["f16_activations"] = bench_f16(layers, args.steps, args.warmup)

    cpu = None
    if not args.no_cpu:
        log("[bench] CPU baseline")
        res, threads = cpu_baseline(layers[0])
        v1, vt = res[1], res[threads]
        cpu = {"value": round(vt[0], 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"one layer's 7 projections (122.8 MB packed) at M=1: {vt[1]} passes in {vt[2]:.1f} s on "
                         f"{threads} threads ({v1[1]} passes in {v1[2]:.1f} s on 1 thread: "
                         f"{v1[0]:.3f} GB/s); restated MLX CPU _qmm_t loop (oracle/eq_oracle.c or_qmm_t_f32), "
                         f"f32 accumulate",
               "single_thread_GB/s": round(v1[0], 3), "host": host_cpu(),
               "threads_note": "threads = min(16, CPUs in this process's affinity): 16 is the GPU box's CPU share "
                               "per GPU"}
        log("[bench] CPU baseline, prefill qmm")
        cpu["prefill_qmm_M512"] = cpu_baseline_prefill(threads)
        log("[bench] CPU baseline, GGUF convert")
        cpu["gguf_convert"] = cpu_baseline_gguf()
    del layers
    torch.cuda.empty_cache()
    if not args.quick:
        log("[bench] qmm prefill")
        detail["qmm"] = bench_qmm(args.steps, args.warmup)
        log("[bench] qmm prefill, other widths")
        detail["qmm_widths"] = bench_qmm_widths(args.steps, args.warmup)
        log("[bench] gguf")
        detail["gguf"] = bench_gguf(args.steps, args.warmup)
        log("[bench] gguf mixture-of-experts linear")
        detail["gguf_grouped"] = bench_gguf_grouped(args.steps, args.warmup)
        log("[bench] gguf native embedding")
        detail["gguf_embedding"] = bench_gguf_embedding(args.steps, args.warmup)
        log("[bench] gguf streaming load")
        detail["gguf_stream"] = bench_gguf_stream()
        log("[bench] affine dequantize / quantize")
        detail["affine_codec"] = bench_affine_codec(args.steps, args.warmup)
        log("[bench] gather_qmm routed-expert decode")
        detail["gather_qmm"] = bench_gather(args.steps, args.warmup)
        log("[bench] transpose = false (qmm_n)")
        detail["qmm_n"] = bench_qmm_n(args.steps, args.warmup)
        log("[bench] mxfp4 mode")
        detail["mxfp4"] = bench_mxfp4(args.steps, args.warmup)

    per_launch_bytes = nbytes / launches
    avg_launch_us = ms * 1e3 / launches
    achieved = per_launch_bytes / (avg_launch_us * 1e-6) / 1e9
    line = {
        "metric": "4-bit qmv achieved HBM GB/s (% peak); decode tok/s for 8B-shaped 4-bit stack",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "timing": "median over the timed replays of one HIP graph per step (HIP events around each replay)",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random 4-bit codes, bf16 scales/biases, x ~ N(0,1) bf16)",
        "config": {
            "workload": "decode qmv sweep (configs[1]): Llama-3-8B projections q,k,v,o,gate,up,down x 32 layers, "
                        "M=1, 4-bit group-64, bf16 activations/scales/biases; one grouped launch per input-sharing "
                        "set {q,k,v},{o},{gate,up},{down}; one HIP graph per step",
            "M": 1, "layers": LAYERS, "bits": BITS, "group_size": GS,
            "bytes_per_step": nbytes, "launches_per_step": launches,
        },
        "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": "qmv_lds_kernel<4,64,BF16T,1,true,false,0,BF16T,0>",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic(),
            "traffic_source": "profiles/qmv_lds_decode_M1_grouped.md (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)",
            "per_launch_bytes": int(per_launch_bytes),
            "avg_launch_us": round(avg_launch_us, 3),
        },
        "cpu_baseline": cpu,
        "detail": detail,
    }
    dropin = detail.get("decode_M1_per_projection")
    if dropin:  # the path unchanged eredu callers take: one eq_quantized_matmul per projection
        line["roofline"]["dropin_per_projection"] = {"GB/s": dropin["GB/s"],
                                                     "frac": round(dropin["GB/s"] / HBM_PEAK_GBS, 4),
                                                     "launches": dropin["launches"]}
    if step is not None:  # the metric's second figure: end-to-end decode of configs[4]
        line["decode_tok_s"] = step["tok/s"]
        line["decode_tok_s_frac_roofline"] = round(step["tok/s"] / step["roofline_tok/s"], 4)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

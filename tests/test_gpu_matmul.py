"""Parity of the HIP quantized matmul (qmv / qmm / general kernels) with the
fp64 oracle, through the C ABI (via the eredu_amd host mirror).

Tolerance (written here, as the rule the north star states): elementwise
|y - y_ref| <= 1e-2 * RMS(y_ref) + 1/2 ulp_bf16(y_ref) for bf16 outputs
(the half-ulp is the unavoidable rounding of the bf16 result), and the
strict |y - y_ref| <= 1e-2 * RMS(y_ref) for f32 outputs.  y_ref is the exact
(f64) product of the same packed inputs.
"""
import numpy as np
import pytest
import torch

from eredu_amd import (EreduError, QuantizedLinear, dequantize_with_mode, quantized_matmul, quantized_matmul_batched,
                       quantized_matmul_with_mode)
from oracle import oracle as orc
from tests.fixtures import (dev_bf16, dev_param, dev_words, host_bits16, host_f32, synthetic_linear,
                            synthetic_x)

pytestmark = pytest.mark.gpu

LLAMA_SHAPES = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]


def run_case(M, N, K, gs, bits, sdt=orc.BF16, xdt=orc.BF16, seed=0, transpose=True, biases=True):
    print(f"[case] M={M} N={N} K={K} gs={gs} bits={bits} sdt={sdt} xdt={xdt} transpose={transpose}", flush=True)
    if transpose:
        w, s, b = synthetic_linear(N, K, gs, bits, seed, scale_dtype=sdt)
    else:
        w, s, b = synthetic_linear(K, N, gs, bits, seed, scale_dtype=sdt)
    if not biases:
        b = None
    xb = synthetic_x(M, K, seed + 1)
    if xdt == orc.BF16:
        x_host, xd = xb, dev_bf16(xb)
    else:
        xf = orc.bf16_bits_to_f32(xb)
        if xdt == orc.F16:
            x_host = xf.astype(np.float16).view(np.uint16)
        else:
            x_host = xf
        xd = dev_param(x_host, xdt)
    y = quantized_matmul_with_mode(xd, dev_words(w), dev_param(s, sdt), None if b is None else dev_param(b, sdt),
                                   transpose, gs, bits)
    torch.cuda.synchronize()
    y_ref = orc.quantized_matmul_f64(x_host, xdt, w, s, b, sdt, transpose, gs, bits, N, K)
    ok, worst, rms = orc.matmul_within_tolerance(host_f32(y), y_ref, out_is_bf16=(xdt != orc.F32))
    assert y.shape == (M, N)
    assert ok, f"max|err|/RMS = {worst:.3e} (RMS {rms:.3f})"
    return worst


@pytest.mark.parametrize("N,K", LLAMA_SHAPES)
@pytest.mark.parametrize("M", [1, 8])
def test_qmv_llama_shapes(cuda, M, N, K):
    run_case(M, N, K, 64, 4, seed=N + K + M)


@pytest.mark.parametrize("M", list(range(1, 17)))
def test_qmv_every_small_batch(cuda, M):
    run_case(M, 256, 1024, 64, 4, seed=M)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("sdt", [orc.BF16, orc.F16])
@pytest.mark.parametrize("M", [1, 5])
def test_qmv_contract_grid(cuda, bits, gs, sdt, M):
    run_case(M, 128, 2048, gs, bits, sdt=sdt, seed=bits * gs + M)


# K not a multiple of the 64-byte-per-row span (and K shorter than one span);
# only K that hold whole groups are valid shapes, so only those are generated
RAGGED_K = [(K, bits, gs) for K in (32, 64, 96, 160, 192, 4160, 4224)
            for bits, gs in ((4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)) if K % gs == 0]


@pytest.mark.parametrize("K,bits,gs", RAGGED_K)
@pytest.mark.parametrize("M", [1, 3])
def test_qmv_ragged_k(cuda, K, bits, gs, M):
    run_case(M, 48, K, gs, bits, seed=K + bits + gs + M)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("M", [17, 128, 300])
def test_qmm_grid(cuda, bits, gs, M):
    run_case(M, 256, 1024, gs, bits, seed=bits + gs + M)


@pytest.mark.parametrize("bits", [4, 8])
def test_qmm_prefill_shape(cuda, bits):
    run_case(512, 4096, 4096, 64, bits, seed=bits)


def test_qmm_f16_scales(cuda):
    run_case(64, 256, 512, 32, 4, sdt=orc.F16, seed=3)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("K", [64, 128, 192, 256, 320, 448])
def test_qmm_pipeline_depths(cuda, bits, K):
    # 1..7 chunks of 64 in one workgroup (too few to split K): every position
    # of the three-slot load ring, including the wrap-around
    run_case(40, 256, K, 64, bits, seed=K + bits)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,gs", [(65, 64), (100, 64), (100, 32)])
def test_qmm_tiles_ragged(cuda, bits, M, gs):
    # N = 384: three 64 x 128 tiles (group 64) or two 128 x 256 tiles, the
    # second half past N (group 32, which keeps the large tile); M not a
    # multiple of either tile height; K split 4 ways in both plans
    run_case(M, 384, 2048, gs, bits, seed=M + gs + bits)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("M,N,K", [(500, 3968, 4096), (400, 3968, 14336)])
def test_qmm_mid_tiles_ragged(cuda, bits, M, N, K):
    # 128 x 128 tiles with K split twice, M not a multiple of 128 and N of
    # 256 (31 column tiles): in place of the 64 x 128 tiles at K = 4096 and
    # of the 128 x 256 tiles' 4-way split at K = 14336.  (Seed 4476 at
    # M = 500, N = 3968, K = 4096, 8 bits puts one of the 2e6 outputs just
    # over the rule: the matrix-core path rounds each dequantized weight to
    # bf16, and the 64 x 128 plan gives that element the same value.)
    run_case(M, N, K, 64, bits, seed=1 + bits)


@pytest.mark.parametrize("bits", [4, 8])
def test_qmm_split_k(cuda, bits):
    # 6 output tiles, 32 chunks: K split 8 ways, partial tiles summed in order
    run_case(300, 512, 2048, 64, bits, seed=bits + 77)


@pytest.mark.parametrize("xdt", [orc.F32, orc.F16])
@pytest.mark.parametrize("M", [1, 33])
def test_general_activation_dtypes(cuda, xdt, M):
    # f32 activations give f32 output and must meet the strict 1e-2*RMS rule
    run_case(M, 64, 512, 64, 4, xdt=xdt, seed=M)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_general_bits_and_f32_scales(cuda, bits):
    run_case(3, 48, 256, 64, bits, sdt=orc.F32, seed=bits)


@pytest.mark.parametrize("M", [1, 7, 20])
def test_transpose_false(cuda, M):
    # W stored [K, N] packed along N (quantized KV attention, tensor.rs:133-140)
    run_case(M, 128, 192, 64, 4, transpose=False, seed=M)


# transpose = false, bf16 x: M = 1 takes qmm_n_m1 (128-column tiles: N = 64
# fills half of one, 384 three, 4096 thirty-two; K = 96 is two row runs of 64
# and 32, the others 8 to 56 runs of 64 to 256 rows, added by the last
# workgroup of each tile), M = 2..8 qmm_n_small (16 / 32 / 64 word columns per
# workgroup; partial sums through the workspace); M > 8 runs qmm_n_small on
# 8-row batches over the one weight matrix plus a launch for the rest.
@pytest.mark.parametrize("N,K", [(64, 96), (384, 1024), (4096, 4096), (128, 4096), (1024, 14336)])
@pytest.mark.parametrize("M", [1, 2, 5, 8, 9])
def test_transpose_false_small_m(cuda, N, K, M):
    run_case(M, N, K, 64, 4, transpose=False, seed=N + K + M)


@pytest.mark.parametrize("N,K", [(384, 1024), (4096, 4096)])
@pytest.mark.parametrize("M", [16, 23, 64])
def test_transpose_false_row_chunks(cuda, N, K, M):
    run_case(M, N, K, 64, 4, transpose=False, seed=N + K + M)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("sdt", [orc.BF16, orc.F16])
@pytest.mark.parametrize("M", [1, 3])
def test_transpose_false_contract_grid(cuda, bits, gs, sdt, M):
    # M = 1 takes qmm_n_m1 (16-byte words per lane), M = 3 qmm_n_small
    run_case(M, 256, 2048, gs, bits, sdt=sdt, transpose=False, seed=bits * gs + M, biases=(gs != 32))


def test_ragged_n_and_no_biases(cuda):
    run_case(2, 40, 256, 32, 4, seed=9, biases=False)   # N % 16 != 0 -> general kernel
    run_case(2, 64, 256, 32, 4, seed=10, biases=False)  # qmv without biases
    run_case(40, 256, 256, 64, 4, seed=11, biases=False)  # qmm without biases


def test_all_zero_codes_give_bias_term(cuda):
    N, K, gs = 64, 512, 64
    s = orc.f32_to_bf16_bits(np.full((N, K // gs), 0.5, np.float32))
    b = orc.f32_to_bf16_bits(np.random.default_rng(0).normal(0, 0.1, (N, K // gs)).astype(np.float32))
    w = np.zeros((N, K // 8), np.uint32)
    for M in (1, 9, 64):
        xb = synthetic_x(M, K, M)
        y = quantized_matmul(dev_bf16(xb), dev_words(w), dev_bf16(s), dev_bf16(b), transpose=True, group_size=gs)
        xs = orc.bf16_bits_to_f32(xb).astype(np.float64).reshape(M, K // gs, gs).sum(-1)
        ref = xs @ orc.bf16_bits_to_f32(b).astype(np.float64).T
        assert orc.matmul_within_tolerance(host_f32(y), ref, True)[0]


def test_batch_dims_flatten_into_m(cuda):
    N, K = 128, 256
    w, s, b = synthetic_linear(N, K, 64, 4, 1)
    xb = synthetic_x(6, K, 2)
    lin = QuantizedLinear(dev_words(w), dev_bf16(s), dev_bf16(b), 64, 4)
    y = lin(dev_bf16(xb).view(2, 3, K))
    assert y.shape == (2, 3, N)
    y_ref = orc.quantized_matmul_f64(xb, orc.BF16, w, s, b, orc.BF16, True, 64, 4, N, K)
    assert orc.matmul_within_tolerance(host_f32(y).reshape(6, N), y_ref, True)[0]


def test_dequantize_bit_exact(cuda):
    for bits, gs, sdt in [(4, 64, orc.BF16), (8, 32, orc.F16), (2, 128, orc.F32), (4, 32, orc.F16)]:
        rows, cols = 96, 512
        w, s, b = synthetic_linear(rows, cols, gs, bits, bits + gs, scale_dtype=sdt)
        ref = orc.affine_dequant_f32(w, s, b, sdt, rows, cols, gs, bits)
        out = dequantize_with_mode(dev_words(w), dev_param(s, sdt), dev_param(b, sdt), gs, bits, dtype=torch.float32)
        assert np.array_equal(out.cpu().numpy(), ref)
        out16 = dequantize_with_mode(dev_words(w), dev_param(s, sdt), dev_param(b, sdt), gs, bits,
                                     dtype=torch.bfloat16)
        assert np.array_equal(host_bits16(out16), orc.f32_to_bf16_bits(ref))


def test_errors_surface_as_exceptions(cuda):
    x = torch.zeros(1, 96, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(16, 12, dtype=torch.int32, device="cuda")
    s = torch.zeros(16, 2, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(EreduError, match="group_size"):
        quantized_matmul(x, w, s, s, transpose=True, group_size=48)
    with pytest.raises(EreduError, match="incompatible"):
        quantized_matmul(x[:, :64], w, s, s, transpose=True, group_size=48)


def _batch_problems(specs, M, gs, bits, sdt=orc.BF16, seed=0, biases=True):
    """(x, w, s, b) device tensors plus host copies for each (N, K) in specs;
    problems with equal K share one activation tensor (as q/k/v do)."""
    xs, probs, host = {}, [], []
    for i, (N, K) in enumerate(specs):
        if K not in xs:
            xb = synthetic_x(M, K, seed + K)
            xs[K] = (xb, dev_bf16(xb))
        w, s, b = synthetic_linear(N, K, gs, bits, seed + 31 * i, scale_dtype=sdt)
        bd = dev_param(b, sdt) if biases or i % 2 else None
        probs.append((xs[K][1], dev_words(w), dev_param(s, sdt), bd))
        host.append((xs[K][0], w, s, b if bd is not None else None, N, K))
    return probs, host


@pytest.mark.parametrize("M", [1, 3, 8, 12, 16])
def test_batched_equals_separate_calls_bitwise(cuda, M):
    # a decoder layer's projections: q, k, v, o, gate, up (x of K=4096) and down (K=14336), scaled down.
    # Above 8 rows (two passes of the 4-bit group-64 decode kernel) the separate calls take the prefill
    # kernel where N % 128 == 0 and the decode kernel otherwise (N = 48): the batched call must match both.
    specs = [(512, 1024), (128, 1024), (128, 1024), (512, 512), (1792, 1024), (1792, 1024), (1024, 3584)]
    if M > 8:
        specs.append((48, 1024))
    probs, host = _batch_problems(specs, M, 64, 4, seed=M, biases=False)
    ys = quantized_matmul_batched(probs, transpose=True, group_size=64, bits=4)
    torch.cuda.synchronize()
    for (x, w, s, b), y, (xh, wh, sh, bh, N, K) in zip(probs, ys, host):
        y1 = quantized_matmul_with_mode(x, w, s, b, True, 64, 4)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y1.view(torch.int16))
        ref = orc.quantized_matmul_f64(xh, orc.BF16, wh, sh, bh, orc.BF16, True, 64, 4, N, K)
        assert orc.matmul_within_tolerance(host_f32(y), ref, True)[0]


@pytest.mark.parametrize("bits,gs,sdt", [(8, 32, orc.F16), (4, 128, orc.BF16), (4, 32, orc.F16)])
def test_batched_more_than_one_launch_and_contract_grid(cuda, bits, gs, sdt):
    # 11 problems (more than one grouped launch) with M = 5
    specs = [(16 * (i + 1), 256 * (1 + i % 3)) for i in range(11)]
    probs, host = _batch_problems(specs, 5, gs, bits, sdt=sdt, seed=bits + gs)
    ys = quantized_matmul_batched(probs, transpose=True, group_size=gs, bits=bits)
    torch.cuda.synchronize()
    for y, (xh, wh, sh, bh, N, K) in zip(ys, host):
        ref = orc.quantized_matmul_f64(xh, orc.BF16, wh, sh, bh, sdt, True, gs, bits, N, K)
        assert orc.matmul_within_tolerance(host_f32(y), ref, True)[0]


def test_batched_falls_back_per_problem(cuda):
    # transpose=False and N % 16 != 0 are not decode-grouped; results still match
    specs = [(40, 256), (48, 256)]
    probs, host = _batch_problems(specs, 2, 32, 4, seed=5)
    ys = quantized_matmul_batched(probs, transpose=True, group_size=32, bits=4)
    torch.cuda.synchronize()
    for y, (xh, wh, sh, bh, N, K) in zip(ys, host):
        ref = orc.quantized_matmul_f64(xh, orc.BF16, wh, sh, bh, orc.BF16, True, 32, 4, N, K)
        assert orc.matmul_within_tolerance(host_f32(y), ref, True)[0]
    with pytest.raises(EreduError, match="same number of activation rows"):
        x2 = torch.zeros(2, 256, dtype=torch.bfloat16, device="cuda")
        x3 = torch.zeros(3, 256, dtype=torch.bfloat16, device="cuda")
        quantized_matmul_batched([(x2, probs[0][1], probs[0][2], None), (x3, probs[0][1], probs[0][2], None)],
                                 group_size=32)


@pytest.mark.parametrize("M,K,gs,bits", [(8, 14336, 64, 4), (8, 14336, 64, 8), (5, 14336, 64, 4), (16, 8192, 128, 4),
                                         (2, 98304, 64, 4), (8, 12288, 64, 4)])
def test_qmv_activations_staged_in_k_phases(cuda, M, K, gs, bits):
    """Activations longer than one workgroup's LDS (M x K x 2 bytes) on a
    problem of at most one tile per workgroup: the decode kernel stages them
    in K phases (the down projection at batch 8 among them)."""
    run_case(M, 256, K, gs, bits, seed=M + K + bits)


@pytest.mark.parametrize("sdt", [orc.BF16, orc.F16])
@pytest.mark.parametrize("M,K", [(6, 2048), (8, 4096), (7, 2080), (8, 14336)])
def test_qmv_group32_two_row_sets(cuda, sdt, M, K):
    """4-bit group 32 at 5-8 activation rows: one pass of the decode kernel
    takes them as two sets of four rows (K a whole number of 512-code blocks;
    K = 2080 runs as 4-row passes, K = 14336 stages its activations in K
    phases).  Against the oracle, and each row bit-equal to the same row
    computed alone (M = 1), whichever pass structure took it."""
    N = 256
    w, s, b = synthetic_linear(N, K, 32, 4, seed=M + K, scale_dtype=sdt)
    xb = synthetic_x(M, K, seed=K + 3)
    wd, sd, bd = dev_words(w), dev_param(s, sdt), dev_param(b, sdt)
    y = quantized_matmul_with_mode(dev_bf16(xb), wd, sd, bd, True, 32, 4)
    torch.cuda.synchronize()
    ref = orc.quantized_matmul_f64(xb, orc.BF16, w, s, b, sdt, True, 32, 4, N, K)
    ok, worst, rms = orc.matmul_within_tolerance(host_f32(y), ref, True)
    assert ok, f"max|err|/RMS = {worst:.3e}"
    for m in range(M):
        y1 = quantized_matmul_with_mode(dev_bf16(xb[m:m + 1]), wd, sd, bd, True, 32, 4)
        torch.cuda.synchronize()
        assert torch.equal(y[m:m + 1].view(torch.int16), y1.view(torch.int16)), f"row {m}"


def test_batched_group32_two_row_sets_equal_separate_calls(cuda):
    # 8 rows of 4-bit group-32 problems whose K are whole blocks: the grouped
    # launch and the separate calls both take one two-row-set pass
    specs = [(256, 1024), (128, 1024), (384, 2048)]
    probs, host = _batch_problems(specs, 8, 32, 4, seed=32, biases=True)
    ys = quantized_matmul_batched(probs, transpose=True, group_size=32, bits=4)
    torch.cuda.synchronize()
    for (x, w, s, b), y, (xh, wh, sh, bh, N, K) in zip(probs, ys, host):
        y1 = quantized_matmul_with_mode(x, w, s, b, True, 32, 4)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y1.view(torch.int16))
        ref = orc.quantized_matmul_f64(xh, orc.BF16, wh, sh, bh, orc.BF16, True, 32, 4, N, K)
        assert orc.matmul_within_tolerance(host_f32(y), ref, True)[0]

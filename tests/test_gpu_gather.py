"""Parity of gather_qmm (eq_gather_qmm through the eredu_amd mirror) with the
oracle's fp64 gather_qmm_f64 on the same packed expert banks.

Tolerance (the matmul rule, per output batch): |y - y_ref| <= 1e-2 *
RMS(y_ref[b]) + 1/2 ulp_bf16(y_ref) for bf16 outputs, 1e-2 * RMS for f32.
Cases: the routed-expert decode of eredu/src/backend/mlx/nn/moe.rs:121-139
(x [routes, 1, K], lhs = arange, rhs = expert per route; the persistent
decode kernel where N % 16 == 0 and K is whole blocks, the team kernel
otherwise),
the general kernels (M > 1, transpose = false, f16 / f32 activations, 2-bit),
MLX's index broadcasting, out-of-range indices (zero rows), launches split at
65535 batches, and the sorted_indices hint.
"""
import numpy as np
import pytest
import torch

from eredu_amd import EreduError, gather_qmm, gather_qmm_with_mode
from oracle import oracle as orc
from tests.fixtures import dev_bf16, dev_param, dev_words, host_f32, synthetic_linear, synthetic_x

pytestmark = pytest.mark.gpu


def expert_bank(E, N, K, gs, bits, sdt, seed, transpose=True):
    rows, cols = (N, K) if transpose else (K, N)
    parts = [synthetic_linear(rows, cols, gs, bits, seed + e, scale_dtype=sdt) for e in range(E)]
    return tuple(np.stack([p[i] for p in parts]) for i in range(3))


def activations(Bx, M, K, xdt, seed):
    xb = synthetic_x(Bx * M, K, seed).reshape(Bx, M, K)
    if xdt == orc.BF16:
        return xb, dev_bf16(xb)
    xf = orc.bf16_bits_to_f32(xb)
    host = xf.astype(np.float16).view(np.uint16) if xdt == orc.F16 else xf
    return host, dev_param(host, xdt)


def check(y, y_ref, out_is_bf16):
    got = host_f32(y).reshape(-1, *y_ref.shape[-2:])
    ref = y_ref.reshape(-1, *y_ref.shape[-2:])
    for b in range(ref.shape[0]):
        if not ref[b].any():
            assert not got[b].any(), f"batch {b}: expected zero rows"
            continue
        ok, worst, _ = orc.matmul_within_tolerance(got[b], ref[b], out_is_bf16=out_is_bf16)
        assert ok, f"batch {b}: max|err|/RMS = {worst:.3e}"


def run(E, N, K, gs, bits, lhs, rhs, Bx, M=1, sdt=orc.BF16, xdt=orc.BF16, transpose=True, biases=True,
        seed=0, sorted_indices=False):
    print(f"[case] gather E={E} N={N} K={K} gs={gs} bits={bits} M={M} Bx={Bx} transpose={transpose} "
          f"xdt={xdt} sdt={sdt}", flush=True)
    w, s, b = expert_bank(E, N, K, gs, bits, sdt, seed, transpose)
    if not biases:
        b = None
    x_host, xd = activations(Bx, M, K, xdt, seed + 100)
    lt = None if lhs is None else torch.as_tensor(np.asarray(lhs), dtype=torch.int32).cuda()
    rt = None if rhs is None else torch.as_tensor(np.asarray(rhs), dtype=torch.int32).cuda()
    y = gather_qmm(xd, dev_words(w), dev_param(s, sdt), None if b is None else dev_param(b, sdt), lt, rt,
                   transpose=transpose, group_size=gs, bits=bits, sorted_indices=sorted_indices)
    torch.cuda.synchronize()
    y_ref = orc.gather_qmm_f64(x_host, xdt, w, s, b, sdt, lhs, rhs, transpose, gs, bits, N, K)
    assert tuple(y.shape) == y_ref.shape
    check(y, y_ref, out_is_bf16=xdt != orc.F32)
    return y


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("sdt", [orc.BF16, orc.F16])
def test_routed_decode(cuda, bits, gs, sdt):
    """12 routes over 8 experts (repeats included), N = 390 (a partial team)."""
    rhs = np.array([5, 0, 7, 5, 2, 2, 1, 6, 3, 0, 4, 7])
    run(8, 390, 1024, gs, bits, np.arange(12), rhs, Bx=12, sdt=sdt, seed=bits * gs, biases=(gs != 128))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("sdt", [orc.BF16, orc.F16])
def test_routed_decode_on_the_decode_kernel(cuda, bits, gs, sdt):
    """N % 16 == 0 and K whole blocks: the persistent decode kernel with the
    indices read on the device.  12 routes (two launches of up to 8), repeated
    experts and x rows, one x index and one expert index out of range (zero
    rows)."""
    lhs = np.array([0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 13, 2])
    rhs = np.array([5, 0, 7, 5, 2, -1, 1, 6, 3, 0, 4, 7])
    run(8, 256, 1024, gs, bits, lhs, rhs, Bx=12, sdt=sdt, seed=bits * gs + 5, biases=(gs != 128))


@pytest.mark.parametrize("K", [4096, 8192, 12288])
def test_routed_decode_team_counts(cuda, K):
    """4-bit chunks per row: 128, 256, 384 -> 4, 2, 1 teams per workgroup (two
    chunks per lane per step; at 384 a lane's second chunk is sometimes absent)."""
    run(3, 200, K, 64, 4, np.arange(4), np.array([2, 0, 1, 2]), Bx=4, seed=K)


def test_shared_activation_row(cuda):
    """One token routed to top-4 experts: x [1, 1, K], lhs absent (broadcast 0)."""
    run(6, 256, 2048, 64, 4, None, np.array([4, 1, 5, 0]), Bx=1)


def test_llama_sized_experts(cuda):
    """Two routes over two 4096 x 4096 experts (a Mixtral-like projection)."""
    run(2, 4096, 4096, 64, 4, np.arange(2), np.array([1, 0]), Bx=2, seed=11)


@pytest.mark.parametrize("transpose", [True, False])
@pytest.mark.parametrize("xdt,bits", [(orc.BF16, 4), (orc.F16, 8), (orc.F32, 2)])
def test_general_paths(cuda, transpose, xdt, bits):
    """M = 3 (the general kernels), both weight layouts, f16 / f32 activations."""
    run(4, 160, 256, 32, bits, np.array([2, 0, 1]), np.array([3, 3, 0]), Bx=3, M=3, xdt=xdt,
        transpose=transpose, seed=bits)


def test_broadcast_index_shapes(cuda):
    """lhs [2, 1] and rhs [1, 3] broadcast to a [2, 3] output batch."""
    y = run(4, 64, 128, 64, 4, np.array([[1], [0]]), np.array([[3, 0, 2]]), Bx=2, M=1, seed=5)
    assert tuple(y.shape) == (2, 3, 1, 64)


@pytest.mark.parametrize("M,transpose", [(1, True), (2, True), (2, False)])
def test_out_of_range_index_gives_zero_rows(cuda, M, transpose):
    run(3, 96, 128, 32, 4, np.array([0, 1, 5, 1]), np.array([2, -1, 0, 3]), Bx=2, M=M, transpose=transpose, seed=9)


@pytest.mark.parametrize("transpose", [True, False])
def test_batches_beyond_one_launch(cuda, transpose):
    """70000 batches: two launches (65535 + 4465); every batch checked."""
    E, N, K, gs, bits, B = 3, 32, 64, 32, 4, 70000
    print(f"[case] gather {B} batches transpose={transpose}", flush=True)
    w, s, b = expert_bank(E, N, K, gs, bits, orc.BF16, 21, transpose)
    x_host, xd = activations(7, 1, K, orc.BF16, 22)
    rng = np.random.default_rng(23)
    lhs, rhs = rng.integers(0, 7, B), rng.integers(0, E, B)
    y = gather_qmm(xd, dev_words(w), dev_bf16(s), dev_bf16(b), torch.as_tensor(lhs, dtype=torch.int32).cuda(),
                   torch.as_tensor(rhs, dtype=torch.int32).cuda(), transpose=transpose, group_size=gs, bits=bits)
    rows, cols = (N, K) if transpose else (K, N)
    W = np.stack([orc.affine_dequant_f64(w[e], s[e], b[e], orc.BF16, rows, cols, gs, bits) for e in range(E)])
    if transpose:
        W = W.transpose(0, 2, 1)  # [E, K, N]
    X = orc.bf16_bits_to_f32(x_host).astype(np.float64)[:, 0, :]  # [7, K]
    per = np.einsum("ik,ekn->ien", X, W)  # every (x row, expert) product
    y_ref = per[lhs, rhs][:, None, :]
    got = host_f32(y)
    ok, worst, _ = orc.matmul_within_tolerance(got, y_ref, out_is_bf16=True)
    assert ok, f"max|err|/RMS = {worst:.3e}"


def test_sorted_hint_does_not_change_results(cuda):
    w, s, b = expert_bank(4, 128, 512, 64, 4, orc.BF16, 31)
    _, xd = activations(6, 1, 512, orc.BF16, 32)
    rhs = torch.tensor([0, 0, 1, 2, 2, 3], dtype=torch.int32).cuda()
    args = (xd, dev_words(w), dev_bf16(s), dev_bf16(b), torch.arange(6, dtype=torch.int32).cuda(), rhs)
    y0 = gather_qmm(*args, sorted_indices=False)
    y1 = gather_qmm(*args, sorted_indices=True)
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))


def test_mirror_rejects_bad_arguments(cuda):
    w, s, b = expert_bank(2, 64, 128, 64, 4, orc.BF16, 41)
    _, xd = activations(2, 1, 128, orc.BF16, 42)
    W, S, B = dev_words(w), dev_bf16(s), dev_bf16(b)
    with pytest.raises(EreduError, match="broadcast"):
        gather_qmm(xd, W, S, B, torch.zeros(3, dtype=torch.int32).cuda(), torch.zeros(2, dtype=torch.int32).cuda())
    with pytest.raises(EreduError, match="integer"):
        gather_qmm(xd, W, S, B, None, torch.zeros(2).cuda())
    with pytest.raises(EreduError, match="batch dimensions"):
        gather_qmm(xd, W, S[:1], B)
    with pytest.raises(EreduError, match="no biases"):
        gather_qmm_with_mode(xd, W, S, B, None, None, True, 32, 4, False, mode=_mxfp4())


def _mxfp4():
    from eredu_amd import QuantizationMode

    return QuantizationMode("mxfp4")


@pytest.mark.parametrize("bits,gs", [(4, 64), (8, 32)])
def test_batched_quantized_matmul_kv_attention(cuda, bits, gs):
    """The quantized KV attention of eredu/src/backend/mlx/nn/tensor.rs:76-150
    at one decode position: queries [1, n_kv, n_rep, 1, D] against keys and
    values [1, n_kv, 1, T, D*bits/32] through quantized_matmul's batch
    broadcasting (scores with transpose = true, then softmax, then the values
    with transpose = false); each product against gather_qmm_f64 with the
    broadcast indices, and the whole attention against an f64 softmax."""
    from eredu_amd import quantized_matmul

    n_kv, n_rep, T, D = 2, 4, 256, 128
    print(f"[case] quantized KV attention bits={bits} gs={gs} T={T}", flush=True)
    keys = expert_bank(n_kv, T, D, gs, bits, orc.BF16, 51, transpose=True)       # [n_kv, T, D*bits/32]
    vals = expert_bank(n_kv, D, T, gs, bits, orc.BF16, 61, transpose=False)      # [n_kv, T, D*bits/32]
    q_host, qd = activations(n_kv * n_rep, 1, D, orc.BF16, 71)
    lhs = np.arange(n_kv * n_rep).reshape(1, n_kv, n_rep)
    rhs = np.arange(n_kv).reshape(1, n_kv, 1)

    def dev(bank):
        w, s, b = bank
        shape = (1, n_kv, 1)
        return (dev_words(w).reshape(*shape, *w.shape[1:]), dev_bf16(s).reshape(*shape, *s.shape[1:]),
                dev_bf16(b).reshape(*shape, *b.shape[1:]))

    kw, ks, kb = dev(keys)
    vw, vs, vb = dev(vals)
    q5 = qd.reshape(1, n_kv, n_rep, 1, D)
    scores = quantized_matmul(q5, kw, ks, kb, transpose=True, group_size=gs, bits=bits)
    assert tuple(scores.shape) == (1, n_kv, n_rep, 1, T)
    s_ref = orc.gather_qmm_f64(q_host, orc.BF16, *keys, orc.BF16, lhs, rhs, True, gs, bits, T, D)
    check(scores, s_ref, out_is_bf16=True)

    probs = torch.softmax(scores.float() / np.sqrt(D), dim=-1).to(torch.bfloat16)
    out = quantized_matmul(probs, vw, vs, vb, transpose=False, group_size=gs, bits=bits)
    assert tuple(out.shape) == (1, n_kv, n_rep, 1, D)
    p_host = host_f32(probs).reshape(n_kv * n_rep, 1, T)
    p_bits = orc.f32_to_bf16_bits(p_host)
    o_ref = orc.gather_qmm_f64(p_bits, orc.BF16, *vals, orc.BF16, lhs, rhs, False, gs, bits, D, T)
    check(out, o_ref, out_is_bf16=True)

    # the composition against an f64 attention over the dequantized caches;
    # tolerance 2e-2 RMS: the bf16 roundings of the scores and probabilities
    # (2^-9 relative each) come on top of the two products' own 1e-2 rule
    Kd = [orc.affine_dequant_f64(keys[0][h], keys[1][h], keys[2][h], orc.BF16, T, D, gs, bits) for h in range(n_kv)]
    Vd = [orc.affine_dequant_f64(vals[0][h], vals[1][h], vals[2][h], orc.BF16, T, D, gs, bits) for h in range(n_kv)]
    q64 = orc.bf16_bits_to_f32(q_host).astype(np.float64).reshape(n_kv, n_rep, D)
    att = np.empty((n_kv, n_rep, D))
    for h in range(n_kv):
        sc = q64[h] @ Kd[h].T / np.sqrt(D)
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        att[h] = (p / p.sum(axis=1, keepdims=True)) @ Vd[h]
    got = host_f32(out).reshape(n_kv, n_rep, D)
    rms = np.sqrt(np.mean(att ** 2))
    assert np.max(np.abs(got - att)) <= 2e-2 * rms, np.max(np.abs(got - att)) / rms


# ------------------------------------------------ grouped (sorted, many routes)
# sorted_indices with >= 64 routes and >= 2 routes per expert: the routes of
# an expert run as one MFMA GEMM (qmm_mfma_kernel over a device-built tile
# list).  Same tolerance rule; experts with 0, 1..127 and > 128 routes.

def sorted_routes(E, R, seed, lo=0, hi=None):
    rng = np.random.default_rng(seed)
    hi = E if hi is None else hi
    # skewed: expert 1 gets many routes (several 128-row tiles), expert E-1 none
    r = np.concatenate([np.full(R // 3, 1), rng.integers(lo, hi - 1, R - R // 3)])
    return np.sort(r)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("sdt", [orc.BF16, orc.F16])
def test_grouped_routes(cuda, bits, gs, sdt):
    E, R = 6, 420
    rhs = sorted_routes(E, R, seed=bits + gs)
    run(E, 384, 512, gs, bits, np.arange(R), rhs, Bx=R, sdt=sdt, seed=bits * gs + 7, sorted_indices=True,
        biases=(gs != 32))


def test_grouped_routes_out_of_range_and_shared_rows(cuda):
    """Sorted expert ids with -1 at the front and 99 at the back (zero rows),
    one lhs out of range (zero row), lhs repeating rows (a token routed to
    several experts)."""
    E, R = 4, 200
    rhs = np.concatenate([[-1, -1], sorted_routes(E, R - 5, seed=3), [99, 99, 99]])
    lhs = np.arange(R) // 2
    lhs[10] = 10_000
    run(E, 256, 256, 64, 4, lhs, rhs, Bx=R // 2, seed=13, sorted_indices=True)


def test_grouped_and_per_route_paths_on_a_mixtral_like_layout(cuda):
    """8 experts of 1024 x 4096, 256 sorted routes: the grouped GEMM (sorted
    hint) and the per-route kernel (no hint) each within the matmul rule of
    the fp64 oracle (two bf16 results may differ by one ulp of each other)."""
    E, R, N, K = 8, 256, 1024, 4096
    w, s, b = expert_bank(E, N, K, 64, 4, orc.BF16, 77)
    x_host, xd = activations(R, 1, K, orc.BF16, 78)
    rhs_np = sorted_routes(E, R, seed=79)
    rhs = torch.as_tensor(rhs_np, dtype=torch.int32).cuda()
    lhs = torch.arange(R, dtype=torch.int32).cuda()
    args = (xd, dev_words(w), dev_bf16(s), dev_bf16(b), lhs, rhs)
    y_ref = orc.gather_qmm_f64(x_host, orc.BF16, w, s, b, orc.BF16, np.arange(R), rhs_np, True, 64, 4, N, K)
    for hint in (True, False):
        y = gather_qmm(*args, sorted_indices=hint)
        check(y, y_ref, out_is_bf16=True)

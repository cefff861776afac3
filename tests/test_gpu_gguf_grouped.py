"""Native GGUF grouped linear on the device (eq_gguf_grouped_linear,
gguf.native_grouped_linear): y[r] = x[r] . W[ids[r]]^T over an expert bank
kept in its blocks, against the fp64 product with the oracle's native decode
of each route's expert, within the matmul rule (|y - ref| <= 1e-2 RMS(ref) +
1/2 ulp bf16).  Both regimes: up to 16 routes (each route's matrix copied and
run through the native M = 1 linear) and more (the bank re-packed once, then
the grouped matrix-core product for sorted ids or the gathered product for
unsorted ones)."""
import numpy as np
import pytest
import torch

from eredu_amd import EreduError, _native
from eredu_amd import gguf as G
from oracle import oracle as orc
from tests.fixtures import dev_bf16, dev_u8, host_f32, synthetic_blocks, synthetic_x

pytestmark = pytest.mark.gpu

T = G.GgmlType


def bank(ty, experts, N, K, seed):
    vals, _ = ty.block_and_bytes()
    raw = synthetic_blocks(int(ty), experts * N * K // vals, seed=seed)
    w = orc.gguf_dequant_f32(int(ty), raw, 1).astype(np.float64).reshape(experts, N, K)
    return raw, w


def run(ty, experts, N, K, ids, seed, repacked=False):
    """Against the fp64 product with each route's native expert (1e-2 for
    the native kernels).  repacked (more than 16 routes): the kernel takes
    the affine route's weights (f16 group factors, as convert_affine), so it
    is held to 1e-2 against that product, and to 3e-2 against the native one (on these synthetic blocks the f16 rounding of
    Q4_K's d * sc alone reaches 2.3e-2 at K = 512)."""
    raw, w = bank(ty, experts, N, K, seed)
    nt = G.NativeTensor("blk.0.ffn_gate_exps.weight", [experts, N, K], ty, G.Endian.Little, dev_u8(raw))
    xb = synthetic_x(len(ids), K, seed + 1)
    y = host_f32(G.native_grouped_linear(dev_bf16(xb), nt, torch.tensor(ids, device="cuda")))
    xf = orc.bf16_bits_to_f32(xb).astype(np.float64)
    ref = np.stack([xf[r] @ w[e].T for r, e in enumerate(ids)])
    ok, worst, _ = orc.matmul_within_tolerance(y, ref, True, rel=3e-2 if repacked else 1e-2)
    assert ok, (ty.name, len(ids), worst)
    if repacked:
        # the matrix-core kernels (sorted ids, >= 64 routes) take the weights
        # in bf16, the gathered vector kernels (fewer or unsorted routes)
        # apply the f16 factors in f32: within 1e-2 of the product it computes
        wa = orc.gguf_dequant_f32(int(ty), raw, 0).reshape(experts, N, K)
        worsts = []
        for w_model in (wa.astype(np.float64), orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(wa)).astype(np.float64)):
            ref = np.stack([xf[r] @ w_model[e].T for r, e in enumerate(ids)])
            worsts.append(orc.matmul_within_tolerance(y, ref, True))
        assert any(ok for ok, _, _ in worsts), (ty.name, len(ids), "repacked", [w for _, w, _ in worsts])


@pytest.mark.parametrize("ty", [T.Q4K, T.Q5K, T.Q6K, T.Q5_1, T.Q8_0, T.IQ4NL, T.IQ4XS])
def test_decode_routes(cuda, ty):
    print(f"[case] grouped decode {ty.name}", flush=True)
    run(ty, 4, 200, 512, [2, 0, 3, 2], seed=int(ty))  # unsorted, repeated
    run(ty, 4, 256, 1024, [1], seed=int(ty) + 7)


@pytest.mark.parametrize("ty", [T.Q4K, T.Q5K, T.Q6K, T.Q5_1, T.Q8_0, T.IQ4NL, T.IQ4XS])
def test_prefill_routes_sorted_and_unsorted(cuda, ty):
    rng = np.random.default_rng(int(ty))
    ids = np.sort(rng.integers(0, 4, 96)).tolist()  # sorted: the grouped matrix-core product
    print(f"[case] grouped prefill {ty.name} sorted", flush=True)
    run(ty, 4, 256, 512, ids, seed=int(ty) + 3, repacked=True)
    print(f"[case] grouped prefill {ty.name} unsorted", flush=True)
    run(ty, 4, 256, 512, rng.permutation(ids).tolist(), seed=int(ty) + 4, repacked=True)
    print(f"[case] grouped prefill {ty.name} 20 routes", flush=True)
    run(ty, 3, 128, 256, rng.integers(0, 3, 20).tolist(), seed=int(ty) + 5, repacked=True)


def test_errors_and_out_of_range_rows(cuda):
    raw, w = bank(T.Q8_0, 2, 128, 256, seed=1)
    nt = G.NativeTensor("e", [2, 128, 256], T.Q8_0, G.Endian.Little, dev_u8(raw))
    x = dev_bf16(synthetic_x(3, 256, 2))
    with pytest.raises(EreduError, match=r"native grouped expert 2 is outside 0\.\.2"):
        G.native_grouped_linear(x, nt, torch.tensor([0, 2, 1], device="cuda"))
    with pytest.raises(EreduError, match="shape mismatch"):
        G.native_grouped_linear(x, nt, torch.tensor([0, 1], device="cuda"))
    # through the C ABI an id outside the bank gives a +0 row, in both regimes
    for routes in (3, 40):
        ids = torch.tensor(([0, 5, 1] * 14)[:routes], dtype=torch.int32, device="cuda")
        xb = synthetic_x(routes, 256, 3)
        xd = dev_bf16(xb)
        y = torch.full((routes, 128), 1.0, dtype=torch.bfloat16, device="cuda")
        d = dev_u8(raw)
        _native.check(_native.lib().eq_gguf_grouped_linear(
            y.data_ptr(), xd.data_ptr(), d.data_ptr(), d.numel(), int(T.Q8_0), 2, 128, 256, ids.data_ptr(), routes,
            0, _native.EQ_DTYPE_BF16, False, torch.cuda.current_stream().cuda_stream))
        got = host_f32(y)
        idl = ids.cpu().numpy()
        assert np.all(got[idl == 5].view(np.uint32) == 0)
        xf = orc.bf16_bits_to_f32(xb).astype(np.float64)
        good = np.nonzero(idl != 5)[0]
        ref = np.stack([xf[r] @ w[idl[r]].T for r in good])
        ok, worst, _ = orc.matmul_within_tolerance(got[good], ref, True)
        assert ok, (routes, worst)

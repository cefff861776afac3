"""Pins of the oracle's gather_qmm restatement (CPU only): closed forms that
fail if lhs and rhs are swapped, broadcast wrongly or an index is dropped."""
import numpy as np

from oracle import oracle as O


def _constant_experts(E, N, K, gs, bits):
    """Expert e dequantizes to the constant e + 1 everywhere: codes 0, scale 0,
    bias e + 1 (f32 parameters)."""
    w = np.zeros((E, N, K * bits // 32), dtype=np.uint32)
    s = np.zeros((E, N, K // gs), dtype=np.float32)
    b = np.stack([np.full((N, K // gs), e + 1.0, dtype=np.float32) for e in range(E)])
    return w, s, b


def test_gather_closed_form_and_broadcast():
    E, N, K, gs, bits, M = 5, 3, 64, 32, 4, 2
    w, s, b = _constant_experts(E, N, K, gs, bits)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((4, M, K)).astype(np.float32)
    lhs = np.array([[3], [0]])          # [2, 1]
    rhs = np.array([[4, 1, 2]])         # [1, 3]
    y = O.gather_qmm_f64(x, O.F32, w, s, b, O.F32, lhs, rhs, True, gs, bits, N, K)
    assert y.shape == (2, 3, M, N)
    for i in range(2):
        for j in range(3):
            expect = (rhs[0, j] + 1) * x[lhs[i, 0]].astype(np.float64).sum(axis=1)
            assert np.allclose(y[i, j], expect[:, None] * np.ones((1, N)))


def test_gather_defaults_and_out_of_range():
    E, N, K, gs, bits, M = 3, 2, 32, 32, 8, 1
    w, s, b = _constant_experts(E, N, K, gs, bits)
    x = np.arange(3 * M * K, dtype=np.float32).reshape(3, M, K) / 100.0
    y = O.gather_qmm_f64(x, O.F32, w, s, b, O.F32, None, None, True, gs, bits, N, K)  # b -> (b, b)
    for e in range(3):
        assert np.allclose(y[e], (e + 1) * x[e].astype(np.float64).sum())
    y = O.gather_qmm_f64(x, O.F32, w, s, b, O.F32, np.array([0, 1]), np.array([2, 7]), True, gs, bits, N, K)
    assert np.allclose(y[0], 3 * x[0].astype(np.float64).sum())
    assert np.all(y[1] == 0.0)  # expert 7 does not exist


def test_gather_transpose_false_closed_form():
    E, N, K, gs, bits, M = 2, 64, 8, 32, 4, 3
    w = np.zeros((E, K, N * bits // 32), dtype=np.uint32)
    s = np.zeros((E, K, N // gs), dtype=np.float32)
    b = np.stack([np.full((K, N // gs), 2.0 * e - 1.0, dtype=np.float32) for e in range(E)])
    x = np.random.default_rng(1).standard_normal((1, M, K)).astype(np.float32)
    y = O.gather_qmm_f64(x, O.F32, w, s, b, O.F32, np.array([0, 0]), np.array([1, 0]), False, gs, bits, N, K)
    sums = x[0].astype(np.float64).sum(axis=1)[:, None]
    assert np.allclose(y[0], 1.0 * sums) and np.allclose(y[1], -1.0 * sums)

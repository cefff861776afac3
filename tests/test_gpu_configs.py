"""Parity at the measured configurations themselves (BASELINE configs[2] and
configs[4]), against the fp64 oracle on the same packed inputs.

* configs[2] prefill: M in {128, 512, 2048} x the four Llama-3-8B shapes x
  4- and 8-bit codes, group 64 -- every launch plan the bench times (split K
  at small grids, the unsplit kernel at M = 2048 with K = 4096 and 14336).
  y is checked on a seeded subset of 64 rows (every column), including the
  first and last row of a 128-row tile.
* configs[4] decode: the 4-bit LM head at N = 128256 (8016 row tiles, a
  262 MB weight buffer) on a seeded subset of output features; one
  full-size layer (H 4096, 32/8 heads, FFN 14336, 1024 cached positions)
  against oracle/decode_oracle.py, fused and unfused; three such layers in
  one step against the oracle (the residual stream and the fused decoder's
  buffer alternation across layers); and the whole 32-layer,
  vocab-128256 step, where the fused and unfused decoders must agree on the
  greedy token over three consecutive positions.

Tolerance (the north star's rule, written here): elementwise
|y - y_ref| <= 1e-2 * RMS(y_ref) + 1/2 ulp_bf16(y_ref) for a bf16 result of
one quantized matmul; logits after a layer of bf16-rounded ops within
2e-2 * RMS(ref) + 1/2 ulp (as tests/test_gpu_decode.py states).
"""
import numpy as np
import pytest
import torch

from eredu_amd import decode as E
from eredu_amd import quantized_matmul_with_mode
from oracle import decode_oracle as D
from oracle import oracle as orc
from tests.fixtures import (dev_bf16, dev_words, device_random_linear, host_bits16, host_f32, host_rows,
                            synthetic_linear, synthetic_x)

pytestmark = pytest.mark.gpu

LLAMA_SHAPES = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]


def row_subset(M, seed, count=64):
    rng = np.random.default_rng(seed)
    edges = {0, min(127, M - 1), min(128, M - 1), M - 1}
    picks = set(rng.choice(M, size=min(count, M), replace=False).tolist()) | edges
    return np.array(sorted(picks))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("N,K", LLAMA_SHAPES)
def test_prefill_config2(cuda, N, K, bits):
    w, s, b = synthetic_linear(N, K, 64, bits, seed=N + 3 * K + bits)
    W = orc.affine_dequant_f64(w, s, b, orc.BF16, N, K, 64, bits)
    wd, sd, bd = dev_words(w), dev_bf16(s), dev_bf16(b)
    for M in (128, 512, 2048):
        print(f"[case] prefill M={M} N={N} K={K} bits={bits}", flush=True)
        xb = synthetic_x(M, K, seed=M + N + bits)
        y = quantized_matmul_with_mode(dev_bf16(xb), wd, sd, bd, True, 64, bits)
        torch.cuda.synchronize()
        rows = row_subset(M, seed=M + K)
        ref = orc.bf16_bits_to_f32(xb[rows]).astype(np.float64) @ W.T
        got = host_f32(y)[rows]
        ok, worst, _ = orc.matmul_within_tolerance(got, ref, out_is_bf16=True)
        assert ok, f"M={M}: max|err|/RMS = {worst:.3e}"


def test_lm_head_vocab_128256(cuda):
    N, K = 128256, 4096
    print(f"[case] LM head qmv N={N} K={K}", flush=True)
    w, s, b = device_random_linear(N, K, 64, 4, seed=11)
    xb = synthetic_x(1, K, seed=12)
    y = quantized_matmul_with_mode(dev_bf16(xb), w, s, b, True, 64, 4)
    torch.cuda.synchronize()
    rng = np.random.default_rng(13)
    n_sel = np.unique(np.concatenate([rng.choice(N, 4096, replace=False), [0, 15, 16, 8015 * 16, N - 1]]))
    wr, sr, br = host_rows(w, s, b, n_sel)
    ref = orc.quantized_matmul_f64(xb, orc.BF16, wr, sr, br, orc.BF16, True, 64, 4, len(n_sel), K)
    got = host_f32(y).reshape(-1)[n_sel]
    ok, worst, _ = orc.matmul_within_tolerance(got.reshape(1, -1), ref, out_is_bf16=True)
    assert ok, f"max|err|/RMS = {worst:.3e}"


@pytest.mark.parametrize("M", [1, 32])
def test_weight_beyond_2_31_bytes(cuda, M):
    """An 8-bit 262144 x 8192 weight holds 2^31 bytes of codes, past the
    32-bit buffer offsets of the kernels: the prefill launcher runs it in row
    pieces of 261888 rows (multiples of the 256-column tile), the decode
    launcher in row chunks below 2^31 bytes.  Output features on both sides
    of the piece boundary, the first and the last are checked against the
    oracle."""
    N, K, bits = 262144, 8192, 8
    boundary = ((2**31 - 1) // K) // 256 * 256  # 261888
    print(f"[case] weight beyond 2^31 bytes M={M} N={N} K={K} bits={bits}", flush=True)
    w, s, b = device_random_linear(N, K, 64, bits, seed=31 + M)
    assert w.numel() * 4 == 2**31
    xb = synthetic_x(M, K, seed=32 + M)
    y = quantized_matmul_with_mode(dev_bf16(xb), w, s, b, True, 64, bits)
    torch.cuda.synchronize()
    rng = np.random.default_rng(33)
    n_sel = np.unique(np.concatenate([np.arange(boundary - 160, boundary + 160), [0, 1, N - 2, N - 1],
                                      rng.choice(N, 256, replace=False)]))
    wr, sr, br = host_rows(w, s, b, n_sel)
    ref = orc.quantized_matmul_f64(xb, orc.BF16, wr, sr, br, orc.BF16, True, 64, bits, len(n_sel), K)
    got = host_f32(y)[:, n_sel]
    del w, s, b, y
    torch.cuda.empty_cache()
    ok, worst, _ = orc.matmul_within_tolerance(got, ref, out_is_bf16=True)
    assert ok, f"max|err|/RMS = {worst:.3e}"


def _bits(x):
    return orc.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


@pytest.fixture(scope="module")
def full_layer_model():
    """One Llama-3-8B-sized layer (host weights from the oracle's quantizer),
    a 1024-row vocabulary and caches holding 1024 positions."""
    H, nh, nkv, F, V, max_seq = 4096, 32, 8, 14336, 1024, 1040
    rng = np.random.default_rng(21)

    def lin(N, K, seed):
        w, sc, b = synthetic_linear(N, K, 64, 4, seed)
        return {"w": w, "s": sc, "b": b, "bits": 4, "gs": 64}

    host = {"hidden": H, "n_heads": nh, "n_kv_heads": nkv, "eps": 1e-5,
            "freqs": D.llama3_rope_freqs(128, 500000.0),
            "embed": _bits(rng.standard_normal((V, H))), "final_norm": _bits(1.0 + 0.1 * rng.standard_normal(H)),
            "layers": [{"in_norm": _bits(1.0 + 0.1 * rng.standard_normal(H)),
                        "post_norm": _bits(1.0 + 0.1 * rng.standard_normal(H)),
                        "q": lin(nh * 128, H, 1), "k": lin(nkv * 128, H, 2), "v": lin(nkv * 128, H, 3),
                        "o": lin(H, nh * 128, 4), "gate": lin(F, H, 5), "up": lin(F, H, 6), "down": lin(H, F, 7)}],
            "lm_head": lin(V, H, 8)}
    kc = _bits(np.random.default_rng(22).standard_normal((nkv, max_seq, 128)))
    vc = _bits(np.random.default_rng(23).standard_normal((nkv, max_seq, 128)))
    return host, kc, vc, max_seq


@pytest.mark.parametrize("fused", [False, True])
def test_full_size_layer_against_the_oracle(cuda, full_layer_model, fused):
    host, kc, vc, max_seq = full_layer_model
    pos, token = 1024, 77
    print(f"[case] full-size layer fused={fused} pos={pos}", flush=True)

    def qlin(d):
        return E.QLinear(dev_words(d["w"]), dev_bf16(d["s"]), dev_bf16(d["b"]), 4, 64)

    L = host["layers"][0]
    layer = E.DecoderLayer(dev_bf16(L["in_norm"]), dev_bf16(L["post_norm"]),
                           *(qlin(L[p]) for p in ("q", "k", "v", "o", "gate", "up", "down")))
    dec = E.LlamaDecoder([layer], dev_bf16(host["embed"]), dev_bf16(host["final_norm"]), qlin(host["lm_head"]),
                         n_heads=32, n_kv_heads=8, eps=1e-5, freqs=host["freqs"], max_seq=max_seq,
                         k_caches=[dev_bf16(kc)], v_caches=[dev_bf16(vc)], fused=fused)
    dec.token.fill_(token)
    dec.step(pos)
    torch.cuda.synchronize()
    kcs, vcs = [kc.copy()], [vc.copy()]
    logits_ref, _ = D.decode_step(host, token, pos, kcs, vcs)
    got = host_f32(dec.logits)
    rms = np.sqrt(np.mean(logits_ref ** 2))
    err = np.abs(got - logits_ref)
    assert np.all(err <= 2e-2 * rms + orc.bf16_half_ulp(logits_ref)), f"max|err|/RMS = {err.max() / rms:.3e}"
    # the cache row written at pos holds the value projection (one quantized
    # matmul: the matmul rule against the oracle's f64 product)
    v_ref = orc.bf16_bits_to_f32(vcs[0][:, pos]).astype(np.float64).reshape(1, -1)
    v_got = orc.bf16_bits_to_f32(host_bits16(dec.v_caches[0])[:, pos]).reshape(1, -1)
    assert orc.matmul_within_tolerance(v_got, v_ref, out_is_bf16=True, rel=1e-2)[0]


@pytest.fixture(scope="module")
def three_layer_model():
    """Three Llama-3-8B-sized layers (host weights from the oracle's
    quantizer, each layer its own seeds), a 1024-row vocabulary and caches
    holding 1024 positions per layer."""
    H, nh, nkv, F, V, max_seq, layers = 4096, 32, 8, 14336, 1024, 1040, 3
    rng = np.random.default_rng(41)

    def lin(N, K, seed):
        w, sc, b = synthetic_linear(N, K, 64, 4, seed)
        return {"w": w, "s": sc, "b": b, "bits": 4, "gs": 64}

    host = {"hidden": H, "n_heads": nh, "n_kv_heads": nkv, "eps": 1e-5,
            "freqs": D.llama3_rope_freqs(128, 500000.0),
            "embed": _bits(rng.standard_normal((V, H))), "final_norm": _bits(1.0 + 0.1 * rng.standard_normal(H)),
            "layers": [{"in_norm": _bits(1.0 + 0.1 * rng.standard_normal(H)),
                        "post_norm": _bits(1.0 + 0.1 * rng.standard_normal(H)),
                        "q": lin(nh * 128, H, 50 + 10 * i), "k": lin(nkv * 128, H, 51 + 10 * i),
                        "v": lin(nkv * 128, H, 52 + 10 * i), "o": lin(H, nh * 128, 53 + 10 * i),
                        "gate": lin(F, H, 54 + 10 * i), "up": lin(F, H, 55 + 10 * i), "down": lin(H, F, 56 + 10 * i)}
                       for i in range(layers)],
            "lm_head": lin(V, H, 49)}
    kcs = [_bits(np.random.default_rng(60 + i).standard_normal((nkv, max_seq, 128))) for i in range(layers)]
    vcs = [_bits(np.random.default_rng(70 + i).standard_normal((nkv, max_seq, 128))) for i in range(layers)]
    return host, kcs, vcs, max_seq


@pytest.mark.parametrize("fused", [False, True])
def test_three_full_size_layers_against_the_oracle(cuda, three_layer_model, fused):
    """Three layers in one step against oracle/decode_oracle.py: what one
    layer cannot show -- the residual stream carried from layer to layer, the
    fused decoder's hidden state alternating between its two buffers (layer
    0 reads the embedding row, later layers the other buffer) and each
    layer's cache -- with every projection kernel the 32-layer step runs.
    The final hidden state (bf16, after three layers' roundings) and the
    logits are checked against the oracle's: RMS(err) <= 2e-2 * RMS(ref) and
    every |err| <= 8e-2 * RMS(ref) + 1/2 ulp -- a one-ulp bf16 difference
    where device and oracle round a sum on opposite sides of a tie grows
    through the later layers (measured: RMS 7.6e-3, max 2.9e-2 of RMS),
    while a wrong buffer, residual or cache makes errors of the order of
    the values themselves.  Every layer's new cache row (one value
    projection each) is checked at the matmul rule."""
    host, kcs0, vcs0, max_seq = three_layer_model
    pos, token = 1024, 321
    print(f"[case] three full-size layers fused={fused} pos={pos}", flush=True)

    def qlin(d):
        return E.QLinear(dev_words(d["w"]), dev_bf16(d["s"]), dev_bf16(d["b"]), 4, 64)

    layers = [E.DecoderLayer(dev_bf16(L["in_norm"]), dev_bf16(L["post_norm"]),
                             *(qlin(L[p]) for p in ("q", "k", "v", "o", "gate", "up", "down")))
              for L in host["layers"]]
    dec = E.LlamaDecoder(layers, dev_bf16(host["embed"]), dev_bf16(host["final_norm"]), qlin(host["lm_head"]),
                         n_heads=32, n_kv_heads=8, eps=1e-5, freqs=host["freqs"], max_seq=max_seq,
                         k_caches=[dev_bf16(k) for k in kcs0], v_caches=[dev_bf16(v) for v in vcs0], fused=fused)
    assert dec.swiglu == fused
    dec.token.fill_(token)
    dec.step(pos)
    torch.cuda.synchronize()
    kcs, vcs = [k.copy() for k in kcs0], [v.copy() for v in vcs0]
    logits_ref, x_ref = D.decode_step(host, token, pos, kcs, vcs)
    # the hidden state after the last layer: the residual sum the final norm
    # writes back (unfused: dec.x; fused: the buffer the LM head's prologue
    # reads plus the last down projection -- compared through the logits)
    got = host_f32(dec.logits)
    rms = np.sqrt(np.mean(logits_ref ** 2))
    err = np.abs(got - logits_ref)
    print(f"  logits max|err|/RMS = {err.max() / rms:.3e}, RMS(err)/RMS = {np.sqrt(np.mean(err ** 2)) / rms:.3e}",
          flush=True)
    assert np.sqrt(np.mean(err ** 2)) <= 2e-2 * rms, f"RMS(err)/RMS = {np.sqrt(np.mean(err ** 2)) / rms:.3e}"
    assert np.all(err <= 8e-2 * rms + orc.bf16_half_ulp(logits_ref)), f"max|err|/RMS = {err.max() / rms:.3e}"
    if not fused:
        hx = orc.bf16_bits_to_f32(host_bits16(dec.x)).astype(np.float64)
        hr = orc.bf16_bits_to_f32(x_ref).astype(np.float64)
        hrms = np.sqrt(np.mean(hr ** 2))
        herr = np.abs(hx - hr)
        print(f"  hidden max|err|/RMS = {herr.max() / hrms:.3e}", flush=True)
        assert np.sqrt(np.mean(herr ** 2)) <= 2e-2 * hrms, "hidden RMS(err)"
        assert np.all(herr <= 8e-2 * hrms + orc.bf16_half_ulp(hr)), f"hidden max|err|/RMS = {herr.max() / hrms:.3e}"
    for li in range(len(layers)):
        v_ref = orc.bf16_bits_to_f32(vcs[li][:, pos]).astype(np.float64).reshape(1, -1)
        v_got = orc.bf16_bits_to_f32(host_bits16(dec.v_caches[li])[:, pos]).reshape(1, -1)
        assert orc.matmul_within_tolerance(v_got, v_ref, out_is_bf16=True, rel=2e-2)[0], f"layer {li} value row"
        # rows other than pos are untouched
        assert np.array_equal(host_bits16(dec.v_caches[li])[:, :pos], vcs0[li][:, :pos]), f"layer {li} cache"


def test_full_model_fused_and_unfused_agree(cuda):
    """configs[4] at full size: 32 layers, vocabulary 128256, 1024 cached
    positions; both decoders step three positions from the same token and
    caches and must pick the same greedy tokens.  The two differ only in
    the order of the RMSNorm sums of squares, so their logits differ by bf16
    roundings that 32 random layers amplify: RMS(fused - unfused) must stay
    within 3e-2 * RMS(logits), and a near-tie -- the unfused logits of the
    two candidates closer than twice the largest fused/unfused difference --
    counts as agreement (both then continue from the fused token)."""
    H, nh, nkv, F, V, layers, max_seq = 4096, 32, 8, 14336, 128256, 32, 1040
    g = torch.Generator(device="cuda").manual_seed(31)
    bf = torch.bfloat16

    def qlin(N, K, seed):
        w, s, b = device_random_linear(N, K, 64, 4, seed)
        return E.QLinear(w, s, b, 4, 64)

    def norm():
        return (1.0 + 0.1 * torch.randn(H, device="cuda", generator=g)).to(bf)

    dev_layers = [E.DecoderLayer(norm(), norm(), qlin(nh * 128, H, 100 + 10 * i), qlin(nkv * 128, H, 101 + 10 * i),
                                 qlin(nkv * 128, H, 102 + 10 * i), qlin(H, nh * 128, 103 + 10 * i),
                                 qlin(F, H, 104 + 10 * i), qlin(F, H, 105 + 10 * i), qlin(H, F, 106 + 10 * i))
                  for i in range(layers)]
    embed = torch.randn((V, H), device="cuda", generator=g).to(bf)
    final_norm = norm()
    lm_head = qlin(V, H, 7)
    kcs = [torch.randn((nkv, max_seq, 128), device="cuda", generator=g).to(bf) for _ in range(layers)]
    vcs = [torch.randn((nkv, max_seq, 128), device="cuda", generator=g).to(bf) for _ in range(layers)]
    freqs = D.llama3_rope_freqs(128, 500000.0)
    decs = [E.LlamaDecoder(dev_layers, embed, final_norm, lm_head, n_heads=nh, n_kv_heads=nkv, eps=1e-5, freqs=freqs,
                           max_seq=max_seq, k_caches=[k.clone() for k in kcs], v_caches=[v.clone() for v in vcs],
                           fused=f) for f in (True, False)]
    token = 1234
    for pos in (1024, 1025, 1026):
        print(f"[case] 32-layer step pos={pos} token={token}", flush=True)
        for d in decs:
            d.token.fill_(token)
            d.step(pos)
        torch.cuda.synchronize()
        lf, lu = host_f32(decs[0].logits), host_f32(decs[1].logits)
        rms = float(np.sqrt(np.mean(lu.astype(np.float64) ** 2)))
        assert np.isfinite(lf).all() and np.isfinite(lu).all()
        d = (lf - lu).astype(np.float64)
        rel = float(np.sqrt(np.mean(d ** 2))) / rms
        print(f"  RMS(fused - unfused) / RMS = {rel:.3e}, max = {np.max(np.abs(d)) / rms:.3e}", flush=True)
        assert rel <= 3e-2, f"fused vs unfused logits: {rel:.3e}"
        tf, tu = int(decs[0].token.item()), int(decs[1].token.item())
        assert tf == int(np.argmax(lf)) and tu == int(np.argmax(lu))
        if tf != tu:  # only a near-tie may separate them
            assert float(lu[tu]) - float(lu[tf]) <= 2 * np.max(np.abs(d)), f"tokens {tf} vs {tu} at pos {pos}"
        token = tf

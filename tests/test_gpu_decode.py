"""Parity of the decode-step kernels (include/eredu_hip.h: eq_rms_norm,
eq_rope_attention_decode, eq_silu_mul, eq_embedding, eq_argmax) and of a
whole batch-1 decode step of a small Llama-shaped model with the oracle
(oracle/decode_oracle.py), through the C ABI via eredu_amd.decode.

Tolerances (written here): bf16 results that the reference rounds once from
an exact value -- residual sums, embedding rows, stored values, argmax -- are
bit-exact; results that pass through transcendental functions or an f32 sum
of another order (RMSNorm output, rotated keys, silu) are within 1 bf16 ulp
of the oracle; attention outputs and logits are within
1e-2 * RMS(ref) + 1/2 ulp_bf16(ref) elementwise (the matmul rule), with the
decode step's logits compared after two layers of bf16 roundings at
2e-2 * RMS(ref).
"""
import numpy as np
import pytest
import torch

from eredu_amd import decode as E
from oracle import decode_oracle as D
from oracle import oracle as orc
from tests.fixtures import dev_bf16, dev_words, host_bits16, host_f32, synthetic_linear

pytestmark = pytest.mark.gpu


def bits(x):
    return orc.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


def randn_bits(shape, seed, std=1.0):
    return bits(np.random.default_rng(seed).standard_normal(shape) * std)


def ulp_bf16(v):
    a = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 1e-30)))
    return np.where(a > 0, 2.0 ** (e - 7), 2.0 ** -133)


def within_ulps(got_bits, ref_f64, n=1):
    got = D.bits_to_f64(got_bits)
    return np.all(np.abs(got - ref_f64) <= n * ulp_bf16(ref_f64) + 1e-30)


@pytest.mark.parametrize("dim", [64, 512, 4096, 14336, 40000])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rms_norm(cuda, dim, with_residual):
    print(f"[case] rms_norm dim={dim} residual={with_residual}", flush=True)
    x = randn_bits(dim, dim)
    w = bits(1.0 + 0.1 * np.random.default_rng(dim + 1).standard_normal(dim))
    r = randn_bits(dim, dim + 2) if with_residual else None
    xd, wd = dev_bf16(x), dev_bf16(w)
    out = E.rms_norm(xd, wd, 1e-5, dev_bf16(r) if r is not None else None)
    torch.cuda.synchronize()
    hid_ref, out_ref = D.rms_norm_bf16(x, w, 1e-5, r)
    assert np.array_equal(host_bits16(xd), hid_ref)  # residual sum: exact
    ref = D.rms_norm(D.bits_to_f64(hid_ref), D.bits_to_f64(w), 1e-5)
    assert within_ulps(host_bits16(out), ref, 1)


@pytest.mark.parametrize("n_heads,n_kv", [(32, 8), (4, 1), (4, 4), (8, 4)])
@pytest.mark.parametrize("pos", [0, 5, 31, 32, 33, 100, 1024])
def test_rope_attention_decode(cuda, n_heads, n_kv, pos):
    print(f"[case] attention heads={n_heads}/{n_kv} pos={pos}", flush=True)
    max_seq = 1100
    seed = pos * 7 + n_heads
    q = randn_bits(n_heads * 128, seed)
    kn = randn_bits(n_kv * 128, seed + 1)
    vn = randn_bits(n_kv * 128, seed + 2)
    kc = randn_bits((n_kv, max_seq, 128), seed + 3)
    vc = randn_bits((n_kv, max_seq, 128), seed + 4)
    freqs = D.llama3_rope_freqs(128, 500000.0)
    scale = 1.0 / np.sqrt(128.0)
    kcd, vcd = dev_bf16(kc), dev_bf16(vc)
    out = E.rope_attention_decode(dev_bf16(q), dev_bf16(kn), dev_bf16(vn), kcd, vcd,
                                  torch.from_numpy(freqs).cuda(), pos, n_heads, n_kv, scale)
    torch.cuda.synchronize()
    ref, kc_ref, vc_ref = D.attention_decode(q, kn, vn, kc, vc, freqs, pos, n_heads, n_kv, scale)
    got_k, got_v = host_bits16(kcd), host_bits16(vcd)
    assert np.array_equal(got_v, vc_ref)
    mask = np.ones(max_seq, dtype=bool)
    mask[pos] = False
    assert np.array_equal(got_k[:, mask], kc[:, mask])
    rot = D.rope(D.bits_to_f64(kn).reshape(n_kv, 128), pos, freqs)
    assert within_ulps(got_k[:, pos], rot, 1)
    # the oracle with the GPU's stored key (a 1-ulp rotation difference moves
    # the scores a little; the output rule below absorbs it either way)
    ok, worst, rms = orc.matmul_within_tolerance(host_f32(out).reshape(n_heads, 128), ref, out_is_bf16=True)
    assert ok, f"max|err|/RMS = {worst:.3e}"


@pytest.mark.parametrize("n_heads,n_kv,max_seq", [(32, 8, 1100), (4, 1, 1100), (8, 4, 4000), (32, 8, 64)])
@pytest.mark.parametrize("pos", [0, 5, 31, 32, 33, 100, 1024, 2500])
def test_rope_attention_decode_at_device_position(cuda, n_heads, n_kv, max_seq, pos):
    """eq_rope_attention_decode_at: the position read from device memory by
    the kernels, whose grid covers every chunk of max_seq.  Same oracle and
    cache rules as the by-value entry point, and bit-equal to it; a position
    outside the cache writes nothing and gives zeros."""
    print(f"[case] attention at device pos heads={n_heads}/{n_kv} max_seq={max_seq} pos={pos}", flush=True)
    seed = pos * 5 + n_heads + max_seq
    q = randn_bits(n_heads * 128, seed)
    kn = randn_bits(n_kv * 128, seed + 1)
    vn = randn_bits(n_kv * 128, seed + 2)
    kc = randn_bits((n_kv, max_seq, 128), seed + 3)
    vc = randn_bits((n_kv, max_seq, 128), seed + 4)
    freqs = D.llama3_rope_freqs(128, 500000.0)
    scale = 1.0 / np.sqrt(128.0)
    kcd, vcd = dev_bf16(kc), dev_bf16(vc)
    pos_d = torch.tensor([pos], dtype=torch.int32, device="cuda")
    out = E.rope_attention_decode_at(dev_bf16(q), dev_bf16(kn), dev_bf16(vn), kcd, vcd,
                                     torch.from_numpy(freqs).cuda(), pos_d, n_heads, n_kv, scale)
    torch.cuda.synchronize()
    got_k, got_v = host_bits16(kcd), host_bits16(vcd)
    if pos >= max_seq:
        assert np.array_equal(got_k, kc) and np.array_equal(got_v, vc)
        assert not host_f32(out).any()
        return
    ref, kc_ref, vc_ref = D.attention_decode(q, kn, vn, kc, vc, freqs, pos, n_heads, n_kv, scale)
    assert np.array_equal(got_v, vc_ref)
    mask = np.ones(max_seq, dtype=bool)
    mask[pos] = False
    assert np.array_equal(got_k[:, mask], kc[:, mask])
    rot = D.rope(D.bits_to_f64(kn).reshape(n_kv, 128), pos, freqs)
    assert within_ulps(got_k[:, pos], rot, 1)
    ok, worst, rms = orc.matmul_within_tolerance(host_f32(out).reshape(n_heads, 128), ref, out_is_bf16=True)
    assert ok, f"max|err|/RMS = {worst:.3e}"
    kc2, vc2 = dev_bf16(kc), dev_bf16(vc)
    out2 = E.rope_attention_decode(dev_bf16(q), dev_bf16(kn), dev_bf16(vn), kc2, vc2,
                                   torch.from_numpy(freqs).cuda(), pos, n_heads, n_kv, scale)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
    assert torch.equal(kcd, kc2) and torch.equal(vcd, vc2)


@pytest.mark.parametrize("pos", [64 * 32 - 1, 64 * 32, 100000])
def test_rope_attention_decode_long_context(cuda, pos):
    """Positions whose chunks outnumber the 64 softmax states per head: each
    state merges several chunks (up to 49 at pos 100000) before the combine;
    at 2047 every state holds one chunk, at 2048 state 0 holds two."""
    print(f"[case] attention long context pos={pos}", flush=True)
    n_heads, n_kv, max_seq = 4, 1, pos + 1
    q = randn_bits(n_heads * 128, pos)
    kn, vn = randn_bits(n_kv * 128, pos + 1), randn_bits(n_kv * 128, pos + 2)
    kc = randn_bits((n_kv, max_seq, 128), pos + 3)
    vc = randn_bits((n_kv, max_seq, 128), pos + 4)
    freqs = D.llama3_rope_freqs(128, 500000.0)
    scale = 1.0 / np.sqrt(128.0)
    kcd, vcd = dev_bf16(kc), dev_bf16(vc)
    out = E.rope_attention_decode(dev_bf16(q), dev_bf16(kn), dev_bf16(vn), kcd, vcd,
                                  torch.from_numpy(freqs).cuda(), pos, n_heads, n_kv, scale)
    torch.cuda.synchronize()
    ref, kc_ref, vc_ref = D.attention_decode(q, kn, vn, kc, vc, freqs, pos, n_heads, n_kv, scale)
    assert np.array_equal(host_bits16(vcd), vc_ref)
    ok, worst, rms = orc.matmul_within_tolerance(host_f32(out).reshape(n_heads, 128), ref, out_is_bf16=True)
    assert ok, f"max|err|/RMS = {worst:.3e}"


def test_attention_matches_torch_sdpa(cuda):
    """Cross-check with torch's own attention in f32 on the rotated inputs."""
    n_heads, n_kv, pos, max_seq = 32, 8, 777, 1024
    q = randn_bits(n_heads * 128, 11)
    kn, vn = randn_bits(n_kv * 128, 12), randn_bits(n_kv * 128, 13)
    kc, vc = randn_bits((n_kv, max_seq, 128), 14), randn_bits((n_kv, max_seq, 128), 15)
    freqs = D.llama3_rope_freqs(128, 500000.0)
    scale = 1.0 / np.sqrt(128.0)
    kcd, vcd = dev_bf16(kc), dev_bf16(vc)
    out = E.rope_attention_decode(dev_bf16(q), dev_bf16(kn), dev_bf16(vn), kcd, vcd, torch.from_numpy(freqs).cuda(),
                                  pos, n_heads, n_kv, scale)
    qr = torch.from_numpy(D.rope(D.bits_to_f64(q).reshape(n_heads, 128), pos, freqs)).float()
    K = torch.from_numpy(D.bits_to_f64(host_bits16(kcd))[:, : pos + 1]).float()
    V = torch.from_numpy(D.bits_to_f64(host_bits16(vcd))[:, : pos + 1]).float()
    K = K.repeat_interleave(n_heads // n_kv, dim=0)
    V = V.repeat_interleave(n_heads // n_kv, dim=0)
    ref = torch.softmax((K @ qr.unsqueeze(-1)).squeeze(-1) * scale, dim=-1).unsqueeze(1) @ V
    ok, worst, _ = orc.matmul_within_tolerance(host_f32(out).reshape(n_heads, 128), ref.squeeze(1).double().numpy(),
                                               out_is_bf16=True)
    assert ok, worst


@pytest.mark.parametrize("n", [8, 14336, 65536 + 8])
def test_silu_mul(cuda, n):
    print(f"[case] silu_mul n={n}", flush=True)
    g = randn_bits(n, n, std=3.0)
    u = randn_bits(n, n + 1)
    out = E.silu_mul(dev_bf16(g), dev_bf16(u))
    torch.cuda.synchronize()
    ref_bits = D.silu_mul_bf16(g, u)
    got = host_bits16(out)
    # the three roundings are the reference's; the sigmoid's f32 exp may differ
    # from the oracle's f64 one in the last place before rounding
    assert within_ulps(got, D.bits_to_f64(ref_bits), 1)
    assert np.mean(got == ref_bits) > 0.99


def test_embedding_and_argmax(cuda):
    vocab, dim = 1000, 256
    table = randn_bits((vocab, dim), 3)
    ids = np.array([0, 999, 17, -1, 1000, 5], dtype=np.int32)
    out = E.embedding(dev_bf16(table), torch.from_numpy(ids).cuda())
    got = host_bits16(out)
    for t, i in enumerate(ids):
        expect = table[i] if 0 <= i < vocab else np.zeros(dim, dtype=np.uint16)
        assert np.array_equal(got[t], expect)
    logits = randn_bits((3, 128256), 4)
    logits[1, 5] = bits([100.0])[0]
    logits[1, 70000] = bits([100.0])[0]  # tie: the first index wins
    logits[2, 128255] = bits([1000.0])[0]
    idx = E.argmax(dev_bf16(logits)).cpu().numpy()
    ref = np.argmax(D.bits_to_f64(logits), axis=1)
    assert list(idx) == list(ref) and idx[1] == 5 and idx[2] == 128255


def tiny_model(seed=0, layers=2, n_heads=4, n_kv=2, ffn=1024, vocab=1024, max_seq=64, fused=None):
    H = n_heads * 128
    rng = np.random.default_rng(seed)
    host = {"hidden": H, "n_heads": n_heads, "n_kv_heads": n_kv, "eps": 1e-5,
            "freqs": D.llama3_rope_freqs(128, 500000.0)}

    def lin(N, K, s):
        w, sc, b = synthetic_linear(N, K, 64, 4, s)
        return {"w": w, "s": sc, "b": b, "bits": 4, "gs": 64}

    host["embed"] = bits(rng.standard_normal((vocab, H)))
    host["final_norm"] = bits(1.0 + 0.1 * rng.standard_normal(H))
    host["layers"] = []
    for li in range(layers):
        s0 = seed * 100 + li * 10
        host["layers"].append({
            "in_norm": bits(1.0 + 0.1 * rng.standard_normal(H)), "post_norm": bits(1.0 + 0.1 * rng.standard_normal(H)),
            "q": lin(n_heads * 128, H, s0), "k": lin(n_kv * 128, H, s0 + 1), "v": lin(n_kv * 128, H, s0 + 2),
            "o": lin(H, n_heads * 128, s0 + 3), "gate": lin(ffn, H, s0 + 4), "up": lin(ffn, H, s0 + 5),
            "down": lin(H, ffn, s0 + 6)})
    host["lm_head"] = lin(vocab, H, seed * 100 + 99)
    kcs = [randn_bits((n_kv, max_seq, 128), seed + 500 + i) for i in range(layers)]
    vcs = [randn_bits((n_kv, max_seq, 128), seed + 600 + i) for i in range(layers)]

    def qlin(d):
        return E.QLinear(dev_words(d["w"]), dev_bf16(d["s"]), dev_bf16(d["b"]), d["bits"], d["gs"])

    dev_layers = [E.DecoderLayer(dev_bf16(L["in_norm"]), dev_bf16(L["post_norm"]), *(qlin(L[p]) for p in
                                 ("q", "k", "v", "o", "gate", "up", "down"))) for L in host["layers"]]
    dec = E.LlamaDecoder(dev_layers, dev_bf16(host["embed"]), dev_bf16(host["final_norm"]), qlin(host["lm_head"]),
                         n_heads=n_heads, n_kv_heads=n_kv, eps=1e-5, freqs=host["freqs"], max_seq=max_seq,
                         k_caches=[dev_bf16(k) for k in kcs], v_caches=[dev_bf16(v) for v in vcs], fused=fused)
    return host, dec, kcs, vcs


@pytest.mark.parametrize("fused", [False, True])
def test_decode_step_end_to_end(cuda, fused):
    host, dec, kcs, vcs = tiny_model(fused=fused)
    assert dec.fused == fused
    assert dec.swiglu == fused  # the fused step folds SiLU-mul into the gate/up launch
    kcs = [k.copy() for k in kcs]
    vcs = [v.copy() for v in vcs]
    token = 7
    dec.token.fill_(token)
    for pos in (10, 11, 12):
        print(f"[case] decode step pos={pos} token={token}", flush=True)
        dec.step(pos)
        torch.cuda.synchronize()
        logits_ref, _ = D.decode_step(host, token, pos, kcs, vcs)
        got = host_f32(dec.logits)
        rms = np.sqrt(np.mean(logits_ref ** 2))
        err = np.abs(got - logits_ref)
        assert np.all(err <= 2e-2 * rms + 0.5 * ulp_bf16(logits_ref)), f"max|err|/RMS = {err.max() / rms:.3e}"
        nxt = int(dec.token.cpu().numpy()[0])
        assert logits_ref[nxt] >= logits_ref.max() - 4e-2 * rms  # greedy pick agrees up to near-ties
        # the oracle continues from the GPU's token so the two stay in step
        token = nxt


@pytest.mark.parametrize("fused", [False, True])
def test_decode_step_graph_replay(cuda, fused):
    """The step captured in a HIP graph and replayed matches the eager step."""
    _, dec, _, _ = tiny_model(seed=3, fused=fused)
    _, dec2, _, _ = tiny_model(seed=3, fused=fused)
    for d in (dec, dec2):
        d.token.fill_(5)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        dec.step(20)  # first call outside capture (workspace)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            dec.step(21)
        torch.cuda.synchronize()
    dec2.step(20)
    toks, toks2 = [], []
    for _ in range(3):
        with torch.cuda.stream(st):
            g.replay()
        torch.cuda.synchronize()
        dec2.step(21)
        torch.cuda.synchronize()
        toks.append(int(dec.token.item()))
        toks2.append(int(dec2.token.item()))
        assert torch.equal(dec.logits, dec2.logits)
    assert toks == toks2


@pytest.mark.parametrize("fused", [False, True])
def test_one_graph_decodes_successive_positions(cuda, fused):
    """step_device() reads the position from device memory and advances it:
    one captured graph, replayed three times from position p, gives the
    tokens and logits of eager device-position steps at p, p + 1, p + 2, and
    the same caches; the first of those steps is also checked against the
    oracle at p."""
    host, dec, kcs, vcs = tiny_model(seed=4, fused=fused)
    _, dec2, _, _ = tiny_model(seed=4, fused=fused)
    p0 = 17
    for d in (dec, dec2):
        d.token.fill_(9)
        d.set_position(p0)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        # one eager step first (workspace and counters of this stream), at a
        # position the replays overwrite; then back to p0
        dec.step_device()
        torch.cuda.synchronize()
        dec.token.fill_(9)
        dec.set_position(p0)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            dec.step_device()
    torch.cuda.synchronize()
    assert int(dec.position.item()) == p0  # capture runs nothing
    kref = [k.copy() for k in kcs]
    vref = [v.copy() for v in vcs]
    for i in range(3):
        print(f"[case] one-graph decode fused={fused} pos={p0 + i}", flush=True)
        token_in = int(dec2.token.item())
        with torch.cuda.stream(st):
            g.replay()
        torch.cuda.synchronize()
        dec2.step_device()
        torch.cuda.synchronize()
        assert int(dec.position.item()) == p0 + i + 1 == int(dec2.position.item())
        assert torch.equal(dec.logits, dec2.logits), f"replay {i}"
        assert int(dec.token.item()) == int(dec2.token.item())
        if i == 0:
            logits_ref, _ = D.decode_step(host, token_in, p0, kref, vref)
            got = host_f32(dec.logits)
            rms = np.sqrt(np.mean(logits_ref ** 2))
            err = np.abs(got - logits_ref)
            assert np.all(err <= 2e-2 * rms + 0.5 * ulp_bf16(logits_ref)), f"max|err|/RMS = {err.max() / rms:.3e}"
    for a, b in zip(dec.k_caches + dec.v_caches, dec2.k_caches + dec2.v_caches):
        assert torch.equal(a, b)


def _prologue_call(problems, lins, pro):
    from eredu_amd import _native as n

    arr = (n.QmmProblem * len(problems))()
    for i, (x, lin, y) in enumerate(problems):
        arr[i] = n.QmmProblem(y.data_ptr(), x.data_ptr(), lin.w.data_ptr(), lin.scales.data_ptr(),
                              lin.biases.data_ptr(), lin.N, lin.K)
    import ctypes
    n.check(n.lib().eq_quantized_matmul_batched_prologue(arr, len(problems), 1, True, 64, lins[0].bits, b"affine",
                                                         n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, ctypes.byref(pro), None))


def _qlin(N, K, seed, bits=4):
    w, s, b = synthetic_linear(N, K, 64, bits, seed)
    return E.QLinear(dev_words(w), dev_bf16(s), dev_bf16(b), bits, 64), (w, s, b)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("K", [1024, 14336])
def test_prologue_silu_mul(cuda, bits, K):
    """down_proj(silu(gate) * up) in one launch equals eq_silu_mul then the matmul, bit for bit."""
    from eredu_amd import _native as n

    print(f"[case] prologue silu_mul bits={bits} K={K}", flush=True)
    lin, (w, s, b) = _qlin(4096, K, K + bits, bits)
    g, u = dev_bf16(randn_bits(K, 1, std=2.0)), dev_bf16(randn_bits(K, 2))
    y = torch.empty(4096, dtype=torch.bfloat16, device="cuda")
    _prologue_call([(g, lin, y)], [lin], n.ActivationPrologue(n.EQ_PROLOGUE_SILU_MUL, u.data_ptr(), None, None, 0.0))
    act = E.silu_mul(g, u)
    y2 = torch.empty_like(y)
    _prologue_call_plain = n.lib().eq_quantized_matmul(y2.data_ptr(), act.data_ptr(), lin.w.data_ptr(),
                                                        lin.scales.data_ptr(), lin.biases.data_ptr(), 1, 4096, K, True,
                                                        64, bits, b"affine", n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, None)
    n.check(_prologue_call_plain)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    ref = orc.quantized_matmul_f64(host_bits16(act), orc.BF16, w, s, b, orc.BF16, True, 64, bits, 4096, K)
    ok, worst, _ = orc.matmul_within_tolerance(host_f32(y).reshape(1, -1), ref, out_is_bf16=True)
    assert ok, worst


@pytest.mark.parametrize("K", [512, 4096])
@pytest.mark.parametrize("with_residual", [False, True])
def test_prologue_rms_norm(cuda, K, with_residual):
    """q/k/v of RMSNorm(x + r) in one launch: hidden_out bit-exact, the
    normalized row within 1 ulp of eq_rms_norm's (sum order), outputs within
    the matmul rule of the oracle on the oracle's normalized row."""
    from eredu_amd import _native as n

    print(f"[case] prologue rms_norm K={K} residual={with_residual}", flush=True)
    shapes = [(K, K), (K // 4, K), (K // 4, K)]
    lins = [_qlin(N, K_, 100 + i) for i, (N, K_) in enumerate(shapes)]
    xb, rb = randn_bits(K, 7), randn_bits(K, 8)
    wb = bits(1.0 + 0.1 * np.random.default_rng(9).standard_normal(K))
    x, r, nw = dev_bf16(xb), dev_bf16(rb), dev_bf16(wb)
    hid = torch.empty(K, dtype=torch.bfloat16, device="cuda")
    ys = [torch.empty(N, dtype=torch.bfloat16, device="cuda") for N, _ in shapes]
    pro = n.ActivationPrologue(n.EQ_PROLOGUE_RMS_NORM, r.data_ptr() if with_residual else None, nw.data_ptr(),
                               hid.data_ptr() if with_residual else None, 1e-5)
    _prologue_call([(x, l, y) for (l, _), y in zip(lins, ys)], [l for l, _ in lins], pro)
    torch.cuda.synchronize()
    hid_ref, h_ref = D.rms_norm_bf16(xb, wb, 1e-5, rb if with_residual else None)
    if with_residual:
        assert np.array_equal(host_bits16(hid), hid_ref)
    assert np.array_equal(host_bits16(x), xb)  # the input row is not modified
    for (lin, (w, s, b)), y, (N, K_) in zip(lins, ys, shapes):
        ref = orc.quantized_matmul_f64(h_ref, orc.BF16, w, s, b, orc.BF16, True, 64, 4, N, K_)
        ok, worst, _ = orc.matmul_within_tolerance(host_f32(y).reshape(1, -1), ref, out_is_bf16=True)
        assert ok, worst


@pytest.mark.parametrize("nbits", [4, 8])
@pytest.mark.parametrize("F,K", [(1024, 512), (14336, 4096)])
@pytest.mark.parametrize("with_norm", [False, True])
def test_swiglu_equals_gate_up_then_silu_mul(cuda, nbits, F, K, with_norm):
    """eq_quantized_matmul_swiglu on the interleaved gate/up matrix equals the
    gate and up projections (eq_quantized_matmul_batched, or its RMSNorm
    prologue) followed by eq_silu_mul, bit for bit; the RMSNorm prologue's
    hidden_out bit-equal too; and the result within the matmul rule of the
    oracle (f64 projections of the oracle's normalized row, the oracle's
    silu_mul roundings)."""
    from eredu_amd import _native as n

    print(f"[case] swiglu bits={nbits} F={F} K={K} norm={with_norm}", flush=True)
    (gate, (wg, sg, bg)), (up, (wu, su, bu)) = _qlin(F, K, 300 + nbits, nbits), _qlin(F, K, 400 + nbits, nbits)
    gu = E.interleave_gate_up(gate, up)
    xb, rb = randn_bits(K, 11), randn_bits(K, 12)
    wb = bits(1.0 + 0.1 * np.random.default_rng(13).standard_normal(K))
    x, r, nw = dev_bf16(xb), dev_bf16(rb), dev_bf16(wb)
    hid, hid2 = (torch.empty(K, dtype=torch.bfloat16, device="cuda") for _ in range(2))
    g, u = (torch.empty(F, dtype=torch.bfloat16, device="cuda") for _ in range(2))
    if with_norm:
        pro = n.ActivationPrologue(n.EQ_PROLOGUE_RMS_NORM, r.data_ptr(), nw.data_ptr(), hid.data_ptr(), 1e-5)
        pro2 = n.ActivationPrologue(n.EQ_PROLOGUE_RMS_NORM, r.data_ptr(), nw.data_ptr(), hid2.data_ptr(), 1e-5)
        out = E.gate_up_swiglu(x, gu, pro)
        _prologue_call([(x, gate, g), (x, up, u)], [gate, up], pro2)
    else:
        out = E.gate_up_swiglu(x, gu)
        arr = (n.QmmProblem * 2)()
        for i, (lin, y) in enumerate(((gate, g), (up, u))):
            arr[i] = n.QmmProblem(y.data_ptr(), x.data_ptr(), lin.w.data_ptr(), lin.scales.data_ptr(),
                                  lin.biases.data_ptr(), F, K)
        n.check(n.lib().eq_quantized_matmul_batched(arr, 2, 1, True, 64, nbits, b"affine", n.EQ_DTYPE_BF16,
                                                    n.EQ_DTYPE_BF16, None))
    ref = E.silu_mul(g, u)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    if with_norm:
        assert torch.equal(hid.view(torch.int16), hid2.view(torch.int16))
        _, h_ref = D.rms_norm_bf16(xb, wb, 1e-5, rb)
    else:
        h_ref = xb
    gr = orc.quantized_matmul_f64(h_ref, orc.BF16, wg, sg, bg, orc.BF16, True, 64, nbits, F, K)
    ur = orc.quantized_matmul_f64(h_ref, orc.BF16, wu, su, bu, orc.BF16, True, 64, nbits, F, K)
    act_ref = orc.bf16_bits_to_f32(D.silu_mul_bf16(orc.f32_to_bf16_bits(gr.astype(np.float32)),
                                                   orc.f32_to_bf16_bits(ur.astype(np.float32)))).astype(np.float64)
    got = host_f32(out).astype(np.float64)
    rms = float(np.sqrt(np.mean(act_ref.reshape(-1) ** 2)))
    assert np.max(np.abs(got - act_ref.reshape(-1))) <= 2e-2 * rms + 1e-6


def test_swiglu_rejects_unsupported(cuda):
    from eredu_amd import _native as n
    import ctypes

    (gate, _), (up, _) = _qlin(512, 8192, 5), _qlin(512, 8192, 6)
    gu = E.interleave_gate_up(gate, up)
    x = dev_bf16(randn_bits(8192, 1))
    out = torch.empty(512, dtype=torch.bfloat16, device="cuda")
    call = lambda pro=None, F=512, gs=64: n.lib().eq_quantized_matmul_swiglu(
        out.data_ptr(), x.data_ptr(), gu.w.data_ptr(), gu.scales.data_ptr(), gu.biases.data_ptr(), F, 8192, gs, 4,
        b"affine", n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, ctypes.byref(pro) if pro is not None else None, None)
    wv = dev_bf16(randn_bits(8192, 2))
    assert call(n.ActivationPrologue(n.EQ_PROLOGUE_RMS_NORM, None, wv.data_ptr(), None, 1e-5)) == 1
    assert "4096" in n.lib().eq_last_error().decode()
    assert call(n.ActivationPrologue(n.EQ_PROLOGUE_SILU_MUL, wv.data_ptr(), None, None, 0.0)) == 1
    assert "RMS_NORM" in n.lib().eq_last_error().decode()
    assert call(F=508) == 1 and "multiple of 8" in n.lib().eq_last_error().decode()
    assert call() == 0, n.lib().eq_last_error()  # K = 8192 without the prologue runs
    torch.cuda.synchronize()


def test_prologue_rejects_unsupported(cuda):
    from eredu_amd import _native as n
    import ctypes

    lin, _ = _qlin(512, 8192, 5)
    x = dev_bf16(randn_bits(8192, 1))
    y = torch.empty(512, dtype=torch.bfloat16, device="cuda")
    arr = (n.QmmProblem * 1)()
    arr[0] = n.QmmProblem(y.data_ptr(), x.data_ptr(), lin.w.data_ptr(), lin.scales.data_ptr(), lin.biases.data_ptr(),
                          512, 8192)
    call = lambda pro, M=1: n.lib().eq_quantized_matmul_batched_prologue(arr, 1, M, True, 64, 4, b"affine",
                                                                         n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16,
                                                                         ctypes.byref(pro), None)
    wv = dev_bf16(randn_bits(8192, 2))
    assert call(n.ActivationPrologue(n.EQ_PROLOGUE_RMS_NORM, None, wv.data_ptr(), None, 1e-5)) == 1
    assert "4096" in n.lib().eq_last_error().decode()
    assert call(n.ActivationPrologue(7, None, None, None, 0.0)) == 1
    assert call(n.ActivationPrologue(n.EQ_PROLOGUE_SILU_MUL, wv.data_ptr(), None, None, 0.0), M=2) == 1
    # the hidden output may not alias the input it is computed from
    lin2, _ = _qlin(512, 4096, 6)
    x2 = dev_bf16(randn_bits(4096, 3))
    arr[0] = n.QmmProblem(y.data_ptr(), x2.data_ptr(), lin2.w.data_ptr(), lin2.scales.data_ptr(),
                          lin2.biases.data_ptr(), 512, 4096)
    assert call(n.ActivationPrologue(n.EQ_PROLOGUE_RMS_NORM, None, wv.data_ptr(), x2.data_ptr(), 1e-5)) == 1
    assert "overlap" in n.lib().eq_last_error().decode()


@pytest.mark.parametrize("n", [16384, 128256, 200000, 1000])
def test_argmax_wide_rows_ties_and_nans(cuda, n):
    """Rows long enough to be split over workgroups (and one short row that is
    not): ties resolve to the first index across workgroup boundaries, NaNs are
    skipped, a row of NaNs gives 0, -inf counts as a value."""
    print(f"[case] argmax n={n}", flush=True)
    rows = 5
    x = randn_bits((rows, n), n)
    big = bits([50.0])[0]
    x[0, n - 1] = big                      # the last element
    x[1, 3] = big
    x[1, n // 2 + 3] = big                 # a tie in a later workgroup: the first wins
    x[2, :] = 0x7FC0                       # all NaN
    x[3, :] = bits([-np.inf])[0]           # all -inf: index 0
    x[4, 7] = 0x7FC0                       # a NaN before the maximum is skipped
    x[4, n - 2] = big
    got = E.argmax(dev_bf16(x)).cpu().numpy()
    assert list(got) == [n - 1, 3, 0, 0, n - 2]

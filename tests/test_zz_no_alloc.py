"""eq_rope_attention_decode_noalloc (the allocation-free variant of
eq_rope_attention_decode) through the C ABI: its outputs and cache writes
equal the allocating entry point's bit for bit (both run the same kernels on
the same inputs; only the scratch differs), on two calls in a row, the
second at a smaller position, and once under HIP graph capture with replays;
calls past its 8 MiB scratch (n_heads * 64 * 520 bytes of softmax states) are
rejected with a message."""
import ctypes

import numpy as np
import pytest
import torch

from eredu_amd import _native as n

pytestmark = pytest.mark.gpu


def _inputs(n_heads, n_kv, max_seq, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    bf = torch.bfloat16
    q = torch.randn(n_heads * 128, device="cuda", generator=g).to(bf)
    kn = torch.randn(n_kv * 128, device="cuda", generator=g).to(bf)
    vn = torch.randn(n_kv * 128, device="cuda", generator=g).to(bf)
    kc = torch.randn((n_kv, max_seq, 128), device="cuda", generator=g).to(bf)
    vc = torch.randn((n_kv, max_seq, 128), device="cuda", generator=g).to(bf)
    return q, kn, vn, kc, vc


def _call(fn, out, q, kn, vn, kc, vc, freqs, pos, max_seq, n_heads, n_kv, st):
    return fn(out.data_ptr(), q.data_ptr(), kn.data_ptr(), vn.data_ptr(), kc.data_ptr(), vc.data_ptr(),
              freqs.data_ptr(), pos, max_seq, n_heads, n_kv, 128, ctypes.c_float(1.0 / np.sqrt(128.0)),
              n.EQ_DTYPE_BF16, st)


def _freqs():
    from oracle import decode_oracle as D

    return torch.from_numpy(D.llama3_rope_freqs(128, 500000.0)).cuda()


def test_noalloc_equals_the_allocating_entry_point(cuda):
    L = n.lib()
    freqs = _freqs()
    n_heads, n_kv, max_seq = 32, 8, 4200
    for pos in (4100, 37):  # the second call smaller than the first
        print(f"[case] noalloc attention pos={pos}", flush=True)
        q, kn, vn, kc, vc = _inputs(n_heads, n_kv, max_seq, seed=pos)
        kc2, vc2 = kc.clone(), vc.clone()
        out_a = torch.empty(n_heads * 128, dtype=torch.bfloat16, device="cuda")
        out_b = torch.empty_like(out_a)
        assert _call(L.eq_rope_attention_decode, out_a, q, kn, vn, kc, vc, freqs, pos, max_seq, n_heads, n_kv,
                     None) == 0, L.eq_last_error()
        assert _call(L.eq_rope_attention_decode_noalloc, out_b, q, kn, vn, kc2, vc2, freqs, pos, max_seq, n_heads,
                     n_kv, None) == 0, L.eq_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))
        assert torch.equal(kc.view(torch.int16), kc2.view(torch.int16))
        assert torch.equal(vc.view(torch.int16), vc2.view(torch.int16))


def test_noalloc_under_graph_capture(cuda):
    """Captured on a fresh stream (whose workspace has never been grown),
    replayed three times with eager work in between."""
    L = n.lib()
    freqs = _freqs()
    n_heads, n_kv, max_seq, pos = 32, 8, 3000, 2999
    q, kn, vn, kc0, vc0 = _inputs(n_heads, n_kv, max_seq, seed=5)
    kc, vc = kc0.clone(), vc0.clone()
    ref = torch.empty(n_heads * 128, dtype=torch.bfloat16, device="cuda")
    assert _call(L.eq_rope_attention_decode, ref, q, kn, vn, kc, vc, freqs, pos, max_seq, n_heads, n_kv, None) == 0
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    out = torch.empty_like(ref)
    kg, vg = kc0.clone(), vc0.clone()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            rc = _call(L.eq_rope_attention_decode_noalloc, out, q, kn, vn, kg, vg, freqs, pos, max_seq, n_heads,
                       n_kv, stream.cuda_stream)
    assert rc == 0, L.eq_last_error()
    torch.cuda.synchronize()
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {rep}"
        assert torch.equal(kg.view(torch.int16), kc.view(torch.int16))
        # eager work between replays
        other = torch.empty_like(ref)
        assert _call(L.eq_rope_attention_decode_noalloc, other, q, kn, vn, kc0.clone(), vc0.clone(), freqs, 10,
                     max_seq, n_heads, n_kv, None) == 0
        torch.cuda.synchronize()


def test_noalloc_rejects_head_counts_past_its_scratch(cuda):
    L = n.lib()
    freqs = _freqs()
    max_seq, pos = 64, 40
    # 256 heads * 64 states * 520 B > 8 MiB
    q, kn, vn, kc, vc = _inputs(256, 64, max_seq, seed=9)
    out = torch.empty(256 * 128, dtype=torch.bfloat16, device="cuda")
    assert _call(L.eq_rope_attention_decode_noalloc, out, q, kn, vn, kc, vc, freqs, pos, max_seq, 256, 64, None) == 1
    assert "scratch" in L.eq_last_error().decode()
    # the largest head count that fits (252 * 64 * 520 B) still runs, equal to
    # the allocating entry point
    q, kn, vn, kc, vc = _inputs(252, 63, max_seq, seed=10)
    kc2, vc2 = kc.clone(), vc.clone()
    out = torch.empty(252 * 128, dtype=torch.bfloat16, device="cuda")
    ref = torch.empty_like(out)
    assert _call(L.eq_rope_attention_decode_noalloc, out, q, kn, vn, kc, vc, freqs, pos, max_seq, 252, 63,
                 None) == 0, L.eq_last_error()
    assert _call(L.eq_rope_attention_decode, ref, q, kn, vn, kc2, vc2, freqs, pos, max_seq, 252, 63, None) == 0
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))

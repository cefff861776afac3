"""The library workspace under HIP graph capture: a graph captured with a
split-K prefill matmul and a decode attention call keeps its workspace
address; a later, larger call on the same stream grows the workspace, and
the old buffer must stay valid for the graph's replays (results bit-equal to
the eager calls).  Each replay is followed by eager work and a
synchronisation before it is checked."""
import numpy as np
import pytest
import torch

from eredu_amd import _native as n
from tests.fixtures import dev_bf16, dev_words, synthetic_linear, synthetic_x

pytestmark = pytest.mark.gpu


def qmm_call(y, x, w, s, b, M, N, K, st):
    n.check(n.lib().eq_quantized_matmul(y.data_ptr(), x.data_ptr(), w.data_ptr(), s.data_ptr(), b.data_ptr(), M, N, K,
                                        True, 64, 4, b"affine", n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, st))


def attn_call(out, q, k, v, kc, vc, freqs, pos, max_seq, st):
    n.check(n.lib().eq_rope_attention_decode(out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(),
                                             vc.data_ptr(), freqs.data_ptr(), pos, max_seq, 32, 8, 128,
                                             1.0 / np.sqrt(128.0), n.EQ_DTYPE_BF16, st))


def test_graph_replays_survive_workspace_growth(cuda):
    stream = torch.cuda.Stream()
    st = stream.cuda_stream
    # split-K prefill (6 tiles on a GPU of 256 CUs: K split several ways)
    M, N, K = 300, 512, 2048
    w, s, b = synthetic_linear(N, K, 64, 4, seed=1)
    wd, sd, bd = dev_words(w), dev_bf16(s), dev_bf16(b)
    x = dev_bf16(synthetic_x(M, K, seed=2))
    y_eager, y_graph = (torch.empty((M, N), dtype=torch.bfloat16, device="cuda") for _ in range(2))
    # decode attention at position 100 (its partials live in the workspace)
    max_seq = 1024
    g = torch.Generator(device="cuda").manual_seed(3)
    q = torch.randn(32 * 128, device="cuda", generator=g).to(torch.bfloat16)
    kn, vn = (torch.randn(8 * 128, device="cuda", generator=g).to(torch.bfloat16) for _ in range(2))
    kc0 = torch.randn((8, max_seq, 128), device="cuda", generator=g).to(torch.bfloat16)
    vc0 = torch.randn((8, max_seq, 128), device="cuda", generator=g).to(torch.bfloat16)
    from oracle import decode_oracle as D

    freqs = torch.from_numpy(D.llama3_rope_freqs(128, 500000.0)).cuda()
    kc, vc = kc0.clone(), vc0.clone()
    a_eager, a_graph = (torch.empty(32 * 128, dtype=torch.bfloat16, device="cuda") for _ in range(2))
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        qmm_call(y_eager, x, wd, sd, bd, M, N, K, st)
        attn_call(a_eager, q, kn, vn, kc, vc, freqs, 100, max_seq, st)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            qmm_call(y_graph, x, wd, sd, bd, M, N, K, st)
            attn_call(a_graph, q, kn, vn, kc, vc, freqs, 100, max_seq, st)
    torch.cuda.synchronize()
    # a much larger split-K call on the same stream grows its workspace
    # (8 x 16 tiles, K split twice: 2 x 1024 x 4096 x 4 bytes of partials)
    M2, N2, K2 = 1024, 4096, 4096
    w2, s2, b2 = synthetic_linear(N2, K2, 64, 4, seed=4)
    x2 = dev_bf16(synthetic_x(M2, K2, seed=5))
    y2 = torch.empty((M2, N2), dtype=torch.bfloat16, device="cuda")
    with torch.cuda.stream(stream):
        qmm_call(y2, x2, dev_words(w2), dev_bf16(s2), dev_bf16(b2), M2, N2, K2, st)
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"[case] replay {rep}", flush=True)
        y_graph.zero_()
        a_graph.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph.view(torch.int16), y_eager.view(torch.int16)), f"qmm replay {rep}"
        assert torch.equal(a_graph.view(torch.int16), a_eager.view(torch.int16)), f"attention replay {rep}"
        # eager work on the stream between replays
        with torch.cuda.stream(stream):
            qmm_call(y2, x2, dev_words(w2), dev_bf16(s2), dev_bf16(b2), M2, N2, K2, st)
        torch.cuda.synchronize()

"""The library workspace and arrival counters under HIP graph capture and
concurrent streams.  A graph captured with a split-K prefill matmul and a
decode attention call keeps its workspace address; a later, larger call on
the same stream grows the workspace, and the old buffer must stay valid for
the graph's replays (results bit-equal to the eager calls).  Kernels that
combine K runs in their last workgroup must keep two streams apart and leave
their counters at zero for the next replay.  Each replay is followed by
eager work and a synchronisation before it is checked."""
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
    # (4 x 32 tiles of 128 x 128, K split twice: 2 x 512 x 4096 x 4 bytes of partials)
    M2, N2, K2 = 512, 4096, 4096
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


def qmm_n_call(y, x, w, s, b, N, K, st):
    n.check(n.lib().eq_quantized_matmul(y.data_ptr(), x.data_ptr(), w.data_ptr(), s.data_ptr(), b.data_ptr(), 1, N, K,
                                        False, 64, 4, b"affine", n.EQ_DTYPE_BF16, n.EQ_DTYPE_BF16, st))


def test_streams_keep_apart_and_replays_reset_counters(cuda):
    """transpose = false at M = 1 splits K into runs that the last workgroup
    of each column tile adds up, counting arrivals in its stream's counter
    block and keeping the runs in its stream's workspace.  Two streams
    running such calls (and split-K prefill) at the same time must not see
    each other's counters or partials, and graph replays must find every
    counter back at zero."""
    N, K = 4096, 4096
    probs = []
    for seed in (11, 12):
        w, s, b = synthetic_linear(K, N, 64, 4, seed=seed)  # W [K, N] packed along N
        probs.append((dev_words(w), dev_bf16(s), dev_bf16(b), dev_bf16(synthetic_x(1, K, seed=seed + 10))))
    Mq, Nq, Kq = 300, 512, 2048
    wq, sq, bq = synthetic_linear(Nq, Kq, 64, 4, seed=13)
    wq, sq, bq = dev_words(wq), dev_bf16(sq), dev_bf16(bq)
    xq = dev_bf16(synthetic_x(Mq, Kq, seed=14))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    refs, outs = [], []
    for i, (w, s, b, x) in enumerate(probs):
        y = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
        streams[i].wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(streams[i]):
            qmm_n_call(y, x, w, s, b, N, K, streams[i].cuda_stream)
        torch.cuda.synchronize()
        refs.append(y.clone())
        outs.append(torch.empty_like(y))
    yq_ref = torch.empty((Mq, Nq), dtype=torch.bfloat16, device="cuda")
    with torch.cuda.stream(streams[0]):
        qmm_call(yq_ref, xq, wq, sq, bq, Mq, Nq, Kq, streams[0].cuda_stream)
    torch.cuda.synchronize()
    yq = torch.empty_like(yq_ref)
    for rep in range(8):
        print(f"[case] concurrent streams, round {rep}", flush=True)
        for o in outs:
            o.zero_()
        yq.zero_()
        torch.cuda.synchronize()
        for it in range(3):  # both streams busy at once, several calls each
            for i, (w, s, b, x) in enumerate(probs):
                with torch.cuda.stream(streams[i]):
                    qmm_n_call(outs[i], x, w, s, b, N, K, streams[i].cuda_stream)
                    if i == 1:
                        qmm_call(yq, xq, wq, sq, bq, Mq, Nq, Kq, streams[i].cuda_stream)
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(outs[i].view(torch.int16), refs[i].view(torch.int16)), f"stream {i} round {rep}"
        assert torch.equal(yq.view(torch.int16), yq_ref.view(torch.int16)), f"split-K prefill round {rep}"
    # graph replays of the counting kernel on a stream that already has its counters
    w, s, b, x = probs[0]
    yg = torch.empty_like(outs[0])
    with torch.cuda.stream(streams[0]):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=streams[0]):
            qmm_n_call(yg, x, w, s, b, N, K, streams[0].cuda_stream)
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"[case] counter replay {rep}", flush=True)
        yg.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(streams[0]):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg.view(torch.int16), refs[0].view(torch.int16)), f"replay {rep}"
        with torch.cuda.stream(streams[0]):  # eager work between replays
            qmm_n_call(outs[1], probs[1][3], probs[1][0], probs[1][1], probs[1][2], N, K, streams[0].cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(outs[1].view(torch.int16), refs[1].view(torch.int16)), f"eager after replay {rep}"


def test_captured_qmm_runs_the_eager_plan(cuda):
    """M = 128 x 4096 x 4096 splits K through the stream's workspace.  On a
    fresh stream the workspace cannot grow while capturing, so the capture
    fails with a message instead of recording an unsplit plan (which would
    sum in another order than the eager call).  After one eager call on the
    stream, the captured call runs the eager plan: every replay equals the
    eager result bit for bit."""
    M, N, K = 128, 4096, 4096
    w, s, b = synthetic_linear(N, K, 64, 4, seed=21)
    wd, sd, bd = dev_words(w), dev_bf16(s), dev_bf16(b)
    x = dev_bf16(synthetic_x(M, K, seed=22))
    y_eager, y_graph = (torch.empty((M, N), dtype=torch.bfloat16, device="cuda") for _ in range(2))
    stream = torch.cuda.Stream()
    st = stream.cuda_stream
    stream.wait_stream(torch.cuda.current_stream())
    print("[case] capture on a fresh stream", flush=True)
    with torch.cuda.stream(stream):
        graph = torch.cuda.CUDAGraph()
        with pytest.raises(n.EreduError, match="cannot grow while the stream is capturing"):
            with torch.cuda.graph(graph, stream=stream):
                qmm_call(y_graph, x, wd, sd, bd, M, N, K, st)
    torch.cuda.synchronize()
    print("[case] capture after an eager call", flush=True)
    with torch.cuda.stream(stream):
        qmm_call(y_eager, x, wd, sd, bd, M, N, K, st)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            qmm_call(y_graph, x, wd, sd, bd, M, N, K, st)
    torch.cuda.synchronize()
    other = torch.empty_like(y_eager)
    for rep in range(3):
        y_graph.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph.view(torch.int16), y_eager.view(torch.int16)), f"replay {rep}"
        with torch.cuda.stream(stream):  # eager work between replays
            qmm_call(other, x, wd, sd, bd, M, N, K, st)
        torch.cuda.synchronize()
        assert torch.equal(other.view(torch.int16), y_eager.view(torch.int16)), f"eager after replay {rep}"

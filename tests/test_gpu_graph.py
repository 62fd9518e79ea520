"""HIP graphs of the compute stream (we_graph_begin / end / launch / destroy).

A graph captures split-K fp8 GEMM (two kernels), the int4 decode GEMV, bf16 attention (the ping-pong kernel),
RMSNorm and an elementwise op. It is replayed several times; before each replay the inputs are
rewritten (eager uploads, a sync), and every replay's outputs must equal, bit for bit, the same calls run
eagerly on the same inputs.
"""
import numpy as np
import pytest

import oracle_lib as O
import we

pytestmark = pytest.mark.gpu


def _inputs(rng):
    m, n, k = 64, 3072, 3072
    x = rng.standard_normal(m * k).astype(np.float16)
    w = rng.integers(0, 254, n * k).astype(np.uint8)
    w = (w + (w >= 0x7F)).astype(np.uint8)
    n4, k4 = 2048, 3584
    w4 = rng.integers(0, 2 ** 32, n4 * k4 // 8, dtype=np.uint64).astype(np.uint32)
    s4 = np.abs(rng.normal(0, 0.01, n4 * k4 // 64)).astype(np.float16)
    x4 = rng.standard_normal(k4).astype(np.float16)
    t, hd, heads = 300, 128, 4
    q = O.bf16_rne(rng.standard_normal(t * heads * hd).astype(np.float32))
    kk = O.bf16_rne(rng.standard_normal(t * heads * hd).astype(np.float32))
    v = O.bf16_rne(rng.standard_normal(t * heads * hd).astype(np.float32))
    xn = rng.standard_normal(7 * 3072).astype(np.float32)
    return dict(x=x, w=w, w4=w4, s4=s4, x4=x4, q=q, k=kk, v=v, xn=xn)


def test_graph_replays_equal_eager_runs(graph):
    rng = np.random.default_rng(0)
    data = _inputs(rng)
    mark = graph.mark()
    b = {name: graph.buffer(arr) for name, arr in data.items()}
    nw = graph.buffer(rng.uniform(-.3, .3, 3072).astype(np.float32))
    out = dict(y=graph.buffer(64 * 3072 * 2), y4=graph.buffer(2048 * 2), o=graph.buffer(300 * 4 * 128 * 2),
               yn=graph.buffer(7 * 3072 * 4), ye=graph.buffer(7 * 3072 * 4))
    p = we.matmul_params(64, 3072, 3072, 0.02, graph=graph)
    p4 = we.matmul_params(1, 2048, 3584, 1.0, graph=graph)

    def step():
        graph.matmul(p, we.F16, b["x"], we.FP8, b["w"], we.F16, out["y"])
        graph.matmul(p4, we.F16, b["x4"], we.INT4, b["w4"], we.F16, out["y4"], scales=b["s4"], group=64)
        graph.attention(300, 4, 4, 128, False, we.BF16, b["q"], b["k"], b["v"], out["o"])
        graph.rmsnorm(7, 3072, 1e-6, 1.0, we.F32, b["xn"], nw, None, None, out["yn"])
        graph.elementwise(we.OP_SILU, 7 * 3072, 1, we.F32, out["yn"], None, None, out["ye"])

    def snapshot():
        return {name: graph.read(buf).copy() for name, buf in out.items()}

    step()  # eager first: grows the context scratch outside the capture
    graph.sync()
    graph.graph_begin()
    step()
    g = graph.graph_end()
    try:
        for rep in range(3):
            fresh = _inputs(np.random.default_rng(100 + rep))
            for name, arr in fresh.items():
                graph.write(b[name], arr)
            graph.sync()
            step()
            want = snapshot()
            for buf in out.values():  # the replay must rewrite every output
                graph.write(buf, np.zeros(buf.size, np.uint8))
            graph.graph_launch(g)
            got = snapshot()
            for name in out:
                assert np.array_equal(got[name], want[name]), (rep, name)
    finally:
        graph.graph_destroy(g)
        graph.release(mark)


def test_capture_refuses_allocation_and_host_traffic(graph):
    mark = graph.mark()
    x = graph.buffer(np.ones(256, np.float32))
    w = graph.buffer(np.ones(256, np.float32))
    y = graph.buffer(256 * 4)
    graph.graph_begin()
    try:
        with pytest.raises(we.WeError, match="not allowed while a graph is being captured"):
            graph.buffer(64)
        with pytest.raises(we.WeError, match="not allowed while a graph is being captured"):
            graph.sync()
        with pytest.raises(we.WeError, match="already being captured"):
            graph.graph_begin()
        graph.rmsnorm(1, 256, 1e-5, 1.0, we.F32, x, w, None, None, y)
    finally:
        g = graph.graph_end()
    graph.graph_launch(g)
    got = graph.read(y, dtype=np.float32, count=256)
    graph.graph_destroy(g)
    assert np.allclose(got, 2.0)  # x / rms(x) * (1 + w) = 2
    graph.release(mark)


def test_graph_keeps_its_scratch_when_an_eager_call_outgrows_it():
    """A graph captured with a split-K GEMM (partial sums in the context scratch) still replays correctly after an
    eager split-K GEMM with more slices and rows grew the scratch past the 16 MiB first allocation: the graph holds
    its scratch block until it is destroyed. A graph captured on compute stream 1 is refused on stream 0."""
    g = we.Graph(0)  # a fresh context: its scratch starts at the minimum size
    try:
        rng = np.random.default_rng(3)
        m, n, k = 64, 3072, 3072
        x = g.buffer(rng.standard_normal(m * k).astype(np.float16))
        w = rng.integers(0, 254, n * k).astype(np.uint8)
        w = g.buffer((w + (w >= 0x7F)).astype(np.uint8))
        y_eager, y_graph = g.buffer(m * n * 2), g.buffer(m * n * 2)
        p = we.matmul_params(m, n, k, 0.02, graph=g)
        g.matmul(p, we.F16, x, we.FP8, w, we.F16, y_eager)  # eager first: the scratch exists before capture
        g.sync()
        g.graph_begin()
        g.matmul(p, we.F16, x, we.FP8, w, we.F16, y_graph)
        gr = g.graph_end()
        # M = 512, N = 3072, K = 12288 splits K into several slices of 512 x 3072 f32 partial sums (over 16 MiB)
        m2, k2 = 512, 12288
        w2 = rng.integers(0, 254, n * k2).astype(np.uint8)
        g.matmul(we.matmul_params(m2, n, k2, 0.02, graph=g), we.F16,
                 g.buffer(rng.standard_normal(m2 * k2).astype(np.float16)), we.FP8,
                 g.buffer((w2 + (w2 >= 0x7F)).astype(np.uint8)), we.F16, g.buffer(m2 * n * 2))
        g.sync()
        want = g.read(y_eager).copy()
        for _ in range(2):
            g.write(y_graph, np.zeros(m * n * 2, np.uint8))
            g.sync()
            g.graph_launch(gr)
            assert np.array_equal(g.read(y_graph), want)
        g.graph_destroy(gr)
        # captured on stream 1: refused on stream 0, runs on stream 1
        g.stream(1)
        g.matmul(p, we.F16, x, we.FP8, w, we.F16, y_graph)
        g.graph_begin()
        g.matmul(p, we.F16, x, we.FP8, w, we.F16, y_graph)
        gr1 = g.graph_end()
        g.stream(0)
        with pytest.raises(we.WeError, match="captured on compute stream 1"):
            g.graph_launch(gr1)
        g.stream(1)
        g.write(y_graph, np.zeros(m * n * 2, np.uint8))
        g.graph_launch(gr1)
        g.sync()
        assert np.array_equal(g.read(y_graph), want)
        g.graph_destroy(gr1)
        g.stream(0)
    finally:
        g.destroy()

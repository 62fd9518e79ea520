"""The context's two compute streams (we_stream_select / we_stream_fork / we_stream_join): work queued on
stream 1 after a fork sees stream 0's results, stream 0 after a join sees stream 1's, each stream's split-K
GEMMs use their own scratch, and the calls are refused where they cannot be honoured."""
import numpy as np
import pytest

import oracle_lib as O
import we

pytestmark = pytest.mark.gpu


def _fp8_weights(rng, n, k):
    w = rng.integers(0, 254, n * k).astype(np.uint8)
    return (w + (w >= 0x7F)).astype(np.uint8)


def test_fork_and_join_order_dependent_work(graph):
    """x -> (stream 0) GEMM a -> fork -> (stream 1) norm of a, split-K GEMM b -> join -> (stream 0) GEMM c of b.
    Every step reads the previous one's output; the result equals the same steps on one stream, bit for bit."""
    rng = np.random.default_rng(11)
    m, k, n = 64, 3072, 3072
    x = O.bf16_rne(rng.standard_normal(m * k).astype(np.float32))
    w1, w2, w3 = (_fp8_weights(rng, n, k) for _ in range(3))
    nw = rng.uniform(-0.2, 0.2, n).astype(np.float32)
    mark = graph.mark()
    xb, w1b, w2b, w3b, nwb = (graph.buffer(v) for v in (x, w1, w2, w3, nw))
    p = we.matmul_params(m, n, k, 0.02, graph=graph)
    outs = []
    for streams in (False, True):
        a, h, b, c = (graph.buffer(m * n * 2) for _ in range(4))
        graph.matmul(p, we.BF16, xb, we.FP8, w1b, we.BF16, a)
        if streams:
            graph.fork()
            graph.stream(1)
        try:
            graph.rmsnorm(m, n, 1e-6, 1.0, we.BF16, a, nwb, None, None, h)
            graph.matmul(p, we.BF16, h, we.FP8, w2b, we.BF16, b)  # M = 64: split-K on this stream's scratch
        finally:
            if streams:
                graph.stream(0)
                graph.join()
        graph.matmul(p, we.BF16, b, we.FP8, w3b, we.BF16, c)
        outs.append(graph.read(c, dtype=np.uint16))
    assert np.array_equal(outs[0], outs[1])
    assert np.isfinite(O.bf16_to_f32(outs[1])).all() and outs[1].any()
    graph.release(mark)


def test_stream_calls_refused_where_they_cannot_hold(graph):
    with pytest.raises(we.WeError, match="stream must be 0 or 1"):
        graph.stream(2)
    graph.graph_begin()
    try:
        for call in (lambda: graph.stream(1), graph.fork, graph.join):
            with pytest.raises(we.WeError, match="not allowed while a graph is being captured"):
                call()
    finally:
        g = graph.graph_end()
    graph.graph_destroy(g)
    graph.stream(0)  # selecting the current stream is a no-op


def test_timestamp_slots_time_work_in_stream_order(graph):
    """we_timer_mark records a timestamp on the compute stream without waiting (the block benchmark's per-op timings,
    src/bench/block.ts:17-95, without a host round trip per op): intervals add up, the interval around queued GEMMs
    covers them, and slots outside the range or never marked are refused."""
    rng = np.random.default_rng(5)
    m, k, n = 256, 3072, 3072
    mark = graph.mark()
    xb = graph.buffer(O.bf16_rne(rng.standard_normal(m * k).astype(np.float32)))
    wb = graph.buffer(_fp8_weights(rng, n, k))
    yb = graph.buffer(m * n * 2)
    p = we.matmul_params(m, n, k, 0.02, graph=graph)
    graph.sync()
    graph.timer_mark(10)
    for _ in range(4):
        graph.matmul(p, we.BF16, xb, we.FP8, wb, we.BF16, yb)
    graph.timer_mark(11)
    graph.timer_mark(12)
    a, b, whole = graph.timer_between(10, 11), graph.timer_between(11, 12), graph.timer_between(10, 12)
    graph.release(mark)
    assert a > 0 and b >= 0 and abs(whole - (a + b)) < 1e-3
    assert b < a  # nothing queued between 11 and 12
    with pytest.raises(we.WeError, match="out of range"):
        graph.timer_mark(we.TIMER_MARKS)
    with pytest.raises(we.WeError):
        graph.timer_between(10, we.TIMER_MARKS)

"""we_matmul_noalloc: the GEMM entry point that allocates nothing, for callers that cannot allocate (graph
capture, serving loops). Its split-K partial sums live in a fixed per-GPU device array; the results must equal
we_matmul's bit for bit (same kernels, same split plan), call after call, a smaller call after a larger one
included (the array keeps the last call's contents), and match the oracle at the GEMM bars."""
import numpy as np
import pytest

import oracle_lib as O
import we

pytestmark = pytest.mark.gpu


def _decode(raw, dt):
    if dt == we.F32:
        return raw.view(np.float32).astype(np.float64)
    if dt == we.F16:
        return raw.view(np.float16).astype(np.float64)
    return O.bf16_to_f32(raw.view(np.uint16)).astype(np.float64)


def _operands(rng, m, n, k, x_dt):
    xf = rng.standard_normal(m * k).astype(np.float32)
    if x_dt == we.F16:
        x = xf.astype(np.float16).view(np.uint16)
        ox = O.F16
    else:
        x = O.bf16_rne(xf)
        ox = O.BF16
    w = rng.integers(0, 254, n * k).astype(np.uint8)
    w = (w + (w >= 0x7F)).astype(np.uint8)
    return x, ox, w


# (m, n, k, x dtype, y dtype, flags): the second call is smaller than the first, so it runs over the first call's
# leftovers in the array
CASES = [(64, 3072, 3072, we.F16, we.F16, 0), (16, 1024, 2048, we.BF16, we.F32, we.EPI_BIAS | we.EPI_GELU)]


def test_noalloc_equals_we_matmul_on_two_calls_in_a_row(graph):
    rng = np.random.default_rng(21)
    for m, n, k, x_dt, y_dt, flags in CASES:
        x, ox, w = _operands(rng, m, n, k, x_dt)
        bias = rng.normal(0, 1, n).astype(np.float32) if flags & we.EPI_BIAS else None
        p = we.matmul_params(m, n, k, 0.02, graph=graph)
        mark = graph.mark()
        xb, wb = graph.buffer(x), graph.buffer(w)
        bb = graph.buffer(bias) if bias is not None else None
        y_ref, y_na = graph.buffer(m * n * we.ELEM_BYTES[y_dt]), graph.buffer(m * n * we.ELEM_BYTES[y_dt])
        graph.matmul(p, x_dt, xb, we.FP8, wb, y_dt, y_ref, bias=bb, flags=flags)
        created = graph.stats["created"]
        graph.matmul_noalloc(p, x_dt, xb, we.FP8, wb, y_dt, y_na, bias=bb, flags=flags)
        assert graph.stats["created"] == created
        ref, got = graph.read(y_ref), graph.read(y_na)
        graph.release(mark)
        assert np.array_equal(got, ref), (m, n, k)
        want = O.matmul(O.matmul_params(m, n, k, 0.02), ox, x, O.FP8, w)
        if bias is not None:
            want = want + np.tile(bias.astype(np.float64), m)
        if flags & we.EPI_GELU:
            want = O.gelu_tanh(want)
        tol = 1e-4 if flags & we.EPI_GELU else {we.F32: 1e-5, we.F16: 2e-3, we.BF16: 1e-2}[y_dt]
        assert O.rel_error(_decode(got, y_dt), want) < tol, (m, n, k)


def test_noalloc_replays_under_graph_capture(graph):
    """Captured in a HIP graph (where no allocation may happen) and replayed over new inputs: every replay equals
    we_matmul run eagerly on the same inputs."""
    rng = np.random.default_rng(22)
    m, n, k = 64, 3072, 3072
    x, _, w = _operands(rng, m, n, k, we.F16)
    p = we.matmul_params(m, n, k, 0.02, graph=graph)
    mark = graph.mark()
    xb, wb = graph.buffer(x), graph.buffer(w)
    y_ref, y_na = graph.buffer(m * n * 2), graph.buffer(m * n * 2)
    graph.sync()
    graph.graph_begin()
    graph.matmul_noalloc(p, we.F16, xb, we.FP8, wb, we.F16, y_na)
    gr = graph.graph_end()
    try:
        for rep in range(2):
            graph.write(xb, rng.standard_normal(m * k).astype(np.float16))
            graph.matmul(p, we.F16, xb, we.FP8, wb, we.F16, y_ref)
            graph.graph_launch(gr)
            assert np.array_equal(graph.read(y_na), graph.read(y_ref)), rep
    finally:
        graph.graph_destroy(gr)
        graph.release(mark)


def test_noalloc_refuses_a_split_plan_beyond_its_array(graph):
    """512 x 3072 x 3072 (few 128 x 128 tiles: six K slices of partial sums, 37.7 MB) needs more than the 16 MiB
    array: a clear error, and we_matmul runs the same GEMM."""
    m, n, k = 512, 3072, 3072
    rng = np.random.default_rng(23)
    x, _, w = _operands(rng, m, n, k, we.BF16)
    p = we.matmul_params(m, n, k, 0.02, graph=graph)
    mark = graph.mark()
    xb, wb, y = graph.buffer(x), graph.buffer(w), graph.buffer(m * n * 2)
    with pytest.raises(we.WeError, match=r"needs \d+ bytes of split-K scratch; the allocation-free entry point has "
                                         r"16777216"):
        graph.matmul_noalloc(p, we.BF16, xb, we.FP8, wb, we.BF16, y)
    graph.matmul(p, we.BF16, xb, we.FP8, wb, we.BF16, y)
    graph.sync()
    graph.release(mark)


def test_noalloc_refuses_the_second_stream_and_other_contexts(graph):
    """Every call on a GPU shares its fixed array, so calls that could overlap are refused rather than raced: a call
    while compute stream 1 is selected fails, and so does a call from a second live context while this one holds
    the array; we_matmul runs in both places, and this context's calls on stream 0 go on working."""
    m, n, k = 16, 1024, 2048
    rng = np.random.default_rng(24)
    x, _, w = _operands(rng, m, n, k, we.BF16)
    p = we.matmul_params(m, n, k, 0.02, graph=graph)
    mark = graph.mark()
    xb, wb, y, y2 = graph.buffer(x), graph.buffer(w), graph.buffer(m * n * 2), graph.buffer(m * n * 2)
    graph.matmul_noalloc(p, we.BF16, xb, we.FP8, wb, we.BF16, y)  # this context now holds the device's array
    graph.stream(1)
    try:
        with pytest.raises(we.WeError, match="compute stream 0 only"):
            graph.matmul_noalloc(p, we.BF16, xb, we.FP8, wb, we.BF16, y2)
    finally:
        graph.stream(0)
    other = we.Graph(0)
    try:
        op = we.matmul_params(m, n, k, 0.02, graph=other)
        ox, ow, oy = other.buffer(x), other.buffer(w), other.buffer(m * n * 2)
        with pytest.raises(we.WeError, match="belongs to another live context"):
            other.matmul_noalloc(op, we.BF16, ox, we.FP8, ow, we.BF16, oy)
        other.matmul(op, we.BF16, ox, we.FP8, ow, we.BF16, oy)
        other_y = other.read(oy)
    finally:
        other.destroy()
    graph.matmul_noalloc(p, we.BF16, xb, we.FP8, wb, we.BF16, y2)
    assert np.array_equal(graph.read(y2), graph.read(y))
    assert np.array_equal(other_y, graph.read(y))
    graph.release(mark)

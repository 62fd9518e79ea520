"""Elementwise ops, layerSum, the Graph buffer semantics and weight streaming on the GPU.
Mirrors tests/gpu/elementwise.test.ts:15-40, tests/gpu/text.test.ts:56-60 and tests/gpu/graph.test.ts."""
import numpy as np
import pytest

import oracle_lib as O
import we

pytestmark = pytest.mark.gpu


def centered(seed, n, size=16):
    return ((O.lcg(seed, n) - 0.5) * size).astype(np.float32)


@pytest.mark.parametrize("dtype", [we.F32, we.BF16])
def test_elementwise_ops(graph, dtype):
    n, d = 1000, 40
    a, b, g = centered(1, n), centered(2, n), centered(7, d, 2)
    if dtype == we.BF16:
        a, b = O.bf16_to_f32(O.bf16_rne(a)), O.bf16_to_f32(O.bf16_rne(b))
    store = (lambda v: v) if dtype == we.F32 else O.bf16_rne
    A, B = graph.buffer(store(a)), graph.buffer(store(b))
    G = graph.buffer(g)
    cases = [
        (we.swiglu(graph, A, B, n, dtype), O.elementwise(O.SWIGLU, a, b), 1e-4),
        (we.sigmoid_gate(graph, A, B, n, dtype), O.elementwise(O.SIGMOID_GATE, a, b), 1e-5),
        (we.gated_add(graph, A, B, G, n, d, dtype), O.elementwise(O.GATED_ADD, a, b, g, d), 1e-5),
        (we.add_bias(graph, A, G, n, d, dtype), O.elementwise(O.ADD_BIAS, a, g, d=d), 1e-6),
        (we.add(graph, A, B, n, dtype), O.elementwise(O.ADD, a, b), 1e-6),
        (we.silu(graph, A, n, dtype), O.elementwise(O.SILU, a), 1e-5),
    ]
    for buf, want, tol in cases:
        raw = graph.read(buf)
        got = raw.view(np.float32).astype(np.float64) if dtype == we.F32 else O.bf16_to_f32(
            raw.view(np.uint16)).astype(np.float64)
        bound = tol if dtype == we.F32 else 2 ** -8 * np.abs(want) + 1e-5
        assert np.all(np.abs(got - want) <= bound)


def test_gelu_far_from_zero(graph):  # tests/gpu/text.test.ts:56-60
    x = np.concatenate([centered(8, 200), np.array([-60, 60, 0], np.float32)])
    got = graph.read(we.gelu(graph, graph.buffer(x), x.size), dtype=np.float32, count=x.size)
    want = np.array([O.lib.or_gelu_tanh(float(v)) for v in x])
    assert np.abs(got - want).max() < 1e-5


def test_layer_sum(graph):  # src/kernels/text.ts:67-84
    t, layers, dim = 9, 4, 33
    x = centered(3, t * layers * dim)
    w = np.array([1.0, -0.5, 2.0, 0.25], np.float32)
    out = graph.buffer(t * dim * 4)
    graph.layer_sum(t, layers, dim, graph.buffer(x), graph.buffer(w), out)
    got = graph.read(out, dtype=np.float32, count=t * dim)
    assert np.abs(got - O.layer_sum(t, layers, dim, x, w)).max() < 1e-5


def test_reused_buffers_come_back_zeroed(graph):  # tests/gpu/graph.test.ts (reuse + zeroing)
    before = graph.stats
    a = graph.buffer(np.arange(1000, dtype=np.float32))
    graph.free(a)
    b = graph.buffer(4000)
    assert b.ptr == a.ptr
    assert not graph.read(b).any()
    after = graph.stats
    assert after["reused"] == before["reused"] + 1
    mark = graph.mark()
    keep = graph.buffer(16)
    drop = graph.buffer(16)
    graph.release(mark, [keep])
    again = graph.buffer(16)
    assert again.ptr == drop.ptr
    graph.free(keep)
    graph.free(again)
    graph.free(b)


def test_copy_is_ordered_with_dispatches(graph):  # tests/gpu/graph.test.ts (copy order)
    src = graph.buffer(np.arange(64, dtype=np.float32))
    dst = graph.buffer(256)
    out = we.add(graph, src, src, 64)  # 2 * src
    graph.copy(out, 0, dst, 0, 256)
    assert np.array_equal(graph.read(dst, dtype=np.float32, count=64), 2 * np.arange(64, dtype=np.float32))


def test_stream_copy_double_buffer(graph):
    """Pinned host -> device on the copy stream into two slots, compute waiting on each copy's ticket
    and each slot refilled only after the compute that read it (the double buffer the layer loop uses)."""
    n = 1 << 20
    layers = [np.full(n, i + 1, np.float32) for i in range(5)]
    pinned = [graph.host_alloc(n * 4) for _ in range(2)]
    slots = [graph.buffer(n * 4) for _ in range(2)]
    acc = graph.buffer(np.zeros(n, np.float32))
    done = [0, 0]
    import ctypes
    for i, data in enumerate(layers):
        s = i % 2
        if done[s]:
            graph.sync()  # the host may overwrite a pinned slot only after its copy finished
        ctypes.memmove(pinned[s], data.ctypes.data, n * 4)
        t = graph.stream_copy(slots[s], pinned[s], n * 4, after=done[s])
        graph.wait_ticket(t)
        nxt = we.add(graph, acc, slots[s], n)
        graph.copy(nxt, 0, acc, 0, n * 4)
        graph.free(nxt)
        done[s] = graph.record_compute()
    got = graph.read(acc, dtype=np.float32, count=n)
    assert np.all(got == 15.0)
    assert graph.ticket_done(done[0]) and graph.ticket_done(done[1])
    for p in pinned:
        graph.host_free(p)

"""Failure injection through the C-ABI (we_set_alloc_cap, we_set_poison).

An allocation cap forces the out-of-memory paths a full device would take, in buffer creation and in the kernel
scratch a split-K GEMM grows; each must fail with WE_ENOMEM and a message, and leave the context usable. Poison
mode fills freed and released buffers with 0xff bytes, so a stale read sees NaN, while a reused buffer still
starts zeroed (src/gpu/graph.ts:48-51). Every kernel here runs in bounds and ends normally: the failures are
refused on the host before any launch.
"""
import numpy as np
import pytest

import oracle_lib as O
import we

pytestmark = pytest.mark.gpu

KIB = 1024


@pytest.fixture
def ctx():
    g = we.Graph(0)
    yield g
    g.destroy()


def test_buffer_creation_past_the_cap_fails_and_the_context_recovers(ctx):
    held0 = ctx.set_alloc_cap(0)
    ctx.set_alloc_cap(held0 + 1024 * KIB)
    a = ctx.buffer(512 * KIB)
    with pytest.raises(we.WeError) as err:
        ctx.buffer(768 * KIB)
    assert err.value.code == 2  # WE_ENOMEM
    assert str(err.value).startswith("hipMalloc(786432): ") and str(err.value).endswith("(allocation cap set)")
    # the pool still serves: a buffer of a freed size allocates nothing and is never refused
    ctx.free(a)
    before = ctx.stats
    b = ctx.buffer(np.arange(512 * KIB // 4, dtype=np.float32))
    assert ctx.stats["reused"] == before["reused"] + 1 and ctx.stats["created"] == before["created"]
    assert np.array_equal(ctx.read(b, dtype=np.float32), np.arange(512 * KIB // 4, dtype=np.float32))
    # lifting the cap lets the refused size through; the held count went up by exactly the two creations
    assert ctx.set_alloc_cap(0) == held0 + 512 * KIB
    c = ctx.buffer(768 * KIB)
    assert ctx.set_alloc_cap(0) == held0 + 512 * KIB + 768 * KIB
    assert not ctx.read(c).any()


def test_split_k_scratch_past_the_cap_fails_before_launch_and_then_runs(ctx):
    m, n, k = 64, 3072, 3072  # split-K at M = 64: partial sums in the context's kernel scratch (>= 16 MiB)
    rng = np.random.default_rng(3)
    x = rng.standard_normal(m * k).astype(np.float16)
    w = rng.integers(0, 254, n * k).astype(np.uint8)
    w = (w + (w >= 0x7F)).astype(np.uint8)
    bx, bw = ctx.buffer(x), ctx.buffer(w)
    y = ctx.buffer(m * n * 4)
    p = we.matmul_params(m, n, k, 0.02, graph=ctx)
    held = ctx.set_alloc_cap(0)
    ctx.set_alloc_cap(held + 4 * 1024 * KIB)
    with pytest.raises(we.WeError) as err:
        ctx.matmul(p, we.F16, bx, we.FP8, bw, we.F32, y)
    assert err.value.code == 2
    assert str(err.value).startswith("scratch of ") and str(err.value).endswith("(allocation cap set)")
    assert not ctx.read(y).any()  # nothing was launched
    ctx.set_alloc_cap(0)
    ctx.matmul(p, we.F16, bx, we.FP8, bw, we.F32, y)
    got = ctx.read(y, dtype=np.float32).astype(np.float64)
    rows = O.matmul_rows(O.matmul_params(m, n, k, 0.02), O.F16, x.view(np.uint16), O.FP8, w, 0, 4)[: 4 * n]
    assert O.rel_error(got[: 4 * n], rows) < 1e-5


def test_poison_fills_freed_and_released_buffers_with_nan(ctx):
    data = np.linspace(-3, 3, 4096, dtype=np.float32)
    # off (the default): a freed buffer keeps its bytes until it is reused
    a = ctx.buffer(data)
    ctx.free(a)
    assert np.array_equal(ctx.read(a, dtype=np.float32), data)
    ctx.buffer(data.nbytes)  # takes `a` back from the pool
    ctx.set_poison(True)
    b = ctx.buffer(data)
    ctx.free(b)
    stale = ctx.read(b, dtype=np.uint8)
    assert (stale == 0xFF).all() and np.isnan(stale.view(np.float32)).all()
    again = ctx.buffer(data.nbytes)  # the same block, zeroed again on reuse
    assert again.ptr == b.ptr and not ctx.read(again).any()
    mark = ctx.mark()
    kept, dropped = ctx.buffer(data), ctx.buffer(data[::-1].copy())
    ctx.release(mark, keep=[kept])
    assert np.array_equal(ctx.read(kept, dtype=np.float32), data)
    assert (ctx.read(dropped, dtype=np.uint8) == 0xFF).all()
    ctx.set_poison(False)

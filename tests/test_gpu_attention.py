"""Attention on the GPU through the C-ABI, against the float64 oracle.

Mirrors tests/gpu/attention.test.ts (its shapes, its LCG inputs, its 1e-5 bound for f32) and adds 16-bit
operands (bf16 / f16, fp32 softmax and accumulation) at ragged, GQA, causal and full double-stream-block
sizes, plus q/k/v read in place from a fused QKV row.

Tolerances: f32 max|out - ref| < 1e-5 (the reference's bar); 16-bit max|out - ref| / max|ref| < 1e-2
(the bar for matmul-class outputs) against the oracle run on the same rounded inputs.
"""
import numpy as np
import pytest

import oracle_lib as O
import we

pytestmark = pytest.mark.gpu


def lcg_random(seed, sizes, scale=2.0):
    """tests/gpu/attention.test.ts:6-7: one LCG stream, ((u * 2) - 1) * size as f32, drawn in order."""
    u = O.lcg(seed, sum(sizes))
    out, i = [], 0
    for n in sizes:
        out.append(((u[i:i + n] * 2 - 1) * scale).astype(np.float32))
        i += n
    return out


def run(graph, q, k, v, shape, dtype):
    mark = graph.mark()
    out = we.attention(graph, graph.buffer(q), graph.buffer(k), graph.buffer(v), shape, dtype)
    raw = graph.read(out)
    graph.release(mark)
    return decode(raw, dtype)


def decode(raw, dtype):
    if dtype == we.F32:
        return raw.view(np.float32).astype(np.float64)
    if dtype == we.F16:
        return raw.view(np.float16).astype(np.float64)
    return O.bf16_to_f32(raw.view(np.uint16)).astype(np.float64)


def to16(x32, dtype):
    """f32 -> (storage, exact f64 values the kernel sees)"""
    if dtype == we.F16:
        h = x32.astype(np.float16)
        return h.view(np.uint16), h.astype(np.float64)
    b = O.bf16_rne(x32)
    return b, O.bf16_to_f32(b).astype(np.float64)


@pytest.mark.parametrize("tokens,heads,kv_heads,dim", [(37, 4, 1, 128), (64, 8, 2, 128)])
def test_matches_cpu_reference(graph, tokens, heads, kv_heads, dim):  # tests/gpu/attention.test.ts:35-54
    q, k, v = lcg_random(1, [tokens * heads * dim, tokens * kv_heads * dim, tokens * kv_heads * dim])
    shape = we.AttentionShape(tokens, heads, kv_heads, dim)
    got = run(graph, q, k, v, shape, we.F32)
    want = O.attention(q, k, v, tokens, heads, kv_heads, dim)
    assert np.abs(got - want).max() < 1e-5


def test_refuses_heads_not_split_over_kv_heads(graph):  # tests/gpu/attention.test.ts:56-61
    b = graph.buffer(4)
    with pytest.raises(we.WeError, match="multiple"):
        we.attention(graph, b, b, b, we.AttentionShape(1, 3, 2, 4))
    with pytest.raises(we.WeError, match="heads must be a multiple of kvHeads"):
        graph.attention(1, 3, 2, 4, False, we.F32, b, b, b, b)


def test_query_chunks_give_the_same_result(graph):  # tests/gpu/attention.test.ts:64-84
    tokens, heads, kv_heads, dim = 50, 2, 1, 16
    q, k, v = lcg_random(5, [tokens * heads * dim, tokens * kv_heads * dim, tokens * kv_heads * dim])
    whole = run(graph, q, k, v, we.AttentionShape(tokens, heads, kv_heads, dim), we.F32)
    chunked = run(graph, q, k, v, we.AttentionShape(tokens, heads, kv_heads, dim, chunk=16), we.F32)
    assert np.abs(chunked - whole).max() < 1e-6
    assert np.abs(chunked - O.attention(q, k, v, tokens, heads, kv_heads, dim)).max() < 1e-5


@pytest.mark.parametrize("chunk", [None, 7])
def test_causal_only_looks_at_earlier_tokens(graph, chunk):  # tests/gpu/attention.test.ts:87-101
    tokens, heads, kv_heads, dim = 19, 4, 1, 128
    q, k, v = lcg_random(9, [tokens * heads * dim, tokens * kv_heads * dim, tokens * kv_heads * dim])
    got = run(graph, q, k, v, we.AttentionShape(tokens, heads, kv_heads, dim, chunk=chunk, causal=True), we.F32)
    assert np.abs(got - O.attention(q, k, v, tokens, heads, kv_heads, dim, causal=True)).max() < 1e-5


@pytest.mark.parametrize("tokens,heads,kv_heads,dim,causal", [
    (37, 4, 1, 128, False), (200, 6, 2, 64, False), (300, 4, 4, 128, True), (129, 3, 1, 32, False),
    (65, 2, 1, 16, True), (1000, 2, 1, 128, False), (513, 4, 2, 96, True)])
@pytest.mark.parametrize("dtype", [we.BF16, we.F16])
def test_16bit_operands(graph, tokens, heads, kv_heads, dim, causal, dtype):
    rng = np.random.default_rng(tokens * 7 + heads + dim)
    q, qv = to16(rng.standard_normal(tokens * heads * dim).astype(np.float32) * 2, dtype)
    k, kv = to16(rng.standard_normal(tokens * kv_heads * dim).astype(np.float32) * 2, dtype)
    v, vv = to16(rng.standard_normal(tokens * kv_heads * dim).astype(np.float32), dtype)
    got = run(graph, q, k, v, we.AttentionShape(tokens, heads, kv_heads, dim, causal=causal), dtype)
    want = O.attention(qv, kv, vv, tokens, heads, kv_heads, dim, causal)
    assert O.rel_error(got, want) < 1e-2


def test_f32_ragged_and_gqa(graph):
    tokens, heads, kv_heads, dim = 130, 6, 3, 64
    q, k, v = lcg_random(13, [tokens * heads * dim, tokens * kv_heads * dim, tokens * kv_heads * dim])
    for causal in (False, True):
        got = run(graph, q, k, v, we.AttentionShape(tokens, heads, kv_heads, dim, causal=causal), we.F32)
        assert np.abs(got - O.attention(q, k, v, tokens, heads, kv_heads, dim, causal)).max() < 1e-5


def test_fused_qkv_rows_in_place(graph):
    """q, k and v read as column slices of one [tokens, 3 * heads * dim] projection, out written into a wider
    row: the result equals the dense layout's bit for bit."""
    tokens, heads, dim = 300, 4, 128
    row = heads * dim
    rng = np.random.default_rng(1)
    qkv = O.bf16_rne(rng.standard_normal(tokens * 3 * row).astype(np.float32))
    parts = qkv.reshape(tokens, 3, row)
    q, k, v = (np.ascontiguousarray(parts[:, i]) for i in range(3))
    dense = run(graph, q, k, v, we.AttentionShape(tokens, heads, heads, dim), we.BF16)
    mark = graph.mark()
    buf = graph.buffer(qkv)
    out = graph.buffer(tokens * (row + 64) * 2)
    graph.attention(tokens, heads, heads, dim, False, we.BF16, buf, we.Graph.slice(buf, row * 2, 0),
                    we.Graph.slice(buf, 2 * row * 2, 0), out, q_stride=3 * row, k_stride=3 * row, v_stride=3 * row,
                    out_stride=row + 64)
    raw = graph.read(out).view(np.uint16).reshape(tokens, row + 64)
    graph.release(mark)
    assert np.array_equal(O.bf16_to_f32(raw[:, :row]).astype(np.float64).ravel(), dense)
    assert not raw[:, row:].any()  # the gap between rows is untouched


def test_double_stream_block_shape_sampled_rows(graph):
    """The block's joint attention: 512 text + 4096 image tokens, 24 heads of 128, bf16. Every output is
    computed; three blocks of query rows (first, middle, last) are checked against the oracle."""
    tokens, heads, dim = 4608, 24, 128
    rng = np.random.default_rng(4608)
    q, qv = to16(rng.standard_normal(tokens * heads * dim).astype(np.float32) * 2, we.BF16)
    k, kv = to16(rng.standard_normal(tokens * heads * dim).astype(np.float32) * 2, we.BF16)
    v, vv = to16(rng.standard_normal(tokens * heads * dim).astype(np.float32), we.BF16)
    got = run(graph, q, k, v, we.AttentionShape(tokens, heads, heads, dim), we.BF16).reshape(tokens, -1)
    assert np.isfinite(got).all()
    for b, e in [(0, 24), (2300, 2324), (4584, 4608)]:
        want = O.attention(qv, kv, vv, tokens, heads, heads, dim, rows=(b, e))
        assert O.rel_error(got[b:e].ravel(), want) < 1e-2, (b, e)


@pytest.mark.parametrize("tokens,heads,kv_heads,causal,dtype", [
    (4608, 24, 24, False, we.BF16), (300, 4, 2, True, we.F16), (65, 3, 1, False, we.BF16), (1000, 8, 8, True, we.BF16),
    (257, 2, 2, False, we.F16), (64, 1, 1, False, we.BF16), (200, 2, 1, True, we.BF16), (2048, 4, 2, True, we.F16)])
def test_dma_ring_path_equals_register_path(graph, tune, tokens, heads, kv_heads, causal, dtype):
    """Head dim 128 with 16-bit operands: the default ping-pong kernel on 32x32x16 MFMAs and the single-phase
    DMA-ring kernel (attn_path 2) share the register-staged kernel's per-tile arithmetic, so their outputs equal it
    bit for bit. The ping-pong kernel on 16x16x32 MFMAs (attn_path 3) sums the same products in another order
    inside its MFMAs: it matches the register path to within two output roundings (and the oracle, below)."""
    rng = np.random.default_rng(tokens + heads)
    q, qv = to16(rng.standard_normal(tokens * heads * 128).astype(np.float32) * 2, dtype)
    k, kv = to16(rng.standard_normal(tokens * kv_heads * 128).astype(np.float32) * 2, dtype)
    v, vv = to16(rng.standard_normal(tokens * kv_heads * 128).astype(np.float32), dtype)
    shape = we.AttentionShape(tokens, heads, kv_heads, 128, causal=causal)
    pp32 = run(graph, q, k, v, shape, dtype)
    tune(attn_path=3)
    pp16 = run(graph, q, k, v, shape, dtype)
    tune(attn_path=2)
    ring = run(graph, q, k, v, shape, dtype)
    tune(attn_path=1)
    reg = run(graph, q, k, v, shape, dtype)
    assert np.array_equal(ring, reg)
    assert np.array_equal(pp32, reg)
    ulp = 2.0 ** -8 if dtype == we.BF16 else 2.0 ** -11
    assert O.rel_error(pp16, reg) < 2 * ulp, O.rel_error(pp16, reg)
    rows = (0, min(tokens, 16))
    want = O.attention(qv, kv, vv, tokens, heads, kv_heads, 128, causal, rows=rows)
    assert O.rel_error(pp16.reshape(tokens, -1)[rows[0]:rows[1]].ravel(), want) < 1e-2


@pytest.mark.parametrize("tokens", [1, 2, 63, 255, 256])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", [we.BF16, we.F32])
def test_tiny_and_block_edge_token_counts(graph, tokens, causal, dtype):
    """Token counts at the edges of the kernels' work units: one and two tokens (a single key tile, most rows of
    the workgroup past the end), one short of a key tile, and one short of / exactly a 256-query block. Head dim
    128, 2 query heads over 1 kv head; every output against the oracle. f32 takes the reference test's inputs
    (one LCG stream, uniform in [-2, 2]), which its 1e-5 bar is set for; 16-bit takes normal inputs."""
    heads, kv_heads, dim = 2, 1, 128
    sizes = [tokens * heads * dim, tokens * kv_heads * dim, tokens * kv_heads * dim]
    shape = we.AttentionShape(tokens, heads, kv_heads, dim, causal=causal)
    if dtype == we.F32:
        q32, k32, v32 = lcg_random(tokens * 2 + causal + 1, sizes)
        got = run(graph, q32, k32, v32, shape, dtype)
        want = O.attention(q32, k32, v32, tokens, heads, kv_heads, dim, causal)
        assert np.abs(got - want).max() < 1e-5
    else:
        rng = np.random.default_rng(tokens * 2 + causal)
        q32, k32 = (rng.standard_normal(n).astype(np.float32) * 2 for n in sizes[:2])
        v32 = rng.standard_normal(sizes[2]).astype(np.float32)
        (q, qv), (k, kv), (v, vv) = (to16(x, dtype) for x in (q32, k32, v32))
        got = run(graph, q, k, v, shape, dtype)
        want = O.attention(qv, kv, vv, tokens, heads, kv_heads, dim, causal)
        assert O.rel_error(got, want) < 1e-2

"""Whole blocks on the GPU against the float64 oracle compositions.

- The Krea single-stream block with tests/gpu/block.test.ts's own tiny configuration and LCG inputs, to its
  bars (cosine > 0.99999, L2-relative error < 1e-4), and its temporary-freeing check.
- The double-stream DiT block: tiny in f32 (same bars) and bf16; full hidden size with few tokens (bf16); the
  full 512 + 4096-token shape (finite, zero gates give the input back bit for bit); a forward that allocates
  nothing; and weights streamed from pinned host memory giving the resident result bit for bit.

bf16 bars: cosine > 0.9999 and L2-relative error < 1e-2 against the oracle on the same bf16-rounded inputs;
the block rounds its activations to bf16 after every step (norms, projections, attention, residuals).
"""
import numpy as np
import pytest

import block as B
import oracle_lib as O
import we

pytestmark = pytest.mark.gpu


def read_as_f64(graph, buf, dtype, count):
    raw = graph.read(buf)
    if dtype == we.F32:
        return raw.view(np.float32)[:count].astype(np.float64)
    return O.bf16_to_f32(raw.view(np.uint16)[:count]).astype(np.float64)


# ------------------------------------------------------------------------------------------ Krea block

KREA_TINY = B.BlockConfig(64, 96, 4, 2, 16, 1e-5)  # tests/gpu/block.test.ts:11
AXES = [4, 6, 6]


class _Draws:
    """tests/gpu/block.test.ts:14-21: one LCG stream; floats(n, size) = rand() * size, fp8 bytes
    floor((rand() + 1) * 128) & 0xff with the NaN codes moved down by one."""

    def __init__(self, seed):
        self.s = seed

    def _u(self, n):
        out = np.empty(n, np.float64)
        s = self.s
        for i in range(n):
            s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
            out[i] = s / 2 ** 32
        self.s = s
        return out

    def floats(self, n, size):
        return ((self._u(n) * 2 - 1) * size).astype(np.float32)

    def fp8(self, n):
        b = (np.floor(self._u(n) * 256).astype(np.int64) & 0xFF).astype(np.uint8)
        b[(b & 0x7F) == 0x7F] -= 1
        return b


def _krea_case(graph):
    cfg = KREA_TINY
    H, M, hd = cfg.hidden, cfg.mlp, cfg.head_dim
    d = _Draws(1)
    shapes = [("wq", cfg.heads * hd, H), ("wk", cfg.kv_heads * hd, H), ("wv", cfg.kv_heads * hd, H), ("gate", H, H),
              ("wo", H, H), ("mlp_gate", M, H), ("mlp_up", M, H), ("mlp_down", H, M)]
    cpu_w = {name: (d.fp8(n * k), 0.002, n, k) for name, n, k in shapes}
    vecs = dict(norm1=d.floats(H, 0.5), norm2=d.floats(H, 0.5), norm_q=d.floats(hd, 0.5), norm_k=d.floats(hd, 0.5),
                table=d.floats(6 * H, 0.3))
    temb = d.floats(6 * H, 0.3)
    pos = B.positions(3, 2, 3)
    cos, sin, pairs = B.rope_tables(pos, AXES, 1000.0)
    tokens = pos.shape[0]
    x = d.floats(tokens * H, 2)
    return cfg, cpu_w, vecs, temb, cos, sin, pairs, tokens, x


def test_krea_block_like_the_reference(graph):  # tests/gpu/block.test.ts:102-138
    cfg, cpu_w, vecs, temb, cos, sin, pairs, tokens, x = _krea_case(graph)
    mark = graph.mark()
    lin = {n: we.Linear(graph.buffer(b), "fp8", s, nn, k) for n, (b, s, nn, k) in cpu_w.items()}
    w = B.BlockWeights(**lin, **{n: graph.buffer(v) for n, v in vecs.items()})
    rope = we.Rope(graph.buffer(cos), graph.buffer(sin), pairs, tokens)
    out = B.block(graph, w, cfg, graph.buffer(x), graph.buffer(temb), rope)
    got = graph.read(out, dtype=np.float32, count=tokens * cfg.hidden).astype(np.float64)
    graph.release(mark)
    order = ["wq", "wk", "wv", "gate", "wo", "mlp_gate", "mlp_up", "mlp_down"]
    want = O.krea_block(cfg, tokens, x.astype(np.float64), [cpu_w[n] for n in order], vecs["norm1"], vecs["norm2"],
                        vecs["norm_q"], vecs["norm_k"], vecs["table"], temb, cos, sin)
    r = O.compare(got, want)
    assert r["cosine"] > 0.99999 and r["relativeError"] < 1e-4, r


def test_krea_block_frees_its_temporaries():  # tests/gpu/block.test.ts:141-180
    cfg = KREA_TINY

    class KeepAll(we.Graph):
        def free(self, buf):  # every temporary stays until the end
            pass

    def block_bytes(graph):
        tokens = 48
        lin = lambda n, k: we.Linear(graph.buffer(n * k), "fp8", 1.0, n, k)  # noqa: E731
        H, M, hd = cfg.hidden, cfg.mlp, cfg.head_dim
        w = B.BlockWeights(lin(cfg.heads * hd, H), lin(cfg.kv_heads * hd, H), lin(cfg.kv_heads * hd, H), lin(H, H),
                           lin(H, cfg.heads * hd), lin(M, H), lin(M, H), lin(H, M), graph.buffer(H * 4),
                           graph.buffer(H * 4), graph.buffer(hd * 4), graph.buffer(hd * 4), graph.buffer(6 * H * 4))
        cos, sin, pairs = B.rope_tables(B.positions(0, 6, 8), AXES, 1000.0)
        rope = we.Rope(graph.buffer(cos), graph.buffer(sin), pairs, tokens)
        x, tvec = graph.buffer(tokens * H * 4), graph.buffer(6 * H * 4)
        before = graph.stats["createdBytes"]
        B.block(graph, w, cfg, x, tvec, rope)
        graph.sync()
        used = graph.stats["createdBytes"] - before
        graph.destroy()
        return used

    freed, kept = block_bytes(we.Graph(0)), block_bytes(KeepAll(0))
    assert freed < 0.6 * kept, (freed, kept)


# ------------------------------------------------------------------------------------------ double-stream block

def _double_weights(rng, cfg):
    """Per stream: fp8 linears (bytes, scale, n, k) and f32 vectors, as the oracle takes them."""
    H, M, hd = cfg.hidden, cfg.mlp, cfg.head_dim

    def lin(n, k):
        b = rng.integers(0, 254, n * k, dtype=np.uint8)
        return (b + (b >= 0x7f)).astype(np.uint8), float(np.float32(2.0 / np.sqrt(k) / 200)), n, k

    v = lambda n, s: rng.uniform(-s, s, n).astype(np.float32)  # noqa: E731
    return [dict(qkv=lin(3 * H, H), proj=lin(H, H), up=lin(M, H), down=lin(H, M), norm1=v(H, .3), norm2=v(H, .3),
                 norm_q=v(hd, .3), norm_k=v(hd, .3), table=v(6 * H, .2)) for _ in range(2)]


def _upload_stream(graph, sw):
    lin = lambda name: we.Linear(graph.buffer(sw[name][0]), "fp8", sw[name][1], sw[name][2], sw[name][3])  # noqa
    return B.StreamWeights(lin("qkv"), lin("proj"), lin("up"), lin("down"),
                           *[graph.buffer(sw[n]) for n in ("norm1", "norm2", "norm_q", "norm_k", "table")])


def _store(x32, dtype):
    if dtype == we.F32:
        return x32, x32.astype(np.float64)
    b = O.bf16_rne(x32)
    return b, O.bf16_to_f32(b).astype(np.float64)


def _run_double(graph, cfg, tt, rows, cols, dtype, seed):
    ti = rows * cols
    rng = np.random.default_rng(seed)
    wt, wi = _double_weights(rng, cfg)
    tvec = rng.uniform(-.2, .2, 6 * cfg.hidden).astype(np.float32)
    xt, xt64 = _store(rng.uniform(-2, 2, tt * cfg.hidden).astype(np.float32), dtype)
    xi, xi64 = _store(rng.uniform(-2, 2, ti * cfg.hidden).astype(np.float32), dtype)
    rope = B.rope_for_image(graph, rows, cols, axes=(cfg.head_dim // 2, cfg.head_dim // 2))
    mark = graph.mark()
    blk = B.DoubleBlock(graph, cfg, tt, ti, dtype)
    e = we.ELEM_BYTES[dtype]
    out_t, out_i = graph.buffer(tt * cfg.hidden * e), graph.buffer(ti * cfg.hidden * e)
    blk.forward(_upload_stream(graph, wt), _upload_stream(graph, wi), graph.buffer(xt), graph.buffer(xi),
                graph.buffer(tvec), rope, out_t, out_i)
    got_t = read_as_f64(graph, out_t, dtype, tt * cfg.hidden)
    got_i = read_as_f64(graph, out_i, dtype, ti * cfg.hidden)
    graph.release(mark)
    cos, sin, _ = B.rope_tables(B.positions(0, rows, cols)[:, 1:], (cfg.head_dim // 2, cfg.head_dim // 2), 10000.0)
    want_t, want_i = O.double_block(cfg, tt, ti, xt64, xi64, wt, wi, tvec, cos, sin)
    return O.compare(np.concatenate([got_t, got_i]), np.concatenate([want_t, want_i]))


def test_double_block_tiny_f32(graph):
    r = _run_double(graph, B.BlockConfig(256, 512, 2, 2, 128, 1e-6), 24, 5, 8, we.F32, 1)
    assert r["cosine"] > 0.99999 and r["relativeError"] < 1e-4, r


def test_double_block_tiny_bf16(graph):
    r = _run_double(graph, B.BlockConfig(256, 512, 2, 2, 128, 1e-6), 24, 5, 8, we.BF16, 2)
    print(f"[bf16 tiny] {r}", flush=True)
    assert r["cosine"] > 0.9999 and r["relativeError"] < 1e-2, r


def test_double_block_full_hidden_few_tokens(graph):
    r = _run_double(graph, B.DIT_DOUBLE_BLOCK, 8, 4, 6, we.BF16, 3)
    print(f"[bf16 full hidden] {r}", flush=True)
    assert r["cosine"] > 0.9999 and r["relativeError"] < 1e-2, r


def _layout_weights(graph, cfg, rng, gates_zero=False, tvec=None):
    layout = B.StreamLayout(cfg)
    host = np.empty(layout.nbytes, np.uint8)
    layout.fill(host, rng)
    if gates_zero:  # table gate rows = -tvec: pregate = postgate = 0
        H = cfg.hidden
        for s, name, off, nbytes in layout.fields:
            if name == "table":
                t = host[off:off + nbytes].view(np.float32).reshape(6, H)
                t[2], t[5] = -tvec.reshape(6, H)[2], -tvec.reshape(6, H)[5]
    scales = {s: {n: 0.02 / np.sqrt(cfg.mlp if n == "down" else cfg.hidden) for n in ("qkv", "proj", "up", "down")}
              for s in ("txt", "img")}
    return layout, host, scales


def test_double_block_full_shape_runs_and_zero_gates_are_identity(graph):
    """512 text + 4096 image tokens (a 64 x 64 patch grid), hidden 3072, bf16: every output finite, and with
    both gates zero the block returns its input exactly (x + 0 * branch)."""
    cfg, tt, rows, cols = B.DIT_DOUBLE_BLOCK, 512, 64, 64
    ti, H = rows * cols, cfg.hidden
    rng = np.random.default_rng(5)
    tvec = rng.uniform(-.2, .2, 6 * H).astype(np.float32)
    mark = graph.mark()
    rope = B.rope_for_image(graph, rows, cols)
    xt = O.bf16_rne(rng.standard_normal(tt * H).astype(np.float32))
    xi = O.bf16_rne(rng.standard_normal(ti * H).astype(np.float32))
    blk = B.DoubleBlock(graph, cfg, tt, ti, we.BF16)
    bx_t, bx_i, tv = graph.buffer(xt), graph.buffer(xi), graph.buffer(tvec)
    out_t, out_i = graph.buffer(tt * H * 2), graph.buffer(ti * H * 2)
    for zero in (False, True):
        layout, host, scales = _layout_weights(graph, cfg, rng, gates_zero=zero, tvec=tvec)
        slot = graph.buffer(host)
        w_t, w_i = layout.weights(slot, scales)
        created = graph.stats["created"]
        blk.forward(w_t, w_i, bx_t, bx_i, tv, rope, out_t, out_i)
        assert graph.stats["created"] == created  # the forward allocates nothing
        gt = graph.read(out_t).view(np.uint16)
        gi = graph.read(out_i).view(np.uint16)
        if zero:
            assert np.array_equal(gt, xt) and np.array_equal(gi, xi)
        else:
            assert np.isfinite(O.bf16_to_f32(gt)).all() and np.isfinite(O.bf16_to_f32(gi)).all()
            assert not np.array_equal(gi, xi)
        graph.free(slot)
    graph.release(mark)


def _layout_streams(layout, host, scales):
    """The per-stream weights of a block image in the oracle's form: fp8 linears (bytes, scale, n, k), f32 vectors."""
    out = {"txt": {}, "img": {}}
    for s, name, off, nbytes in layout.fields:
        data = host[off:off + nbytes]
        if name in layout.FP8_FIELDS:
            n, k = layout._shape(name)
            out[s][name] = (data, float(np.float32(scales[s][name])), n, k)
        else:
            out[s][name] = data.view(np.float32)
    return out["txt"], out["img"]


def test_double_block_full_shape_sampled_rows_match_the_oracle(graph):
    """The block exactly as benchmarked (512 text + 4096 image tokens, hidden 3072, 24 heads of 128, fp8 weights,
    bf16 activations, non-zero gates, both streams overlapped) against the float64 composition on sampled text
    and image rows (first, last and tile-boundary rows); K and V of all 4608 tokens enter every checked row. The
    bars are those of the few-token full-hidden case: cosine > 0.9999, L2-relative error < 1e-2."""
    cfg, tt, rows, cols = B.DIT_DOUBLE_BLOCK, 512, 64, 64
    ti, H = rows * cols, cfg.hidden
    rng = np.random.default_rng(12)
    tvec = rng.uniform(-.2, .2, 6 * H).astype(np.float32)
    xt = O.bf16_rne(rng.standard_normal(tt * H).astype(np.float32))
    xi = O.bf16_rne(rng.standard_normal(ti * H).astype(np.float32))
    layout, host, scales = _layout_weights(graph, cfg, rng)
    mark = graph.mark()
    rope = B.rope_for_image(graph, rows, cols)
    blk = B.DoubleBlock(graph, cfg, tt, ti, we.BF16)
    slot = graph.buffer(host)
    w_t, w_i = layout.weights(slot, scales)
    out_t, out_i = graph.buffer(tt * H * 2), graph.buffer(ti * H * 2)
    blk.forward(w_t, w_i, graph.buffer(xt), graph.buffer(xi), graph.buffer(tvec), rope, out_t, out_i)
    got_t = O.bf16_to_f32(graph.read(out_t).view(np.uint16)).astype(np.float64).reshape(tt, H)
    got_i = O.bf16_to_f32(graph.read(out_i).view(np.uint16)).astype(np.float64).reshape(ti, H)
    graph.release(mark)
    rt, ri = [0, 1, 255, 256, 511], [0, 63, 64, 255, 256, 2047, 4032, 4095]
    cos, sin, _ = B.rope_tables(B.positions(0, rows, cols)[:, 1:], (cfg.head_dim // 2, cfg.head_dim // 2), 10000.0)
    wt, wi = _layout_streams(layout, host, scales)
    want_t, want_i = O.double_block_rows(cfg, tt, ti, O.bf16_to_f32(xt), O.bf16_to_f32(xi), wt, wi, tvec, cos, sin,
                                         rt, ri)
    for name, got, want in (("text", got_t[rt], want_t), ("image", got_i[ri], want_i)):
        r = O.compare(got.ravel(), want.ravel())
        print(f"[full block {name} rows] {r}", flush=True)
        assert r["cosine"] > 0.9999 and r["relativeError"] < 1e-2, (name, r)
        # the branch really contributes: the output is not the input
        assert np.abs(want - (O.bf16_to_f32(xt if name == "text" else xi).astype(np.float64).reshape(-1, H)[
            rt if name == "text" else ri])).max() > 0.1


@pytest.mark.parametrize("grouped", [False, True])
def test_double_block_overlapped_streams_equal_serial(graph, tune, grouped):
    """The text stream on the second compute stream beside the image stream gives the serial block's outputs bit
    for bit at the full shape (512 + 4096 tokens, hidden 3072, bf16), forward after forward (the text GEMMs'
    split-K slices use that stream's own scratch). With the QKV, output, up and down projections of the two streams
    grouped into one launch each (the default), the text tiles run in the image's tile shape with all of K, so
    the serial block is run with that tile shape and no split-K (gemm_cfg, gemm_splitk) for the
    comparison."""
    if grouped:
        tune(gemm_cfg=0, gemm_splitk=0)
    cfg, tt, rows, cols = B.DIT_DOUBLE_BLOCK, 512, 64, 64
    ti, H = rows * cols, cfg.hidden
    rng = np.random.default_rng(9)
    tvec = rng.uniform(-.2, .2, 6 * H).astype(np.float32)
    mark = graph.mark()
    rope = B.rope_for_image(graph, rows, cols)
    xt = O.bf16_rne(rng.standard_normal(tt * H).astype(np.float32))
    xi = O.bf16_rne(rng.standard_normal(ti * H).astype(np.float32))
    bx_t, bx_i, tv = graph.buffer(xt), graph.buffer(xi), graph.buffer(tvec)
    layout, host, scales = _layout_weights(graph, cfg, rng)
    slot = graph.buffer(host)
    w_t, w_i = layout.weights(slot, scales)
    outs = {}
    for overlap in (False, True):
        blk = B.DoubleBlock(graph, cfg, tt, ti, we.BF16, overlap=overlap, grouped=grouped)
        assert blk.grouped == (grouped and overlap)
        out_t, out_i = graph.buffer(tt * H * 2), graph.buffer(ti * H * 2)
        for _ in range(2):
            blk.forward(w_t, w_i, bx_t, bx_i, tv, rope, out_t, out_i)
        outs[overlap] = (graph.read(out_t).view(np.uint16), graph.read(out_i).view(np.uint16))
    assert np.array_equal(outs[True][0], outs[False][0])
    assert np.array_equal(outs[True][1], outs[False][1])
    assert not np.array_equal(outs[True][1], xi)
    graph.release(mark)


@pytest.mark.parametrize("shape", ["small", "full"])
def test_streamed_weights_give_the_resident_result(graph, shape):
    """Three blocks whose weights stream through two device slots from pinned host memory equal the same blocks
    run from resident copies of their weights, bit for bit: at hidden 256 with 48 tokens, and at the benchmarked
    shape (512 text + 4096 image tokens, hidden 3072, 226.7 MB of weights per block), where the copy of block
    i + 1 runs on the copy stream while block i computes."""
    if shape == "small":
        cfg, tt, rows, cols = B.BlockConfig(256, 512, 2, 2, 128, 1e-6), 16, 4, 8
    else:
        cfg, tt, rows, cols = B.DIT_DOUBLE_BLOCK, 512, 64, 64
    ti, H = rows * cols, cfg.hidden
    rng = np.random.default_rng(6)
    tvec = graph.buffer(rng.uniform(-.2, .2, 6 * H).astype(np.float32))
    rope = B.rope_for_image(graph, rows, cols)
    blk = B.DoubleBlock(graph, cfg, tt, ti, we.BF16)
    x0t = graph.buffer(O.bf16_rne(rng.standard_normal(tt * H).astype(np.float32)))
    x0i = graph.buffer(O.bf16_rne(rng.standard_normal(ti * H).astype(np.float32)))
    hosts = [_layout_weights(graph, cfg, rng) for _ in range(3)]
    layout, scales = hosts[0][0], hosts[0][2]

    def chain(weights_of):
        xs = [(x0t, x0i)] + [(graph.buffer(tt * H * 2), graph.buffer(ti * H * 2)) for _ in range(3)]

        def compute(i, slot):
            w_t, w_i = layout.weights(slot, scales)
            blk.forward(w_t, w_i, xs[i][0], xs[i][1], tvec, rope, xs[i + 1][0], xs[i + 1][1])

        weights_of(compute)
        return np.concatenate([graph.read(xs[3][0]), graph.read(xs[3][1])])

    def resident(compute):
        for i, (_, host, _) in enumerate(hosts):
            slot = graph.buffer(host)
            compute(i, slot)
            graph.sync()
            graph.free(slot)

    pinned = []
    for _, host, _ in hosts:
        p = graph.host_alloc(layout.nbytes)
        graph.host_view(p, layout.nbytes)[:] = host
        pinned.append(p)
    streamer = B.BlockStreamer(graph, layout)
    try:
        want = chain(resident)
        got = chain(lambda compute: streamer.run(pinned, compute))
    finally:
        graph.sync()
        streamer.free()
        for p in pinned:
            graph.host_free(p)
    assert np.array_equal(got, want)


def test_blocks_streamed_from_a_file_give_the_resident_result(graph, tmp_path):
    """Two blocks written to one .safetensors file (prefixes double_blocks.0. / .1.), read by the native reader
    straight into pinned host memory and streamed through the device slots, equal the same blocks run from
    resident copies of the in-memory weights, bit for bit."""
    import weights as W
    cfg, tt, rows, cols = B.BlockConfig(256, 512, 2, 2, 128, 1e-6), 16, 4, 8
    ti, H = rows * cols, cfg.hidden
    rng = np.random.default_rng(8)
    tvec = graph.buffer(rng.uniform(-.2, .2, 6 * H).astype(np.float32))
    rope = B.rope_for_image(graph, rows, cols)
    blk = B.DoubleBlock(graph, cfg, tt, ti, we.BF16)
    x0t = graph.buffer(O.bf16_rne(rng.standard_normal(tt * H).astype(np.float32)))
    x0i = graph.buffer(O.bf16_rne(rng.standard_normal(ti * H).astype(np.float32)))
    hosts = [_layout_weights(graph, cfg, rng) for _ in range(2)]
    layout = hosts[0][0]
    tensors = {}
    for i, (_, host, scales) in enumerate(hosts):
        tensors.update(layout.file_tensors(host, scales, f"double_blocks.{i}."))
    W.save(tmp_path / "model.safetensors", tensors)

    def chain(weights_of):
        xs = [(x0t, x0i)] + [(graph.buffer(tt * H * 2), graph.buffer(ti * H * 2)) for _ in range(2)]

        def compute(i, slot, scales):
            w_t, w_i = layout.weights(slot, scales)
            blk.forward(w_t, w_i, xs[i][0], xs[i][1], tvec, rope, xs[i + 1][0], xs[i + 1][1])

        weights_of(compute)
        return np.concatenate([graph.read(xs[2][0]), graph.read(xs[2][1])])

    def resident(compute):
        for i, (_, host, scales) in enumerate(hosts):
            slot = graph.buffer(host)
            compute(i, slot, scales)
            graph.sync()
            graph.free(slot)

    pinned = [graph.host_alloc(layout.nbytes) for _ in hosts]
    streamer = B.BlockStreamer(graph, layout)
    try:
        with W.read_header(tmp_path / "model.safetensors") as st:
            file_scales = [layout.fill_from_file(st, f"double_blocks.{i}.", p) for i, p in enumerate(pinned)]
        want = chain(resident)
        got = chain(lambda compute: streamer.run(pinned, lambda i, slot: compute(i, slot, file_scales[i])))
    finally:
        graph.sync()
        streamer.free()
        for p in pinned:
            graph.host_free(p)
    assert np.array_equal(got, want)

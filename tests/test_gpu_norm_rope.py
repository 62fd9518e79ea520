"""RMSNorm, RoPE and the fused per-head norm + RoPE on the GPU against the float64 oracle.
Mirrors tests/gpu/rmsnorm.test.ts:25-53 and tests/gpu/rope.test.ts:5-42 (tolerances 1e-5 / 1e-6 abs
for f32; bf16 storage adds one bf16 rounding, 2^-8 of the value)."""
import numpy as np
import pytest

import oracle_lib as O
import we

pytestmark = pytest.mark.gpu


def lcg_centered(seed, n, size):
    """rng(seed) of tests/gpu/rmsnorm.test.ts:5-8: (lcg - 0.5) * size, as f32."""
    return ((O.lcg(seed, n) - 0.5) * size).astype(np.float32)


def test_rmsnorm_krea_rows_with_modulation(graph):  # tests/gpu/rmsnorm.test.ts:25-31
    d = 6144
    u = O.lcg(1, 3 * d + 3 * d)
    x = ((u[: 3 * d] - 0.5) * 8).astype(np.float32)
    w = ((u[3 * d: 4 * d] - 0.5) * 0.2).astype(np.float32)
    sc = ((u[4 * d: 5 * d] - 0.5) * 2).astype(np.float32)
    sh = ((u[5 * d:] - 0.5) * 2).astype(np.float32)
    out = we.norm(graph, graph.buffer(x), graph.buffer(w), 3, d, we.Mod(graph.buffer(sc), graph.buffer(sh)))
    got = graph.read(out, dtype=np.float32, count=3 * d)
    assert np.abs(got - O.rmsnorm(x, w, 1e-5, 1.0, sc, sh)).max() < 1e-5


def test_rmsnorm_per_head_plain(graph):  # tests/gpu/rmsnorm.test.ts:33-40
    d = 128
    u = O.lcg(2, 101 * d)
    x = ((u[: 100 * d] - 0.5) * 2).astype(np.float32)
    w = ((u[100 * d:] - 0.5) * 2).astype(np.float32)
    out = we.norm(graph, graph.buffer(x), graph.buffer(w), 100, d, we.no_mod(graph, d), offset=0.0)
    got = graph.read(out, dtype=np.float32, count=100 * d)
    assert np.abs(got - O.rmsnorm(x, w, 1e-5, 0.0)).max() < 1e-5


def test_rmsnorm_short_odd_rows(graph):  # tests/gpu/rmsnorm.test.ts:42-48
    u = O.lcg(3, 6 * 37)
    x = ((u[: 5 * 37] - 0.5) * 2).astype(np.float32)
    w = ((u[5 * 37:] - 0.5) * 2).astype(np.float32)
    out = we.norm(graph, graph.buffer(x), graph.buffer(w), 5, 37, None)
    got = graph.read(out, dtype=np.float32, count=5 * 37)
    assert np.abs(got - O.rmsnorm(x, w, 1e-5, 1.0)).max() < 1e-5


@pytest.mark.parametrize("rows,d", [(4608, 3072), (110592 // 8, 128), (7, 2000)])
def test_rmsnorm_bf16_storage(graph, rows, d):
    rng = np.random.default_rng(d)
    x = O.bf16_rne(rng.standard_normal(rows * d).astype(np.float32) * 3)
    w = rng.uniform(-0.2, 0.2, d).astype(np.float32)
    out = we.norm(graph, graph.buffer(x), graph.buffer(w), rows, d, None, eps=1e-6, dtype=we.BF16)
    got = O.bf16_to_f32(graph.read(out, dtype=np.uint16, count=rows * d)).astype(np.float64)
    want = O.rmsnorm(O.bf16_to_f32(x), w, 1e-6, 1.0)
    assert np.all(np.abs(got - want) <= 2 ** -8 * np.abs(want) + 1e-6)


@pytest.mark.parametrize("dtype,d", [(we.BF16, 3072), (we.F16, 2048), (we.BF16, 4096), (we.F16, 4104), (we.BF16, 6144)])
def test_rmsnorm_16bit_modulated_rows(graph, dtype, d):
    """The double-stream block's modulated norm on 16-bit rows (one wave per row, 16-byte accesses): weight,
    scale and shift per column, against the f64 oracle at one rounding of the output type. d <= 4096 stages the
    per-column factors in LDS; 4104 and 6144 take the kernel that loads them per row."""
    rows = 37
    rng = np.random.default_rng(d + dtype)
    x32 = rng.standard_normal(rows * d).astype(np.float32) * 3
    w = rng.uniform(-0.2, 0.2, d).astype(np.float32)
    sc = rng.uniform(-1, 1, d).astype(np.float32)
    sh = rng.uniform(-1, 1, d).astype(np.float32)
    if dtype == we.BF16:
        x = O.bf16_rne(x32)
        xv = O.bf16_to_f32(x)
    else:
        x = x32.astype(np.float16).view(np.uint16)
        xv = x32.astype(np.float16).astype(np.float32)
    out = we.norm(graph, graph.buffer(x), graph.buffer(w), rows, d, we.Mod(graph.buffer(sc), graph.buffer(sh)),
                  eps=1e-6, dtype=dtype)
    raw = graph.read(out, dtype=np.uint16, count=rows * d)
    got = (O.bf16_to_f32(raw) if dtype == we.BF16 else raw.view(np.float16).astype(np.float32)).astype(np.float64)
    want = O.rmsnorm(xv, w, 1e-6, 1.0, sc, sh)
    ulp = 2 ** -8 if dtype == we.BF16 else 2 ** -11
    assert np.all(np.abs(got - want) <= ulp * np.abs(want) + 1e-5)


def test_rope_interleaved_three_axes(graph):  # tests/gpu/rope.test.ts:5-22
    heads = 3
    pos = O.rope_positions(2, 3, 4, 3)
    cos, sin, pairs = O.rope_tables(pos, [32, 48, 48], 1000.0)
    tokens = pos.shape[0]
    x = (O.lcg(1, tokens * heads * 128) * 2 - 1).astype(np.float32)
    r = we.Rope(graph.buffer(cos), graph.buffer(sin), pairs, tokens)
    got = graph.read(we.rotate(graph, graph.buffer(x), heads, r), dtype=np.float32, count=x.size)
    want = O.rope_rotate(x, tokens, heads, pairs, cos, sin)
    assert np.abs(got - want).max() < 1e-6
    assert np.array_equal(got[: 2 * heads * 128], x[: 2 * heads * 128])  # text tokens unchanged


def test_rope_half_pairs(graph):  # tests/gpu/rope.test.ts:24-42
    heads = 2
    pos = np.array([[0.0], [1.0], [5.0], [40.0]])
    cos, sin, pairs = O.rope_tables(pos, [128], 5e6)
    x = (O.lcg(7, 4 * heads * 128) * 2 - 1).astype(np.float32)
    r = we.Rope(graph.buffer(cos), graph.buffer(sin), pairs, 4)
    got = graph.read(we.rotate(graph, graph.buffer(x), heads, r, "half"), dtype=np.float32, count=x.size)
    want = O.rope_rotate(x, 4, heads, pairs, cos, sin, half=True)
    assert np.abs(got - want).max() < 1e-5


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("dtype", [we.F32, we.BF16, we.F16])
def test_fused_qk_norm_rope(graph, half, dtype):
    """RMSNorm per head (offset 1, eps 1e-6) then 2D-axial RoPE (theta 10000) on the image tokens only,
    as the q/k path of attend() (src/model/block.ts:53-56) composes it."""
    text, rows, cols, heads, hd = 8, 6, 10, 4, 128
    tokens = text + rows * cols
    pos = O.rope_positions(0, rows, cols, 2)
    cos, sin, pairs = O.rope_tables(pos, [64, 64], 10000.0)
    rng = np.random.default_rng(3)
    x32 = rng.standard_normal(tokens * heads * hd).astype(np.float32) * 2
    w = rng.uniform(-0.3, 0.3, hd).astype(np.float32)
    if dtype == we.F32:
        x, xs = x32, x32
    elif dtype == we.BF16:
        x = O.bf16_rne(x32)
        xs = O.bf16_to_f32(x)
    else:
        x = x32.astype(np.float16).view(np.uint16)
        xs = x32.astype(np.float16).astype(np.float32)
    out = graph.buffer(x.nbytes)
    graph.qk_norm_rope(tokens, heads, hd, 1e-6, 1.0, graph.buffer(w), text, half, graph.buffer(cos),
                       graph.buffer(sin), dtype, graph.buffer(x), out)
    raw = graph.read(out)
    if dtype == we.F32:
        got = raw.view(np.float32).astype(np.float64)
    elif dtype == we.BF16:
        got = O.bf16_to_f32(raw.view(np.uint16)).astype(np.float64)
    else:
        got = raw.view(np.float16).astype(np.float64)
    normed = O.rmsnorm(xs, w, 1e-6, 1.0).astype(np.float32)  # [tokens * heads, hd]
    img = normed.reshape(tokens, heads * hd)[text:].ravel()
    rot = O.rope_rotate(img, rows * cols, heads, pairs, cos, sin, half=half)
    want = np.concatenate([normed.reshape(tokens, heads * hd)[:text].ravel().astype(np.float64), rot])
    tol = {we.F32: 2e-5, we.BF16: 2 ** -8, we.F16: 2 ** -10}[dtype]
    assert np.all(np.abs(got - want) <= tol * np.maximum(np.abs(want), 1.0))


@pytest.mark.parametrize("hd", [64, 128])
def test_fused_qk_norm_rope_strided_in_place(graph, hd):
    """q/k normalized and rotated in place inside a fused [tokens, 3 * heads * head_dim] QKV row: the k slice
    equals the dense result, the q and v slices are untouched."""
    text, rows, cols, heads = 4, 3, 5, 2
    tokens, row = text + rows * cols, heads * hd
    pos = O.rope_positions(0, rows, cols, 2)
    cos, sin, pairs = O.rope_tables(pos, [hd // 2, hd // 2], 10000.0)
    rng = np.random.default_rng(8)
    qkv = O.bf16_rne(rng.standard_normal(tokens * 3 * row).astype(np.float32))
    w = rng.uniform(-0.3, 0.3, hd).astype(np.float32)
    kpart = np.ascontiguousarray(qkv.reshape(tokens, 3, row)[:, 1])
    wb, cb, sb = graph.buffer(w), graph.buffer(cos), graph.buffer(sin)
    dense = graph.buffer(kpart.nbytes)
    graph.qk_norm_rope(tokens, heads, hd, 1e-6, 1.0, wb, text, False, cb, sb, we.BF16, graph.buffer(kpart), dense)
    buf = graph.buffer(qkv)
    kslice = we.Graph.slice(buf, row * 2, 0)
    graph.qk_norm_rope(tokens, heads, hd, 1e-6, 1.0, wb, text, False, cb, sb, we.BF16, kslice, kslice,
                       x_stride=3 * row, out_stride=3 * row)
    got = graph.read(buf).view(np.uint16).reshape(tokens, 3, row)
    assert np.array_equal(got[:, 1], graph.read(dense).view(np.uint16).reshape(tokens, row))
    assert np.array_equal(got[:, 0], qkv.reshape(tokens, 3, row)[:, 0])
    assert np.array_equal(got[:, 2], qkv.reshape(tokens, 3, row)[:, 2])


@pytest.mark.parametrize("dtype,rows,d", [(we.F32, 7, 640), (we.F32, 5, 3072), (we.BF16, 300, 3072),
                                          (we.F16, 9, 1000), (we.BF16, 4096, 3072)])
def test_rmsnorm_mod_equals_the_add_then_the_norm(graph, dtype, rows, d):
    """we_rmsnorm_mod (src/model/block.ts:33-37 folded into norm1, :96) writes mod = tvec + table and the
    modulated norm; both equal, bit for bit, the separate add pass followed by we_rmsnorm on mod's first two
    parts (every norm kernel: one wave per row, one block per row, the 16-bit vector kernel)."""
    rng = np.random.default_rng(rows + d)
    x = rng.standard_normal(rows * d).astype(np.float32)
    if dtype == we.BF16:
        x = O.bf16_rne(x)
    elif dtype == we.F16:
        x = x.astype(np.float16)
    w = rng.uniform(-.3, .3, d).astype(np.float32)
    tvec = rng.uniform(-1, 1, 6 * d).astype(np.float32)
    table = rng.uniform(-1, 1, 6 * d).astype(np.float32)
    mark = graph.mark()
    xb, wb, tb, tab = graph.buffer(x), graph.buffer(w), graph.buffer(tvec), graph.buffer(table)
    esz = we.ELEM_BYTES[dtype]
    mod_f, out_f = graph.buffer(6 * d * 4), graph.buffer(rows * d * esz)
    graph.rmsnorm_mod(rows, d, 1e-6, 1.0, dtype, xb, wb, tb, tab, 6 * d, mod_f, out_f)
    mod_s, out_s = graph.buffer(6 * d * 4), graph.buffer(rows * d * esz)
    graph.elementwise(we.OP_ADD, 6 * d, 1, we.F32, tb, tab, None, mod_s)
    graph.rmsnorm(rows, d, 1e-6, 1.0, dtype, xb, wb, we.Graph.slice(mod_s, 0, d * 4), we.Graph.slice(mod_s, d * 4, d * 4),
                  out_s)
    got = [graph.read(b) for b in (mod_f, out_f, mod_s, out_s)]
    graph.release(mark)
    assert np.array_equal(got[0], got[2]) and np.array_equal(got[1], got[3])
    assert np.array_equal(got[0].view(np.float32), tvec + table)


def test_rmsnorm_mod_refuses_overlap_and_short_mod(graph):
    d = 64
    mark = graph.mark()
    x, w, t = graph.buffer(d * 4), graph.buffer(d * 4), graph.buffer(6 * d * 4)
    mod, out = graph.buffer(6 * d * 4), graph.buffer(d * 4)
    with pytest.raises(we.WeError, match="may not overlap"):
        graph.rmsnorm_mod(1, d, 1e-6, 1.0, we.F32, x, w, t, t, 6 * d, t, out)
    with pytest.raises(we.WeError, match="less than 2 d"):
        graph.rmsnorm_mod(1, d, 1e-6, 1.0, we.F32, x, w, t, t, d, mod, out)
    with pytest.raises(we.WeError, match="must be positive"):
        graph.rmsnorm_mod(0, d, 1e-6, 1.0, we.F32, x, w, t, t, 6 * d, mod, out)
    graph.release(mark)

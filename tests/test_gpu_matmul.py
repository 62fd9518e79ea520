"""GEMM parity on the GPU through the C-ABI, against the float64 oracle.
Mirrors tests/gpu/matmul.test.ts (shapes, LCG inputs, error definition) and adds the dtype matrix,
every tile configuration, the fused epilogues and full-size shapes (sampled rows + exact properties).

Tolerances (max|y - ref| / max|ref|, tests/gpu/matmul.test.ts:38-46):
  * f32 / f16 / bf16 inputs with an f32 output: 1e-5, the reference's own bar (f32 operands are split
    into three bf16 terms, exact; every other operand is exact in the MFMA type; only the f32
    accumulation rounds);
  * f16 output: 2e-3 (one f16 rounding is 2^-11 of the value);  bf16 output: 1e-2 (2^-8 of the value).
"""
import ctypes

import numpy as np
import pytest

import oracle_lib as O
import we

pytestmark = pytest.mark.gpu
TOL_F32_OUT = 1e-5
TOL = {we.F32: TOL_F32_OUT, we.F16: 2e-3, we.BF16: 1e-2}


def decode(arr, dt):
    if dt == we.F32:
        return arr.view(np.float32).astype(np.float64)
    if dt == we.F16:
        return arr.view(np.float16).astype(np.float64)
    return O.bf16_to_f32(arr.view(np.uint16)).astype(np.float64)


def encode_act(x32, dt):
    """f32 values -> storage for dtype dt, and the exact values the kernel sees (for the oracle)."""
    if dt == we.F32:
        return x32.astype(np.float32), x32.astype(np.float32), O.F32
    if dt == we.F16:
        h = x32.astype(np.float16)
        return h, h.view(np.uint16), O.F16
    b = O.bf16_rne(x32)
    return b, b, O.BF16


def run(graph, p, x, x_dt, w, w_dt, y_dt=we.F32, flags=0, bias=None, y_init=None, rows=None):
    rows = rows if rows is not None else p.m * (p.k_split if flags & we.EPI_SPLIT_K else 1)
    ylen = (rows - 1) * p.y_stride + p.n + p.y_offset
    esz = we.ELEM_BYTES[y_dt]
    mark = graph.mark()
    xb, wb = graph.buffer(x), graph.buffer(w)
    yb = graph.buffer(y_init) if y_init is not None else graph.buffer(ylen * esz)
    bb = graph.buffer(np.asarray(bias, np.float32)) if bias is not None else None
    graph.matmul(p, x_dt, xb, w_dt, wb, y_dt, yb, bias=bb, flags=flags)
    out = graph.read(yb, nbytes=ylen * esz)
    graph.release(mark)
    return decode(out, y_dt)


REF_SHAPES = [(1, 1, 4), (37, 70, 100), (64, 64, 64), (130, 65, 36), (200, 260, 84)]


@pytest.mark.parametrize("m,n,k", REF_SHAPES)
def test_fp8_matches_reference_test_shapes(graph, m, n, k):  # tests/gpu/matmul.test.ts:49-59
    x, w = O.matmul_test_data(m, n, k, 1)
    got = we.matmul_fp8(graph, x, w, 0.002, m, n, k)
    want = O.matmul(O.matmul_params(m, n, k, 0.002), O.F32, x, O.FP8, w)
    assert O.rel_error(got.astype(np.float64), want) < TOL_F32_OUT


def test_fp8_krea_layer_shape(graph):  # tests/gpu/matmul.test.ts:61-66
    m, n, k, s = 8, 1536, 6144, 0.0018833705689758062
    x, w = O.matmul_test_data(m, n, k, 7)
    got = we.matmul_fp8(graph, x, w, s, m, n, k)
    want = O.matmul(O.matmul_params(m, n, k, s), O.F32, x, O.FP8, w)
    assert O.rel_error(got.astype(np.float64), want) < TOL_F32_OUT


def test_refuses_bad_params_and_short_buffers(graph):  # tests/gpu/matmul.test.ts:68-72
    p = we.MatmulParams(1, 1, 6, 1.0, 6, 6, 1, 0, 0, 0, 0, 0, 1)
    x, w, y = graph.buffer(64), graph.buffer(64), graph.buffer(64)
    with pytest.raises(we.WeError, match="K must be a multiple of 4, got 6"):
        graph.matmul(p, we.F32, x, we.FP8, w, we.F32, y)
    p = we.matmul_params(4, 4, 8, 1.0)
    with pytest.raises(we.WeError, match="y is too small"):
        graph.matmul(p, we.F32, graph.buffer(4 * 8 * 4), we.FP8, graph.buffer(32), we.F32, graph.buffer(8))
    with pytest.raises(we.WeError, match="not a buffer of this context"):
        graph.matmul(p, we.F32, we.Buffer(16, 128), we.FP8, w, we.F32, y)


def test_f32_head_pick_with_strides_and_offsets(graph):  # tests/gpu/matmul.test.ts:93-109
    tokens, heads, kv, dim = 20, 4, 2, 128
    u = O.lcg(3, tokens * heads * dim)
    q = (u * 2 - 1).astype(np.float32)
    kk = (O.lcg(4, tokens * kv * dim) * 2 - 1).astype(np.float32)
    h, g = 2, 1
    got = we.matmul_f32(graph, q, kk, 1.0, tokens, tokens, dim, output_length=tokens * 24, x_stride=heads * dim,
                        x_offset=h * dim, w_stride=kv * dim, w_offset=g * dim, y_stride=24).reshape(tokens, 24)
    want = q.reshape(tokens, heads, dim)[:, h].astype(np.float64) @ kk.reshape(tokens, kv, dim)[:, g].astype(
        np.float64).T
    assert np.abs(got[:, :tokens] - want).max() < 1e-4


@pytest.mark.parametrize("m,n,k", [(37, 70, 100), (8, 1536, 6144)])
def test_bf16_weights(graph, m, n, k):  # tests/gpu/matmul.test.ts:112-127
    u = O.lcg(9, m * k + n * k)
    x = (u[: m * k] * 2 - 1).astype(np.float32)
    wf = (u[m * k:] * 2 - 1).astype(np.float32)
    wb = (wf.view(np.uint32) >> 16).astype(np.uint16)
    got = we.matmul_bf16(graph, x, wb, 0.5, m, n, k)
    want = O.matmul(O.matmul_params(m, n, k, 0.5), O.F32, x, O.BF16, wb)
    assert O.rel_error(got.astype(np.float64), want) < TOL_F32_OUT


def test_split_k_partials(graph):  # tests/gpu/matmul.test.ts:131-149
    m, n, k, split, scale = 5, 12, 200, 3, 0.5
    x, w = O.matmul_test_data(m, n, k, 3)
    p = we.matmul_params(m, n, k, scale, k_split=split, graph=graph)
    parts = run(graph, p, x, we.F32, w, we.FP8, flags=we.EPI_SPLIT_K).reshape(split, m * n)
    op = O.matmul_params(m, n, k, scale, k_split=split)
    want_parts = O.matmul(op, O.F32, x, O.FP8, w, split=True).reshape(split, m * n)
    want = O.matmul(O.matmul_params(m, n, k, scale), O.F32, x, O.FP8, w)
    assert np.abs(parts - want_parts).max() < 1e-5 * np.abs(want).max()
    assert np.abs(parts.sum(0) - want).max() < 5e-4  # toBeCloseTo(want, 3)
    assert abs(parts[0, 0] - want[0]) > 1e-3


def test_accumulate_adds_exactly(graph):  # tests/gpu/matmul.test.ts:159-175
    m, n, k, scale = 3, 6, 8, 0.25
    x = (np.arange(m * k) % 5 - 2).astype(np.float32)
    w = ((np.arange(n * k) * 3) % 7 - 3).astype(np.float32)
    start = np.arange(m * n, dtype=np.float32)
    p = we.matmul_params(m, n, k, scale, graph=graph)
    plain = run(graph, p, x, we.F32, w, we.F32)
    got = run(graph, p, x, we.F32, w, we.F32, flags=we.EPI_ACCUMULATE, y_init=start)
    assert np.array_equal(got.astype(np.float32), (plain.astype(np.float32) + start))


W_KINDS = [we.FP8, we.BF16, we.F16, we.F32]


def make_weights(rng, n, k, w_dt):
    if w_dt == we.FP8:
        b = rng.integers(0, 256, n * k).astype(np.uint8)
        b[(b & 0x7F) == 0x7F] -= 1
        return b, b, O.FP8
    vals = rng.normal(0, 0.05, n * k).astype(np.float32)
    if w_dt == we.BF16:
        h = O.bf16_rne(vals)
        return h, h, O.BF16
    if w_dt == we.F16:
        h = vals.astype(np.float16).view(np.uint16)
        return h, h, O.F16
    return vals, vals, O.F32


@pytest.mark.parametrize("x_dt", [we.F32, we.F16, we.BF16])
@pytest.mark.parametrize("w_dt", W_KINDS)
@pytest.mark.parametrize("y_dt", [we.F32, we.BF16, we.F16])
def test_dtype_matrix(graph, x_dt, w_dt, y_dt):
    m, n, k = 130, 200, 320
    rng = np.random.default_rng(x_dt * 100 + w_dt * 10 + y_dt)
    x_store, x_oracle, ox = encode_act(rng.standard_normal(m * k).astype(np.float32), x_dt)
    w_store, w_oracle, ow = make_weights(rng, n, k, w_dt)
    scale = 0.02 if w_dt == we.FP8 else 1.0
    p = we.matmul_params(m, n, k, scale, graph=graph)
    got = run(graph, p, x_store, x_dt, w_store, w_dt, y_dt)
    want = O.matmul(O.matmul_params(m, n, k, scale), ox, x_oracle, ow, w_oracle)
    err = O.rel_error(got, want)
    assert err < TOL[y_dt], err


@pytest.mark.parametrize("path", ["fast", "generic"])
@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("x_dt,w_dt", [(we.BF16, we.FP8), (we.BF16, we.BF16), (we.F16, we.FP8), (we.F16, we.F16)])
def test_every_tile_config_with_ragged_edges(graph, cfg, x_dt, w_dt, path):
    """Both kernels (the straight-line fast path and the general one) in every tile shape, with partial
    tiles in M and N and a partial last K block (K = 208 = 3 * 64 + 16)."""
    m, n, k = 300, 520, 208
    rng = np.random.default_rng(cfg)
    x_store, x_oracle, ox = encode_act(rng.standard_normal(m * k).astype(np.float32), x_dt)
    w_store, w_oracle, ow = make_weights(rng, n, k, w_dt)
    p = we.matmul_params(m, n, k, 0.5, graph=graph)
    with graph.tuned(gemm_cfg=cfg, gemm_generic=int(path == "generic")):
        got = run(graph, p, x_store, x_dt, w_store, w_dt, we.F32)
    want = O.matmul(O.matmul_params(m, n, k, 0.5), ox, x_oracle, ow, w_oracle)
    assert O.rel_error(got, want) < TOL_F32_OUT


def test_unaligned_offsets_and_strides(graph):
    # multiples of 4 (the reference's only rule) but not of 16 bytes: the element-wise loader path
    m, n, k = 33, 47, 68
    rng = np.random.default_rng(5)
    xs, ws, ys = k + 4, k + 12, n + 3
    x = rng.standard_normal(4 + m * xs).astype(np.float32)
    w = rng.integers(0, 256, 4 + n * ws).astype(np.uint8)
    w[(w & 0x7F) == 0x7F] -= 1
    p = we.matmul_params(m, n, k, 0.1, x_stride=xs, w_stride=ws, y_stride=ys, x_offset=4, w_offset=4, y_offset=2,
                         graph=graph)
    got = run(graph, p, x, we.F32, w, we.FP8)
    op = O.matmul_params(m, n, k, 0.1, x_stride=xs, w_stride=ws, y_stride=ys, x_offset=4, w_offset=4, y_offset=2)
    want = O.matmul(op, O.F32, x, O.FP8, w, out_len=got.size)
    assert O.rel_error(got, want) < TOL_F32_OUT


def test_bias_and_gelu_epilogue(graph):  # src/model/ops.ts:65 + src/kernels/elementwise.ts:25-29, fused
    m, n, k = 96, 160, 256
    rng = np.random.default_rng(7)
    x_store, x_oracle, ox = encode_act(rng.standard_normal(m * k).astype(np.float32), we.BF16)
    w = rng.integers(0, 256, n * k).astype(np.uint8)
    w[(w & 0x7F) == 0x7F] -= 1
    bias = rng.normal(0, 1, n).astype(np.float32)
    p = we.matmul_params(m, n, k, 0.02, graph=graph)
    got = run(graph, p, x_store, we.BF16, w, we.FP8, we.F32, flags=we.EPI_BIAS | we.EPI_GELU, bias=bias)
    lin = O.matmul(O.matmul_params(m, n, k, 0.02), ox, x_oracle, O.FP8, w) + np.tile(bias.astype(np.float64), m)
    want = np.array([O.lib.or_gelu_tanh(v) for v in lin])
    assert np.abs(got - want).max() < 1e-4 * np.abs(want).max()


def test_scale_is_linear_exactly(graph):
    m, n, k = 64, 128, 192
    rng = np.random.default_rng(11)
    x = O.bf16_rne(rng.standard_normal(m * k).astype(np.float32))
    w = rng.integers(0, 0x7E, n * k).astype(np.uint8)
    a = run(graph, we.matmul_params(m, n, k, 0.25, graph=graph), x, we.BF16, w, we.FP8, we.F32)
    b = run(graph, we.matmul_params(m, n, k, 0.5, graph=graph), x, we.BF16, w, we.FP8, we.F32)
    assert np.array_equal(2 * a, b)


def test_nan_codes_decode_like_the_shader(graph):
    # the reference shader has no NaN branch: 0x7f / 0xff weigh +-480 (src/kernels/fp8.ts:12-20)
    m, n, k = 4, 8, 64
    x = np.ones(m * k, np.float32)
    w = np.full(n * k, 0x38, np.uint8)  # 1.0
    w[0] = 0x7F
    w[k + 5] = 0xFF
    got = run(graph, we.matmul_params(m, n, k, 1.0, graph=graph), x, we.F32, w, we.FP8).reshape(m, n)
    assert got[0, 0] == 63 + 480 and got[0, 1] == 63 - 480 and got[0, 2] == 64


@pytest.mark.parametrize("y_dt", [we.BF16, we.F32, we.F16])
@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("cfg", [None, 0])
def test_fast_epilogue_gelu_without_bias(graph, tune, y_dt, gated, cfg):
    """The fast kernel's whole-sub-tile epilogue with GELU and no bias: the up-projection as benchmarked (256 x 256
    ping-pong tiles, bf16 out) and the gated form, against the oracle product followed by or_gelu_tanh (and the
    reference's gatedAdd). 512 x 768 outputs are 2 x 3 whole 256 x 256 tiles; cfg None takes the default pick."""
    m, n, k = 512, 768, 512
    rng = np.random.default_rng(31 + y_dt + 3 * gated)
    x_store, x_oracle, ox = encode_act(rng.standard_normal(m * k).astype(np.float32), we.BF16)
    w = rng.integers(0, 254, n * k).astype(np.uint8)
    w = (w + (w >= 0x7F)).astype(np.uint8)
    gate = rng.uniform(-1.5, 1.5, n).astype(np.float32) if gated else None
    res_store, res_vals = _store(rng.standard_normal(m * n), y_dt) if gated else (None, None)
    if cfg is not None:
        tune(gemm_cfg=cfg)
    p = we.matmul_params(m, n, k, 0.02, graph=graph)
    mark = graph.mark()
    yb = graph.buffer(m * n * we.ELEM_BYTES[y_dt])
    graph.matmul(p, we.BF16, graph.buffer(x_store), we.FP8, graph.buffer(w), y_dt, yb, flags=we.EPI_GELU,
                 gate=graph.buffer(gate) if gated else None, residual=graph.buffer(res_store) if gated else None)
    got = decode(graph.read(yb), y_dt)
    graph.release(mark)
    v = O.gelu_tanh(O.matmul(O.matmul_params(m, n, k, 0.02), ox, x_oracle, O.FP8, w))
    want = (res_vals + np.tile(gate.astype(np.float64), m) * v) if gated else v
    tol = 1e-4 if y_dt == we.F32 else TOL[y_dt]
    assert O.rel_error(got, want) < tol


@pytest.mark.parametrize("name,m,n,k,w_dt,flags", [("C3 up", 4096, 12288, 3072, we.FP8, we.EPI_GELU),
                                                   ("C3 down", 4096, 3072, 12288, we.FP8, 0),
                                                   ("C2 qkv", 4096, 9216, 3072, we.BF16, 0)])
def test_full_size_sampled_rows(graph, name, m, n, k, w_dt, flags):
    """Full-size GEMMs: every output is computed, 6 whole rows (incl. the first and last) are checked
    against the f64 oracle, and the row sums of y equal x @ rowsum(W) (a checksum over all outputs).
    Then the GEMM exactly as bench.py runs it (bf16 output, default tile pick; the up-projection with GELU
    fused and no bias): its sampled rows against the oracle (+ GELU) at the bf16 bar, and every one of its
    outputs against the f32-output run above passed through GELU in float64 and rounded to bf16. Both runs take
    the same tile pick and the same accumulation order, so they agree to the rounding of the output: exactly
    without GELU, within one bf16 step with it."""
    rng = np.random.default_rng(m + n + k)
    x = O.bf16_rne(rng.standard_normal(m * k).astype(np.float32))
    if w_dt == we.FP8:
        w = rng.integers(0, 256, n * k, dtype=np.uint8)
        w[(w & 0x7F) == 0x7F] -= 1
        ow = O.FP8
    else:
        w = O.bf16_rne(rng.normal(0, 0.02, n * k).astype(np.float32))
        ow = O.BF16
    scale = 0.02 if w_dt == we.FP8 else 1.0
    p = we.matmul_params(m, n, k, scale, graph=graph)
    got = run(graph, p, x, we.BF16, w, w_dt, we.F32).reshape(m, n)
    op = O.matmul_params(m, n, k, scale)
    rows = [0, 1, 777, 2049, m - 2, m - 1]
    for r in rows:
        want = O.matmul_rows(op, O.BF16, x, ow, w, r, r + 1).reshape(m, n)[r]
        assert O.rel_error(got[r], want) < TOL_F32_OUT, (name, r)
    # checksum of checksums: y @ 1 = x @ (W^T 1) * scale, for every row
    wdec = (O.e4m3_table()[w] if w_dt == we.FP8 else O.bf16_to_f32(w).astype(np.float64)).reshape(n, k)
    xs = O.bf16_to_f32(x).astype(np.float64).reshape(m, k)
    want_sum = xs @ wdec.sum(0) * scale
    assert np.abs(got.sum(1) - want_sum).max() < 1e-4 * np.abs(want_sum).max() + 1e-3
    # ---- the benchmarked variant: bf16 out (+ fused GELU for the up-projection)
    bench = run(graph, p, x, we.BF16, w, w_dt, we.BF16, flags=flags).reshape(m, n)
    gelu = (lambda v: O.gelu_tanh(v)) if flags & we.EPI_GELU else (lambda v: v)  # noqa: E731
    for r in rows:
        want = gelu(O.matmul_rows(op, O.BF16, x, ow, w, r, r + 1).reshape(m, n)[r])
        assert O.rel_error(bench[r], want) < TOL[we.BF16], (name, r)
    expect = O.bf16_to_f32(O.bf16_rne(gelu(got).astype(np.float32))).astype(np.float64)
    if flags & we.EPI_GELU:
        diff = np.abs(bench - expect)
        assert (diff <= 2.0 ** -7 * np.abs(expect) + 1e-30).all(), (name, float(diff.max()))
        # a one-step difference only where GELU's last f32 bits meet a rounding tie (outputs that underflow
        # f32 aside)
        assert ((diff == 0) | (np.abs(expect) < 1e-30)).mean() > 0.99, name
    else:
        assert np.array_equal(bench, expect), name


# ------------------------------------------------------------------ LoRA through linear() (tests/gpu/lora.test.ts)

def rms_rel(got, want):
    """src/model/compare.ts:2-17 relativeError: sqrt(sum (a - b)^2 / sum b^2)."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.sqrt(((got - want) ** 2).sum() / (want ** 2).sum()))


class LcgDraws:
    """tests/gpu/lora.test.ts:12-21: one LCG stream; floats in [-1, 1) as f32, bf16 as the top half of such
    a float (truncated), fp8 bytes floor((r + 1) * 60) (no NaN codes)."""

    def __init__(self, seed, total):
        self.u, self.i = O.lcg(seed, total), 0

    def _take(self, n):
        u = self.u[self.i:self.i + n]
        self.i += n
        assert u.size == n
        return u

    def floats(self, n):
        return (self._take(n) * 2 - 1).astype(np.float32)

    def bf16(self, n):
        bits = (self.floats(n).view(np.uint32) >> 16).astype(np.uint16)
        return bits, O.bf16_to_f32(bits).astype(np.float64)

    def fp8(self, n):
        return np.floor(self._take(n) * 120).astype(np.uint8)


def lora_reference(x, w, w_scale, down, up, s, m, n, k, r):
    """tests/gpu/lora.test.ts:23-38 in float64."""
    x = x.astype(np.float64).reshape(m, k)
    t = x @ down.reshape(r, k).T
    return ((x @ w.reshape(n, k).T) * w_scale + s * (t @ up.reshape(n, r).T)).ravel()


def test_lora_on_fp8_linear_bf16_and_f32_weights(graph):  # tests/gpu/lora.test.ts:40-78
    m, n, k, r, s = 5, 12, 16, 4, 0.8 * 0.5
    d = LcgDraws(7, m * k + n * k + r * k + n * r)
    x, w = d.floats(m * k), d.fp8(n * k)
    (down_b, down_v), (up_b, up_v) = d.bf16(r * k), d.bf16(n * r)
    mark = graph.mark()
    base = we.Linear(graph.buffer(w), "fp8", 0.25, n, k)
    lora_bf = (we.Linear(graph.buffer(down_b), "bf16", 1.0, r, k), we.Linear(graph.buffer(up_b), "bf16", s, n, r))
    lora_f32 = (we.Linear(graph.buffer(down_v.astype(np.float32)), "f32", 1.0, r, k),
                we.Linear(graph.buffer(up_v.astype(np.float32)), "f32", s, n, r))
    want = lora_reference(x, O.e4m3_table()[w], 0.25, down_v, up_v, s, m, n, k, r)
    for lora in (lora_bf, lora_f32):
        lin = we.Linear(base.buffer, "fp8", 0.25, n, k, lora=lora)
        got = graph.read(we.linear(graph, graph.buffer(x), lin, m), dtype=np.float32, count=m * n)
        assert rms_rel(got, want) < 1e-6
    plain = graph.read(we.linear(graph, graph.buffer(x), base, m), dtype=np.float32, count=m * n)
    assert rms_rel(plain, want) > 1e-3  # the update is really there
    graph.release(mark)


@pytest.mark.parametrize("y_dt", [we.F32, we.BF16])
def test_lora_with_gelu_applies_gelu_to_the_sum(graph, y_dt):
    """linear(..., gelu_tanh=True) with LoRA returns gelu(x W^T s + bias + lora), as a caller of the reference
    applies GELU to what linear returns (src/model/ops.ts:61-73); the fused GELU stays off the base GEMM."""
    m, n, k, r, s = 6, 40, 64, 4, 0.6
    d = LcgDraws(13, m * k + n * k + r * k + n * r + n)
    x, w = d.floats(m * k), d.fp8(n * k)
    (down_b, down_v), (up_b, up_v) = d.bf16(r * k), d.bf16(n * r)
    bias = d.floats(n)
    mark = graph.mark()
    lora = (we.Linear(graph.buffer(down_b), "bf16", 1.0, r, k), we.Linear(graph.buffer(up_b), "bf16", s, n, r))
    lin = we.Linear(graph.buffer(w), "fp8", 0.25, n, k, bias=graph.buffer(bias), lora=lora)
    got = decode(graph.read(we.linear(graph, graph.buffer(x), lin, m, y_dtype=y_dt, gelu_tanh=True)), y_dt)
    graph.release(mark)
    lin_sum = lora_reference(x, O.e4m3_table()[w], 0.25, down_v, up_v, s, m, n, k, r) + np.tile(bias, m)
    want = O.gelu_tanh(lin_sum)
    assert rms_rel(got, want) < (1e-6 if y_dt == we.F32 else 1e-2)
    wrong = O.gelu_tanh(lin_sum - lora_reference(x, O.e4m3_table()[w] * 0, 0.0, down_v, up_v, s, m, n, k, r)) + \
        lora_reference(x, O.e4m3_table()[w] * 0, 0.0, down_v, up_v, s, m, n, k, r)
    assert rms_rel(wrong, want) > 1e-3  # the order matters for these inputs


def test_lora_rank_not_multiple_of_4_is_rejected(graph):  # tests/gpu/lora.test.ts:80-89
    mark = graph.mark()
    lin = lambda n, k, scale=1.0: we.Linear(graph.buffer(n * k * 4), "f32", scale, n, k)  # noqa: E731
    w = lin(8, 8)
    w.lora = (lin(3, 8), lin(8, 3))
    with pytest.raises(we.WeError, match="LoRA shapes do not fit the linear layer"):
        we.linear(graph, graph.buffer(8 * 4), w, 1)
    graph.release(mark)


def test_lora_down_split_over_long_k(graph):  # tests/gpu/lora.test.ts:120-146
    m, n, k, r, s = 5, 8, 1024, 4, 0.3
    assert we.k_split_for(m, r, k) == 4
    d = LcgDraws(11, m * k + n * k + r * k + n * r)
    x = d.floats(m * k)
    (w_b, w_v), (down_b, down_v), (up_b, up_v) = d.bf16(n * k), d.bf16(r * k), d.bf16(n * r)
    mark = graph.mark()
    lora = (we.Linear(graph.buffer(down_b), "bf16", 1.0, r, k), we.Linear(graph.buffer(up_b), "bf16", s, n, r))
    lin = we.Linear(graph.buffer(w_b), "bf16", 1.0, n, k, lora=lora)
    got = graph.read(we.linear(graph, graph.buffer(x), lin, m), dtype=np.float32, count=m * n)
    assert rms_rel(got, lora_reference(x, w_v, 1.0, down_v, up_v, s, m, n, k, r)) < 1e-6
    graph.release(mark)


# ------------------------------------------------------------------ small M: K split over workgroups, reduced in-kernel

@pytest.mark.parametrize("m,n,k,x_dt,y_dt,flags", [
    (64, 3072, 3072, we.F16, we.F16, 0),                      # the single fp8 matmul at M = 64
    (37, 70, 1024, we.BF16, we.F32, we.EPI_BIAS | we.EPI_GELU),
    (1, 300, 2048, we.BF16, we.BF16, 0),
    (64, 1000, 4096, we.F16, we.F32, we.EPI_ACCUMULATE),
    (33, 129, 768, we.F16, we.F16, we.EPI_BIAS),
    (256, 384, 2048, we.BF16, we.F32, we.EPI_GELU), (256, 384, 2048, we.BF16, we.BF16, 0),
    (200, 1000, 1024, we.BF16, we.F32, we.EPI_BIAS)])
def test_small_m_split_k_reduction(graph, tune, m, n, k, x_dt, y_dt, flags):
    """fp8 GEMMs whose tiles fill few workgroup slots (small M; or M > 64 with few tiles, like the
    double-stream block's 512-token text projections) split K across workgroups and a reduce pass adds the
    slices. The result matches the oracle, repeats bit for bit (slices are summed in slice order), and
    matches the unsplit kernel within the same bar."""
    rng = np.random.default_rng(m * 7 + n + k)
    x_store, x_oracle, ox = encode_act(rng.standard_normal(m * k).astype(np.float32), x_dt)
    w = rng.integers(0, 254, n * k).astype(np.uint8)
    w = (w + (w >= 0x7F)).astype(np.uint8)
    bias = rng.normal(0, 1, n).astype(np.float32) if flags & we.EPI_BIAS else None
    start = rng.standard_normal(m * n).astype(np.float32) if flags & we.EPI_ACCUMULATE else None
    y_init = start if start is not None else None
    p = we.matmul_params(m, n, k, 0.02, graph=graph)
    runs = [run(graph, p, x_store, x_dt, w, we.FP8, y_dt, flags=flags, bias=bias, y_init=y_init) for _ in range(2)]
    assert np.array_equal(runs[0], runs[1])
    lin = O.matmul(O.matmul_params(m, n, k, 0.02), ox, x_oracle, O.FP8, w)
    if bias is not None:
        lin = lin + np.tile(bias.astype(np.float64), m)
    want = np.array([O.lib.or_gelu_tanh(v) for v in lin]) if flags & we.EPI_GELU else lin
    if start is not None:
        want = want + start
    tol = 1e-4 if flags & we.EPI_GELU else TOL[y_dt]
    assert O.rel_error(runs[0], want) < tol
    tune(gemm_splitk=0)
    unsplit = run(graph, p, x_store, x_dt, w, we.FP8, y_dt, flags=flags, bias=bias, y_init=y_init)
    assert O.rel_error(unsplit, want) < tol


# ---- gated residual epilogue (we_matmul_gated): gatedAdd (src/kernels/elementwise.ts:52-58) after the GEMM ----

def _store(vals, dt):
    """f64 values -> (storage of dtype dt, the exact values stored)"""
    s, exact, _ = encode_act(vals.astype(np.float32), dt)
    return s, decode(np.ascontiguousarray(s).view(np.uint8), dt)


@pytest.mark.parametrize("case", ["fast_full", "fast_ragged", "small_m_split", "generic_f32", "f16_out", "gelu_bias"])
def test_gated_residual_equals_gemm_then_gated_add(graph, case, tune):
    """y = residual + gate * v (v: scale, bias, GELU of the product), against the f64 oracle of the product followed
    by the reference's gatedAdd, on every epilogue: the fast kernel's whole-tile and per-value paths, the split-K
    reduce pass (small M), the general kernel (f32 operands) and f16 output."""
    shapes = {"fast_full": (512, 384, 256, we.BF16, we.FP8, we.BF16), "fast_ragged": (300, 520, 208, we.BF16, we.FP8, we.BF16),
              "small_m_split": (48, 3072, 3072, we.F16, we.FP8, we.F16), "generic_f32": (70, 90, 128, we.F32, we.F32, we.F32),
              "f16_out": (256, 256, 192, we.F16, we.F16, we.F16), "gelu_bias": (512, 384, 256, we.BF16, we.FP8, we.BF16)}
    m, n, k, x_dt, w_dt, y_dt = shapes[case]
    flags = we.EPI_BIAS | we.EPI_GELU if case == "gelu_bias" else 0
    rng = np.random.default_rng(len(case))
    x_store, x_oracle, ox = encode_act(rng.standard_normal(m * k).astype(np.float32), x_dt)
    w_store, w_oracle, ow = make_weights(rng, n, k, w_dt)
    scale = 0.05 if w_dt == we.FP8 else 1.0
    gate = rng.uniform(-1.5, 1.5, n).astype(np.float32)
    bias = rng.uniform(-.5, .5, n).astype(np.float32) if flags & we.EPI_BIAS else None
    res_store, res_vals = _store(rng.standard_normal(m * n), y_dt)
    p = we.matmul_params(m, n, k, scale, graph=graph)
    mark = graph.mark()
    xb, wb, gb, rb = graph.buffer(x_store), graph.buffer(w_store), graph.buffer(gate), graph.buffer(res_store)
    yb = graph.buffer(m * n * we.ELEM_BYTES[y_dt])
    bb = graph.buffer(bias) if bias is not None else None
    if case == "generic_f32":
        tune(gemm_generic=1)
    graph.matmul(p, x_dt, xb, w_dt, wb, y_dt, yb, bias=bb, flags=flags, gate=gb, residual=rb)
    got = decode(graph.read(yb), y_dt)
    graph.release(mark)
    v = O.matmul(O.matmul_params(m, n, k, scale), ox, x_oracle, ow, w_oracle).reshape(m, n)
    if bias is not None:
        v = v + bias
    if flags & we.EPI_GELU:
        v = np.vectorize(O.lib.or_gelu_tanh)(v)
    want = (res_vals.reshape(m, n) + gate.astype(np.float64) * v).ravel()
    assert O.rel_error(got, want) < TOL[y_dt], case


def test_gated_residual_in_place_and_accumulate(graph):
    """residual = y (the block's x += gate * proj(...)), and no residual with ACCUMULATE: both equal the gatedAdd
    of the plain product onto y's old values, bit for bit across the two forms."""
    m, n, k = 512, 384, 256
    rng = np.random.default_rng(7)
    x = O.bf16_rne(rng.standard_normal(m * k).astype(np.float32))
    w, _, _ = make_weights(rng, n, k, we.FP8)
    gate = rng.uniform(-1, 1, n).astype(np.float32)
    y0, y0_vals = _store(rng.standard_normal(m * n), we.BF16)
    p = we.matmul_params(m, n, k, 0.05, graph=graph)
    mark = graph.mark()
    xb, wb, gb = graph.buffer(x), graph.buffer(w), graph.buffer(gate)
    y1, y2 = graph.buffer(y0), graph.buffer(y0)
    graph.matmul(p, we.BF16, xb, we.FP8, wb, we.BF16, y1, gate=gb, residual=y1)
    graph.matmul(p, we.BF16, xb, we.FP8, wb, we.BF16, y2, flags=we.EPI_ACCUMULATE, gate=gb)
    a, b = graph.read(y1), graph.read(y2)
    graph.release(mark)
    assert np.array_equal(a, b)
    v = O.matmul(O.matmul_params(m, n, k, 0.05), O.BF16, x, O.FP8, w).reshape(m, n)
    assert O.rel_error(decode(a, we.BF16), (y0_vals.reshape(m, n) + gate * v).ravel()) < TOL[we.BF16]


def test_gated_residual_int4(graph):
    m, n, k, group = 8, 640, 1024, 64
    rng = np.random.default_rng(9)
    words = rng.integers(0, 2 ** 32, n * k // 8, dtype=np.uint64).astype(np.uint32)
    scales = np.abs(rng.normal(0, 0.01, n * k // group)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(m * k).astype(np.float16)
    gate = rng.uniform(-1, 1, n).astype(np.float32)
    res = rng.standard_normal(m * n).astype(np.float32)
    p = we.matmul_params(m, n, k, 1.0, graph=graph)
    mark = graph.mark()
    yb = graph.buffer(m * n * 4)
    graph.matmul(p, we.F16, graph.buffer(x), we.INT4, graph.buffer(words), we.F32, yb, scales=graph.buffer(scales),
                 group=group, gate=graph.buffer(gate), residual=graph.buffer(res))
    got = graph.read(yb).view(np.float32).astype(np.float64)
    graph.release(mark)
    v = O.matmul(O.matmul_params(m, n, k, 1.0), O.F16, x.view(np.uint16), O.INT4, words, scales=scales, group=group)
    want = res.astype(np.float64) + (gate.astype(np.float64) * v.reshape(m, n)).ravel()
    assert O.rel_error(got, want) < TOL_F32_OUT


def test_gated_residual_refusals(graph):
    p = we.matmul_params(4, 4, 4, 1.0, graph=graph)
    b = graph.buffer(64)
    with pytest.raises(we.WeError, match="gate is null"):
        graph.check(graph.lib.we_matmul_gated(graph.ctx, ctypes.byref(p), we.F32, we._addr(b), we.F32, we._addr(b),
                                              None, 0, we.F32, we._addr(b), None, 0, None, None))
    with pytest.raises(we.WeError, match="split-K"):
        graph.matmul(p, we.F32, b, we.F32, b, we.F32, b, flags=we.EPI_SPLIT_K, gate=b)
    with pytest.raises(we.WeError, match="residual replaces accumulate"):
        graph.matmul(p, we.F32, b, we.F32, b, we.F32, b, flags=we.EPI_ACCUMULATE, gate=b, residual=b)


def _sigmoid(v):
    with np.errstate(over="ignore"):  # exp(-v) -> inf for very negative v: sigmoid -> 0, its limit
        return 1.0 / (1.0 + np.exp(-v))


@pytest.mark.parametrize("mul", [we.MUL_SWIGLU, we.MUL_SIGMOID_GATE])
@pytest.mark.parametrize("case", ["fast_full", "fast_ragged", "small_m_split", "generic_f32", "f16_out", "bias"])
def test_product_epilogue_equals_gemm_then_the_elementwise_step(graph, case, mul, tune):
    """y = silu(aux) * v (swiglu with the GEMM as `up`) or aux * sigmoid(v) (sigmoidGate with the GEMM as `gate`),
    v the scaled (biased) product, against the f64 oracle of the product followed by the reference's formula
    (src/kernels/elementwise.ts:38-50), on every epilogue: the fast kernel's whole-tile and per-value paths, the
    split-K reduce pass (small M), the general kernel (f32 operands) and f16 output."""
    shapes = {"fast_full": (512, 384, 256, we.BF16, we.FP8, we.BF16), "fast_ragged": (300, 520, 208, we.BF16, we.FP8, we.BF16),
              "small_m_split": (48, 3072, 3072, we.F16, we.FP8, we.F16), "generic_f32": (70, 90, 128, we.F32, we.F32, we.F32),
              "f16_out": (256, 256, 192, we.F16, we.F16, we.F16), "bias": (512, 384, 256, we.BF16, we.FP8, we.F32)}
    m, n, k, x_dt, w_dt, y_dt = shapes[case]
    rng = np.random.default_rng(len(case) + 10 * mul)
    x_store, x_oracle, ox = encode_act(rng.standard_normal(m * k).astype(np.float32), x_dt)
    w_store, w_oracle, ow = make_weights(rng, n, k, w_dt)
    scale = 0.05 if w_dt == we.FP8 else 1.0
    bias = rng.uniform(-.5, .5, n).astype(np.float32) if case == "bias" else None
    aux_store, aux_vals = _store(rng.standard_normal(m * n) * 2, y_dt)
    p = we.matmul_params(m, n, k, scale, graph=graph)
    mark = graph.mark()
    xb, wb, ab = graph.buffer(x_store), graph.buffer(w_store), graph.buffer(aux_store)
    yb = graph.buffer(m * n * we.ELEM_BYTES[y_dt])
    bb = graph.buffer(bias) if bias is not None else None
    if case == "generic_f32":
        tune(gemm_generic=1)
    graph.matmul(p, x_dt, xb, w_dt, wb, y_dt, yb, bias=bb, flags=we.EPI_BIAS if bias is not None else 0, mul=mul, aux=ab)
    got = decode(graph.read(yb), y_dt)
    graph.release(mark)
    v = O.matmul(O.matmul_params(m, n, k, scale), ox, x_oracle, ow, w_oracle)
    if bias is not None:
        v = v + np.tile(bias.astype(np.float64), m)
    want = aux_vals * _sigmoid(aux_vals) * v if mul == we.MUL_SWIGLU else aux_vals * _sigmoid(v)
    assert O.rel_error(got, want) < TOL[y_dt], (case, mul)


@pytest.mark.parametrize("mul", [we.MUL_SWIGLU, we.MUL_SIGMOID_GATE])
def test_product_epilogue_in_place_and_against_the_unfused_pair(graph, mul):
    """aux = y (the block writes the product over the gate / attention output) gives the same bits as a separate
    aux buffer; with f32 output the fused result equals linear + the elementwise kernel to f32 rounding."""
    m, n, k = 512, 384, 256
    rng = np.random.default_rng(20 + mul)
    x = O.bf16_rne(rng.standard_normal(m * k).astype(np.float32))
    w, _, _ = make_weights(rng, n, k, we.FP8)
    aux = rng.standard_normal(m * n).astype(np.float32) * 2
    p = we.matmul_params(m, n, k, 0.05, graph=graph)
    mark = graph.mark()
    xb, wb = graph.buffer(x), graph.buffer(w)
    sep, inplace, v, pair = graph.buffer(m * n * 4), graph.buffer(aux), graph.buffer(m * n * 4), graph.buffer(m * n * 4)
    ab = graph.buffer(aux)
    graph.matmul(p, we.BF16, xb, we.FP8, wb, we.F32, sep, mul=mul, aux=ab)
    graph.matmul(p, we.BF16, xb, we.FP8, wb, we.F32, inplace, mul=mul, aux=inplace)
    graph.matmul(p, we.BF16, xb, we.FP8, wb, we.F32, v)
    op = we.OP_SWIGLU if mul == we.MUL_SWIGLU else we.OP_SIGMOID_GATE
    graph.elementwise(op, m * n, 1, we.F32, ab, v, None, pair)
    a, b, c = (graph.read(t, dtype=np.float32).astype(np.float64) for t in (sep, inplace, pair))
    graph.release(mark)
    assert np.array_equal(a, b)
    assert O.rel_error(a, c) < 1e-6


def test_product_epilogue_refusals(graph):
    p = we.matmul_params(4, 4, 4, 1.0, graph=graph)
    b = graph.buffer(64)
    with pytest.raises(we.WeError, match="aux is null"):
        graph.matmul(p, we.F32, b, we.F32, b, we.F32, b, mul=we.MUL_SWIGLU, aux=None)
    with pytest.raises(we.WeError, match="unknown product epilogue 3"):
        graph.matmul(p, we.F32, b, we.F32, b, we.F32, b, mul=3, aux=b)
    for flags in (we.EPI_GELU, we.EPI_ACCUMULATE, we.EPI_SPLIT_K):
        with pytest.raises(we.WeError, match="takes only WE_EPI_BIAS"):
            graph.matmul(p, we.F32, b, we.F32, b, we.F32, b, flags=flags, mul=we.MUL_SIGMOID_GATE, aux=b)
    with pytest.raises(we.WeError, match="int4 weights have no product epilogue") as e:
        graph.matmul(p, we.F16, b, we.INT4, b, we.F32, b, scales=b, group=64, mul=we.MUL_SWIGLU, aux=b)
    assert e.value.code == 4


# ---- the conv3x3 input mode (src/kernels/matmul.ts:74-83, conv3x3Params :268-272) ----

def test_conv3x3_matches_the_direct_convolution(graph):  # tests/gpu/image.test.ts:11-30
    h, w, cin, cout = 5, 7, 8, 12
    u = O.lcg(5, h * w * cin + cout * 9 * cin)
    x = (u[: h * w * cin] * 2 - 1).astype(np.float32)
    wt = (u[h * w * cin:] * 2 - 1).astype(np.float32)
    mark = graph.mark()
    y = we.conv3x3(graph, graph.buffer(x), graph.buffer(wt), h, w, cin, cout)
    got = graph.read(y, dtype=np.float32).astype(np.float64)
    graph.release(mark)
    want = O.matmul(O.conv3x3_params(h, w, cin, cout), O.F32, x, O.F32, wt)
    assert np.abs(got - want).max() < 1e-5  # the reference test's bar


@pytest.mark.parametrize("x_dt,w_dt,y_dt,flags", [(we.BF16, we.FP8, we.BF16, 0), (we.F16, we.F16, we.F32, we.EPI_BIAS),
                                                  (we.F32, we.BF16, we.F32, we.EPI_GELU),
                                                  (we.BF16, we.FP8, we.F32, we.EPI_SPLIT_K)])
def test_conv3x3_dtypes_ragged_and_epilogues(graph, x_dt, w_dt, y_dt, flags):
    """cin = 12 (8-value chunks straddle two taps), odd height and width, several tiles; against the oracle's
    conv addressing (itself pinned by a direct convolution in test_oracle.py)."""
    h, w, cin, cout = 19, 23, 12, 70
    rng = np.random.default_rng(x_dt * 10 + w_dt)
    x_store, x_oracle, ox = encode_act(rng.standard_normal(h * w * cin).astype(np.float32), x_dt)
    w_store, w_oracle, ow = make_weights(rng, cout, 9 * cin, w_dt)
    p = we.conv3x3_params(h, w, cin, cout, graph=graph)
    p.scale = 0.05
    bias = rng.uniform(-1, 1, cout).astype(np.float32) if flags & we.EPI_BIAS else None
    op = O.conv3x3_params(h, w, cin, cout)
    op.scale = 0.05
    if flags & we.EPI_SPLIT_K:
        p.k_split = op.k_split = 3
    got = run(graph, p, x_store, x_dt, w_store, w_dt, y_dt, flags=flags, bias=bias)
    want = O.matmul(op, ox, x_oracle, ow, w_oracle, split=bool(flags & we.EPI_SPLIT_K))
    if bias is not None:
        want = want + np.tile(bias.astype(np.float64), h * w)
    if flags & we.EPI_GELU:
        want = O.gelu_tanh(want)
    tol = 1e-4 if flags & we.EPI_GELU else TOL[y_dt]
    assert O.rel_error(got, want) < tol


def test_conv3x3_refusals(graph):
    with pytest.raises(we.WeError, match="cin must be a multiple of 4, got 6"):
        we.conv3x3_params(4, 4, 6, 8, graph=graph)
    p = we.conv3x3_params(4, 4, 8, 8, graph=graph)
    b = graph.buffer(65536)
    p.k = 64
    with pytest.raises(we.WeError, match="K = 9 \\* cin"):
        graph.matmul(p, we.F32, b, we.F32, b, we.F32, b)
    p = we.conv3x3_params(4, 4, 8, 8, graph=graph)
    with pytest.raises(we.WeError, match="int4 weights have no 3x3 convolution input"):
        graph.matmul(p, we.F16, b, we.INT4, b, we.F32, b, scales=b, group=64)


F32_FAST_CASES = [
    # (m, n, k, weights, flags): ragged tiles, the small-M split-K plan over the planes, the reference's Krea layer
    # shape, bf16 weights, and the fused epilogues
    (300, 520, 192, we.FP8, 0), (64, 3072, 3072, we.FP8, 0), (8, 1536, 6144, we.FP8, 0), (130, 200, 320, we.BF16, 0),
    (512, 768, 512, we.FP8, we.EPI_BIAS | we.EPI_GELU), (256, 512, 1024, we.BF16, we.EPI_ACCUMULATE),
]


@pytest.mark.parametrize("m,n,k,w_dt,flags", F32_FAST_CASES)
def test_f32_activations_on_the_fast_path(graph, tune, m, n, k, w_dt, flags):
    """f32 x, the reference's own activation dtype (src/kernels/matmul.ts:129-131), with fp8 or bf16 weights and K a
    multiple of 64: split into three exact bf16 planes and run by the fast kernel over 3K. It matches the float64
    oracle at the reference's 1e-5 bar, and the general kernel (which splits x into the same planes tile by tile)
    to 4e-6: every product is exact in both, only the f32 summation order differs (at K = 3072, sums of ~200 move by
    ~1.5e-6 of max|y| between two orders)."""
    rng = np.random.default_rng(m + n + k)
    x = rng.standard_normal(m * k).astype(np.float32)
    w_store, w_oracle, ow = make_weights(rng, n, k, w_dt)
    scale = 0.02 if w_dt == we.FP8 else 1.0
    bias = rng.normal(0, 1, n).astype(np.float32) if flags & we.EPI_BIAS else None
    y0 = rng.standard_normal(m * n).astype(np.float32) if flags & we.EPI_ACCUMULATE else None
    p = we.matmul_params(m, n, k, scale, graph=graph)
    got = run(graph, p, x, we.F32, w_store, w_dt, we.F32, flags=flags, bias=bias, y_init=y0)
    want = O.matmul(O.matmul_params(m, n, k, scale), O.F32, x, ow, w_oracle)
    if bias is not None:
        want = want + np.tile(bias.astype(np.float64), m)
    if flags & we.EPI_GELU:
        want = O.gelu_tanh(want)
    if y0 is not None:
        want = want + y0.astype(np.float64)
    tol = 1e-4 if flags & we.EPI_GELU else TOL_F32_OUT
    assert O.rel_error(got, want) < tol
    tune(gemm_generic=1)
    general = run(graph, p, x, we.F32, w_store, w_dt, we.F32, flags=flags, bias=bias, y_init=y0)
    assert O.rel_error(got, general) < 4e-6


# ---- the ping-pong tiles (16x16x32 accumulator layout) through every epilogue ----

PP_CASES = {  # x dtype, weight dtype, y dtype, epilogue
    "plain_bf16": (we.BF16, we.FP8, we.BF16, "plain"), "plain_bf16_weights": (we.BF16, we.BF16, we.BF16, "plain"),
    "gelu_bf16": (we.BF16, we.FP8, we.BF16, "gelu"), "bias_gelu_f32": (we.BF16, we.FP8, we.F32, "bias_gelu"),
    "gated_bf16": (we.BF16, we.FP8, we.BF16, "gated"), "gated_f32_f16x": (we.F16, we.FP8, we.F32, "gated"),
    "swiglu_bf16": (we.BF16, we.FP8, we.BF16, "swiglu"), "sigmoid_gate_f16": (we.F16, we.F16, we.F16, "sigmoid"),
    "accumulate_f32": (we.BF16, we.FP8, we.F32, "accumulate"), "split_partials": (we.BF16, we.FP8, we.F32, "partials"),
    "reduce_pass_bf16": (we.BF16, we.FP8, we.BF16, "reduce"),
}


@pytest.mark.parametrize("shape", ["whole", "ragged"])
@pytest.mark.parametrize("cfg", [0, 5])
@pytest.mark.parametrize("case", list(PP_CASES))
def test_pingpong_tiles_every_epilogue(graph, tune, cfg, shape, case):
    """The ping-pong tiles (gemm_cfg 0: 256 x 256, 5: 256 x 192; 16x16x32 MFMAs, whose accumulator blocks hold one
    run of 4 columns per lane) through every epilogue, on whole tiles (the per-row fast paths, the LDS-staged
    16-bit stores) and ragged ones (the per-value path, a partial last K block): against the oracle's product
    followed by the reference's epilogue formulas (bias and GELU src/kernels/elementwise.ts:25-29, gatedAdd :52-58,
    swiglu :38-43, sigmoidGate :45-50, accumulate and split-K partials src/kernels/matmul.ts:159-175)."""
    x_dt, w_dt, y_dt, epi = PP_CASES[case]
    m, n, k = (512, 768, 256) if shape == "whole" else (300, 520, 208)
    if epi == "reduce":  # the split-K reduce plan needs K >= 512
        k += 256 if shape == "whole" else 320
    rng = np.random.default_rng(cfg * 100 + len(case) + (7 if shape == "whole" else 0))
    x_store, x_oracle, ox = encode_act(rng.standard_normal(m * k).astype(np.float32), x_dt)
    w_store, w_oracle, ow = make_weights(rng, n, k, w_dt)
    scale = 0.05 if w_dt == we.FP8 else 1.0
    tune(gemm_cfg=cfg, gemm_splitk=2 if epi == "reduce" else 0)
    split = 2 if epi == "partials" else 1
    p = we.matmul_params(m, n, k, scale, k_split=split, graph=graph)
    flags = {"gelu": we.EPI_GELU, "bias_gelu": we.EPI_BIAS | we.EPI_GELU, "accumulate": we.EPI_ACCUMULATE,
             "partials": we.EPI_SPLIT_K}.get(epi, 0)
    bias = rng.uniform(-.5, .5, n).astype(np.float32) if flags & we.EPI_BIAS else None
    gate = rng.uniform(-1.5, 1.5, n).astype(np.float32) if epi == "gated" else None
    other_store, other = _store(rng.standard_normal(m * n), y_dt) if epi in ("gated", "swiglu", "sigmoid",
                                                                               "accumulate") else (None, None)
    mark = graph.mark()
    xb, wb = graph.buffer(x_store), graph.buffer(w_store)
    yb = graph.buffer(other_store) if epi == "accumulate" else graph.buffer(m * split * n * we.ELEM_BYTES[y_dt])
    bb = graph.buffer(bias) if bias is not None else None
    kw = {}
    if epi == "gated":
        kw = {"gate": graph.buffer(gate), "residual": graph.buffer(other_store)}
    elif epi in ("swiglu", "sigmoid"):
        kw = {"mul": we.MUL_SWIGLU if epi == "swiglu" else we.MUL_SIGMOID_GATE, "aux": graph.buffer(other_store)}
    graph.matmul(p, x_dt, xb, w_dt, wb, y_dt, yb, bias=bb, flags=flags, **kw)
    got = decode(graph.read(yb), y_dt)
    graph.release(mark)
    if epi == "partials":
        want = O.matmul(O.matmul_params(m, n, k, scale, k_split=split), ox, x_oracle, ow, w_oracle, split=True)
        full = O.matmul(O.matmul_params(m, n, k, scale), ox, x_oracle, ow, w_oracle)
        assert np.abs(got - want).max() < TOL_F32_OUT * np.abs(full).max(), (cfg, shape)
        return
    v = O.matmul(O.matmul_params(m, n, k, scale), ox, x_oracle, ow, w_oracle)
    if bias is not None:
        v = v + np.tile(bias.astype(np.float64), m)
    if flags & we.EPI_GELU:
        v = np.vectorize(O.lib.or_gelu_tanh)(v)
    if epi == "gated":
        v = other + np.tile(gate.astype(np.float64), m) * v
    elif epi == "swiglu":
        v = other * _sigmoid(other) * v
    elif epi == "sigmoid":
        v = other * _sigmoid(v)
    elif epi == "accumulate":
        v = other + v
    assert O.rel_error(got, v) < TOL[y_dt], (cfg, shape, case)


@pytest.mark.parametrize("m,n,k", [(1, 1, 4), (1, 1, 64), (2, 3, 8), (5, 1, 68), (1, 7, 260), (3, 2, 128), (9, 1, 192)])
@pytest.mark.parametrize("w_dt,x_dt", [(we.FP8, we.BF16), (we.FP8, we.F32), (we.BF16, we.F16)])
def test_tiny_shapes(graph, m, n, k, w_dt, x_dt):
    """Shapes far below every tile: one output column, one row, K of a single vec4 (the reference's smallest
    unit, matmulParams' K % 4 rule) and K one vec4 past a 64-k block. f32 output against the oracle."""
    rng = np.random.default_rng(m * 100 + n * 10 + k)
    x_store, x_oracle, ox = encode_act(rng.standard_normal(m * k).astype(np.float32), x_dt)
    if w_dt == we.FP8:
        w = rng.integers(0, 254, n * k).astype(np.uint8)
        w = (w + (w >= 0x7F)).astype(np.uint8)
        ow = O.FP8
    else:
        w = O.bf16_rne(rng.standard_normal(n * k).astype(np.float32))
        ow = O.BF16
    p = we.matmul_params(m, n, k, 0.5, graph=graph)
    got = run(graph, p, x_store, x_dt, w, w_dt, we.F32)
    want = O.matmul(O.matmul_params(m, n, k, 0.5), ox, x_oracle, ow, w)
    assert O.rel_error(got, want) < TOL_F32_OUT

"""Pins the CPU oracle before the GPU tests compare the HIP path against it.

Sources of truth, none of them the oracle itself:
  * known-answer values from the reference's own tests (tests/fp8.test.ts, tests/noise.test.ts,
    tests/rope.test.ts, tests/gpu/fp8.test.ts, tests/gpu/matmul.test.ts, tests/gpu/rmsnorm.test.ts);
  * the reference's fixture tests/fixtures/torch-randn.json (copied to tests/golden/);
  * torch's float8_e4m3fn / bfloat16 / float16 / tanh-GELU (tests/golden/*.json, see make_golden.py);
  * numpy float64 library routines (matmul, einsum, complex rotation, scipy's expit) on the same inputs.
Each "plausible mistake" check shows that a dropped term, a transposed operand or a wrong index would
fail the same comparison.
"""
import json
import math
import pathlib

import numpy as np
import pytest
from scipy.special import expit

import oracle_lib as O

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def load(name):
    return json.loads((GOLDEN / name).read_text())


E4M3_TORCH = np.array([float("nan") if v == "nan" else float(v) for v in load("e4m3fn.json")["decode"]])


# ---------------------------------------------------------------------------------------------- decoders

@pytest.mark.parametrize("byte,value", [(0x00, 0.0), (0x38, 1.0), (0xC0, -2.0), (0x7E, 448.0), (0x01, 2.0 ** -9),
                                        (0x08, 2.0 ** -6), (0x3C, 1.5)])
def test_e4m3_known_answers(byte, value):  # tests/fp8.test.ts:5-19
    assert O.e4m3(byte) == value


def test_e4m3_negative_zero_nan_no_infinity():  # tests/fp8.test.ts:21-25
    assert O.e4m3(0x80) == 0.0 and math.copysign(1.0, O.e4m3(0x80)) < 0
    assert math.isnan(O.e4m3(0x7F)) and math.isnan(O.e4m3(0xFF))


def test_e4m3_all_codes_match_torch():
    ours = O.e4m3_table()
    nan = np.isnan(E4M3_TORCH)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], E4M3_TORCH[~nan])
    assert np.array_equal(np.signbit(ours[~nan]), np.signbit(E4M3_TORCH[~nan]))


def test_shader_decoder_equals_cpu_decoder_and_has_no_nan_branch():  # tests/gpu/fp8.test.ts:21-28, kernels/fp8.ts:12-20
    gpu = O.e4m3_gpu_table().astype(np.float64)
    ref = E4M3_TORCH
    ok = ~np.isnan(ref)
    assert np.array_equal(gpu[ok], ref[ok])
    assert np.array_equal(np.signbit(gpu[ok]), np.signbit(ref[ok]))
    assert gpu[0x7F] == 480.0 and gpu[0xFF] == -480.0


@pytest.mark.parametrize("byte,value", [(0x00, 0.0), (0x3C, 1.0), (0x7B, 57344.0), (0x01, 2.0 ** -16), (0xC0, -2.0),
                                        (0x7C, math.inf), (0xFC, -math.inf)])
def test_e5m2_known_answers(byte, value):  # tests/fp8.test.ts:27-41
    assert O.lib.or_e5m2(byte) == value
    assert math.isnan(O.lib.or_e5m2(0x7E))


def test_f16_and_bf16_known_answers():  # tests/fp8.test.ts:44-50
    assert [O.lib.or_bf16(h) for h in (0x3F80, 0xC000)] == [1.0, -2.0]
    assert [O.lib.or_f16(h) for h in (0x3C00, 0xC000, 0x0001, 0x7C00)] == [1.0, -2.0, 2.0 ** -24, math.inf]
    every = np.arange(65536, dtype=np.uint16)
    ours = np.array([O.lib.or_f16(int(h)) for h in every])
    lib = every.view(np.float16).astype(np.float64)
    ok = ~np.isnan(lib)
    assert np.array_equal(np.isnan(ours), ~ok) and np.array_equal(ours[ok], lib[ok])


def test_unpack_fp8_scale_and_odd_length():  # tests/gpu/fp8.test.ts:30-37
    s = 0.0018833705689758062
    got = O.unpack_fp8(np.array([0x38, 0xC0, 0x7E], np.uint8), s)
    want = np.array([1.0, -2.0, 448.0], np.float32) * np.float32(s)
    assert np.array_equal(got, want)
    assert O.unpack_fp8(np.array([0x38, 0x38, 0x38, 0x38, 0x40], np.uint8), 1.0).tolist() == [1, 1, 1, 1, 2]


def test_float_conversions_match_torch():
    g = load("convert.json")
    f = np.array(g["f32_bits"], np.uint32).view(np.float32)
    assert O.to_bf16(f).tolist() == g["bf16"]
    assert O.bf16_rne(f).tolist() == g["bf16"]
    assert O.to_f16(f).tolist() == g["f16"]
    # numpy's own float16 rounding agrees as a second library
    with np.errstate(over="ignore"):
        assert np.array_equal(O.to_f16(f), f.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------------------------------------- generators

def test_lcg_sequence():  # tests/gpu/matmul.test.ts:10-12
    s, want = 1, []
    for _ in range(5):
        s = (s * 1664525 + 1013904223) % 2 ** 32
        want.append(s / 2 ** 32)
    assert O.lcg(1, 5).tolist() == want
    st = __import__("ctypes").c_uint32(1)
    assert [O.lib.or_lcg_uniform(__import__("ctypes").byref(st)) for _ in range(5)] == want


def test_matmul_test_data_layout():  # tests/gpu/matmul.test.ts:14-23: x first, then w; no NaN codes
    m, n, k = 37, 70, 100
    x, w = O.matmul_test_data(m, n, k, 1)
    u = O.lcg(1, m * k + n * k)
    assert np.array_equal(x, (u[: m * k] * 2 - 1).astype(np.float32))
    b = np.floor(u[m * k:] * 256).astype(np.int64)
    b = np.where((b & 0x7F) == 0x7F, b - 1, b)
    assert np.array_equal(w, b.astype(np.uint8))
    assert not np.any((w & 0x7F) == 0x7F)


def test_mt19937_known_answers():  # tests/noise.test.ts:11-20
    import ctypes
    mt = (ctypes.c_uint32 * 625)()
    O.lib.or_mt_seed(mt, 5489)
    last = 0
    for _ in range(10000):
        last = O.lib.or_mt_next(mt)
    assert last == 4123659995
    a, b = (ctypes.c_uint32 * 625)(), (ctypes.c_uint32 * 625)()
    O.lib.or_mt_seed(a, 2 ** 32 + 7)
    O.lib.or_mt_seed(b, 7)
    assert O.lib.or_mt_next(a) == O.lib.or_mt_next(b)


def test_torch_randn_known_answers_and_fixture():  # tests/noise.test.ts:25-45
    r4 = lambda a: [round(float(v), 4) for v in a]
    assert r4(O.torch_randn(6, 0)) == [1.541, -0.2934, -2.1788, 0.5684, -1.0845, -1.3986]
    assert r4(O.torch_randn(3, 42)) == [0.3367, 0.1288, 0.2345]
    assert r4(O.torch_randn(16, 0)) == [-1.1258, -1.1524, -0.2506, -0.4339, 0.8487, 0.692, -0.316, -2.1152, 0.3223,
                                        -1.2633, 0.35, 0.3081, 0.1198, 1.2377, 1.1168, -0.2473]
    for case in load("torch-randn.json")["cases"]:
        a = O.torch_randn(case["n"], case["seed"])
        for i, v in case["values"].items():
            assert abs(a[int(i)] - v) < 5e-7, (case["n"], case["seed"], i)


# ---------------------------------------------------------------------------------------------- matmul

def np_matmul(x, wdec, m, n, k, scale):
    return (x.astype(np.float64).reshape(m, k) @ wdec.astype(np.float64).reshape(n, k).T * scale).ravel()


@pytest.mark.parametrize("m,n,k,scale,seed", [(1, 1, 4, 0.002, 1), (37, 70, 100, 0.002, 1), (64, 64, 64, 0.002, 1),
                                              (130, 65, 36, 0.002, 1), (200, 260, 84, 0.002, 1),
                                              (8, 1536, 512, 0.0018833705689758062, 7)])
def test_fp8_matmul_oracle_matches_numpy(m, n, k, scale, seed):  # tests/gpu/matmul.test.ts:49-66
    x, w = O.matmul_test_data(m, n, k, seed)
    p = O.matmul_params(m, n, k, scale)
    got = O.matmul(p, O.F32, x, O.FP8, w)
    want = np_matmul(x, E4M3_TORCH[w], m, n, k, np.float32(scale))
    assert O.rel_error(got, want) < 1e-12
    if min(n, k) > 1 and n != k:  # a transposed W cannot pass
        wrong = np_matmul(x, E4M3_TORCH[w].reshape(n, k).T.copy().ravel()[: n * k], m, n, k, np.float32(scale))
        assert O.rel_error(got, wrong) > 1e-3
    if k > 4:  # a dropped last k term cannot pass
        wd = E4M3_TORCH[w].reshape(n, k).copy()
        wd[:, -1] = 0
        assert O.rel_error(got, np_matmul(x, wd.ravel(), m, n, k, np.float32(scale))) > 1e-6


def test_matmul_params_validation():  # tests/gpu/matmul.test.ts:68-72, kernels/matmul.ts:205-207
    with pytest.raises(ValueError, match="K must be a multiple of 4, got 6"):
        O.matmul_params(1, 1, 6, 1.0)
    with pytest.raises(ValueError, match="xStride"):
        O.matmul_params(1, 1, 4, 1.0, x_stride=6)
    with pytest.raises(ValueError, match="wOffset"):
        O.matmul_params(1, 1, 4, 1.0, w_offset=2)
    p = O.matmul_params(3, 5, 8, 0.5)
    assert (p.x_stride, p.w_stride, p.y_stride, p.k_split) == (8, 8, 5, 1)


def test_ksplit_known_answers():  # tests/gpu/matmul.test.ts:151-156
    assert O.ksplit_for(1088, 64, 6144) == 24
    assert O.ksplit_for(4160, 64, 16384) == 8
    assert O.ksplit_for(4160, 6144, 6144) == 1
    assert O.ksplit_for(5, 12, 16) == 1
    assert O.ksplit_chunk(200, 3) == 80  # slices of 80, 80, 40 (tests/gpu/matmul.test.ts:133)


def test_split_k_partials_sum_to_the_full_product():  # tests/gpu/matmul.test.ts:131-149
    m, n, k, split, scale = 5, 12, 200, 3, 0.5
    x, w = O.matmul_test_data(m, n, k, 3)
    p = O.matmul_params(m, n, k, scale, k_split=split)
    parts = O.matmul(p, O.F32, x, O.FP8, w, split=True).reshape(split, m * n)
    want = np_matmul(x, E4M3_TORCH[w], m, n, k, scale)
    assert np.allclose(parts.sum(0), want, rtol=0, atol=1e-9)
    assert abs(parts[0, 0] - want[0]) > 1e-3
    wd = E4M3_TORCH[w].reshape(n, k)
    assert np.allclose(parts[2], np_matmul(x.reshape(m, k)[:, 160:].ravel(), wd[:, 160:].ravel(), m, n, 40, scale))


def test_accumulate_adds_to_y():  # tests/gpu/matmul.test.ts:159-175
    m, n, k, scale = 3, 6, 8, 0.25
    x = (np.arange(m * k) % 5 - 2).astype(np.float32)
    w = ((np.arange(n * k) * 3) % 7 - 3).astype(np.float32)
    start = np.arange(m * n, dtype=np.float64)
    p = O.matmul_params(m, n, k, scale)
    plain = O.matmul(p, O.F32, x, O.F32, w)
    got = O.matmul(p, O.F32, x, O.F32, w, accumulate=True, y=start)
    assert np.array_equal(got, plain + start)


def test_strided_head_pick():  # tests/gpu/matmul.test.ts:93-109
    tokens, heads, kv, dim = 20, 4, 2, 128
    rng = np.random.default_rng(3)
    q = rng.uniform(-1, 1, tokens * heads * dim).astype(np.float32)
    kk = rng.uniform(-1, 1, tokens * kv * dim).astype(np.float32)
    h, g = 2, 1
    p = O.matmul_params(tokens, tokens, dim, 1.0, x_stride=heads * dim, x_offset=h * dim, w_stride=kv * dim,
                        w_offset=g * dim, y_stride=24)
    got = O.matmul(p, O.F32, q, O.F32, kk, out_len=tokens * 24).reshape(tokens, 24)[:, :tokens]
    want = q.reshape(tokens, heads, dim)[:, h].astype(np.float64) @ kk.reshape(tokens, kv, dim)[:, g].astype(np.float64).T
    assert np.abs(got - want).max() < 1e-9


def test_bf16_and_half_activation_matmul():  # tests/gpu/matmul.test.ts:112-127
    m, n, k = 37, 70, 100
    rng = np.random.default_rng(9)
    x = rng.uniform(-1, 1, m * k).astype(np.float32)
    wf = rng.uniform(-1, 1, n * k).astype(np.float32)
    wb = (wf.view(np.uint32) >> 16).astype(np.uint16)  # truncation, as the reference test does
    p = O.matmul_params(m, n, k, 0.5)
    got = O.matmul(p, O.F32, x, O.BF16, wb)
    assert O.rel_error(got, np_matmul(x, O.bf16_to_f32(wb), m, n, k, 0.5)) < 1e-12
    xh = x.astype(np.float16)
    got = O.matmul(p, O.F16, xh.view(np.uint16), O.BF16, wb)
    assert O.rel_error(got, np_matmul(xh.astype(np.float32), O.bf16_to_f32(wb), m, n, k, 0.5)) < 1e-12
    xb = O.to_bf16(x)
    got = O.matmul(p, O.BF16, xb, O.FP8, np.zeros(n * k, np.uint8) + 0x38)
    assert O.rel_error(got, np_matmul(O.bf16_to_f32(xb), np.ones(n * k), m, n, k, 0.5)) < 1e-12


def np_int4_dequant(words, scales, rows, k, group):
    nib = (words[:, None] >> (4 * np.arange(8, dtype=np.uint32))[None, :]) & 0xF
    q = np.where(nib >= 8, nib.astype(np.int64) - 16, nib.astype(np.int64)).reshape(rows, k)
    s = scales.view(np.float16).astype(np.float64).reshape(rows, k // group)
    return q * np.repeat(s, group, axis=1)


def test_int4_every_code_and_scale():
    scales = np.array([0x3C00, 0x2E66, 0x1400, 0x8001, 0xBC00, 0x0000], np.uint16)
    for s in scales:
        for code in range(16):
            word = code << 12  # nibble 3
            q = code - 16 if code >= 8 else code
            v = O.lib.or_int4_value(word, 3, int(s))
            assert v == np.float32(q * float(np.array([s], np.uint16).view(np.float16)[0]))


@pytest.mark.parametrize("m,n,k,group", [(1, 40, 128, 64), (8, 33, 256, 64), (16, 17, 192, 64), (3, 9, 96, 32)])
def test_int4_gemv_oracle_matches_numpy(m, n, k, group):
    rng = np.random.default_rng(m * 100 + n)
    words = rng.integers(0, 2 ** 32, n * k // 8, dtype=np.uint64).astype(np.uint32)
    scales = np.abs(rng.normal(0, 0.01, n * k // group)).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(m * k).astype(np.float16)
    p = O.matmul_params(m, n, k, 1.0)
    got = O.matmul(p, O.F16, x.view(np.uint16), O.INT4, words, scales=scales, group=group)
    wd = np_int4_dequant(words, scales, n, k, group)
    want = (x.astype(np.float64).reshape(m, k) @ wd.T).ravel()
    assert O.rel_error(got, want) < 1e-12
    assert np.array_equal(O.dequant_int4(words, scales, n, k, group), wd.astype(np.float32).ravel())
    # a wrong nibble order (high nibble first) cannot pass
    swapped = ((words & 0x0F0F0F0F) << 4) | ((words >> 4) & 0x0F0F0F0F)
    wrong = (x.astype(np.float64).reshape(m, k) @ np_int4_dequant(swapped, scales, n, k, group).T).ravel()
    assert O.rel_error(got, wrong) > 1e-3


def test_layer_sum_matches_einsum():  # src/kernels/text.ts:67-84
    t, layers, dim = 7, 3, 11
    rng = np.random.default_rng(1)
    x = rng.standard_normal(t * layers * dim).astype(np.float32)
    w = np.array([1.0, 0.5, -2.0], np.float32)
    want = np.einsum("tld,l->td", x.reshape(t, layers, dim).astype(np.float64), w.astype(np.float64)).ravel()
    assert np.abs(O.layer_sum(t, layers, dim, x, w) - want).max() < 1e-12


# ---------------------------------------------------------------------------------------------- rmsnorm / rope / elementwise

def np_rmsnorm(x, w, d, eps, offset, scale, shift):
    xr = x.astype(np.float64).reshape(-1, d)
    inv = 1.0 / np.sqrt((xr * xr).mean(1, keepdims=True) + eps)
    return (xr * inv * (offset + w.astype(np.float64)) * (1 + scale.astype(np.float64)) + shift).ravel()


@pytest.mark.parametrize("rows,d,offset,mod", [(3, 6144, 1.0, True), (100, 128, 0.0, False), (5, 37, 1.0, False)])
def test_rmsnorm_oracle(rows, d, offset, mod):  # tests/gpu/rmsnorm.test.ts:25-48
    rng = np.random.default_rng(d)
    x = rng.uniform(-4, 4, rows * d).astype(np.float32)
    w = rng.uniform(-0.1, 0.1, d).astype(np.float32)
    sc = rng.uniform(-1, 1, d).astype(np.float32) if mod else np.zeros(d, np.float32)
    sh = rng.uniform(-1, 1, d).astype(np.float32) if mod else np.zeros(d, np.float32)
    got = O.rmsnorm(x, w, 1e-5, offset, sc if mod else None, sh if mod else None)
    want = np_rmsnorm(x, w, d, 1e-5, offset, sc, sh)
    assert np.abs(got - want).max() < 1e-12
    assert np.abs(got - np_rmsnorm(x, w, d, 1e-5, 1.0 - offset, sc, sh)).max() > 1e-3  # offset matters


def test_rope_positions_known_answer():  # tests/rope.test.ts:4-17
    assert O.rope_positions(2, 2, 3, 3).tolist() == [[0, 0, 0], [0, 0, 0], [0, 0, 0], [0, 0, 1], [0, 0, 2], [0, 1, 0],
                                                    [0, 1, 1], [0, 1, 2]]


def test_rope_tables_known_answers():  # tests/rope.test.ts:19-39
    cos, sin, pairs = O.rope_tables(np.zeros((1, 3)), [32, 48, 48], 1000.0)
    assert pairs == 64 and cos.tolist() == [1.0] * 64 and sin.tolist() == [0.0] * 64
    cos, sin, _ = O.rope_tables(np.array([[0.0, 3.0, 5.0]]), [32, 48, 48], 1000.0)
    ang = lambda pos, j, dim: pos * 1000.0 ** (-(2 * j) / dim)
    assert sin[0] == 0
    assert abs(cos[16] - math.cos(ang(3, 0, 48))) < 5e-7
    assert abs(sin[16 + 5] - math.sin(ang(3, 5, 48))) < 5e-7
    assert abs(sin[40 + 23] - math.sin(ang(5, 23, 48))) < 5e-7
    with pytest.raises(ValueError, match="even"):
        O.rope_tables(np.zeros((1, 3)), [31, 48, 49], 1000.0)


@pytest.mark.parametrize("half", [False, True])
def test_rope_rotation_matches_complex_multiply(half):  # tests/gpu/rope.test.ts:5-42
    pos = O.rope_positions(2, 3, 4, 3)
    tokens, heads = pos.shape[0], 3
    cos, sin, pairs = O.rope_tables(pos, [32, 48, 48], 1000.0)
    rng = np.random.default_rng(1)
    x = rng.uniform(-1, 1, tokens * heads * pairs * 2).astype(np.float32)
    got = O.rope_rotate(x, tokens, heads, pairs, cos, sin, half)
    xr = x.astype(np.float64).reshape(tokens, heads, 2, pairs) if half else x.astype(np.float64).reshape(
        tokens, heads, pairs, 2)
    z = xr[:, :, 0, :] + 1j * xr[:, :, 1, :] if half else xr[..., 0] + 1j * xr[..., 1]
    e = (cos.astype(np.float64) + 1j * sin.astype(np.float64)).reshape(tokens, 1, pairs)
    r = z * e
    want = np.stack([r.real, r.imag], axis=2 if half else 3).ravel()
    assert np.abs(got - want).max() < 1e-12
    assert np.array_equal(got[: 2 * heads * pairs * 2], x[: 2 * heads * pairs * 2])  # text tokens unchanged
    wrong = np.stack([r.real, -r.imag], axis=2 if half else 3).ravel()  # the opposite rotation cannot pass
    assert np.abs(got - wrong).max() > 1e-3


def test_gelu_matches_torch_and_shader_form():  # tests/gpu/text.test.ts:56-60, kernels/elementwise.ts:25-29
    g = load("gelu.json")
    ours = np.array([O.lib.or_gelu_tanh(v) for v in g["x"]])
    assert np.abs(ours - np.array(g["gelu"])).max() < 1e-12
    shader = np.array([O.lib.or_gelu_tanh_shader(v) for v in g["x"]], np.float64)
    assert np.abs(shader - np.array(g["gelu"])).max() < 1e-5
    # the vectorized form used over whole GEMM outputs equals the C oracle, and the torch golden
    v = np.concatenate([np.array(g["x"]), np.random.default_rng(3).normal(0, 4, 5000)])
    assert np.abs(O.gelu_tanh(v) - np.array([O.lib.or_gelu_tanh(t) for t in v])).max() < 1e-12
    assert np.abs(O.gelu_tanh(g["x"]) - np.array(g["gelu"])).max() < 1e-12
    assert np.abs(O.gelu_tanh(v) - v).max() > 0.1  # not the identity


def test_elementwise_ops_match_scipy():  # src/kernels/elementwise.ts:38-84, tests/gpu/elementwise.test.ts:15-40
    n, d = 1000, 40
    rng = np.random.default_rng(1)
    a, b = (rng.uniform(-8, 8, n).astype(np.float32) for _ in range(2))
    g = rng.uniform(-1, 1, d).astype(np.float32)
    A, B, G = a.astype(np.float64), b.astype(np.float64), g.astype(np.float64)
    cases = {
        O.SWIGLU: (A * expit(A) * B, dict(b=b)),
        O.SIGMOID_GATE: (A * expit(B), dict(b=b)),
        O.GATED_ADD: (A + np.tile(G, n // d) * B, dict(b=b, c=g, d=d)),
        O.ADD_BIAS: (A + np.tile(G, n // d), dict(b=g, d=d)),
        O.ADD: (A + B, dict(b=b)),
        O.SILU: (A * expit(A), {}),
    }
    for op, (want, kw) in cases.items():
        assert np.abs(O.elementwise(op, a, **kw) - want).max() < 1e-12, op


def test_compare_known_answers():  # src/model/compare.ts:2-17
    a = np.array([1.0, 2.0, 3.0])
    r = O.compare(a, a)
    assert r["cosine"] == pytest.approx(1.0) and r["maxError"] == 0 and r["relativeError"] == 0
    r = O.compare(2 * a, a)
    assert r["cosine"] == pytest.approx(1.0) and r["maxError"] == 3 and r["relativeError"] == pytest.approx(1.0)
    r = O.compare(np.array([1.0, 0.0]), np.array([0.0, 1.0]))
    assert r["cosine"] == 0 and r["relativeError"] == pytest.approx(math.sqrt(2))
    assert O.rel_error(np.array([1.0, 2.5]), np.array([1.0, 2.0])) == pytest.approx(0.25)


# ----------------------------------------------------------------------------------- attention oracle

def _attention_numpy(q, k, v, tokens, heads, kv_heads, dim, causal):
    """Independent formulation: batched einsum scores, scipy softmax, masked by an upper-triangular -inf."""
    from scipy.special import softmax
    q = q.reshape(tokens, heads, dim)
    k = np.repeat(k.reshape(tokens, kv_heads, dim), heads // kv_heads, axis=1)
    v = np.repeat(v.reshape(tokens, kv_heads, dim), heads // kv_heads, axis=1)
    s = np.einsum("ihd,jhd->hij", q, k) / np.sqrt(dim)
    if causal:
        s = s + np.triu(np.full((tokens, tokens), -np.inf), 1)
    return np.einsum("hij,jhd->ihd", softmax(s, axis=-1), v).ravel()


@pytest.mark.parametrize("tokens,heads,kv_heads,dim,causal", [(37, 4, 1, 16, False), (64, 8, 2, 32, False),
                                                              (19, 4, 1, 24, True), (50, 6, 3, 8, True)])
def test_attention_oracle_matches_numpy(tokens, heads, kv_heads, dim, causal):  # tests/gpu/attention.test.ts:9-32
    u = O.lcg(tokens + dim, tokens * (heads + 2 * kv_heads) * dim) * 4 - 2
    q = u[: tokens * heads * dim]
    k = u[tokens * heads * dim: tokens * (heads + kv_heads) * dim]
    v = u[tokens * (heads + kv_heads) * dim:]
    got = O.attention(q, k, v, tokens, heads, kv_heads, dim, causal)
    assert np.abs(got - _attention_numpy(q, k, v, tokens, heads, kv_heads, dim, causal)).max() < 1e-12
    b, e = 5, 17
    part = O.attention(q, k, v, tokens, heads, kv_heads, dim, causal, rows=(b, e))
    assert np.array_equal(part, got.reshape(tokens, -1)[b:e].ravel())


def test_attention_oracle_closed_forms():
    rng = np.random.default_rng(0)
    tokens, heads, kv_heads, dim = 9, 4, 2, 8
    v = rng.standard_normal(tokens * kv_heads * dim)
    q = rng.standard_normal(tokens * heads * dim)
    # equal keys: uniform weights, every query gets the mean of its kv head's values
    k = np.tile(rng.standard_normal(kv_heads * dim), tokens)
    out = O.attention(q, k, v, tokens, heads, kv_heads, dim).reshape(tokens, heads, dim)
    mean = v.reshape(tokens, kv_heads, dim).mean(0)
    for h in range(heads):
        assert np.allclose(out[:, h], mean[h // 2], atol=1e-12)  # query head h reads kv head h // (heads / kv)
    # causal: query 0 sees only key 0
    k = rng.standard_normal(tokens * kv_heads * dim)
    out = O.attention(q, k, v, tokens, heads, kv_heads, dim, causal=True).reshape(tokens, heads, dim)
    for h in range(heads):
        assert np.array_equal(out[0, h], v.reshape(tokens, kv_heads, dim)[0, h // 2])
    # one dominant key: q . k_3 / sqrt(dim) exceeds the others by ~1000, so the output is v_3
    k = np.zeros(tokens * kv_heads * dim)
    k.reshape(tokens, kv_heads, dim)[3] = 1.0
    q1 = np.full(tokens * heads * dim, 1000.0 * np.sqrt(dim) / dim)
    out = O.attention(q1, k, v, tokens, heads, kv_heads, dim).reshape(tokens, heads, dim)
    assert np.allclose(out, v.reshape(tokens, kv_heads, dim)[3][[0, 0, 1, 1]][None], atol=1e-12)


# ----------------------------------------------------------------------------------- block oracles

def _np_rms(x, w, d, eps, scale=None, shift=None):
    x = x.reshape(-1, d)
    y = x / np.sqrt((x * x).mean(1, keepdims=True) + eps) * (1.0 + w.astype(np.float64))
    if scale is not None:
        y = y * (1.0 + scale) + shift
    return y.ravel()


def _np_rope(x, tokens, heads, pairs, cos, sin):
    z = x.reshape(tokens, heads, pairs, 2)
    c = cos.reshape(tokens, 1, pairs).astype(np.float64)
    s = sin.reshape(tokens, 1, pairs).astype(np.float64)
    rot = (z[..., 0] + 1j * z[..., 1]) * (c + 1j * s)  # a rotation is a complex multiplication
    return np.stack([rot.real, rot.imag], -1).ravel()


def _np_mm(x, lin, m):
    b, s, n, k = lin
    return (x.reshape(m, k) @ O.e4m3_table()[b].reshape(n, k).T * s).ravel()


class _Cfg:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def _draw_linear(rng, n, k):
    b = rng.integers(0, 254, n * k).astype(np.uint8)
    return (b + (b >= 0x7f)).astype(np.uint8), float(np.float32(rng.uniform(0.001, 0.004))), n, k


def _krea_inputs(rng, cfg, tokens):
    H, M, hd = cfg.hidden, cfg.mlp, cfg.head_dim
    shapes = [(cfg.heads * hd, H), (cfg.kv_heads * hd, H), (cfg.kv_heads * hd, H), (H, H), (H, H), (M, H), (M, H),
              (H, M)]
    lins = [_draw_linear(rng, n, k) for n, k in shapes]
    v = lambda n, s: rng.uniform(-s, s, n).astype(np.float32)  # noqa: E731
    vecs = dict(norm1=v(H, .5), norm2=v(H, .5), norm_q=v(hd, .5), norm_k=v(hd, .5), table=v(6 * H, .3),
                temb=v(6 * H, .3))
    pos = O.rope_positions(3, 2, (tokens - 3) // 2, 3)
    cos, sin, _ = O.rope_tables(pos, [4, 6, 6], 1000.0)
    return lins, vecs, cos, sin, rng.uniform(-2, 2, tokens * H)


def test_krea_block_oracle_matches_numpy_composition():  # tests/gpu/block.test.ts:60-100
    cfg = _Cfg(hidden=64, mlp=96, heads=4, kv_heads=2, head_dim=16, eps=1e-5)
    tokens, H, hd = 9, 64, 16
    rng = np.random.default_rng(1)
    lins, vc, cos, sin, x = _krea_inputs(rng, cfg, tokens)
    got = O.krea_block(cfg, tokens, x, lins, vc["norm1"], vc["norm2"], vc["norm_q"], vc["norm_k"], vc["table"],
                       vc["temb"], cos, sin)
    mod = (vc["temb"].astype(np.float64) + vc["table"]).reshape(6, H)
    h = _np_rms(x, vc["norm1"], H, cfg.eps, mod[0], mod[1])
    q = _np_rope(_np_rms(_np_mm(h, lins[0], tokens), vc["norm_q"], hd, cfg.eps), tokens, 4, hd // 2, cos, sin)
    k = _np_rope(_np_rms(_np_mm(h, lins[1], tokens), vc["norm_k"], hd, cfg.eps), tokens, 2, hd // 2, cos, sin)
    v = _np_mm(h, lins[2], tokens)
    g = _np_mm(h, lins[3], tokens)
    o = _attention_numpy(q, k, v, tokens, 4, 2, hd, False) / (1 + np.exp(-g))
    x1 = x + np.tile(mod[2], tokens) * _np_mm(o, lins[4], tokens)
    h2 = _np_rms(x1, vc["norm2"], H, cfg.eps, mod[3], mod[4])
    gg, uu = _np_mm(h2, lins[5], tokens), _np_mm(h2, lins[6], tokens)
    want = x1 + np.tile(mod[5], tokens) * _np_mm(gg / (1 + np.exp(-gg)) * uu, lins[7], tokens)
    assert np.abs(got - want).max() < 1e-10 * np.abs(want).max()
    # zero gates (table = -temb on the gate rows): the block is the identity
    table = vc["table"].copy().reshape(6, H)
    table[2], table[5] = -vc["temb"].reshape(6, H)[2], -vc["temb"].reshape(6, H)[5]
    same = O.krea_block(cfg, tokens, x, lins, vc["norm1"], vc["norm2"], vc["norm_q"], vc["norm_k"], table.ravel(),
                        vc["temb"], cos, sin)
    assert np.array_equal(same, x)


def _double_inputs(rng, cfg):
    H, M, hd = cfg.hidden, cfg.mlp, cfg.head_dim
    v = lambda n, s: rng.uniform(-s, s, n).astype(np.float32)  # noqa: E731
    return [dict(qkv=_draw_linear(rng, 3 * H, H), proj=_draw_linear(rng, H, H), up=_draw_linear(rng, M, H),
                 down=_draw_linear(rng, H, M), norm1=v(H, .5), norm2=v(H, .5), norm_q=v(hd, .5), norm_k=v(hd, .5),
                 table=v(6 * H, .3)) for _ in range(2)]


def test_double_block_oracle_matches_numpy_composition():
    cfg = _Cfg(hidden=64, mlp=128, heads=2, kv_heads=2, head_dim=32, eps=1e-6)
    H, hd, heads, tt, rows, cols = 64, 32, 2, 5, 3, 4
    ti = rows * cols
    rng = np.random.default_rng(2)
    wt, wi = _double_inputs(rng, cfg)
    tvec = rng.uniform(-.3, .3, 6 * H).astype(np.float32)
    cos, sin, _ = O.rope_tables(O.rope_positions(0, rows, cols, 2), [16, 16], 10000.0)
    xt, xi = rng.uniform(-2, 2, tt * H), rng.uniform(-2, 2, ti * H)
    got_t, got_i = O.double_block(cfg, tt, ti, xt, xi, wt, wi, tvec, cos, sin)
    qs, ks, vs, mods = [], [], [], []
    for w, x, n, rot in ((wt, xt, tt, False), (wi, xi, ti, True)):
        mod = (tvec.astype(np.float64) + w["table"]).reshape(6, H)
        mods.append(mod)
        qkv = _np_mm(_np_rms(x, w["norm1"], H, cfg.eps, mod[0], mod[1]), w["qkv"], n).reshape(n, 3, H)
        q = _np_rms(qkv[:, 0].ravel(), w["norm_q"], hd, cfg.eps)
        k = _np_rms(qkv[:, 1].ravel(), w["norm_k"], hd, cfg.eps)
        if rot:
            q, k = _np_rope(q, n, heads, hd // 2, cos, sin), _np_rope(k, n, heads, hd // 2, cos, sin)
        qs.append(q)
        ks.append(k)
        vs.append(qkv[:, 2].ravel())
    o = _attention_numpy(np.concatenate(qs), np.concatenate(ks), np.concatenate(vs), tt + ti, heads, heads, hd,
                         False).reshape(tt + ti, H)
    gelu = lambda u: 0.5 * u * (1 + np.tanh(np.sqrt(2 / np.pi) * (u + 0.044715 * u ** 3)))  # noqa: E731
    for w, x, n, r0, mod, got in ((wt, xt, tt, 0, mods[0], got_t), (wi, xi, ti, tt, mods[1], got_i)):
        x1 = x + np.tile(mod[2], n) * _np_mm(o[r0:r0 + n].ravel(), w["proj"], n)
        h2 = _np_rms(x1, w["norm2"], H, cfg.eps, mod[3], mod[4])
        want = x1 + np.tile(mod[5], n) * _np_mm(gelu(_np_mm(h2, w["up"], n)), w["down"], n)
        assert np.abs(got - want).max() < 1e-10 * np.abs(want).max()
    # the streams meet only in attention: new image MLP weights leave the text output unchanged
    wi2 = dict(wi, up=_draw_linear(rng, cfg.mlp, H))
    got_t2, got_i2 = O.double_block(cfg, tt, ti, xt, xi, wt, wi2, tvec, cos, sin)
    assert np.array_equal(got_t2, got_t) and not np.array_equal(got_i2, got_i)


def test_double_block_rows_equal_the_oracle_rows():
    """The sampled-row composition (used to check the full 512 + 4096-token block on the GPU) equals
    or_double_block_f64 on every row it is asked for, text and image, including first and last rows."""
    cfg = _Cfg(hidden=64, mlp=128, heads=2, kv_heads=2, head_dim=32, eps=1e-6)
    H, tt, rows, cols = 64, 5, 3, 4
    ti = rows * cols
    rng = np.random.default_rng(4)
    wt, wi = _double_inputs(rng, cfg)
    tvec = rng.uniform(-.3, .3, 6 * H).astype(np.float32)
    cos, sin, _ = O.rope_tables(O.rope_positions(0, rows, cols, 2), [16, 16], 10000.0)
    xt, xi = rng.uniform(-2, 2, tt * H), rng.uniform(-2, 2, ti * H)
    full_t, full_i = O.double_block(cfg, tt, ti, xt, xi, wt, wi, tvec, cos, sin)
    rt, ri = [0, 3, 4], [0, 5, 7, 11]
    got_t, got_i = O.double_block_rows(cfg, tt, ti, xt, xi, wt, wi, tvec, cos, sin, rt, ri)
    want_t, want_i = full_t.reshape(tt, H)[rt], full_i.reshape(ti, H)[ri]
    assert np.abs(got_t - want_t).max() < 1e-10 * np.abs(want_t).max()
    assert np.abs(got_i - want_i).max() < 1e-10 * np.abs(want_i).max()
    # a rotation left out of the image keys cannot pass
    no_rope = O.double_block_rows(cfg, tt, ti, xt, xi, wt, wi, tvec, np.ones_like(cos), np.zeros_like(sin), rt, ri)
    assert np.abs(no_rope[1] - want_i).max() > 1e-3 * np.abs(want_i).max()


def test_rmsnorm_oracle_matches_torch_golden():
    """or_rmsnorm_f64 against torch.nn.functional.rms_norm (tests/golden/rmsnorm.json, written by make_golden.py
    without the oracle): plain (offset 0 and 1) and Krea-modulated rows, d from 7 to 512, eps 1e-5 and 1e-6."""
    for c in load("rmsnorm.json")["cases"]:
        x, w = np.array(c["x"], np.float32), np.array(c["weight"], np.float32)
        sc, sh = np.array(c["scale"], np.float32), np.array(c["shift"], np.float32)
        got = O.rmsnorm(x, w, c["eps"], c["offset"], sc if c["modulated"] else None, sh if c["modulated"] else None)
        want = np.array(c["out"])
        assert np.abs(got - want).max() < 1e-12 * np.abs(want).max(), (c["rows"], c["d"])
        # a dropped offset or eps cannot pass
        assert np.abs(O.rmsnorm(x, w, c["eps"], 1.0 - c["offset"], sc if c["modulated"] else None,
                                sh if c["modulated"] else None) - want).max() > 1e-3


def _direct_conv3x3(x, weight, h, w, cin, cout):
    """tests/gpu/image.test.ts:16-28: the direct 3x3 convolution with zero padding, channel-last, in float64."""
    xi = x.astype(np.float64).reshape(h, w, cin)
    wt = weight.astype(np.float64).reshape(cout, 3, 3, cin)
    pad = np.zeros((h + 2, w + 2, cin))
    pad[1:-1, 1:-1] = xi
    out = np.zeros((h, w, cout))
    for ky in range(3):
        for kx in range(3):
            out += pad[ky:ky + h, kx:kx + w] @ wt[:, ky, kx, :].T
    return out.ravel()


def test_conv3x3_input_mode_equals_the_direct_convolution():
    """The im2col addressing of the conv3x3 input (src/kernels/matmul.ts:74-83) through the oracle's GEMM equals
    a direct convolution, on the reference test's data (tests/gpu/image.test.ts:11-30: LCG seed 5, x then weight,
    values 2u - 1 as f32) and on a larger ragged case; the params carry the reference's check."""
    h, w, cin, cout = 5, 7, 8, 12
    u = O.lcg(5, h * w * cin + cout * 9 * cin)
    x = (u[: h * w * cin] * 2 - 1).astype(np.float32)
    wt = (u[h * w * cin:] * 2 - 1).astype(np.float32)
    got = O.matmul(O.conv3x3_params(h, w, cin, cout), O.F32, x, O.F32, wt)
    assert np.abs(got - _direct_conv3x3(x, wt, h, w, cin, cout)).max() < 1e-12
    rng = np.random.default_rng(4)
    h, w, cin, cout = 9, 13, 12, 20
    x = rng.standard_normal(h * w * cin).astype(np.float32)
    wt = rng.standard_normal(cout * 9 * cin).astype(np.float32)
    got = O.matmul(O.conv3x3_params(h, w, cin, cout), O.F32, x, O.F32, wt)
    assert np.abs(got - _direct_conv3x3(x, wt, h, w, cin, cout)).max() < 1e-10
    # a mistake check: the taps are (ky, kx) = (tap / 3, tap % 3), not transposed
    wrong = _direct_conv3x3(x, wt.reshape(cout, 3, 3, cin).transpose(0, 2, 1, 3).copy(), h, w, cin, cout)
    assert np.abs(got - wrong).max() > 1.0
    with pytest.raises(ValueError, match="cin must be a multiple of 4, got 6"):
        O.conv3x3_params(4, 4, 6, 8)

"""Dequantization kernels on the GPU, bit-exact against the oracle.
Mirrors tests/gpu/fp8.test.ts:21-37 (unpackFp8) and pins the int4 format (no reference counterpart)."""
import numpy as np
import pytest

import oracle_lib as O
import we

pytestmark = pytest.mark.gpu


def test_unpack_every_byte_exactly(graph):  # tests/gpu/fp8.test.ts:21-28
    allb = np.arange(256, dtype=np.uint8)
    got = we.unpack_fp8(graph, allb, 1.0)
    want = O.unpack_fp8(allb, 1.0)  # the shader formula: NaN codes decode to +-480
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    cpu = O.e4m3_table()
    ok = ~np.isnan(cpu)
    assert np.array_equal(got[ok].astype(np.float64), cpu[ok])
    assert got[0x7F] == 480.0 and got[0xFF] == -480.0


def test_unpack_applies_scale_and_handles_odd_length(graph):  # tests/gpu/fp8.test.ts:30-37
    s = 0.0018833705689758062
    got = we.unpack_fp8(graph, np.array([0x38, 0xC0, 0x7E], np.uint8), s)
    assert np.array_equal(got, np.array([1, -2, 448], np.float32) * np.float32(s))
    assert we.unpack_fp8(graph, np.array([0x38] * 4 + [0x40], np.uint8), 1.0).tolist() == [1, 1, 1, 1, 2]


def test_unpack_large_random(graph):
    rng = np.random.default_rng(3)
    data = rng.integers(0, 256, 1 << 20, dtype=np.uint8)
    got = we.unpack_fp8(graph, data, 0.02)
    assert np.array_equal(got.view(np.uint32), O.unpack_fp8(data, 0.02).view(np.uint32))


@pytest.mark.parametrize("rows,k,group", [(3, 64, 64), (17, 256, 64), (5, 384, 128), (2, 96, 32)])
def test_int4_dequant_bit_exact(graph, rows, k, group):
    rng = np.random.default_rng(rows * k)
    words = rng.integers(0, 2 ** 32, rows * k // 8, dtype=np.uint64).astype(np.uint32)
    scales = np.abs(rng.normal(0, 0.01, rows * k // group)).astype(np.float16).view(np.uint16)
    scales[0] = 0x3C00  # 1.0: the raw codes -8..7
    wb, sb = graph.buffer(words), graph.buffer(scales)
    out = graph.buffer(rows * k * 4)
    graph.dequant_int4_raw(wb, sb, rows, k, group, out)
    got = graph.read(out, dtype=np.float32, count=rows * k)
    want = O.dequant_int4(words, scales, rows, k, group)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---- the GEMM's own fp8 decode (tests/gpu/fp8.test.ts:21-28 checks every byte through e4m3_to_f32, the function
# matmulWgsl inlines, src/kernels/matmul.ts:40-47). x is the identity, so y[r, c] = 1.0 * decode(W[c, r]) * 1.0
# with one nonzero product per output: the f32 result is the decoded byte itself, whatever the summation order.
# Every column of W holds all 256 byte values (twice), so every tile, wave and lane position sees every code.
ONE_HOT_K, ONE_HOT_N = 512, 256


def _one_hot_gemm(graph, tune, x_dt, cfg, w, splitk=None):
    k, n = ONE_HOT_K, ONE_HOT_N
    if x_dt == we.F32:  # f32 x runs as three bf16 planes (1.0, 0, 0) over 3K with the weights repeating every K
        x = np.eye(k, dtype=np.float32)
    else:
        x = np.zeros((k, k), np.uint16)
        x[np.arange(k), np.arange(k)] = 0x3F80 if x_dt == we.BF16 else 0x3C00  # 1.0 as bf16 / f16
    tune(gemm_cfg=cfg)
    if splitk is not None:
        tune(gemm_splitk=splitk)
    p = we.matmul_params(k, n, k, 1.0, graph=graph)
    mark = graph.mark()
    y = graph.buffer(k * n * 4)
    graph.matmul(p, x_dt, graph.buffer(x.ravel()), we.FP8, graph.buffer(w.ravel()), we.F32, y)
    got = graph.read(y, dtype=np.float32, count=k * n).reshape(k, n)
    graph.release(mark)
    return got


def _codes(with_nan):
    k, n = ONE_HOT_K, ONE_HOT_N
    w = ((np.arange(k)[None, :] + 7 * np.arange(n)[:, None]) % 256).astype(np.uint8)  # W [N, K]
    if not with_nan:
        w[(w & 0x7F) == 0x7F] -= 1  # 0x7f -> 0x7e, 0xff -> 0xfe: the finite codes only
    return w


@pytest.mark.parametrize("with_nan", [False, True])
@pytest.mark.parametrize("x_dt", [we.BF16, we.F16, we.F32])
@pytest.mark.parametrize("cfg", [0, 1, 2, 3, 4, 5])
def test_gemm_fp8_decode_every_byte_exactly(graph, tune, cfg, x_dt, with_nan):
    """Every byte through the fast GEMM's in-register decode, in every tile configuration (0 256x256 and 5 256x192
    ping-pong, 1 256x128, 2 128x128, 3 64x64, 4 32x64), bit for bit against the shader formula
    (src/kernels/fp8.ts:12-20). Without 0x7f / 0xff the hardware converter decodes all 254 finite codes, the
    subnormals 0x01-0x07 and 0x81-0x87 included; with them, the waves that meet a NaN recompute with the shader's
    decoding, which must give +-480 and every other code unchanged. f32 x takes the plane path (the weights read
    at k mod K, in the main loop and in the recompute)."""
    w = _codes(with_nan)
    got = _one_hot_gemm(graph, tune, x_dt, cfg, w)
    want = O.e4m3_gpu_table()[w.T]  # [K, N]: y[r, c] = decode(W[c, r])
    assert np.array_equal(got, want), (cfg, x_dt, with_nan, np.argwhere(got != want)[:5])
    if with_nan:
        assert (got[w.T == 0x7F] == 480.0).all() and (got[w.T == 0xFF] == -480.0).all()
    else:
        cpu = O.e4m3_table()[w.T]  # the CPU decoder of src/weights/fp8.ts:4-11 (no NaN codes here)
        assert np.array_equal(got.astype(np.float64), cpu)
        assert set(np.unique(w)) == set(range(256)) - {0x7F, 0xFF}


@pytest.mark.parametrize("with_nan", [False, True])
@pytest.mark.parametrize("cfg,slices", [(3, 4), (4, 8), (2, 2)])
def test_gemm_fp8_decode_every_byte_through_split_k(graph, tune, cfg, slices, with_nan):
    """The same through a split-K slice plan (slices of K in separate workgroups, raw f32 partial sums, the reduce
    pass adding them in slice order): still exactly the decoded byte."""
    w = _codes(with_nan)
    got = _one_hot_gemm(graph, tune, we.BF16, cfg, w, splitk=slices)
    want = O.e4m3_gpu_table()[w.T]
    assert np.array_equal(got, want), (cfg, slices, with_nan, np.argwhere(got != want)[:5])


def test_gemm_fp8_nan_codes_in_one_column_leave_other_waves_on_the_converter(graph, tune):
    """NaN codes confined to one column send only the waves holding that column through the recompute; the other
    waves' hardware decode and the recomputed values meet in one output, each exactly the shader's value."""
    w = _codes(False)
    w[37, 5], w[37, 300] = 0x7F, 0xFF
    for cfg in (0, 2, 5):
        got = _one_hot_gemm(graph, tune, we.BF16, cfg, w)
        want = O.e4m3_gpu_table()[w.T]
        assert np.array_equal(got, want), cfg
        assert got[5, 37] == 480.0 and got[300, 37] == -480.0

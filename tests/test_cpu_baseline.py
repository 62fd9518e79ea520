"""The strong CPU baseline bench.py times (oracle/cpu_gemm.c: all threads, f32 accumulation, AVX-512 when the
host has it) computes the same product as the faithful float64 loop of tests/gpu/matmul.test.ts:26-35
(or_matmul_f64): every weight dtype, ragged M / N / K (tails of the 6-row strip, the 64-column block and the
128-k block), 16-bit outputs, one and several threads, the AVX-512 and portable strips."""
import numpy as np
import pytest

import oracle_lib as O


def _data(rng, m, n, k, x_dt, w_dt, group):
    x = rng.standard_normal(m * k).astype(np.float32)
    if x_dt == O.F16:
        x = x.astype(np.float16).view(np.uint16)
    elif x_dt == O.BF16:
        x = (x.view(np.uint32) >> 16).astype(np.uint16)
    scales = None
    if w_dt == O.FP8:
        w = rng.choice(np.setdiff1d(np.arange(256), [0x7F, 0xFF]), n * k).astype(np.uint8)
    elif w_dt == O.BF16:
        w = (rng.standard_normal(n * k).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    elif w_dt == O.F16:
        w = rng.standard_normal(n * k).astype(np.float16).view(np.uint16)
    elif w_dt == O.INT4:
        w = rng.integers(0, 2 ** 32, n * k // 8, dtype=np.uint64).astype(np.uint32)
        scales = np.abs(rng.normal(0, 0.01, n * k // group)).astype(np.float16).view(np.uint16)
    else:
        w = rng.standard_normal(n * k).astype(np.float32)
    return x, w, scales


@pytest.mark.parametrize("m,n,k,x_dt,w_dt", [
    (7, 70, 200, O.F32, O.FP8), (6, 64, 256, O.BF16, O.FP8), (13, 130, 520, O.F16, O.BF16),
    (1, 33, 192, O.F16, O.INT4), (16, 100, 640, O.F16, O.INT4), (5, 17, 12, O.F32, O.F32), (64, 65, 300, O.F16, O.F16),
])
@pytest.mark.parametrize("threads,avx512", [(1, True), (3, True), (2, False)])
def test_matches_the_float64_loop(m, n, k, x_dt, w_dt, threads, avx512):
    rng = np.random.default_rng(m * 1000 + n + k)
    group = 64 if w_dt == O.INT4 else 0
    x, w, scales = _data(rng, m, n, k, x_dt, w_dt, group)
    want = O.matmul(O.matmul_params(m, n, k, 0.02), x_dt, x, w_dt, w, scales=scales, group=group)
    got = O.cpu_matmul(m, n, k, 0.02, x_dt, x, w_dt, w, scales, group, O.F32, threads, avx512).astype(np.float64)
    # f32 accumulation over K terms against float64: relative to the row's scale of values
    assert np.abs(got - want).max() <= 2e-6 * np.sqrt(k) * np.abs(want).max()


def test_16_bit_outputs_are_the_rounded_f32_result():
    rng = np.random.default_rng(5)
    m, n, k = 9, 80, 300
    x, w, _ = _data(rng, m, n, k, O.F16, O.FP8, 0)
    f32 = O.cpu_matmul(m, n, k, 0.02, O.F16, x, O.FP8, w, threads=2)
    for dt, conv in ((O.F16, O.lib.or_f32_to_f16), (O.BF16, O.lib.or_f32_to_bf16)):
        got = O.cpu_matmul(m, n, k, 0.02, O.F16, x, O.FP8, w, y_dtype=dt, threads=2)
        assert got.tolist() == [conv(float(v)) for v in f32]


def test_gelu_epilogue_is_gelu_of_the_product():
    rng = np.random.default_rng(8)
    m, n, k = 7, 90, 260
    x, w, _ = _data(rng, m, n, k, O.BF16, O.FP8, 0)
    v = O.cpu_matmul(m, n, k, 0.05, O.BF16, x, O.FP8, w, threads=2).astype(np.float64)
    got = O.cpu_matmul(m, n, k, 0.05, O.BF16, x, O.FP8, w, threads=2, gelu=True).astype(np.float64)
    want = np.array([O.lib.or_gelu_tanh(t) for t in v])
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


def test_avx512_and_portable_strips_agree():
    if not O.lib.cb_has_avx512():
        pytest.skip("host has no AVX-512")
    rng = np.random.default_rng(6)
    m, n, k = 11, 129, 513
    x, w, _ = _data(rng, m, n, k, O.BF16, O.FP8, 0)
    a = O.cpu_matmul(m, n, k, 0.5, O.BF16, x, O.FP8, w, threads=2, avx512=True)
    b = O.cpu_matmul(m, n, k, 0.5, O.BF16, x, O.FP8, w, threads=2, avx512=False)
    assert np.abs(a - b).max() <= 1e-5 * np.abs(b).max()


def test_refuses_bad_arguments():
    with pytest.raises(ValueError):
        O.cpu_matmul(2, 8, 100, 1.0, O.F16, np.zeros(200, np.uint16), O.INT4, np.zeros(100, np.uint32),
                     np.zeros(16, np.uint16), 64)  # K not a multiple of the group

"""int4-weight GEMV / skinny GEMM on the GPU against the float64 oracle.

The reference has no int4 code (its matmul takes fp8 / bf16 / f32), so this format is pinned by the
oracle's definition, itself checked against a numpy brute force in test_oracle.py. Tolerance: f32 output
1e-5 (the reference's bar), f16 output 2e-3 (one f16 rounding of the value)."""
import numpy as np
import pytest

import oracle_lib as O
import we

pytestmark = pytest.mark.gpu


def make(rng, m, n, k, group, x_dt=we.F16):
    words = rng.integers(0, 2 ** 32, n * k // 8, dtype=np.uint64).astype(np.uint32)
    scales = np.abs(rng.normal(0, 0.01, n * k // group)).astype(np.float16).view(np.uint16)
    x32 = rng.standard_normal(m * k).astype(np.float32)
    if x_dt == we.F16:
        x = x32.astype(np.float16).view(np.uint16)
        ox = O.F16
    elif x_dt == we.BF16:
        x = O.bf16_rne(x32)
        ox = O.BF16
    else:
        x = x32
        ox = O.F32
    return words, scales, x, ox


def run(graph, m, n, k, group, words, scales, x, x_dt, y_dt, bias=None, flags=0, scale=1.0):
    mark = graph.mark()
    wb, sb, xb = graph.buffer(words), graph.buffer(scales), graph.buffer(x)
    yb = graph.buffer(m * n * we.ELEM_BYTES[y_dt])
    bb = graph.buffer(np.asarray(bias, np.float32)) if bias is not None else None
    graph.matmul(we.matmul_params(m, n, k, scale, graph=graph), x_dt, xb, we.INT4, wb, y_dt, yb, scales=sb,
                 group=group, bias=bb, flags=flags)
    raw = graph.read(yb)
    graph.release(mark)
    if y_dt == we.F32:
        return raw.view(np.float32).astype(np.float64)
    if y_dt == we.F16:
        return raw.view(np.float16).astype(np.float64)
    return O.bf16_to_f32(raw.view(np.uint16)).astype(np.float64)


@pytest.mark.parametrize("m", [1, 8, 16])
def test_qwen2_decode_shape_full(graph, m):
    """The decode shape K = 3584, N = 18944, group 64, every output checked."""
    n, k, group = 18944, 3584, 64
    rng = np.random.default_rng(m)
    words, scales, x, ox = make(rng, m, n, k, group)
    got = run(graph, m, n, k, group, words, scales, x, we.F16, we.F16)
    want = O.matmul(O.matmul_params(m, n, k, 1.0), ox, x, O.INT4, words, scales=scales, group=group)
    assert O.rel_error(got, want) < 2e-3
    got32 = run(graph, m, n, k, group, words, scales, x, we.F16, we.F32)
    assert O.rel_error(got32, want) < 1e-5


@pytest.mark.parametrize("m,n,k,group,x_dt", [(1, 40, 128, 64, we.F16), (1, 100, 1024, 128, we.F16),
                                              (1, 37, 4096, 64, we.F16), (1, 50, 576, 64, we.F16),
                                              (1, 24, 640, 320, we.F16), (3, 33, 192, 64, we.F16),
                                              (32, 64, 256, 128, we.F16), (33, 70, 320, 64, we.F16),
                                              (70, 31, 128, 64, we.F16), (5, 64, 256, 64, we.BF16),
                                              (9, 50, 192, 64, we.F32)])
def test_small_and_ragged(graph, m, n, k, group, x_dt):
    rng = np.random.default_rng(m * 1000 + n)
    words, scales, x, ox = make(rng, m, n, k, group, x_dt)
    got = run(graph, m, n, k, group, words, scales, x, x_dt, we.F32)
    want = O.matmul(O.matmul_params(m, n, k, 1.0), ox, x, O.INT4, words, scales=scales, group=group)
    assert O.rel_error(got, want) < 1e-5


def test_every_code_and_epilogue(graph):
    m, n, k, group = 2, 16, 64, 64
    # row j of W holds code (j - 8) everywhere; x = 1 in row 0, 2 in row 1 -> y = 64 * code * s * x
    words = np.repeat(np.array([(((j - 8) & 0xF) * 0x11111111) for j in range(16)], np.uint32), k // 8)
    scales = np.full(n, 0x3C00, np.uint16)  # 1.0
    x = np.concatenate([np.ones(k), 2 * np.ones(k)]).astype(np.float16).view(np.uint16)
    got = run(graph, m, n, k, group, words, scales, x, we.F16, we.F32).reshape(m, n)
    codes = np.arange(16) - 8
    assert np.array_equal(got[0], 64.0 * codes) and np.array_equal(got[1], 128.0 * codes)
    bias = np.arange(n, dtype=np.float32)
    got = run(graph, m, n, k, group, words, scales, x, we.F16, we.F32, bias=bias, flags=we.EPI_BIAS,
              scale=0.5).reshape(m, n)
    assert np.array_equal(got[0], 32.0 * codes + bias)


def test_refuses_unsupported_layouts(graph):
    wb, sb, xb, yb = graph.buffer(4096), graph.buffer(4096), graph.buffer(4096), graph.buffer(4096)
    with pytest.raises(we.WeError, match="group"):
        graph.matmul(we.matmul_params(1, 8, 96, 1.0, graph=graph), we.F16, xb, we.INT4, wb, we.F32, yb, scales=sb,
                     group=32)
    with pytest.raises(we.WeError, match="split-K"):
        graph.matmul(we.matmul_params(1, 8, 128, 1.0, k_split=2, graph=graph), we.F16, xb, we.INT4, wb, we.F32, yb,
                     scales=sb, group=64, flags=we.EPI_SPLIT_K)


@pytest.mark.parametrize("k", [256, 2048, 2304, 3072, 3584])
def test_decode_kernel_matches_general_kernel(graph, k, tune):
    """M = 1 runs the pipelined decode kernel (x staged in LDS, weights through an LDS ring); it must give
    the general kernel's results at every K, including K whose x staging spans several passes per thread
    and whose blocks span several ring chunks (both sum exact f32 products; only the order inside an MFMA
    may differ, hence the 1e-6 bound)."""
    n = 80
    rng = np.random.default_rng(k)
    words, scales, x, _ = make(rng, 1, n, k, 64)
    fast = run(graph, 1, n, k, 64, words, scales, x, we.F16, we.F32)
    tune(int4_path=1)
    general = run(graph, 1, n, k, 64, words, scales, x, we.F16, we.F32)
    assert O.rel_error(fast, general) < 1e-6


@pytest.mark.parametrize("m,n,k,group,x_dt", [
    (2, 80, 256, 64, we.F16), (8, 100, 2304, 64, we.F16), (16, 64, 3584, 64, we.F16), (13, 200, 4096, 128, we.F16),
    (16, 33, 192, 64, we.BF16), (5, 70, 3072, 256, we.F16), (16, 130, 3584, 64, we.BF16), (1, 96, 1024, 64, we.F16),
    (4, 64, 18944, 512, we.F16), (9, 190, 64, 64, we.F16)])
def test_shared_x_kernel_matches_general_kernel(graph, m, n, k, group, x_dt, tune):
    """2 <= M <= 16 with 16-bit x runs the shared-x kernel (x rows and weights through one LDS ring; 32 columns,
    8 x rows and 8 waves per workgroup for M <= 8, 64 columns, 16 rows and 16 waves above); forced at M = 1 as
    well here, with ragged N, K of one block up to
    18944 and scale groups of 64-512. It must match the oracle and the general kernel (same exact products,
    1e-6 for the summation order)."""
    rng = np.random.default_rng(m * 100 + k)
    words, scales, x, ox = make(rng, m, n, k, group, x_dt)
    want = O.matmul(O.matmul_params(m, n, k, 1.0), ox, x, O.INT4, words, scales=scales, group=group)
    tune(int4_path=1)
    general = run(graph, m, n, k, group, words, scales, x, x_dt, we.F32)
    tune(int4_path=2)
    got = run(graph, m, n, k, group, words, scales, x, x_dt, we.F32)
    assert O.rel_error(got, want) < 1e-5
    assert O.rel_error(got, general) < 1e-6


def test_f32_activations_keep_every_mantissa_bit(graph):
    """f32 x enters the int4 kernel as three bf16 planes whose sum is the f32 value exactly, so each product with a
    code keeps all 24 bits of x. Every code is +1 (nibbles 1) with scale 1.0, and x alternates
    1 + 2^-9 + (r + 1) 2^-20 and -1 in row r, so the large parts cancel and y[r, :] = 32 (2^-9 + (r + 1) 2^-20)
    exactly (every partial sum is exact in f32). The 2^-20 terms lie below the second plane: two planes would give
    32 * 2^-9 in every row, 2e-3 off."""
    m, n, k, group = 4, 16, 64, 64
    words = np.full(n * k // 8, 0x11111111, np.uint32)
    scales = np.full(n * k // group, 0x3C00, np.uint16)
    x = np.empty((m, k), np.float32)
    for r in range(m):
        x[r, 0::2] = np.float32(1 + 2.0 ** -9 + (r + 1) * 2.0 ** -20)
        x[r, 1::2] = -1.0
    assert np.float64(x[0, 0]) == 1 + 2.0 ** -9 + 2.0 ** -20  # exact in f32
    exact = np.repeat([32 * (2.0 ** -9 + (r + 1) * 2.0 ** -20) for r in range(m)], n)
    want = O.matmul(O.matmul_params(m, n, k, 1.0), O.F32, x.ravel(), O.INT4, words, scales=scales, group=group)
    assert np.array_equal(want, exact)
    got = run(graph, m, n, k, group, words, scales, x.ravel(), we.F32, we.F32)
    assert np.array_equal(got, exact), np.abs(got - exact).max()


@pytest.mark.parametrize("m,n,k,group", [(1, 1, 64, 64), (1, 3, 128, 64), (2, 1, 64, 64), (16, 1, 128, 128),
                                         (17, 2, 64, 64), (1, 17, 192, 64)])
def test_tiny_shapes(graph, m, n, k, group):
    """One or a few output columns (most of the kernels' 16-row work units past N), a single scale group, and M
    on both sides of the shared-x kernel's range."""
    rng = np.random.default_rng(m * 10 + n + k)
    words, scales, x, ox = make(rng, m, n, k, group)
    got = run(graph, m, n, k, group, words, scales, x, we.F16, we.F32)
    want = O.matmul(O.matmul_params(m, n, k, 1.0), ox, x, O.INT4, words, scales=scales, group=group)
    assert O.rel_error(got, want) < 1e-5

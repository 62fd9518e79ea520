"""The peak probes (we_peak, we_read_peak; timePeak, src/bench/peak.ts:69-109) compute what they claim: the float
chains reach their exact fixed point, the int8 chains match a CPU emulation of dot4, the MFMA chains are linear in
the iteration count, and the streaming read sums every word of the buffer once."""
import numpy as np
import pytest

import we

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", [we.PEAK_F32, we.PEAK_F16])
def test_float_chains_reach_the_fixed_point(graph, kind):
    # a -> 0.5 a + 0.25 reaches 0.5 exactly; each thread folds 8 chains x 4 values: 16.0
    out = graph.buffer(64 * 8 * 4)
    ops = graph.peak(kind, 8, 200, out)
    assert ops == 8 * 64 * 200 * 64
    assert np.all(graph.read(out).view(np.float32) == 16.0)


def _sdot4(a, b):
    """v_dot4_i32_i8 without clamping: a + sum of the signed byte products (int32 wrap)."""
    s = 0
    for i in range(4):
        x = ((a >> (8 * i)) & 0xFF) - (256 if (a >> (8 * i)) & 0x80 else 0)
        y = ((b >> (8 * i)) & 0xFF) - (256 if (b >> (8 * i)) & 0x80 else 0)
        s += x * y
    return s


def test_int8_chains_match_a_cpu_emulation(graph):
    out = graph.buffer(64 * 2 * 4)
    graph.peak(we.PEAK_I8, 2, 5, out)
    got = graph.read(out).view(np.uint32)
    y = 0x0302FF01
    for tid in range(128):
        total = 0
        for j in range(8):
            a = (tid % 16) + j
            for _ in range(5):
                a = (a + _sdot4(a & 0xFFFFFFFF, y)) & 0xFFFFFFFF
            total = (total + a) & 0xFFFFFFFF
        assert got[tid] == total, tid


def test_mfma_chains_are_linear_in_the_iterations(graph):
    out1, out2 = graph.buffer(256 * 4 * 4), graph.buffer(256 * 4 * 4)
    assert graph.peak(we.PEAK_MFMA_BF16, 4, 3, out1) == 4 * 256 * 3 * 4096
    graph.peak(we.PEAK_MFMA_BF16, 4, 6, out2)
    a, b = graph.read(out1).view(np.float32), graph.read(out2).view(np.float32)
    assert np.all(np.isfinite(a)) and np.all(a > 0)
    assert np.array_equal(2 * a, b)


def test_mfma_on_gemm_like_operands_is_deterministic_and_finite(graph):
    """The MFMA probe on the fp8-weight GEMM's operand statistics: same operation count as the constant-operand
    probe, finite results (random signs keep the sums small), different per thread, the same on a second run, and
    different from the constant-operand probe's."""
    out1, out2, out3 = graph.buffer(256 * 4 * 4), graph.buffer(256 * 4 * 4), graph.buffer(256 * 4 * 4)
    assert graph.peak(we.PEAK_MFMA_BF16_DATA, 4, 19, out1) == 4 * 256 * 19 * 4096  # two groups of 8 and a rest of 3
    graph.peak(we.PEAK_MFMA_BF16_DATA, 4, 19, out2)
    graph.peak(we.PEAK_MFMA_BF16, 4, 19, out3)
    a, b, c = (graph.read(o).view(np.float32) for o in (out1, out2, out3))
    assert np.all(np.isfinite(a)) and np.array_equal(a, b)
    assert len(np.unique(a)) > 900 and not np.array_equal(a, c)


def test_streaming_read_sums_every_word(graph):
    # 64 MB plus a ragged tail (not a whole number of waves' worth)
    words = np.random.default_rng(0).integers(0, 2 ** 32, (64 << 20) // 4 + 4 * 333, dtype=np.uint64).astype(np.uint32)
    buf = graph.buffer(words)
    out = graph.buffer(we.read_peak_out_words(words.nbytes) * 4)
    graph.read_peak(buf, words.nbytes, out)
    got = int(graph.read(out).view(np.uint32).astype(np.uint64).sum()) & 0xFFFFFFFF
    assert got == int(words.astype(np.uint64).sum()) & 0xFFFFFFFF

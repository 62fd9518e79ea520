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

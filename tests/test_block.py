"""CPU checks of the block module's host logic: RoPE positions and tables (src/kernels/rope.ts:14-36) against
the oracle, and the streamed weight layout."""
import numpy as np
import pytest

import block as B
import oracle_lib as O


def test_positions_match_the_oracle():  # tests/rope.test.ts:4-17
    assert np.array_equal(B.positions(3, 2, 3), O.rope_positions(3, 2, 3, 3))
    assert np.array_equal(B.positions(0, 64, 64)[:, 1:], O.rope_positions(0, 64, 64, 2))


@pytest.mark.parametrize("axes,theta", [([32, 48, 48], 1000.0), ([4, 6, 6], 1000.0), ([64, 64], 10000.0)])
def test_rope_tables_match_the_oracle(axes, theta):  # tests/rope.test.ts:19-39
    pos = B.positions(5, 7, 9)[:, -len(axes):] if len(axes) == 2 else B.positions(5, 7, 9)
    cos, sin, pairs = B.rope_tables(pos, axes, theta)
    ocos, osin, opairs = O.rope_tables(pos, axes, theta)
    assert pairs == opairs
    assert np.abs(cos.ravel() - ocos).max() <= 2 ** -23 and np.abs(sin.ravel() - osin).max() <= 2 ** -23
    with pytest.raises(ValueError, match="even number"):
        B.rope_tables(pos, [3] + axes[1:], theta)


def test_stream_layout_is_aligned_and_complete():
    cfg = B.DIT_DOUBLE_BLOCK
    lay = B.StreamLayout(cfg)
    H, M = cfg.hidden, cfg.mlp
    assert lay.fp8_bytes == 2 * (9216 * 3072 + 3072 * 3072 + 2 * 12288 * 3072) == 226_492_416
    ends = 0
    for s, name, off, nbytes in lay.fields:
        assert off % 256 == 0 and off >= ends
        ends = off + nbytes
    assert ends <= lay.nbytes < ends + 256
    assert sum(n for _, name, _, n in lay.fields if name in ("qkv", "proj", "up", "down")) == lay.fp8_bytes
    small = B.StreamLayout(B.BlockConfig(64, 128, 2, 2, 32))
    host = np.zeros(small.nbytes, np.uint8)
    small.fill(host, np.random.default_rng(0))
    for s, name, off, nbytes in small.fields:
        if name in ("qkv", "proj", "up", "down"):
            assert not ((host[off:off + nbytes] & 0x7F) == 0x7F).any()  # no NaN codes
        else:
            v = host[off:off + nbytes].view(np.float32)
            assert np.abs(v).max() <= 0.3 and H * M > 0

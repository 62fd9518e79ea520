"""The fused QKV projection (we_matmul_qk_norm_rope) against the float64 oracle and against the unfused pair.

The q/k path of attend() (src/model/block.ts:53-56) is linear -> per-head RMSNorm -> RoPE. Fused, the norm and
the rotation run in the GEMM's epilogue on head-aligned tiles (256 x 128, 128 x 128); elsewhere the
call runs the GEMM and then the q/k pass (the ping-pong 256 x 256 and 256 x 192 tiles among them). Checks:
  * every tile the epilogue runs on, ragged M, partial RoPE (rows >= rope_from), no RoPE, bias, bf16 / f16 output:
    q / k heads within 2^-7 (bf16) / 2^-9 (f16) of the oracle's norm + rotation of the f64 product, relative to the
    rotated pair's magnitude (at least 1: values are ~1 after the norm), v columns within the GEMM's own bar;
  * which path ran: the fused epilogue normalizes the unrounded f32 value, so it differs in some bits from the
    pair (GEMM rounded to bf16, then the pass), while the fallback (a 256 x 192 tile) equals the pair bit for bit.
"""
import numpy as np
import pytest

import oracle_lib as O
import we

pytestmark = pytest.mark.gpu


def _decode(raw, dt):
    if dt == we.F16:
        return raw.view(np.float16).astype(np.float64)
    if dt == we.BF16:
        return O.bf16_to_f32(raw.view(np.uint16)).astype(np.float64)
    return raw.view(np.float32).astype(np.float64)


CASES = {
    # name: (cfg, m, heads, k, y dtype, rope_from (None: no RoPE), bias)
    "128x128_ragged_partial_rope": (2, 300, 3, 256, we.BF16, 50, False),
    "256x128_f16_bias": (1, 512, 4, 256, we.F16, 0, True),  # K < 512: never a split-K plan
    "fallback_256x256": (0, 512, 4, 256, we.BF16, 0, False),
    "256x128_no_rope": (1, 256, 3, 256, we.BF16, None, False),
    "auto_text_shape": (None, 512, 24, 3072, we.BF16, None, False),
    "fallback_256x192": (5, 300, 3, 256, we.BF16, 50, False),
    "fallback_f32": (None, 130, 2, 128, we.F32, 10, False),
}


@pytest.mark.parametrize("case", list(CASES))
def test_fused_qkv_projection(graph, tune, case):
    cfg, m, heads, k, y_dt, rope_from, with_bias = CASES[case]
    hid = heads * 128
    n = 3 * hid
    rng = np.random.default_rng(len(case))
    x = O.bf16_rne(rng.standard_normal(m * k).astype(np.float32))
    w = rng.integers(0, 254, n * k).astype(np.uint8)
    w = (w + (w >= 0x7F)).astype(np.uint8)
    scale = 0.05
    nq, nk = (rng.uniform(-.3, .3, 128).astype(np.float32) for _ in range(2))
    bias = rng.uniform(-.5, .5, n).astype(np.float32) if with_bias else None
    rot_rows = m - rope_from if rope_from is not None else 0
    cos = rng.uniform(-1, 1, max(rot_rows, 1) * 64).astype(np.float32)
    sin = np.sqrt(1 - cos.astype(np.float64) ** 2).astype(np.float32)
    if cfg is not None:
        tune(gemm_cfg=cfg)
    x_dt = we.BF16
    p = we.matmul_params(m, n, k, scale, graph=graph)
    mark = graph.mark()
    xb, wb, qb, kb = graph.buffer(x), graph.buffer(w), graph.buffer(nq), graph.buffer(nk)
    cb, sb = graph.buffer(cos), graph.buffer(sin)
    bb = graph.buffer(bias) if bias is not None else None
    esz = we.ELEM_BYTES[y_dt]
    fused, pair = graph.buffer(m * n * esz), graph.buffer(m * n * esz)
    rf = rope_from if rope_from is not None else 0
    c_arg, s_arg = (cb, sb) if rope_from is not None else (None, None)
    graph.matmul_qk_norm_rope(p, x_dt, xb, we.FP8, wb, y_dt, fused, heads, heads, 1e-6, 1.0, qb, kb, rf, c_arg, s_arg,
                              bias=bb, flags=we.EPI_BIAS if bias is not None else 0)
    # the unfused pair: GEMM, then the q/k pass over q and k in place
    graph.matmul(p, x_dt, xb, we.FP8, wb, y_dt, pair, bias=bb, flags=we.EPI_BIAS if bias is not None else 0)
    for part, nw in ((0, qb), (1, kb)):
        sl = we.Graph.slice(pair, part * hid * esz, 0)
        graph.qk_norm_rope(m, heads, 128, 1e-6, 1.0, nw, rope_from if rope_from is not None else m, False,
                           c_arg, s_arg, y_dt, sl, sl, x_stride=n, out_stride=n)
    got_raw, pair_raw = graph.read(fused), graph.read(pair)
    graph.release(mark)

    # the oracle on sampled rows (all rows of the small cases): first / last rows, both sides of rope_from, tile edges
    if m * n * k <= 2 ** 28:
        rows = np.arange(m)
    else:
        rows = np.unique(np.concatenate([[0, 1, 127, 128, 255, 256, m - 1], rng.integers(0, m, 17)]))
    op = O.matmul_params(m, n, k, scale)
    v = np.stack([O.matmul_rows(op, O.BF16, x, O.FP8, w, r, r + 1)[r * n:(r + 1) * n] for r in rows])
    if bias is not None:
        v = v + bias.astype(np.float64)
    want = v.copy()
    for part, nw in ((0, nq), (1, nk)):
        heads_v = v[:, part * hid:(part + 1) * hid].reshape(len(rows), heads, 128)
        inv = 1.0 / np.sqrt((heads_v ** 2).mean(axis=2, keepdims=True) + 1e-6)
        normed = heads_v * inv * (1.0 + nw.astype(np.float64))
        if rope_from is not None:
            sel = rows >= rope_from
            t = rows[sel] - rope_from
            c = cos.astype(np.float64).reshape(rot_rows, 64)[t][:, None, :]
            s = sin.astype(np.float64).reshape(rot_rows, 64)[t][:, None, :]
            a, b = normed[sel, :, 0::2].copy(), normed[sel, :, 1::2].copy()
            normed[sel, :, 0::2] = a * c - b * s
            normed[sel, :, 1::2] = b * c + a * s
        want[:, part * hid:(part + 1) * hid] = normed.reshape(len(rows), hid)
    got = _decode(got_raw, y_dt).reshape(m, n)[rows]
    tol = {we.BF16: 2 ** -7, we.F16: 2 ** -9, we.F32: 2e-5}[y_dt]
    qk = slice(0, 2 * hid)
    # the rotation mixes the two values of a pair, so an error relative to one value is bounded by the pair's
    # magnitude sqrt(a^2 + b^2) (the pass rounds the GEMM value before it: two roundings of 2^-9 in bf16)
    wq = want[:, qk]
    mag = np.repeat(np.hypot(wq[:, 0::2], wq[:, 1::2]), 2, axis=1)
    assert np.all(np.abs(got[:, qk] - wq) <= tol * np.maximum(mag, 1.0)), case
    vt = {we.BF16: 1e-2, we.F16: 2e-3, we.F32: 1e-5}[y_dt]
    assert O.rel_error(got[:, 2 * hid:].ravel(), want[:, 2 * hid:].ravel()) < vt, case
    if case.startswith("fallback"):
        assert np.array_equal(got_raw, pair_raw), case
    else:
        assert not np.array_equal(got_raw, pair_raw), case  # the epilogue ran: no rounding before the norm
        assert np.array_equal(got_raw.reshape(m, n * esz)[:, 2 * hid * esz:], pair_raw.reshape(m, n * esz)[:, 2 * hid * esz:])


def test_fused_qkv_refusals(graph):
    p = we.matmul_params(4, 384, 4, 1.0, graph=graph)
    b = graph.buffer(4096)
    with pytest.raises(we.WeError, match="exceed the 384 output columns"):
        graph.matmul_qk_norm_rope(p, we.BF16, b, we.FP8, b, we.BF16, b, 2, 2, 1e-6, 1.0, b, b)
    with pytest.raises(we.WeError, match="takes only WE_EPI_BIAS"):
        graph.matmul_qk_norm_rope(p, we.BF16, b, we.FP8, b, we.BF16, b, 1, 1, 1e-6, 1.0, b, b, flags=we.EPI_GELU)
    with pytest.raises(we.WeError, match="cos and sin go together"):
        graph.matmul_qk_norm_rope(p, we.BF16, b, we.FP8, b, we.BF16, b, 1, 1, 1e-6, 1.0, b, b, 0, b, None)

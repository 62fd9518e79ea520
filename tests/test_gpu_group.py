"""Two GEMMs as one launch (we_matmul_group) against separate calls and the float64 oracle.

The double-stream block's text and image streams project with their own weights but the same N and K; grouped,
the tiles of both run in one launch (full K per tile). Checks:
  * a qualifying pair (16-bit x, fp8 / 16-bit weights, aligned rows) equals two separate calls that use the same
    tile shape (gemm_cfg) with split-K off (gemm_splitk 0), bit for bit, on every epilogue the block uses
    (plain, GELU, bias, gated residual with the residual in place or separate) and on ragged row counts, and is
    within the GEMM's own bar of the f64 oracle (gatedAdd of src/kernels/elementwise.ts:52-58 after the product);
  * the default tile pick for the pair gives the oracle's result too (the block's shapes: 512 + 4096 rows);
  * pairs that do not qualify (f32 x, different K) run as separate calls: bit for bit those calls;
  * refusals come before any launch: a bad item leaves both outputs untouched.
"""
import numpy as np
import pytest

import oracle_lib as O
import we
from test_gpu_matmul import TOL, decode, encode_act, make_weights

pytestmark = pytest.mark.gpu


def _problem(graph, rng, m, n, k, x_dt, w_dt, y_dt, gated, bias, in_place, scale):
    x_store, x_oracle, ox = encode_act(rng.standard_normal(m * k).astype(np.float32), x_dt)
    w_store, w_oracle, ow = make_weights(rng, n, k, w_dt)
    res_vals = O.bf16_rne(rng.standard_normal(m * n).astype(np.float32)).astype(np.float32)
    res_store, res_exact, _ = encode_act(res_vals, y_dt)
    d = {"m": m, "p": we.matmul_params(m, n, k, scale, graph=graph), "x": graph.buffer(x_store),
         "w": graph.buffer(w_store), "oracle": (ox, x_oracle, ow, w_oracle), "scale": scale}
    d["gate"] = rng.uniform(-1.5, 1.5, n).astype(np.float32) if gated else None
    d["bias"] = rng.uniform(-.5, .5, n).astype(np.float32) if bias else None
    d["res0"] = res_store if gated else None
    d["res_vals"] = decode(np.ascontiguousarray(res_store).view(np.uint8), y_dt) if gated else None
    d["in_place"] = in_place
    return d


def _buffers(graph, d, y_dt, n):
    """fresh y (holding the residual when in place) and the item dict for matmul / matmul_group"""
    esz = we.ELEM_BYTES[y_dt]
    y = graph.buffer(d["res0"]) if d["gate"] is not None and d["in_place"] else graph.buffer(d["m"] * n * esz)
    item = {"params": d["p"], "x": d["x"], "w": d["w"], "y": y}
    if d["bias"] is not None:
        item["bias"] = graph.buffer(d["bias"])
    if d["gate"] is not None:
        item["gate"] = graph.buffer(d["gate"])
        item["residual"] = y if d["in_place"] else graph.buffer(d["res0"])
    return item


def _oracle(d, n, k, flags):
    ox, xo, ow, wo = d["oracle"]
    v = O.matmul(O.matmul_params(d["m"], n, k, d["scale"]), ox, xo, ow, wo).reshape(d["m"], n)
    if d["bias"] is not None:
        v = v + d["bias"]
    if flags & we.EPI_GELU:
        v = np.vectorize(O.lib.or_gelu_tanh)(v)
    if d["gate"] is not None:
        v = d["res_vals"].reshape(d["m"], n) + d["gate"].astype(np.float64) * v
    return v.ravel()


CASES = {
    # name: (m0, m1, n, k, x dtype, w dtype, y dtype, flags, gated, bias, in place, cfg)
    "gated_in_place_256x256": (512, 1024, 768, 512, we.BF16, we.FP8, we.BF16, 0, True, False, True, 0),
    "gated_ragged_256x192": (300, 700, 576, 256, we.BF16, we.FP8, we.BF16, 0, True, False, False, 5),
    "gelu_bias_128x128": (130, 512, 384, 256, we.F16, we.FP8, we.F16, we.EPI_GELU | we.EPI_BIAS, False, True, False, 2),
    "plain_bf16_weights_256x128": (256, 512, 512, 320, we.BF16, we.BF16, we.BF16, 0, False, False, False, 1),
    "f32_out_64x64": (64, 200, 256, 128, we.BF16, we.FP8, we.F32, 0, True, False, True, 3),
}


@pytest.mark.parametrize("case", list(CASES))
def test_pair_equals_separate_calls_and_the_oracle(graph, tune, case):
    m0, m1, n, k, x_dt, w_dt, y_dt, flags, gated, bias, in_place, cfg = CASES[case]
    rng = np.random.default_rng(len(case))
    scale = 0.05 if w_dt == we.FP8 else 1.0
    tune(gemm_cfg=cfg, gemm_splitk=0)
    mark = graph.mark()
    probs = [_problem(graph, rng, m, n, k, x_dt, w_dt, y_dt, gated, bias, in_place, scale) for m in (m0, m1)]
    sep = [_buffers(graph, d, y_dt, n) for d in probs]
    grp = [_buffers(graph, d, y_dt, n) for d in probs]
    for it in sep:
        graph.matmul(it["params"], x_dt, it["x"], w_dt, it["w"], y_dt, it["y"], bias=it.get("bias"), flags=flags,
                     gate=it.get("gate"), residual=it.get("residual"))
    graph.matmul_group(grp, x_dt, w_dt, y_dt, flags)
    for d, a, b in zip(probs, sep, grp):
        ra, rb = graph.read(a["y"]), graph.read(b["y"])
        assert np.array_equal(ra, rb), (case, d["m"])
        got = decode(rb, y_dt)
        err = O.rel_error(got, _oracle(d, n, k, flags))
        print(f"[group {case} m={d['m']}] rel error {err:.2e}", flush=True)
        assert err < TOL[y_dt], (case, d["m"], err)
    graph.release(mark)


def test_block_shaped_pair_with_the_default_pick_matches_the_oracle(graph):
    """The block's down projections as one launch: 512 text + 4096 image rows, N = 3072, K = 12288, gated residual
    in place; the oracle on sampled rows of each (first, last, tile boundaries)."""
    n, k = 3072, 12288
    rng = np.random.default_rng(5)
    mark = graph.mark()
    probs = [_problem(graph, rng, m, n, k, we.BF16, we.FP8, we.BF16, True, False, True, 0.01) for m in (512, 4096)]
    items = [_buffers(graph, d, we.BF16, n) for d in probs]
    graph.matmul_group(items, we.BF16, we.FP8, we.BF16)
    for d, it in zip(probs, items):
        got = decode(graph.read(it["y"]), we.BF16).reshape(d["m"], n)
        rows = np.unique(np.array([0, 1, 255, 256, d["m"] - 1, d["m"] // 2]))
        ox, xo, ow, wo = d["oracle"]
        op = O.matmul_params(d["m"], n, k, d["scale"])
        v = np.stack([O.matmul_rows(op, ox, xo, ow, wo, r, r + 1)[r * n:(r + 1) * n] for r in rows])
        want = d["res_vals"].reshape(d["m"], n)[rows] + d["gate"].astype(np.float64) * v
        err = O.rel_error(got[rows].ravel(), want.ravel())
        print(f"[group block down m={d['m']}] rel error {err:.2e}", flush=True)
        assert err < TOL[we.BF16], (d["m"], err)
    graph.release(mark)


@pytest.mark.parametrize("why", ["f32_x", "different_k"])
def test_pairs_that_do_not_qualify_run_as_separate_calls(graph, why):
    rng = np.random.default_rng(3)
    n = 256
    x_dt = we.F32 if why == "f32_x" else we.BF16
    ks = (128, 128) if why == "f32_x" else (128, 256)
    mark = graph.mark()
    probs = [_problem(graph, rng, m, n, kk, x_dt, we.FP8, we.BF16, True, True, False, 0.05)
             for m, kk in zip((96, 160), ks)]
    sep = [_buffers(graph, d, we.BF16, n) for d in probs]
    grp = [_buffers(graph, d, we.BF16, n) for d in probs]
    for it in sep:
        graph.matmul(it["params"], x_dt, it["x"], we.FP8, it["w"], we.BF16, it["y"], bias=it["bias"], flags=we.EPI_BIAS,
                     gate=it["gate"], residual=it["residual"])
    graph.matmul_group(grp, x_dt, we.FP8, we.BF16, we.EPI_BIAS)
    for d, a, b, kk in zip(probs, sep, grp, ks):
        assert np.array_equal(graph.read(a["y"]), graph.read(b["y"])), why
        assert O.rel_error(decode(graph.read(b["y"]), we.BF16), _oracle(d, n, kk, we.EPI_BIAS)) < TOL[we.BF16]
    graph.release(mark)


def test_group_refusals_launch_nothing(graph):
    rng = np.random.default_rng(4)
    mark = graph.mark()
    probs = [_problem(graph, rng, m, 256, 128, we.BF16, we.FP8, we.BF16, False, False, False, 0.05) for m in (64, 128)]
    items = [_buffers(graph, d, we.BF16, 256) for d in probs]
    with pytest.raises(we.WeError, match="holds 1 or 2 GEMMs"):
        graph.matmul_group(items + items[:1], we.BF16, we.FP8, we.BF16)
    with pytest.raises(we.WeError, match="a residual needs a gate"):
        graph.matmul_group([items[0], dict(items[1], residual=items[1]["y"])], we.BF16, we.FP8, we.BF16)
    short = graph.buffer(64)
    with pytest.raises(we.WeError, match="y is too small"):  # the second item's output is too short: the first is not run
        graph.matmul_group([items[0], dict(items[1], y=short)], we.BF16, we.FP8, we.BF16)
    assert not graph.read(items[0]["y"]).any()
    with pytest.raises(we.WeError, match="split-K"):
        graph.matmul_group([dict(items[0], gate=graph.buffer(np.ones(256, np.float32)))], we.BF16, we.FP8, we.BF16,
                           we.EPI_SPLIT_K)
    graph.release(mark)


def test_dependent_pair_runs_in_order(graph):
    """Item 1 reads item 0's output as its x (a chained pair): the paired launch would run both GEMMs' tiles at
    once, so the call runs them in order instead. The result equals two separate calls, and item 1's output is
    the oracle's product of item 0's output (rounded to bf16 as stored) with its own weights."""
    m, n, k = 256, 512, 512  # n == k: item 0's output [m, n] is item 1's x [m, k]
    rng = np.random.default_rng(77)
    x0 = O.bf16_rne(rng.standard_normal(m * k).astype(np.float32))
    w0, w1 = (make_weights(rng, n, k, we.FP8)[0] for _ in range(2))
    p = we.matmul_params(m, n, k, 0.05, graph=graph)
    mark = graph.mark()
    xb, w0b, w1b = graph.buffer(x0), graph.buffer(w0), graph.buffer(w1)
    outs = []
    for grouped in (False, True):
        mid, out = graph.buffer(m * n * 2), graph.buffer(m * n * 2)
        items = [{"params": p, "x": xb, "w": w0b, "y": mid}, {"params": p, "x": mid, "w": w1b, "y": out}]
        if grouped:
            graph.matmul_group(items, we.BF16, we.FP8, we.BF16)
        else:
            for it in items:
                graph.matmul(it["params"], we.BF16, it["x"], we.FP8, it["w"], we.BF16, it["y"])
        outs.append((graph.read(mid), graph.read(out)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    h = outs[1][0].view(np.uint16)
    want = O.matmul(O.matmul_params(m, n, k, 0.05), O.BF16, h, O.FP8, w1)
    assert O.rel_error(decode(outs[1][1], we.BF16), want) < TOL[we.BF16]
    graph.release(mark)


def test_pair_writing_the_other_items_residual_runs_in_order(graph):
    """Item 0's output is item 1's residual (bytes item 1 reads): ordered calls, item 0 first."""
    m, n, k = 256, 512, 256
    rng = np.random.default_rng(78)
    xs = [O.bf16_rne(rng.standard_normal(m * k).astype(np.float32)) for _ in range(2)]
    ws = [make_weights(rng, n, k, we.FP8)[0] for _ in range(2)]
    gate = rng.uniform(-1, 1, n).astype(np.float32)
    p = we.matmul_params(m, n, k, 0.05, graph=graph)
    mark = graph.mark()
    xb = [graph.buffer(x) for x in xs]
    wb = [graph.buffer(w) for w in ws]
    gb = graph.buffer(gate)
    got = []
    for grouped in (False, True):
        y0, y1 = graph.buffer(m * n * 2), graph.buffer(m * n * 2)
        items = [{"params": p, "x": xb[0], "w": wb[0], "y": y0},
                 {"params": p, "x": xb[1], "w": wb[1], "y": y1, "gate": gb, "residual": y0}]
        if grouped:
            graph.matmul_group(items, we.BF16, we.FP8, we.BF16)
        else:
            graph.matmul(p, we.BF16, xb[0], we.FP8, wb[0], we.BF16, y0)
            graph.matmul(p, we.BF16, xb[1], we.FP8, wb[1], we.BF16, y1, gate=gb, residual=y0)
        got.append(graph.read(y1))
    assert np.array_equal(got[0], got[1])
    assert np.abs(decode(got[1], we.BF16)).max() > 0
    graph.release(mark)

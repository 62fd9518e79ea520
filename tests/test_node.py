"""The Node N-API addon (web-engine_amd/node): the binding a TypeScript host of the reference uses.

CPU: the addon loads under `node`, exports one function per entry point of include/we.h, its host logic
(matmulParams image and messages, kSplitFor) equals the oracle's, and index.js readHeader / readTensor read
.safetensors files through the native reader with the reference's messages.
GPU: tests/node_driver.js runs linear (fp8 + bias, fp8 + GELU, fp8 + LoRA, int4), norm, rotate, attention, the
elementwise ops and a pinned-host stream copy through the addon, then the reference's own call shapes:
Graph.run(code, bindings, workgroups) keyed by shader source (linear + addBias, LoRA, split-K + layer sum, norm
with Params from device.queue.writeBuffer, rotate, elementwise with a { buffer, offset, size } binding),
`await graph.device.queue.onSubmittedWorkDone()` and concurrent asynchronous reads; the results are checked here
against the oracle with the bars of the matching C-ABI tests (test_gpu_matmul, test_gpu_int4, test_gpu_norm_rope,
test_gpu_elementwise, test_gpu_attention)."""
import json
import pathlib
import shutil
import subprocess

import numpy as np
import pytest

import oracle_lib as O
import we
from test_gpu_matmul import LcgDraws, lora_reference, rms_rel

ROOT = pathlib.Path(__file__).resolve().parents[1]
NODE_DIR = ROOT / "web-engine_amd" / "node"
ADDON = NODE_DIR / "we_node.node"
NODE = shutil.which("node")

pytestmark = pytest.mark.skipif(NODE is None or not ADDON.exists(),
                                reason="node or the built addon (web-engine_amd/node/we_node.node) is missing")

# include/we.h entry point -> addon export
EXPORTS = {
    "we_ctx_create": "create", "we_ctx_destroy": "destroy", "we_device_info": "deviceInfo", "we_sync": "sync",
    "we_buf_alloc": "bufAlloc", "we_buf_free": "bufFree", "we_buf_upload": "upload", "we_buf_download": "download",
    "we_buf_copy": "copy", "we_mark": "mark", "we_release": "release", "we_stats": "stats",
    "we_host_alloc": "hostAlloc", "we_host_free": "hostFree", "we_host_span": "hostSpan", "we_stream_copy": "streamCopy",
    "we_wait_ticket": "waitTicket", "we_ticket_done": "ticketDone", "we_record_compute": "recordCompute",
    "we_timer_start": "timerStart", "we_timer_stop": "timerStop", "we_matmul_params_make": "matmulParams",
    "we_ksplit_for": "kSplitFor", "we_conv3x3_params": "conv3x3Params", "we_matmul": "matmul", "we_matmul_noalloc": "matmulNoalloc", "we_matmul_gated": "matmulGated", "we_matmul_group": "matmulGroup", "we_matmul_mul": "matmulMul", "we_matmul_qk_norm_rope": "matmulQkNormRope", "we_rmsnorm": "rmsnorm", "we_rmsnorm_mod": "rmsnormMod",
    "we_rope": "rope",
    "we_qk_norm_rope": "qkNormRope", "we_attention": "attention", "we_elementwise": "elementwise", "we_layer_sum": "layerSum",
    "we_unpack_fp8": "unpackFp8", "we_dequant_int4": "dequantInt4", "we_last_error": "lastError",
    "we_graph_begin": "graphBegin", "we_graph_end": "graphEnd", "we_graph_launch": "graphLaunch",
    "we_graph_destroy": "graphDestroy", "we_peak": "peak", "we_read_peak": "readPeak", "we_st_open": "stOpen", "we_st_close": "stClose", "we_st_count": "stCount",
    "we_st_info": "stInfo", "we_st_find": "stFind", "we_st_metadata_count": "stMetadataCount",
    "we_st_metadata_at": "stMetadataAt", "we_st_read": "stRead", "we_stream_select": "streamSelect",
    "we_stream_fork": "streamFork", "we_stream_join": "streamJoin", "we_buf_download_async": "downloadAsync",
    "we_ticket_wait": "waitTicketAsync", "we_record_all": "recordAll", "we_set_alloc_cap": "setAllocCap",
    "we_set_poison": "setPoison", "we_set_tuning": "setTuning", "we_timer_mark": "timerMark",
    "we_timer_between": "timerBetween",
}


def node_eval(script, timeout=60):
    out = subprocess.run([NODE, "-e", script], cwd=NODE_DIR, capture_output=True, text=True, timeout=timeout)
    assert out.returncode == 0, out.stderr
    return json.loads(out.stdout)


def test_addon_exports_every_entry_point():
    assert set(EXPORTS) == set(we.header_functions())
    keys = node_eval('console.log(JSON.stringify(Object.keys(require("./we_node.node"))))')
    assert set(EXPORTS.values()) <= set(keys)


LAYOUTS = [
    dict(m=3, n=5, k=8, scale=0.25),
    dict(m=20, n=20, k=128, scale=1.0, xStride=512, xOffset=256, wStride=256, wOffset=128, yStride=24),
    dict(m=5, n=12, k=200, scale=0.5, kSplit=3),
    dict(m=1, n=1, k=6, scale=1.0),
    dict(m=1, n=1, k=4, scale=1.0, xStride=6),
    dict(m=1, n=1, k=4, scale=1.0, wStride=10),
    dict(m=1, n=1, k=4, scale=1.0, xOffset=1),
    dict(m=1, n=1, k=4, scale=1.0, wOffset=2),
]


def test_matmul_params_image_and_messages_match_the_oracle():  # src/kernels/matmul.ts:198-212
    script = f"""
const we = require("./index.js");
const out = {json.dumps(LAYOUTS)}.map((l) => {{
  try {{ return Array.from(we.matmulParams({{ m: l.m, n: l.n, k: l.k }}, l.scale, l)); }}
  catch (e) {{ return e.message; }}
}});
console.log(JSON.stringify(out));"""
    got = node_eval(script)
    names = dict(xStride="x_stride", wStride="w_stride", yStride="y_stride", xOffset="x_offset", wOffset="w_offset",
                 yOffset="y_offset", kSplit="k_split")
    for layout, g in zip(LAYOUTS, got):
        kw = {names[key]: v for key, v in layout.items() if key in names}
        try:
            p = O.matmul_params(layout["m"], layout["n"], layout["k"], layout["scale"], **kw)
        except ValueError as e:
            assert g == str(e), (layout, g)
            continue
        assert np.frombuffer(bytes(p), np.uint32).tolist() == g, layout


def test_ksplit_for_matches_the_oracle():  # src/model/ops.ts:42-45
    grid = [(m, n, k) for m in (1, 5, 64, 1088, 4160) for n in (4, 64, 300) for k in (64, 1024, 6144, 16384)]
    got = node_eval(f'const a = require("./we_node.node"); '
                    f'console.log(JSON.stringify({json.dumps(grid)}.map(([m, n, k]) => a.kSplitFor(m, n, k))))')
    assert got == [O.ksplit_for(m, n, k) for m, n, k in grid]
    assert got[grid.index((1088, 64, 6144))] == 24 and got[grid.index((4160, 64, 16384))] == 8


def test_context_free_errors_throw_with_the_message():
    got = node_eval('const a = require("./we_node.node"); const r = [];'
                    'try { a.matmul(null, new Uint32Array(13), 0, null, 3, null, null, 0, 0, null, null, 0); }'
                    'catch (e) { r.push(e.message); }'
                    'try { a.bufAlloc(null, 16); } catch (e) { r.push(e.message); }'
                    'console.log(JSON.stringify(r));')
    assert got == ["context is null", "context is null"]


def test_graph_run_table_and_its_errors():
    """registerKernels maps every reference export name it is given; Graph.run refuses an unregistered shader
    and a wrong binding count before touching the device (a Graph without a context is enough here)."""
    got = node_eval('''
const we = require("./index.js");
const ref = { matmulWgsl: (w, i = "rows", { splitK = false, accumulate = false } = {}) => `m ${w} ${splitK} ${accumulate}`,
  rmsnormWgsl: "n", ropeKernel: (p) => `r ${p}`, ropeWgsl: "r interleaved", layerSumWgsl: "l", swigluWgsl: "s",
  conv3x3Wgsl: "c3",
  sigmoidGateWgsl: "sg", gatedAddWgsl: "ga", addBiasWgsl: "ab", geluTanhWgsl: "g", addWgsl: "a", siluWgsl: "si" };
const out = { count: we.registerKernels(ref) };
const g = Object.create(we.Graph.prototype);
try { g.run("unknown\\nsecond line", [], [1]); } catch (e) { out.unknown = e.message; }
try { g.run("n", [null, null], [1]); } catch (e) { out.count6 = e.message; }
try { g.run("ga", [null, null, null, null], [1]); } catch (e) { out.count5 = e.message; }
try { we.registerKernels({ rmsnormWgsl: 3 }); } catch (e) { out.notText = e.message; }
console.log(JSON.stringify(out));''')
    assert got["count"] == 21
    assert got["unknown"].startswith('Graph.run: no MI355X kernel is registered for this shader ("unknown");')
    assert got["count6"] == "Graph.run: rmsnorm takes 6 bindings (Params first), got 2"
    assert got["count5"] == "Graph.run: elementwise takes 5 bindings (Params first), got 4"
    assert got["notText"] == "registerKernels: rmsnormWgsl is not WGSL source text"


def test_type_declarations_cover_the_module():
    """index.d.ts declares exactly what index.js exports, and every Graph method it declares exists."""
    import re
    dts = (NODE_DIR / "index.d.ts").read_text()
    declared = set(re.findall(r"^export (?:const|function|class) (\w+)", dts, re.M))
    body = dts[dts.index("export class Graph {"):]
    body = body[: body.index("\n}\n")]
    methods = set(re.findall(r"^  (?:static )?(\w+)\(", body, re.M)) - {"constructor"}
    got = node_eval('const w = require("./index.js"); const g = Object.create(w.Graph.prototype);'
                    'console.log(JSON.stringify({ keys: Object.keys(w), methods: %s.filter((m) => '
                    'typeof g[m] !== "function" && typeof w.Graph[m] !== "function") }))' % json.dumps(sorted(methods)))
    assert declared == set(got["keys"])
    assert got["methods"] == []
    assert {"run", "read", "onSubmittedWorkDone", "writeBuffer", "buffer", "slice", "copy", "release"} <= methods


def test_safetensors_through_the_addon(tmp_path):
    """readHeader / readTensor from index.js (the native reader) on files written here: tensors, offsets,
    metadata, bytes (whole, limited, into a caller's array) and the reference's error messages and class."""
    import weights as W
    rng = np.random.default_rng(2)
    big = rng.integers(0, 256, 20 * 1024 * 1024 + 7, dtype=np.uint8)
    good = tmp_path / "good.safetensors"
    W.save(good, {"a": ("F8_E4M3", [2, 2], bytes([1, 2, 3, 4])), "b": ("F32", [1], np.float32([1.5]).view(np.uint8)),
                  "big": ("U8", [big.size], big)}, {"format": "pt"})
    bad = tmp_path / "bad.safetensors"
    text = b'{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}}'
    bad.write_bytes(len(text).to_bytes(8, "little") + text + bytes(4))
    got = node_eval(
        'const w = require("./index.js"); const st = w.readHeader(%s); const out = {};'
        'out.tensors = [...st.tensors.values()]; out.metadata = st.metadata;'
        'out.a = Array.from(w.readTensor(st, st.tensors.get("a"))); out.a2 = Array.from(w.readTensor(st, st.tensors.get("a"), 2));'
        'const big = w.readTensor(st, st.tensors.get("big"), undefined, undefined, 8);'
        'let sum = 0; for (let i = 0; i < big.length; i++) sum = (sum * 31 + big[i]) %% 1000000007; out.sum = sum;'
        'const dst = new Uint8Array(4); w.readTensor(st, st.tensors.get("b"), undefined, dst);'
        'out.b = Array.from(new Float32Array(dst.buffer)); st.close();'
        'try { w.readHeader(%s); } catch (e) { out.err = [e.name, e.message, e instanceof w.SafetensorsError]; }'
        'try { w.readHeader(%s); } catch (e) { out.missing = e.name; }'
        'console.log(JSON.stringify(out));' % (json.dumps(str(good)), json.dumps(str(bad)),
                                               json.dumps(str(tmp_path / "absent"))))
    st = W.read_header(good)
    assert got["tensors"] == [dict(name=t.name, dtype=t.dtype, shape=list(t.shape), offset=t.offset, size=t.size, index=i)
                              for i, t in enumerate(st.tensors.values())]
    assert got["metadata"] == {"format": "pt"}
    assert got["a"] == [1, 2, 3, 4] and got["a2"] == [1, 2] and got["b"] == [1.5]
    s = 0
    for v in big.tolist():
        s = (s * 31 + v) % 1000000007
    assert got["sum"] == s
    assert got["err"] == ["SafetensorsError", "a: has 4 bytes, its shape needs 8 bytes", True]
    assert got["missing"] == "Error"


# ------------------------------------------------------------------------------------------------ GPU

def _write(tmp, name, arr):
    np.ascontiguousarray(arr).tofile(tmp / name)
    return name


@pytest.mark.gpu
def test_graph_steps_through_the_addon(tmp_path):
    cases, checks = [], {}
    # fp8 linear + fused bias (tests/gpu/matmul.test.ts shapes; bias as ops.ts:65)
    m, n, k = 37, 70, 100
    x, w = O.matmul_test_data(m, n, k, 1)
    bias = ((O.lcg(5, n) - 0.5) * 4).astype(np.float32)
    base = O.matmul(O.matmul_params(m, n, k, 0.002), O.F32, x, O.FP8, w) + np.tile(bias.astype(np.float64), m)
    wspec = dict(file=_write(tmp_path, "w8", w), dtype="fp8", scale=0.002, n=n, k=k, bias=_write(tmp_path, "b", bias))
    cases.append(dict(name="fp8_bias", op="linear", m=m, x=_write(tmp_path, "x", x), xDtype=we.F32,
                      yDtype=we.F32, w=wspec))
    checks["fp8_bias"] = (np.float32, lambda g: O.rel_error(g, base) < 1e-5)
    gel = np.array([O.lib.or_gelu_tanh(v) for v in base])
    cases.append(dict(cases[-1], name="fp8_gelu", geluTanh=True))
    checks["fp8_gelu"] = (np.float32, lambda g: np.abs(g - gel).max() < 1e-4 * np.abs(gel).max())

    # LoRA on an fp8 linear (tests/gpu/lora.test.ts:40-78)
    m2, n2, k2, r, s = 5, 12, 16, 4, 0.4
    d = LcgDraws(7, m2 * k2 + n2 * k2 + r * k2 + n2 * r)
    x2, w2 = d.floats(m2 * k2), d.fp8(n2 * k2)
    (db, dv), (ub, uv) = d.bf16(r * k2), d.bf16(n2 * r)
    lora_want = lora_reference(x2, O.e4m3_table()[w2], 0.25, dv, uv, s, m2, n2, k2, r)
    lora = dict(down=dict(file=_write(tmp_path, "down", db), dtype="bf16", scale=1.0, n=r, k=k2),
                up=dict(file=_write(tmp_path, "up", ub), dtype="bf16", scale=s, n=n2, k=r))
    cases.append(dict(name="lora", op="linear", m=m2, x=_write(tmp_path, "x2", x2), xDtype=we.F32, yDtype=we.F32,
                      w=dict(file=_write(tmp_path, "w2", w2), dtype="fp8", scale=0.25, n=n2, k=k2, lora=lora)))
    checks["lora"] = (np.float32, lambda g: rms_rel(g, lora_want) < 1e-6)
    bad = dict(down=dict(lora["down"], n=3), up=dict(lora["up"], k=3))
    cases.append(dict(cases[-1], name="lora_rank3", expectError=True, w=dict(cases[-1]["w"], lora=bad)))

    # int4 weights, f16 activations, ragged N (the additive int4 format)
    m3, n3, k3, group = 3, 33, 192, 64
    rng = np.random.default_rng(3)
    words = rng.integers(0, 2 ** 32, n3 * k3 // 8, dtype=np.uint64).astype(np.uint32)
    scales = np.abs(rng.normal(0, 0.01, n3 * k3 // group)).astype(np.float16).view(np.uint16)
    x3 = rng.standard_normal(m3 * k3).astype(np.float16).view(np.uint16)
    i4_want = O.matmul(O.matmul_params(m3, n3, k3, 1.0), O.F16, x3, O.INT4, words, scales=scales, group=group)
    cases.append(dict(name="int4", op="linear", m=m3, x=_write(tmp_path, "x3", x3), xDtype=we.F16, yDtype=we.F32,
                      w=dict(file=_write(tmp_path, "w4", words), dtype="int4", scale=1.0, n=n3, k=k3,
                             scales=_write(tmp_path, "s4", scales), group=group)))
    checks["int4"] = (np.float32, lambda g: O.rel_error(g, i4_want) < 1e-5)

    # norm with modulation (tests/gpu/rmsnorm.test.ts:25-31)
    dn = 6144
    u = O.lcg(1, 6 * dn)
    xn = ((u[: 3 * dn] - 0.5) * 8).astype(np.float32)
    wn = ((u[3 * dn: 4 * dn] - 0.5) * 0.2).astype(np.float32)
    sc = ((u[4 * dn: 5 * dn] - 0.5) * 2).astype(np.float32)
    sh = ((u[5 * dn:] - 0.5) * 2).astype(np.float32)
    norm_want = O.rmsnorm(xn, wn, 1e-5, 1.0, sc, sh)
    cases.append(dict(name="norm", op="norm", rows=3, d=dn, eps=1e-5, offset=1.0, x=_write(tmp_path, "xn", xn),
                      weight=_write(tmp_path, "wn", wn), scale=_write(tmp_path, "sc", sc),
                      shift=_write(tmp_path, "sh", sh)))
    checks["norm"] = (np.float32, lambda g: np.abs(g - norm_want).max() < 1e-5)

    # rotate, interleaved pairs over three axes (tests/gpu/rope.test.ts:5-22)
    heads = 3
    pos = O.rope_positions(2, 3, 4, 3)
    cos, sin, pairs = O.rope_tables(pos, [32, 48, 48], 1000.0)
    tokens = pos.shape[0]
    xr = (O.lcg(1, tokens * heads * 128) * 2 - 1).astype(np.float32)
    rope_want = O.rope_rotate(xr, tokens, heads, pairs, cos, sin)
    cases.append(dict(name="rotate", op="rotate", tokens=tokens, heads=heads, pairs=pairs, pairing="interleaved",
                      x=_write(tmp_path, "xr", xr), cos=_write(tmp_path, "cos", np.asarray(cos, np.float32)),
                      sin=_write(tmp_path, "sin", np.asarray(sin, np.float32))))
    checks["rotate"] = (np.float32, lambda g: np.abs(g - rope_want).max() < 1e-6)

    # attention, causal, grouped kv heads (tests/gpu/attention.test.ts:87-101 shape, f32)
    ta, ha, kva, da = 19, 4, 1, 128
    ua = O.lcg(9, ta * (ha + 2 * kva) * da)
    qa = ((ua[: ta * ha * da] * 2 - 1) * 2).astype(np.float32)
    ka = ((ua[ta * ha * da: ta * (ha + kva) * da] * 2 - 1) * 2).astype(np.float32)
    va = ((ua[ta * (ha + kva) * da:] * 2 - 1) * 2).astype(np.float32)
    att_want = O.attention(qa, ka, va, ta, ha, kva, da, causal=True)
    cases.append(dict(name="attention", op="attention", tokens=ta, heads=ha, kvHeads=kva, dim=da, causal=True,
                      q=_write(tmp_path, "qa", qa), k=_write(tmp_path, "ka", ka), v=_write(tmp_path, "va", va)))
    checks["attention"] = (np.float32, lambda g: np.abs(g - att_want).max() < 1e-5)

    # elementwise (tests/gpu/elementwise.test.ts:15-40)
    ne, de = 1000, 40
    a = ((O.lcg(1, ne) - 0.5) * 16).astype(np.float32)
    b = ((O.lcg(2, ne) - 0.5) * 16).astype(np.float32)
    gg = ((O.lcg(7, de) - 0.5) * 2).astype(np.float32)
    fa, fb, fg = _write(tmp_path, "ea", a), _write(tmp_path, "eb", b), _write(tmp_path, "eg", gg)
    for fn, inputs, sizes, want, tol in [
        ("swiglu", [fa, fb], [ne], O.elementwise(O.SWIGLU, a, b), 1e-4),
        ("sigmoidGate", [fa, fb], [ne], O.elementwise(O.SIGMOID_GATE, a, b), 1e-5),
        ("gatedAdd", [fa, fb, fg], [ne, de], O.elementwise(O.GATED_ADD, a, b, gg, de), 1e-5),
        ("addBias", [fa, fg], [ne, de], O.elementwise(O.ADD_BIAS, a, gg, d=de), 1e-6),
        ("add", [fa, fb], [ne], O.elementwise(O.ADD, a, b), 1e-6),
        ("gelu", [fa], [ne], O.elementwise(O.GELU_TANH, a), 1e-5),
        ("silu", [fa], [ne], O.elementwise(O.SILU, a), 1e-5),
    ]:
        cases.append(dict(name=fn, op="elementwise", fn=fn, inputs=inputs, sizes=sizes))
        checks[fn] = (np.float32, lambda g, want=want, tol=tol: np.abs(g - want).max() <= tol)

    # pinned host memory -> device over the copy stream (src/model/weights.ts:124-129)
    blob = np.random.default_rng(9).integers(0, 256, (1 << 20) + 12, dtype=np.uint8)
    cases.append(dict(name="stream", op="stream", x=_write(tmp_path, "blob", blob)))
    checks["stream"] = (np.uint8, lambda g: np.array_equal(g, blob))

    # the same steps as Graph.run(code, bindings, workgroups) calls keyed by the reference's shader sources
    by_name = {c["name"]: c for c in cases}
    cases.append(dict(by_name["fp8_bias"], name="run_fp8_bias", op="runLinear"))
    checks["run_fp8_bias"] = checks["fp8_bias"]
    cases.append(dict(by_name["lora"], name="run_lora", op="runLinear"))
    checks["run_lora"] = checks["lora"]
    ms, ns, ks = 5, 12, 1024  # kSplitFor(5, 12, 1024) = 4: split-K partials, then the layer sum
    xs = (rng.standard_normal(ms * ks)).astype(np.float32)
    ws = (rng.standard_normal(ns * ks).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    split_want = O.matmul(O.matmul_params(ms, ns, ks, 0.5), O.F32, xs, O.BF16, ws)
    cases.append(dict(name="run_split", op="runNarrow", m=ms, x=_write(tmp_path, "xs", xs),
                      w=dict(file=_write(tmp_path, "ws", ws), dtype="bf16", scale=0.5, n=ns, k=ks)))
    checks["run_split"] = (np.float32, lambda g: O.rel_error(g, split_want) < 1e-5)
    cases.append(dict(by_name["norm"], name="run_norm", op="runNorm"))
    checks["run_norm"] = checks["norm"]
    cases.append(dict(by_name["rotate"], name="run_rotate", op="runRotate"))
    checks["run_rotate"] = checks["rotate"]
    cases.append(dict(name="run_gatedAdd", op="runElementwise", code="gatedAddWgsl", inputs=[fa, fb, fg],
                      sizes=[ne, de], sliceLast=True))
    checks["run_gatedAdd"] = checks["gatedAdd"]
    cases.append(dict(name="run_swiglu", op="runElementwise", code="swigluWgsl", inputs=[fa, fb], sizes=[ne]))
    checks["run_swiglu"] = checks["swiglu"]
    # a 3x3 convolution through Graph.run(conv3x3Wgsl) (tests/gpu/image.test.ts:11-30 data and bar)
    hc, wc, cin, cout = 5, 7, 8, 12
    uc = O.lcg(5, hc * wc * cin + cout * 9 * cin)
    xc = (uc[: hc * wc * cin] * 2 - 1).astype(np.float32)
    wcv = (uc[hc * wc * cin:] * 2 - 1).astype(np.float32)
    conv_want = O.matmul(O.conv3x3_params(hc, wc, cin, cout), O.F32, xc, O.F32, wcv)
    cases.append(dict(name="run_conv", op="runConv", h=hc, w=wc, cin=cin, cout=cout, x=_write(tmp_path, "xc", xc),
                      weight=_write(tmp_path, "wc", wcv)))
    checks["run_conv"] = (np.float32, lambda g: np.abs(g - conv_want).max() < 1e-5)
    cases.append(dict(name="run_unknown", op="runUnknown", expectError=True))

    # two GEMMs as one launch (matmulGroup, we_matmul_group): bf16 x, fp8 weights, f32 y; the second with the gated
    # residual, written after the first in one y
    mg0, mg1, ng, kg = 64, 300, 256, 256
    rng = np.random.default_rng(11)
    xg0, xg1 = (O.bf16_rne(rng.standard_normal(mm * kg).astype(np.float32)) for mm in (mg0, mg1))
    wg0, wg1 = ((lambda v: (v + (v >= 0x7F)).astype(np.uint8))(rng.integers(0, 254, ng * kg)) for _ in range(2))
    gg = rng.uniform(-1, 1, ng).astype(np.float32)
    resg = np.zeros((mg0 + mg1) * ng, np.float32)
    resg[mg0 * ng:] = rng.standard_normal(mg1 * ng).astype(np.float32)
    v0 = O.matmul(O.matmul_params(mg0, ng, kg, 0.05), O.BF16, xg0, O.FP8, wg0)
    v1 = O.matmul(O.matmul_params(mg1, ng, kg, 0.03), O.BF16, xg1, O.FP8, wg1).reshape(mg1, ng)
    group_want = np.concatenate([v0, (resg[mg0 * ng:].reshape(mg1, ng) + gg.astype(np.float64) * v1).ravel()])
    cases.append(dict(name="group", op="group", m0=mg0, m1=mg1, n=ng, k=kg, scale0=0.05, scale1=0.03,
                      x0=_write(tmp_path, "xg0", xg0.view(np.uint16)), x1=_write(tmp_path, "xg1", xg1.view(np.uint16)),
                      w0=_write(tmp_path, "wg0", wg0), w1=_write(tmp_path, "wg1", wg1), gate=_write(tmp_path, "gg", gg),
                      res=_write(tmp_path, "resg", resg)))
    checks["group"] = (np.float32, lambda g: O.rel_error(g, group_want) < 1e-5)

    (tmp_path / "spec.json").write_text(json.dumps(dict(cases=cases)))
    print(f"[node] {len(cases)} cases in {tmp_path}", flush=True)
    out = subprocess.run([NODE, str(ROOT / "tests" / "node_driver.js"), str(tmp_path)], capture_output=True,
                         text=True, timeout=100)
    print(out.stdout[-2000:], out.stderr[-2000:], flush=True)
    assert out.returncode == 0
    result = json.loads((tmp_path / "result.json").read_text())
    assert result["device"]["arch"].startswith("gfx950")
    assert result["errors"]["lora_rank3"] == "LoRA shapes do not fit the linear layer"
    assert result["errors"]["run_unknown"].startswith("Graph.run: no MI355X kernel is registered for this shader")
    assert len(result["errors"]) == 2
    assert result["registered"] == 21  # 9 matmul variants, conv3x3, rmsnorm, 2 rope pairings, layer sum, 7 elementwise
    assert result["concurrentReads"] == [1, 2, 3]
    assert result["reusedDelta"] >= 1 and result["zeroed"]
    failed = []
    for name, (dtype, ok) in checks.items():
        got = np.fromfile(tmp_path / f"{name}.out", dtype)
        if dtype == np.float32:
            got = got.astype(np.float64)
        if not ok(got):
            failed.append(name)
    assert not failed, failed

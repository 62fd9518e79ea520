"use strict";
/*
 * Runs the graph steps of web-engine_amd/node (the N-API addon) on cuda:0 from a case list written by
 * tests/test_node.py: node tests/node_driver.js <dir>. Inputs are raw little-endian files in <dir>, each
 * case's output goes to <dir>/<name>.out, and <dir>/result.json gets the device info and pool statistics.
 */
const fs = require("fs");
const path = require("path");
const we = require("../web-engine_amd/node/index.js");

// Stand-ins for the reference's WGSL exports (src/kernels/*.ts), by their reference names: Graph.run keys on the
// source text, so distinct strings exercise the same dispatch the real shader sources would.
const REF = {
  matmulWgsl: (w, input = "rows", { splitK = false, accumulate = false } = {}) =>
    `// matmul ${w} ${input}${splitK ? " splitK" : ""}${accumulate ? " accumulate" : ""}`,
  rmsnormWgsl: "// rmsnorm", ropeKernel: (pairing) => `// rope ${pairing}`, layerSumWgsl: "// layer sum",
  swigluWgsl: "// swiglu", sigmoidGateWgsl: "// sigmoid gate", gatedAddWgsl: "// gated add", addBiasWgsl: "// add bias",
  geluTanhWgsl: "// gelu tanh", addWgsl: "// add", siluWgsl: "// silu",
};
REF.matmulFp8Wgsl = REF.matmulWgsl("fp8");
REF.matmulBf16Wgsl = REF.matmulWgsl("bf16");
REF.matmulF32Wgsl = REF.matmulWgsl("f32");
REF.conv3x3Wgsl = REF.matmulWgsl("f32", "conv3x3");
const registered = we.registerKernels(REF);

/** src/kernels/rmsnorm.ts:52-57 */
function rmsnormParams(rows, d, eps, offset) {
  const params = new Uint32Array(4);
  params.set([rows, d]);
  new Float32Array(params.buffer).set([eps, offset], 2);
  return params;
}

/** The reference's linear / narrowLinear (src/model/ops.ts:48-73) as Graph.run calls: matmul, addBias, LoRA. */
function runLinear(graph, x, w, m) {
  const shape = { m, n: w.n, k: w.k };
  const y = graph.buffer(m * w.n * 4);
  const MATMUL = { fp8: REF.matmulFp8Wgsl, bf16: REF.matmulBf16Wgsl, f32: REF.matmulF32Wgsl };
  graph.run(MATMUL[w.dtype], [graph.buffer(we.matmulParams(shape, w.scale)), x, w.buffer, y], [1, 1]);
  let out = y;
  if (w.bias) {
    out = graph.buffer(m * w.n * 4);
    graph.run(REF.addBiasWgsl, [graph.buffer(new Uint32Array([m * w.n, w.n])), y, w.bias, out], [1]);
  }
  if (!w.lora) return out;
  const { down, up } = w.lora;
  const t = runNarrow(graph, x, down, m);
  graph.run(REF.matmulWgsl(up.dtype, "rows", { accumulate: true }),
            [graph.buffer(we.matmulParams({ m, n: up.n, k: up.k }, up.scale)), t, up.buffer, out], [1, 1]);
  return out;
}

function runNarrow(graph, x, w, m) {
  const split = we.kSplitFor(m, w.n, w.k);
  if (split === 1) return runLinear(graph, x, w, m);
  const shape = { m, n: w.n, k: w.k };
  const partials = graph.buffer(split * m * w.n * 4);
  graph.run(REF.matmulWgsl(w.dtype, "rows", { splitK: true }),
            [graph.buffer(we.matmulParams(shape, w.scale, { kSplit: split })), x, w.buffer, partials], [1, 1, split]);
  const y = graph.buffer(m * w.n * 4);
  graph.run(REF.layerSumWgsl, [graph.buffer(new Uint32Array([1, split, m * w.n])), partials,
                               graph.buffer(new Float32Array(split).fill(1)), y], [1]);
  return y;
}

const dir = process.argv[2];
const spec = JSON.parse(fs.readFileSync(path.join(dir, "spec.json"), "utf8"));
const load = (graph, file) => (file == null ? null : graph.buffer(fs.readFileSync(path.join(dir, file))));

function linearOf(graph, w) {
  if (w == null) return null;
  const lin = { buffer: load(graph, w.file), dtype: w.dtype, scale: w.scale, n: w.n, k: w.k };
  if (w.bias) lin.bias = load(graph, w.bias);
  if (w.scales) lin.scales = load(graph, w.scales);
  if (w.group) lin.group = w.group;
  if (w.lora) lin.lora = { down: linearOf(graph, w.lora.down), up: linearOf(graph, w.lora.up) };
  return lin;
}

async function runCase(graph, c) {
  switch (c.op) {
    case "linear":
      return we.linear(graph, load(graph, c.x), linearOf(graph, c.w), c.m,
                       { xDtype: c.xDtype, yDtype: c.yDtype, geluTanh: !!c.geluTanh });
    case "norm": {
      const mod = c.scale ? { scale: load(graph, c.scale), shift: load(graph, c.shift) } : we.noMod(graph, c.d);
      return we.norm(graph, load(graph, c.x), load(graph, c.weight), c.rows, c.d, mod, c.eps, c.offset);
    }
    case "rotate": {
      const rope = { cos: load(graph, c.cos), sin: load(graph, c.sin), pairs: c.pairs, tokens: c.tokens };
      return we.rotate(graph, load(graph, c.x), c.heads, rope, c.pairing);
    }
    case "attention":
      return we.attention(graph, load(graph, c.q), load(graph, c.k), load(graph, c.v),
                          { tokens: c.tokens, heads: c.heads, kvHeads: c.kvHeads, dim: c.dim, causal: c.causal });
    case "elementwise":
      return we[c.fn](graph, ...c.inputs.map((f) => load(graph, f)), ...c.sizes);
    case "stream": {  // pinned host memory -> device on the copy stream, ordered by a ticket
      const data = fs.readFileSync(path.join(dir, c.x));
      const pinned = graph.hostAlloc(data.length);
      graph.hostWrite(pinned, 0, data);
      const dst = graph.buffer(data.length);
      const ticket = graph.streamCopy(dst, pinned, data.length, 0);
      graph.waitTicket(ticket);
      graph.sync();
      graph.hostFree(pinned);
      return dst;
    }
    // the same steps through Graph.run(code, bindings, workgroups), as the reference's ops.ts issues them
    case "runLinear":
      return runLinear(graph, load(graph, c.x), linearOf(graph, c.w), c.m);
    case "runNarrow":
      return runNarrow(graph, load(graph, c.x), linearOf(graph, c.w), c.m);
    case "runNorm": {  // Params written with device.queue.writeBuffer (no host copy: run() downloads them)
      const params = graph.buffer(16);
      graph.device.queue.writeBuffer(params, 0, rmsnormParams(c.rows, c.d, c.eps, c.offset));
      const out = graph.buffer(c.rows * c.d * 4);
      graph.run(REF.rmsnormWgsl, [params, load(graph, c.x), load(graph, c.weight), load(graph, c.scale),
                                  load(graph, c.shift), out], [c.rows]);
      return out;
    }
    case "runRotate": {
      const out = graph.buffer(c.tokens * c.heads * c.pairs * 2 * 4);
      graph.run(REF.ropeKernel(c.pairing), [graph.buffer(new Uint32Array([c.tokens, c.heads, c.pairs])),
                                           load(graph, c.x), load(graph, c.cos), load(graph, c.sin), out], [1, 1]);
      return out;
    }
    case "runElementwise": {  // src/model/ops.ts:95-99, with the modulation slice form { buffer, offset, size }
      const inputs = c.inputs.map((f) => load(graph, f));
      if (c.sliceLast) {
        const last = inputs[inputs.length - 1];
        const wide = graph.buffer(last.size + 256);
        graph.copy(last, 0, wide, 256, last.size);
        inputs[inputs.length - 1] = { buffer: wide, offset: 256, size: last.size };
      }
      const out = graph.buffer(c.sizes[0] * 4);
      graph.run(REF[c.code], [graph.buffer(new Uint32Array([c.sizes[0], c.sizes[1] || 1])), ...inputs, out], [1]);
      return out;
    }
    case "runConv": {  // src/model/vae.ts:134-135: conv3x3Params, then Graph.run(conv3x3Wgsl, ...)
      const { shape, params } = we.conv3x3Params(c.h, c.w, c.cin, c.cout, graph);
      const y = graph.buffer(shape.m * shape.n * 4);
      graph.run(REF.conv3x3Wgsl, [graph.buffer(params), load(graph, c.x), load(graph, c.weight), y], [1, 1]);
      return y;
    }
    case "group": {  // two GEMMs as one launch (matmulGroup): item 0 plain, item 1 with a gated residual, one y
      const y = graph.buffer((c.m0 + c.m1) * c.n * 4);
      const res = load(graph, c.res);
      graph.matmulGroup([
        { params: we.matmulParams({ m: c.m0, n: c.n, k: c.k }, c.scale0, {}, graph), x: load(graph, c.x0),
          w: load(graph, c.w0), y },
        { params: we.matmulParams({ m: c.m1, n: c.n, k: c.k }, c.scale1, { yOffset: c.m0 * c.n }, graph),
          x: load(graph, c.x1), w: load(graph, c.w1), y, gate: load(graph, c.gate), residual: res },
      ], we.BF16, we.FP8, we.F32);
      return y;
    }
    case "runUnknown":
      graph.run("// a shader with no MI355X kernel", [graph.buffer(new Uint32Array(2))], [1]);
      return null;
    default:
      throw new Error(`unknown op ${c.op}`);
  }
}

(async () => {
  const graph = new we.Graph(0);
  const result = { device: graph.deviceInfo(), errors: {} };
  try {
    for (const c of spec.cases) {
      console.log(`[node case] ${c.name}`);
      const mark = graph.mark();
      try {
        const y = await runCase(graph, c);
        if (c.op.startsWith("run")) await graph.device.queue.onSubmittedWorkDone(); // src/model/weights.ts:128
        fs.writeFileSync(path.join(dir, `${c.name}.out`), Buffer.from(await graph.read(y)));
      } catch (e) {
        if (!c.expectError) throw e;
        result.errors[c.name] = e.message;
      }
      graph.release(mark);
    }
    const before = graph.stats;
    const mark = graph.mark();
    graph.buffer(4096);
    graph.release(mark);
    const again = graph.buffer(4096);  // same size class: taken from the pool, zeroed
    result.reusedDelta = graph.stats.reused - before.reused;
    result.zeroed = new Uint8Array(await graph.read(again)).every((b) => b === 0);
    result.registered = registered;
    // reads in flight together, each resolving to its own bytes, while the event loop keeps turning
    const bufs = [1, 2, 3].map((v) => graph.buffer(new Float32Array(1 << 16).fill(v)));
    let ticks = 0;
    const timer = setInterval(() => ticks++, 0);
    const reads = await Promise.all(bufs.map((b) => graph.read(b)));
    clearInterval(timer);
    result.concurrentReads = reads.map((r) => new Float32Array(r).every((v, _, a) => v === a[0]) && new Float32Array(r)[0]);
  } finally {
    graph.destroy();
  }
  fs.writeFileSync(path.join(dir, "result.json"), JSON.stringify(result));
  console.log("[node] done");
})().catch((e) => {
  console.error(e);
  process.exit(1);
});

"use strict";
/*
 * Runs the graph steps of web-engine_amd/node (the N-API addon) on cuda:0 from a case list written by
 * tests/test_node.py: node tests/node_driver.js <dir>. Inputs are raw little-endian files in <dir>, each
 * case's output goes to <dir>/<name>.out, and <dir>/result.json gets the device info and pool statistics.
 */
const fs = require("fs");
const path = require("path");
const we = require("../web-engine_amd/node/index.js");

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
  } finally {
    graph.destroy();
  }
  fs.writeFileSync(path.join(dir, "result.json"), JSON.stringify(result));
  console.log("[node] done");
})().catch((e) => {
  console.error(e);
  process.exit(1);
});

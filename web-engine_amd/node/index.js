"use strict";
/*
 * CommonJS glue over we_node.node: a Graph with the method names of the reference's WebGPU Graph
 * (src/gpu/graph.ts:26-160) and the graph steps of src/model/ops.ts, running on the MI355X kernels of libwe.so.
 * A buffer is { ptr: BigInt, size: number } in place of a GPUBuffer; Graph.slice gives a binding into one.
 */
const addon = require("./we_node.node");

const F32 = 0, F16 = 1, BF16 = 2, FP8 = 3, INT4 = 4;
const DTYPES = { f32: F32, f16: F16, bf16: BF16, fp8: FP8, int4: INT4 };
const ELEM_BYTES = { [F32]: 4, [F16]: 2, [BF16]: 2, [FP8]: 1 };
const EPI = { ACCUMULATE: 1, SPLIT_K: 2, BIAS: 4, GELU_TANH: 8 };
const OP = { SWIGLU: 0, SIGMOID_GATE: 1, GATED_ADD: 2, ADD_BIAS: 3, GELU_TANH: 4, ADD: 5, SILU: 6 };
const MUL = { SWIGLU: 1, SIGMOID_GATE: 2 };
// kernel-choice switches (we_set_tuning, WE_TUNE_* of include/we.h)
const TUNE = { gemmCfg: 0, gemmGeneric: 1, gemmSplitK: 2, gemmReduceXcd: 3, attnPath: 4, int4Path: 5 };

// A binding is a buffer { ptr, size }, a Graph.slice of one, the reference's { buffer, offset, size } form, or a
// BigInt address.
const ptrOf = (b) =>
  b == null ? null : typeof b === "bigint" ? b : b.buffer !== undefined ? b.buffer.ptr + BigInt(b.offset || 0) : b.ptr;
const ownerOf = (b) => (b != null && typeof b === "object" && b.buffer !== undefined ? b.buffer : b);
const offsetOf = (b) => (b != null && typeof b === "object" && b.buffer !== undefined ? b.offset || 0 : 0);

// Graph.run's table: the WGSL source text of a reference shader -> the MI355X kernel computing the same thing.
const KERNELS = new Map();
// the reference's elementwise exports (src/kernels/elementwise.ts:38-86): [name, op, inputs between params and out]
const ELEMENTWISE = [
  ["swigluWgsl", OP.SWIGLU, 2], ["sigmoidGateWgsl", OP.SIGMOID_GATE, 2], ["gatedAddWgsl", OP.GATED_ADD, 3],
  ["addBiasWgsl", OP.ADD_BIAS, 2], ["geluTanhWgsl", OP.GELU_TANH, 1], ["addWgsl", OP.ADD, 2], ["siluWgsl", OP.SILU, 1],
];
const PARAM_BYTES = { matmul: 52, rmsnorm: 16, rope: 12, layerSum: 12, elementwise: 8 };
const SHADOW_MAX = 256; // buffers made from data up to this size keep a host copy, so run() reads Params without a sync

/**
 * Fills Graph.run's table from the reference's kernel exports, given by their reference names (e.g. the modules
 * src/kernels/matmul.ts, rmsnorm.ts, rope.ts, elementwise.ts and text.ts spread into one object):
 *   matmulWgsl (the function, src/kernels/matmul.ts:118: fp8 / bf16 / f32 weights x plain, splitK, accumulate),
 *   matmulFp8Wgsl / matmulBf16Wgsl / matmulF32Wgsl, conv3x3Wgsl, rmsnormWgsl, ropeKernel or ropeWgsl / ropeHalfWgsl,
 *   layerSumWgsl, and swigluWgsl, sigmoidGateWgsl, gatedAddWgsl, addBiasWgsl, geluTanhWgsl, addWgsl, siluWgsl.
 * Returns how many sources the table maps. Shaders outside this list (attention parts, the VAE's others) have
 * no MI355X kernel here, and Graph.run throws for them.
 */
function registerKernels(ref) {
  const put = (name, code, kernel) => {
    if (typeof code !== "string") throw new TypeError(`registerKernels: ${name} is not WGSL source text`);
    KERNELS.set(code, kernel);
  };
  if (ref.matmulWgsl !== undefined) {
    for (const w of ["fp8", "bf16", "f32"]) {
      put(`matmulWgsl("${w}")`, ref.matmulWgsl(w, "rows", {}), { op: "matmul", weights: DTYPES[w], flags: 0 });
      put(`matmulWgsl("${w}", splitK)`, ref.matmulWgsl(w, "rows", { splitK: true }),
          { op: "matmul", weights: DTYPES[w], flags: EPI.SPLIT_K });
      put(`matmulWgsl("${w}", accumulate)`, ref.matmulWgsl(w, "rows", { accumulate: true }),
          { op: "matmul", weights: DTYPES[w], flags: EPI.ACCUMULATE });
    }
  }
  // conv3x3Wgsl (src/kernels/matmul.ts:183) is the f32 matmul with the conv input; its Params say so
  for (const [name, w] of [["matmulFp8Wgsl", FP8], ["matmulBf16Wgsl", BF16], ["matmulF32Wgsl", F32], ["conv3x3Wgsl", F32]])
    if (ref[name] !== undefined) put(name, ref[name], { op: "matmul", weights: w, flags: 0 });
  if (ref.rmsnormWgsl !== undefined) put("rmsnormWgsl", ref.rmsnormWgsl, { op: "rmsnorm" });
  if (ref.ropeKernel !== undefined) {
    put('ropeKernel("interleaved")', ref.ropeKernel("interleaved"), { op: "rope", half: false });
    put('ropeKernel("half")', ref.ropeKernel("half"), { op: "rope", half: true });
  }
  if (ref.ropeWgsl !== undefined) put("ropeWgsl", ref.ropeWgsl, { op: "rope", half: false });
  if (ref.ropeHalfWgsl !== undefined) put("ropeHalfWgsl", ref.ropeHalfWgsl, { op: "rope", half: true });
  if (ref.layerSumWgsl !== undefined) put("layerSumWgsl", ref.layerSumWgsl, { op: "layerSum" });
  for (const [name, op, inputs] of ELEMENTWISE)
    if (ref[name] !== undefined) put(name, ref[name], { op: "elementwise", kind: op, inputs });
  return KERNELS.size;
}

const bindingCount = (k) => (k.op === "matmul" ? 4 : k.op === "rmsnorm" ? 6 : k.op === "rope" ? 5 : k.op === "layerSum" ? 4 : k.inputs + 2);

class Graph {
  /** src/gpu/graph.ts:35: one context (device, streams, pool) per graph. */
  constructor(device = 0) {
    this.ctx = addon.create(device);
    this.shadow = new WeakMap(); // buffer -> host copy of its bytes (small buffers made from data: Params)
    this.staging = new Map();    // size -> free pinned blocks for read()
    this.pending = 0;            // reads and onSubmittedWorkDone waits not yet settled
    // graph.device.queue as the reference's callers use it (src/model/weights.ts:128, src/gpu/graph.ts:47)
    this.device = {
      queue: {
        writeBuffer: (buffer, offset, data, dataOffset, size) => this.writeBuffer(buffer, offset, data, dataOffset, size),
        onSubmittedWorkDone: () => this.onSubmittedWorkDone(),
        submit: () => {},
      },
    };
  }

  /** src/gpu/graph.ts:38-54: a device buffer with this data, or zeroed with this many bytes (pooled by size). */
  buffer(data) {
    const bytes = typeof data === "number" ? data : data.byteLength;
    const size = Math.max(4, Math.ceil(bytes / 4) * 4);
    const ptr = addon.bufAlloc(this.ctx, size);
    const buffer = { ptr, size };
    if (typeof data !== "number" && data.byteLength) {
      addon.upload(this.ctx, ptr, 0, data);
      if (data.byteLength <= SHADOW_MAX) {
        const view = ArrayBuffer.isView(data) ? new Uint8Array(data.buffer, data.byteOffset, data.byteLength) : new Uint8Array(data);
        this.shadow.set(buffer, Uint8Array.from(view));
      }
    }
    return buffer;
  }

  /**
   * GPUQueue.writeBuffer: `data` at byte `offset` of `buffer`; `dataOffset` and `size` count elements of a typed
   * array, bytes of an ArrayBuffer (WebGPU's rule). The upload is done when this returns.
   */
  writeBuffer(buffer, offset, data, dataOffset = 0, size) {
    const unit = ArrayBuffer.isView(data) ? data.BYTES_PER_ELEMENT || 1 : 1;
    const base = ArrayBuffer.isView(data) ? data.byteOffset : 0;
    const raw = ArrayBuffer.isView(data) ? data.buffer : data;
    const total = ArrayBuffer.isView(data) ? data.byteLength : data.byteLength;
    const begin = dataOffset * unit;
    const bytes = size === undefined ? total - begin : size * unit;
    if (begin < 0 || bytes < 0 || begin + bytes > total) throw new RangeError("writeBuffer: range runs past the data");
    const view = new Uint8Array(raw, base + begin, bytes);
    const owner = ownerOf(buffer);
    const at = offsetOf(buffer) + offset;
    addon.upload(this.ctx, ptrOf(owner), at, view);
    const sh = this.shadow.get(owner);
    if (sh !== undefined) {
      if (at + bytes <= sh.byteLength) sh.set(view, at);
      else this.shadow.delete(owner);
    }
  }

  /** The first `bytes` of a Params binding: the host copy when there is one, else a (waiting) download. */
  paramsOf(binding, bytes) {
    const owner = ownerOf(binding), off = offsetOf(binding);
    const sh = this.shadow.get(owner);
    if (sh !== undefined && off + bytes <= sh.byteLength) return sh.slice(off, off + bytes).buffer;
    return addon.download(this.ctx, ptrOf(binding), 0, bytes);
  }

  /**
   * src/gpu/graph.ts:76-89: queues one dispatch of a reference shader, with its bindings in order (Params first).
   * The shader is looked up in the table registerKernels fills and runs as the MI355X kernel that computes the
   * same thing; its Params are decoded here. `workgroups` is accepted for the reference's signature: the MI355X
   * kernels size their own grids (a split-K matmul takes its slice count from Params.k_split, as the reference's
   * kernel does).
   */
  run(code, bindings, workgroups) {
    const k = KERNELS.get(code);
    if (k === undefined) {
      const head = typeof code === "string" ? code.trim().split("\n")[0].slice(0, 60) : String(code);
      throw new Error(`Graph.run: no MI355X kernel is registered for this shader ("${head}"); registerKernels maps the reference's WGSL exports`);
    }
    if (!Array.isArray(bindings) || bindings.length !== bindingCount(k))
      throw new Error(`Graph.run: ${k.op} takes ${bindingCount(k)} bindings (Params first), got ${Array.isArray(bindings) ? bindings.length : typeof bindings}`);
    const raw = this.paramsOf(bindings[0], PARAM_BYTES[k.op]);
    const u = new Uint32Array(raw), f = new Float32Array(raw);
    const b = (i) => ptrOf(bindings[i]);
    let out;
    switch (k.op) {
      case "matmul": // [p, x, w, y]: f32 x and y (src/kernels/matmul.ts:127-132)
        addon.matmul(this.ctx, u, F32, b(1), k.weights, b(2), null, 0, F32, b(3), null, k.flags);
        out = 3;
        break;
      case "rmsnorm": // [p, x, weight, scale, shift, out], Params { rows, d, eps: f32, offset: f32 }
        addon.rmsnorm(this.ctx, u[0], u[1], f[2], f[3], F32, b(1), b(2), b(3), b(4), b(5));
        out = 5;
        break;
      case "rope": // [p, x, cos, sin, out], Params { tokens, heads, pairs }
        addon.rope(this.ctx, u[0], u[1], u[2], k.half ? 1 : 0, F32, b(1), b(2), b(3), b(4));
        out = 4;
        break;
      case "layerSum": // [p, x, w, out], Params { tokens, layers, dim }
        addon.layerSum(this.ctx, u[0], u[1], u[2], b(1), b(2), b(3));
        out = 3;
        break;
      default: // elementwise: [p, inputs..., out], Params { n, d }
        addon.elementwise(this.ctx, k.kind, u[0], u[1], F32, b(1), k.inputs > 1 ? b(2) : null,
                          k.inputs > 2 ? b(3) : null, b(k.inputs + 1));
        out = k.inputs + 1;
    }
    this.shadow.delete(ownerOf(bindings[out])); // the kernel writes it: a host copy would go stale
  }

  /** src/gpu/graph.ts:57-60 */
  static slice(buffer, offset, size) {
    return { ptr: buffer.ptr + BigInt(offset), size };
  }

  /** Work is queued on the context's stream as it is issued; nothing is held back. */
  submit() {}

  /**
   * src/gpu/graph.ts:109-119: copies `bytes` of `buffer` back after everything queued before. The copy goes to
   * pinned memory on the selected compute stream and the wait runs on a worker thread, so the event loop keeps
   * running meanwhile; the Promise resolves to an ArrayBuffer.
   */
  async read(buffer, bytes = buffer.size) {
    if (bytes === 0) return new ArrayBuffer(0);
    const size = Math.max(4096, 2 ** Math.ceil(Math.log2(bytes)));
    const free = this.staging.get(size);
    const pinned = free !== undefined && free.length ? free.pop() : addon.hostAlloc(this.ctx, size);
    const ticket = addon.downloadAsync(this.ctx, ptrOf(buffer), 0, pinned, bytes);
    this.pending++;
    try {
      await addon.waitTicketAsync(this.ctx, ticket);
      return addon.hostRead(this.ctx, pinned, bytes);
    } finally {
      this.pending--;
      if (this.ctx !== null) {
        if (!this.staging.has(size)) this.staging.set(size, []);
        this.staging.get(size).push(pinned);
      }
    }
  }

  /**
   * GPUQueue.onSubmittedWorkDone (src/model/weights.ts:128, src/gpu/run-ahead.ts:5): resolves once the work queued
   * so far on both compute streams and the copy stream has finished; waits on worker threads.
   */
  onSubmittedWorkDone() {
    const tickets = addon.recordAll(this.ctx);
    this.pending++;
    return Promise.all(tickets.map((t) => addon.waitTicketAsync(this.ctx, t))).then(
      () => { this.pending--; },
      (e) => { this.pending--; throw e; });
  }

  copy(src, srcOffset, dst, dstOffset, size) {
    addon.copy(this.ctx, ptrOf(src), srcOffset, ptrOf(dst), dstOffset, size);
    this.shadow.delete(ownerOf(dst));
  }

  mark() {
    return addon.mark(this.ctx);
  }

  release(mark, keep = []) {
    addon.release(this.ctx, mark, keep.map((b) => b.ptr));
  }

  free(buffer) {
    addon.bufFree(this.ctx, buffer.ptr);
  }

  /** Failure injection: device allocations past `bytes` held (0 = no cap) throw as a full device does. */
  setAllocCap(bytes) {
    return addon.setAllocCap(this.ctx, bytes);
  }

  /** Debugging: freed and released buffers are filled with NaN bytes once pooled. */
  setPoison(on) {
    addon.setPoison(this.ctx, on ? 1 : 0);
  }

  /** Pins a kernel choice (a TUNE key: gemmCfg, gemmGeneric, gemmSplitK, gemmReduceXcd, attnPath, int4Path);
   *  returns the previous value. */
  setTuning(key, value) {
    const k = typeof key === "string" ? TUNE[key] : key;
    if (k === undefined) throw new Error(`unknown tuning key ${key}`);
    return addon.setTuning(this.ctx, k, value);
  }

  /** src/gpu/graph.ts:32: buffers created vs taken from the pool, and bytes created. */
  get stats() {
    return addon.stats(this.ctx);
  }

  /** Frees everything. Settle (await) every read() and onSubmittedWorkDone() first: their waits use the context. */
  destroy() {
    if (this.pending) throw new Error(`Graph.destroy: ${this.pending} read() / onSubmittedWorkDone() promises still pending; await them first`);
    if (this.ctx !== null) addon.destroy(this.ctx); // frees the pinned staging blocks with the context
    this.ctx = null;
    this.staging.clear();
  }

  sync() {
    addon.sync(this.ctx);
  }

  /** Two compute streams: later calls queue on stream `which` (0: main, 1: second). */
  stream(which) {
    addon.streamSelect(this.ctx, which);
  }

  /** Stream 1 waits for the work queued so far on stream 0. */
  fork() {
    addon.streamFork(this.ctx);
  }

  /** Stream 0 waits for the work queued so far on stream 1. */
  join() {
    addon.streamJoin(this.ctx);
  }

  deviceInfo() {
    return addon.deviceInfo(this.ctx);
  }

  // ---- the kernels, one call each ----
  // gate (f32 [N]) given: y = residual + gate * v, the gatedAdd of src/model/block.ts:60-64 fused (matmulGated);
  // mul given: y = silu(aux) * v (MUL.SWIGLU) or aux * sigmoid(v) (MUL.SIGMOID_GATE) (matmulMul)
  matmul(params, xDtype, x, wDtype, w, yDtype, y,
         { scales = null, group = 0, bias = null, flags = 0, gate = null, residual = null, mul = 0, aux = null } = {}) {
    if (mul) {
      addon.matmulMul(this.ctx, params, xDtype, ptrOf(x), wDtype, ptrOf(w), ptrOf(scales), group, yDtype, ptrOf(y),
                      ptrOf(bias), flags, mul, ptrOf(aux));
    } else if (gate === null) {
      addon.matmul(this.ctx, params, xDtype, ptrOf(x), wDtype, ptrOf(w), ptrOf(scales), group, yDtype, ptrOf(y),
                   ptrOf(bias), flags);
    } else {
      addon.matmulGated(this.ctx, params, xDtype, ptrOf(x), wDtype, ptrOf(w), ptrOf(scales), group, yDtype, ptrOf(y),
                        ptrOf(bias), flags, ptrOf(gate), ptrOf(residual));
    }
  }

  /** One or two GEMMs of one N, K, dtypes and flags as one launch (matmulGroup): items are
   * { params, x, w, y, bias, gate, residual } (bias, gate and residual optional, as in matmul). */
  matmulGroup(items, xDtype, wDtype, yDtype, flags = 0) {
    const args = [];
    for (const it of items) {
      args.push(it.params, ptrOf(it.x), ptrOf(it.w), ptrOf(it.y), ptrOf(it.bias), ptrOf(it.gate),
                ptrOf(it.residual));
    }
    addon.matmulGroup(this.ctx, items.length, xDtype, wDtype, yDtype, flags, ...args);
  }

  /** A QKV projection with the per-head RMSNorm + RoPE of its q / k heads (128 wide) fused in (the q/k path of
   * attend(), src/model/block.ts:53-56). */
  matmulQkNormRope(params, xDtype, x, wDtype, w, yDtype, y, qHeads, kHeads, eps, offset, normQ, normK,
                   { ropeFrom = 0, cos = null, sin = null, bias = null, flags = 0 } = {}) {
    addon.matmulQkNormRope(this.ctx, params, xDtype, ptrOf(x), wDtype, ptrOf(w), yDtype, ptrOf(y), ptrOf(bias), flags,
                           qHeads, kHeads, eps, offset, ptrOf(normQ), ptrOf(normK), ropeFrom, ptrOf(cos), ptrOf(sin));
  }

  rmsnorm(rows, d, eps, offset, dtype, x, weight, scale, shift, out) {
    addon.rmsnorm(this.ctx, rows, d, eps, offset, dtype, ptrOf(x), ptrOf(weight), ptrOf(scale), ptrOf(shift),
                  ptrOf(out));
  }

  /** mod = tvec + table (modN f32) and out = rmsnorm(x) modulated by mod[0:d], mod[d:2d], in one launch */
  rmsnormMod(rows, d, eps, offset, dtype, x, weight, tvec, table, modN, mod, out) {
    addon.rmsnormMod(this.ctx, rows, d, eps, offset, dtype, ptrOf(x), ptrOf(weight), ptrOf(tvec), ptrOf(table), modN,
                     ptrOf(mod), ptrOf(out));
  }

  rope(tokens, heads, pairs, half, dtype, x, cos, sin, out) {
    addon.rope(this.ctx, tokens, heads, pairs, half ? 1 : 0, dtype, ptrOf(x), ptrOf(cos), ptrOf(sin), ptrOf(out));
  }

  qkNormRope(tokens, heads, headDim, eps, offset, weight, ropeFrom, half, cos, sin, dtype, x, out, xStride = 0,
             outStride = 0) {
    addon.qkNormRope(this.ctx, tokens, heads, headDim, eps, offset, ptrOf(weight), ropeFrom, half ? 1 : 0, ptrOf(cos),
                     ptrOf(sin), dtype, ptrOf(x), xStride, ptrOf(out), outStride);
  }

  attention(tokens, heads, kvHeads, dim, causal, dtype, q, k, v, out,
            { qStride = 0, kStride = 0, vStride = 0, outStride = 0 } = {}) {
    addon.attention(this.ctx, tokens, heads, kvHeads, dim, causal ? 1 : 0, dtype, ptrOf(q), qStride, ptrOf(k), kStride,
                    ptrOf(v), vStride, ptrOf(out), outStride);
  }

  elementwise(op, n, d, dtype, a, b, c, out) {
    addon.elementwise(this.ctx, op, n, d, dtype, ptrOf(a), ptrOf(b), ptrOf(c), ptrOf(out));
  }

  layerSum(tokens, layers, dim, x, w, out) {
    addon.layerSum(this.ctx, tokens, layers, dim, ptrOf(x), ptrOf(w), ptrOf(out));
  }

  // ---- pinned host memory and the copy stream (src/model/weights.ts:124-129, src/gpu/run-ahead.ts:7-21) ----
  /** Pinned host memory: { ptr, size, ctx }; hostWrite and readTensor check every write against it. */
  hostAlloc(bytes) {
    return { ptr: addon.hostAlloc(this.ctx, bytes), size: bytes, ctx: this.ctx };
  }

  hostWrite(pinned, offset, data) {
    if (pinned.freed) throw new Error("pinned buffer was freed");
    if (!(Number.isInteger(offset) && offset >= 0 && offset + data.byteLength <= pinned.size))
      throw new RangeError(`write of ${data.byteLength} bytes at ${offset} runs past the ${pinned.size}-byte pinned buffer`);
    addon.hostWrite(this.ctx, pinned.ptr, offset, data);  // checked again natively against the live block
  }

  hostFree(pinned) {
    addon.hostFree(this.ctx, pinned.ptr);
    pinned.freed = true;
  }

  streamCopy(dst, pinnedSrc, bytes, after = 0) {
    return addon.streamCopy(this.ctx, ptrOf(dst), ptrOf(pinnedSrc), bytes, after);
  }

  waitTicket(ticket) {
    addon.waitTicket(this.ctx, ticket);
  }

  ticketDone(ticket) {
    return addon.ticketDone(this.ctx, ticket);
  }

  recordCompute() {
    return addon.recordCompute(this.ctx);
  }

  // ---- HIP graphs of the compute stream: capture a fixed sequence of graph steps once, replay it
  graphBegin() {
    addon.graphBegin(this.ctx);
  }

  graphEnd() {
    return addon.graphEnd(this.ctx);
  }

  graphLaunch(graph) {
    addon.graphLaunch(this.ctx, graph);
  }

  graphDestroy(graph) {
    addon.graphDestroy(this.ctx, graph);
  }
}

/** src/kernels/matmul.ts:198-212: the 13 x u32 Params image, with the same defaults and errors. */
function matmulParams({ m, n, k }, scale, layout = {}, graph = null) {
  const l = layout;
  return addon.matmulParams(graph ? graph.ctx : null, m, n, k, scale, l.xStride, l.wStride, l.yStride, l.xOffset,
                            l.wOffset, l.yOffset, l.kSplit == null ? 1 : l.kSplit);
}

/** src/kernels/matmul.ts:268-272: { shape, params } of a 3x3 convolution as a GEMM, with the same error. */
function conv3x3Params(height, width, cin, cout, graph = null) {
  const params = addon.conv3x3Params(graph ? graph.ctx : null, height, width, cin, cout);
  return { shape: { m: height * width, n: cout, k: 9 * cin }, params };
}

/** src/model/ops.ts:42-45 */
const kSplitFor = (m, n, k) => addon.kSplitFor(m, n, k);

const wdt = (dtype) => (typeof dtype === "string" ? DTYPES[dtype] : dtype);

/** src/model/ops.ts:48-58: split-K partials, then a layer sum over them. */
function narrowLinear(graph, x, w, m, xDtype = F32) {
  const split = kSplitFor(m, w.n, w.k);
  if (split === 1) return linear(graph, x, w, m, { xDtype });
  const shape = { m, n: w.n, k: w.k };
  const partials = graph.buffer(split * m * w.n * 4);
  graph.matmul(matmulParams(shape, w.scale, { kSplit: split }, graph), xDtype, x, wdt(w.dtype), w.buffer, F32, partials,
               { flags: EPI.SPLIT_K });
  const y = graph.buffer(m * w.n * 4);
  graph.layerSum(1, split, m * w.n, partials, graph.buffer(new Float32Array(split).fill(1)), y);
  return y;
}

/**
 * src/model/ops.ts:61-73: y[m, n] = x[m, k] . W^T (+ bias) (+ up.scale * (x . down^T) . up^T, added in place).
 * The bias (and, on request, the tanh GELU) run in the GEMM epilogue. `w.dtype` may also be "int4" with
 * `w.scales` (f16 [n, k / group]) and `w.group`.
 */
function linear(graph, x, w, m, { xDtype = F32, yDtype = F32, geluTanh = false, swigluGate = null, sigmoidGateOf = null,
                                  out = null } = {}) {
  const shape = { m, n: w.n, k: w.k };
  if (swigluGate !== null || sigmoidGateOf !== null) {
    // the consumer fused: swiglu(swigluGate, linear) or sigmoidGate(sigmoidGateOf, linear) (src/model/ops.ts:102-104)
    if (geluTanh || (swigluGate !== null && sigmoidGateOf !== null)) throw new Error("one fused consumer at a time, and not with GELU");
    const aux = swigluGate !== null ? swigluGate : sigmoidGateOf;
    const mul = swigluGate !== null ? MUL.SWIGLU : MUL.SIGMOID_GATE;
    const y = out !== null ? out : graph.buffer(m * w.n * ELEM_BYTES[yDtype]);
    if (!w.lora && wdt(w.dtype) !== INT4) {
      graph.matmul(matmulParams(shape, w.scale, {}, graph), xDtype, x, wdt(w.dtype), w.buffer, yDtype, y,
                   { bias: w.bias, flags: w.bias ? EPI.BIAS : 0, mul, aux });
      return y;
    }
    const v = linear(graph, x, w, m, { xDtype, yDtype });
    graph.elementwise(mul === MUL.SWIGLU ? OP.SWIGLU : OP.SIGMOID_GATE, m * w.n, 1, yDtype, aux, v, null, y);
    graph.free(v);
    return y;
  }
  const y = out !== null ? out : graph.buffer(m * w.n * ELEM_BYTES[yDtype]);
  // GELU applies to the whole sum (a caller of the reference applies it to what linear returns): with LoRA it
  // runs in place after the update is added, not in the base GEMM's epilogue
  const flags = (w.bias ? EPI.BIAS : 0) | (geluTanh && !w.lora ? EPI.GELU_TANH : 0);
  const int4 = wdt(w.dtype) === INT4;
  graph.matmul(matmulParams(shape, w.scale, {}, graph), xDtype, x, wdt(w.dtype), w.buffer, yDtype, y,
               { scales: w.scales, group: int4 ? (w.group == null ? 64 : w.group) : 0, bias: w.bias, flags });
  if (!w.lora) return y;
  const { down, up } = w.lora;
  if (down.k !== w.k || up.n !== w.n || up.k !== down.n || down.n % 4) throw new Error("LoRA shapes do not fit the linear layer");
  const t = narrowLinear(graph, x, down, m, xDtype);
  graph.matmul(matmulParams({ m, n: up.n, k: up.k }, up.scale, {}, graph), F32, t, wdt(up.dtype), up.buffer, yDtype, y,
               { flags: EPI.ACCUMULATE });
  if (geluTanh) graph.elementwise(OP.GELU_TANH, m * w.n, 1, yDtype, y, null, null, y);
  return y;
}

/** src/model/ops.ts:78-82 */
function norm(graph, x, weight, rows, d, mod, eps = 1e-5, offset = 1, dtype = F32) {
  const out = graph.buffer(rows * d * ELEM_BYTES[dtype]);
  graph.rmsnorm(rows, d, eps, offset, dtype, x, weight, mod ? mod.scale : null, mod ? mod.shift : null, out);
  return out;
}

/** src/model/ops.ts:85 */
const noMod = (graph, d) => ({ scale: graph.buffer(d * 4), shift: graph.buffer(d * 4) });

/** src/model/ops.ts:89-93 */
function rotate(graph, x, heads, rope, pairing = "interleaved", dtype = F32) {
  const out = graph.buffer(rope.tokens * heads * rope.pairs * 2 * ELEM_BYTES[dtype]);
  graph.rope(rope.tokens, heads, rope.pairs, pairing === "half", dtype, x, rope.cos, rope.sin, out);
  return out;
}

/** src/kernels/attention.ts:20-51: shape { tokens, heads, kvHeads, dim, chunk?, causal? } -> new out buffer. */
function attention(graph, q, k, v, shape, dtype = F32) {
  const { tokens, heads, kvHeads, dim } = shape;
  if (!kvHeads || heads % kvHeads) throw new Error("heads must be a multiple of kvHeads");
  const out = graph.buffer(tokens * heads * dim * ELEM_BYTES[dtype]);
  graph.attention(tokens, heads, kvHeads, dim, !!shape.causal, dtype, q, k, v, out);
  return out;
}

function elementwise(graph, op, inputs, n, d = 1, dtype = F32) {
  const out = graph.buffer(n * ELEM_BYTES[dtype]);
  graph.elementwise(op, n, d, dtype, inputs[0], inputs.length > 1 ? inputs[1] : null,
                    inputs.length > 2 ? inputs[2] : null, out);
  return out;
}

// src/model/ops.ts:102-113
const swiglu = (graph, gate, up, n, dtype = F32) => elementwise(graph, OP.SWIGLU, [gate, up], n, 1, dtype);
const sigmoidGate = (graph, a, gate, n, dtype = F32) => elementwise(graph, OP.SIGMOID_GATE, [a, gate], n, 1, dtype);
const gatedAdd = (graph, x, h, g, n, d, dtype = F32) => elementwise(graph, OP.GATED_ADD, [x, h, g], n, d, dtype);
const addBias = (graph, x, b, n, d, dtype = F32) => elementwise(graph, OP.ADD_BIAS, [x, b], n, d, dtype);
const add = (graph, x, h, n, dtype = F32) => elementwise(graph, OP.ADD, [x, h], n, 1, dtype);
const gelu = (graph, x, n, dtype = F32) => elementwise(graph, OP.GELU_TANH, [x], n, 1, dtype);
const silu = (graph, x, n, dtype = F32) => elementwise(graph, OP.SILU, [x], n, 1, dtype);

// ---- .safetensors files: readHeader / readTensor (src/weights/safetensors.ts:28-70), on a path ----
// The header is read and checked natively (libwe's we_st_*), with the reference's messages; tensor bytes are
// read on request, with parallel positional reads, into a Uint8Array or straight into pinned host memory.
class SafetensorsError extends Error {
  constructor(message) {
    super(message);
    this.name = "SafetensorsError";
  }
}

function readHeader(path) {
  let handle;
  try {
    handle = addon.stOpen(path);
  } catch (e) {
    if (e.name === "SafetensorsError") throw new SafetensorsError(e.message);
    throw e;
  }
  const tensors = new Map();
  const n = addon.stCount(handle);
  for (let i = 0; i < n; i++) {
    const t = addon.stInfo(handle, i);
    tensors.set(t.name, { name: t.name, dtype: t.dtype, shape: t.shape, offset: t.offset, size: t.size, index: i });
  }
  const metadata = {};
  const m = addon.stMetadataCount(handle);
  for (let i = 0; i < m; i++) {
    const [k, v] = addon.stMetadataAt(handle, i);
    metadata[k] = v;
  }
  return { tensors, metadata, handle, close: () => addon.stClose(handle) };
}

/** The raw bytes of one tensor, or only its first `limit` bytes; `dst` (a Uint8Array, or pinned memory from
 * Graph.hostAlloc, optionally with a byte `offset` into it) receives them when given. */
function readTensor(st, tensor, limit, dst, threads, offset = 0) {
  const n = Math.min(limit === undefined ? tensor.size : limit, tensor.size);
  if (dst === undefined) dst = new Uint8Array(n);
  if (ArrayBuffer.isView(dst)) {
    addon.stRead(st.handle, tensor.index, 0, n, dst, threads || 0);
    return dst;
  }
  if (typeof dst !== "object" || dst.ctx == null) throw new TypeError("readTensor: dst must be a TypedArray or pinned memory from Graph.hostAlloc");
  if (dst.freed) throw new Error("pinned buffer was freed");
  if (offset + n > dst.size) throw new RangeError(`${n} bytes at ${offset} run past the ${dst.size}-byte pinned buffer`);
  addon.stRead(st.handle, tensor.index, 0, n, dst.ptr + BigInt(offset), threads || 0, dst.ctx);
  return dst;
}

module.exports = {
  addon, Graph, F32, F16, BF16, FP8, INT4, DTYPES, EPI, OP, MUL, TUNE,
  matmulParams, conv3x3Params, kSplitFor, linear, norm, noMod, rotate, attention,
  swiglu, sigmoidGate, gatedAdd, addBias, add, gelu, silu,
  SafetensorsError, readHeader, readTensor, registerKernels,
  lastError: (graph) => addon.lastError(graph ? graph.ctx : null),
};

/**
 * Types of index.js: the reference's Graph (src/gpu/graph.ts) and graph steps (src/model/ops.ts), with the same
 * names and argument meaning, on the MI355X kernels of libwe.so. A TypeScript caller of the reference switches by
 * importing Graph and the steps from here; its own ops.ts keeps working through Graph.run once registerKernels has
 * been given the reference's shader exports.
 */

/** A device buffer (in place of a GPUBuffer): its address and its size in bytes. */
export interface Buffer {
  readonly ptr: bigint;
  readonly size: number;
}

/** src/gpu/graph.ts:24: a whole buffer, or a part of it (offset and size in bytes). */
export type Binding = Buffer | { buffer: Buffer; offset: number; size: number };

/** Pinned host memory from Graph.hostAlloc. */
export interface Pinned {
  readonly ptr: bigint;
  readonly size: number;
  readonly ctx: bigint;
  freed?: boolean;
}

export const F32: 0;
export const F16: 1;
export const BF16: 2;
export const FP8: 3;
export const INT4: 4;
export type DType = 0 | 1 | 2 | 3 | 4;
export const DTYPES: { f32: 0; f16: 1; bf16: 2; fp8: 3; int4: 4 };
/** Epilogue flags of Graph.matmul: += into y, split-K partial planes, + bias[n], tanh GELU. */
export const EPI: { ACCUMULATE: 1; SPLIT_K: 2; BIAS: 4; GELU_TANH: 8 };
export const OP: { SWIGLU: 0; SIGMOID_GATE: 1; GATED_ADD: 2; ADD_BIAS: 3; GELU_TANH: 4; ADD: 5; SILU: 6 };
/** Product epilogues of Graph.matmul: y = silu(aux) * v, or aux * sigmoid(v). */
export const MUL: { SWIGLU: 1; SIGMOID_GATE: 2 };
export const TUNE: { gemmCfg: 0; gemmGeneric: 1; gemmSplitK: 2; gemmReduceXcd: 3; attnPath: 4; int4Path: 5 };

/** The subset of GPUQueue the reference's callers use. */
export interface Queue {
  writeBuffer(buffer: Binding, offset: number, data: ArrayBufferView | ArrayBuffer, dataOffset?: number, size?: number): void;
  onSubmittedWorkDone(): Promise<void>;
  submit(): void;
}

/**
 * The shader exports of the reference (src/kernels/matmul.ts, rmsnorm.ts, rope.ts, elementwise.ts, text.ts) under
 * their reference names; each one given is mapped to its MI355X kernel.
 */
export interface ReferenceKernels {
  matmulWgsl?: (weights: "fp8" | "bf16" | "f32", input?: "rows", mode?: { splitK?: boolean; accumulate?: boolean }) => string;
  matmulFp8Wgsl?: string;
  matmulBf16Wgsl?: string;
  matmulF32Wgsl?: string;
  conv3x3Wgsl?: string;
  rmsnormWgsl?: string;
  ropeKernel?: (pairing: "interleaved" | "half") => string;
  ropeWgsl?: string;
  ropeHalfWgsl?: string;
  layerSumWgsl?: string;
  swigluWgsl?: string;
  sigmoidGateWgsl?: string;
  gatedAddWgsl?: string;
  addBiasWgsl?: string;
  geluTanhWgsl?: string;
  addWgsl?: string;
  siluWgsl?: string;
}

/** Fills Graph.run's table; returns how many shader sources it maps. */
export function registerKernels(ref: ReferenceKernels): number;

export class Graph {
  /** One context (device, two compute streams, a copy stream, the buffer pool) per graph. */
  constructor(device?: number);
  readonly ctx: bigint | null;
  /** graph.device.queue as src/model/weights.ts:128 and src/gpu/graph.ts:47 use it. */
  readonly device: { queue: Queue };
  /** src/gpu/graph.ts:38 */
  buffer(data: ArrayBufferView | number): Buffer;
  /** src/gpu/graph.ts:57 */
  static slice(buffer: Buffer, offset: number, size: number): Buffer;
  /** src/gpu/graph.ts:76: one dispatch of a registered reference shader, bindings in order (Params first). */
  run(code: string, bindings: Binding[], workgroups: [number, number?, number?]): void;
  /** src/gpu/graph.ts:92 */
  copy(src: Binding, srcOffset: number, dst: Binding, dstOffset: number, size: number): void;
  /** src/gpu/graph.ts:100: work is queued as it is issued, so this does nothing. */
  submit(): void;
  /** src/gpu/graph.ts:109: resolves after the work queued before it, without blocking the event loop. */
  read(buffer: Binding, bytes?: number): Promise<ArrayBuffer>;
  writeBuffer(buffer: Binding, offset: number, data: ArrayBufferView | ArrayBuffer, dataOffset?: number, size?: number): void;
  onSubmittedWorkDone(): Promise<void>;
  /** src/gpu/graph.ts:122-139 */
  mark(): number;
  release(mark: number, keep?: Buffer[]): void;
  free(buffer: Buffer): void;
  /** src/gpu/graph.ts:32 */
  readonly stats: { created: number; reused: number; createdBytes: number };
  /** Failure injection: device allocations past `bytes` held (0 = no cap) throw; returns the bytes held now. */
  setAllocCap(bytes: number): number;
  /** Debugging: freed and released buffers are filled with NaN bytes once pooled. */
  setPoison(on: boolean): void;
  /** Pins a kernel choice (a TUNE key or its name); returns the previous value. */
  setTuning(key: keyof typeof TUNE | number, value: number): number;
  /** Every read() and onSubmittedWorkDone() promise must have settled first. */
  destroy(): void;
  sync(): void;
  stream(which: 0 | 1): void;
  fork(): void;
  join(): void;
  deviceInfo(): { arch: string; computeUnits: number; ldsBytes: number };

  matmul(params: Uint32Array, xDtype: DType, x: Binding, wDtype: DType, w: Binding, yDtype: DType, y: Binding,
         opts?: { scales?: Binding | null; group?: number; bias?: Binding | null; flags?: number; gate?: Binding | null;
                  residual?: Binding | null; mul?: 0 | 1 | 2; aux?: Binding | null }): void;
  /** One or two GEMMs of one N, K, dtypes and flags as one launch (we_matmul_group). */
  matmulGroup(items: Array<{ params: Uint32Array; x: Binding; w: Binding; y: Binding; bias?: Binding | null;
                             gate?: Binding | null; residual?: Binding | null }>,
              xDtype: DType, wDtype: DType, yDtype: DType, flags?: number): void;
  /** A QKV projection with the per-head RMSNorm + RoPE of its q / k heads (128 wide) fused in. */
  matmulQkNormRope(params: Uint32Array, xDtype: DType, x: Binding, wDtype: DType, w: Binding, yDtype: DType, y: Binding,
                   qHeads: number, kHeads: number, eps: number, offset: number, normQ: Binding, normK: Binding,
                   opts?: { ropeFrom?: number; cos?: Binding | null; sin?: Binding | null; bias?: Binding | null;
                            flags?: number }): void;
  rmsnorm(rows: number, d: number, eps: number, offset: number, dtype: DType, x: Binding, weight: Binding,
          scale: Binding | null, shift: Binding | null, out: Binding): void;
  /** mod = tvec + table (modN f32) and out = rmsnorm(x) modulated by mod[0:d], mod[d:2d], in one launch. */
  rmsnormMod(rows: number, d: number, eps: number, offset: number, dtype: DType, x: Binding, weight: Binding,
             tvec: Binding, table: Binding, modN: number, mod: Binding, out: Binding): void;
  rope(tokens: number, heads: number, pairs: number, half: boolean, dtype: DType, x: Binding, cos: Binding,
       sin: Binding, out: Binding): void;
  qkNormRope(tokens: number, heads: number, headDim: number, eps: number, offset: number, weight: Binding,
             ropeFrom: number, half: boolean, cos: Binding, sin: Binding, dtype: DType, x: Binding, out: Binding,
             xStride?: number, outStride?: number): void;
  attention(tokens: number, heads: number, kvHeads: number, dim: number, causal: boolean, dtype: DType, q: Binding,
            k: Binding, v: Binding, out: Binding,
            strides?: { qStride?: number; kStride?: number; vStride?: number; outStride?: number }): void;
  elementwise(op: number, n: number, d: number, dtype: DType, a: Binding, b: Binding | null, c: Binding | null,
              out: Binding): void;
  layerSum(tokens: number, layers: number, dim: number, x: Binding, w: Binding, out: Binding): void;

  hostAlloc(bytes: number): Pinned;
  hostWrite(pinned: Pinned, offset: number, data: ArrayBufferView): void;
  hostFree(pinned: Pinned): void;
  streamCopy(dst: Binding, pinnedSrc: Pinned | bigint, bytes: number, after?: number): number;
  waitTicket(ticket: number): void;
  ticketDone(ticket: number): boolean;
  recordCompute(): number;
  graphBegin(): void;
  graphEnd(): bigint;
  graphLaunch(graph: bigint): void;
  graphDestroy(graph: bigint): void;
}

/** src/model/ops.ts:25-34, plus int4 weights (f16 scales per group of K). */
export type Linear = {
  buffer: Buffer;
  dtype: "fp8" | "bf16" | "f32" | "int4";
  scale: number;
  n: number;
  k: number;
  bias?: Buffer;
  scales?: Buffer;
  group?: number;
  lora?: { down: Linear; up: Linear };
};
export type Mod = { scale: Binding; shift: Binding };
export type Rope = { cos: Buffer; sin: Buffer; pairs: number; tokens: number };
export type Pairing = "interleaved" | "half";

/** src/kernels/matmul.ts:198-212 */
export function matmulParams(shape: { m: number; n: number; k: number }, scale: number,
                             layout?: { xStride?: number; wStride?: number; yStride?: number; xOffset?: number;
                                        wOffset?: number; yOffset?: number; kSplit?: number },
                             graph?: Graph | null): Uint32Array;
/** src/kernels/matmul.ts:268-272 */
export function conv3x3Params(height: number, width: number, cin: number, cout: number, graph?: Graph | null):
  { shape: { m: number; n: number; k: number }; params: Uint32Array };
/** src/model/ops.ts:42 */
export function kSplitFor(m: number, n: number, k: number): number;
/** src/model/ops.ts:61 */
export function linear(graph: Graph, x: Binding, w: Linear, m: number,
                       opts?: { xDtype?: DType; yDtype?: DType; geluTanh?: boolean; swigluGate?: Binding | null;
                                sigmoidGateOf?: Binding | null; out?: Buffer | null }): Buffer;
/** src/model/ops.ts:78 */
export function norm(graph: Graph, x: Binding, weight: Binding, rows: number, d: number, mod: Mod | null, eps?: number,
                     offset?: number, dtype?: DType): Buffer;
/** src/model/ops.ts:85 */
export function noMod(graph: Graph, d: number): Mod;
/** src/model/ops.ts:89 */
export function rotate(graph: Graph, x: Binding, heads: number, rope: Rope, pairing?: Pairing, dtype?: DType): Buffer;
/** src/kernels/attention.ts:20 */
export function attention(graph: Graph, q: Binding, k: Binding, v: Binding,
                          shape: { tokens: number; heads: number; kvHeads: number; dim: number; causal?: boolean },
                          dtype?: DType): Buffer;
/** src/model/ops.ts:102-113 */
export function swiglu(graph: Graph, gate: Binding, up: Binding, n: number, dtype?: DType): Buffer;
export function sigmoidGate(graph: Graph, a: Binding, gate: Binding, n: number, dtype?: DType): Buffer;
export function gatedAdd(graph: Graph, x: Binding, h: Binding, g: Binding, n: number, d: number, dtype?: DType): Buffer;
export function addBias(graph: Graph, x: Binding, b: Binding, n: number, d: number, dtype?: DType): Buffer;
export function add(graph: Graph, x: Binding, h: Binding, n: number, dtype?: DType): Buffer;
export function gelu(graph: Graph, x: Binding, n: number, dtype?: DType): Buffer;
export function silu(graph: Graph, x: Binding, n: number, dtype?: DType): Buffer;

/** src/weights/safetensors.ts:28-70, on a path, with the reference's messages. */
export class SafetensorsError extends Error {}
export type TensorInfo = { name: string; dtype: string; shape: number[]; offset: number; size: number; index: number };
export function readHeader(path: string): { tensors: Map<string, TensorInfo>; metadata: Record<string, string>;
                                            handle: bigint; close(): void };
export function readTensor(st: { handle: bigint }, tensor: TensorInfo, limit?: number, dst?: Uint8Array | Pinned,
                           threads?: number, offset?: number): Uint8Array | Pinned;
export function lastError(graph?: Graph | null): string;
export const addon: Record<string, (...args: unknown[]) => unknown>;

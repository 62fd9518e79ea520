/*
 * we.h — C ABI of the MI355X (gfx950) quantized-weight matmul path.
 *
 * Plain C: pointers, sizes and integer status codes; no PyTorch or HIP types in any signature.
 * Every entry point returns WE_OK (0) or an error code and leaves a message in we_last_error(ctx).
 * Device buffers are plain device pointers owned by the context (like the reference's Graph owns its
 * GPUBuffers). All work is queued in order on the context's compute stream; results are visible to
 * the host after we_buf_download or we_sync.
 *
 * Each declaration names the reference interface it replaces (paths in the dotstories/web-engine tree).
 */
#ifndef WE_H
#define WE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define WE_OK 0
#define WE_EINVAL 1       /* bad shape / stride / alignment / argument; message = the reference's text */
#define WE_ENOMEM 2       /* device or pinned-host allocation failed */
#define WE_EHIP 3         /* a HIP runtime call failed; message carries hipGetErrorString */
#define WE_EUNSUPPORTED 4 /* a dtype combination or mode the library does not implement */
#define WE_EFORMAT 5      /* not a valid .safetensors file; message = the reference's SafetensorsError text */
#define WE_EIO 6          /* a file could not be opened or read */
#define WE_ENOTFOUND 7    /* no tensor of that name */

/* dtype tags (activations, weights, outputs) */
#define WE_F32 0
#define WE_F16 1
#define WE_BF16 2
#define WE_FP8_E4M3 3 /* OCP float8_e4m3fn, one byte per value, K contiguous */
#define WE_INT4 4     /* 8 two's-complement nibbles per LE u32 along K, low nibble first; f16 scale per group */

/* matmul epilogue flags (combinable; applied in this order: scale, bias, gelu, accumulate) */
#define WE_EPI_ACCUMULATE 1u /* y += ... (src/kernels/matmul.ts:145) */
#define WE_EPI_SPLIT_K 2u    /* slice z of K into rows z*M.. of y (src/kernels/matmul.ts:155-159) */
#define WE_EPI_BIAS 4u       /* + bias[col] (f32), the addBias pass of src/model/ops.ts:65 fused */
#define WE_EPI_GELU_TANH 8u  /* tanh GELU of the result (src/kernels/elementwise.ts:25-29) fused */

/* elementwise ops (src/kernels/elementwise.ts:38-84) */
#define WE_OP_SWIGLU 0       /* out = silu(a) * b */
#define WE_OP_SIGMOID_GATE 1 /* out = a * sigmoid(b) */
#define WE_OP_GATED_ADD 2    /* out = a + c[i % d] * b */
#define WE_OP_ADD_BIAS 3     /* out = a + b[i % d] */
#define WE_OP_GELU_TANH 4    /* out = gelu_tanh(a) */
#define WE_OP_ADD 5          /* out = a + b */
#define WE_OP_SILU 6         /* out = a * sigmoid(a) */

typedef struct we_ctx we_ctx;

/* Binary image of the reference's matmul Params buffer: 13 x u32, scale stored as f32
 * (src/kernels/matmul.ts:120-126). Strides and offsets are in values, not bytes. */
typedef struct we_matmul_params {
  uint32_t m, n, k;
  float scale;
  uint32_t x_stride, w_stride, y_stride;
  uint32_t x_offset, w_offset, y_offset;
  uint32_t width, cin; /* 3x3 convolution input (we_conv3x3_params, src/kernels/matmul.ts:74-83); 0 for a GEMM */
  uint32_t k_split;
} we_matmul_params;

/* ---- context: replaces getDevice (src/gpu/compute.ts:6-20) and the Graph object (src/gpu/graph.ts:26-35) ---- */
int we_ctx_create(int device, we_ctx** out);
int we_ctx_destroy(we_ctx* ctx);
const char* we_last_error(const we_ctx* ctx); /* ctx = NULL: the last context-free failure of this thread */
/* device name, compute-unit count, LDS bytes per workgroup (for reports) */
int we_device_info(we_ctx* ctx, char* name, size_t name_len, int* compute_units, int* lds_bytes);

/* ---- buffers: Graph.buffer / free / release / mark / copy / read / stats (src/gpu/graph.ts:38-139) ---- */
int we_buf_alloc(we_ctx* ctx, size_t bytes, void** out);  /* zeroed, size-keyed pool */
int we_buf_free(we_ctx* ctx, void* buf);                   /* back to the pool; later use is stream-ordered */
int we_buf_upload(we_ctx* ctx, void* buf, size_t offset, const void* src, size_t bytes); /* queue.writeBuffer */
int we_buf_download(we_ctx* ctx, const void* buf, size_t offset, void* dst, size_t bytes); /* Graph.read */
int we_buf_copy(we_ctx* ctx, const void* src, size_t src_offset, void* dst, size_t dst_offset, size_t bytes);
/* Graph.read without blocking (src/gpu/graph.ts:109-119, whose mapAsync resolves later): queues the copy of
 * `bytes` at buf + offset into pinned memory of this context (we_host_alloc) after the work queued so far, and
 * returns a ticket; the data is there once we_ticket_wait (or we_ticket_done) reports the ticket done. */
int we_buf_download_async(we_ctx* ctx, const void* buf, size_t offset, void* pinned_dst, size_t bytes,
                          uint64_t* ticket);
int we_mark(we_ctx* ctx, size_t* mark);                                         /* Graph.mark */
int we_release(we_ctx* ctx, size_t mark, void* const* keep, size_t n_keep);     /* Graph.release */
int we_stats(we_ctx* ctx, uint64_t* created, uint64_t* reused, uint64_t* created_bytes); /* Graph.stats */
/* Failure injection and debugging, additive (the reference meets these failures through WebGPU's out-of-memory
 * error scope, src/probe/measure.ts:27-38, and hides stale data by zeroing reused buffers, src/gpu/graph.ts:48-51):
 *  - we_set_alloc_cap: the device bytes the context may hold at once (pool buffers + kernel scratch; 0 = no cap).
 *    An allocation past it fails as a full device does: WE_ENOMEM, and the context stays usable. `held` (may be
 *    NULL) receives the bytes held now. Taking a buffer from the pool allocates nothing and is never refused.
 *  - we_set_poison: on (1), we_buf_free and we_release fill each buffer they pool with 0xff bytes (NaN as f32,
 *    bf16, f16 and e4m3) on the compute stream, after the work queued so far, so a kernel that reads a freed
 *    buffer reads NaN instead of stale plausible values. Reused buffers are still zeroed by we_buf_alloc. */
int we_set_alloc_cap(we_ctx* ctx, uint64_t bytes, uint64_t* held);
int we_set_poison(we_ctx* ctx, int on);

/* Kernel-choice switches, per context. Additive: the reference's tuner (src/bench/tune.ts:5-30) compiles shader
 * variants from TUNE_CONFIGS (src/kernels/matmul-tuned.ts:13-125); here the variants are built in and a switch pins
 * one, for tile sweeps, measurements and tests. A context starts from the environment as it is at we_ctx_create
 * (WE_GEMM_CFG=<id>, WE_GEMM_PATH=generic, WE_GEMM_SPLITK=off|<slices>, WE_GEMM_REDUCE_XCD=off,
 * WE_ATTN_PATH=registers|ring|mfma16, WE_INT4_PATH=generic|shared|pipe); launches read the context, never the environment.
 * we_set_tuning sets one key (WE_EINVAL for an unknown key or a value out of range) and returns the old value in
 * `previous` (may be NULL). */
#define WE_TUNE_GEMM_CFG 0        /* fast-GEMM tile: 0 256x256, 1 256x128, 2 128x128, 3 64x64, 4 32x64, 5 256x192; -1 by shape */
#define WE_TUNE_GEMM_GENERIC 1    /* 1: the general GEMM kernel only */
#define WE_TUNE_GEMM_SPLITK 2     /* -1: split-K plan by shape, 0: off, n > 0: n slices */
#define WE_TUNE_GEMM_REDUCE_XCD 3 /* 1: the split-K reduce reads each tile on its XCD where that pays, 0: never */
#define WE_TUNE_ATTN_PATH 4       /* 0: default, 1: register-staged kernel, 2: DMA ring with a V^T pre-pass,
                                     3: ping-pong kernel on 16x16x32 MFMAs */
#define WE_TUNE_INT4_PATH 5       /* 0: by shape, 1: general kernel, 2: shared-x kernel, 3: LDS-ring decode kernel */
int we_set_tuning(we_ctx* ctx, int key, int value, int* previous);

int we_sync(we_ctx* ctx); /* device.queue.onSubmittedWorkDone(), called from src/model/weights.ts:128 */

/* Two compute streams. No counterpart in the reference, whose WebGPU queue is one ordered stream: for
 * callers that overlap independent work, like the double-stream block's text and image streams.
 * we_stream_select picks the stream that later calls queue on (0: the main stream, 1: the second one);
 * each stream has its own kernel scratch. we_stream_fork makes stream 1 wait for the work queued so far on
 * stream 0; we_stream_join makes stream 0 wait for the work queued so far on stream 1. Work on the two
 * streams is ordered only through these two calls (we_sync waits for both). Buffers that stream 1 uses, or
 * that are allocated while it is selected (they are zeroed on it), are ready for stream 0 after a join; do
 * not free or release them before one. Timers, tickets, downloads and graph capture use the selected
 * stream; selecting, forking and joining are refused during a capture. */
int we_stream_select(we_ctx* ctx, int stream);
int we_stream_fork(we_ctx* ctx);
int we_stream_join(we_ctx* ctx);

/* ---- pinned host memory and weight streaming: replaces the per-block upload pacing of
 * loadTransformer (src/model/weights.ts:124-129) and runAhead (src/gpu/run-ahead.ts:7-21) ---- */
int we_host_alloc(we_ctx* ctx, size_t bytes, void** out); /* pinned (hipHostMalloc) */
int we_host_free(we_ctx* ctx, void* ptr);
/* WE_OK when [p, p + bytes) lies inside one live we_host_alloc block of this context, else WE_EINVAL. No
 * counterpart in the reference (WebGPU owns its staging memory): bindings call it before they write into
 * pinned memory on a script's behalf, so a wrong offset or length, or a write after we_host_free, is refused. */
int we_host_span(we_ctx* ctx, const void* p, size_t bytes);
/* enqueue dst <- pinned src on the copy stream after the compute work recorded by `after` (0 = none);
 * returns a ticket that compute can wait on */
int we_stream_copy(we_ctx* ctx, void* dst, const void* pinned_src, size_t bytes, uint64_t after, uint64_t* ticket);
int we_wait_ticket(we_ctx* ctx, uint64_t ticket);   /* compute stream waits for a copy ticket */
int we_record_compute(we_ctx* ctx, uint64_t* ticket); /* ticket for the compute work queued so far */
int we_ticket_done(we_ctx* ctx, uint64_t ticket, int* done);
/* Blocks the calling host thread until the ticket's work is done: the wait behind a Promise of
 * device.queue.onSubmittedWorkDone() (src/model/weights.ts:128) or of an asynchronous read. It touches only the
 * ticket's event, so a binding may call it from a worker thread while its main thread keeps using ctx; a failure's
 * message is in we_last_error(NULL) of the waiting thread. Tickets live in a ring of 1024 events: a wait must start
 * before 1024 newer tickets exist and should end before that many more are made (the slot is then re-recorded). */
int we_ticket_wait(we_ctx* ctx, uint64_t ticket);
/* Three tickets, for the work queued so far on compute stream 0, compute stream 1 and the copy stream: all three
 * done is device.queue.onSubmittedWorkDone() (src/model/weights.ts:128, src/gpu/run-ahead.ts:5). */
int we_record_all(we_ctx* ctx, uint64_t tickets[3]);

/* ---- timing on the compute stream (hipEvents) ---- */
int we_timer_start(we_ctx* ctx);
int we_timer_stop(we_ctx* ctx, float* ms);
/* Timestamps between kernels without a host round trip, for harnesses that time each step of a running sequence (the
 * per-op timings of profileBlock, src/bench/block.ts:17-95, which the reference takes with submit-and-wait):
 * we_timer_mark records a timestamp into slot (0 .. WE_TIMER_MARKS - 1) after the work queued so far on the selected
 * compute stream, without waiting; we_timer_between waits for slot `to` and returns the milliseconds from slot `from`
 * to it. A slot keeps its last mark. */
#define WE_TIMER_MARKS 256
int we_timer_mark(we_ctx* ctx, uint32_t slot);
int we_timer_between(we_ctx* ctx, uint32_t from, uint32_t to, float* ms);

/* ---- HIP graphs of the compute stream: no counterpart in the reference (WebGPU records a command buffer
 * per submit). For launch-bound loops (decode steps, small GEMMs) and callers that replay a fixed sequence:
 * we_graph_begin starts capturing the kernels later calls queue on the compute stream; we_graph_end
 * instantiates them; we_graph_launch replays them in stream order. Between begin and end only kernel-
 * queuing calls and we_buf_copy are allowed: allocation, host transfers, syncs, tickets and timers fail.
 * A replay reads and writes the buffers the captured calls named, with their contents at replay time.
 * Kernels that need scratch (split-K partial sums, attention's V^T) replay into the scratch block of the stream
 * they were captured on: a graph keeps that block alive until we_graph_destroy, also when a later eager call
 * outgrows it, and we_graph_launch refuses to run a graph while the other compute stream is selected. Replays
 * of graphs captured on one stream share that stream's scratch, so they run one after another in its order. */
typedef struct we_graph we_graph;
int we_graph_begin(we_ctx* ctx);
int we_graph_end(we_ctx* ctx, we_graph** graph);
int we_graph_launch(we_ctx* ctx, we_graph* graph);
int we_graph_destroy(we_ctx* ctx, we_graph* graph);

/* ---- matmul: matmulParams (src/kernels/matmul.ts:198-212) and kSplitFor (src/model/ops.ts:42-45) ---- */
/* negative stride/offset = the reference's default; fails with "<name> must be a multiple of 4, got v" */
int we_matmul_params_make(we_ctx* ctx, uint32_t m, uint32_t n, uint32_t k, float scale, int64_t x_stride,
                          int64_t w_stride, int64_t y_stride, int64_t x_offset, int64_t w_offset, int64_t y_offset,
                          int64_t k_split, we_matmul_params* out);
uint32_t we_ksplit_for(uint32_t m, uint32_t n, uint32_t k);
/* conv3x3Params (src/kernels/matmul.ts:268-272): the Params of a 3x3 convolution with padding 1 as a GEMM:
 * M = height * width pixels, N = cout, K = 9 * cin, width and cin set; fails with "cin must be a multiple of 4,
 * got <cin>". we_matmul with these Params reads x as a channel-last image [height, width, cin] (row m a pixel,
 * k over (tap, channel), the 9 neighbours gathered in the kernel with zeros outside the image: the conv3x3 input
 * of src/kernels/matmul.ts:74-83) and W as [cout, (ky, kx, cin)]. Plain epilogues only (scale, bias, GELU,
 * accumulate, split-K); no int4 weights. */
int we_conv3x3_params(we_ctx* ctx, uint32_t height, uint32_t width, uint32_t cin, uint32_t cout,
                      we_matmul_params* out);

/* y = x . W^T * scale with W [N, K] as stored (fp8 / bf16 / f16 / f32 / int4). Replaces matmulWgsl
 * (src/kernels/matmul.ts:118-178) dispatched by linear() (src/model/ops.ts:61-73).
 * x: x_dtype in {F32, F16, BF16}; y: y_dtype in {F32, F16, BF16}; w_scales: int4 only, f16 [N, K/group];
 * bias: f32 [N] with WE_EPI_BIAS. Accumulation is fp32 on bf16/f16 MFMA (f32 operands are split into
 * three bf16 planes whose sum is the f32 value exactly, so every product keeps all 24 mantissa bits). */
int we_matmul(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
              const void* w_scales, uint32_t group, int y_dtype, void* y, const float* bias, uint32_t flags);
/* we_matmul that allocates nothing. No counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving or decode loops, harnesses that forbid hipMalloc). Same arguments,
 * kernels and results as we_matmul; the split-K partial sums that small-M GEMMs (M <= 64, and larger M with few
 * output tiles) keep in scratch go to a fixed per-GPU device array of 16 MiB instead of the context's scratch,
 * which holds every M <= 64 shape. A GEMM whose split plan needs more fails with WE_EINVAL, "... needs <n> bytes of
 * split-K scratch; the allocation-free entry point has 16777216 (use we_matmul)". Every call on one GPU shares that
 * GPU's array, so calls that could overlap are refused rather than raced: the array belongs to the first live
 * context that calls this on the GPU until that context is destroyed (another context's call fails with WE_EINVAL),
 * and a call while compute stream 1 is selected fails with WE_EINVAL. Calls of the owning context on stream 0 run
 * in stream order; each call's split-K slices write every partial sum before its reduce pass reads them, so what a
 * previous call left in the array is never read. */
int we_matmul_noalloc(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                      const void* w_scales, uint32_t group, int y_dtype, void* y, const float* bias, uint32_t flags);
/* we_matmul with the gated residual of the reference's gatedAdd (src/kernels/elementwise.ts:52-58, used after the
 * attention output and MLP down projections, src/model/block.ts:60-64 and :80) fused into the epilogue:
 *   y = residual + gate[col] * v,  v = the value we_matmul would store (scale, bias, GELU)
 * gate: f32 [N]; residual: y's dtype and layout (y_offset, y_stride), may be y itself; residual NULL: y = gate * v,
 * or y += gate * v with WE_EPI_ACCUMULATE. Not with WE_EPI_SPLIT_K. No reference entry point: the reference runs
 * gatedAdd as its own pass over the GEMM's output. */
int we_matmul_gated(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                    const void* w_scales, uint32_t group, int y_dtype, void* y, const float* bias, uint32_t flags,
                    const float* gate, const void* residual);

/* we_matmul with the elementwise step that consumes its output fused into the epilogue, as a product with a second
 * operand `aux` of y's dtype and layout (y_offset, y_stride; aux may be y itself):
 *   WE_MUL_SWIGLU:       y = silu(aux) * v, swiglu(gate, up) (src/kernels/elementwise.ts:38-43) with this GEMM as
 *                        `up` and the gate projection's output as aux (the MLP of src/model/block.ts:74-81);
 *   WE_MUL_SIGMOID_GATE: y = aux * sigmoid(v), sigmoidGate(a, gate) (elementwise.ts:45-50) with this GEMM as `gate`
 *                        and the attention output as aux (src/model/block.ts:60-62).
 * v is the value we_matmul would store (scale, then bias with WE_EPI_BIAS); other flags are refused, and int4
 * weights give WE_EUNSUPPORTED. v is not rounded to y's dtype before the product (the unfused pair rounds it
 * once more). No reference entry point: the reference runs these steps as their own passes. */
#define WE_MUL_SWIGLU 1
#define WE_MUL_SIGMOID_GATE 2
int we_matmul_mul(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                  const void* w_scales, uint32_t group, int y_dtype, void* y, const float* bias, uint32_t flags, int mul,
                  const void* aux);

/* A fused QKV projection with the q/k path of attend() (src/model/block.ts:53-56: per-head RMSNorm of q and k, then
 * RoPE) in its epilogue. Output columns [0, q_heads * 128) are q heads, the next k_heads * 128 are k heads, the rest
 * (v) is stored as we_matmul stores it. Each q / k head (128 values of a row t) is RMS-normalized (eps, offset,
 * weight norm_q / norm_k f32 [128]) and, when cos / sin are given, rotated on rows t >= rope_from with interleaved
 * pairs and cos / sin row t - rope_from (f32 [rows, 64]); the formulas of we_qk_norm_rope. x 16-bit, any weight but
 * int4; flags: WE_EPI_BIAS only. Where the GEMM's tile is aligned to heads (256 x 128 or 128 x 128 tiles, no
 * split-K plan; 16-bit y; e.g. a 512-token text stream) the norm and rotation run in the epilogue, and the value is not rounded to y's
 * dtype before the norm; otherwise the call runs the GEMM and then we_qk_norm_rope over the q and k columns, in
 * place. No reference entry point: the reference runs linear, norm and rotate as separate passes. */
int we_matmul_qk_norm_rope(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype,
                           const void* w, int y_dtype, void* y, const float* bias, uint32_t flags, uint32_t q_heads,
                           uint32_t k_heads, float eps, float offset, const float* norm_q, const float* norm_k,
                           uint32_t rope_from, const float* cos_t, const float* sin_t);

/* Two GEMMs of one N, K, dtypes and flags as one launch. No counterpart in the reference, which dispatches every
 * linear() on its own (src/model/ops.ts:61-73): for callers with independent GEMMs of one shape, like a double-stream
 * block whose text and image streams project with their own weights. Each item holds the arguments of one
 * we_matmul_gated call (gate and residual NULL: a plain epilogue; bias with WE_EPI_BIAS). With 16-bit x, fp8 or
 * matching 16-bit weights and 16-byte aligned rows, the tiles of both run in one launch with all of K per tile (no
 * split-K), in the tile shape picked for the two row counts together: a small GEMM beside a large one then adds no
 * launch and no partly empty round of tiles of its own. Each result equals a separate we_matmul_gated call made
 * with that tile shape (WE_TUNE_GEMM_CFG) and no split-K plan. A pair whose items depend on each other (one item's
 * y overlaps the other's y, x, w, bias, gate or residual bytes), any other pair, and count 1 run as separate calls
 * in order, item 0 first. Every item is checked before anything is launched; count must be 1 or 2. */
typedef struct we_matmul_item {
  const we_matmul_params* p;
  const void* x;
  const void* w;
  void* y;
  const float* bias;
  const float* gate;
  const void* residual;
} we_matmul_item;
int we_matmul_group(we_ctx* ctx, uint32_t count, const we_matmul_item* items, int x_dtype, int w_dtype, int y_dtype,
                    uint32_t flags);

/* ---- norms and rotary: rmsnormWgsl (src/kernels/rmsnorm.ts:13-48) / norm() (src/model/ops.ts:78-82),
 * ropeKernel (src/kernels/rope.ts:59-77) / rotate() (src/model/ops.ts:89-93) ---- */
/* out = x / sqrt(mean(x^2) + eps) * (offset + weight) * (1 + scale) + shift; scale/shift may be NULL */
int we_rmsnorm(we_ctx* ctx, uint32_t rows, uint32_t d, float eps, float offset, int dtype, const void* x,
               const float* weight, const float* scale, const float* shift, void* out);
/* The modulation add of src/model/block.ts:33-37 (mod = tvec + table, the six vectors of a block) folded into the
 * norm that first consumes it (block.ts:96: norm1 with prescale / preshift), one launch:
 *   mod[j] = tvec[j] + table[j] for j < mod_n (for the block's later consumers: gates, norm2);
 *   out = we_rmsnorm(x) with scale = mod[0:d], shift = mod[d:2d], computed in the kernel with the same f32 adds.
 * tvec, table, mod: f32 [mod_n], mod_n >= 2 d; mod may not overlap tvec, table, x or out. rows, d >= 1. */
int we_rmsnorm_mod(we_ctx* ctx, uint32_t rows, uint32_t d, float eps, float offset, int dtype, const void* x,
                   const float* weight, const float* tvec, const float* table, uint32_t mod_n, float* mod, void* out);
/* x [tokens, heads, 2*pairs]; cos/sin f32 [tokens, pairs]; half = 0 interleaved pairs, 1 (j, j+pairs) */
int we_rope(we_ctx* ctx, uint32_t tokens, uint32_t heads, uint32_t pairs, int half, int dtype, const void* x,
            const float* cos_t, const float* sin_t, void* out);
/* the q/k path of attend() (src/model/block.ts:53-56) in one pass: per-head RMSNorm (offset, eps) of
 * x [tokens, heads, head_dim], then RoPE on tokens >= rope_from (earlier tokens are only normalized);
 * cos/sin row r belongs to token rope_from + r. Token t's heads start at t * x_stride of x and
 * t * out_stride of out (0 = heads * head_dim), so q and k can be read from a fused QKV row. */
int we_qk_norm_rope(we_ctx* ctx, uint32_t tokens, uint32_t heads, uint32_t head_dim, float eps, float offset,
                    const float* weight, uint32_t rope_from, int half, const float* cos_t, const float* sin_t,
                    int dtype, const void* x, uint32_t x_stride, void* out, uint32_t out_stride);

/* ---- attention: attention(graph, q, k, v, shape) (src/kernels/attention.ts:20-51) ---- */
/* out[t, h] = softmax(q[t, h] . k[j, g]^T / sqrt(dim)) . v[j, g] over keys j (causal: j <= t), g = h / (heads /
 * kv_heads); fails with "heads must be a multiple of kvHeads" (attention.ts:23). Token t of q starts at
 * t * q_stride elements (0 = heads * dim; k and v: 0 = kv_heads * dim; out: 0 = heads * dim), so q, k and v
 * may be slices of one fused QKV row. dtype F32 (exact f32 products), BF16 or F16 (fp32 scores, softmax and
 * accumulation; probabilities rounded to the operand type). dim: a multiple of 8 (F32: 4), at most 128.
 * The reference's `chunk` only bounds its score buffer; no score matrix exists here, so it has no analogue. */
int we_attention(we_ctx* ctx, uint32_t tokens, uint32_t heads, uint32_t kv_heads, uint32_t dim, int causal, int dtype,
                 const void* q, uint32_t q_stride, const void* k, uint32_t k_stride, const void* v, uint32_t v_stride,
                 void* out, uint32_t out_stride);

/* ---- elementwise and reductions (src/kernels/elementwise.ts:38-84, src/kernels/text.ts:67-84) ---- */
int we_elementwise(we_ctx* ctx, int op, size_t n, size_t d, int dtype, const void* a, const void* b, const void* c,
                   void* out);
int we_layer_sum(we_ctx* ctx, uint32_t tokens, uint32_t layers, uint32_t dim, const float* x, const float* w,
                 float* out);

/* ---- dequantization test kernels: unpackFp8 (src/kernels/fp8.ts:24-36) and the int4 format ---- */
int we_unpack_fp8(we_ctx* ctx, const void* packed, size_t n, const float* scale, float* out);
int we_dequant_int4(we_ctx* ctx, const uint32_t* words, const uint16_t* scales, uint32_t rows, uint32_t k,
                    uint32_t group, float* out);

/* ---- peak probes: timePeak (src/bench/peak.ts:69-109) ----
 * One dispatch of a math-peak kernel on the compute stream (time it with we_timer_start / we_timer_stop).
 * F32 / F16 / I8 as the reference: workgroups of 64 threads, each thread `iters` iterations of 64 operations
 * (8 independent chains of fma / packed-f16 fma / int8 dot4); F32 uses scalar FMAs. MFMA_BF16: workgroups of
 * 256 threads, each wave 8 independent chains of v_mfma_f32_32x32x16_bf16 per iteration (4096 FLOP per thread
 * per iteration) on small constant operands: the ceiling of the matmul's MFMA loop. MFMA_BF16_DATA: the same work
 * on v_mfma_f32_16x16x32_bf16 (the large GEMM tiles' shape) on operands with the fp8-weight GEMM's bit statistics
 * (random bf16 activations, weights decoded from random e4m3fn codes, rotated every MFMA): the ceiling at the power
 * those data draw. out: u32 [workgroups x threads]
 * receives each thread's folded result; *ops (may be NULL) the operation count of the dispatch. No counterpart in
 * the reference for the two MFMA kinds (src/bench/peak.ts times the shader ALUs only). */
#define WE_PEAK_F32 0
#define WE_PEAK_F16 1
#define WE_PEAK_I8 2
#define WE_PEAK_MFMA_BF16 3
#define WE_PEAK_MFMA_BF16_DATA 4
int we_peak(we_ctx* ctx, int kind, uint32_t workgroups, uint32_t iters, uint32_t* out, double* ops);
/* One streaming read of `bytes` (a multiple of 16, 16-byte aligned) from buf, every load in flight at once; each
 * wave's sum of the words it read goes to out (u32 [4 * ceil(bytes / 32768)]): the HBM read ceiling the int4 GEMV
 * is measured against (over more than the 256 MB Infinity Cache). */
int we_read_peak(we_ctx* ctx, const void* buf, size_t bytes, uint32_t* out);

/* ---- .safetensors files: readHeader / readTensor (src/weights/safetensors.ts:28-70) ----
 * we_st_open reads and validates the header (8-byte LE size, JSON object of {dtype, shape, data_offsets}
 * entries plus optional __metadata__) with the reference's checks and messages: "File is too small to be a
 * .safetensors file", "Bad header size: n" (over 100,000,000 or past the end), "Header is not valid JSON",
 * "Header is not an object", "<name>: unknown dtype <d>", "<name>: bad shape", "<name>: bad data_offsets",
 * "<name>: has n bytes, its shape needs m bytes", "<name>: data goes past the end of the file", "<a> and <b>
 * overlap" (WE_EFORMAT; we_last_error(NULL)). Tensors are listed in the order the reference's Map holds them;
 * offsets are absolute file offsets. Nothing but the header is read until we_st_read, which reads bytes
 * [begin, begin + bytes) of one tensor straight into dst (any host memory, e.g. from we_host_alloc) with up to
 * `threads` parallel positional reads (0 = 8). A handle is read-only after open: reads may run concurrently.
 * Strings and shapes returned stay valid until we_st_close. */
typedef struct we_safetensors we_safetensors;
typedef struct we_tensor_info {
  const char* name;
  const char* dtype; /* "F8_E4M3", "BF16", "F32", ... (DTYPE_BYTES, src/weights/safetensors.ts:8-11) */
  uint32_t ndim;
  const uint64_t* shape;
  uint64_t offset; /* absolute file offset of the first byte */
  uint64_t size;   /* bytes */
} we_tensor_info;
int we_st_open(const char* path, we_safetensors** out);
int we_st_close(we_safetensors* st);
int we_st_count(const we_safetensors* st, uint32_t* n);
int we_st_info(const we_safetensors* st, uint32_t index, we_tensor_info* out);
int we_st_find(const we_safetensors* st, const char* name, uint32_t* index); /* WE_ENOTFOUND: "Missing tensor <name>" */
int we_st_metadata_count(const we_safetensors* st, uint32_t* n);             /* the string entries of __metadata__ */
int we_st_metadata_at(const we_safetensors* st, uint32_t index, const char** key, const char** value);
int we_st_read(const we_safetensors* st, uint32_t index, uint64_t begin, uint64_t bytes, void* dst, uint32_t threads);

#ifdef __cplusplus
}
#endif
#endif

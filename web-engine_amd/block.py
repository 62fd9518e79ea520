"""Transformer blocks on the MI355X kernels, and per-block weight streaming from pinned host memory.

- `positions`, `rope_tables`: src/kernels/rope.ts:14-36 (host-side, f64 angles stored as f32).
- `block`: the Krea single-stream block of src/model/block.ts:91-105 (attend :40-65, mlp :74-81, modulation
  :33-37), step for step through the operator API of we.py, freeing each temporary after its last use; the
  sigmoid gate runs in the gate projection's epilogue and SwiGLU in the up projection's, each writing over its
  first input instead of a new buffer.
- `DoubleBlock`: the double-stream DiT block (text and image streams with their own weights, one joint
  attention), built from the same steps with a persistent workspace so a forward allocates nothing:
    mod_s = tvec + table_s;  h_s = norm1_s(x_s) * (1 + prescale_s) + preshift_s  (one launch: the norm writes mod_s)
    [q|k|v]_s = h_s . qkv_s^T (both streams write one [text + image, 3 hidden] buffer, text rows first)
    q_s, k_s: per-head RMSNorm, then RoPE on the image rows (in the QKV GEMM's epilogue for the text stream,
    whose 128 x 128 tiles align with heads; in place right after it for the image stream)
    o = attention(q, k, v) read straight from the fused rows;  x1_s = x_s + pregate_s * (o_s . proj_s^T)
    out_s = x1_s + postgate_s * down_s(gelu_tanh(up_s(norm2_s(x1_s) * (1 + postscale_s) + postshift_s)))
  The GELU runs in the up projection's epilogue, and both gated residuals in the epilogues of the output
  projection and the down projection (we_matmul_gated): no elementwise pass touches the residual stream.
- `BlockStreamer`: src/model/weights.ts:94-131 loads every block before the first step and paces uploads
  with onSubmittedWorkDone; src/gpu/run-ahead.ts:7-21 keeps one block of CPU encoding ahead. Here a block's
  weights live in pinned host memory and are copied on the copy stream into one of two device slots while
  the block before computes from the other slot.
"""
import numpy as np

import we

MOD = ("prescale", "preshift", "pregate", "postscale", "postshift", "postgate")  # src/model/block.ts:30


class BlockConfig:
    """src/model/block.ts:6 (hidden, mlp, heads, kvHeads, headDim, eps)."""

    def __init__(self, hidden, mlp, heads, kv_heads, head_dim, eps=1e-5):
        self.hidden, self.mlp, self.heads, self.kv_heads, self.head_dim, self.eps = (hidden, mlp, heads, kv_heads,
                                                                                      head_dim, eps)


KREA_BLOCK = BlockConfig(6144, 16384, 48, 12, 128, 1e-5)  # src/model/block.ts:8
DIT_DOUBLE_BLOCK = BlockConfig(3072, 12288, 24, 24, 128, 1e-6)  # 24 heads x 128, RMSNorm eps 1e-6


# ------------------------------------------------------------------------------------------------ RoPE tables

def positions(text_tokens, rows, columns):
    """src/kernels/rope.ts:14-18: text tokens at (0, 0, 0), image token i at (0, i // columns, i % columns)."""
    text = np.zeros((text_tokens, 3))
    i = np.arange(rows * columns)
    image = np.stack([np.zeros(rows * columns), i // columns, i % columns], axis=1)
    return np.concatenate([text, image]).astype(np.float64)


def rope_tables(pos, axes, theta):
    """src/kernels/rope.ts:20-36: per axis of dim D, angle = pos * theta^(-2j / D), cos/sin as f32 [tokens, pairs]."""
    if any(d % 2 for d in axes):
        raise ValueError("Every RoPE axis needs an even number of dims")
    pos = np.asarray(pos, np.float64)
    cols = []
    for axis, dim in enumerate(axes):
        j = np.arange(dim // 2, dtype=np.float64)
        cols.append(pos[:, axis:axis + 1] * theta ** (-(2 * j) / dim))
    angle = np.concatenate(cols, axis=1)
    return np.cos(angle).astype(np.float32), np.sin(angle).astype(np.float32), sum(axes) // 2


# ------------------------------------------------------------------------------------------ Krea single stream

class BlockWeights:
    """src/model/block.ts:11-28: the eight linears (we.Linear), norm1, norm2, normQ, normK and table buffers."""

    def __init__(self, wq, wk, wv, gate, wo, mlp_gate, mlp_up, mlp_down, norm1, norm2, norm_q, norm_k, table):
        self.wq, self.wk, self.wv, self.gate, self.wo = wq, wk, wv, gate, wo
        self.mlp_gate, self.mlp_up, self.mlp_down = mlp_gate, mlp_up, mlp_down
        self.norm1, self.norm2, self.norm_q, self.norm_k, self.table = norm1, norm2, norm_q, norm_k, table


def modulation(graph, tvec, table, hidden):
    """src/model/block.ts:33-37: mod = tvec + table; the six vectors as slices of it."""
    mod = we.add(graph, tvec, table, 6 * hidden)
    return _mod_parts(mod, hidden), mod


def _mod_parts(mod, hidden):
    return {name: we.Graph.slice(mod, i * hidden * 4, hidden * 4) for i, name in enumerate(MOD)}


def _used(graph, x, f):
    """src/model/block.ts:68-72: f(x), then x is freed."""
    y = f(x)
    graph.free(x)
    return y


def _attend(graph, w, cfg, h, rows, rope, dtype):
    """src/model/block.ts:40-65. The per-head norm and the RoPE of q and k run as one pass, in place."""
    def projected(lin, n, norm_w):
        y = we.linear(graph, h, lin, rows, x_dtype=dtype, y_dtype=dtype)
        graph.qk_norm_rope(rows, n, cfg.head_dim, cfg.eps, 1.0, norm_w, 0 if rope else rows, False,
                           rope.cos if rope else None, rope.sin if rope else None, dtype, y, y)
        return y

    q = projected(w.wq, cfg.heads, w.norm_q)
    k = projected(w.wk, cfg.kv_heads, w.norm_k)
    v = we.linear(graph, h, w.wv, rows, x_dtype=dtype, y_dtype=dtype)
    o = we.attention(graph, q, k, v, we.AttentionShape(rows, cfg.heads, cfg.kv_heads, cfg.head_dim), dtype)
    for b in (q, k, v):
        graph.free(b)
    # o * sigmoid(h . gate^T): the sigmoid gate in the gate projection's epilogue, written over o
    we.linear(graph, h, w.gate, rows, x_dtype=dtype, y_dtype=dtype, sigmoid_gate_of=o, out=o)
    return _used(graph, o, lambda y: we.linear(graph, y, w.wo, rows, x_dtype=dtype, y_dtype=dtype))


def _mlp(graph, w, cfg, h, rows, dtype):
    """src/model/block.ts:74-81"""
    gate = we.linear(graph, h, w.mlp_gate, rows, x_dtype=dtype, y_dtype=dtype)
    # silu(gate) * (h . up^T): swiglu in the up projection's epilogue, written over gate
    we.linear(graph, h, w.mlp_up, rows, x_dtype=dtype, y_dtype=dtype, swiglu_gate=gate, out=gate)
    return _used(graph, gate, lambda y: we.linear(graph, y, w.mlp_down, rows, x_dtype=dtype, y_dtype=dtype))


def block(graph, w, cfg, x, tvec, rope, dtype=we.F32):
    """src/model/block.ts:91-105: one Krea single-stream block; x [tokens, hidden] -> new [tokens, hidden]."""
    t, hidden = rope.tokens, cfg.hidden
    # modulation (block.ts:33-37) folded into norm1 (block.ts:96): one launch writes mod and h
    mod_buf = graph.buffer(6 * hidden * 4)
    h = graph.buffer(t * hidden * we.ELEM_BYTES[dtype])
    graph.rmsnorm_mod(t, hidden, cfg.eps, 1.0, dtype, x, w.norm1, tvec, w.table, 6 * hidden, mod_buf, h)
    mod = _mod_parts(mod_buf, hidden)
    a = _used(graph, h, lambda y: _attend(graph, w, cfg, y, t, rope, dtype))
    x1 = _used(graph, a, lambda y: we.gated_add(graph, x, y, mod["pregate"], t * hidden, hidden, dtype))
    h2 = we.norm(graph, x1, w.norm2, t, hidden, we.Mod(mod["postscale"], mod["postshift"]), cfg.eps, 1.0, dtype)
    m = _used(graph, h2, lambda y: _mlp(graph, w, cfg, y, t, dtype))
    out = we.gated_add(graph, x1, m, mod["postgate"], t * hidden, hidden, dtype)
    for b in (m, x1, mod_buf):
        graph.free(b)
    return out


# ------------------------------------------------------------------------------------------ double stream (DiT)

class StreamWeights:
    """One stream's weights: qkv [3 hidden, hidden], proj [hidden, hidden], up [mlp, hidden], down [hidden, mlp]
    (we.Linear, fp8), and f32 vectors norm1, norm2 [hidden], norm_q, norm_k [head_dim], table [6 hidden]."""

    def __init__(self, qkv, proj, up, down, norm1, norm2, norm_q, norm_k, table):
        self.qkv, self.proj, self.up, self.down = qkv, proj, up, down
        self.norm1, self.norm2, self.norm_q, self.norm_k, self.table = norm1, norm2, norm_q, norm_k, table


class DoubleBlock:
    """The double-stream block at fixed token counts, with its workspace allocated once. With overlap (the
    default) the text stream's steps run on the context's second compute stream, beside the image stream's:
    the two streams meet only in the joint attention, and the text stream's small GEMMs fill workgroup slots
    the image stream leaves free. With grouped (the default, with overlap) the QKV, output, up and down
    projections of the two streams run as one launch each (we_matmul_group), the QKV launch followed by the q / k
    RMSNorm (+ RoPE) passes. The result is the same bit for bit as serial calls that use the same tile shapes."""

    def __init__(self, graph, cfg, txt_tokens, img_tokens, dtype=we.BF16, overlap=True, grouped=True):
        if cfg.heads != cfg.kv_heads or cfg.heads * cfg.head_dim != cfg.hidden:
            raise ValueError("the double-stream block needs heads == kvHeads and heads * headDim == hidden")
        self.graph, self.cfg, self.dtype = graph, cfg, dtype
        self.rows = (txt_tokens, img_tokens)
        self.row0 = (0, txt_tokens)
        self.tokens = txt_tokens + img_tokens
        H, e = cfg.hidden, we.ELEM_BYTES[dtype]
        big = max(self.rows)
        self.qkv = graph.buffer(self.tokens * 3 * H * e)
        self.o = graph.buffer(self.tokens * H * e)
        self.overlap = overlap
        self.grouped = grouped and overlap  # the grouped projections use each stream's own buffers
        self.group_qkv = self.grouped  # the QKV projections grouped as well (then q / k normalized by passes)
        if overlap:  # each stream its own norm output and MLP hidden
            self.h = [graph.buffer(r * H * e) for r in self.rows]
            self.u = [graph.buffer(r * cfg.mlp * e) for r in self.rows]
        else:
            h, u = graph.buffer(big * H * e), graph.buffer(big * cfg.mlp * e)
            self.h, self.u = [h, h], [u, u]
        self.x1 = [graph.buffer(r * H * e) for r in self.rows]
        self.mod = [graph.buffer(6 * H * 4) for _ in self.rows]

    def free(self):
        for b in [self.qkv, self.o] + list({id(b): b for b in self.h + self.u}.values()) + self.x1 + self.mod:
            self.graph.free(b)

    def _streams(self, step):
        """step(s) for the text (s = 0) and image (s = 1) streams: text on the second compute stream when
        overlapping, then stream 0 waits for it."""
        g = self.graph
        if not self.overlap:
            step(0)
            step(1)
            return
        g.fork()
        g.stream(1)
        try:
            step(0)
        finally:
            g.stream(0)
        step(1)
        g.join()

    def forward(self, w_txt, w_img, x_txt, x_img, tvec, rope_img, out_txt, out_img):
        """x_s, out_s: [rows_s, hidden] of the block's dtype; tvec f32 [6 hidden]; rope_img: we.Rope over the
        image tokens (interleaved pairs). out_s may not alias x_s."""
        g, cfg, dt = self.graph, self.cfg, self.dtype
        H, hd, heads, e = cfg.hidden, cfg.head_dim, cfg.heads, we.ELEM_BYTES[dt]
        sl = we.Graph.slice
        ws, xs, outs = (w_txt, w_img), (x_txt, x_img), (out_txt, out_img)

        def qkv_step(s):
            w, rows, r0, h = ws[s], self.rows[s], self.row0[s], self.h[s]
            # mod = tvec + table (for the gates and norm2 below) written by norm1, which folds the add in
            g.rmsnorm_mod(rows, H, cfg.eps, 1.0, dt, xs[s], w.norm1, tvec, w.table, 6 * H, self.mod[s], h)
            # the fused QKV projection: per-head RMSNorm of q and k (and RoPE on the image stream) in the GEMM's
            # epilogue where its tile is head-aligned (the text stream), else a pass right after it
            p = we.matmul_params(rows, 3 * H, H, w.qkv.scale, y_offset=r0 * 3 * H, graph=g)
            rotate = s == 1
            cos, sin = (rope_img.cos, rope_img.sin) if rotate else (None, None)
            if hd == 128:
                g.matmul_qk_norm_rope(p, dt, h, we.FP8, w.qkv.buffer, dt, self.qkv, heads, heads, cfg.eps, 1.0,
                                      w.norm_q, w.norm_k, 0, cos, sin)
                return
            g.matmul(p, dt, h, we.FP8, w.qkv.buffer, dt, self.qkv)
            for part, norm_w in ((0, w.norm_q), (1, w.norm_k)):
                base = sl(self.qkv, (r0 * 3 * H + part * H) * e, 0)
                g.qk_norm_rope(rows, heads, hd, cfg.eps, 1.0, norm_w, 0 if rotate else rows, False, cos, sin, dt, base,
                               base, x_stride=3 * H, out_stride=3 * H)

        def out_step(s):
            w, rows, r0, mod, h, u = ws[s], self.rows[s], self.row0[s], self.mod[s], self.h[s], self.u[s]
            # x1 = x + gate1 * proj(o), the gated residual in the projection's epilogue
            p = we.matmul_params(rows, H, H, w.proj.scale, x_offset=r0 * H, graph=g)
            g.matmul(p, dt, self.o, we.FP8, w.proj.buffer, dt, self.x1[s], gate=sl(mod, 2 * H * 4, H * 4),
                     residual=xs[s])
            g.rmsnorm(rows, H, cfg.eps, 1.0, dt, self.x1[s], w.norm2, sl(mod, 3 * H * 4, H * 4),
                      sl(mod, 4 * H * 4, H * 4), h)
            g.matmul(we.matmul_params(rows, cfg.mlp, H, w.up.scale, graph=g), dt, h, we.FP8, w.up.buffer, dt,
                     u, flags=we.EPI_GELU)
            # out = x1 + gate2 * down(u), fused likewise
            g.matmul(we.matmul_params(rows, H, cfg.mlp, w.down.scale, graph=g), dt, u, we.FP8, w.down.buffer, dt,
                     outs[s], gate=sl(mod, 5 * H * 4, H * 4), residual=self.x1[s])

        def out_grouped():
            # the output and down projections of the two streams share N and K: each pair runs as one launch
            # (we_matmul_group), the text tiles beside the image tiles in one round, with the gated residuals
            # x1 = x + gate1 * proj(o) and out = x1 + gate2 * down(u) in the epilogues
            g.matmul_group([dict(params=we.matmul_params(self.rows[s], H, H, ws[s].proj.scale, x_offset=self.row0[s] * H,
                                                         graph=g),
                                 x=self.o, w=ws[s].proj.buffer, y=self.x1[s], gate=sl(self.mod[s], 2 * H * 4, H * 4),
                                 residual=xs[s]) for s in (0, 1)], dt, we.FP8, dt)
            for s in (0, 1):
                g.rmsnorm(self.rows[s], H, cfg.eps, 1.0, dt, self.x1[s], ws[s].norm2, sl(self.mod[s], 3 * H * 4, H * 4),
                          sl(self.mod[s], 4 * H * 4, H * 4), self.h[s])
            # the up projections share N and K too: one launch with GELU in its epilogue
            g.matmul_group([dict(params=we.matmul_params(self.rows[s], cfg.mlp, H, ws[s].up.scale, graph=g),
                                 x=self.h[s], w=ws[s].up.buffer, y=self.u[s]) for s in (0, 1)], dt, we.FP8, dt,
                           we.EPI_GELU)
            g.matmul_group([dict(params=we.matmul_params(self.rows[s], H, cfg.mlp, ws[s].down.scale, graph=g),
                                 x=self.u[s], w=ws[s].down.buffer, y=outs[s], gate=sl(self.mod[s], 5 * H * 4, H * 4),
                                 residual=self.x1[s]) for s in (0, 1)], dt, we.FP8, dt)

        def qkv_grouped():
            # the two QKV projections share N and K: one launch (we_matmul_group) writes both streams' rows of the
            # shared [text + image, 3 hidden] buffer; then the per-head RMSNorm of q and k (and RoPE on the image
            # rows) as passes, in place
            self._streams(lambda s: g.rmsnorm_mod(self.rows[s], H, cfg.eps, 1.0, dt, xs[s], ws[s].norm1, tvec,
                                                  ws[s].table, 6 * H, self.mod[s], self.h[s]))
            g.matmul_group([dict(params=we.matmul_params(self.rows[s], 3 * H, H, ws[s].qkv.scale,
                                                         y_offset=self.row0[s] * 3 * H, graph=g),
                                 x=self.h[s], w=ws[s].qkv.buffer, y=self.qkv) for s in (0, 1)], dt, we.FP8, dt)
            for s in (0, 1):
                rotate = s == 1
                cos, sin = (rope_img.cos, rope_img.sin) if rotate else (None, None)
                for part, norm_w in ((0, ws[s].norm_q), (1, ws[s].norm_k)):
                    base = sl(self.qkv, (self.row0[s] * 3 * H + part * H) * e, 0)
                    g.qk_norm_rope(self.rows[s], heads, hd, cfg.eps, 1.0, norm_w, 0 if rotate else self.rows[s], False,
                                   cos, sin, dt, base, base, x_stride=3 * H, out_stride=3 * H)

        if self.group_qkv:
            qkv_grouped()
        else:
            self._streams(qkv_step)
        g.attention(self.tokens, heads, heads, hd, False, dt, self.qkv, sl(self.qkv, H * e, 0),
                    sl(self.qkv, 2 * H * e, 0), self.o, q_stride=3 * H, k_stride=3 * H, v_stride=3 * H, out_stride=H)
        if self.grouped:
            out_grouped()
        else:
            self._streams(out_step)

    def profile(self, w_txt, w_img, x_txt, x_img, tvec, rope_img, out_txt, out_img, reps=5, warm=None):
        """Where the block's time goes (profileBlock, src/bench/block.ts:17-95): the steps of forward() in its
        order, each run on its own on compute stream 0 (`reps` back-to-back calls between HIP events, after one
        untimed call, or after warm(step) where given: a caller's untimed run-up, e.g. until the clocks settle),
        per stream, without the overlap and grouping of forward(). Every step rewrites its outputs from inputs it
        does not write, so repeating it changes nothing. Returns [{name, kind, us}], kind one of linear /
        attention / other as in the reference."""
        g, cfg, dt = self.graph, self.cfg, self.dtype
        H, hd, heads, e = cfg.hidden, cfg.head_dim, cfg.heads, we.ELEM_BYTES[dt]
        sl = we.Graph.slice
        ws, xs, outs, names = (w_txt, w_img), (x_txt, x_img), (out_txt, out_img), ("text", "image")
        steps = []
        for s in (0, 1):
            w, rows, r0, h, u, mod = ws[s], self.rows[s], self.row0[s], self.h[s], self.u[s], self.mod[s]
            cos, sin = (rope_img.cos, rope_img.sin) if s == 1 else (None, None)
            steps += [
                (f"norm 1 + modulation ({names[s]})", "other",
                 lambda w=w, rows=rows, h=h, mod=mod, s=s: g.rmsnorm_mod(rows, H, cfg.eps, 1.0, dt, xs[s], w.norm1,
                                                                          tvec, w.table, 6 * H, mod, h)),
                (f"qkv + q/k norm{' + rope' if s else ''} ({names[s]})", "linear",
                 lambda w=w, rows=rows, r0=r0, h=h, cos=cos, sin=sin: g.matmul_qk_norm_rope(
                     we.matmul_params(rows, 3 * H, H, w.qkv.scale, y_offset=r0 * 3 * H, graph=g), dt, h, we.FP8,
                     w.qkv.buffer, dt, self.qkv, heads, heads, cfg.eps, 1.0, w.norm_q, w.norm_k, 0, cos, sin))]
        steps.append(("attention (joint)", "attention",
                      lambda: g.attention(self.tokens, heads, heads, hd, False, dt, self.qkv, sl(self.qkv, H * e, 0),
                                          sl(self.qkv, 2 * H * e, 0), self.o, q_stride=3 * H, k_stride=3 * H,
                                          v_stride=3 * H, out_stride=H)))
        for s in (0, 1):
            w, rows, r0, h, u, mod = ws[s], self.rows[s], self.row0[s], self.h[s], self.u[s], self.mod[s]
            steps += [
                (f"out + gated residual ({names[s]})", "linear",
                 lambda w=w, rows=rows, r0=r0, mod=mod, s=s: g.matmul(
                     we.matmul_params(rows, H, H, w.proj.scale, x_offset=r0 * H, graph=g), dt, self.o, we.FP8,
                     w.proj.buffer, dt, self.x1[s], gate=sl(mod, 2 * H * 4, H * 4), residual=xs[s])),
                (f"norm 2 ({names[s]})", "other",
                 lambda w=w, rows=rows, h=h, mod=mod, s=s: g.rmsnorm(rows, H, cfg.eps, 1.0, dt, self.x1[s], w.norm2,
                                                                      sl(mod, 3 * H * 4, H * 4),
                                                                      sl(mod, 4 * H * 4, H * 4), h)),
                (f"mlp up + gelu ({names[s]})", "linear",
                 lambda w=w, rows=rows, h=h, u=u: g.matmul(we.matmul_params(rows, cfg.mlp, H, w.up.scale, graph=g), dt,
                                                           h, we.FP8, w.up.buffer, dt, u, flags=we.EPI_GELU)),
                (f"mlp down + gated residual ({names[s]})", "linear",
                 lambda w=w, rows=rows, u=u, mod=mod, s=s: g.matmul(
                     we.matmul_params(rows, H, cfg.mlp, w.down.scale, graph=g), dt, u, we.FP8, w.down.buffer, dt,
                     outs[s], gate=sl(mod, 5 * H * 4, H * 4), residual=self.x1[s]))]
        out = []
        for name, kind, fn in steps:
            if warm is None:
                fn()
            else:
                warm(fn)
            g.sync()
            g.timer_start()
            for _ in range(reps):
                fn()
            out.append({"name": name, "kind": kind, "us": g.timer_stop() / reps * 1e3})
        return out


# ------------------------------------------------------------------------------------------ weight streaming

def _align(n, a=256):
    return (n + a - 1) // a * a


class StreamLayout:
    """Byte layout of one double-stream block's weights, identical in pinned host memory and in a device
    slot: per stream qkv, proj, up, down (fp8), then norm1, norm2, norm_q, norm_k, table (f32)."""

    def __init__(self, cfg):
        H, M, hd = cfg.hidden, cfg.mlp, cfg.head_dim
        self.cfg = cfg
        self.fields, off = [], 0
        for s in ("txt", "img"):
            for name, nbytes in (("qkv", 3 * H * H), ("proj", H * H), ("up", M * H), ("down", H * M),
                                 ("norm1", 4 * H), ("norm2", 4 * H), ("norm_q", 4 * hd), ("norm_k", 4 * hd),
                                 ("table", 24 * H)):
                self.fields.append((s, name, off, nbytes))
                off = _align(off + nbytes)
        self.nbytes = off
        self.fp8_bytes = 2 * (3 * H * H + H * H + 2 * M * H)

    def weights(self, base, scales):
        """StreamWeights (text, image) over the buffer at `base`; scales[s][name] = per-tensor fp8 scale."""
        views = {}
        for s, name, off, nbytes in self.fields:
            views[(s, name)] = we.Graph.slice(base, off, nbytes)
        cfg = self.cfg
        H, M = cfg.hidden, cfg.mlp
        out = []
        for s in ("txt", "img"):
            lin = lambda name, n, k: we.Linear(views[(s, name)], "fp8", scales[s][name], n, k)  # noqa: E731
            out.append(StreamWeights(lin("qkv", 3 * H, H), lin("proj", H, H), lin("up", M, H), lin("down", H, M),
                                     views[(s, "norm1")], views[(s, "norm2")], views[(s, "norm_q")],
                                     views[(s, "norm_k")], views[(s, "table")]))
        return out

    # tensor names of one block in a .safetensors file, after the block's prefix ("double_blocks.7."): per stream
    # "<txt|img>_" + the name below; fp8 weights carry "<name>.weight" and "<name>.weight_scale" (F32 [1], or
    # ".scale_weight"), norms [H] / [head_dim] and the modulation table [6, H] any float dtype
    FILE_NAMES = {"qkv": "attn.qkv", "proj": "attn.proj", "up": "mlp.0", "down": "mlp.2", "norm1": "norm1.weight",
                  "norm2": "norm2.weight", "norm_q": "attn.norm_q.weight", "norm_k": "attn.norm_k.weight",
                  "table": "mod.table"}
    FP8_FIELDS = ("qkv", "proj", "up", "down")

    def _shape(self, name):
        H, M, hd = self.cfg.hidden, self.cfg.mlp, self.cfg.head_dim
        return {"qkv": (3 * H, H), "proj": (H, H), "up": (M, H), "down": (H, M), "norm1": (H,), "norm2": (H,),
                "norm_q": (hd,), "norm_k": (hd,), "table": (6, H)}[name]

    def fill_from_file(self, st, prefix, dst, threads=0):
        """One block's weights from an open weights.Safetensors into the host image at address `dst` (pinned
        memory, so the streamer copies them to HBM as they are): fp8 weights are read from the file straight
        into place, small float tensors are converted to f32. Returns the scales (for `weights`)."""
        import weights as W
        scales = {"txt": {}, "img": {}}
        for s, name, off, nbytes in self.fields:
            fname = f"{prefix}{s}_{self.FILE_NAMES[name]}"
            if name in self.FP8_FIELDS:
                n, k = self._shape(name)
                scales[s][name] = W.load_linear_fp8(st, fname, n, k, int(dst) + off, threads)
            else:
                W.load_floats_into(st, fname, nbytes // 4, int(dst) + off)
        return scales

    def file_tensors(self, image, scales, prefix):
        """The tensors of one block image (a uint8 array of nbytes) under the names fill_from_file reads, for
        weights.save."""
        out = {}
        for s, name, off, nbytes in self.fields:
            fname = f"{prefix}{s}_{self.FILE_NAMES[name]}"
            data = image[off:off + nbytes]
            if name in self.FP8_FIELDS:
                out[fname + ".weight"] = ("F8_E4M3", self._shape(name), data)
                out[fname + ".weight_scale"] = ("F32", (1,), np.array([scales[s][name]], np.float32).view(np.uint8))
            else:
                out[fname] = ("F32", self._shape(name), data)
        return out

    def fill(self, dst, rng, vec_scale=0.3):
        """Random-init weights into a uint8 view `dst` of nbytes: fp8 codes uniform over the 254 finite ones,
        norm weights and tables uniform in +-vec_scale."""
        for s, name, off, nbytes in self.fields:
            if name in ("qkv", "proj", "up", "down"):
                b = rng.integers(0, 254, nbytes, dtype=np.uint8)
                dst[off:off + nbytes] = b + (b >= 0x7f) + (b >= 0xfe)  # skip 0x7f and 0xff
            else:
                dst[off:off + nbytes] = ((rng.random(nbytes // 4) * 2 - 1) * vec_scale).astype(np.float32).view(
                    np.uint8)


class BlockStreamer:
    """Double-buffered weight streaming: block i's weights are copied from its pinned host buffer into device
    slot i % 2 on the copy stream, once the block that last used that slot has been queued; the compute
    stream waits for the copy of block i only when it reaches block i."""

    def __init__(self, graph, layout, slots=2):
        self.graph, self.layout = graph, layout
        self.slots = [graph.buffer(layout.nbytes) for _ in range(slots)]

    def run(self, pinned, compute, start=0, blocks=None):
        """pinned: host buffers of the blocks (we.Graph.host_alloc results); block i's weights are
        pinned[i % len(pinned)]; blocks: how many blocks to run (default len(pinned)); compute(i, slot_buffer)
        queues block i's work; start: a compute ticket the first copies wait for (0 = none). Returns after
        queuing everything."""
        g, n = self.graph, len(self.slots)
        blocks = len(pinned) if blocks is None else blocks
        src = lambda i: pinned[i % len(pinned)]  # noqa: E731
        tickets = {}
        for i in range(min(n, blocks)):
            tickets[i] = g.stream_copy(self.slots[i], src(i), self.layout.nbytes, start)
        for i in range(blocks):
            g.wait_ticket(tickets.pop(i))
            compute(i, self.slots[i % n])
            if i + n < blocks:
                done = g.record_compute()
                tickets[i + n] = g.stream_copy(self.slots[i % n], src(i + n), self.layout.nbytes, done)

    def free(self):
        for b in self.slots:
            self.graph.free(b)


def rope_for_image(graph, rows, columns, axes=(64, 64), theta=10000.0):
    """2D-axial RoPE of a rows x columns image grid ((row, column) axes), as a we.Rope over the image tokens."""
    pos = positions(0, rows, columns)[:, 1:]
    cos, sin, pairs = rope_tables(pos, axes, theta)
    return we.Rope(graph.buffer(cos), graph.buffer(sin), pairs, rows * columns)


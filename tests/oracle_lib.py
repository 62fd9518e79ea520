"""ctypes binding of the CPU oracle (oracle/liboracle.so). Test infrastructure only: results are checked against it."""
import ctypes
import pathlib
import subprocess

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[1]
LIB_PATH = ROOT / "oracle" / "liboracle.so"

F32, F16, BF16, FP8, INT4 = 0, 1, 2, 3, 4
SWIGLU, SIGMOID_GATE, GATED_ADD, ADD_BIAS, GELU_TANH, ADD, SILU = range(7)


class Params(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("m", "n", "k")] + [("scale", ctypes.c_float)] + [
        (n, ctypes.c_uint32) for n in ("x_stride", "w_stride", "y_stride", "x_offset", "w_offset", "y_offset", "width",
                                       "cin", "k_split")]


class Linear(ctypes.Structure):
    _fields_ = [("bytes", ctypes.c_void_p), ("scale", ctypes.c_float), ("n", ctypes.c_uint32), ("k", ctypes.c_uint32)]


class BlockCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("hidden", "mlp", "heads", "kv_heads", "head_dim")] + [
        ("eps", ctypes.c_double)]


class StreamW(ctypes.Structure):
    _fields_ = [(n, Linear) for n in ("qkv", "proj", "up", "down")] + [
        (n, ctypes.c_void_p) for n in ("norm1", "norm2", "norm_q", "norm_k", "table")]


def _load():
    if not LIB_PATH.exists():
        subprocess.run(["make", "-C", str(LIB_PATH.parent)], check=True, capture_output=True)
    lib = ctypes.CDLL(str(LIB_PATH))
    P = ctypes.c_void_p
    u8, u16, u32, i64, f, d, sz = (ctypes.c_uint8, ctypes.c_uint16, ctypes.c_uint32, ctypes.c_int64, ctypes.c_float,
                                   ctypes.c_double, ctypes.c_size_t)
    sig = {
        "or_e4m3": (d, [u8]), "or_e4m3_gpu": (f, [u8]), "or_e5m2": (d, [u8]), "or_f16": (d, [u16]),
        "or_bf16": (f, [u16]), "or_f32_to_bf16": (u16, [f]), "or_f32_to_f16": (u16, [f]),
        "or_unpack_fp8": (None, [P, sz, f, P]), "or_int4_value": (f, [u32, ctypes.c_int, u16]),
        "or_dequant_int4": (None, [P, P, sz, sz, sz, P]),
        "or_lcg_next": (u32, [P]), "or_lcg_uniform": (d, [P]), "or_lcg_fill": (None, [u32, sz, P]),
        "or_matmul_test_data": (None, [u32, u32, u32, u32, P, P]),
        "or_mt_seed": (None, [P, ctypes.c_uint64]), "or_mt_next": (u32, [P]),
        "or_torch_randn": (None, [sz, ctypes.c_uint64, P]),
        "or_matmul_params_make": (ctypes.c_int, [u32, u32, u32, f, i64, i64, i64, i64, i64, i64, i64, P, P, sz]),
        "or_ksplit_for": (u32, [u32, u32, u32]), "or_ksplit_chunk": (u32, [u32, u32]),
        "or_conv3x3_params": (ctypes.c_int, [u32, u32, u32, u32, P, P, sz]),
        "or_matmul_f64": (None, [P, ctypes.c_int, P, ctypes.c_int, P, P, u32, ctypes.c_int, P]),
        "or_matmul_f64_rows": (None, [P, ctypes.c_int, P, ctypes.c_int, P, P, u32, u32, u32, P]),
        "or_layer_sum": (None, [u32, u32, u32, P, P, P]),
        "or_rmsnorm_f64": (None, [sz, sz, d, d, P, P, P, P, P]),
        "or_rope_positions": (None, [u32, u32, u32, u32, P]),
        "or_rope_tables": (ctypes.c_int, [P, u32, P, u32, d, P, P]),
        "or_rope_rotate_f64": (None, [u32, u32, u32, ctypes.c_int, P, P, P, P]),
        "or_attention_f64": (None, [u32, u32, u32, u32, ctypes.c_int, u32, u32, P, P, P, P]),
        "or_krea_block_f64": (None, [P, u32, P, P, P, P, P, P, P, P, P, P, P]),
        "or_double_block_f64": (None, [P, u32, u32, P, P, P, P, P, P, P, P, P]),
        "or_gelu_tanh": (d, [d]), "or_gelu_tanh_shader": (f, [f]), "or_sigmoid": (d, [d]),
        "or_elementwise_f64": (None, [ctypes.c_int, sz, sz, P, P, P, P]),
        "or_rel_error": (d, [P, P, sz]), "or_compare": (None, [P, P, sz, P, P, P]),
        "cb_matmul": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, u32, u32, u32, f, ctypes.c_int, P, ctypes.c_int, P,
                                     P, u32, ctypes.c_int, ctypes.c_int, P]),
        "cb_has_avx512": (ctypes.c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def c_contig(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def e4m3(b):
    return lib.or_e4m3(b)


def e4m3_table():
    return np.array([lib.or_e4m3(b) for b in range(256)])


def e4m3_gpu_table():
    return np.array([lib.or_e4m3_gpu(b) for b in range(256)], dtype=np.float32)


def unpack_fp8(data, scale):
    data = c_contig(data, np.uint8)
    out = np.empty(data.size, np.float32)
    lib.or_unpack_fp8(ptr(data), data.size, scale, ptr(out))
    return out


def to_bf16(a):
    a = c_contig(a, np.float32).ravel()
    return np.array([lib.or_f32_to_bf16(float(v)) for v in a], dtype=np.uint16)


def to_f16(a):
    a = c_contig(a, np.float32).ravel()
    return np.array([lib.or_f32_to_f16(float(v)) for v in a], dtype=np.uint16)


def bf16_to_f32(h):
    h = np.asarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def matmul_test_data(m, n, k, seed=1):
    x = np.empty(m * k, np.float32)
    w = np.empty(n * k, np.uint8)
    lib.or_matmul_test_data(m, n, k, seed, ptr(x), ptr(w))
    return x, w


def lcg(seed, count):
    out = np.empty(count, np.float64)
    lib.or_lcg_fill(seed, count, ptr(out))
    return out


def bf16_rne(a):
    """Vectorised f32 -> bf16 bits, round to nearest even (checked against or_f32_to_bf16 in test_oracle)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def torch_randn(n, seed):
    out = np.empty(n, np.float32)
    lib.or_torch_randn(n, seed, ptr(out))
    return out


def matmul_params(m, n, k, scale, x_stride=-1, w_stride=-1, y_stride=-1, x_offset=-1, w_offset=-1, y_offset=-1,
                  k_split=1):
    p = Params()
    msg = ctypes.create_string_buffer(256)
    rc = lib.or_matmul_params_make(m, n, k, scale, x_stride, w_stride, y_stride, x_offset, w_offset, y_offset,
                                   k_split, ctypes.byref(p), msg, 256)
    if rc:
        raise ValueError(msg.value.decode())
    return p


def matmul(p, x_dtype, x, w_dtype, w, scales=None, group=0, split=False, accumulate=False, y=None, out_len=None):
    """Float64 oracle matmul; returns the whole y buffer (size out_len, default rows * y_stride + y_offset)."""
    rows = p.m * (p.k_split if split else 1)
    if y is None:
        y = np.zeros(out_len if out_len is not None else rows * p.y_stride + p.y_offset, np.float64)
    else:
        y = c_contig(y, np.float64).copy()
    flags = (1 if split else 0) | (2 if accumulate else 0)
    lib.or_matmul_f64(ctypes.byref(p), x_dtype, ptr(x), w_dtype, ptr(w), ptr(scales), group, flags, ptr(y))
    return y


def matmul_rows(p, x_dtype, x, w_dtype, w, row_begin, row_end, scales=None, group=0):
    y = np.zeros(p.m * p.y_stride + p.y_offset, np.float64)
    lib.or_matmul_f64_rows(ctypes.byref(p), x_dtype, ptr(x), w_dtype, ptr(w), ptr(scales), group, row_begin, row_end,
                           ptr(y))
    return y


def cpu_matmul(m, n, k, scale, x_dtype, x, w_dtype, w, scales=None, group=0, y_dtype=F32, threads=1, avx512=True,
               gelu=False):
    """The strong CPU baseline (oracle/cpu_gemm.c): f32 accumulation on `threads` host threads; contiguous
    x [m, k], W [n, k]; tanh GELU on the result when `gelu`; returns y [m * n] as float32 (F32) or the 16-bit
    codes (F16 / BF16)."""
    y = np.empty(m * n, np.float32 if y_dtype == F32 else np.uint16)
    rc = lib.cb_matmul(threads, 1 if avx512 else 0, m, n, k, scale, x_dtype, ptr(x), w_dtype, ptr(w), ptr(scales),
                       group, y_dtype, 1 if gelu else 0, ptr(y))
    if rc != 0:
        raise ValueError("cb_matmul refused its arguments")
    return y


def conv3x3_params(height, width, cin, cout):
    """conv3x3Params (src/kernels/matmul.ts:268-272); raises ValueError with the reference's message."""
    p = Params()
    msg = ctypes.create_string_buffer(200)
    if lib.or_conv3x3_params(height, width, cin, cout, ctypes.byref(p), msg, 200):
        raise ValueError(msg.value.decode())
    return p


def ksplit_for(m, n, k):
    return lib.or_ksplit_for(m, n, k)


def ksplit_chunk(k, split):
    return lib.or_ksplit_chunk(k, split)


def layer_sum(tokens, layers, dim, x, w):
    out = np.empty(tokens * dim, np.float64)
    lib.or_layer_sum(tokens, layers, dim, ptr(c_contig(x, np.float32)), ptr(c_contig(w, np.float32)), ptr(out))
    return out


def rmsnorm(x, weight, eps=1e-5, offset=1.0, scale=None, shift=None):
    x = c_contig(x, np.float32)
    weight = c_contig(weight, np.float32)
    d = weight.size
    rows = x.size // d
    out = np.empty(x.size, np.float64)
    sc = None if scale is None else c_contig(scale, np.float32)
    sh = None if shift is None else c_contig(shift, np.float32)
    lib.or_rmsnorm_f64(rows, d, eps, offset, ptr(x), ptr(weight), ptr(sc), ptr(sh), ptr(out))
    return out


def rope_positions(text_tokens, rows, columns, axes):
    pos = np.empty((text_tokens + rows * columns) * axes, np.float64)
    lib.or_rope_positions(text_tokens, rows, columns, axes, ptr(pos))
    return pos.reshape(-1, axes)


def rope_tables(pos, axes, theta):
    pos = c_contig(pos, np.float64)
    tokens = pos.shape[0]
    ax = np.array(axes, dtype=np.uint32)
    pairs = int(sum(axes) // 2)
    cos = np.empty(tokens * pairs, np.float32)
    sin = np.empty(tokens * pairs, np.float32)
    rc = lib.or_rope_tables(ptr(pos), tokens, ptr(ax), len(axes), theta, ptr(cos), ptr(sin))
    if rc < 0:
        raise ValueError("Every RoPE axis needs an even number of dims")
    return cos, sin, pairs


def rope_rotate(x, tokens, heads, pairs, cos, sin, half=False):
    x = c_contig(x, np.float32)
    out = np.empty(x.size, np.float64)
    lib.or_rope_rotate_f64(tokens, heads, pairs, 1 if half else 0, ptr(x), ptr(c_contig(cos, np.float32)),
                           ptr(c_contig(sin, np.float32)), ptr(out))
    return out


def attention(q, k, v, tokens, heads, kv_heads, dim, causal=False, rows=None):
    """f64 attention of dense q [tokens, heads, dim], k/v [tokens, kv_heads, dim]; rows = (begin, end) of the
    query rows to compute (default all). Returns [rows, heads, dim] flattened."""
    q, k, v = (c_contig(a, np.float64) for a in (q, k, v))
    b, e = rows if rows is not None else (0, tokens)
    out = np.empty((e - b) * heads * dim, np.float64)
    lib.or_attention_f64(tokens, heads, kv_heads, dim, 1 if causal else 0, b, e, ptr(q), ptr(k), ptr(v), ptr(out))
    return out


def _lin(bytes_, scale, n, k, keep):
    b = c_contig(bytes_, np.uint8)
    keep.append(b)
    return Linear(b.ctypes.data, scale, n, k)


def _cfg(cfg):
    return BlockCfg(cfg.hidden, cfg.mlp, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.eps)


def krea_block(cfg, tokens, x, lins, norm1, norm2, norm_q, norm_k, table, temb, cos, sin):
    """lins: 8 (bytes, scale, n, k) in the order wq, wk, wv, gate, wo, mlpGate, mlpUp, mlpDown."""
    keep = []
    arr = (Linear * 8)(*[_lin(b, s, n, k, keep) for b, s, n, k in lins])
    vecs = [c_contig(v, np.float32) for v in (norm1, norm2, norm_q, norm_k, table, temb, cos, sin)]
    x = c_contig(x, np.float64)
    out = np.empty(tokens * cfg.hidden, np.float64)
    c = _cfg(cfg)
    lib.or_krea_block_f64(ctypes.byref(c), tokens, ptr(x), arr, *[ptr(v) for v in vecs], ptr(out))
    return out


def _stream(sw, keep):
    """sw: dict with qkv/proj/up/down = (bytes, scale, n, k) and f32 vectors norm1/norm2/norm_q/norm_k/table."""
    vecs = {n: c_contig(sw[n], np.float32) for n in ("norm1", "norm2", "norm_q", "norm_k", "table")}
    keep.extend(vecs.values())
    lins = {n: _lin(*sw[n], keep) for n in ("qkv", "proj", "up", "down")}
    return StreamW(**lins, **{n: v.ctypes.data for n, v in vecs.items()})


def double_block(cfg, txt_tokens, img_tokens, x_txt, x_img, w_txt, w_img, tvec, cos_img, sin_img):
    keep = []
    st, si = _stream(w_txt, keep), _stream(w_img, keep)
    x_txt, x_img = c_contig(x_txt, np.float64), c_contig(x_img, np.float64)
    tv, cs, sn = (c_contig(v, np.float32) for v in (tvec, cos_img, sin_img))
    out_t = np.empty(txt_tokens * cfg.hidden, np.float64)
    out_i = np.empty(img_tokens * cfg.hidden, np.float64)
    c = _cfg(cfg)
    lib.or_double_block_f64(ctypes.byref(c), txt_tokens, img_tokens, ptr(x_txt), ptr(x_img), ctypes.byref(st),
                            ctypes.byref(si), ptr(tv), ptr(cs), ptr(sn), ptr(out_t), ptr(out_i))
    return out_t, out_i


def double_block_rows(cfg, txt_tokens, img_tokens, x_txt, x_img, w_txt, w_img, tvec, cos_img, sin_img, rows_txt,
                      rows_img):
    """Outputs of the double-stream block for selected rows only (text rows `rows_txt`, image rows `rows_img`),
    composed in float64 numpy from the steps of or_double_block_f64: K and V of every token (attention needs all
    of them), everything else only for the selected rows. It makes the full 512 + 4096-token shape checkable on
    the CPU in seconds. Pinned to or_double_block_f64 row for row (test_oracle)."""
    H, hd, heads, eps = cfg.hidden, cfg.head_dim, cfg.heads, cfg.eps
    table = e4m3_table()
    T = txt_tokens + img_tokens

    def mm(x, lin, rows=None):
        b, scale, n, k = lin
        w = np.asarray(b, np.uint8).reshape(n, k)
        if rows is not None:
            w = w[rows]
        return (x @ table[w].T) * float(scale)

    def rms(x, w, scale=None, shift=None):
        x = np.asarray(x, np.float64)
        inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
        y = x * inv * (1.0 + np.asarray(w, np.float64))
        if scale is not None:
            y = y * (1.0 + scale) + shift
        return y

    def rope(x, c, s):  # x [rows, heads, hd], interleaved pairs; c, s [rows, hd / 2]
        a, b = x[..., 0::2], x[..., 1::2]
        c, s = c[:, None, :].astype(np.float64), s[:, None, :].astype(np.float64)
        out = np.empty_like(x)
        out[..., 0::2] = a * c - b * s
        out[..., 1::2] = b * c + a * s
        return out

    ws, xs = (w_txt, w_img), (np.asarray(x_txt, np.float64).reshape(-1, H), np.asarray(x_img, np.float64).reshape(-1, H))
    picks, row0 = (np.asarray(rows_txt, np.int64), np.asarray(rows_img, np.int64)), (0, txt_tokens)
    k_all, v_all = np.empty((T, heads, hd)), np.empty((T, heads, hd))
    q_sel, mods = [], []
    cos_img = np.asarray(cos_img, np.float32).reshape(img_tokens, hd // 2)
    sin_img = np.asarray(sin_img, np.float32).reshape(img_tokens, hd // 2)
    for s in range(2):
        w, x = ws[s], xs[s]
        mod = (np.asarray(tvec, np.float64) + np.asarray(w["table"], np.float64)).reshape(6, H)
        mods.append(mod)
        h = rms(x, w["norm1"], mod[0], mod[1])
        kv = mm(h, w["qkv"], np.arange(H, 3 * H))
        k = rms(kv[:, :H].reshape(-1, heads, hd), w["norm_k"])
        v = kv[:, H:].reshape(-1, heads, hd)
        q = rms(mm(h[picks[s]], w["qkv"], np.arange(0, H)).reshape(-1, heads, hd), w["norm_q"])
        if s == 1:
            k = rope(k, cos_img, sin_img)
            q = rope(q, cos_img[picks[s]], sin_img[picks[s]])
        k_all[row0[s]:row0[s] + x.shape[0]], v_all[row0[s]:row0[s] + x.shape[0]] = k, v
        q_sel.append(q)
    outs = []
    for s in range(2):
        w, mod, q = ws[s], mods[s], q_sel[s]
        sc = np.einsum("rhd,thd->rht", q, k_all) / np.sqrt(hd)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        o = np.einsum("rht,thd->rhd", p / p.sum(-1, keepdims=True), v_all).reshape(-1, H)
        x1 = xs[s][picks[s]] + mod[2] * mm(o, w["proj"])
        u = gelu_tanh(mm(rms(x1, w["norm2"], mod[3], mod[4]), w["up"]))
        outs.append(x1 + mod[5] * mm(u, w["down"]))
    return outs[0], outs[1]


def elementwise(op, a, b=None, c=None, d=1):
    a = c_contig(a, np.float32)
    bb = None if b is None else c_contig(b, np.float32)
    cc = None if c is None else c_contig(c, np.float32)
    out = np.empty(a.size, np.float64)
    lib.or_elementwise_f64(op, a.size, d, ptr(a), ptr(bb), ptr(cc), ptr(out))
    return out


def dequant_int4(words, scales, rows, k, group):
    words = c_contig(words, np.uint32)
    scales = c_contig(scales, np.uint16)
    out = np.empty(rows * k, np.float32)
    lib.or_dequant_int4(ptr(words), ptr(scales), rows, k, group, ptr(out))
    return out


def gelu_tanh(v):
    """Vectorized float64 tanh GELU (PyTorch gelu(approximate="tanh"), src/kernels/elementwise.ts:25-29), for checks
    over millions of outputs: 0.5 v (1 + tanh u) written as v / (1 + e^(-2u)), the same function without the
    cancellation of 1 + tanh u for negative v (below v = -5 the tanh form rounds to 0 where the value is ~1e-10
    and smaller). Pinned to or_gelu_tanh (to 1e-12) and the torch golden in test_oracle."""
    v = np.asarray(v, np.float64)
    u = np.sqrt(2.0 / np.pi) * (v + 0.044715 * v * v * v)
    with np.errstate(over="ignore"):
        return v / (1.0 + np.exp(-2.0 * u))


def rel_error(got, ref):
    got = c_contig(got, np.float64)
    ref = c_contig(ref, np.float64)
    return lib.or_rel_error(ptr(got), ptr(ref), ref.size)


def compare(result, reference):
    a = c_contig(result, np.float64)
    b = c_contig(reference, np.float64)
    cs, mx, rel = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    lib.or_compare(ptr(a), ptr(b), a.size, ctypes.byref(cs), ctypes.byref(mx), ctypes.byref(rel))
    return {"cosine": cs.value, "maxError": mx.value, "relativeError": rel.value}

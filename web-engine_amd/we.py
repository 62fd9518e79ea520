"""Python host side of the MI355X matmul path: a ctypes binding of libwe.so (include/we.h) and a
mirror of the reference's operator API over it.

  Graph                 src/gpu/graph.ts:26-155   (buffer / read / free / mark / release / copy / destroy / stats)
  matmul_params         src/kernels/matmul.ts:198-212
  k_split_for           src/model/ops.ts:42-45
  Linear, linear        src/model/ops.ts:24-32, 48-73 (bias fused in the GEMM epilogue; LoRA via split-K + accumulate)
  norm, no_mod          src/model/ops.ts:78-85
  rotate                src/model/ops.ts:89-93
  swiglu, sigmoid_gate, gated_add, add, gelu, silu      src/model/ops.ts:101-113
  matmul_fp8 / matmul_bf16 / matmul_f32 one-shots        src/kernels/matmul.ts:223-265
  unpack_fp8 one-shot   src/kernels/fp8.ts:24-36

Every op runs the hand-written gfx950 kernels in libwe.so; there is no CPU fallback. Importing works
without a GPU (the symbol checks use that); creating a Graph needs the library and a GPU and raises
otherwise.
"""
import contextlib
import ctypes
import os
import pathlib
import re

import numpy as np

PKG = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG / "libwe.so"
HEADER = PKG.parent / "include" / "we.h"

F32, F16, BF16, FP8, INT4 = 0, 1, 2, 3, 4
DTYPES = {"f32": F32, "f16": F16, "bf16": BF16, "fp8": FP8, "int4": INT4}
ELEM_BYTES = {F32: 4, F16: 2, BF16: 2, FP8: 1}
EPI_ACCUMULATE, EPI_SPLIT_K, EPI_BIAS, EPI_GELU = 1, 2, 4, 8
TIMER_MARKS = 256  # timestamp slots (WE_TIMER_MARKS)
# kernel-choice switches (we_set_tuning, WE_TUNE_* of include/we.h)
TUNE_KEYS = {"gemm_cfg": 0, "gemm_generic": 1, "gemm_splitk": 2, "gemm_reduce_xcd": 3, "attn_path": 4, "int4_path": 5}
MUL_SWIGLU, MUL_SIGMOID_GATE = 1, 2
OP_SWIGLU, OP_SIGMOID_GATE, OP_GATED_ADD, OP_ADD_BIAS, OP_GELU_TANH, OP_ADD, OP_SILU = range(7)
PEAK_F32, PEAK_F16, PEAK_I8, PEAK_MFMA_BF16, PEAK_MFMA_BF16_DATA = range(5)


def read_peak_out_words(nbytes):
    """u32 results of we_read_peak over nbytes (one per wave of 64 threads x 8 chunks of 16 bytes)"""
    return 4 * ((nbytes // 16 + 2047) // 2048)
ERRORS = {1: "WE_EINVAL", 2: "WE_ENOMEM", 3: "WE_EHIP", 4: "WE_EUNSUPPORTED", 5: "WE_EFORMAT", 6: "WE_EIO",
          7: "WE_ENOTFOUND"}
WE_EINVAL = 1
TILE = 128  # the reference's matmul tile (src/kernels/matmul.ts:33), used by k_split_for


class WeError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(message)
        self.code = code
        self.name = ERRORS.get(code, str(code))


class MatmulParams(ctypes.Structure):
    """Binary image of the reference's 13 x u32 matmul Params (src/kernels/matmul.ts:120-126)."""
    _fields_ = [("m", ctypes.c_uint32), ("n", ctypes.c_uint32), ("k", ctypes.c_uint32), ("scale", ctypes.c_float),
                ("x_stride", ctypes.c_uint32), ("w_stride", ctypes.c_uint32), ("y_stride", ctypes.c_uint32),
                ("x_offset", ctypes.c_uint32), ("w_offset", ctypes.c_uint32), ("y_offset", ctypes.c_uint32),
                ("width", ctypes.c_uint32), ("cin", ctypes.c_uint32), ("k_split", ctypes.c_uint32)]


class MatmulItem(ctypes.Structure):
    """we_matmul_item: the arguments of one GEMM of a we_matmul_group call."""
    _fields_ = [("p", ctypes.POINTER(MatmulParams)), ("x", ctypes.c_void_p), ("w", ctypes.c_void_p),
                ("y", ctypes.c_void_p), ("bias", ctypes.c_void_p), ("gate", ctypes.c_void_p),
                ("residual", ctypes.c_void_p)]


_P, _I, _U32, _U64, _SZ, _F, _I64 = (ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t,
                                     ctypes.c_float, ctypes.c_int64)
SIGNATURES = {
    "we_ctx_create": (_I, [_I, _P]),
    "we_ctx_destroy": (_I, [_P]),
    "we_last_error": (ctypes.c_char_p, [_P]),
    "we_device_info": (_I, [_P, ctypes.c_char_p, _SZ, _P, _P]),
    "we_buf_alloc": (_I, [_P, _SZ, _P]),
    "we_buf_free": (_I, [_P, _P]),
    "we_buf_upload": (_I, [_P, _P, _SZ, _P, _SZ]),
    "we_buf_download": (_I, [_P, _P, _SZ, _P, _SZ]),
    "we_buf_copy": (_I, [_P, _P, _SZ, _P, _SZ, _SZ]),
    "we_mark": (_I, [_P, _P]),
    "we_release": (_I, [_P, _SZ, _P, _SZ]),
    "we_stats": (_I, [_P, _P, _P, _P]),
    "we_sync": (_I, [_P]),
    "we_stream_select": (_I, [_P, ctypes.c_int]),
    "we_stream_fork": (_I, [_P]),
    "we_stream_join": (_I, [_P]),
    "we_host_alloc": (_I, [_P, _SZ, _P]),
    "we_host_free": (_I, [_P, _P]),
    "we_host_span": (_I, [_P, _P, ctypes.c_size_t]),
    "we_buf_download_async": (_I, [_P, _P, ctypes.c_size_t, _P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint64)]),
    "we_ticket_wait": (_I, [_P, ctypes.c_uint64]),
    "we_record_all": (_I, [_P, _P]),
    "we_set_alloc_cap": (_I, [_P, _U64, _P]),
    "we_set_poison": (_I, [_P, ctypes.c_int]),
    "we_set_tuning": (_I, [_P, ctypes.c_int, ctypes.c_int, _P]),
    "we_timer_mark": (_I, [_P, _U32]),
    "we_timer_between": (_I, [_P, _U32, _U32, _P]),
    "we_stream_copy": (_I, [_P, _P, _P, _SZ, _U64, _P]),
    "we_wait_ticket": (_I, [_P, _U64]),
    "we_record_compute": (_I, [_P, _P]),
    "we_ticket_done": (_I, [_P, _U64, _P]),
    "we_timer_start": (_I, [_P]),
    "we_timer_stop": (_I, [_P, _P]),
    "we_matmul_params_make": (_I, [_P, _U32, _U32, _U32, _F, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "we_ksplit_for": (_U32, [_U32, _U32, _U32]),
    "we_conv3x3_params": (_I, [_P, _U32, _U32, _U32, _U32, _P]),
    "we_matmul": (_I, [_P, _P, _I, _P, _I, _P, _P, _U32, _I, _P, _P, _U32]),
    "we_matmul_gated": (_I, [_P, _P, _I, _P, _I, _P, _P, _U32, _I, _P, _P, _U32, _P, _P]),
    "we_matmul_mul": (_I, [_P, _P, _I, _P, _I, _P, _P, _U32, _I, _P, _P, _U32, _I, _P]),
    "we_matmul_group": (_I, [_P, _U32, _P, _I, _I, _I, _U32]),
    "we_matmul_qk_norm_rope": (_I, [_P, _P, _I, _P, _I, _P, _I, _P, _P, _U32, _U32, _U32, _F, _F, _P, _P, _U32, _P,
                                    _P]),
    "we_matmul_noalloc": (_I, [_P, _P, _I, _P, _I, _P, _P, _U32, _I, _P, _P, _U32]),
    "we_rmsnorm": (_I, [_P, _U32, _U32, _F, _F, _I, _P, _P, _P, _P, _P]),
    "we_rmsnorm_mod": (_I, [_P, _U32, _U32, _F, _F, _I, _P, _P, _P, _P, _U32, _P, _P]),
    "we_rope": (_I, [_P, _U32, _U32, _U32, _I, _I, _P, _P, _P, _P]),
    "we_qk_norm_rope": (_I, [_P, _U32, _U32, _U32, _F, _F, _P, _U32, _I, _P, _P, _I, _P, _U32, _P, _U32]),
    "we_attention": (_I, [_P, _U32, _U32, _U32, _U32, _I, _I, _P, _U32, _P, _U32, _P, _U32, _P, _U32]),
    "we_elementwise": (_I, [_P, _I, _SZ, _SZ, _I, _P, _P, _P, _P]),
    "we_layer_sum": (_I, [_P, _U32, _U32, _U32, _P, _P, _P]),
    "we_unpack_fp8": (_I, [_P, _P, _SZ, _P, _P]),
    "we_dequant_int4": (_I, [_P, _P, _P, _U32, _U32, _U32, _P]),
    "we_graph_begin": (_I, [_P]),
    "we_graph_end": (_I, [_P, _P]),
    "we_graph_launch": (_I, [_P, _P]),
    "we_graph_destroy": (_I, [_P, _P]),
    "we_peak": (_I, [_P, _I, _U32, _U32, _P, _P]),
    "we_read_peak": (_I, [_P, _P, _SZ, _P]),
    "we_st_open": (_I, [ctypes.c_char_p, _P]),
    "we_st_close": (_I, [_P]),
    "we_st_count": (_I, [_P, _P]),
    "we_st_info": (_I, [_P, _U32, _P]),
    "we_st_find": (_I, [_P, ctypes.c_char_p, _P]),
    "we_st_metadata_count": (_I, [_P, _P]),
    "we_st_metadata_at": (_I, [_P, _U32, _P, _P]),
    "we_st_read": (_I, [_P, _U32, _U64, _U64, _P, _U32]),
}

_lib = None


def header_functions():
    """Names of every function declared in include/we.h."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|uint32_t|const char\*)\s+(we_\w+)\s*\(", text, re.M)))


def load_library(path=None):
    """Loads libwe.so (raising if it is missing) and declares every entry point's signature."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = pathlib.Path(path or os.environ.get("WE_LIB", LIB_PATH))
    if not p.exists():
        raise RuntimeError(f"{p} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


class Buffer:
    """A device buffer (or a slice of one, like Graph.slice): address and size in bytes."""
    __slots__ = ("ptr", "size", "base")

    def __init__(self, ptr, size, base=None):
        self.ptr, self.size, self.base = ptr, size, base

    def __int__(self):
        return self.ptr

    def __repr__(self):
        return f"Buffer(0x{self.ptr:x}, {self.size})"


def _addr(b):
    if b is None:
        return None
    if isinstance(b, Buffer):
        return ctypes.c_void_p(b.ptr)
    return ctypes.c_void_p(int(b))


class Graph:
    """Mirror of the reference's Graph (src/gpu/graph.ts:26-155) over one we_ctx: buffers stay on the GPU,
    work is queued in order on one compute stream, freed buffers are pooled by size and come back zeroed."""

    def __init__(self, device=0):
        self.lib = load_library()
        ctx = ctypes.c_void_p()
        rc = self.lib.we_ctx_create(device, ctypes.byref(ctx))
        if rc:
            raise WeError(rc, f"we_ctx_create(device={device}) failed with {ERRORS.get(rc, rc)}: no usable gfx950 GPU")
        self.ctx = ctx

    # ---- errors
    def check(self, rc):
        if rc:
            raise WeError(rc, self.lib.we_last_error(self.ctx).decode())

    # ---- Graph API
    def buffer(self, data=None, nbytes=None):
        """A zeroed buffer of `nbytes` bytes, or one holding `data` (a numpy array or bytes)."""
        arr = None
        if data is not None and not isinstance(data, int):
            arr = np.ascontiguousarray(data)
            nbytes = arr.nbytes
        elif isinstance(data, int):
            nbytes = data
        p = ctypes.c_void_p()
        self.check(self.lib.we_buf_alloc(self.ctx, nbytes, ctypes.byref(p)))
        buf = Buffer(p.value, nbytes)
        if arr is not None and nbytes:
            self.check(self.lib.we_buf_upload(self.ctx, _addr(buf), 0, arr.ctypes.data_as(ctypes.c_void_p), nbytes))
        return buf

    upload = buffer

    def write(self, buf, data, offset=0):
        arr = np.ascontiguousarray(data)
        self.check(self.lib.we_buf_upload(self.ctx, _addr(buf), offset, arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes))

    @staticmethod
    def slice(buf, offset, size):
        return Buffer(buf.ptr + offset, size, base=buf)

    def read(self, buf, nbytes=None, dtype=np.uint8, count=None):
        nbytes = buf.size if nbytes is None else nbytes
        if count is not None:
            nbytes = count * np.dtype(dtype).itemsize
        out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype)
        self.check(self.lib.we_buf_download(self.ctx, _addr(buf), 0, out.ctypes.data_as(ctypes.c_void_p), out.nbytes))
        return out

    def copy(self, src, src_offset, dst, dst_offset, size):
        self.check(self.lib.we_buf_copy(self.ctx, _addr(src), src_offset, _addr(dst), dst_offset, size))

    def free(self, buf):
        self.check(self.lib.we_buf_free(self.ctx, _addr(buf)))

    def mark(self):
        m = ctypes.c_size_t()
        self.check(self.lib.we_mark(self.ctx, ctypes.byref(m)))
        return m.value

    def release(self, mark, keep=()):
        arr = (ctypes.c_void_p * max(1, len(keep)))(*[b.ptr for b in keep])
        self.check(self.lib.we_release(self.ctx, mark, arr, len(keep)))

    @property
    def stats(self):
        c, r, b = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        self.check(self.lib.we_stats(self.ctx, ctypes.byref(c), ctypes.byref(r), ctypes.byref(b)))
        return {"created": c.value, "reused": r.value, "createdBytes": b.value}

    def sync(self):
        self.check(self.lib.we_sync(self.ctx))

    # ---- two compute streams (we_stream_select / fork / join)
    def stream(self, which):
        """Queue later calls on compute stream `which` (0: main, 1: second)."""
        self.check(self.lib.we_stream_select(self.ctx, which))

    def fork(self):
        """Stream 1 waits for the work queued so far on stream 0."""
        self.check(self.lib.we_stream_fork(self.ctx))

    def join(self):
        """Stream 0 waits for the work queued so far on stream 1."""
        self.check(self.lib.we_stream_join(self.ctx))

    on_submitted_work_done = sync

    def device_info(self):
        name = ctypes.create_string_buffer(64)
        cu, lds = ctypes.c_int(), ctypes.c_int()
        self.check(self.lib.we_device_info(self.ctx, name, 64, ctypes.byref(cu), ctypes.byref(lds)))
        return {"arch": name.value.decode(), "compute_units": cu.value, "lds_bytes": lds.value}

    def destroy(self):
        if getattr(self, "ctx", None):
            self.lib.we_ctx_destroy(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()

    # ---- pinned host memory and streaming
    def set_alloc_cap(self, nbytes):
        """Failure injection: allocations past `nbytes` device bytes held (0 = no cap) fail with WE_ENOMEM.
        Returns the bytes the context holds now."""
        held = ctypes.c_uint64()
        self.check(self.lib.we_set_alloc_cap(self.ctx, nbytes, ctypes.byref(held)))
        return held.value

    def set_poison(self, on):
        """Debugging: freed / released buffers are filled with 0xff bytes (NaN) once pooled."""
        self.check(self.lib.we_set_poison(self.ctx, 1 if on else 0))

    def set_tuning(self, key, value):
        """Sets one kernel-choice switch of this context (a TUNE_* key or its name, e.g. "gemm_cfg") and returns
        the previous value. The context starts from the WE_* environment variables as they were when it was made."""
        k = TUNE_KEYS[key] if isinstance(key, str) else int(key)
        prev = ctypes.c_int()
        self.check(self.lib.we_set_tuning(self.ctx, k, int(value), ctypes.byref(prev)))
        return prev.value

    @contextlib.contextmanager
    def tuned(self, **switches):
        """Pins kernel choices for the calls queued inside the block, e.g. graph.tuned(gemm_cfg=0, gemm_splitk=0);
        the previous values come back on exit."""
        old = []
        try:
            for name, value in switches.items():
                old.append((name, self.set_tuning(name, value)))
            yield self
        finally:
            for name, value in reversed(old):
                self.set_tuning(name, value)

    def host_alloc(self, nbytes):
        p = ctypes.c_void_p()
        self.check(self.lib.we_host_alloc(self.ctx, nbytes, ctypes.byref(p)))
        return p.value

    @staticmethod
    def host_view(ptr, nbytes):
        """A numpy uint8 view of pinned host memory from host_alloc (valid until host_free)."""
        return np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(ptr))

    def host_free(self, ptr):
        self.check(self.lib.we_host_free(self.ctx, ctypes.c_void_p(ptr)))

    def stream_copy(self, dst, pinned_src, nbytes, after=0):
        t = ctypes.c_uint64()
        self.check(self.lib.we_stream_copy(self.ctx, _addr(dst), ctypes.c_void_p(pinned_src), nbytes, after,
                                           ctypes.byref(t)))
        return t.value

    def wait_ticket(self, ticket):
        self.check(self.lib.we_wait_ticket(self.ctx, ticket))

    def record_compute(self):
        t = ctypes.c_uint64()
        self.check(self.lib.we_record_compute(self.ctx, ctypes.byref(t)))
        return t.value

    def ticket_done(self, ticket):
        d = ctypes.c_int()
        self.check(self.lib.we_ticket_done(self.ctx, ticket, ctypes.byref(d)))
        return bool(d.value)

    # ---- HIP graphs of the compute stream
    def graph_begin(self):
        self.check(self.lib.we_graph_begin(self.ctx))

    def graph_end(self):
        g = ctypes.c_void_p()
        self.check(self.lib.we_graph_end(self.ctx, ctypes.byref(g)))
        return g.value

    def graph_launch(self, graph):
        self.check(self.lib.we_graph_launch(self.ctx, ctypes.c_void_p(graph)))

    def graph_destroy(self, graph):
        self.check(self.lib.we_graph_destroy(self.ctx, ctypes.c_void_p(graph)))

    # ---- timing
    def timer_start(self):
        self.check(self.lib.we_timer_start(self.ctx))

    def timer_stop(self):
        ms = ctypes.c_float()
        self.check(self.lib.we_timer_stop(self.ctx, ctypes.byref(ms)))
        return ms.value

    def timer_mark(self, slot):
        """Timestamp into `slot` after the work queued so far (no wait)."""
        self.check(self.lib.we_timer_mark(self.ctx, slot))

    def timer_between(self, a, b):
        """Milliseconds from timestamp slot a to slot b (waits for b)."""
        ms = ctypes.c_float()
        self.check(self.lib.we_timer_between(self.ctx, a, b, ctypes.byref(ms)))
        return ms.value

    # ---- raw ops (one dispatch each)
    def matmul(self, params, x_dtype, x, w_dtype, w, y_dtype, y, scales=None, group=0, bias=None, flags=0, gate=None,
               residual=None, mul=0, aux=None):
        """we_matmul; with `gate` (f32 [N]) we_matmul_gated: y = residual + gate * v (gatedAdd fused); with `mul`
        we_matmul_mul: y = silu(aux) * v (MUL_SWIGLU) or aux * sigmoid(v) (MUL_SIGMOID_GATE)."""
        if mul:
            self.check(self.lib.we_matmul_mul(self.ctx, ctypes.byref(params), x_dtype, _addr(x), w_dtype, _addr(w),
                                              _addr(scales), group, y_dtype, _addr(y), _addr(bias), flags, mul,
                                              _addr(aux)))
        elif gate is None:
            self.check(self.lib.we_matmul(self.ctx, ctypes.byref(params), x_dtype, _addr(x), w_dtype, _addr(w),
                                          _addr(scales), group, y_dtype, _addr(y), _addr(bias), flags))
        else:
            self.check(self.lib.we_matmul_gated(self.ctx, ctypes.byref(params), x_dtype, _addr(x), w_dtype, _addr(w),
                                                _addr(scales), group, y_dtype, _addr(y), _addr(bias), flags,
                                                _addr(gate), _addr(residual)))

    def matmul_group(self, items, x_dtype, w_dtype, y_dtype, flags=0):
        """we_matmul_group: one or two GEMMs of one N, K, dtypes and flags; items are dicts with params, x, w, y and
        optionally bias, gate, residual (the arguments of matmul). Two qualifying GEMMs run as one launch."""
        arr = (MatmulItem * len(items))()
        keep = []
        for i, it in enumerate(items):
            p = it["params"]
            keep.append(p)
            arr[i].p = ctypes.pointer(p)
            for f in ("x", "w", "y", "bias", "gate", "residual"):
                a = _addr(it.get(f))
                setattr(arr[i], f, a.value if a is not None else None)
        self.check(self.lib.we_matmul_group(self.ctx, len(items), arr, x_dtype, w_dtype, y_dtype, flags))

    def matmul_qk_norm_rope(self, params, x_dtype, x, w_dtype, w, y_dtype, y, q_heads, k_heads, eps, offset, norm_q,
                            norm_k, rope_from=0, cos=None, sin=None, bias=None, flags=0):
        """we_matmul_qk_norm_rope: a QKV projection whose q / k heads (128 wide) are RMS-normalized and rotated in
        the GEMM's epilogue (or by a pass after it where no head-aligned tile fits)."""
        self.check(self.lib.we_matmul_qk_norm_rope(self.ctx, ctypes.byref(params), x_dtype, _addr(x), w_dtype, _addr(w),
                                                   y_dtype, _addr(y), _addr(bias), flags, q_heads, k_heads, eps,
                                                   offset, _addr(norm_q), _addr(norm_k), rope_from, _addr(cos),
                                                   _addr(sin)))

    def matmul_noalloc(self, params, x_dtype, x, w_dtype, w, y_dtype, y, scales=None, group=0, bias=None, flags=0):
        """we_matmul_noalloc: we_matmul with its split-K scratch in the GPU's fixed array (allocates nothing)."""
        self.check(self.lib.we_matmul_noalloc(self.ctx, ctypes.byref(params), x_dtype, _addr(x), w_dtype, _addr(w),
                                              _addr(scales), group, y_dtype, _addr(y), _addr(bias), flags))

    def peak(self, kind, workgroups, iters, out):
        """One dispatch of a peak kernel (timePeak, src/bench/peak.ts): returns its operation count."""
        ops = ctypes.c_double()
        self.check(self.lib.we_peak(self.ctx, kind, workgroups, iters, _addr(out), ctypes.byref(ops)))
        return ops.value

    def read_peak(self, buf, nbytes, out):
        self.check(self.lib.we_read_peak(self.ctx, _addr(buf), nbytes, _addr(out)))

    def rmsnorm(self, rows, d, eps, offset, dtype, x, weight, scale, shift, out):
        self.check(self.lib.we_rmsnorm(self.ctx, rows, d, eps, offset, dtype, _addr(x), _addr(weight), _addr(scale),
                                       _addr(shift), _addr(out)))

    def rmsnorm_mod(self, rows, d, eps, offset, dtype, x, weight, tvec, table, mod_n, mod, out):
        """we_rmsnorm_mod: mod = tvec + table (mod_n f32) and out = rmsnorm(x) modulated by mod[0:d], mod[d:2d]."""
        self.check(self.lib.we_rmsnorm_mod(self.ctx, rows, d, eps, offset, dtype, _addr(x), _addr(weight), _addr(tvec),
                                           _addr(table), mod_n, _addr(mod), _addr(out)))

    def rope(self, tokens, heads, pairs, half, dtype, x, cos, sin, out):
        self.check(self.lib.we_rope(self.ctx, tokens, heads, pairs, 1 if half else 0, dtype, _addr(x), _addr(cos),
                                    _addr(sin), _addr(out)))

    def qk_norm_rope(self, tokens, heads, head_dim, eps, offset, weight, rope_from, half, cos, sin, dtype, x, out,
                     x_stride=0, out_stride=0):
        self.check(self.lib.we_qk_norm_rope(self.ctx, tokens, heads, head_dim, eps, offset, _addr(weight), rope_from,
                                            1 if half else 0, _addr(cos), _addr(sin), dtype, _addr(x), x_stride,
                                            _addr(out), out_stride))

    def attention(self, tokens, heads, kv_heads, dim, causal, dtype, q, k, v, out, q_stride=0, k_stride=0,
                  v_stride=0, out_stride=0):
        self.check(self.lib.we_attention(self.ctx, tokens, heads, kv_heads, dim, 1 if causal else 0, dtype, _addr(q),
                                         q_stride, _addr(k), k_stride, _addr(v), v_stride, _addr(out), out_stride))

    def elementwise(self, op, n, d, dtype, a, b, c, out):
        self.check(self.lib.we_elementwise(self.ctx, op, n, d, dtype, _addr(a), _addr(b), _addr(c), _addr(out)))

    def layer_sum(self, tokens, layers, dim, x, w, out):
        self.check(self.lib.we_layer_sum(self.ctx, tokens, layers, dim, _addr(x), _addr(w), _addr(out)))

    def unpack_fp8_raw(self, packed, n, scale, out):
        self.check(self.lib.we_unpack_fp8(self.ctx, _addr(packed), n, _addr(scale), _addr(out)))

    def dequant_int4_raw(self, words, scales, rows, k, group, out):
        self.check(self.lib.we_dequant_int4(self.ctx, _addr(words), _addr(scales), rows, k, group, _addr(out)))


# ------------------------------------------------------------------------------------------ operator API

def matmul_params(m, n, k, scale, x_stride=None, w_stride=None, y_stride=None, x_offset=None, w_offset=None,
                  y_offset=None, k_split=1, graph=None):
    """src/kernels/matmul.ts:198-212, with its validation messages."""
    lib = load_library()
    p = MatmulParams()
    d = lambda v: -1 if v is None else v
    ctx = graph.ctx if graph is not None else None
    rc = lib.we_matmul_params_make(ctx, m, n, k, scale, d(x_stride), d(w_stride), d(y_stride), d(x_offset),
                                   d(w_offset), d(y_offset), k_split, ctypes.byref(p))
    if rc:
        raise WeError(rc, lib.we_last_error(ctx).decode())  # ctx None: this thread's context-free message
    return p


def conv3x3_params(height, width, cin, cout, graph=None):
    """conv3x3Params (src/kernels/matmul.ts:268-272): Params under which matmul is a 3x3 convolution (padding 1)
    of a channel-last image [height, width, cin] with W [cout, (ky, kx, cin)]."""
    lib = load_library()
    p = MatmulParams()
    ctx = graph.ctx if graph is not None else None
    rc = lib.we_conv3x3_params(ctx, height, width, cin, cout, ctypes.byref(p))
    if rc:
        raise WeError(rc, lib.we_last_error(ctx).decode())
    return p


def conv3x3(graph, x, w, height, width, cin, cout, x_dtype=F32, w_dtype=F32, y_dtype=F32, scale=1.0):
    """The one-shot conv3x3 of src/kernels/matmul.ts:275-279 on device buffers: y [height * width, cout]."""
    p = conv3x3_params(height, width, cin, cout, graph=graph)
    p.scale = scale
    y = graph.buffer(height * width * cout * ELEM_BYTES[y_dtype])
    graph.matmul(p, x_dtype, x, w_dtype, w, y_dtype, y)
    return y


def k_split_for(m, n, k):
    """src/model/ops.ts:42-45"""
    return load_library().we_ksplit_for(m, n, k)


class Linear:
    """src/model/ops.ts:24-32, plus the additive int4 dtype (scales f16 [n, k / group])."""

    def __init__(self, buffer, dtype, scale, n, k, bias=None, lora=None, scales=None, group=64):
        self.buffer, self.dtype, self.scale, self.n, self.k = buffer, dtype, scale, n, k
        self.bias, self.lora, self.scales, self.group = bias, lora, scales, group


def _wdt(dtype):
    return DTYPES[dtype] if isinstance(dtype, str) else dtype


def linear(graph, x, w, m, x_dtype=F32, y_dtype=F32, gelu_tanh=False, swiglu_gate=None, sigmoid_gate_of=None,
           out=None):
    """y[m, n] = x[m, k] . W^T (+ bias) (+ lora up.scale * (x . down^T) . up^T, added in place): src/model/ops.ts:61-73.
    The bias (and optional tanh GELU) run in the GEMM epilogue instead of separate passes. GELU applies to the whole
    sum, as a caller of the reference applies it to what linear returns: with LoRA it runs after the update is added
    (one in-place pass), not in the base GEMM's epilogue.
    The step that consumes the result may be fused too: swiglu_gate=g returns swiglu(g, linear) (src/model/ops.ts:102)
    and sigmoid_gate_of=a returns sigmoidGate(a, linear) (ops.ts:104), both in the epilogue when there is no LoRA.
    `out` (optional) receives the result instead of a new buffer; it may be the gate / a operand itself."""
    if swiglu_gate is not None or sigmoid_gate_of is not None:
        if gelu_tanh or (swiglu_gate is not None and sigmoid_gate_of is not None):
            raise WeError(1, "one fused consumer at a time, and not with GELU")
        aux = swiglu_gate if swiglu_gate is not None else sigmoid_gate_of
        mul = MUL_SWIGLU if swiglu_gate is not None else MUL_SIGMOID_GATE
        y = out if out is not None else graph.buffer(m * w.n * ELEM_BYTES[y_dtype])
        if w.lora is None and _wdt(w.dtype) != INT4:
            graph.matmul(matmul_params(m, w.n, w.k, w.scale, graph=graph), x_dtype, x, _wdt(w.dtype), w.buffer,
                         y_dtype, y, bias=w.bias, flags=EPI_BIAS if w.bias is not None else 0, mul=mul, aux=aux)
            return y
        v = linear(graph, x, w, m, x_dtype, y_dtype)
        op = OP_SWIGLU if mul == MUL_SWIGLU else OP_SIGMOID_GATE
        graph.elementwise(op, m * w.n, 1, y_dtype, aux, v, None, y)  # swiglu(gate=aux, up=v), sigmoidGate(a=aux, gate=v)
        graph.free(v)
        return y
    y = out if out is not None else graph.buffer(m * w.n * ELEM_BYTES[y_dtype])
    fuse_gelu = gelu_tanh and w.lora is None
    flags = (EPI_BIAS if w.bias is not None else 0) | (EPI_GELU if fuse_gelu else 0)
    graph.matmul(matmul_params(m, w.n, w.k, w.scale, graph=graph), x_dtype, x, _wdt(w.dtype), w.buffer, y_dtype, y,
                 scales=w.scales, group=w.group if _wdt(w.dtype) == INT4 else 0, bias=w.bias, flags=flags)
    if w.lora is None:
        return y
    down, up = w.lora
    if down.k != w.k or up.n != w.n or up.k != down.n or down.n % 4:
        raise WeError(1, "LoRA shapes do not fit the linear layer")
    t = _narrow_linear(graph, x, down, m, x_dtype)
    graph.matmul(matmul_params(m, up.n, up.k, up.scale, graph=graph), F32, t, _wdt(up.dtype), up.buffer, y_dtype, y,
                 flags=EPI_ACCUMULATE)
    if gelu_tanh:
        graph.elementwise(OP_GELU_TANH, m * w.n, 1, y_dtype, y, None, None, y)
    return y


def _narrow_linear(graph, x, w, m, x_dtype):
    """src/model/ops.ts:48-58: split-K partials, then layerSum over them."""
    split = k_split_for(m, w.n, w.k)
    if split == 1:
        return linear(graph, x, w, m, x_dtype, F32)
    partials = graph.buffer(split * m * w.n * 4)
    graph.matmul(matmul_params(m, w.n, w.k, w.scale, k_split=split, graph=graph), x_dtype, x, _wdt(w.dtype), w.buffer,
                 F32, partials, flags=EPI_SPLIT_K)
    y = graph.buffer(m * w.n * 4)
    ones = graph.buffer(np.ones(split, np.float32))
    graph.layer_sum(1, split, m * w.n, partials, ones, y)
    return y


class Mod:
    def __init__(self, scale, shift):
        self.scale, self.shift = scale, shift


def no_mod(graph, d):
    """src/model/ops.ts:85"""
    return Mod(graph.buffer(d * 4), graph.buffer(d * 4))


def norm(graph, x, weight, rows, d, mod, eps=1e-5, offset=1.0, dtype=F32):
    """src/model/ops.ts:78-82"""
    out = graph.buffer(rows * d * ELEM_BYTES[dtype])
    graph.rmsnorm(rows, d, eps, offset, dtype, x, weight, mod.scale if mod else None, mod.shift if mod else None, out)
    return out


class Rope:
    def __init__(self, cos, sin, pairs, tokens):
        self.cos, self.sin, self.pairs, self.tokens = cos, sin, pairs, tokens


def rotate(graph, x, heads, rope, pairing="interleaved", dtype=F32):
    """src/model/ops.ts:89-93"""
    out = graph.buffer(rope.tokens * heads * rope.pairs * 2 * ELEM_BYTES[dtype])
    graph.rope(rope.tokens, heads, rope.pairs, pairing == "half", dtype, x, rope.cos, rope.sin, out)
    return out


class AttentionShape:
    """src/kernels/attention.ts:7: tokens, heads, kvHeads, dim, chunk (accepted; nothing to bound here), causal."""

    def __init__(self, tokens, heads, kv_heads, dim, chunk=None, causal=False):
        self.tokens, self.heads, self.kv_heads, self.dim = tokens, heads, kv_heads, dim
        self.chunk, self.causal = chunk, causal


def attention(graph, q, k, v, shape, dtype=F32):
    """src/kernels/attention.ts:20-51: q [tokens, heads, dim], k/v [tokens, kvHeads, dim] -> new out
    [tokens, heads, dim]; raises "heads must be a multiple of kvHeads" like the reference."""
    s = shape
    if s.kv_heads == 0 or s.heads % s.kv_heads:
        raise WeError(1, "heads must be a multiple of kvHeads")
    out = graph.buffer(s.tokens * s.heads * s.dim * ELEM_BYTES[dtype])
    graph.attention(s.tokens, s.heads, s.kv_heads, s.dim, s.causal, dtype, q, k, v, out)
    return out


def _elementwise(graph, op, a, b, c, n, d=1, dtype=F32):
    out = graph.buffer(n * ELEM_BYTES[dtype])
    graph.elementwise(op, n, d, dtype, a, b, c, out)
    return out


def swiglu(graph, gate, up, n, dtype=F32):
    return _elementwise(graph, OP_SWIGLU, gate, up, None, n, 1, dtype)


def sigmoid_gate(graph, a, gate, n, dtype=F32):
    return _elementwise(graph, OP_SIGMOID_GATE, a, gate, None, n, 1, dtype)


def gated_add(graph, x, h, g, n, d, dtype=F32):
    return _elementwise(graph, OP_GATED_ADD, x, h, g, n, d, dtype)


def add_bias(graph, x, b, n, d, dtype=F32):
    return _elementwise(graph, OP_ADD_BIAS, x, b, None, n, d, dtype)


def add(graph, x, h, n, dtype=F32):
    return _elementwise(graph, OP_ADD, x, h, None, n, 1, dtype)


def gelu(graph, x, n, dtype=F32):
    return _elementwise(graph, OP_GELU_TANH, x, None, None, n, 1, dtype)


def silu(graph, x, n, dtype=F32):
    return _elementwise(graph, OP_SILU, x, None, None, n, 1, dtype)


# ------------------------------------------------------------------------------------------ one-shots (tests)

def _oneshot(graph, x, w_bytes, w_dtype, scale, m, n, k, x_dtype=F32, y_dtype=F32, **layout):
    p = matmul_params(m, n, k, scale, graph=graph, **layout)
    xb = graph.buffer(x)
    wb = graph.buffer(w_bytes)
    rows = m * (p.k_split if layout.get("k_split", 1) > 1 else 1)
    y = graph.buffer(max(1, rows * p.y_stride + p.y_offset) * ELEM_BYTES[y_dtype])
    graph.matmul(p, x_dtype, xb, w_dtype, wb, y_dtype, y)
    return y


def matmul_fp8(graph, x, w, scale, m, n, k):
    """src/kernels/matmul.ts:223-233"""
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.uint8)
    if x.size != m * k or w.size != n * k:
        raise WeError(1, "x or w does not match the shape")
    return graph.read(_oneshot(graph, x, w, FP8, scale, m, n, k), dtype=np.float32, count=m * n)


def matmul_bf16(graph, x, w, scale, m, n, k):
    """src/kernels/matmul.ts:236-246 (w: raw little-endian bf16 bytes or uint16 values)"""
    x = np.asarray(x, np.float32)
    w = np.asarray(w)
    if x.size != m * k or w.nbytes != n * k * 2:
        raise WeError(1, "x or w does not match the shape")
    return graph.read(_oneshot(graph, x, w, BF16, scale, m, n, k), dtype=np.float32, count=m * n)


def matmul_f32(graph, x, w, scale, m, n, k, output_length=None, **layout):
    """src/kernels/matmul.ts:249-265"""
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    y = _oneshot(graph, x, w, F32, scale, m, n, k, **layout)
    return graph.read(y, dtype=np.float32, count=output_length or m * n)


def unpack_fp8(graph, data, scale):
    """src/kernels/fp8.ts:24-36 one-shot: out[i] = e4m3(byte i) * scale."""
    data = np.asarray(data, np.uint8)
    packed = graph.buffer(np.pad(data, (0, (-data.size) % 4)) if data.size else np.zeros(4, np.uint8))
    sc = graph.buffer(np.array([scale], np.float32))
    out = graph.buffer(max(4, data.size * 4))
    graph.unpack_fp8_raw(packed, data.size, sc, out)
    return graph.read(out, dtype=np.float32, count=data.size)

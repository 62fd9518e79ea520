"""Model files over the native .safetensors reader of libwe.so (we_st_*):

  Safetensors, read_header, read_tensor   src/weights/safetensors.ts:28-70 (header checked in libwe.so with the
                                          reference's messages; bytes read on request, in parallel, straight into
                                          any host memory, e.g. pinned buffers for the weight streamer)
  fp8_weights, block_groups               src/weights/inspect.ts (fp8 weight + scale pairing, repeated blocks)
  to_float32                              src/weights/fp8.ts:4-54 (the CPU decoders)
  load_linear_fp8                         src/model/weights.ts:26-50 (an fp8 [n, k] weight and its weight_scale)

Reading needs the library but no GPU.
"""
import collections
import ctypes
import json
import re

import numpy as np

import we

# DTYPE_BYTES (src/weights/safetensors.ts:8-11)
DTYPE_BYTES = {"F64": 8, "F32": 4, "F16": 2, "BF16": 2, "F8_E4M3": 1, "F8_E5M2": 1, "I64": 8, "I32": 4, "I16": 2,
               "I8": 1, "U64": 8, "U32": 4, "U16": 2, "U8": 1, "BOOL": 1}
WE_EFORMAT, WE_EIO, WE_ENOTFOUND = 5, 6, 7

TensorInfo = collections.namedtuple("TensorInfo", "name dtype shape offset size")
Fp8Weight = collections.namedtuple("Fp8Weight", "weight scale")
BlockGroup = collections.namedtuple("BlockGroup", "prefix count")


class SafetensorsError(we.WeError):
    """A file that is not a valid .safetensors file (src/weights/safetensors.ts:18-20)."""


class _Info(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_char_p), ("ndim", ctypes.c_uint32),
                ("shape", ctypes.POINTER(ctypes.c_uint64)), ("offset", ctypes.c_uint64), ("size", ctypes.c_uint64)]


def _raise(lib, rc):
    msg = (lib.we_last_error(None) or b"").decode(errors="replace")
    raise (SafetensorsError if rc == WE_EFORMAT else we.WeError)(rc, msg)


class Safetensors:
    """An open .safetensors file: `tensors` (name -> TensorInfo, in the reference's Map order; offsets are
    absolute file offsets) and `metadata` (the string entries of __metadata__). Only the header has been
    read; `read` / `read_into` fetch tensor bytes."""

    def __init__(self, path):
        self._lib = lib = we.load_library()
        h = ctypes.c_void_p()
        rc = lib.we_st_open(str(path).encode(), ctypes.byref(h))
        if rc:
            _raise(lib, rc)
        self._h = h
        self.path = str(path)
        n = ctypes.c_uint32()
        self._check(lib.we_st_count(h, ctypes.byref(n)))
        self.tensors = {}
        self._index = {}
        info = _Info()
        for i in range(n.value):
            self._check(lib.we_st_info(h, i, ctypes.byref(info)))
            name = info.name.decode()
            shape = tuple(int(info.shape[d]) for d in range(info.ndim))
            self.tensors[name] = TensorInfo(name, info.dtype.decode(), shape, int(info.offset), int(info.size))
            self._index[name] = i
        self._check(lib.we_st_metadata_count(h, ctypes.byref(n)))
        self.metadata = {}
        k, v = ctypes.c_char_p(), ctypes.c_char_p()
        for i in range(n.value):
            self._check(lib.we_st_metadata_at(h, i, ctypes.byref(k), ctypes.byref(v)))
            self.metadata[k.value.decode()] = v.value.decode()

    def _check(self, rc):
        if rc:
            _raise(self._lib, rc)

    def info(self, name):
        t = self.tensors.get(name)
        if t is None:
            raise we.WeError(WE_ENOTFOUND, f"Missing tensor {name}")
        return t

    def read_into(self, name, dst, begin=0, nbytes=None, threads=0):
        """Reads bytes [begin, begin + nbytes) of a tensor (default: all of it from `begin`) to the host
        address `dst` (an int, e.g. a pinned buffer from Graph.host_alloc plus an offset)."""
        t = self.info(name)
        nbytes = t.size - begin if nbytes is None else nbytes
        self._check(self._lib.we_st_read(self._h, self._index[name], begin, nbytes, ctypes.c_void_p(int(dst)), threads))
        return nbytes

    def read(self, name, limit=None, threads=0):
        """The raw bytes of one tensor, or only its first `limit` bytes (readTensor)."""
        t = self.info(name)
        n = t.size if limit is None else min(limit, t.size)
        out = np.empty(n, np.uint8)
        if n:
            self.read_into(name, out.ctypes.data, 0, n, threads)
        return out

    def close(self):
        if getattr(self, "_h", None):
            self._lib.we_st_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()


def read_header(path):
    return Safetensors(path)


def read_tensor(st, tensor, limit=None):
    return st.read(tensor.name if isinstance(tensor, TensorInfo) else tensor, limit)


# ---- src/weights/inspect.ts -------------------------------------------------------------------------------

SCALE_SUFFIXES = (".scale_weight", ".weight_scale")


def fp8_weights(st):
    """fp8 weights with their per-layer scale (ComfyUI fp8_scaled: real weight = fp8 x scale), sorted by
    weight name (code-point order; the reference's localeCompare agrees on names of letters, digits, '.' and
    '_' of one case)."""
    pairs = []
    for t in st.tensors.values():
        if not t.dtype.startswith("F8_") or not t.name.endswith(".weight"):
            continue
        base = t.name[:-len(".weight")]
        scale = next((st.tensors[base + s] for s in SCALE_SUFFIXES if base + s in st.tensors), None)
        pairs.append(Fp8Weight(t, scale))
    return sorted(pairs, key=lambda p: p.weight.name)


def block_groups(names):
    """Repeated blocks ("x.blocks.0...", "x.blocks.1...") and how many of each, biggest first."""
    groups = {}
    for name in names:
        m = re.match(r"^(.*?)\.(\d+)\.", name)
        if not m:
            continue
        groups.setdefault(m.group(1), set()).add(m.group(2))
    return sorted((BlockGroup(p, len(ids)) for p, ids in groups.items()), key=lambda g: -g.count)


# ---- src/weights/fp8.ts ---------------------------------------------------------------------------------

def _table(decode):
    return np.array([decode(b) for b in range(256)], np.float32)


def _e4m3(b):  # bias 7, no infinity, 0x7f / 0xff are NaN
    sign = -1.0 if b & 0x80 else 1.0
    e, m = (b >> 3) & 0xF, b & 7
    if e == 0xF and m == 7:
        return np.nan
    return sign * (m / 8) * 2.0 ** -6 if e == 0 else sign * (1 + m / 8) * 2.0 ** (e - 7)


def _e5m2(b):  # bias 15, IEEE-style infinity and NaN
    sign = -1.0 if b & 0x80 else 1.0
    e, m = (b >> 2) & 0x1F, b & 3
    if e == 0x1F:
        return np.nan if m else sign * np.inf
    return sign * (m / 4) * 2.0 ** -14 if e == 0 else sign * (1 + m / 4) * 2.0 ** (e - 15)


_E4M3 = _table(_e4m3)
_E5M2 = _table(_e5m2)


def to_float32(dtype, raw):
    """Little-endian tensor bytes -> f32 (toFloat32)."""
    if dtype not in ("F32", "BF16", "F16", "F8_E4M3", "F8_E5M2"):
        raise ValueError(f"Can't decode {dtype} as floats")
    raw = np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray, memoryview)) else np.asarray(raw, np.uint8)
    raw = np.ascontiguousarray(raw)
    if dtype == "F32":
        return raw.view(np.float32).copy()
    if dtype == "BF16":
        return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    if dtype == "F16":
        return raw.view(np.float16).astype(np.float32)
    if dtype == "F8_E4M3":
        return _E4M3[raw]
    return _E5M2[raw]


# ---- src/model/weights.ts -------------------------------------------------------------------------------

def load_scale(st, base):
    """The f32 per-tensor scale of the fp8 weight `base`.weight (weight_scale, or scale_weight)."""
    for s in (".weight_scale", ".scale_weight"):
        t = st.tensors.get(base + s)
        if t is not None:
            return float(to_float32(t.dtype, st.read(t.name))[0])
    raise we.WeError(WE_ENOTFOUND, f"Missing tensor {base}.weight_scale")


def load_linear_fp8(st, name, n, k, dst, threads=0):
    """Reads `name`.weight (F8_E4M3 [n, k]) to the host address `dst` and returns its scale (loadLinear's
    checks, for the fp8 layout the streamer moves)."""
    w = st.info(f"{name}.weight")
    if w.dtype != "F8_E4M3" or w.shape != (n, k):
        raise we.WeError(we.WE_EINVAL,
                         f"{name}.weight: expected a 2D F8_E4M3 tensor of shape [{n}, {k}], got {w.dtype} {list(w.shape)}")
    st.read_into(w.name, dst, threads=threads)
    return load_scale(st, name)


def load_floats_into(st, name, count, dst):
    """A small float tensor of `count` values (norm weights, modulation tables) as f32 at the host address
    `dst` (loadFloats)."""
    t = st.info(name)
    v = to_float32(t.dtype, st.read(name))
    if v.size != count:
        raise we.WeError(we.WE_EINVAL, f"{name}: expected {count} values, got {v.size}")
    ctypes.memmove(int(dst), v.ctypes.data, 4 * count)


def save(path, tensors, metadata=None):
    """Writes a .safetensors file: tensors = {name: (dtype, shape, bytes-like)} in file order (for exporting
    a weight image; the reference itself only reads these files)."""
    header = {"__metadata__": dict(metadata)} if metadata else {}
    off, blobs = 0, []
    for name, (dtype, shape, data) in tensors.items():
        b = np.ascontiguousarray(np.frombuffer(memoryview(data).cast("B"), np.uint8))
        need = int(np.prod(shape, dtype=np.int64)) * DTYPE_BYTES[dtype]
        if b.size != need:
            raise ValueError(f"{name}: has {b.size} bytes, its shape needs {need} bytes")
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + b.size]}
        off += b.size
        blobs.append(b)
    text = json.dumps(header, separators=(",", ":")).encode()
    text += b" " * (-(8 + len(text)) % 8)  # data starts 8-byte aligned
    with open(path, "wb") as f:
        f.write(len(text).to_bytes(8, "little"))
        f.write(text)
        for b in blobs:
            f.write(b.tobytes())

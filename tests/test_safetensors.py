"""The native .safetensors reader (we_st_* in libwe.so) and its Python mirror (web-engine_amd/weights.py), on
the CPU: no GPU work is involved.

Mirrors tests/safetensors.test.ts (every case, with its files built byte for byte as tests/helpers.ts builds
them: compact JSON header, no padding), tests/inspect.test.ts (fp8Weights, blockGroups) and the toFloat32 cases
of tests/fp8.test.ts; adds hostile headers beyond the reference's list, parallel reads of a large tensor, and a
double-stream block image written to a file and read back into a host image, byte for byte.
"""
import json
import struct

import numpy as np
import pytest

import block as B
import oracle_lib as O
import we
import weights as W


def make_safetensors(path, tensors, metadata=None):
    """tests/helpers.ts:2-16: 8-byte LE size, JSON.stringify(header) (no padding), the data in order."""
    header = {"__metadata__": metadata} if metadata else {}
    off = 0
    for name, (dtype, shape, data) in tensors.items():
        header[name] = {"dtype": dtype, "shape": shape, "data_offsets": [off, off + len(data)]}
        off += len(data)
    text = json.dumps(header, separators=(",", ":")).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text + b"".join(bytes(d) for _, _, d in tensors.values()))
    return path


def raw_safetensors(path, header_text, data=b"", size_override=None):
    """tests/helpers.ts:19-24: a raw file, 8-byte size + the given header text + data."""
    text = header_text.encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text) if size_override is None else size_override) + text + bytes(data))
    return path


@pytest.fixture
def path(tmp_path):
    return tmp_path / "t.safetensors"


# ---- tests/safetensors.test.ts ------------------------------------------------------------------------------

def test_lists_tensors_with_absolute_file_offsets(path):  # :8-18
    make_safetensors(path, {"a": ("F8_E4M3", [2, 2], [1, 2, 3, 4]), "b": ("F32", [1], [0, 0, 128, 63])},
                     {"format": "pt"})
    st = W.read_header(path)
    start = path.stat().st_size - 8  # data starts after size + header
    assert st.metadata == {"format": "pt"}
    assert st.tensors["a"] == W.TensorInfo("a", "F8_E4M3", (2, 2), start, 4)
    assert (st.tensors["b"].offset, st.tensors["b"].size) == (start + 4, 4)


def test_reads_one_tensors_bytes(path):  # :20-24
    make_safetensors(path, {"a": ("U8", [2], [7, 8]), "b": ("U8", [3], [9, 10, 11])})
    st = W.read_header(path)
    assert W.read_tensor(st, st.tensors["b"]).tolist() == [9, 10, 11]


def test_accepts_a_file_without_tensors(path):  # :26-28
    assert len(W.read_header(make_safetensors(path, {})).tensors) == 0


@pytest.mark.parametrize("case,message", [
    ("too_small", "too small"), ("header_bigger_than_file", "header size"), ("header_over_100MB", "header size"),
    ("not_json", "not valid JSON"), ("not_object", "not an object"), ("unknown_dtype", "unknown dtype"),
    ("bad_shape", "bad shape"), ("size_mismatch", "8 bytes"), ("past_the_end", "past the end"),
    ("overlap", "overlap")])
def test_rejects_broken_or_hostile_files(path, case, message):  # :30-52
    if case == "too_small":
        path.write_bytes(bytes([1, 2]))
    elif case == "header_bigger_than_file":
        raw_safetensors(path, "{}", size_override=1000)
    elif case == "header_over_100MB":
        raw_safetensors(path, "{}", size_override=200_000_000)
    elif case == "not_json":
        raw_safetensors(path, "nope")
    elif case == "not_object":
        raw_safetensors(path, "[1]")
    elif case == "unknown_dtype":
        raw_safetensors(path, '{"a":{"dtype":"X9","shape":[1],"data_offsets":[0,1]}}', bytes(1))
    elif case == "bad_shape":
        raw_safetensors(path, '{"a":{"dtype":"U8","shape":[-1],"data_offsets":[0,1]}}', bytes(1))
    elif case == "size_mismatch":
        raw_safetensors(path, '{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}}', bytes(4))
    elif case == "past_the_end":
        raw_safetensors(path, '{"a":{"dtype":"U8","shape":[4],"data_offsets":[0,4]}}', bytes(1))
    else:
        raw_safetensors(path, '{"a":{"dtype":"U8","shape":[2],"data_offsets":[0,2]},'
                              '"b":{"dtype":"U8","shape":[2],"data_offsets":[1,3]}}', bytes(3))
    with pytest.raises(W.SafetensorsError, match=message) as e:
        W.read_header(path)
    assert e.value.code == W.WE_EFORMAT


def test_errors_are_safetensors_errors(path):  # :51
    path.write_bytes(b"")
    with pytest.raises(W.SafetensorsError):
        W.read_header(path)


def test_read_tensor_with_a_limit(path):  # :55-61
    make_safetensors(path, {"a": ("U8", [4], [1, 2, 3, 4])})
    st = W.read_header(path)
    assert W.read_tensor(st, st.tensors["a"], 2).tolist() == [1, 2]


# ---- exact messages and the rest of the reference's rules ---------------------------------------------------

@pytest.mark.parametrize("header,data,message", [
    ('{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}}', 4, "a: has 4 bytes, its shape needs 8 bytes"),
    ('{"a":{"dtype":"U8","shape":[2],"data_offsets":[3,1]}}', 4, "a: has -2 bytes, its shape needs 2 bytes"),
    ('{"a":{"dtype":"X9","shape":[1],"data_offsets":[0,1]}}', 1, "a: unknown dtype X9"),
    ('{"a":{"shape":[1],"data_offsets":[0,1]}}', 1, "a: unknown dtype undefined"),
    ('{"a":{"dtype":7,"shape":[1],"data_offsets":[0,1]}}', 1, "a: unknown dtype 7"),
    ('{"a":{"dtype":["F","32"],"shape":[1],"data_offsets":[0,1]}}', 1, "a: unknown dtype F,32"),
    ('{"a":null}', 1, "a: unknown dtype undefined"),
    ('{"a":{"dtype":"U8","shape":[1.5],"data_offsets":[0,1]}}', 1, "a: bad shape"),
    ('{"a":{"dtype":"U8","shape":"1","data_offsets":[0,1]}}', 1, "a: bad shape"),
    ('{"a":{"dtype":"U8","shape":[1],"data_offsets":[0]}}', 1, "a: bad data_offsets"),
    ('{"a":{"dtype":"U8","shape":[1],"data_offsets":[-1,0]}}', 1, "a: bad data_offsets"),
    ('{"a":{"dtype":"U8","shape":[1],"data_offsets":[0,9007199254740992]}}', 1, "a: bad data_offsets"),
    ('{"a":{"dtype":"U8","shape":[3],"data_offsets":[0,3]}}', 2, "a: data goes past the end of the file"),
    ('{"x":{"dtype":"U8","shape":[2],"data_offsets":[0,2]},"y":{"dtype":"U8","shape":[2],"data_offsets":[1,3]}}', 3,
     "x and y overlap"),
    # integer-like keys come first in JavaScript's object order: "5" is checked before "a"
    ('{"a":{"dtype":"X1","shape":[1],"data_offsets":[0,1]},"5":{"dtype":"X2","shape":[1],"data_offsets":[0,1]}}', 1,
     "5: unknown dtype X2"),
    ('{"a":1,}', 0, "Header is not valid JSON"),
    ("", 0, "Header is not valid JSON"),
    ('"str"', 0, "Header is not an object"),
    # nesting is bounded at 256 levels (JSON.parse would accept this header and the reference then report
    # "Header is not an object": both reject the file)
    ("[" * 5000 + "]" * 5000, 0, "Header is not valid JSON"),
])
def test_exact_messages(path, header, data, message):
    raw_safetensors(path, header, bytes(data))
    with pytest.raises(W.SafetensorsError) as e:
        W.read_header(path)
    assert str(e.value) == message


def test_header_size_message_and_limit(path):
    raw_safetensors(path, "{}", size_override=100_000_001)
    with pytest.raises(W.SafetensorsError, match=r"^Bad header size: 100000001$"):
        W.read_header(path)
    path.write_bytes(bytes(7))
    with pytest.raises(W.SafetensorsError, match=r"^File is too small to be a \.safetensors file$"):
        W.read_header(path)


def test_json_details(path):
    # escapes and non-ASCII names, float-valued counts, padding, duplicate keys (the last value wins, in the
    # first one's place), zero-size tensors, a non-string metadata value (kept out of the string map)
    text = ('﻿ {"__metadata__":{"k":"v","n":3},"w\\u00e9ight\\ud83d\\ude00":{"dtype":"U8","shape":[2.0],'
            '"data_offsets":[0,2e0]},"z":{"dtype":"F32","shape":[0,5],"data_offsets":[2,2]},'
            '"d":{"dtype":"X","shape":[1],"data_offsets":[0,1]},"d":{"dtype":"U8","shape":[1],"data_offsets":[2,3]}}   ')
    raw_safetensors(path, text, bytes([5, 6, 7]))
    st = W.read_header(path)
    assert list(st.tensors) == ["wéight\U0001F600", "z", "d"]
    assert st.tensors["wéight\U0001F600"].shape == (2,) and st.read("wéight\U0001F600").tolist() == [5, 6]
    assert st.tensors["z"].size == 0 and st.read("z").size == 0
    assert st.read("d").tolist() == [7]
    assert st.metadata == {"k": "v"}


def test_zero_size_tensor_order_decides_overlap(path):
    # the reference's stable sort by offset: a zero-size tensor listed after a tensor at the same offset
    # starts inside it
    raw_safetensors(path, '{"a":{"dtype":"U8","shape":[0],"data_offsets":[0,0]},'
                          '"b":{"dtype":"U8","shape":[2],"data_offsets":[0,2]}}', bytes(2))
    assert len(W.read_header(path).tensors) == 2
    raw_safetensors(path, '{"b":{"dtype":"U8","shape":[2],"data_offsets":[0,2]},'
                          '"a":{"dtype":"U8","shape":[0],"data_offsets":[0,0]}}', bytes(2))
    with pytest.raises(W.SafetensorsError, match="^b and a overlap$"):
        W.read_header(path)


def test_reads_are_bounded_and_missing_names_fail(path):
    make_safetensors(path, {"a": ("U8", [4], [1, 2, 3, 4])})
    st = W.read_header(path)
    out = np.zeros(8, np.uint8)
    with pytest.raises(we.WeError, match=r"a: bytes \[2, 6\) are outside its 4 bytes"):
        st.read_into("a", out.ctypes.data, begin=2, nbytes=4)
    assert st.read_into("a", out.ctypes.data, begin=1, nbytes=3) == 3 and out[:3].tolist() == [2, 3, 4]
    with pytest.raises(we.WeError, match="Missing tensor nope") as e:
        st.info("nope")
    assert e.value.code == W.WE_ENOTFOUND
    with pytest.raises(we.WeError) as e:
        W.read_header(path.parent / "absent.safetensors")
    assert e.value.code == W.WE_EIO


def test_parallel_read_of_a_large_tensor(path):
    rng = np.random.default_rng(0)
    big = rng.integers(0, 256, 40 * 1024 * 1024 + 12345, dtype=np.uint8)
    W.save(path, {"pad": ("U8", [3], bytes(3)), "big": ("U8", [big.size], big)})
    st = W.read_header(path)
    for threads in (1, 3, 8, 16):
        assert np.array_equal(st.read("big", threads=threads), big)
    part = np.zeros(1000, np.uint8)
    st.read_into("big", part.ctypes.data, begin=big.size - 1000, threads=8)
    assert np.array_equal(part, big[-1000:])


def test_parallel_read_covers_every_byte_when_pieces_round_down(path):
    """64 MiB + 3 bytes over 8 threads: floor(bytes / 8) is already page-aligned, so pieces of that size would
    leave the last 3 bytes unread. Every byte arrives, for the whole tensor and for a sub-range with the same
    property."""
    rng = np.random.default_rng(1)
    big = rng.integers(1, 256, 64 * 1024 * 1024 + 3, dtype=np.uint8)  # no zero bytes: a skipped byte shows
    W.save(path, {"big": ("U8", [big.size], big)})
    st = W.read_header(path)
    for threads in (8, 7, 16):
        assert np.array_equal(st.read("big", threads=threads), big), threads
    sub = np.zeros(32 * 1024 * 1024 + 5, np.uint8)
    st.read_into("big", sub.ctypes.data, begin=17, nbytes=sub.size, threads=4)
    assert np.array_equal(sub, big[17:17 + sub.size])


# ---- tests/inspect.test.ts ----------------------------------------------------------------------------------

def _t(dtype, shape):
    n = int(np.prod(shape)) * {"F32": 4, "BF16": 2}.get(dtype, 1)
    return (dtype, shape, bytes(n))


def _krea(path):  # inspect.test.ts:8-20
    return W.read_header(make_safetensors(path, {
        "model.diffusion_model.txtfusion.projector.weight": _t("BF16", [4, 2]),
        "model.diffusion_model.blocks.0.attn.qkv.weight": _t("F8_E4M3", [6, 2]),
        "model.diffusion_model.blocks.0.attn.qkv.scale_weight": _t("F32", [1]),
        "model.diffusion_model.blocks.1.attn.qkv.weight": _t("F8_E4M3", [6, 2]),
        "model.diffusion_model.blocks.1.attn.qkv.weight_scale": _t("F32", [1]),
        "model.diffusion_model.blocks.1.norm.weight": _t("BF16", [2]),
        "model.diffusion_model.final.weight": _t("F8_E4M3", [2, 2]),
        "scaled_fp8": _t("F8_E4M3", [0]),
    }))


def test_fp8_weights_pairs_each_weight_with_its_scale(path):  # inspect.test.ts:22-32
    short = lambda t: t.name.replace("model.diffusion_model.", "") if t else None  # noqa: E731
    assert [(short(p.weight), short(p.scale)) for p in W.fp8_weights(_krea(path))] == [
        ("blocks.0.attn.qkv.weight", "blocks.0.attn.qkv.scale_weight"),
        ("blocks.1.attn.qkv.weight", "blocks.1.attn.qkv.weight_scale"),
        ("final.weight", None)]


def test_fp8_weights_skips_the_scaled_fp8_marker(path):  # inspect.test.ts:34-36
    assert not any(p.weight.name == "scaled_fp8" for p in W.fp8_weights(_krea(path)))


def test_block_groups():  # inspect.test.ts:39-50
    assert W.block_groups(["m.blocks.0.a", "m.blocks.0.b", "m.blocks.1.a", "m.blocks.2.a", "m.txt.0.x", "other"]) == [
        W.BlockGroup("m.blocks", 3), W.BlockGroup("m.txt", 1)]
    assert W.block_groups(["m.blocks.0.mlp.1.w", "m.blocks.1.mlp.0.w"]) == [W.BlockGroup("m.blocks", 2)]


# ---- tests/fp8.test.ts (toFloat32) --------------------------------------------------------------------------

def test_to_float32():
    le = lambda *w: np.array(w, np.uint16).view(np.uint8)  # noqa: E731
    assert W.to_float32("F32", np.array([1.5, -2], np.float32).view(np.uint8)).tolist() == [1.5, -2]
    assert W.to_float32("BF16", le(0x3F80, 0xC000)).tolist() == [1, -2]
    assert W.to_float32("F16", le(0x3C00, 0xC000, 0x0001, 0x7C00)).tolist() == [1, -2, 2.0 ** -24, np.inf]
    assert W.to_float32("F8_E4M3", [0x38, 0x7E]).tolist() == [1, 448]
    assert W.to_float32("F8_E5M2", [0x3C]).tolist() == [1]
    with pytest.raises(ValueError, match="I64"):
        W.to_float32("I64", bytes(8))


def test_fp8_tables_match_the_oracle_on_every_code():
    codes = np.arange(256, dtype=np.uint8)
    assert np.array_equal(W.to_float32("F8_E4M3", codes), np.array([O.lib.or_e4m3(int(b)) for b in codes], np.float32),
                          equal_nan=True)
    assert np.array_equal(W.to_float32("F8_E5M2", codes), np.array([O.lib.or_e5m2(int(b)) for b in codes], np.float32),
                          equal_nan=True)
    assert np.signbit(W.to_float32("F8_E4M3", [0x80])[0])


# ---- a double-stream block image through a file ---------------------------------------------------------------

def test_block_image_round_trips_through_a_file(path):
    cfg = B.BlockConfig(256, 512, 2, 2, 128, 1e-6)
    layout = B.StreamLayout(cfg)
    image = np.zeros(layout.nbytes, np.uint8)
    layout.fill(image, np.random.default_rng(3))
    scales = {s: {n: 0.01 * (i + 1) + (s == "img") for i, n in enumerate(layout.FP8_FIELDS)} for s in ("txt", "img")}
    W.save(path, layout.file_tensors(image, scales, "double_blocks.4."))
    back = np.full(layout.nbytes, 0xAB, np.uint8)
    with W.read_header(path) as st:
        got = layout.fill_from_file(st, "double_blocks.4.", back.ctypes.data)
    for s, name, off, nbytes in layout.fields:
        assert np.array_equal(back[off:off + nbytes], image[off:off + nbytes]), (s, name)
    assert got == {s: {n: float(np.float32(v)) for n, v in d.items()} for s, d in scales.items()}


def test_block_loader_checks_shapes_and_names(path):
    cfg = B.BlockConfig(256, 512, 2, 2, 128, 1e-6)
    layout = B.StreamLayout(cfg)
    image = np.zeros(layout.nbytes, np.uint8)
    tensors = layout.file_tensors(image, {s: dict.fromkeys(layout.FP8_FIELDS, 1.0) for s in ("txt", "img")}, "b.")
    dtype, shape, data = tensors["b.img_mlp.0.weight"]
    tensors["b.img_mlp.0.weight"] = ("BF16", (shape[0] // 2, shape[1]), data)
    W.save(path, tensors)
    with W.read_header(path) as st, pytest.raises(we.WeError, match=r"b.img_mlp.0.weight: expected a 2D F8_E4M3 tensor"):
        layout.fill_from_file(st, "b.", image.ctypes.data)
    with W.read_header(path) as st, pytest.raises(we.WeError, match="Missing tensor c.txt_attn.qkv.weight"):
        layout.fill_from_file(st, "c.", image.ctypes.data)

"""CPU checks of the C-ABI library: it loads, exports every function include/we.h declares, and its pure
host logic (parameter validation, kSplitFor) matches the reference without touching a GPU."""
import ctypes
import subprocess

import pytest

import we


def test_library_exports_every_declared_symbol():
    lib = we.load_library()
    declared = we.header_functions()
    assert len(declared) >= 30
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing, missing
    assert set(declared) == set(we.SIGNATURES), set(declared) ^ set(we.SIGNATURES)
    out = subprocess.run(["nm", "-D", "--defined-only", str(we.LIB_PATH)], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}
    assert set(declared) <= exported


def test_library_has_gfx950_code_object():
    blob = we.LIB_PATH.read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    assert b"amdgcn-amd-amdhsa--gfx942" not in blob  # built for MI355X only


def test_params_validation_messages_without_gpu():  # tests/gpu/matmul.test.ts:68-72
    with pytest.raises(we.WeError, match="K must be a multiple of 4, got 6"):
        we.matmul_params(1, 1, 6, 1.0)
    with pytest.raises(we.WeError, match="xStride must be a multiple of 4, got 6"):
        we.matmul_params(1, 1, 4, 1.0, x_stride=6)
    with pytest.raises(we.WeError, match="wOffset must be a multiple of 4, got 2"):
        we.matmul_params(1, 1, 4, 1.0, w_offset=2)
    p = we.matmul_params(3, 5, 8, 0.25, k_split=2)
    assert (p.m, p.n, p.k, p.x_stride, p.w_stride, p.y_stride, p.k_split) == (3, 5, 8, 8, 8, 5, 2)
    assert ctypes.sizeof(we.MatmulParams) == 52  # 13 x u32, like the reference's Params buffer
    assert ctypes.c_uint32.from_buffer_copy(bytes(p)[12:16]).value == ctypes.c_uint32.from_buffer_copy(
        ctypes.c_float(0.25)).value


def test_ksplit_for_known_answers():  # tests/gpu/matmul.test.ts:151-156
    assert we.k_split_for(1088, 64, 6144) == 24
    assert we.k_split_for(4160, 64, 16384) == 8
    assert we.k_split_for(4160, 6144, 6144) == 1
    assert we.k_split_for(5, 12, 16) == 1

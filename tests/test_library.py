"""CPU checks of the product library: it is built, loads, and exports every entry point the C
header declares (no compute call: there is no GPU here)."""

import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fusor_gpu.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fg_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_symbols()
    for want in ("fg_table_create", "fg_matmul", "fg_quantize_rows", "fg_dequantize_row", "fg_encode",
                 "fg_qwen2_step", "fg_last_error"):
        assert want in names


def test_library_loads_and_exports_every_declared_symbol():
    from fusor_kernels import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(lib, name), name
    # the binding declares exactly the header's entry points
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_version_and_error_calls_need_no_gpu():
    from fusor_kernels import _lib
    lib = _lib.lib()
    assert lib.fg_version() == 1
    assert lib.fg_table_byte_len(1, 4864, 896) == 4864 * 896 + 4864 * 896 // 32 * 4
    # the reference's message for a matrix of partial groups (tensor.rs:332-361), from argument
    # checks that run before any device call
    rc = lib.fg_encode(3, 1, 64, None, None, None)
    assert rc == _lib.FG_ERR_FORMAT
    assert lib.fg_last_error().decode() == "a T2b128 tensor of shape [1, 64]: a matrix of whole groups of 128 expected"
    rc = lib.fg_quantize_rows(None, 33, 1, None, None, None, None)
    assert rc == _lib.FG_ERR_SHAPE

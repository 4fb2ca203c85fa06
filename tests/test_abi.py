"""The C-ABI library: it loads, exports every entry point include/ckh.h declares, and
rejects bad arguments with an error code and message -- all without a GPU (argument
validation happens before any HIP call)."""
import ctypes
import re
from pathlib import Path

import pytest

import comfy_kitchen.backends.hip as hb

HEADER = Path(__file__).resolve().parent.parent / "include" / "ckh.h"


def declared_symbols() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ckh_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return hb.load_library()


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(hb.SIGNATURES)


def test_every_declared_symbol_is_exported(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    assert lib.ckh_abi_version() == hb.ABI_VERSION == 8


def test_amax_workspace_size_matches_header():
    m = re.search(r"#define CKH_AMAX_WORKSPACE_BYTES (\d+)", HEADER.read_text())
    assert m and int(m.group(1)) == hb.AMAX_WORKSPACE_BYTES


def test_invalid_arguments_return_error(lib):
    assert lib.ckh_quantize_fp8(None, None, None, 16, 2, 5, 0) == 1
    assert b"null pointer" in lib.ckh_last_error()
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf)
    assert lib.ckh_quantize_fp8(p, p, p, 16, 7, 5, 0) == 1
    assert b"unsupported input dtype" in lib.ckh_last_error()
    assert lib.ckh_dequantize_fp8(p, p, p, 16, 5, 2, 5, 0) == 1
    assert b"unsupported scale dtype" in lib.ckh_last_error()
    assert lib.ckh_apply_rope(p, None, p, p, None, 1, 1, 1, 128, 1, 1, 1, 128, 128, 128, 256, 256, 256, 5, 0, 0) == 1
    assert b"unsupported x dtype" in lib.ckh_last_error()
    assert lib.ckh_quantize_mxfp8(p, p, p, 4, 48, 4, 48, 2, 0) == 1
    assert b"multiple of 32" in lib.ckh_last_error()
    assert lib.ckh_apply_rope(p, None, p, p, p, 1, 1, 1, 128, 1, 1, 1, 128, 128, 128, 256, 256, 256, 2, 0, 0) == 1
    assert b"xk and xk_out" in lib.ckh_last_error()
    assert lib.ckh_apply_rope(p, None, p, p, None, 1, 2, 3, 128, 1, 5, 3, 0, 0, 0, 0, 0, 0, 2, 0, 0) == 1
    assert b"does not broadcast" in lib.ckh_last_error()
    f = lib.ckh_amax_scale
    f.argtypes = hb.SIGNATURES["ckh_amax_scale"][1]
    assert f(p, 16, 2, 448.0, p, None, 0) == 1  # no workspace
    assert b"null pointer" in lib.ckh_last_error()
    assert f(p, 16, 2, 448.0, p, p + 2, 0) == 1
    assert b"misaligned" in lib.ckh_last_error()
    assert f(p, 0, 2, 448.0, p, p, 0) == 1
    assert b"empty tensor" in lib.ckh_last_error()
    g = lib.ckh_amax_scale_noalloc
    assert g(p, 16, 2, 448.0, None, 0) == 1
    assert b"null pointer" in lib.ckh_last_error()
    assert g(p, 0, 2, 448.0, p, 0) == 1
    assert b"empty tensor" in lib.ckh_last_error()
    assert g(p, 16, 3, 448.0, p, 0) == 1
    assert b"unsupported input dtype" in lib.ckh_last_error()


def test_zero_sized_calls_are_noops(lib):
    assert lib.ckh_quantize_fp8(None, None, None, 0, 2, 5, 0) == 0
    assert lib.ckh_dequantize_fp8(None, None, None, 0, 5, 2, 0, 0) == 0


def test_quantize_nvfp4_dynamic_rejects_bad_arguments(lib):
    buf = ctypes.create_string_buffer(256)
    p = ctypes.addressof(buf)
    f = lib.ckh_quantize_nvfp4_dynamic
    assert f(p, 2688.0, p, p, p, 16, 64, 16, 64, 0.0, 2, 1, None, 0) == 1  # no workspace
    assert b"null pointer" in lib.ckh_last_error()
    assert f(p, 2688.0, p, p, p, 0, 64, 0, 64, 0.0, 2, 1, p, 0) == 1
    assert b"empty tensor" in lib.ckh_last_error()
    assert f(p, 2688.0, p, p, p, 16, 40, 16, 40, 0.0, 2, 1, p, 0) == 1
    assert b"multiple of 16" in lib.ckh_last_error()

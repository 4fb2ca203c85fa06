"""Compile oracle/scalar_ref.c into oracle/_build/libscalar_ref.so (test infrastructure).

    python oracle/build_ref.py

gcc with -ffp-contract=off -fno-fast-math: each float operation rounds exactly once.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "scalar_ref.c"
OUT = HERE / "_build" / "libscalar_ref.so"


def build(verbose: bool = True) -> Path:
    OUT.parent.mkdir(exist_ok=True)
    cmd = ["gcc", "-O2", "-std=c11", "-shared", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
           "-o", str(OUT), str(SRC), "-lm"]
    subprocess.run(cmd, check=True)
    if verbose:
        print(f"built {OUT}")
    return OUT


def load():
    """ctypes handle to the scalar reference with argument types bound."""
    import ctypes

    if not OUT.exists():
        build(verbose=False)
    lib = ctypes.CDLL(str(OUT))
    p, i64, f32, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_int
    lib.ref_e4m3_value.restype, lib.ref_e4m3_value.argtypes = ctypes.c_double, [i32]
    lib.ref_e5m2_value.restype, lib.ref_e5m2_value.argtypes = ctypes.c_double, [i32]
    lib.ref_e2m1_value.restype, lib.ref_e2m1_value.argtypes = ctypes.c_double, [i32]
    for fn in ("ref_f32_to_e4m3", "ref_f32_to_e5m2", "ref_f32_to_e2m1"):
        getattr(lib, fn).restype, getattr(lib, fn).argtypes = i32, [f32]
    lib.ref_f32_to_bf16.restype, lib.ref_f32_to_bf16.argtypes = ctypes.c_uint16, [f32]
    lib.ref_quantize_fp8_bf16.restype, lib.ref_quantize_fp8_bf16.argtypes = None, [p, i64, f32, i32, p]
    lib.ref_quantize_mxfp8_row_bf16.restype, lib.ref_quantize_mxfp8_row_bf16.argtypes = None, [p, i64, p, p]
    lib.ref_quantize_nvfp4_row_bf16.restype, lib.ref_quantize_nvfp4_row_bf16.argtypes = None, [p, i64, f32, p, p]
    lib.ref_default_scale.restype, lib.ref_default_scale.argtypes = f32, [f32, f32, i32]
    lib.ref_dequantize_nvfp4_value.restype, lib.ref_dequantize_nvfp4_value.argtypes = f32, [i32, i32, f32, i32]
    return lib


if __name__ == "__main__":
    build()

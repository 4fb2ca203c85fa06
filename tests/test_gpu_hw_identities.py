"""Exhaustive checks of the gfx950 instruction identities the bit-exact fast paths rely on.

The sweeps (tests/hw/identities.hip, built into tests/hw/libckh_hwcheck.so) run the very
helpers the product kernels call (csrc/ckh_common.h, csrc/quant_math.h) against their
software or IEEE definitions over each identity's whole domain:

  e4m3 / e5m2 / bf16 converts   all 2^32 fp32 inputs (after the kernels' clamps)
  E2M1 pack (saturating)        all 2^32 fp32 inputs, both nibble orders
  E4M3 decode                   all 256 codes
  scaled E4M3 convert           all 2^16 bf16 / f16 inputs x all 254 normal E8M0 scales
  rcp + Newton reciprocal       every fp32 T in [2^-70, 2^71)
  Markstein quotient codes      every T significand x every bf16 / f16 v (both signs)
  (amax/6)/g Markstein steps    every f16 amax significand x every g significand
  MXFP8 exponent closed form    every finite amax with biased exponent >= 10
  NVFP4 GEMM operand decode     every code byte x every pair of finite scale bytes

A toolchain or ROCm change that broke one of them would break the quantizers' or the
GEMMs' agreement with the reference silently on data the other tests never hit.
"""
import ctypes
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "hw" / "libckh_hwcheck.so"
SWEEPS = {
    "e4m3_convert": 0, "e5m2_convert": 1, "bf16_convert": 2, "e2m1_pack": 3, "e4m3_decode": 4,
    "scaled_e4m3_bf16": 5, "scaled_e4m3_f16": 6, "rcp_newton": 7, "markstein_bf16": 8,
    "markstein_f16": 9, "nvfp4_scale_steps": 10, "mx_exponent": 11, "nvfp4_gemm_decode": 12,
}
CHUNK = 1 << 34  # indices per launch (each launch well under a second)


@pytest.fixture(scope="module")
def lib(hip):
    if not LIB.exists():
        pytest.fail(f"{LIB} missing: run python comfy-kitchen_amd/build.py")
    h = ctypes.CDLL(str(LIB))
    h.ckh_hw_sweep_size.restype = ctypes.c_uint64
    h.ckh_hw_sweep_size.argtypes = [ctypes.c_int]
    h.ckh_hw_sweep.restype = ctypes.c_int
    h.ckh_hw_sweep.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64]
    return h


@pytest.mark.parametrize("name", list(SWEEPS))
def test_hardware_identity(name, lib):
    which = SWEEPS[name]
    n = lib.ckh_hw_sweep_size(which)
    assert n > 0
    counts = torch.tensor([0, -1], dtype=torch.int64, device="cuda")  # mismatches, smallest bad index
    stream = torch.cuda.current_stream().cuda_stream
    for begin in range(0, n, CHUNK):
        assert lib.ckh_hw_sweep(which, begin, min(n, begin + CHUNK), counts.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    bad, first = counts.cpu().tolist()
    assert bad == 0, f"{name}: {bad} of {n} inputs differ; first at index {first & (2**64 - 1):#x}"

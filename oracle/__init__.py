"""CPU oracle for the quantize / block-scaled GEMM / RoPE path -- TEST INFRASTRUCTURE ONLY.

eager_ref.py restates the reference's eager backend with torch CPU ops; scalar_ref.c is
an independent brute-force scalar restatement used to pin it.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import anything here, and
only as the checker or the timed CPU baseline -- never as the product path.

The reference's own native code (backends/cuda/*.cu, cuBLASLt) needs nvcc, nanobind and
an NVIDIA GPU, none of which exist here, so there is no oracle/_ref build.
"""

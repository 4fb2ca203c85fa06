"""Write tests/golden/checkpoints.safetensors: quantized linear layers in the reference's
checkpoint convention, made by the CPU oracle, with the oracle's expected outputs.

    python tests/golden/make_checkpoints.py

Keys, dtypes and shapes follow the reference layouts' state_dict_tensors
(tensor/fp8.py:74-80, tensor/mxfp8.py:86-87, tensor/nvfp4.py:94-101): per layer
`<layer>.weight` (codes: float8_e4m3fn [N, K], or uint8 [N, K/2] for NVFP4),
`<layer>.weight_scale` (the FP8 tensor scale as a 0-dim fp32; the swizzled block scales as
2-D float8_e8m0fnu / float8_e4m3fn), `<layer>.weight_scale_2` (the NVFP4 tensor scale, 0-dim
fp32), plus `<layer>.input_scale` (NVFP4 static activation scale, fp32 [1], as
samples/nvfp4_linear.py:93-99 writes it) and `<layer>.bias`; samples/nvfp4_linear.py:39-61
loads them.

Layers, each [N=128, K=256] from one bf16 weight `w_bf16`:
  fp8    TensorCoreFP8Layout, tensor scale amax/448
  mxfp8  TensorCoreMXFP8Layout
  nvfp4  TensorCoreNVFP4Layout, weight_scale_2 = amax/2688, input_scale = amax(x)/2688 * 1.25
Also the activation `x` [32, 256] bf16 and, per layer, the oracle's fp32 result of
F.linear(quantize(x), weight) + bias: `<layer>.expected` (the activation quantized with the
layout's default dynamic scale) and, for nvfp4, `nvfp4.expected_static` (with input_scale).
Everything comes from oracle/eager_ref.py (CPU); no GPU code is involved.
"""
from __future__ import annotations

import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))
from oracle import eager_ref as ref  # noqa: E402

OUT = Path(__file__).resolve().parent / "checkpoints.safetensors"
N, K, M = 128, 256, 32


def make() -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(1234)
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16()
    x = (torch.randn(M, K, generator=g) * torch.exp(torch.randn(M, 1, generator=g))).bfloat16()
    bias = (torch.randn(N, generator=g) * 0.1).bfloat16()
    sd = {"w_bf16": w, "x": x}

    # per-tensor FP8 (tensor/fp8.py:74-80: "" and "_scale")
    sw = ref.default_scale(w, 448.0).reshape(())
    qw = ref.quantize_per_tensor_fp8(w, sw.reshape(1))
    sx = ref.default_scale(x, 448.0).reshape(())
    qx = ref.quantize_per_tensor_fp8(x, sx.reshape(1))
    y = (ref.dequantize_per_tensor_fp8(qx, sx.reshape(1), torch.float32)
         @ ref.dequantize_per_tensor_fp8(qw, sw.reshape(1), torch.float32).T) + bias.float()
    sd.update({"fp8.weight": qw, "fp8.weight_scale": sw.reshape(()), "fp8.bias": bias, "fp8.expected": y})

    # MXFP8 (tensor/mxfp8.py:86-87: "" and "_scale", E8M0 bytes swizzled)
    qw, bw = ref.quantize_mxfp8(w)
    qx, bx = ref.quantize_mxfp8(x)
    y = ref.scaled_mm_mxfp8_ref(qx, qw, bx, bw, out_dtype=torch.float32) + bias.float()
    sd.update({"mxfp8.weight": qw, "mxfp8.weight_scale": bw, "mxfp8.bias": bias, "mxfp8.expected": y})

    # NVFP4 (tensor/nvfp4.py:94-101; samples/nvfp4_linear.py:39-61)
    gw = ref.default_scale(w, 2688.0).reshape(1)
    qw, bw = ref.quantize_nvfp4(w, gw)
    gx = ref.default_scale(x, 2688.0).reshape(1)
    qx, bx = ref.quantize_nvfp4(x, gx)
    y = ref.scaled_mm_nvfp4_ref(qx, qw, gx, gw, bx, bw, out_dtype=torch.float32) + bias.float()
    g_in = (gx * 1.25).reshape(1)  # a calibrated static input scale, not the dynamic one
    qs, bs = ref.quantize_nvfp4(x, g_in)
    y_static = ref.scaled_mm_nvfp4_ref(qs, qw, g_in, gw, bs, bw, out_dtype=torch.float32) + bias.float()
    sd.update({"nvfp4.weight": qw, "nvfp4.weight_scale": bw, "nvfp4.weight_scale_2": gw.reshape(()),
               "nvfp4.input_scale": g_in, "nvfp4.bias": bias, "nvfp4.expected": y,
               "nvfp4.expected_static": y_static})
    return {k: v.contiguous().clone() for k, v in sd.items()}


if __name__ == "__main__":
    save_file(make(), str(OUT))
    print(f"wrote {OUT.relative_to(REPO)}")

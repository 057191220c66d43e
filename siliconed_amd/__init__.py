"""siliconed_amd — Siliconed's weight-quantized linear layer, MI355X-native (gfx950).

int8 / fp8-e4m3 weights with per-output-channel fp32 scales × bf16 activations, fp32 sums in the
matrix cores, fused scale + bias + GELU-tanh / SiLU-GLU / SITU-GLU epilogue, fused QKV, and ComfyUI's convrot rotation. The work
is done by the HIP library libsiliconed_q8.so (C ABI: include/siliconed_q8.h); this package holds
its host side. There is no CPU fallback: without the library, importing the operators fails.
"""
from . import _abi as abi
from .tensor_gemm import (PackedWeight, TensorGEMM, context, dequantize, dequantize_rotated, linear, linear_qkv, pack,
                          rotate, round_bf16)

__all__ = ["abi", "PackedWeight", "TensorGEMM", "context", "linear", "linear_qkv", "pack", "dequantize",
           "dequantize_rotated", "rotate", "round_bf16"]

"""Per-tensor FP8 projection module for audited ``nn.Linear`` call sites.

Drop-in for the reference's ``ThorFP8Linear`` (instinctflash/runtime/
torch_fp8_linear.py:10-79) on gfx950: same recipe string, constructor contract
and error behaviour, with the CUDA capability check replaced by a gfx950 check
and ``torch._scaled_mm`` + the Triton packer replaced by this package's HIP
kernels:

  * weight: per-tensor E4M3, scale = max(amax, 1e-12) * fl32(1/448) (the device
    scalar-division semantics of torch_fp8_linear.py:39-48);
  * activations: dynamic per-tensor E4M3 with the same recipe
    (runtime/fp8_pack.py:83-91, NaN anywhere -> NaN scale);
  * out = bf16(acc * scale_a * scale_w + bias), fp32 accumulation
    (torch_fp8_linear.py:75-78).
"""
from __future__ import annotations

import torch
from torch import nn

from .backend import is_gfx950
from .kernels.fp8 import E4M3, Fp8Weight, quant_linear, quantize_tensor


class Gfx950FP8Linear(nn.Module):
    recipe = "e4m3fn_weights_dynamic_per_tensor_activations_fp32_accum_bf16_output"

    def __init__(self, linear_module: nn.Linear, *, device=None, storage_device=None):
        super().__init__()
        if type(linear_module) is not nn.Linear:
            raise TypeError("FP8 packing requires a plain nn.Linear with no custom forward")
        w = linear_module.weight.detach()
        target = torch.device(device) if device is not None else w.device
        if target.type != "cuda" or not is_gfx950(target):
            raise ValueError("FP8 projections require a gfx950 (MI355X) device")
        storage = torch.device(storage_device) if storage_device is not None else target
        if storage != target:
            raise ValueError("Separate packed storage is not supported: pack on the target device")
        if w.dtype != torch.bfloat16:
            raise ValueError("This FP8 recipe requires native BF16 projection weights")
        if linear_module.in_features % 16 or linear_module.out_features % 16:
            raise ValueError("FP8 projection input/output dimensions must be multiples of 16")
        w = w.to(target)
        if not torch.isfinite(w).all():
            raise ValueError("Cannot quantize non-finite projection weights")
        self.in_features, self.out_features = linear_module.in_features, linear_module.out_features
        packed, scale = quantize_tensor(w.contiguous())
        self.register_buffer("weight_fp8", packed)
        self.register_buffer("weight_scale", scale)
        bias = linear_module.bias.detach() if linear_module.bias is not None else None
        if bias is not None and (bias.dtype != torch.bfloat16 or not torch.isfinite(bias).all()):
            raise ValueError("This FP8 recipe requires finite BF16 bias")
        self.register_buffer("bias", bias.to(target).clone() if bias is not None else None)

    @torch.no_grad()
    def forward(self, x):
        if x.ndim < 1 or x.shape[-1] != self.in_features:
            raise ValueError("FP8 projection input has incompatible feature dimension")
        if x.dtype != torch.bfloat16 or x.device != self.weight_fp8.device:
            raise ValueError("FP8 projection input must be BF16 on the packed weight device")
        if self.weight_fp8.dtype != E4M3 or self.weight_scale.dtype != torch.float32:
            raise RuntimeError("FP8 packed buffers were cast after construction; pack after model.to()")
        shape = (*x.shape[:-1], self.out_features)
        if x.numel() == 0:
            return x.new_empty(shape)
        rows = x.reshape(-1, self.in_features).contiguous()
        bias = None if self.bias is None else self.bias.float()
        # dynamic per-tensor activation scale, then the GEMM
        out = quant_linear(rows, Fp8Weight(self.weight_fp8, self.weight_scale, bias), per_tensor=True)
        return out.reshape(shape)

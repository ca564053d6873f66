"""The reference's PyTorch CPU FP8 projection path, timed as bench.py's CPU
baseline -- TEST/BENCH INFRASTRUCTURE ONLY (never part of the product path).

Restates the GI-engine decomposition (instinctflash/kernels/fp8.py:30-53 with the
consumer math of kernels/norm.py:45-58,135-144 and kernels/activation.py:26-40)
with torch CPU operators:
  1. per-token quantization: scale = amax.clamp_min(1e-12) * fl32(1/448) (the
     device scalar-division semantics, instinctflash/runtime/torch_fp8_linear.py:
     39-48), q = (x / scale).clamp(+-448).to(float8_e4m3fn);
  2. torch._scaled_mm(q, W8.t(), scale_a=1, scale_b=1, out_dtype=bf16) -- the
     raw accumulator, exactly as kernels/fp8.py:50-53 (oneDNN on the CPU);
  3. fp32 epilogue: raw * row_scale * col_scale + bias -> activation ->
     gate -> residual -> bf16.
"""
from __future__ import annotations

import torch
import torch.nn.functional as Fn

_INV448 = torch.tensor(1.0 / 448.0, dtype=torch.float32)
_ONE = torch.ones((), dtype=torch.float32)


def quant_rows(x: torch.Tensor):
    xf = x.float()
    scale = xf.abs().amax(dim=1).clamp_min(1e-12) * _INV448
    q = (xf / scale[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q, scale


def _epilogue(y, bias=None, act=None, residual=None, gate=None):
    """fp32 consumer math of the reference (kernels/norm.py:45-58,135-144,
    kernels/activation.py:26-40): + bias, activation (GLU halves: gate rows
    then up rows), * adaLN gate, + residual, then bf16."""
    if bias is not None:
        y = y + bias
    if act == "gelu_tanh":
        y = Fn.gelu(y, approximate="tanh")
    elif act in ("geglu", "swiglu"):
        F = y.shape[1] // 2
        g, u = y[:, :F], y[:, F:]
        y = (Fn.gelu(g, approximate="tanh") if act == "geglu" else Fn.silu(g)) * u
    if gate is not None:
        y = y * gate.float()
    if residual is not None:
        y = residual.float() + y
    return y.to(torch.bfloat16)


def linear(q, sa, w8, sw, bias=None, act=None, residual=None, gate=None):
    raw = torch._scaled_mm(q, w8.t(), scale_a=_ONE, scale_b=_ONE, out_dtype=torch.bfloat16)
    return _epilogue(raw.float() * sa[:, None] * sw[None, :], bias, act, residual, gate)


def c2_unit(xs, w1, s1, w2, s2, res):
    """One timed unit of config C2: 4 flow-matching steps of up(GELU) + down(+res)."""
    out = None
    for x in xs:
        q, sa = quant_rows(x)
        h = linear(q, sa, w1, s1, act="gelu_tanh")
        q2, sa2 = quant_rows(h)
        out = linear(q2, sa2, w2, s2, residual=res)
    return out


def linear_fp32(q, sa, wd, bias=None, act=None, residual=None, gate=None):
    """Dequantize-then-fp32-matmul (benchmarks/native/fp8_probe.py:36): wd is the
    dequantized weight (q_w * s_w) in fp32; the activation is dequantized per row."""
    return _epilogue((q.float() * sa[:, None]) @ wd.t(), bias, act, residual, gate)


def c2_unit_fp32(xs, wd1, wd2, res):
    """C2 unit with the dequantize-then-fp32-matmul CPU path (MKL)."""
    out = None
    for x in xs:
        q, sa = quant_rows(x)
        h = linear_fp32(q, sa, wd1, act="gelu_tanh")
        q2, sa2 = quant_rows(h)
        out = linear_fp32(q2, sa2, wd2, residual=res)
    return out

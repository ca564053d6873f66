"""Consumer-side row kernels of the reference's FP8 pipeline, on HIP.

``row_quant`` and ``dequant_rows`` keep the reference signatures
(instinctflash/kernels/norm.py:150 and :178) so an engine can call them
unchanged. The quantization they perform follows the bit-exact recipe of
``quant_rows`` (scale floor 1e-12, scale = amax * fl32(1/448), IEEE division).
``num_warps`` / ``block`` are accepted for signature compatibility; the HIP
kernels pick their own launch shape.
"""
from __future__ import annotations

import torch

from .. import _lib
from .fp8 import E4M3, _ptr, _rows, _stream, _vec


def row_quant(x, q, q_scale, *, row=None, col=None, bias=None, gelu=False, num_warps=None):
    """q[m] = fp8((x[m] * row[m] * col + bias) [-> gelu_tanh] / s[m]) with per-row s.

    Reference: instinctflash/kernels/norm.py:150-158."""
    M, D, ldx = _rows("x", x, torch.bfloat16)
    _, _, ldq = _rows("q", q, E4M3, x.device, cols=D)
    _vec("q_scale", q_scale, M, device=x.device)
    _vec("row", row, M, device=x.device)
    _vec("col", col, D, device=x.device)
    _vec("bias", bias, D, device=x.device)
    _lib.check(_lib.load().ifx_row_quant(_ptr(x), ldx, M, D, _ptr(row), _ptr(col), _ptr(bias),
                                         1 if gelu else 0, _ptr(q), ldq, _ptr(q_scale),
                                         _stream(x.device)), "ifx_row_quant")


def dequant_rows(x, y, *, row=None, col=None, bias=None, block=None, num_warps=4):
    """y[m] = x[m] * row[m] * col + bias; x bf16, y bf16 or fp32.

    Reference: instinctflash/kernels/norm.py:178-185."""
    M, D, ldx = _rows("x", x, torch.bfloat16)
    if y.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("y must be bf16 or fp32")
    _, _, ldy = _rows("y", y, y.dtype, x.device, cols=D)
    _vec("row", row, M, device=x.device)
    _vec("col", col, D, device=x.device)
    _vec("bias", bias, D, device=x.device)
    dt = _lib.DTYPE_F32 if y.dtype == torch.float32 else _lib.DTYPE_BF16
    _lib.check(_lib.load().ifx_dequant_rows(_ptr(x), ldx, M, D, _ptr(row), _ptr(col), _ptr(bias), _ptr(y),
                                            dt, ldy, _stream(x.device)), "ifx_dequant_rows")

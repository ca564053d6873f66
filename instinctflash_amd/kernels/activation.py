"""Gated MLP activation + per-row FP8 requantization, on HIP.

Keeps the signature of instinctflash/kernels/activation.py:46 so an engine can
call it unchanged. ``gu`` is the raw bf16 gate|up accumulator [M, 2F] in the
reference's (non-interleaved) layout:

    g = gu[m, :F] * row[m] * col[:F]      u = gu[m, F:] * row[m] * col[F:]
    h = act(g) * u,  act in {gelu_tanh, silu}
    q[m], s[m] = quantize(h) with the bit-exact per-row recipe of quant_rows.

The fused alternative is ``linear(..., act="geglu"|"swiglu")`` on a
``pack_glu`` weight followed by ``quant_rows`` of its bf16 output.
"""
from __future__ import annotations

import torch

from .. import _lib
from .fp8 import E4M3, _ptr, _rows, _stream, _vec

GELU_TANH = _lib.ACT_GELU_TANH
SILU = _lib.ACT_SILU


def gated_act_quant(gu, q, q_scale, *, row=None, col=None, act=GELU_TANH, num_warps=None):
    M, F2, ldgu = _rows("gu", gu, torch.bfloat16)
    if F2 % 2:
        raise ValueError("gu must have an even number of columns (gate | up)")
    F = F2 // 2
    if F > 16384:
        # Same width contract as the reference (kernels/activation.py:50-51).
        raise ValueError("gated_act_quant supports hidden widths up to 16384")
    if act not in (GELU_TANH, SILU):
        raise ValueError(f"act must be GELU_TANH ({GELU_TANH}) or SILU ({SILU})")
    _, _, ldq = _rows("q", q, E4M3, gu.device, cols=F)
    _vec("q_scale", q_scale, M, device=gu.device)
    _vec("row", row, M, device=gu.device)
    _vec("col", col, F2, device=gu.device)
    _lib.check(_lib.load().ifx_gated_act_quant(_ptr(gu), ldgu, M, F, _ptr(row), _ptr(col), act, _ptr(q), ldq,
                                               _ptr(q_scale), _stream(gu.device)), "ifx_gated_act_quant")

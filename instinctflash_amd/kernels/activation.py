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
from .fp8 import E4M3, _ptr, _qout, _rows, _stream, _vec

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
    qp, ldq = _qout("q", q, M, F, gu.device)
    _vec("q_scale", q_scale, M, device=gu.device)
    _vec("row", row, M, device=gu.device)
    _vec("col", col, F2, device=gu.device)
    _lib.check(_lib.load().ifx_gated_act_quant(_ptr(gu), ldgu, M, F, _ptr(row), _ptr(col), act, qp, ldq,
                                               _ptr(q_scale), _stream(gu.device)), "ifx_gated_act_quant")


def _f32_matrix(name, t, rows, cols, device):
    if t.dtype != torch.float32 or t.device != device or tuple(t.shape) != (rows, cols) or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 [{rows}, {cols}] tensor on {device}")


def moe_router(x, gate_w, e_bias, route_w, *, top_k, scale):
    """route_w[t, e] = the normalized sigmoid weight of expert e for token t when
    e is among the token's top_k experts by sigmoid(logits) + e_bias, else 0.

    Reference: instinctflash/kernels/activation.py:91-100. logits = x @ gate_w.T
    (x [M, D] bf16 or fp32, gate_w fp32 [E, D]); the weights use the unbiased
    sigmoid and sum to ``scale`` per token; equal selection scores pick the
    lowest expert index first. D <= 16384, E <= 256."""
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("x must be bf16 or fp32")
    M, D, ldx = _rows("x", x, x.dtype)
    dev = x.device
    E = gate_w.shape[0] if gate_w.dim() == 2 else -1
    _f32_matrix("gate_w", gate_w, E, D, dev)
    _vec("e_bias", e_bias, E, device=dev)
    _f32_matrix("route_w", route_w, M, E, dev)
    if not 0 <= int(top_k) <= E:
        raise ValueError(f"top_k must be in [0, {E}]")
    _lib.check(_lib.load().ifx_moe_router(
        _ptr(x), _lib.DTYPE_F32 if x.dtype == torch.float32 else _lib.DTYPE_BF16, ldx, M, D, _ptr(gate_w),
        _ptr(e_bias), _ptr(route_w), E, int(top_k), float(scale), _stream(dev)), "ifx_moe_router")


def moe_act_quant(gu, q, q_scale, route_w, *, row, col, experts, group, n_routed, block=4096, num_warps=8):
    """h = silu(g) * u * route_w[t, min(c // group, experts-1)] for routed columns
    c < n_routed, weight 1 for the shared expert's columns; q, q_scale = per-row
    E4M3 of h.

    Reference: instinctflash/kernels/activation.py:131-137 (same keywords;
    ``block`` and ``num_warps`` are accepted for signature compatibility). ``gu``
    is the raw bf16 [M, 2F] accumulator of the concatenated experts' gate|up
    projection, ``row`` [M] / ``col`` [2F] its dequantization scales. The
    quantization is this package's per-row recipe (as quant_rows)."""
    M, F2, ldgu = _rows("gu", gu, torch.bfloat16)
    if F2 % 2:
        raise ValueError("gu must have an even number of columns (gate | up)")
    F = F2 // 2
    dev = gu.device
    E, G, NR = int(experts), int(group), int(n_routed)
    if E <= 0 or G <= 0 or not 0 <= NR <= F:
        raise ValueError("experts and group must be positive and n_routed in [0, F]")
    qp, ldq = _qout("q", q, M, F, dev)
    _vec("q_scale", q_scale, M, device=dev)
    _vec("row", row, M, device=dev)
    _vec("col", col, F2, device=dev)
    _f32_matrix("route_w", route_w, M, E, dev)
    _lib.check(_lib.load().ifx_moe_act_quant(_ptr(gu), ldgu, M, F, _ptr(row), _ptr(col), _ptr(route_w), E, G, NR,
                                             qp, ldq, _ptr(q_scale), _stream(dev)), "ifx_moe_act_quant")

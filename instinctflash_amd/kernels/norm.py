"""Consumer-side row kernels of the reference's FP8 pipeline, on HIP.

``residual_norm_quant``, ``row_quant`` and ``dequant_rows`` keep the reference
signatures (instinctflash/kernels/norm.py:97, :150 and :178) so an engine can
call them unchanged. The quantization they perform follows the bit-exact recipe of
``quant_rows`` (scale floor 1e-12, scale = amax * fl32(1/448), IEEE division).
``num_warps`` / ``block`` are accepted for signature compatibility; the HIP
kernels pick their own launch shape.
"""
from __future__ import annotations

import torch

from .. import _lib
from .fp8 import E4M3, _ptr, _qout, _rows, _stream, _vec


def row_quant(x, q, q_scale, *, row=None, col=None, bias=None, gelu=False, num_warps=None):
    """q[m] = fp8((x[m] * row[m] * col + bias) [-> gelu_tanh] / s[m]) with per-row s.

    Reference: instinctflash/kernels/norm.py:150-158. ``x`` is bf16, fp16
    (the pi05 engine's attention output, engines/pi05/engine.py:205) or
    float32 (the GR00T engine's encoder rows, engines/groot_n17/engine.py:144)."""
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError("row_quant expects bf16, fp16 or fp32 input")
    M, D, ldx = _rows("x", x, x.dtype)
    qp, ldq = _qout("q", q, M, D, x.device)
    _vec("q_scale", q_scale, M, device=x.device)
    _vec("row", row, M, device=x.device)
    _vec("col", col, D, device=x.device)
    _vec("bias", bias, D, device=x.device)
    flags = (_lib.RQ_GELU if gelu else 0) | (_lib.RQ_F16 if x.dtype == torch.float16 else 0) | \
        (_lib.RQ_F32 if x.dtype == torch.float32 else 0)
    _lib.check(_lib.load().ifx_row_quant(_ptr(x), ldx, M, D, _ptr(row), _ptr(col), _ptr(bias),
                                         flags, qp, ldq, _ptr(q_scale),
                                         _stream(x.device)), "ifx_row_quant")


_FLOAT_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16, torch.float32: _lib.DTYPE_F32}


def dequant_rows(x, y, *, row=None, col=None, bias=None, block=None, num_warps=4):
    """y[m] = x[m] * row[m] * col + bias in float32; x and y bf16, fp16 or fp32
    (any combination).

    Reference: instinctflash/kernels/norm.py:178-185."""
    if x.dtype not in _FLOAT_DTYPES or y.dtype not in _FLOAT_DTYPES:
        raise ValueError("dequant_rows takes bf16, fp16 or fp32 x and y")
    M, D, ldx = _rows("x", x, x.dtype)
    _, _, ldy = _rows("y", y, y.dtype, x.device, cols=D)
    _vec("row", row, M, device=x.device)
    _vec("col", col, D, device=x.device)
    _vec("bias", bias, D, device=x.device)
    _lib.check(_lib.load().ifx_dequant_rows(_ptr(x), _FLOAT_DTYPES[x.dtype], ldx, M, D, _ptr(row), _ptr(col),
                                            _ptr(bias), _ptr(y), _FLOAT_DTYPES[y.dtype], ldy, _stream(x.device)),
               "ifx_dequant_rows")


def _table(name, t, D, rows_from_index, device):
    """An f32 per-column vector [D], or with ``mod_index`` a contiguous [n, D] table."""
    if t is None:
        return None
    if t.device != device or t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 tensor on {device}")
    if rows_from_index:
        if t.numel() % D or t.numel() == 0:
            raise ValueError(f"{name} must be a [n, {D}] table when mod_index is given")
    elif t.numel() != D:
        raise ValueError(f"{name} must have {D} elements")
    if t.data_ptr() % 16:
        raise ValueError(f"{name} must be 16-byte aligned")
    return t


def residual_norm_quant(res, *, delta=None, delta_row=None, delta_col=None, bias=None, gate=None,
                        write_res=True, layernorm=False, weight=None, beta=None,
                        mod_scale=None, mod_shift=None, q=None, q_scale=None, y=None, eps=1e-6,
                        num_warps=None, router=None, mod_index=None):
    """Pre-norm producer, one pass per row of ``res`` [M, D] (fp32, or bf16):

        if delta:  res[m] += (delta[m] * delta_row[m] * delta_col + bias) * gate
        y[m] = norm(res[m])                        RMS, or LayerNorm with layernorm=True
        y[m] = y[m] * weight + beta
        y[m] = y[m] * (1 + mod_scale) + mod_shift
        q[m], q_scale[m] = per-row E4M3 of y[m];   y written when given

    Reference: instinctflash/kernels/norm.py:97-123 (same keywords; ``gate``,
    ``mod_scale`` and ``mod_shift`` are [D], or [n, D] tables indexed per row by
    the int32 ``mod_index``). The quantization is this package's recipe
    (1e-12 floor, scale = amax * fl32(1/448), IEEE division) rather than the
    Triton kernel's 1e-8 floor and 448/amax multiply. ``num_warps`` is accepted
    for signature compatibility. ``router=(gate_w [E, D], e_bias [E], out [M, E],
    top_k, scale)`` also writes the MoE routing weights of ``moe_router``
    computed from the float32 normalized row (norm.py:84-94), equal bit for bit
    to ``moe_router`` on a float32 ``y``."""
    if res.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("res must be float32 or bfloat16")
    M, D, ldres = _rows("res", res, res.dtype)
    dev = res.device
    lddelta = 0
    if delta is not None:
        if delta.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("delta must be bfloat16 or float32")
        Md, _, lddelta = _rows("delta", delta, delta.dtype, dev, cols=D)
        if Md != M:
            raise ValueError("delta must have as many rows as res")
    _vec("delta_row", delta_row, M, device=dev)
    for name, t in (("delta_col", delta_col), ("bias", bias), ("weight", weight), ("beta", beta)):
        _table(name, t, D, False, dev)
    indexed = mod_index is not None
    if indexed:
        _vec("mod_index", mod_index, M, dtype=torch.int32, device=dev)
    for name, t in (("gate", gate), ("mod_scale", mod_scale), ("mod_shift", mod_shift)):
        _table(name, t, D, indexed, dev)
    if (mod_scale is None) != (mod_shift is None):
        raise ValueError("mod_scale and mod_shift come together")
    qp, ldq = None, 0
    if q is not None:
        if q_scale is None:
            raise ValueError("q needs a q_scale vector")
        qp, ldq = _qout("q", q, M, D, dev)
        _vec("q_scale", q_scale, M, device=dev)
    ldy = 0
    if y is not None:
        if y.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("y must be float32 or bfloat16")
        My, _, ldy = _rows("y", y, y.dtype, dev, cols=D)
        if My != M:
            raise ValueError("y must have as many rows as res")
    rw = rb = ro = None
    rE, rK, rS = 0, 0, 1.0
    if router is not None:
        from .activation import _f32_matrix
        if len(router) != 5:
            raise ValueError("router must be (gate_w, e_bias, out, top_k, scale)")
        rw, rb, ro, rK, rS = router
        rE = rw.shape[0] if rw.dim() == 2 else -1
        _f32_matrix("router gate_w", rw, rE, D, dev)
        _vec("router e_bias", rb, rE, device=dev)
        _f32_matrix("router out", ro, M, rE, dev)
        if not 0 <= int(rK) <= rE:
            raise ValueError(f"router top_k must be in [0, {rE}]")
    dt = lambda t: _lib.DTYPE_F32 if t is not None and t.dtype == torch.float32 else _lib.DTYPE_BF16  # noqa: E731
    flags = (_lib.RNQ_WRITE_RES if write_res else 0) | (_lib.RNQ_LAYERNORM if layernorm else 0)
    _lib.check(_lib.load().ifx_residual_norm_quant(
        _ptr(res), dt(res), ldres, _ptr(delta), dt(delta), lddelta, _ptr(delta_row), _ptr(delta_col), _ptr(bias),
        _ptr(gate), _ptr(weight), _ptr(beta), _ptr(mod_scale), _ptr(mod_shift), _ptr(mod_index), flags, float(eps),
        qp, ldq, _ptr(q_scale), _ptr(y), dt(y), ldy, _ptr(rw), _ptr(rb), _ptr(ro), rE, int(rK), float(rS), M, D,
        _stream(dev)), "ifx_residual_norm_quant")

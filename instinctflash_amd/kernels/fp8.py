"""Per-channel FP8 weights, the per-token activation quantizer and the FP8 GEMM
with fused epilogue, on gfx950 HIP kernels.

Public names mirror the reference module instinctflash/kernels/fp8.py
(``E4M3``, ``FP8_MAX``, ``Fp8Weight``, ``quantize_weight``, ``gemm``) so an
engine that imports them runs unchanged; ``quant_rows``, ``linear``,
``pack_glu``, ``pack_skinny``, ``quantize_tensor`` and ``quant_linear`` are the fused
entry points of this build.

Every call validates its tensors on the host and raises ``ValueError`` before
anything is launched; kernels run on the current HIP stream and never allocate
(the split-K / quantization workspace is a cached buffer per stream).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _lib

E4M3 = torch.float8_e4m3fn
FP8_MAX = 448.0

ACTIVATIONS = {None: 0, "none": 0, "gelu_tanh": _lib.EPI_GELU_TANH, "geglu": _lib.EPI_GEGLU,
               "swiglu": _lib.EPI_SWIGLU}


@dataclass
class Fp8Weight:
    """Reference: instinctflash/kernels/fp8.py:19-27.

    ``w`` [N, K] E4M3, K contiguous; ``scale`` [N] FP32 per-output-channel
    dequantization scale; ``bias`` [N] FP32 or None. ``glu`` marks a gate|up
    weight already repacked by :func:`pack_glu` (rows interleaved in blocks of 16).
    ``tiled`` marks a weight repacked by :func:`pack_skinny` for M <= 64 calls:
    ``w`` then holds 2 KB fragment tiles and ``nk`` the logical (N, K).
    ``rope`` = (heads_q, heads_kv, head_dim) marks a fused q|k|v weight whose
    rows were reordered by :func:`~instinctflash_amd.kernels.rope.permute_rope_rows`
    for :func:`~instinctflash_amd.kernels.rope.linear_qkv_rope` only.
    """

    w: torch.Tensor
    scale: torch.Tensor
    bias: torch.Tensor | None = None
    glu: bool = False
    tiled: bool = False
    nk: tuple | None = None
    rope: tuple | None = None

    @property
    def shape(self):
        return tuple(self.nk) if self.tiled else tuple(self.w.shape)


@dataclass
class TiledRows:
    """E4M3 activations [M, K] (M <= 64) in the skinny tile layout written by
    :func:`quant_rows_tiled`: ``q`` holds the tiles, ``M`` / ``K`` the logical
    shape. Accepted by :func:`linear` and :func:`gemm` wherever an [M, K] e4m3
    tensor is."""

    q: torch.Tensor
    M: int
    K: int

    @property
    def shape(self):
        return (self.M, self.K)

    @property
    def device(self):
        return self.q.device


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _on_device(name, t, device=None):
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a tensor on the gfx950 device, got {t.device}")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def _rows(name, t, dtype, device=None, cols=None):
    """2-D tensor with unit column stride (row stride free); returns (rows, cols, ld)."""
    _on_device(name, t, device)
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.shape[1] > 1 and t.stride(1) != 1:
        raise ValueError(f"{name} must have unit column stride")
    if cols is not None and t.shape[1] != cols:
        raise ValueError(f"{name} has {t.shape[1]} columns, expected {cols}")
    ld = t.stride(0) if t.shape[0] > 1 else max(t.shape[1], 1)
    return t.shape[0], t.shape[1], ld


def _vec(name, t, n, dtype=torch.float32, device=None):
    if t is None:
        return None
    _on_device(name, t, device)
    if t.dtype != dtype or t.numel() != n or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {dtype} vector of {n} elements")
    return t


def _qout(name, q, M, K, device):
    """E4M3 output operand [M, K]: a row-strided tensor, or a :class:`TiledRows`
    (the skinny tile layout, M <= 64). Returns (pointer, row stride) with the
    row stride IFX_LD_TILED (0) for the tile layout."""
    if isinstance(q, TiledRows):
        if (q.M, q.K) != (M, K) or q.q.dtype != E4M3 or q.device != device or \
                q.q.numel() != _lib.load().ifx_quant_rows_tiled_bytes(M, K):
            raise ValueError(f"{name} does not hold the tile layout of a [{M}, {K}] operand")
        return q.q.data_ptr(), _lib.LD_TILED
    rows, _, ld = _rows(name, q, E4M3, device, cols=K)
    if rows != M:
        raise ValueError(f"{name} must have {M} rows")
    return q.data_ptr(), ld


_WORKSPACES: dict = {}
_RETIRED: list = []


def _workspace(nbytes: int, device, stream: int):
    """Workspace per (device, stream), reused by every call on that stream
    (calls on one stream are ordered). It holds split-K partial sums, which
    every call writes before it reads them, so it needs no initialisation.

    A buffer outgrown by a later call is kept alive (never freed), because a
    captured HIP graph may still hold its address. Growing while the stream is
    being captured raises instead: run the captured calls once eagerly first,
    so the buffer is already large enough."""
    if nbytes == 0:
        return None
    key = (device.index, stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"the FP8 workspace of this stream must grow to {nbytes} bytes during HIP graph "
                               "capture; run the captured calls once before capturing")
        if ws is not None:
            _RETIRED.append(ws)
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


# ---------------------------------------------------------------------------
# quantizers
# ---------------------------------------------------------------------------

def quant_rows(x: torch.Tensor, q: torch.Tensor | None = None, scale: torch.Tensor | None = None):
    """Per-row dynamic E4M3 quantization (per token for activations).

    scale[m] = max(amax_m, 1e-12) * fl32(1/448); q = e4m3(clamp(x / scale, +-448)).
    Recipe of instinctflash/kernels/fp8.py:30-37 evaluated with device scalar
    semantics (instinctflash/runtime/fp8_pack.py:88-89). x: bf16 or fp32 [M, K].
    """
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"quant_rows expects bf16 or fp32 input, got {x.dtype}")
    M, K, ldx = _rows("x", x, x.dtype)
    if q is None:
        q = torch.empty((M, K), dtype=E4M3, device=x.device)
    if scale is None:
        scale = torch.empty((M,), dtype=torch.float32, device=x.device)
    _, _, ldq = _rows("q", q, E4M3, x.device, cols=K)
    if q.shape[0] != M:
        raise ValueError("q must have as many rows as x")
    _vec("scale", scale, M, device=x.device)
    if M and not K:
        raise ValueError("cannot quantize rows of width 0")
    dt = _lib.DTYPE_BF16 if x.dtype == torch.bfloat16 else _lib.DTYPE_F32
    _lib.check(_lib.load().ifx_quant_rows(_ptr(x), dt, ldx, M, K, _ptr(q), ldq, _ptr(scale),
                                          _stream(x.device)), "ifx_quant_rows")
    return q, scale


def quant_rows_tiled(x: torch.Tensor, q: TiledRows | None = None, scale: torch.Tensor | None = None):
    """``quant_rows`` for M <= 64 rows, writing the skinny tile layout that the
    M <= 64 GEMM reads with 1 KB contiguous loads: same bytes and scales, only
    placed differently. Returns (TiledRows, scale)."""
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"quant_rows_tiled expects bf16 or fp32 input, got {x.dtype}")
    M, K, ldx = _rows("x", x, x.dtype)
    if not 0 < M <= 64 or K % 16:
        raise ValueError("quant_rows_tiled needs 1 <= M <= 64 and K % 16 == 0")
    lib = _lib.load()
    nbytes = lib.ifx_quant_rows_tiled_bytes(M, K)
    if q is None:
        q = TiledRows(torch.empty(nbytes, dtype=E4M3, device=x.device), M, K)
    if (q.M, q.K) != (M, K) or q.q.numel() != nbytes or q.q.dtype != E4M3 or q.device != x.device:
        raise ValueError("q does not hold the tile layout of x's shape")
    if scale is None:
        scale = torch.empty((M,), dtype=torch.float32, device=x.device)
    _vec("scale", scale, M, device=x.device)
    dt = _lib.DTYPE_BF16 if x.dtype == torch.bfloat16 else _lib.DTYPE_F32
    _lib.check(lib.ifx_quant_rows_tiled(_ptr(x), dt, ldx, M, K, _ptr(q.q), _ptr(scale), _stream(x.device)),
               "ifx_quant_rows_tiled")
    return q, scale


def quantize_weight(w: torch.Tensor, bias: torch.Tensor | None = None, device=None) -> Fp8Weight:
    """Quantize ``w`` [N, K] per output channel on ``device`` (reference
    instinctflash/kernels/fp8.py:30-37). BF16 weights are read directly (the
    widening to FP32 is exact); other float dtypes are widened to FP32 first."""
    device = torch.device(device) if device is not None else w.device
    if w.dtype not in (torch.bfloat16, torch.float32):
        w = w.to(torch.float32)
    w = w.to(device=device).contiguous()
    q, scale = quant_rows(w)
    b = None if bias is None else bias.to(device=device, dtype=torch.float32).contiguous()
    return Fp8Weight(q, scale, b)


def quantize_tensor(x: torch.Tensor):
    """Per-tensor dynamic quantization of a contiguous bf16 tensor: one scale
    (shape [1]) for every element. Reference: instinctflash/runtime/fp8_pack.py:83-91."""
    _on_device("x", x)
    if x.dtype != torch.bfloat16 or not x.is_contiguous() or x.numel() == 0:
        raise ValueError("per-tensor FP8 packing requires nonempty contiguous bf16 input")
    lib = _lib.load()
    q = torch.empty_like(x, dtype=E4M3)
    scale = torch.empty((1,), dtype=torch.float32, device=x.device)
    nbytes = lib.ifx_quant_tensor_workspace_size(x.numel())
    part = torch.empty((nbytes,), dtype=torch.uint8, device=x.device)
    _lib.check(lib.ifx_quant_tensor_bf16(_ptr(x), x.numel(), _ptr(q), _ptr(scale), _ptr(part), nbytes,
                                         _stream(x.device)), "ifx_quant_tensor_bf16")
    return q, scale


def pack_tensor(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Pack a contiguous bf16 tensor with a fixed one-element FP32 device scale.
    Reference: instinctflash/runtime/fp8_pack.py:48-60 (pack_bf16_e4m3)."""
    _on_device("x", x)
    if x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("FP8 packing requires contiguous bf16 inputs")
    if scale.dtype != torch.float32 or scale.numel() != 1 or scale.device != x.device:
        raise ValueError("FP8 packing requires one FP32 scale on the input device")
    q = torch.empty_like(x, dtype=E4M3)
    _lib.check(_lib.load().ifx_pack_tensor_bf16(_ptr(x), x.numel(), _ptr(scale), _ptr(q), _stream(x.device)),
               "ifx_pack_tensor_bf16")
    return q


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------

def _epilogue(M, K, device, w: Fp8Weight, out, flags, residual, gate, use_scales):
    """Validates the weight, output and epilogue operands of a projection of M
    rows; returns (flags, N, ldw, sw, bias, ldr, ldo)."""
    if w.tiled:
        N, Kw = w.nk
        _on_device("w.w", w.w, device)
        if w.w.dtype != E4M3 or not w.w.is_contiguous() or w.w.numel() != _lib.load().ifx_fp8_skinny_tiled_bytes(N, Kw):
            raise ValueError("w.w is not a pack_skinny tile array for the recorded (N, K)")
        if M > 64:
            raise ValueError("a pack_skinny weight serves M <= 64 only")
        ldw = 0
        flags |= _lib.EPI_W_TILED
    else:
        N, Kw, ldw = _rows("w.w", w.w, E4M3, device)
    if Kw != K:
        raise ValueError(f"the activations have K={K} but the weight has K={Kw}")
    glu = bool(flags & (_lib.EPI_GEGLU | _lib.EPI_SWIGLU))
    if glu and not w.glu:
        raise ValueError("GeGLU/SwiGLU epilogues need a weight repacked with pack_glu()")
    if not glu and w.glu:
        raise ValueError("this weight is GLU-interleaved; use a GeGLU/SwiGLU epilogue")
    if N % 16 or K % 16 or (glu and N % 32):
        raise ValueError(f"FP8 GEMM needs N % {32 if glu else 16} == 0 and K % 16 == 0, got N={N}, K={K}")
    n_out = N // 2 if glu else N
    if out.dtype == torch.float32:
        flags |= _lib.EPI_OUT_F32
    elif out.dtype == torch.float16:
        flags |= _lib.EPI_OUT_F16
    elif out.dtype != torch.bfloat16:
        raise ValueError(f"out must be bf16, fp16 or fp32, got {out.dtype}")
    Mo, _, ldo = _rows("out", out, out.dtype, device, cols=n_out)
    if Mo != M:
        raise ValueError(f"out has {Mo} rows, expected {M}")
    sw = None
    if use_scales:
        # per-channel [N] scales or one shared value (per-tensor recipe,
        # reference runtime/torch_fp8_linear.py:75-78)
        if w.scale.numel() == 1 and N != 1:
            sw = _vec("w.scale", w.scale, 1, device=device)
            flags |= _lib.EPI_SCALAR_SW
        else:
            sw = _vec("w.scale", w.scale, N, device=device)
    bias = None
    if use_scales and w.bias is not None:
        bias = _vec("w.bias", w.bias, N, device=device)
        flags |= _lib.EPI_BIAS
    ldr = 0
    if residual is not None:
        if residual.dtype == torch.float32:
            flags |= _lib.EPI_RES_F32
        elif residual.dtype != torch.bfloat16:
            raise ValueError("residual must be bf16 or fp32")
        Mr, _, ldr = _rows("residual", residual, residual.dtype, device, cols=n_out)
        if Mr != M:
            raise ValueError("residual must have M rows")
        flags |= _lib.EPI_RESIDUAL
    if gate is not None:
        _vec("gate", gate, n_out, dtype=torch.bfloat16, device=device)
        flags |= _lib.EPI_GATE
    if M:
        for name, t in (("w.w", w.w), ("out", out)):
            if t.data_ptr() % 16:
                raise ValueError(f"{name} must be 16-byte aligned")
        if (not w.tiled and ldw % 16) or ldo % 8 or (residual is not None and (ldr % 8 or residual.data_ptr() % 16)):
            raise ValueError("row strides must be multiples of 16 bytes (w) and 8 elements (out, residual)")
    return flags, N, ldw, sw, bias, ldr, ldo


def _linear(a, sa, w: Fp8Weight, out, flags, residual=None, gate=None, use_scales=True):
    if w.rope is not None:
        raise ValueError("this weight's rows are reordered for linear_qkv_rope; use that call")
    if isinstance(a, TiledRows):
        M, K, lda = a.M, a.K, 0
        _on_device("a", a.q)
        flags |= _lib.EPI_A_TILED
        a_t = a.q
    else:
        M, K, lda = _rows("a", a, E4M3)
        a_t = a
    flags, N, ldw, sw, bias, ldr, ldo = _epilogue(M, K, a.device, w, out, flags, residual, gate, use_scales)
    if use_scales:
        # per-token [M] scales or one shared value
        if sa is not None and sa.numel() == 1 and M != 1:
            _vec("a_scale", sa, 1, device=a.device)
            flags |= _lib.EPI_SCALAR_SA
        else:
            _vec("a_scale", sa, M, device=a.device)
    if M == 0:
        return out
    if a_t.data_ptr() % 16 or lda % 16:
        raise ValueError("a must be 16-byte aligned with a row stride that is a multiple of 16 bytes")
    lib = _lib.load()
    stream = _stream(a.device)
    nbytes = lib.ifx_fp8_linear_workspace_size(M, N, K, flags)
    ws = _workspace(nbytes, a.device, stream)
    _lib.check(lib.ifx_fp8_linear(_ptr(a_t), lda, _ptr(sa) if use_scales else None, _ptr(w.w), ldw,
                                  _ptr(sw), _ptr(bias), _ptr(residual), ldr, _ptr(gate), flags,
                                  _ptr(out), ldo, M, N, K, _ptr(ws), nbytes, stream), "ifx_fp8_linear")
    return out


def gemm(a: torch.Tensor, w: Fp8Weight, out: torch.Tensor) -> torch.Tensor:
    """out[M, N] = a[M, K] (E4M3) @ w.w[N, K]^T with fp32 accumulation, unscaled.

    Reference: instinctflash/kernels/fp8.py:50-53 (torch._scaled_mm with unit
    scales); ``out`` is bf16 (or fp32) and may be a row-strided view."""
    if w.glu:
        raise ValueError("gemm() writes the raw accumulator of an unpacked weight")
    return _linear(a, None, w, out, 0, use_scales=False)


def linear(a: torch.Tensor, a_scale: torch.Tensor, w: Fp8Weight, out: torch.Tensor | None = None, *,
           act: str | None = None, residual: torch.Tensor | None = None,
           gate: torch.Tensor | None = None, out_dtype=torch.bfloat16) -> torch.Tensor:
    """Fused FP8 projection: out = epilogue(a @ w.w^T * a_scale[m] * w.scale[n]).

    ``a_scale`` is [M] (per token) or [1] (per tensor); ``w.scale`` is [N]
    (per channel) or [1] (per tensor).

    Epilogue order: + w.bias; act (``gelu_tanh``, or ``geglu``/``swiglu`` on a
    :func:`pack_glu` weight, halving the width); * gate[n] (adaLN gate); +
    residual[m, n]. ``out`` may alias ``residual`` for an in-place update.
    Replaces the reference's gemm + consumer pairs (kernels/norm.py:45-58,
    :135-144, :161-175; kernels/activation.py:26-40)."""
    if act not in ACTIVATIONS:
        raise ValueError(f"unknown activation {act!r}; expected one of {sorted(k for k in ACTIVATIONS if k)}")
    flags = ACTIVATIONS[act]
    if out is None:
        n_out = w.shape[0] // 2 if flags & (_lib.EPI_GEGLU | _lib.EPI_SWIGLU) else w.shape[0]
        out = torch.empty((a.shape[0], n_out), dtype=out_dtype, device=a.device)
    return _linear(a, a_scale, w, out, flags, residual=residual, gate=gate)


def quant_linear(x: torch.Tensor, w: Fp8Weight, out: torch.Tensor | None = None, *,
                 act: str | None = None, residual: torch.Tensor | None = None,
                 gate: torch.Tensor | None = None, out_dtype=torch.bfloat16, per_tensor: bool = False,
                 a_scale: torch.Tensor | None = None) -> torch.Tensor:
    """Quantize bf16 activations ``x`` [M, K] to E4M3 (per token, or per tensor
    with ``per_tensor=True``) and project: the result equals
    ``linear(*quant_rows(x), w, ...)`` (or with ``quantize_tensor``'s scale) bit
    for bit; the E4M3 copy lives in the per-stream workspace. ``a_scale`` ([M],
    or [1] per tensor), if given, receives the scales.
    Replaces the reference's producer-quant + gemm pairs and the body of
    ThorFP8Linear.forward (runtime/torch_fp8_linear.py:66-78)."""
    if act not in ACTIVATIONS:
        raise ValueError(f"unknown activation {act!r}; expected one of {sorted(k for k in ACTIVATIONS if k)}")
    M, K, ldx = _rows("x", x, torch.bfloat16)
    flags = ACTIVATIONS[act]
    if out is None:
        n_out = w.shape[0] // 2 if flags & (_lib.EPI_GEGLU | _lib.EPI_SWIGLU) else w.shape[0]
        out = torch.empty((M, n_out), dtype=out_dtype, device=x.device)
    flags, N, ldw, sw, bias, ldr, ldo = _epilogue(M, K, x.device, w, out, flags, residual, gate, True)
    mode = _lib.SCALE_TENSOR if per_tensor else _lib.SCALE_ROW
    if a_scale is not None:
        _vec("a_scale", a_scale, 1 if per_tensor else M, device=x.device)
    if M == 0:
        return out
    if x.data_ptr() % 16 or ldx % 8:
        raise ValueError("x must be 16-byte aligned with a row stride that is a multiple of 8 elements")
    if per_tensor and ldx != K:
        raise ValueError("per-tensor quantization needs contiguous rows")
    lib = _lib.load()
    stream = _stream(x.device)
    nbytes = lib.ifx_quant_linear_workspace_size(M, N, K, flags, mode)
    ws = _workspace(nbytes, x.device, stream)
    _lib.check(lib.ifx_quant_linear(_ptr(x), ldx, mode, _ptr(w.w), ldw, _ptr(sw), _ptr(bias), _ptr(residual), ldr,
                                    _ptr(gate), flags, _ptr(out), ldo, M, N, K, _ptr(a_scale), _ptr(ws), nbytes,
                                    stream), "ifx_quant_linear")
    return out


def pack_glu(w: Fp8Weight) -> Fp8Weight:
    """Repack a gate|up weight (rows [0,F) gate, [F,2F) up, as the reference
    stores it for kernels/activation.py:24-25) into the 16-row interleaved layout
    of the fused GLU epilogue. Output width of the projection is F."""
    if w.glu:
        return w
    if w.tiled:
        raise ValueError("pack_glu must come before pack_skinny")
    N, K, ldw = _rows("w.w", w.w, E4M3)
    if N % 32 or ldw != K:
        raise ValueError("pack_glu needs a contiguous [2F, K] weight with F % 16 == 0")
    _vec("w.scale", w.scale, N, device=w.w.device)
    if w.bias is not None:
        _vec("w.bias", w.bias, N, device=w.w.device)
    wo = torch.empty_like(w.w)
    so = torch.empty_like(w.scale)
    bo = None if w.bias is None else torch.empty_like(w.bias)
    _lib.check(_lib.load().ifx_fp8_pack_glu(_ptr(w.w), _ptr(w.scale), _ptr(w.bias), N // 2, K, _ptr(wo),
                                            _ptr(so), _ptr(bo), _stream(w.w.device)), "ifx_fp8_pack_glu")
    return Fp8Weight(wo, so, bo, glu=True)


def pack_skinny(w: Fp8Weight) -> Fp8Weight:
    """Repack a weight for M <= 64 projections (decode / action-head shapes): each
    16-row block and 128-byte K step becomes one contiguous 2 KB tile in the order
    the matrix-core fragments are loaded, so every load instruction of the skinny
    GEMM reads 1 KB of contiguous memory. Scales, bias and the GLU flag carry
    over; apply after :func:`pack_glu`. Such a weight is rejected for M > 64."""
    if w.tiled:
        return w
    N, K, ldw = _rows("w.w", w.w, E4M3)
    if N % 16 or K % 16:
        raise ValueError("pack_skinny needs N % 16 == 0 and K % 16 == 0")
    if w.w.data_ptr() % 16 or ldw % 16:
        raise ValueError("w.w must be 16-byte aligned with a 16-byte multiple row stride")
    lib = _lib.load()
    out = torch.empty(lib.ifx_fp8_skinny_tiled_bytes(N, K), dtype=E4M3, device=w.w.device)
    _lib.check(lib.ifx_fp8_pack_skinny(_ptr(w.w), ldw, N, K, _ptr(out), _stream(w.w.device)), "ifx_fp8_pack_skinny")
    return Fp8Weight(out, w.scale, w.bias, glu=w.glu, tiled=True, nk=(N, K), rope=w.rope)

"""QKV split consumer of the fused QKV projection, on HIP (gfx950).

Mirrors the reference module instinctflash/kernels/rope.py: ``rope_inv_freq``
and ``qkv_split`` keep their signatures, so an engine's call sites run
unchanged. The kernel rescales the raw accumulator, applies the optional
per-head q/k RMSNorm and the rotary embedding (split-half pairing, FP32 angles,
M-RoPE sections), and writes Q and the K/V cache rows at ``kv_base + t``.
``linear_qkv_rope`` does the same work (without the per-head norms and
sections) inside the skinny FP8 GEMM's epilogue, for weights reordered by
``permute_rope_rows``.
"""
from __future__ import annotations

import torch

from .. import _lib
from .fp8 import _ptr, _rows, _stream, _vec

_OUT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16, torch.float32: _lib.DTYPE_F32}


def rope_inv_freq(head_dim, theta, device):
    """1 / theta^(2i / head_dim), i < head_dim / 2, in float32 (reference rope.py:83-85)."""
    exponent = torch.arange(0, head_dim, 2, dtype=torch.int64, device=device).float() / head_dim
    return (1.0 / (theta ** exponent)).float()


def _heads(name, t, rows, heads, head_dim, device):
    if t.device != device or t.dim() != 3 or t.shape[1:] != (heads, head_dim) or t.stride(2) != 1:
        raise ValueError(f"{name} must be a [rows, {heads}, {head_dim}] tensor with unit last stride on {device}")
    if t.shape[0] < rows:
        raise ValueError(f"{name} has {t.shape[0]} rows, {rows} needed")
    return t.stride(0), t.stride(1)


def qkv_split(qkv, q_out, k_out, v_out, *, heads_q, heads_kv, head_dim, row=None, col=None, bias=None,
              inv_freq=None, pos=None, sections=None, q_norm=None, k_norm=None, norm_eps=1e-6, kv_base=0):
    """q_out [T, HQ, HD]; k_out / v_out [S, HKV, HD] written at rows ``kv_base + t``.

    Reference: instinctflash/kernels/rope.py:89-116. ``qkv`` is the raw (bf16,
    or fp32) accumulator [T, (HQ + 2*HKV) * HD]; ``row`` [T] / ``col`` / ``bias``
    are its dequantization scales and bias; rotary is applied when ``inv_freq``
    is given, with ``pos`` a float32 [T, S] position table and ``sections`` an
    int32 [HD/2] column map; ``kv_base`` is an int or a one-element int32
    device tensor (read on the device, so a captured graph follows it)."""
    if q_out.dtype != k_out.dtype or k_out.dtype != v_out.dtype:
        raise ValueError("q/k/v outputs must share a dtype")
    if q_out.dtype not in _OUT:
        raise ValueError("q/k/v outputs must be bf16, fp16 or fp32")
    if inv_freq is not None and pos is None:
        raise ValueError("rotary needs a position table")
    if (q_norm is None) != (k_norm is None):
        raise ValueError("q_norm and k_norm come together")
    if qkv.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("qkv must be bf16 or fp32")
    HQ, HKV, HD = int(heads_q), int(heads_kv), int(head_dim)
    T, C, ldqkv = _rows("qkv", qkv, qkv.dtype)
    dev = qkv.device
    if C != (HQ + 2 * HKV) * HD:
        raise ValueError(f"qkv has {C} columns, expected (heads_q + 2 * heads_kv) * head_dim = {(HQ + 2 * HKV) * HD}")
    dynamic = torch.is_tensor(kv_base)
    if dynamic:
        if kv_base.device != dev or kv_base.dtype != torch.int32 or kv_base.numel() != 1:
            raise ValueError("a device kv_base must be a one-element int32 tensor on the qkv device")
        base_rows = 0
    else:
        base_rows = int(kv_base)
        if base_rows < 0:
            raise ValueError("kv_base must be >= 0")
    sq = _heads("q_out", q_out, T, HQ, HD, dev)
    sk = _heads("k_out", k_out, base_rows + T, HKV, HD, dev)
    sv = _heads("v_out", v_out, base_rows + T, HKV, HD, dev)
    _vec("row", row, T, device=dev)
    _vec("col", col, C, device=dev)
    _vec("bias", bias, C, device=dev)
    _vec("q_norm", q_norm, HD, device=dev)
    _vec("k_norm", k_norm, HD, device=dev)
    ldpos = 0
    if inv_freq is not None:
        _vec("inv_freq", inv_freq, HD // 2, device=dev)
        if pos.dtype != torch.float32 or pos.device != dev or pos.dim() != 2 or pos.shape[0] < T or \
                (pos.shape[1] > 1 and pos.stride(1) != 1):
            raise ValueError("pos must be a float32 [T, S] device table with unit column stride")
        ldpos = pos.stride(0) if pos.shape[0] > 1 else pos.shape[1]
        if sections is not None:
            _vec("sections", sections, HD // 2, dtype=torch.int32, device=dev)
    _lib.check(_lib.load().ifx_qkv_split(
        _ptr(qkv), _lib.DTYPE_F32 if qkv.dtype == torch.float32 else _lib.DTYPE_BF16, ldqkv, _ptr(row), _ptr(col),
        _ptr(bias), _ptr(q_norm), _ptr(k_norm), float(norm_eps), _ptr(inv_freq),
        _ptr(pos) if inv_freq is not None else None, ldpos, _ptr(sections) if inv_freq is not None else None,
        _ptr(q_out), sq[0], sq[1], _ptr(k_out), sk[0], sk[1], _ptr(v_out), sv[0], sv[1], _OUT[q_out.dtype],
        base_rows, _ptr(kv_base) if dynamic else None, T, HQ, HKV, HD, _stream(dev)), "ifx_qkv_split")


def _rope_row_order(head_dim: int) -> list:
    """Packed row i of a head -> head dim: rows 16k + 4g + (0, 1, 2, 3) hold dims
    d, d + 1, d + HD/2, d + 1 + HD/2 with d = 8k + 2g, so each lane of the
    skinny GEMM's output fragment owns two complete rotary pairs."""
    half = head_dim // 2
    order = []
    for i in range(head_dim):
        d = 8 * (i // 16) + 2 * ((i % 16) // 4)
        r = i % 4
        order.append(d + (r & 1) + (half if r >= 2 else 0))
    return order


def permute_rope_rows(w, heads_q: int, heads_kv: int, head_dim: int):
    """Reorder the rows of a fused q|k|v weight [(HQ + 2*HKV) * HD, K] (with its
    scales and bias) into the order :func:`linear_qkv_rope` reads; apply before
    :func:`~instinctflash_amd.kernels.fp8.pack_skinny`. The result is accepted
    by :func:`linear_qkv_rope` only."""
    from .fp8 import Fp8Weight
    HQ, HKV, HD = int(heads_q), int(heads_kv), int(head_dim)
    if w.tiled or w.glu or w.rope is not None:
        raise ValueError("permute_rope_rows takes a plain (not packed) weight")
    N = w.w.shape[0]
    if HQ < 1 or HKV < 1 or HD % 16 or HD > 256 or N != (HQ + 2 * HKV) * HD:
        raise ValueError(f"need N = (heads_q + 2 * heads_kv) * head_dim with head_dim % 16 == 0 and <= 256, got N={N}")
    order = _rope_row_order(HD)
    idx = torch.tensor([h * HD + o for h in range(HQ + 2 * HKV) for o in order], dtype=torch.int64,
                       device=w.w.device)

    def take(t):
        return None if t is None else (t if t.numel() == 1 else t.index_select(0, idx).contiguous())
    return Fp8Weight(w.w.index_select(0, idx).contiguous(), take(w.scale), take(w.bias), rope=(HQ, HKV, HD))


def linear_qkv_rope(a, a_scale, w, q_out, k_out, v_out, *, inv_freq=None, pos=None, kv_base=0):
    """FP8 QKV projection with ``qkv_split``'s work in the GEMM's epilogue: for a
    weight from :func:`permute_rope_rows` (optionally :func:`pack_skinny`-ed) and
    M <= 64 tokens, y = a @ w^T * a_scale[m] * w.scale (+ bias) in fp32, the
    rotary pairs (i, i + HD/2) of Q and K heads (angle pos[t] * inv_freq[i]),
    then Q into q_out [T, HQ, HD] and K / V into k_out / v_out [S, HKV, HD] at
    rows ``kv_base + t``. Replaces ``gemm`` + ``qkv_split`` (reference
    kernels/fp8.py:50-53, kernels/rope.py:89-116) without the bf16 round trip of
    the raw accumulator; no per-head norms, no position sections."""
    from .fp8 import TiledRows, E4M3, _workspace
    if w.rope is None:
        raise ValueError("linear_qkv_rope needs a weight from permute_rope_rows")
    HQ, HKV, HD = w.rope
    if q_out.dtype != k_out.dtype or k_out.dtype != v_out.dtype or q_out.dtype not in _OUT:
        raise ValueError("q/k/v outputs must share a dtype: bf16, fp16 or fp32")
    if inv_freq is not None and pos is None:
        raise ValueError("rotary needs a position table")
    flags = 0
    if isinstance(a, TiledRows):
        M, K, lda, a_t = a.M, a.K, 0, a.q
        flags |= _lib.EPI_A_TILED
    else:
        M, K, lda = _rows("a", a, E4M3)
        a_t = a
    dev = a_t.device
    if M > 64:
        raise ValueError("linear_qkv_rope serves M <= 64")
    if w.tiled:
        N, Kw = w.nk
        ldw = 0
        flags |= _lib.EPI_W_TILED
    else:
        N, Kw, ldw = _rows("w.w", w.w, E4M3, dev)
    if Kw != K or N != (HQ + 2 * HKV) * HD:
        raise ValueError("weight and activation shapes disagree")
    _vec("a_scale", a_scale, M, device=dev)
    _vec("w.scale", w.scale, N, device=dev)
    if w.bias is not None:
        _vec("w.bias", w.bias, N, device=dev)
        flags |= _lib.EPI_BIAS
    dynamic = torch.is_tensor(kv_base)
    if dynamic:
        if kv_base.device != dev or kv_base.dtype != torch.int32 or kv_base.numel() != 1:
            raise ValueError("a device kv_base must be a one-element int32 tensor on the activation device")
        base_rows = 0
    else:
        base_rows = int(kv_base)
        if base_rows < 0:
            raise ValueError("kv_base must be >= 0")
    sq = _heads("q_out", q_out, M, HQ, HD, dev)
    sk = _heads("k_out", k_out, base_rows + M, HKV, HD, dev)
    sv = _heads("v_out", v_out, base_rows + M, HKV, HD, dev)
    ldpos = 0
    if inv_freq is not None:
        _vec("inv_freq", inv_freq, HD // 2, device=dev)
        if pos.dtype != torch.float32 or pos.device != dev or pos.dim() != 2 or pos.shape[0] < M:
            raise ValueError("pos must be a float32 [T, S] device table (column 0 is used)")
        ldpos = pos.stride(0) if pos.shape[0] > 1 else max(1, pos.shape[1])
    if M == 0:
        return q_out
    lib = _lib.load()
    stream = _stream(dev)
    nbytes = lib.ifx_fp8_linear_workspace_size(M, N, K, 0)
    ws = _workspace(nbytes, dev, stream)
    _lib.check(lib.ifx_fp8_linear_qkv_rope(
        _ptr(a_t), lda, _ptr(a_scale), _ptr(w.w), ldw, _ptr(w.scale), _ptr(w.bias), flags,
        _ptr(pos) if inv_freq is not None else None, ldpos, _ptr(inv_freq), HQ, HKV, HD,
        _ptr(q_out), sq[0], sq[1], _ptr(k_out), sk[0], sk[1], _ptr(v_out), sv[0], sv[1], _OUT[q_out.dtype],
        base_rows, _ptr(kv_base) if dynamic else None, M, K, _ptr(ws), nbytes, stream), "ifx_fp8_linear_qkv_rope")
    return q_out

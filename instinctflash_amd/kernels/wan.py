"""Wan DiT QKV consumer on HIP (gfx950).

Mirrors the reference module instinctflash/kernels/wan.py: ``wan_qkv`` keeps its
signature. For each row of the raw fused projection accumulator ``[Q | K | V]``
(each ``heads * head_dim`` wide) it applies the row/column dequantization and
bias, RMS-normalizes Q and K over their full width, rotates adjacent channel
pairs (2j, 2j+1) of every head by ``pos[t, sections[j]] * inv_freq[j]`` (FP32
angles, accurate cos/sin), and stores Q densely and K/V into per-batch pool rows
``slots[t]`` (t = row % tokens).
"""
from __future__ import annotations

import torch

from .. import _lib
from .fp8 import _ptr, _rows, _stream, _vec
from .rope import _OUT


def wan_qkv(raw, q_out, *, heads, head_dim, tokens, k_pool=None, v_pool=None, slots=None, row=None, col=None,
            bias=None, q_norm=None, k_norm=None, pos=None, sections=None, inv_freq=None, eps=1e-6, num_warps=8):
    """raw [B*T, parts*H*HD] (parts: Q, then K, then V); q_out [B*T, H*HD];
    k_pool / v_pool [B, S, H*HD] written at rows ``slots[t]`` (or ``t``).

    Reference: instinctflash/kernels/wan.py:84-116. ``num_warps`` is accepted for
    signature compatibility. As in the reference launch, the second part is
    always K, so a ``v_pool`` without a ``k_pool`` is not written."""
    if raw.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("raw must be bf16 or fp32")
    if q_out.dtype not in _OUT:
        raise ValueError("q_out must be bf16, fp16 or fp32")
    H, HD, T = int(heads), int(head_dim), int(tokens)
    D = H * HD
    rows, C, ldraw = _rows("raw", raw, raw.dtype)
    dev = raw.device
    parts = 1 + (k_pool is not None) + (v_pool is not None)
    if C < parts * D:
        raise ValueError(f"raw has {C} columns, {parts} parts of {D} needed")
    if T <= 0 or rows % T:
        raise ValueError("rows must be a whole number of batches of `tokens` rows")
    Mq, _, sq = _rows("q_out", q_out, q_out.dtype, dev, cols=D)
    if Mq != rows:
        raise ValueError("q_out must have as many rows as raw")
    B = rows // T
    pool_strides = []
    for name, p in (("k_pool", k_pool), ("v_pool", v_pool)):
        if p is None:
            pool_strides.append((0, 0))
            continue
        if p.dtype != q_out.dtype or p.device != dev or p.dim() != 3 or p.shape[0] < B or p.shape[2] != D or \
                p.stride(2) != 1:
            raise ValueError(f"{name} must be a [B, S, {D}] tensor of q_out's dtype with unit last stride")
        pool_strides.append((p.stride(0), p.stride(1)))
    if slots is not None:
        _vec("slots", slots, slots.numel(), dtype=torch.int32, device=dev)
        if slots.numel() < T:
            raise ValueError("slots needs one entry per token")
    _vec("row", row, rows, device=dev)
    for name, t in (("col", col), ("bias", bias)):
        if t is not None:
            _vec(name, t, t.numel(), device=dev)
            if t.numel() < parts * D:
                raise ValueError(f"{name} must cover the {parts} parts")
    _vec("q_norm", q_norm, D, device=dev)
    _vec("k_norm", k_norm, D, device=dev)
    ldpos = 0
    if inv_freq is not None:
        if pos is None:
            raise ValueError("rotary needs a position table")
        _vec("inv_freq", inv_freq, HD // 2, device=dev)
        if pos.dtype != torch.float32 or pos.device != dev or pos.dim() != 2 or pos.shape[0] < T or \
                (pos.shape[1] > 1 and pos.stride(1) != 1):
            raise ValueError("pos must be a float32 [T, S] device table with unit column stride")
        ldpos = pos.stride(0) if pos.shape[0] > 1 else pos.shape[1]
        if sections is not None:
            _vec("sections", sections, HD // 2, dtype=torch.int32, device=dev)
    (sk_b, sk_s), (sv_b, sv_s) = pool_strides
    _lib.check(_lib.load().ifx_wan_qkv(
        _ptr(raw), _lib.DTYPE_F32 if raw.dtype == torch.float32 else _lib.DTYPE_BF16, ldraw, _ptr(row), _ptr(col),
        _ptr(bias), _ptr(q_norm), _ptr(k_norm), float(eps), _ptr(inv_freq), _ptr(pos) if inv_freq is not None else None,
        ldpos, _ptr(sections) if inv_freq is not None else None, _ptr(q_out), sq, _ptr(k_pool), sk_b, sk_s,
        _ptr(v_pool), sv_b, sv_s, _ptr(slots), _OUT[q_out.dtype], rows, T, H, HD, _stream(dev)), "ifx_wan_qkv")


def wan_rope_tables(head_dim=128, theta=10000.0, device=None):
    """3-D rotary frequency tables for ``wan_qkv`` (reference
    engines/wan_va/weights.py:76-84): the head's channel pairs split into frame /
    height / width sections of HD - 2 (HD // 3), HD // 3 and HD // 3 channels,
    each with its own ladder theta^(-2i / d). Returns (inv_freq float32 [HD / 2],
    sections int32 [HD / 2], 0 = frame, 1 = height, 2 = width)."""
    hw = head_dim // 3
    dims = (head_dim - 2 * hw, hw, hw)
    freqs, secs = [], []
    for s, d in enumerate(dims):
        i = torch.arange(d // 2, dtype=torch.float64)
        freqs.append(theta ** (-2.0 * i / d))
        secs.append(torch.full((d // 2,), s, dtype=torch.int32))
    return torch.cat(freqs).float().to(device), torch.cat(secs).to(device)

"""Attention for short robotics sequences, with split-KV and a fused FP8
output row, on HIP (gfx950).

Mirrors instinctflash/kernels/attention.py: ``attention`` and ``SplitWorkspace``
keep their signatures, so an engine's call sites run unchanged. Grouped-query
heads fold into query rows; query token t sees keys [0, limit_t) with
limit_t = kv_len (+ kv_extra[t]) (min causal_offset + t + 1); ``kv_len`` may be
a one-element int32 device tensor read at execution time (captured graphs follow
it); ``kv_index`` maps key n to cache row kv_index[n]. With ``split`` the keys
of each row block are spread over several workgroups and merged by a second
kernel, which can also emit every token's full output row as per-token E4M3
(``q8``, ``q8_scale``) -- the A operand of the output projection.
"""
from __future__ import annotations

import ctypes

import torch

from .. import _lib
from .fp8 import _on_device, _ptr, _qout, _stream, _vec

_DT = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16}


class SplitWorkspace:
    """Partial-softmax storage for split-KV attention of one geometry
    (reference attention.py:150-159). No initialization is needed."""

    def __init__(self, batch, tq, hq, hkv, head_dim, splits, device):
        self.splits = int(splits)
        if self.splits < 2:
            raise ValueError("a split workspace needs splits >= 2")
        nbytes = _lib.load().ifx_attention_workspace_size(batch, tq, hq, hkv, head_dim, self.splits)
        if nbytes == 0:
            raise ValueError("unsupported split-attention geometry")
        self.geometry = (int(batch), int(tq), int(hq), int(hkv), int(head_dim))
        self.buf = torch.empty(nbytes, dtype=torch.uint8, device=device)


_AUTO_SPLIT: dict = {}


def split_count(B, Tq, Hq, Hkv, Tk) -> int:
    """Key ranges for a launch with few query-row blocks (workgroups of 128 query
    rows): about 256 workgroups in total, at least 64 keys per range, 2..16
    ranges (measured on MI355X: the 51-token pi05 chunk over 882 keys runs best
    at 14, the 800-token prefix at 4-6). 1 when the row blocks alone fill the GPU."""
    blocks = -(-(Tq * (Hq // Hkv)) // 128) * Hkv * B
    if blocks >= 128 or Tk < 128:
        return 1
    return int(max(2, min(16, -(-Tk // 64), round(256 / blocks))))


def _auto_split(B, Tq, Hq, Hkv, D, Tk, device):
    """Split workspace for launches with too few row blocks to fill the GPU
    (:func:`split_count`), allocated once per geometry and device and then
    reused (calls on one device are stream-ordered by the caller)."""
    splits = split_count(B, Tq, Hq, Hkv, Tk)
    if splits < 2 or Hq * splits > 1024:
        return None
    key = (device, B, Tq, Hq, Hkv, D, splits)
    ws = _AUTO_SPLIT.get(key)
    if ws is None:
        ws = _AUTO_SPLIT[key] = SplitWorkspace(B, Tq, Hq, Hkv, D, splits, device)
    return ws


def config_for(head_dim: int, group: int, rows: int):
    """Launch choice of the reference's Triton kernel; the HIP kernel has one
    configuration, so this only keeps the import surface (attention.py:103-106)."""
    return (128, 64, 4, 1)


def _strides(name, t, dev):
    _on_device(name, t, dev)
    if t.dim() != 4 or t.stride(3) != 1:
        raise ValueError(f"{name} must be 4-D with a contiguous last dimension")
    return (ctypes.c_int64 * 3)(t.stride(0), t.stride(1), t.stride(2))


def attention(q, k, v, out=None, *, scale=None, kv_len=None, kv_extra=None, max_extra=0, causal=False,
              causal_offset=0, config=None, tc5=False, split=None, q8=None, q8_scale=None, kv_index=None):
    """Attention of q [B, Tq, Hq, D] over k / v [B, Tk, Hkv, D] (bf16 or fp16).

    Reference: instinctflash/kernels/attention.py:162-213 (same keywords;
    ``config`` and ``tc5`` select Triton launch shapes there and are accepted
    and ignored here; ``max_extra`` only bounds ``kv_extra``). Returns ``out``
    (allocated like q when omitted, unless a split launch writes only q8).
    Without ``split``, a launch with too few query-row blocks to fill the GPU
    splits its keys anyway, through a workspace this module allocates once
    per geometry."""
    if q.dtype not in _DT or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must share a dtype, bf16 or fp16")
    dev = q.device
    B, Tq, Hq, D = q.shape
    if k.dim() != 4 or v.shape != k.shape or k.shape[0] != B or k.shape[3] != D:
        raise ValueError("k and v must be [B, Tk, Hkv, D] matching q")
    Tk, Hkv = k.shape[1], k.shape[2]
    if Hq % Hkv:
        raise ValueError("query heads must be a multiple of KV heads")
    if out is None and (split is None or q8 is None):
        out = torch.empty_like(q)
    if out is not None and (out.dtype != q.dtype or out.shape != q.shape):
        raise ValueError("out must match q in shape and dtype")
    qs, ks, vs = _strides("q", q, dev), _strides("k", k, dev), _strides("v", v, dev)
    os_ = _strides("out", out, dev) if out is not None else None
    if scale is None:
        scale = D ** -0.5
    dynamic = torch.is_tensor(kv_len)
    if dynamic:
        _vec("kv_len", kv_len, 1, dtype=torch.int32, device=dev)
    static_len = Tk if kv_len is None or dynamic else int(kv_len)
    if kv_index is not None:
        _on_device("kv_index", kv_index, dev)
        if kv_index.dtype != torch.int32 or kv_index.dim() != 1 or not kv_index.is_contiguous():
            raise ValueError("kv_index must be a contiguous int32 vector")
    _vec("kv_extra", kv_extra, Tq, dtype=torch.int32, device=dev)
    splits, ws, ws_bytes = 1, None, 0
    if split is None and q8 is None:
        split = _auto_split(B, Tq, Hq, Hkv, D, Tk, dev)
    if split is not None:
        if split.geometry != (B, Tq, Hq, Hkv, D):
            raise ValueError(f"split workspace geometry {split.geometry} does not match {(B, Tq, Hq, Hkv, D)}")
        splits, ws, ws_bytes = split.splits, split.buf, split.buf.numel()
    ldq8 = 0
    if q8 is not None:
        if split is None:
            raise ValueError("the fused FP8 output needs a split workspace")
        if B != 1:
            raise ValueError("fused FP8 output supports batch 1")
        q8p, ldq8 = _qout("q8", q8, Tq, Hq * D, dev)
        _vec("q8_scale", q8_scale, Tq, device=dev)
    _lib.check(_lib.load().ifx_attention(
        _ptr(q), _ptr(k), _ptr(v), _ptr(out), _DT[q.dtype], B, Tq, Hq, Tk, Hkv, D, qs, ks, vs, os_, static_len,
        _ptr(kv_len) if dynamic else None, _ptr(kv_extra), 1 if causal else 0, int(causal_offset), _ptr(kv_index),
        kv_index.numel() if kv_index is not None else 0, float(scale), splits, _ptr(ws), ws_bytes, q8p if q8 is not None else None, ldq8,
        _ptr(q8_scale), _stream(dev)), "ifx_attention")
    return out

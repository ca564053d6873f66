"""The transformer blocks of the LingBot-VA (Wan2.2-style) video/action model on
the gfx950 kernels: the call site that defines config C5 (Wan DiT block
projections, M = batch x tokens rows).

Mirrors the block loop of instinctflash/engines/wan_va/engine.py:205-245
(``_forward``) and the per-layer text K/V of :180-203 (``_prepare_text``):

  * LayerNorm + flow-time modulation (shift, scale rows picked per token through
    ``mod_index``) to per-token FP8 (``residual_norm_quant``);
  * per block: the fused q|k|v projection, ``wan_qkv`` (rescale, bias, full-width
    RMSNorm of Q and K, 3-D rotary, K/V into the self-attention pool at the
    tokens' slots), attention over the live pool slots (``kv_index``), the output
    projection and the gated residual update + affine ``norm2``; cross-attention
    (query projection + ``wan_qkv`` normalization, attention over the 512 text
    rows, output projection, residual + modulated LayerNorm); the GELU-tanh FFN
    and the gated residual + the next block's modulated LayerNorm (or the
    head's, written as float32 ``y`` after the last block).

The residual stream is bf16, as upstream rounds it after every add. The
modulation tables hold per timestep-entry rows [cap, 6, D] (shift, scale, gate,
c_shift, c_scale, c_gate) per block and [cap, 6, D] for the head (shift,
scale); ``mod_index`` holds 6 * entry for each row, so the row of component c
is ``table.view(-1, D)[mod_index + c]`` -- the reference's convention.

``reference_calls=True`` makes exactly the reference's calls. The default lays
the FFN out for gfx950: GELU in the ff1 projection's epilogue (bf16 result) and
``quant_rows`` of it, instead of the raw accumulator and ``row_quant(gelu=True)``.
Weights are random (no checkpoint here) with the published 5B shapes.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .kernels import E4M3, Fp8Weight, attention, gemm, linear, quant_rows, quantize_weight, \
    residual_norm_quant, row_quant, wan_qkv

#: Wan2.2 5B transformer: engines/wan_va/weights.py D, H, HD, FF; engine.py TEXT
WAN_D, WAN_H, WAN_HD, WAN_FF, WAN_TEXT = 3072, 24, 128, 14336, 512
EPS = 1e-6


def wan_rope_tables(head_dim=WAN_HD, theta=10000.0, device=None):
    """3-D rotary frequencies (engines/wan_va/weights.py:76-84): the head's
    channel pairs split into frame / height / width sections of
    HD - 2 (HD // 3), HD // 3 and HD // 3 channels; each section has its own
    frequency ladder theta^(-2i / d). Returns (inv_freq float32 [HD / 2],
    sections int32 [HD / 2] with 0 = frame, 1 = height, 2 = width)."""
    hw = head_dim // 3
    dims = (head_dim - 2 * hw, hw, hw)
    freqs, secs = [], []
    for s, d in enumerate(dims):
        i = torch.arange(d // 2, dtype=torch.float64)
        freqs.append(theta ** (-2.0 * i / d))
        secs.append(torch.full((d // 2,), s, dtype=torch.int32))
    return torch.cat(freqs).float().to(device), torch.cat(secs).to(device)


@dataclass
class WanBlockWeights:
    qkv: Fp8Weight       # [3D, D] + bias
    norm_q: torch.Tensor
    norm_k: torch.Tensor
    o: Fp8Weight
    norm2_w: torch.Tensor
    norm2_b: torch.Tensor
    cq: Fp8Weight
    cnorm_q: torch.Tensor
    ckv: Fp8Weight       # [2D, D] text K | V + bias
    cnorm_k: torch.Tensor
    co: Fp8Weight
    ff1: Fp8Weight       # [FF, D] + bias
    ff2: Fp8Weight       # [D, FF] + bias


def random_wan_blocks(n: int, device, seed=0, D=WAN_D, FF=WAN_FF) -> list:
    """Random blocks with the model's shapes: projections N(0, 0.02) and biases
    N(0, 0.01), quantized per output channel on the device; norm weights
    1 + N(0, 0.1), LayerNorm biases N(0, 0.05)."""
    g = torch.Generator().manual_seed(seed)
    dev = torch.device(device)

    def lin(nout, k):
        w = (torch.randn(nout, k, generator=g) * 0.02).to(torch.bfloat16)
        return quantize_weight(w.to(dev), (torch.randn(nout, generator=g) * 0.01).to(dev), dev)

    def vec(s=0.1, base=1.0):
        return (base + torch.randn(D, generator=g) * s).to(dev)

    return [WanBlockWeights(lin(3 * D, D), vec(), vec(), lin(D, D), vec(), vec(0.05, 0.0), lin(D, D), vec(),
                            lin(2 * D, D), vec(), lin(D, D), lin(FF, D), lin(D, FF)) for _ in range(n)]


class WanStack:
    """The block stack over ``B`` batches of ``T`` tokens (R = B T <= max_batch
    max_tokens rows). State: the bf16 residual stream ``x`` [R, D], the
    self-attention K/V pools ``kpool`` / ``vpool`` [layers, max_batch,
    pool_slots, D] (fp16), the text K/V ``tk`` / ``tv`` [layers, max_batch,
    text, D] (``prepare_text``), and the device tables the graph reads: token
    positions ``pos`` [T, 3] (frame, h, w), pool ``slots`` [T] of this forward's
    tokens, the ``live`` slots attention reads and their count ``n_live``, and
    ``mod_index`` [R]."""

    def __init__(self, blocks: list, device, *, pool_slots: int, max_tokens=512, max_batch=2, text=WAN_TEXT,
                 heads=WAN_H, head_dim=WAN_HD, reference_calls=False):
        self.blocks = blocks
        self.dev = torch.device(device)
        self.reference_calls = bool(reference_calls)
        self.H, self.HD = int(heads), int(head_dim)
        self.D = D = self.H * self.HD
        self.FF = FF = blocks[0].ff1.shape[0]
        self.S, self.TEXT = int(pool_slots), int(text)
        self.max_tokens, self.max_batch = int(max_tokens), int(max_batch)
        dev, f32, f16, bf16 = self.dev, torch.float32, torch.float16, torch.bfloat16
        L, B = len(blocks), self.max_batch
        R = B * self.max_tokens
        RT = max(R, B * self.TEXT)
        self.kpool = torch.zeros(L, B, self.S, D, dtype=f16, device=dev)
        self.vpool = torch.zeros_like(self.kpool)
        self.tk = torch.zeros(L, B, self.TEXT, D, dtype=f16, device=dev)
        self.tv = torch.zeros_like(self.tk)
        self.q8 = torch.zeros(RT * max(FF, D), dtype=E4M3, device=dev)
        self.raw = torch.zeros(RT * 3 * D, dtype=bf16, device=dev)
        self.raw_ff = torch.zeros(R * FF, dtype=bf16, device=dev)
        self.scale = [torch.zeros(RT, dtype=f32, device=dev) for _ in range(2)]
        self.x = torch.zeros(R, D, dtype=bf16, device=dev)
        self.y = torch.zeros(R, D, dtype=f32, device=dev)
        self.q16 = torch.zeros(RT, D, dtype=f16, device=dev)
        self.o16 = torch.zeros(R, D, dtype=f16, device=dev)
        self.pos = torch.zeros(self.max_tokens, 3, dtype=f32, device=dev)
        self.slots = torch.zeros(self.max_tokens, dtype=torch.int32, device=dev)
        self.live = torch.zeros(self.S, dtype=torch.int32, device=dev)
        self.n_live = torch.zeros(1, dtype=torch.int32, device=dev)
        self.mod_index = torch.zeros(R, dtype=torch.int32, device=dev)
        self.inv_freq, self.sections = wan_rope_tables(self.HD, device=dev)

    def q8v(self, rows, cols):
        return self.q8[: rows * cols].view(rows, cols)

    def rawv(self, rows, cols):
        return self.raw[: rows * cols].view(rows, cols)

    def prepare_text(self, text_h: torch.Tensor, on_call=None):
        """Per-layer text K / V of the cross attention (engines/wan_va/engine.py:
        180-203) from the text embedder's output ``text_h`` [B, text, D]
        (float32): per-token FP8, the k|v projection, K through ``wan_qkv``'s
        full-width RMSNorm (``cnorm_k``), V rescaled + bias to fp16."""
        note = on_call or (lambda name, **t: None)
        B = text_h.shape[0]
        if text_h.shape[1:] != (self.TEXT, self.D) or not 1 <= B <= self.max_batch:
            raise ValueError(f"text_h must be [B <= {self.max_batch}, {self.TEXT}, {self.D}]")
        rows, D = B * self.TEXT, self.D
        th = text_h.reshape(rows, D).float().contiguous()
        s = self.scale[0][:rows]
        row_quant(th, self.q8v(rows, D), s)
        note("text_quant", x=th, q=self.q8v(rows, D), s=s)
        for i, blk in enumerate(self.blocks):
            raw = self.rawv(rows, 2 * D)
            gemm(self.q8v(rows, D), blk.ckv, raw)
            note("ckv", a=self.q8v(rows, D), w=blk.ckv, out=raw)
            kq = self.q16[:rows]
            wan_qkv(raw, kq, heads=self.H, head_dim=self.HD, tokens=self.TEXT, row=s, col=blk.ckv.scale,
                    bias=blk.ckv.bias, q_norm=blk.cnorm_k, eps=EPS)
            self.tk[i, :B].copy_(kq.view(B, self.TEXT, D))
            # V: rescale + bias only (wan_qkv without norm or rotary), straight to fp16
            wan_qkv(raw[:, D:], self.tv[i, :B].view(rows, D), heads=self.H, head_dim=self.HD, tokens=self.TEXT,
                    row=s, col=blk.ckv.scale[D:], bias=blk.ckv.bias[D:], eps=EPS)
            note("text_kv", raw=raw, row=s, w=blk.ckv, k=self.tk[i, :B].reshape(rows, D),
                 v=self.tv[i, :B].reshape(rows, D))

    def forward(self, B: int, T: int, block_mod: torch.Tensor, head_mod: torch.Tensor, x=None, on_call=None):
        """One forward of ``B`` x ``T`` tokens (engines/wan_va/engine.py:205-245,
        after the patch / action embedding): ``x`` [B T, D] (any float dtype)
        initialises the residual stream, else it continues from ``self.x``.
        ``block_mod`` [layers, cap, 6, D] and ``head_mod`` [cap, 6, D] are the
        float32 modulation tables; ``pos``, ``slots``, ``live``, ``n_live`` and
        ``mod_index`` must be set. Returns the head's float32 ``y`` [B T, D]."""
        L, D, H, HD, FF = len(self.blocks), self.D, self.H, self.HD, self.FF
        if not (1 <= B <= self.max_batch and 1 <= T <= self.max_tokens):
            raise ValueError("B or T beyond the stack's buffers")
        if block_mod.dim() != 4 or block_mod.shape[0] != L or block_mod.shape[2:] != (6, D) or \
                head_mod.dim() != 3 or head_mod.shape[1:] != (6, D):
            raise ValueError(f"block_mod must be [{L}, cap, 6, {D}] and head_mod [cap, 6, {D}]")
        if not (block_mod.is_contiguous() and head_mod.is_contiguous()):
            raise ValueError("modulation tables must be contiguous")
        R = B * T
        if x is not None:
            self.x[:R].copy_(x)
        note = on_call or (lambda name, **t: None)
        q8, raw, mi = self.q8v, self.rawv, self.mod_index[:R]
        s = [v[:R] for v in self.scale]
        xr = self.x[:R]
        qv = self.q16[:R].view(B, T, H, HD)
        ov = self.o16[:R].view(B, T, H, HD)
        t0 = block_mod[0]
        note("pre_res", res=xr)
        residual_norm_quant(xr, layernorm=True, mod_scale=t0[0, 1], mod_shift=t0[0, 0], mod_index=mi,
                            q=q8(R, D), q_scale=s[0], eps=EPS)
        note("norm0", res=xr, q=q8(R, D), s=s[0], mod=(t0, 0, 1))
        for i, blk in enumerate(self.blocks):
            tb = block_mod[i]
            kp, vp = self.kpool[i, :B], self.vpool[i, :B]
            gemm(q8(R, D), blk.qkv, raw(R, 3 * D))
            note("qkv", a=q8(R, D), w=blk.qkv, out=raw(R, 3 * D))
            wan_qkv(raw(R, 3 * D), self.q16[:R], heads=H, head_dim=HD, tokens=T, k_pool=kp, v_pool=vp,
                    slots=self.slots, row=s[0], col=blk.qkv.scale, bias=blk.qkv.bias, q_norm=blk.norm_q,
                    k_norm=blk.norm_k, pos=self.pos, sections=self.sections, inv_freq=self.inv_freq, eps=EPS)
            note("wan_qkv", raw=raw(R, 3 * D), row=s[0], blk=blk, q=self.q16[:R], kp=kp, vp=vp, T=T)
            attention(qv, kp.view(B, self.S, H, HD), vp.view(B, self.S, H, HD), out=ov, kv_len=self.n_live,
                      kv_index=self.live)
            note("self_attention", q=qv, k=kp.view(B, self.S, H, HD), v=vp.view(B, self.S, H, HD), out=ov)
            row_quant(self.o16[:R], q8(R, D), s[1])
            note("row_quant", x=self.o16[:R], q=q8(R, D), s=s[1])
            gemm(q8(R, D), blk.o, raw(R, D))
            note("o", a=q8(R, D), w=blk.o, out=raw(R, D))
            note("pre_res", res=xr)
            residual_norm_quant(xr, delta=raw(R, D), delta_row=s[1], delta_col=blk.o.scale, bias=blk.o.bias,
                                gate=tb[0, 2], mod_index=mi, layernorm=True, weight=blk.norm2_w, beta=blk.norm2_b,
                                q=q8(R, D), q_scale=s[0], eps=EPS)
            note("norm2", res=xr, delta=raw(R, D), delta_row=s[1], w=blk.o, gate=(tb, 2), weight=blk.norm2_w,
                 beta=blk.norm2_b, q=q8(R, D), s=s[0])
            gemm(q8(R, D), blk.cq, raw(R, D))
            note("cq", a=q8(R, D), w=blk.cq, out=raw(R, D))
            wan_qkv(raw(R, D), self.q16[:R], heads=H, head_dim=HD, tokens=T, row=s[0], col=blk.cq.scale,
                    bias=blk.cq.bias, q_norm=blk.cnorm_q, eps=EPS)
            note("cross_q", raw=raw(R, D), row=s[0], w=blk.cq, norm=blk.cnorm_q, q=self.q16[:R])
            tk = self.tk[i, :B].view(B, self.TEXT, H, HD)
            tv = self.tv[i, :B].view(B, self.TEXT, H, HD)
            attention(qv, tk, tv, out=ov)
            note("cross_attention", q=qv, k=tk, v=tv, out=ov)
            row_quant(self.o16[:R], q8(R, D), s[1])
            note("row_quant", x=self.o16[:R], q=q8(R, D), s=s[1])
            gemm(q8(R, D), blk.co, raw(R, D))
            note("co", a=q8(R, D), w=blk.co, out=raw(R, D))
            note("pre_res", res=xr)
            residual_norm_quant(xr, delta=raw(R, D), delta_row=s[1], delta_col=blk.co.scale, bias=blk.co.bias,
                                layernorm=True, mod_scale=tb[0, 4], mod_shift=tb[0, 3], mod_index=mi,
                                q=q8(R, D), q_scale=s[0], eps=EPS)
            note("norm3", res=xr, delta=raw(R, D), delta_row=s[1], w=blk.co, mod=(tb, 3, 4), q=q8(R, D), s=s[0])
            if self.reference_calls:
                rf = self.raw_ff[: R * FF].view(R, FF)
                gemm(q8(R, D), blk.ff1, rf)
                note("ff1_raw", a=q8(R, D), w=blk.ff1, out=rf)
                row_quant(rf, q8(R, FF), s[1], row=s[0], col=blk.ff1.scale, bias=blk.ff1.bias, gelu=True)
                note("ff1_quant", x=rf, row=s[0], w=blk.ff1, q=q8(R, FF), s=s[1])
            else:
                h = self.raw_ff[: R * FF].view(R, FF)
                linear(q8(R, D), s[0], blk.ff1, out=h, act="gelu_tanh")
                note("ff1", a=q8(R, D), sa=s[0], w=blk.ff1, out=h, act="gelu_tanh")
                quant_rows(h, q8(R, FF), s[1])
                note("quant_h", x=h, q=q8(R, FF), s=s[1])
            gemm(q8(R, FF), blk.ff2, raw(R, D))
            note("ff2", a=q8(R, FF), w=blk.ff2, out=raw(R, D))
            note("pre_res", res=xr)
            if i + 1 < L:
                nt = block_mod[i + 1]
                residual_norm_quant(xr, delta=raw(R, D), delta_row=s[1], delta_col=blk.ff2.scale,
                                    bias=blk.ff2.bias, gate=tb[0, 5], layernorm=True, mod_scale=nt[0, 1],
                                    mod_shift=nt[0, 0], mod_index=mi, q=q8(R, D), q_scale=s[0], eps=EPS)
                note("norm_next", res=xr, delta=raw(R, D), delta_row=s[1], w=blk.ff2, gate=(tb, 5),
                     mod=(nt, 0, 1), q=q8(R, D), s=s[0])
            else:
                residual_norm_quant(xr, delta=raw(R, D), delta_row=s[1], delta_col=blk.ff2.scale,
                                    bias=blk.ff2.bias, gate=tb[0, 5], layernorm=True, mod_scale=head_mod[0, 1],
                                    mod_shift=head_mod[0, 0], mod_index=mi, y=self.y[:R], eps=EPS)
                note("norm_head", res=xr, delta=raw(R, D), delta_row=s[1], w=blk.ff2, gate=(tb, 5),
                     mod=(head_mod, 0, 1), y=self.y[:R])
        return self.y[:R]

"""The GR00T N1.7 action head on the gfx950 kernels: the call site that defines
config C2 (the DiT's 1536 -> 6144 GELU -> 1536 MLP over the action rows).

Mirrors instinctflash/engines/groot_n17/engine.py:92-200:
  * ``vlsa``: LayerNorm of the backbone features (``vlln``), then the 2048-wide
    self-attention blocks over them (q|k|v projection, rescale + bias to fp16
    (``dequant_rows``), attention up to the device-side sequence length, FP8 of
    its output (``row_quant``), output projection, residual + LayerNorm, the
    GELU MLP, residual + the next block's LayerNorm);
  * ``cross_kv``: the valid text rows and image rows gathered to the front of
    two buffers (on the device), per-token FP8 of each, and every cross block's
    K / V projection, rescaled to fp16;
  * ``dit``: the flow steps: state and action encoders (torch, as upstream),
    then the 1536-wide DiT blocks -- odd blocks self-attend over the [state,
    actions] rows, even blocks cross-attend to text (block % 4 == 0) or image
    rows -- each with AdaLN-modulated LayerNorms, and the GELU MLP; after the last
    block the output modulation, the decoder and the Euler update of the actions.

``reference_calls=True`` makes exactly the reference's calls. The default lays the
same math out for gfx950: the q|k|v and cross K/V projections write their
rescaled fp16 rows from the GEMM epilogue (no raw accumulator, no
``dequant_rows``), GELU is applied in the ff1 epilogue, and the DiT (41 rows)
runs in the skinny tile layouts with the attention's split-KV combine writing the
o projection's FP8 operand (7 kernels per block instead of 10).
Weights are random (no checkpoint here) with the published shapes; the model is
built with any number of VLSA / DiT blocks (the published head has 4 and 32).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .kernels import E4M3, Fp8Weight, SplitWorkspace, TiledRows, attention, dequant_rows, gemm, linear, \
    pack_skinny, quant_rows, quantize_weight, residual_norm_quant, row_quant
from .kernels.attention import split_count

#: engines/groot_n17/engine.py:17-21
VL_D, VL_H, VL_HD, VL_FF = 2048, 32, 64, 8192
D, H, HD, FF = 1536, 32, 48, 6144
HORIZON, ACT_DIM = 40, 132
SA = HORIZON + 1
LN_EPS, OUT_EPS = 1e-5, 1e-6


@dataclass
class VlsaBlock:
    ln1_w: torch.Tensor
    ln1_b: torch.Tensor
    qkv: Fp8Weight       # [3 VL_D, VL_D] + bias
    o: Fp8Weight
    ln3_w: torch.Tensor
    ln3_b: torch.Tensor
    ff1: Fp8Weight       # [VL_FF, VL_D] + bias
    ff2: Fp8Weight


@dataclass
class DitBlock:
    cross: bool
    text: bool           # cross blocks: text rows (else image rows)
    qkv: Fp8Weight       # self: [3 D, D]; cross: the query only [D, D]
    kv: Fp8Weight | None  # cross: [2 D, VL_D] over the encoder rows
    o: Fp8Weight
    ff1: Fp8Weight       # [FF, D] + bias
    ff2: Fp8Weight


@dataclass
class GrootWeights:
    vlln_w: torch.Tensor
    vlln_b: torch.Tensor
    vlsa: list
    dit: list
    mod: torch.Tensor        # [steps, blocks, 2, D] (scale, shift)
    out_mod: torch.Tensor    # [steps, 2, D] (shift, scale)
    proj_out_w: torch.Tensor  # [D, 1024] (x @ W layout)
    proj_out_b: torch.Tensor
    pos: torch.Tensor        # [HORIZON, D]
    state_w1: torch.Tensor   # [ACT_DIM, 1024]
    state_b1: torch.Tensor
    state_w2: torch.Tensor   # [1024, D]
    state_b2: torch.Tensor
    act_w: torch.Tensor      # [ACT_DIM, D]
    act_c: torch.Tensor      # [steps, D]
    act_w3: torch.Tensor     # [D, D]
    act_b3: torch.Tensor
    dec_w1: torch.Tensor     # [1024, 1024]
    dec_b1: torch.Tensor
    dec_w2: torch.Tensor     # [1024, ACT_DIM]
    dec_b2: torch.Tensor
    steps: int
    dt: float


def random_groot_weights(device, *, vlsa_blocks=4, dit_blocks=32, steps=4, seed=0) -> GrootWeights:
    """Random weights with the head's shapes: FP8 projections N(0, 0.02) (biases
    N(0, 0.01)) quantized per output channel on the device; LayerNorm weights
    1 + N(0, 0.1); modulations N(0, 0.1); the float32 encoders / decoder
    N(0, 1 / sqrt(fan in)). Block i of the DiT cross-attends when i is even, to
    text rows when i % 4 == 0 (engines/groot_n17/weights.py:139-156)."""
    g = torch.Generator().manual_seed(seed)
    dev = torch.device(device)

    def lin(n, k):
        w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
        return quantize_weight(w.to(dev), (torch.randn(n, generator=g) * 0.01).to(dev), dev)

    def vec(n, s=0.1, base=0.0):
        return (base + torch.randn(n, generator=g) * s).to(dev)

    def dense(k, n):
        return (torch.randn(k, n, generator=g) / k ** 0.5).to(dev)

    vlsa = [VlsaBlock(vec(VL_D, base=1.0), vec(VL_D, 0.05), lin(3 * VL_D, VL_D), lin(VL_D, VL_D), vec(VL_D, base=1.0),
                      vec(VL_D, 0.05), lin(VL_FF, VL_D), lin(VL_D, VL_FF)) for _ in range(vlsa_blocks)]
    dit = []
    for i in range(dit_blocks):
        cross = i % 2 == 0
        dit.append(DitBlock(cross, i % 4 == 0, lin(D, D) if cross else lin(3 * D, D),
                            lin(2 * D, VL_D) if cross else None, lin(D, D), lin(FF, D), lin(D, FF)))
    return GrootWeights(
        vlln_w=vec(VL_D, base=1.0), vlln_b=vec(VL_D, 0.05), vlsa=vlsa, dit=dit,
        mod=(torch.randn(steps, dit_blocks, 2, D, generator=g) * 0.1).to(dev),
        out_mod=(torch.randn(steps, 2, D, generator=g) * 0.1).to(dev),
        proj_out_w=dense(D, 1024), proj_out_b=vec(1024, 0.01), pos=vec(HORIZON * D, 0.02).view(HORIZON, D),
        state_w1=dense(ACT_DIM, 1024), state_b1=vec(1024, 0.01), state_w2=dense(1024, D), state_b2=vec(D, 0.01),
        act_w=dense(ACT_DIM, D), act_c=(torch.randn(steps, D, generator=g) * 0.1).to(dev), act_w3=dense(D, D),
        act_b3=vec(D, 0.01), dec_w1=dense(1024, 1024), dec_b1=vec(1024, 0.01), dec_w2=dense(1024, ACT_DIM),
        dec_b2=vec(ACT_DIM, 0.01), steps=steps, dt=1.0 / steps)


class GrootHead:
    """The action head over up to ``max_seq`` backbone rows. Device state:
    features ``feat`` [S, VL_D] (float32), ``img_mask`` / ``valid`` [S] (bool),
    the sequence length ``seq_len`` [1] (int32), ``state`` [1, ACT_DIM] and
    ``noise`` [HORIZON, ACT_DIM]; ``forward(M)`` (M: the bucketed row count)
    runs ``vlsa``, ``cross_kv`` and ``dit`` and leaves the actions in ``a_t``."""

    def __init__(self, weights: GrootWeights, device, *, max_seq=512, reference_calls=False):
        self.w = weights
        self.dev = torch.device(device)
        self.reference_calls = bool(reference_calls)
        dev, f32, f16, bf16 = self.dev, torch.float32, torch.float16, torch.bfloat16
        S = self.max_seq = int(max_seq)
        rows = max(S, SA)
        self.feat = torch.zeros(S, VL_D, dtype=f32, device=dev)
        self.img_mask = torch.zeros(S, dtype=torch.bool, device=dev)
        self.valid = torch.zeros(S, dtype=torch.bool, device=dev)
        self.seq_len = torch.zeros(1, dtype=torch.int32, device=dev)
        self.n_img = torch.zeros(1, dtype=torch.int32, device=dev)
        self.n_txt = torch.zeros(1, dtype=torch.int32, device=dev)
        self.state = torch.zeros(1, ACT_DIM, dtype=f32, device=dev)
        self.noise = torch.zeros(HORIZON, ACT_DIM, dtype=f32, device=dev)
        self.q8buf = torch.zeros(rows * VL_FF, dtype=E4M3, device=dev)
        self.rawbuf = torch.zeros(rows * VL_FF, dtype=bf16, device=dev)
        self.scale = [torch.zeros(rows, dtype=f32, device=dev) for _ in range(2)]
        self.vx = torch.zeros(S, VL_D, dtype=f32, device=dev)
        self.enc = {k: torch.zeros(S, VL_D, dtype=f32, device=dev) for k in ("text", "image")}
        self.qkv16 = torch.zeros(rows, 3 * VL_D, dtype=f16, device=dev)
        self.o16 = torch.zeros(rows, VL_D, dtype=f16, device=dev)
        n_cross = sum(b.cross for b in weights.dit)
        # cross K and V of a block side by side per row ([..., 0, :, :] K, [..., 1, :, :] V),
        # so one projection writes both
        self.kv16 = torch.zeros(n_cross, S, 2, H, HD, dtype=f16, device=dev)
        self.kc, self.vc = self.kv16[:, :, 0], self.kv16[:, :, 1]
        self.h = torch.zeros(SA, D, dtype=f32, device=dev)
        self.y = torch.zeros(SA, D, dtype=f32, device=dev)
        self.a_t = torch.zeros(HORIZON, ACT_DIM, dtype=f32, device=dev)
        self.state_emb = torch.zeros(1, D, dtype=f32, device=dev)
        self.enc_tmp = torch.zeros(1, 1024, dtype=f32, device=dev)
        if not self.reference_calls:
            from . import _lib
            lib = _lib.load()
            tiled = lambda k: TiledRows(torch.zeros(lib.ifx_quant_rows_tiled_bytes(SA, k), dtype=E4M3,  # noqa: E731
                                                    device=dev), SA, k)
            self.xq, self.oq, self.hq = tiled(D), tiled(D), tiled(FF)
            self.dit_t = [DitBlock(b.cross, b.text, pack_skinny(b.qkv), b.kv, pack_skinny(b.o), pack_skinny(b.ff1),
                                   pack_skinny(b.ff2)) for b in weights.dit]
            self.split_self = SplitWorkspace(1, SA, H, H, HD, max(2, split_count(1, SA, H, H, SA)), dev)
            self.split_cross = SplitWorkspace(1, SA, H, H, HD, max(2, split_count(1, SA, H, H, S)), dev)

    def q8(self, rows, cols):
        return self.q8buf[: rows * cols].view(rows, cols)

    def raw(self, rows, cols):
        return self.rawbuf[: rows * cols].view(rows, cols)

    def set_inputs(self, features, image_mask, attention_mask, state, noise):
        """engines/groot_n17/engine.py:68-88 without the graph: features [n, VL_D];
        masks [n] bool; state [ACT_DIM]; noise [HORIZON, ACT_DIM]."""
        n = int(features.shape[0])
        if not 1 <= n <= self.max_seq:
            raise ValueError(f"1..{self.max_seq} backbone rows supported, got {n}")
        self.feat[:n].copy_(features)
        self.feat[n:].zero_()
        self.img_mask[:n].copy_(image_mask)
        self.img_mask[n:].zero_()
        self.valid[:n].copy_(attention_mask)
        self.valid[n:].zero_()
        self.seq_len.fill_(n)
        self.state.copy_(state.reshape(1, ACT_DIM))
        self.noise.copy_(noise.reshape(HORIZON, ACT_DIM))

    def forward(self, M, on_call=None):
        if not 1 <= M <= self.max_seq:
            raise ValueError(f"M must be in [1, {self.max_seq}]")
        if on_call is not None and not self.reference_calls:
            raise ValueError("on_call needs reference_calls=True")
        note = on_call or (lambda name, **t: None)
        self.vlsa(M, note)
        self.cross_kv(M, note)
        if self.reference_calls:
            self.dit(note)
        else:
            self.dit_fused()
        return self.a_t

    def _mlp(self, note, x_q, x_s, blk, rows, width, ff):
        """The GELU MLP's first half: FP8 hidden rows of blk.ff1 into q8(rows, ff), scales s[1]."""
        q8, raw, s = self.q8, self.raw, self.scale
        if self.reference_calls:
            gemm(x_q, blk.ff1, raw(rows, ff))
            note("ff1_raw", a=x_q, w=blk.ff1, out=raw(rows, ff))
            row_quant(raw(rows, ff), q8(rows, ff), s[1][:rows], row=x_s, col=blk.ff1.scale, bias=blk.ff1.bias,
                      gelu=True)
            note("ff1_quant", x=raw(rows, ff), row=x_s, w=blk.ff1, q=q8(rows, ff), s=s[1][:rows])
        else:
            h = raw(rows, ff)
            linear(x_q, x_s, blk.ff1, out=h, act="gelu_tanh")
            note("ff1", a=x_q, sa=x_s, w=blk.ff1, out=h, act="gelu_tanh")
            quant_rows(h, q8(rows, ff), s[1][:rows])
            note("quant_h", x=h, q=q8(rows, ff), s=s[1][:rows])

    def vlsa(self, M, note=None):
        """engines/groot_n17/engine.py:92-129."""
        note = note or (lambda name, **t: None)
        w, q8, raw = self.w, self.q8, self.raw
        s = [v[:M] for v in self.scale]
        vx = self.vx[:M]
        residual_norm_quant(self.feat[:M], layernorm=True, weight=w.vlln_w, beta=w.vlln_b, y=vx, eps=LN_EPS)
        note("vlln", src=self.feat[:M], y=vx, weight=w.vlln_w, beta=w.vlln_b)
        if not w.vlsa:
            return
        L0 = w.vlsa[0]
        note("pre_res", res=vx)
        residual_norm_quant(vx, layernorm=True, weight=L0.ln1_w, beta=L0.ln1_b, q=q8(M, VL_D), q_scale=s[0],
                            eps=LN_EPS)
        note("norm_vl", res=vx, weight=L0.ln1_w, beta=L0.ln1_b, q=q8(M, VL_D), s=s[0])
        view = (1, M, VL_H, VL_HD)
        for i, L in enumerate(w.vlsa):
            if self.reference_calls:
                gemm(q8(M, VL_D), L.qkv, raw(M, 3 * VL_D))
                note("gemm", a=q8(M, VL_D), w=L.qkv, out=raw(M, 3 * VL_D))
                dequant_rows(raw(M, 3 * VL_D), self.qkv16[:M], row=s[0], col=L.qkv.scale, bias=L.qkv.bias)
                note("dequant", x=raw(M, 3 * VL_D), y=self.qkv16[:M], row=s[0], w=L.qkv)
            else:
                linear(q8(M, VL_D), s[0], L.qkv, out=self.qkv16[:M])
            qkv = self.qkv16[:M].view(1, M, 3, VL_H, VL_HD)
            ov = self.o16[:M].view(view)
            attention(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], out=ov, kv_len=self.seq_len)
            note("attention", q=qkv[:, :, 0], k=qkv[:, :, 1], v=qkv[:, :, 2], out=ov, kv_len=self.seq_len)
            row_quant(self.o16[:M], q8(M, VL_D), s[1])
            note("row_quant", x=self.o16[:M], q=q8(M, VL_D), s=s[1])
            gemm(q8(M, VL_D), L.o, raw(M, VL_D))
            note("gemm", a=q8(M, VL_D), w=L.o, out=raw(M, VL_D))
            note("pre_res", res=vx)
            residual_norm_quant(vx, delta=raw(M, VL_D), delta_row=s[1], delta_col=L.o.scale, bias=L.o.bias,
                                layernorm=True, weight=L.ln3_w, beta=L.ln3_b, q=q8(M, VL_D), q_scale=s[0],
                                eps=LN_EPS)
            note("norm_vl", res=vx, delta=raw(M, VL_D), delta_row=s[1], w=L.o, weight=L.ln3_w, beta=L.ln3_b,
                 q=q8(M, VL_D), s=s[0])
            self._mlp(note, q8(M, VL_D), s[0], L, M, VL_D, VL_FF)
            gemm(q8(M, VL_FF), L.ff2, raw(M, VL_D))
            note("gemm", a=q8(M, VL_FF), w=L.ff2, out=raw(M, VL_D))
            note("pre_res", res=vx)
            nxt = w.vlsa[i + 1] if i + 1 < len(w.vlsa) else None
            if nxt is not None:
                residual_norm_quant(vx, delta=raw(M, VL_D), delta_row=s[1], delta_col=L.ff2.scale, bias=L.ff2.bias,
                                    layernorm=True, weight=nxt.ln1_w, beta=nxt.ln1_b, q=q8(M, VL_D), q_scale=s[0],
                                    eps=LN_EPS)
                note("norm_vl", res=vx, delta=raw(M, VL_D), delta_row=s[1], w=L.ff2, weight=nxt.ln1_w,
                     beta=nxt.ln1_b, q=q8(M, VL_D), s=s[0])
            else:
                residual_norm_quant(vx, delta=raw(M, VL_D), delta_row=s[1], delta_col=L.ff2.scale, bias=L.ff2.bias,
                                    eps=LN_EPS)
                note("res_vl", res=vx, delta=raw(M, VL_D), delta_row=s[1], w=L.ff2)

    def cross_kv(self, M, note=None):
        """engines/groot_n17/engine.py:131-152: valid text / image rows to the
        front of two buffers (stable order, on the device), then each cross
        block's K / V projection of its rows, rescaled + bias to fp16."""
        note = note or (lambda name, **t: None)
        q8, raw = self.q8, self.raw
        s0 = self.scale[0][:M]
        img = self.img_mask[:M] & self.valid[:M]
        txt = ~self.img_mask[:M] & self.valid[:M]
        for key, sel, count in (("image", img, self.n_img), ("text", txt, self.n_txt)):
            order = torch.argsort((~sel).to(torch.int8), stable=True)
            torch.index_select(self.vx[:M], 0, order, out=self.enc[key][:M])
            count.copy_(sel.sum().to(torch.int32).view(1))
        for key in ("text", "image"):
            src = self.enc[key][:M]
            row_quant(src, q8(M, VL_D), s0)
            note("enc_quant", x=src, q=q8(M, VL_D), s=s0)
            for i, blk in enumerate(self.w.dit):
                if not blk.cross or blk.text != (key == "text"):
                    continue
                ci = i // 2
                if not self.reference_calls:
                    linear(q8(M, VL_D), s0, blk.kv, out=self.kv16[ci, :M].view(M, 2 * D))
                    continue
                gemm(q8(M, VL_D), blk.kv, raw(M, 2 * D))
                note("gemm", a=q8(M, VL_D), w=blk.kv, out=raw(M, 2 * D))
                dequant_rows(raw(M, 2 * D)[:, :D], self.kc[ci, :M].view(M, D), row=s0, col=blk.kv.scale[:D],
                             bias=blk.kv.bias[:D])
                dequant_rows(raw(M, 2 * D)[:, D:], self.vc[ci, :M].view(M, D), row=s0, col=blk.kv.scale[D:],
                             bias=blk.kv.bias[D:])
                note("dequant_kv", x=raw(M, 2 * D), k=self.kc[ci, :M].view(M, D), v=self.vc[ci, :M].view(M, D),
                     row=s0, w=blk.kv)

    def dit(self, note=None):
        """engines/groot_n17/engine.py:154-200: ``steps`` flow steps of the DiT."""
        note = note or (lambda name, **t: None)
        w, q8, raw = self.w, self.q8, self.raw
        s = [v[:SA] for v in self.scale]
        torch.addmm(w.state_b1, self.state, w.state_w1, out=self.enc_tmp)
        torch.relu_(self.enc_tmp)
        torch.addmm(w.state_b2, self.enc_tmp, w.state_w2, out=self.state_emb)
        self.a_t.copy_(self.noise)
        view = (1, SA, H, HD)
        qkv16 = self.qkv16[:SA]
        o16 = self.o16[:SA, :D]
        last = len(w.dit) - 1
        for step in range(w.steps):
            mod = w.mod[step]
            self.h[:1].copy_(self.state_emb)
            act = torch.addmm(w.act_c[step], self.a_t, w.act_w)
            act = act * torch.sigmoid(act)
            torch.addmm(w.act_b3, act, w.act_w3, out=self.h[1:])
            self.h[1:].add_(w.pos)
            note("pre_res", res=self.h)
            residual_norm_quant(self.h, layernorm=True, mod_scale=mod[0, 0], mod_shift=mod[0, 1], q=q8(SA, D),
                                q_scale=s[0], eps=LN_EPS)
            note("norm_dit", res=self.h, mod=(mod[0, 0], mod[0, 1]), q=q8(SA, D), s=s[0])
            for i, blk in enumerate(w.dit):
                if blk.cross:
                    gemm(q8(SA, D), blk.qkv, raw(SA, D))
                    note("gemm", a=q8(SA, D), w=blk.qkv, out=raw(SA, D))
                    dequant_rows(raw(SA, D), qkv16[:, :D], row=s[0], col=blk.qkv.scale, bias=blk.qkv.bias)
                    note("dequant", x=raw(SA, D), y=qkv16[:, :D], row=s[0], w=blk.qkv)
                    ci = i // 2
                    n = self.n_txt if blk.text else self.n_img
                    attention(qkv16[:, :D].view(view), self.kc[ci][None], self.vc[ci][None], out=o16.view(view),
                              kv_len=n)
                    note("attention", q=qkv16[:, :D].view(view), k=self.kc[ci][None], v=self.vc[ci][None],
                         out=o16.view(view), kv_len=n)
                else:
                    gemm(q8(SA, D), blk.qkv, raw(SA, 3 * D))
                    note("gemm", a=q8(SA, D), w=blk.qkv, out=raw(SA, 3 * D))
                    dequant_rows(raw(SA, 3 * D), qkv16[:, :3 * D], row=s[0], col=blk.qkv.scale, bias=blk.qkv.bias)
                    note("dequant", x=raw(SA, 3 * D), y=qkv16[:, :3 * D], row=s[0], w=blk.qkv)
                    qkv = qkv16[:, :3 * D].view(1, SA, 3, H, HD)
                    attention(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], out=o16.view(view))
                    note("attention", q=qkv[:, :, 0], k=qkv[:, :, 1], v=qkv[:, :, 2], out=o16.view(view), kv_len=None)
                row_quant(o16, q8(SA, D), s[1])
                note("row_quant", x=o16, q=q8(SA, D), s=s[1])
                gemm(q8(SA, D), blk.o, raw(SA, D))
                note("gemm", a=q8(SA, D), w=blk.o, out=raw(SA, D))
                note("pre_res", res=self.h)
                residual_norm_quant(self.h, delta=raw(SA, D), delta_row=s[1], delta_col=blk.o.scale, bias=blk.o.bias,
                                    layernorm=True, q=q8(SA, D), q_scale=s[0], eps=LN_EPS)
                note("norm_dit", res=self.h, delta=raw(SA, D), delta_row=s[1], w=blk.o, q=q8(SA, D), s=s[0])
                self._mlp(note, q8(SA, D), s[0], blk, SA, D, FF)
                gemm(q8(SA, FF), blk.ff2, raw(SA, D))
                note("gemm", a=q8(SA, FF), w=blk.ff2, out=raw(SA, D))
                note("pre_res", res=self.h)
                if i < last:
                    nm = mod[i + 1]
                    residual_norm_quant(self.h, delta=raw(SA, D), delta_row=s[1], delta_col=blk.ff2.scale,
                                        bias=blk.ff2.bias, layernorm=True, mod_scale=nm[0], mod_shift=nm[1],
                                        q=q8(SA, D), q_scale=s[0], eps=LN_EPS)
                    note("norm_dit", res=self.h, delta=raw(SA, D), delta_row=s[1], w=blk.ff2, mod=(nm[0], nm[1]),
                         q=q8(SA, D), s=s[0])
                else:
                    om = w.out_mod[step]
                    residual_norm_quant(self.h, delta=raw(SA, D), delta_row=s[1], delta_col=blk.ff2.scale,
                                        bias=blk.ff2.bias, layernorm=True, mod_scale=om[1], mod_shift=om[0],
                                        y=self.y, eps=OUT_EPS)
                    note("norm_out", res=self.h, delta=raw(SA, D), delta_row=s[1], w=blk.ff2, mod=(om[1], om[0]),
                         y=self.y)
            out = torch.addmm(w.proj_out_b, self.y[1:], w.proj_out_w)
            v = torch.addmm(w.dec_b2, torch.relu(torch.addmm(w.dec_b1, out, w.dec_w1)), w.dec_w2)
            self.a_t.add_(v, alpha=w.dt)

    def dit_fused(self):
        """``dit`` in the gfx950 layout (same math): tile-layout FP8 rows, fp16
        q|k|v straight from the projection epilogue, the attention combine
        writing the o projection's FP8 operand, GELU in the ff1 epilogue."""
        w, raw = self.w, self.raw
        s = [v[:SA] for v in self.scale]
        xq, oq, hq = self.xq, self.oq, self.hq
        torch.addmm(w.state_b1, self.state, w.state_w1, out=self.enc_tmp)
        torch.relu_(self.enc_tmp)
        torch.addmm(w.state_b2, self.enc_tmp, w.state_w2, out=self.state_emb)
        self.a_t.copy_(self.noise)
        view = (1, SA, H, HD)
        qkv16 = self.qkv16[:SA]
        last = len(self.dit_t) - 1
        for step in range(w.steps):
            mod = w.mod[step]
            self.h[:1].copy_(self.state_emb)
            act = torch.addmm(w.act_c[step], self.a_t, w.act_w)
            act = act * torch.sigmoid(act)
            torch.addmm(w.act_b3, act, w.act_w3, out=self.h[1:])
            self.h[1:].add_(w.pos)
            residual_norm_quant(self.h, layernorm=True, mod_scale=mod[0, 0], mod_shift=mod[0, 1], q=xq,
                                q_scale=s[0], eps=LN_EPS)
            for i, blk in enumerate(self.dit_t):
                if blk.cross:
                    linear(xq, s[0], blk.qkv, out=qkv16[:, :D])
                    ci = i // 2
                    attention(qkv16[:, :D].view(view), self.kc[ci][None], self.vc[ci][None],
                              kv_len=self.n_txt if blk.text else self.n_img, split=self.split_cross, q8=oq,
                              q8_scale=s[1])
                else:
                    linear(xq, s[0], blk.qkv, out=qkv16[:, :3 * D])
                    qkv = qkv16[:, :3 * D].view(1, SA, 3, H, HD)
                    attention(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], split=self.split_self, q8=oq, q8_scale=s[1])
                gemm(oq, blk.o, raw(SA, D))
                residual_norm_quant(self.h, delta=raw(SA, D), delta_row=s[1], delta_col=blk.o.scale, bias=blk.o.bias,
                                    layernorm=True, q=xq, q_scale=s[0], eps=LN_EPS)
                linear(xq, s[0], blk.ff1, out=raw(SA, FF), act="gelu_tanh")
                row_quant(raw(SA, FF), hq, s[1])
                gemm(hq, blk.ff2, raw(SA, D))
                if i < last:
                    nm = mod[i + 1]
                    residual_norm_quant(self.h, delta=raw(SA, D), delta_row=s[1], delta_col=blk.ff2.scale,
                                        bias=blk.ff2.bias, layernorm=True, mod_scale=nm[0], mod_shift=nm[1], q=xq,
                                        q_scale=s[0], eps=LN_EPS)
                else:
                    om = w.out_mod[step]
                    residual_norm_quant(self.h, delta=raw(SA, D), delta_row=s[1], delta_col=blk.ff2.scale,
                                        bias=blk.ff2.bias, layernorm=True, mod_scale=om[1], mod_shift=om[0],
                                        y=self.y, eps=OUT_EPS)
            out = torch.addmm(w.proj_out_b, self.y[1:], w.proj_out_w)
            v = torch.addmm(w.dec_b2, torch.relu(torch.addmm(w.dec_b1, out, w.dec_w1)), w.dec_w2)
            self.a_t.add_(v, alpha=w.dt)

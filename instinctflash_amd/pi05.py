"""The pi05 action expert's flow-matching loop on the gfx950 kernels.

Mirrors the reference engine's expert stage (instinctflash/engines/pi05/
engine.py:212-245) call for call, with this package's kernels behind the same
names: per Euler step, the action-in projection, then per layer the fused QKV
projection, the QKV split with RoPE into the K/V cache after the prefix, the
attention of the 50-token chunk over prefix + chunk, the per-token FP8 of the
attention output, the output projection with the adaLN-gated residual and the
next norm, the GeGLU MLP and the down projection with the next gated residual.
Weights are per-output-channel FP8 (``quantize_weight``); the whole loop is
graph-capturable (the prefix length lives in device memory).

It exists to run the drop-in kernels end to end at the engine's real shapes:
``random_weights`` builds random weights of the published architecture
(Gemma-300M expert: width 1024, MLP 4096, 18 layers, 8 query heads and one KV
head of 256), since no checkpoint is available here.

``reference_calls=True`` makes exactly the reference's calls (row-major FP8
operands, attention into fp16 then ``row_quant``). The default keeps the same
math but lays the loop out for gfx950: weights in the skinny tile layout
(``pack_skinny``), every FP8 activation written by its producer in the tile
layout the M <= 64 GEMM reads with 1 KB loads, the QKV split's rescale, rotary
pairs and cache stores done in the QKV projection's epilogue
(``linear_qkv_rope``), GeGLU in the gate|up projection's epilogue (GLU-packed
weights, then ``row_quant`` of the half-width result instead of
``gated_act_quant`` of the full-width accumulator), and the attention's split-KV
combine emitting the output projection's FP8 operand directly (two kernels per
layer fewer).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .kernels import E4M3, Fp8Weight, SplitWorkspace, TiledRows, attention, gated_act_quant, gemm, linear, \
    linear_qkv_rope, pack_glu, pack_skinny, permute_rope_rows, qkv_split, quantize_weight, residual_norm_quant, \
    rope_inv_freq, row_quant
from .kernels.activation import GELU_TANH
from .kernels.attention import split_count

EX_D, EX_FF = 1024, 4096
HEADS, HEAD_DIM = 8, 256
QKV_N = (HEADS + 2) * HEAD_DIM  # q 2048 | k 256 | v 256
ACTION_DIM = 32


@dataclass
class ExpertLayer:
    qkv: Fp8Weight
    o: Fp8Weight
    gate_up: Fp8Weight
    down: Fp8Weight


@dataclass
class ExpertWeights:
    layers: list
    mod_attn: torch.Tensor   # [steps, L, 3, EX_D]: (scale, shift, gate)
    mod_ffn: torch.Tensor    # [steps, L, 3, EX_D]
    mod_final: torch.Tensor  # [steps, 2, EX_D]
    action_in_w: torch.Tensor   # [EX_D, 32]
    action_in_b: torch.Tensor   # [EX_D]
    action_out_w: torch.Tensor  # [32, EX_D]
    action_out_b: torch.Tensor  # [32]

    @property
    def steps(self) -> int:
        return self.mod_attn.shape[0]


def random_weights(device, layers=18, steps=10, seed=0) -> ExpertWeights:
    """Random weights of the expert's architecture (N(0, 0.02) projections,
    small adaLN tables), quantized per output channel on the device."""
    g = torch.Generator().manual_seed(seed)

    def lin(n, k):
        return quantize_weight((torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16).to(device), None, device)

    ls = [ExpertLayer(lin(QKV_N, EX_D), lin(EX_D, HEADS * HEAD_DIM), lin(2 * EX_FF, EX_D), lin(EX_D, EX_FF))
          for _ in range(layers)]
    f = lambda *s, sc=0.1: (torch.randn(*s, generator=g) * sc).to(device)  # noqa: E731
    gate = lambda *s: (torch.rand(*s, generator=g) * 0.5 + 0.5).to(device)  # noqa: E731
    ma = torch.cat([f(steps, layers, 2, EX_D), gate(steps, layers, 1, EX_D)], 2).contiguous()
    mf = torch.cat([f(steps, layers, 2, EX_D), gate(steps, layers, 1, EX_D)], 2).contiguous()
    return ExpertWeights(ls, ma, mf, f(steps, 2, EX_D).contiguous(), f(EX_D, ACTION_DIM, sc=0.2), f(EX_D, sc=0.01),
                         f(ACTION_DIM, EX_D, sc=0.02), f(ACTION_DIM, sc=0.01))


class Pi05Expert:
    """The expert stage of the pi05 engine over a prefix K/V cache.

    ``kc`` / ``vc`` [layers, smax + chunk, 1, 256] fp16 hold the prefix's keys and
    values (written by the prefix stage in the engine; filled by the caller
    here); ``set_prefix(n)`` sets the valid prefix length (device memory, so a
    captured graph follows it). ``forward(noise)`` runs the Euler steps and
    returns the chunk's actions x_t [chunk, 32] (reference engine.py:212-245).
    """

    def __init__(self, weights: ExpertWeights, device, *, smax=1024, chunk=50, reference_calls=False):
        self.w = weights
        self.reference_calls = bool(reference_calls)
        self.dev = torch.device(device)
        self.chunk = int(chunk)
        self.smax = int(smax)
        L = len(weights.layers)
        dev, f32, f16, bf16 = self.dev, torch.float32, torch.float16, torch.bfloat16
        A = self.chunk
        self.q8 = torch.zeros(A * EX_FF, dtype=E4M3, device=dev)
        self.raw = torch.zeros(A * 2 * EX_FF, dtype=bf16, device=dev)
        self.scale = [torch.zeros(A, dtype=f32, device=dev) for _ in range(2)]
        self.q16 = torch.zeros(A, HEADS, HEAD_DIM, dtype=f16, device=dev)
        self.o16 = torch.zeros(A, HEADS * HEAD_DIM, dtype=f16, device=dev)
        self.kc = torch.zeros(L, self.smax + A, 1, HEAD_DIM, dtype=f16, device=dev)
        self.vc = torch.zeros_like(self.kc)
        self.x_t = torch.zeros(A, ACTION_DIM, dtype=f32, device=dev)
        self.noise = torch.zeros(A, ACTION_DIM, dtype=f32, device=dev)
        self.dx = torch.zeros(A, EX_D, dtype=f32, device=dev)
        self.dy = torch.zeros(A, EX_D, dtype=f32, device=dev)
        self.prefix_len = torch.zeros(1, dtype=torch.int32, device=dev)
        self.kv_len = torch.zeros(1, dtype=torch.int32, device=dev)
        self.inv_freq = rope_inv_freq(HEAD_DIM, 10000.0, dev)
        self.pos_chunk = torch.zeros(A, 1, dtype=f32, device=dev)
        dt = -1.0 / weights.steps
        self.out_w_dt = (weights.action_out_w * dt).t().contiguous()
        self.out_b_dt = (weights.action_out_b * dt).contiguous()
        self.in_w_t = weights.action_in_w.t().contiguous()
        if not self.reference_calls:
            from . import _lib
            lib = _lib.load()
            tiled = lambda k: TiledRows(torch.zeros(lib.ifx_quant_rows_tiled_bytes(A, k), dtype=E4M3,  # noqa: E731
                                                    device=dev), A, k)
            self.xq, self.oq, self.hq = tiled(EX_D), tiled(HEADS * HEAD_DIM), tiled(EX_FF)
            self.layers = [ExpertLayer(pack_skinny(permute_rope_rows(L.qkv, HEADS, 1, HEAD_DIM)), pack_skinny(L.o),
                                       pack_skinny(pack_glu(L.gate_up)), pack_skinny(L.down)) for L in weights.layers]
            splits = max(2, split_count(1, A, HEADS, 1, self.smax + A))
            self.split = SplitWorkspace(1, A, HEADS, 1, HEAD_DIM, splits, dev)

    def q8v(self, rows, cols):
        return self.q8[: rows * cols].view(rows, cols)

    def rawv(self, rows, cols):
        return self.raw[: rows * cols].view(rows, cols)

    def set_prefix(self, n: int):
        """Valid prefix rows n (<= smax): keys 0..n-1 of the caches, chunk rows after them."""
        if not 1 <= n <= self.smax:
            raise ValueError(f"prefix length must be in [1, {self.smax}]")
        self.prefix_len.fill_(n)
        self.kv_len.fill_(n + self.chunk)
        torch.arange(n, n + self.chunk, out=self.pos_chunk[:, 0])

    def forward(self, noise=None, on_call=None):
        """Reference engine.py:212-245 (`_expert`); call for call with
        ``reference_calls``, else the tile-layout form of the same math.
        ``on_call`` (reference calls only) is called after every kernel with its
        name and the buffers it read and wrote, for per-call parity tests."""
        if not self.reference_calls:
            if on_call is not None:
                raise ValueError("on_call needs reference_calls=True")
            return self._forward_tiled(noise)
        note = on_call or (lambda name, **t: None)
        w, A = self.w, self.chunk
        q8, raw, s = self.q8v, self.rawv, self.scale
        if noise is not None:
            self.noise.copy_(noise)
        self.x_t.copy_(self.noise)
        qv = self.q16[:A].view(1, A, HEADS, HEAD_DIM)
        ov = self.o16[:A].view(1, A, HEADS, HEAD_DIM)
        last = len(w.layers) - 1
        for step in range(w.steps):
            torch.addmm(w.action_in_b, self.x_t, self.in_w_t, out=self.dx)
            ma, mf = w.mod_attn[step], w.mod_ffn[step]
            note("pre_res", res=self.dx)
            residual_norm_quant(self.dx, mod_scale=ma[0, 0], mod_shift=ma[0, 1], q=q8(A, EX_D), q_scale=s[0])
            note("norm", res=self.dx, mod=(ma[0, 0], ma[0, 1]), q=q8(A, EX_D), s=s[0])
            for i, L in enumerate(w.layers):
                gemm(q8(A, EX_D), L.qkv, raw(A, QKV_N))
                note("gemm", a=q8(A, EX_D), w=L.qkv, out=raw(A, QKV_N))
                qkv_split(raw(A, QKV_N), self.q16[:A], self.kc[i], self.vc[i], heads_q=HEADS, heads_kv=1,
                          head_dim=HEAD_DIM, inv_freq=self.inv_freq, pos=self.pos_chunk, row=s[0],
                          col=L.qkv.scale, kv_base=self.prefix_len)
                note("qkv_split", raw=raw(A, QKV_N), row=s[0], w=L.qkv, q=self.q16[:A], k=self.kc[i], v=self.vc[i])
                attention(qv, self.kc[i][None], self.vc[i][None], out=ov, kv_len=self.kv_len,
                          scale=HEAD_DIM ** -0.5)
                note("attention", q=qv, k=self.kc[i][None], v=self.vc[i][None], out=ov, kv_len=self.kv_len)
                row_quant(self.o16[:A], q8(A, HEADS * HEAD_DIM), s[1])
                note("row_quant", x=self.o16[:A], q=q8(A, HEADS * HEAD_DIM), s=s[1])
                gemm(q8(A, HEADS * HEAD_DIM), L.o, raw(A, EX_D))
                note("gemm", a=q8(A, HEADS * HEAD_DIM), w=L.o, out=raw(A, EX_D))
                note("pre_res", res=self.dx)
                residual_norm_quant(self.dx, delta=raw(A, EX_D), delta_row=s[1], delta_col=L.o.scale,
                                    gate=ma[i, 2], mod_scale=mf[i, 0], mod_shift=mf[i, 1],
                                    q=q8(A, EX_D), q_scale=s[0])
                note("norm", res=self.dx, delta=raw(A, EX_D), delta_row=s[1], w=L.o, gate=ma[i, 2],
                     mod=(mf[i, 0], mf[i, 1]), q=q8(A, EX_D), s=s[0])
                gemm(q8(A, EX_D), L.gate_up, raw(A, 2 * EX_FF))
                note("gemm", a=q8(A, EX_D), w=L.gate_up, out=raw(A, 2 * EX_FF))
                gated_act_quant(raw(A, 2 * EX_FF), q8(A, EX_FF), s[1], row=s[0], col=L.gate_up.scale,
                                act=GELU_TANH)
                note("gated_act_quant", gu=raw(A, 2 * EX_FF), row=s[0], w=L.gate_up, q=q8(A, EX_FF), s=s[1])
                gemm(q8(A, EX_FF), L.down, raw(A, EX_D))
                note("gemm", a=q8(A, EX_FF), w=L.down, out=raw(A, EX_D))
                note("pre_res", res=self.dx)
                if i < last:
                    residual_norm_quant(self.dx, delta=raw(A, EX_D), delta_row=s[1], delta_col=L.down.scale,
                                        gate=mf[i, 2], mod_scale=ma[i + 1, 0], mod_shift=ma[i + 1, 1],
                                        q=q8(A, EX_D), q_scale=s[0])
                    note("norm", res=self.dx, delta=raw(A, EX_D), delta_row=s[1], w=L.down, gate=mf[i, 2],
                         mod=(ma[i + 1, 0], ma[i + 1, 1]), q=q8(A, EX_D), s=s[0])
                else:
                    mfin = w.mod_final[step]
                    residual_norm_quant(self.dx, delta=raw(A, EX_D), delta_row=s[1], delta_col=L.down.scale,
                                        gate=mf[i, 2], mod_scale=mfin[0], mod_shift=mfin[1], y=self.dy)
                    note("norm", res=self.dx, delta=raw(A, EX_D), delta_row=s[1], w=L.down, gate=mf[i, 2],
                         mod=(mfin[0], mfin[1]), y=self.dy)
            self.x_t.addmm_(self.dy, self.out_w_dt).add_(self.out_b_dt)
        return self.x_t

    def _forward_tiled(self, noise=None):
        w, A = self.w, self.chunk
        raw, s = self.rawv, self.scale
        xq, oq, hq = self.xq, self.oq, self.hq
        if noise is not None:
            self.noise.copy_(noise)
        self.x_t.copy_(self.noise)
        qv = self.q16[:A].view(1, A, HEADS, HEAD_DIM)
        last = len(self.layers) - 1
        for step in range(w.steps):
            torch.addmm(w.action_in_b, self.x_t, self.in_w_t, out=self.dx)
            ma, mf = w.mod_attn[step], w.mod_ffn[step]
            residual_norm_quant(self.dx, mod_scale=ma[0, 0], mod_shift=ma[0, 1], q=xq, q_scale=s[0])
            for i, L in enumerate(self.layers):
                linear_qkv_rope(xq, s[0], L.qkv, self.q16[:A], self.kc[i], self.vc[i], inv_freq=self.inv_freq,
                                pos=self.pos_chunk, kv_base=self.prefix_len)
                attention(qv, self.kc[i][None], self.vc[i][None], kv_len=self.kv_len, scale=HEAD_DIM ** -0.5,
                          split=self.split, q8=oq, q8_scale=s[1])
                gemm(oq, L.o, raw(A, EX_D))
                residual_norm_quant(self.dx, delta=raw(A, EX_D), delta_row=s[1], delta_col=L.o.scale,
                                    gate=ma[i, 2], mod_scale=mf[i, 0], mod_shift=mf[i, 1], q=xq, q_scale=s[0])
                linear(xq, s[0], L.gate_up, out=raw(A, EX_FF), act="geglu")
                row_quant(raw(A, EX_FF), hq, s[1])
                gemm(hq, L.down, raw(A, EX_D))
                if i < last:
                    residual_norm_quant(self.dx, delta=raw(A, EX_D), delta_row=s[1], delta_col=L.down.scale,
                                        gate=mf[i, 2], mod_scale=ma[i + 1, 0], mod_shift=ma[i + 1, 1],
                                        q=xq, q_scale=s[0])
                else:
                    mfin = w.mod_final[step]
                    residual_norm_quant(self.dx, delta=raw(A, EX_D), delta_row=s[1], delta_col=L.down.scale,
                                        gate=mf[i, 2], mod_scale=mfin[0], mod_shift=mfin[1], y=self.dy)
            self.x_t.addmm_(self.dy, self.out_w_dt).add_(self.out_b_dt)
        return self.x_t

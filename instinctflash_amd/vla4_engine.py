"""The LingBot-VLA-4B forward on the gfx950 kernels: the Qwen2.5 text prefix over
the vision + prompt rows and the 36-layer flow-matching expert, one graph.

Mirrors instinctflash/engines/vla4/engine.py:
  * ``prefix`` (:114-139): the vision embeddings (from the model's own bf16 tower,
    an input here as upstream) and the prompt rows, RMS pre-norm to FP8 (the
    norm weights folded into the projections), per layer q|k|v (+ bias), QKV split
    with rotary into the layer's K/V cache, attention up to the device-side prefix
    length, o projection, residual + pre-norm, gate|up, SwiGLU requantization,
    down, residual + pre-norm; the last layer only fills the K/V cache;
  * ``expert`` (:141-177): per Euler step the suffix rows [state, 50 actions]
    (state projection, the action/time MLP, torch as upstream), AdaRMSNorm to
    FP8 (per-step scale / shift tables, no gates), per layer q|k|v (+ bias), QKV
    split into the cache rows after the prefix, attention over the layer's prefix
    K/V plus the suffix (the state row sees the prefix and itself, the actions
    everything: ``kv_extra``), o projection, residual + AdaRMSNorm, gate|up,
    SwiGLU requantization, down, residual + the next AdaRMSNorm or the final
    weight-form RMSNorm (float32 ``y``), then the Euler update.

``reference_calls=True`` makes exactly the reference's calls. The default lays
the same math out for gfx950: SwiGLU in the gate|up projections' epilogues
(GLU-packed weights, half-width bf16, requantized with ``quant_rows`` /
``row_quant``), and in the expert (51 rows) the pi05 expert's forms: weights in
the skinny tile layout, every FP8 activation written by its producer in that
layout, the QKV split in the QKV projection's epilogue (``linear_qkv_rope``) and
the attention's split-KV combine emitting the o projection's FP8 operand.
Weights are random with the published shapes (no checkpoint here).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .kernels import E4M3, Fp8Weight, SplitWorkspace, TiledRows, attention, gated_act_quant, gemm, linear, \
    linear_qkv_rope, pack_glu, pack_skinny, permute_rope_rows, quant_rows, quantize_weight, qkv_split, \
    residual_norm_quant, rope_inv_freq, row_quant
from .kernels.activation import SILU
from .kernels.attention import split_count

#: engines/vla4/engine.py:23-27
VISION_TOKENS = 192
D, FF, EX_D, EX_FF = 2048, 11008, 768, 2752
HQ, HKV, HD = 16, 2, 128
QKV_N = (HQ + 2 * HKV) * HD
STATE_DIM = 75


@dataclass
class Layer:
    qkv: Fp8Weight               # [QKV_N, width] + bias
    o: Fp8Weight | None          # None on the prefix's last layer
    gate_up: Fp8Weight | None    # [2 ff, width], gate rows then up rows
    down: Fp8Weight | None


@dataclass
class Vla4Weights:
    lm: list
    expert: list
    state_w: torch.Tensor        # [EX_D, STATE_DIM]
    state_b: torch.Tensor
    act_w: torch.Tensor          # [EX_D, STATE_DIM]
    act_c: torch.Tensor          # [steps, EX_D]
    mlp_out_w: torch.Tensor      # [EX_D, EX_D]
    mlp_out_b: torch.Tensor
    out_w: torch.Tensor          # [STATE_DIM, EX_D]
    out_b: torch.Tensor
    final_norm: torch.Tensor     # [EX_D]
    mod_attn: torch.Tensor       # [steps, layers, 2, EX_D] (scale, shift)
    mod_ffn: torch.Tensor
    dt: float

    @property
    def steps(self) -> int:
        return self.mod_attn.shape[0]


def random_vla4_weights(device, *, layers=36, steps=10, seed=0) -> Vla4Weights:
    """Random weights with LingBot-VLA-4B's shapes, drawn on the device: FP8
    projections N(0, 0.02) per output channel, q|k|v biases N(0, 0.01), small
    AdaRMSNorm tables (engines/vla4/weights.py:81-110)."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)

    def rn(*shape, s=1.0):
        return torch.randn(*shape, generator=g, device=dev) * s

    def lin(n, k, bias=False):
        return quantize_weight(rn(n, k, s=0.02).to(torch.bfloat16), rn(n, s=0.01) if bias else None, dev)

    lm = [Layer(lin(QKV_N, D, True), lin(D, HQ * HD), lin(2 * FF, D), lin(D, FF)) for _ in range(layers - 1)]
    lm.append(Layer(lin(QKV_N, D, True), None, None, None))
    ex = [Layer(lin(QKV_N, EX_D, True), lin(EX_D, HQ * HD), lin(2 * EX_FF, EX_D), lin(EX_D, EX_FF))
          for _ in range(layers)]
    return Vla4Weights(lm, ex, rn(EX_D, STATE_DIM, s=0.1), rn(EX_D, s=0.01), rn(EX_D, STATE_DIM, s=0.1),
                       rn(steps, EX_D, s=0.1), rn(EX_D, EX_D, s=EX_D ** -0.5), rn(EX_D, s=0.01),
                       rn(STATE_DIM, EX_D, s=0.02), rn(STATE_DIM, s=0.01), 1.0 + rn(EX_D, s=0.1),
                       rn(steps, layers, 2, EX_D, s=0.1).contiguous(), rn(steps, layers, 2, EX_D, s=0.1).contiguous(),
                       -1.0 / steps)


class Vla4Engine:
    """LingBot-VLA-4B over 192 vision rows, up to ``max_lang`` prompt rows (in
    buckets of ``bucket``) and a [state, 50 actions] suffix. Inputs: ``vis``
    [192, D], the prompt rows via ``set_prompt`` ([n, D] embeddings), ``state``
    [1, 75], ``noise`` [50, 75]; ``forward(M)`` leaves the actions in ``x_t``."""

    def __init__(self, weights: Vla4Weights, device, *, max_lang=72, chunk=50, bucket=16, reference_calls=False):
        self.w = weights
        self.dev = torch.device(device)
        self.chunk = int(chunk)
        self.S = self.chunk + 1
        self.max_lang = int(max_lang)
        self.bucket = int(bucket)
        self.reference_calls = bool(reference_calls)
        dev, f32, f16, bf16 = self.dev, torch.float32, torch.float16, torch.bfloat16
        lang_rows = -(-self.max_lang // self.bucket) * self.bucket
        self.smax = VISION_TOKENS + lang_rows
        rows = max(self.smax, self.S)
        self.vis = torch.zeros(VISION_TOKENS, D, dtype=f32, device=dev)
        self.lang = torch.zeros(lang_rows, D, dtype=f32, device=dev)
        self.state = torch.zeros(1, STATE_DIM, dtype=f32, device=dev)
        self.noise = torch.zeros(self.chunk, STATE_DIM, dtype=f32, device=dev)
        self.prefix_len = torch.zeros(1, dtype=torch.int32, device=dev)
        self.q8buf = torch.zeros(rows * FF, dtype=E4M3, device=dev)
        self.rawbuf = torch.zeros(rows * 2 * FF, dtype=bf16, device=dev)
        self.scale = [torch.zeros(rows, dtype=f32, device=dev) for _ in range(2)]
        self.px = torch.zeros(self.smax, D, dtype=f32, device=dev)
        self.q16 = torch.zeros(self.smax, HQ, HD, dtype=f16, device=dev)
        self.o16 = torch.zeros(self.smax, HQ * HD, dtype=f16, device=dev)
        self.kc = torch.zeros(len(weights.lm), self.smax + self.S, HKV, HD, dtype=f16, device=dev)
        self.vc = torch.zeros_like(self.kc)
        self.x_t = torch.zeros(self.chunk, STATE_DIM, dtype=f32, device=dev)
        self.dx = torch.zeros(self.S, EX_D, dtype=f32, device=dev)
        self.dy = torch.zeros(self.S, EX_D, dtype=f32, device=dev)
        self.hid = torch.zeros(self.chunk, EX_D, dtype=f32, device=dev)
        self.state_emb = torch.zeros(1, EX_D, dtype=f32, device=dev)
        self.inv_freq = rope_inv_freq(HD, 10000.0, dev)
        self.pos_prefix = torch.arange(self.smax, dtype=f32, device=dev)[:, None].contiguous()
        self.pos_suffix = torch.zeros(self.S, 1, dtype=f32, device=dev)
        # suffix keys past the prefix: the state row sees itself, the actions all S
        self.kv_extra = torch.full((self.S,), self.S, dtype=torch.int32, device=dev)
        self.kv_extra[0] = 1
        self.act_w_t = weights.act_w.t().contiguous()
        self.mlp_out_w_t = weights.mlp_out_w.t().contiguous()
        self.state_w_t = weights.state_w.t().contiguous()
        self.out_w_dt = (weights.out_w * weights.dt).t().contiguous()
        self.out_b_dt = (weights.out_b * weights.dt).contiguous()
        glu = (lambda L: L) if self.reference_calls else (
            lambda L: Layer(L.qkv, L.o, None if L.gate_up is None else pack_glu(L.gate_up), L.down))
        self.lm = [glu(L) for L in weights.lm]
        self.ex = [glu(L) for L in weights.expert]
        self.h = torch.zeros(rows * FF, dtype=bf16, device=dev)
        self.rows = None
        if not self.reference_calls:
            from . import _lib
            lib = _lib.load()
            S = self.S
            tiled = lambda k: TiledRows(torch.zeros(lib.ifx_quant_rows_tiled_bytes(S, k), dtype=E4M3,  # noqa: E731
                                                    device=dev), S, k)
            self.xq, self.oq, self.hq = tiled(EX_D), tiled(HQ * HD), tiled(EX_FF)
            self.ex_tiled = [Layer(pack_skinny(permute_rope_rows(L.qkv, HQ, HKV, HD)), pack_skinny(L.o),
                                   pack_skinny(pack_glu(L.gate_up)), pack_skinny(L.down)) for L in weights.expert]
            splits = max(2, split_count(1, S, HQ, HKV, self.smax + S))
            self.split = SplitWorkspace(1, S, HQ, HKV, HD, splits, dev)

    def q8(self, rows, cols):
        return self.q8buf[: rows * cols].view(rows, cols)

    def raw(self, rows, cols):
        return self.rawbuf[: rows * cols].view(rows, cols)

    def set_prompt(self, lang_rows: torch.Tensor):
        """engines/vla4/engine.py:85-98 after the token-embedding lookup; returns
        the bucketed prefix row count."""
        n = int(lang_rows.shape[0])
        if not 1 <= n <= self.max_lang:
            raise ValueError(f"1..{self.max_lang} prompt rows supported, got {n}")
        self.lang[:n].copy_(lang_rows)
        self.lang[n:].zero_()
        p = VISION_TOKENS + n
        self.prefix_len.fill_(p)
        torch.arange(p, p + self.S, out=self.pos_suffix[:, 0])
        self.rows = VISION_TOKENS + -(-n // self.bucket) * self.bucket
        return self.rows

    def forward(self, M=None, on_call=None):
        M = self.rows if M is None else int(M)
        if M is None or not VISION_TOKENS < M <= self.smax:
            raise ValueError("set_prompt first (or M out of range)")
        if on_call is not None and not self.reference_calls:
            raise ValueError("on_call needs reference_calls=True")
        note = on_call or (lambda name, **t: None)
        self.prefix(M)
        if self.reference_calls:
            self.expert(note)
        else:
            self.expert_tiled()
        return self.x_t

    def _mlp(self, note, L, rows, width, ff, x_s, ref=None):
        """gate|up + SwiGLU requantization into q8(rows, ff) / scale[1]; ``ref``:
        the layer in the reference layout (the per-call notes carry its weight)."""
        ref = ref or L
        q8, raw, s1 = self.q8, self.raw, self.scale[1][:rows]
        if self.reference_calls:
            gemm(q8(rows, width), L.gate_up, raw(rows, 2 * ff))
            note("gemm", a=q8(rows, width), w=ref.gate_up, out=raw(rows, 2 * ff))
            gated_act_quant(raw(rows, 2 * ff), q8(rows, ff), s1, row=x_s, col=L.gate_up.scale, act=SILU)
            note("gated_act_quant", gu=raw(rows, 2 * ff), row=x_s, w=ref.gate_up, q=q8(rows, ff), s=s1)
        else:
            h = self.h[: rows * ff].view(rows, ff)
            linear(q8(rows, width), x_s, L.gate_up, out=h, act="swiglu")
            note("swiglu", a=q8(rows, width), sa=x_s, w=ref.gate_up, out=h)
            quant_rows(h, q8(rows, ff), s1)
            note("row_quant", x=h, q=q8(rows, ff), s=s1)

    def prefix(self, M):
        q8, raw = self.q8, self.raw
        s = [v[:M] for v in self.scale]
        V = VISION_TOKENS
        self.px[:V].copy_(self.vis)
        self.px[V:M].copy_(self.lang[: M - V])
        residual_norm_quant(self.px[:M], q=q8(M, D), q_scale=s[0])
        qv = self.q16[:M].view(1, M, HQ, HD)
        none = lambda name, **t: None  # noqa: E731
        for i, L in enumerate(self.lm):
            gemm(q8(M, D), L.qkv, raw(M, QKV_N))
            qkv_split(raw(M, QKV_N), self.q16[:M], self.kc[i], self.vc[i], heads_q=HQ, heads_kv=HKV, head_dim=HD,
                      row=s[0], col=L.qkv.scale, bias=L.qkv.bias, inv_freq=self.inv_freq, pos=self.pos_prefix[:M])
            if L.o is None:
                break
            attention(qv, self.kc[i][None], self.vc[i][None], out=self.o16[:M].view(1, M, HQ, HD),
                      kv_len=self.prefix_len)
            row_quant(self.o16[:M], q8(M, HQ * HD), s[1])
            gemm(q8(M, HQ * HD), L.o, raw(M, D))
            residual_norm_quant(self.px[:M], delta=raw(M, D), delta_row=s[1], delta_col=L.o.scale, q=q8(M, D),
                                q_scale=s[0])
            self._mlp(none, L, M, D, FF, s[0])
            gemm(q8(M, FF), L.down, raw(M, D))
            residual_norm_quant(self.px[:M], delta=raw(M, D), delta_row=s[1], delta_col=L.down.scale, q=q8(M, D),
                                q_scale=s[0])

    def expert(self, note=None):
        note = note or (lambda name, **t: None)
        w, q8, raw, S = self.w, self.q8, self.raw, self.S
        s = [v[:S] for v in self.scale]
        torch.addmm(w.state_b, self.state, self.state_w_t, out=self.state_emb)
        self.x_t.copy_(self.noise)
        qv = self.q16[:S].view(1, S, HQ, HD)
        ov = self.o16[:S].view(1, S, HQ, HD)
        last = len(self.ex) - 1
        for step in range(w.steps):
            ma, mf = w.mod_attn[step], w.mod_ffn[step]
            self.dx[:1].copy_(self.state_emb)
            torch.addmm(w.act_c[step], self.x_t, self.act_w_t, out=self.hid)
            torch.nn.functional.silu(self.hid, inplace=True)
            torch.addmm(w.mlp_out_b, self.hid, self.mlp_out_w_t, out=self.dx[1:])
            note("pre_res", res=self.dx)
            residual_norm_quant(self.dx, mod_scale=ma[0, 0], mod_shift=ma[0, 1], q=q8(S, EX_D), q_scale=s[0])
            note("norm", res=self.dx, mod=(ma[0, 0], ma[0, 1]), q=q8(S, EX_D), s=s[0])
            for i, L in enumerate(self.ex):
                gemm(q8(S, EX_D), L.qkv, raw(S, QKV_N))
                note("gemm", a=q8(S, EX_D), w=L.qkv, out=raw(S, QKV_N))
                qkv_split(raw(S, QKV_N), self.q16[:S], self.kc[i], self.vc[i], heads_q=HQ, heads_kv=HKV, head_dim=HD,
                          row=s[0], col=L.qkv.scale, bias=L.qkv.bias, inv_freq=self.inv_freq, pos=self.pos_suffix,
                          kv_base=self.prefix_len)
                note("qkv_split", raw=raw(S, QKV_N), row=s[0], w=L.qkv, q=self.q16[:S], k=self.kc[i], v=self.vc[i])
                attention(qv, self.kc[i][None], self.vc[i][None], out=ov, kv_len=self.prefix_len,
                          kv_extra=self.kv_extra, max_extra=S)
                note("attention", q=qv, k=self.kc[i][None], v=self.vc[i][None], out=ov)
                row_quant(self.o16[:S], q8(S, HQ * HD), s[1])
                note("row_quant", x=self.o16[:S], q=q8(S, HQ * HD), s=s[1])
                gemm(q8(S, HQ * HD), L.o, raw(S, EX_D))
                note("gemm", a=q8(S, HQ * HD), w=L.o, out=raw(S, EX_D))
                note("pre_res", res=self.dx)
                residual_norm_quant(self.dx, delta=raw(S, EX_D), delta_row=s[1], delta_col=L.o.scale,
                                    mod_scale=mf[i, 0], mod_shift=mf[i, 1], q=q8(S, EX_D), q_scale=s[0])
                note("norm", res=self.dx, delta=raw(S, EX_D), delta_row=s[1], w=L.o, mod=(mf[i, 0], mf[i, 1]),
                     q=q8(S, EX_D), s=s[0])
                self._mlp(note, L, S, EX_D, EX_FF, s[0], ref=w.expert[i])
                gemm(q8(S, EX_FF), L.down, raw(S, EX_D))
                note("gemm", a=q8(S, EX_FF), w=L.down, out=raw(S, EX_D))
                note("pre_res", res=self.dx)
                if i < last:
                    residual_norm_quant(self.dx, delta=raw(S, EX_D), delta_row=s[1], delta_col=L.down.scale,
                                        mod_scale=ma[i + 1, 0], mod_shift=ma[i + 1, 1], q=q8(S, EX_D), q_scale=s[0])
                    note("norm", res=self.dx, delta=raw(S, EX_D), delta_row=s[1], w=L.down,
                         mod=(ma[i + 1, 0], ma[i + 1, 1]), q=q8(S, EX_D), s=s[0])
                else:
                    residual_norm_quant(self.dx, delta=raw(S, EX_D), delta_row=s[1], delta_col=L.down.scale,
                                        weight=w.final_norm, y=self.dy)
                    note("norm", res=self.dx, delta=raw(S, EX_D), delta_row=s[1], w=L.down, weight=w.final_norm,
                         y=self.dy)
            self.x_t.addmm_(self.dy[1:], self.out_w_dt).add_(self.out_b_dt)

    def expert_tiled(self):
        """The expert in the gfx950 layout (same math as ``expert``)."""
        w, raw, S = self.w, self.raw, self.S
        s = [v[:S] for v in self.scale]
        xq, oq, hq = self.xq, self.oq, self.hq
        torch.addmm(w.state_b, self.state, self.state_w_t, out=self.state_emb)
        self.x_t.copy_(self.noise)
        qv = self.q16[:S].view(1, S, HQ, HD)
        last = len(self.ex_tiled) - 1
        for step in range(w.steps):
            ma, mf = w.mod_attn[step], w.mod_ffn[step]
            self.dx[:1].copy_(self.state_emb)
            torch.addmm(w.act_c[step], self.x_t, self.act_w_t, out=self.hid)
            torch.nn.functional.silu(self.hid, inplace=True)
            torch.addmm(w.mlp_out_b, self.hid, self.mlp_out_w_t, out=self.dx[1:])
            residual_norm_quant(self.dx, mod_scale=ma[0, 0], mod_shift=ma[0, 1], q=xq, q_scale=s[0])
            for i, L in enumerate(self.ex_tiled):
                linear_qkv_rope(xq, s[0], L.qkv, self.q16[:S], self.kc[i], self.vc[i], inv_freq=self.inv_freq,
                                pos=self.pos_suffix, kv_base=self.prefix_len)
                attention(qv, self.kc[i][None], self.vc[i][None], kv_len=self.prefix_len, kv_extra=self.kv_extra,
                          max_extra=S, split=self.split, q8=oq, q8_scale=s[1])
                gemm(oq, L.o, raw(S, EX_D))
                residual_norm_quant(self.dx, delta=raw(S, EX_D), delta_row=s[1], delta_col=L.o.scale,
                                    mod_scale=mf[i, 0], mod_shift=mf[i, 1], q=xq, q_scale=s[0])
                linear(xq, s[0], L.gate_up, out=raw(S, EX_FF), act="swiglu")
                row_quant(raw(S, EX_FF), hq, s[1])
                gemm(hq, L.down, raw(S, EX_D))
                if i < last:
                    residual_norm_quant(self.dx, delta=raw(S, EX_D), delta_row=s[1], delta_col=L.down.scale,
                                        mod_scale=ma[i + 1, 0], mod_shift=ma[i + 1, 1], q=xq, q_scale=s[0])
                else:
                    residual_norm_quant(self.dx, delta=raw(S, EX_D), delta_row=s[1], delta_col=L.down.scale,
                                        weight=w.final_norm, y=self.dy)
            self.x_t.addmm_(self.dy[1:], self.out_w_dt).add_(self.out_b_dt)

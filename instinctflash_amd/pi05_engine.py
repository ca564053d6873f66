"""The whole pi05 forward on the gfx950 kernels: SigLIP vision tower, Gemma-2B
prefix, Gemma-300M flow-matching expert, captured as one graph.

Mirrors instinctflash/engines/pi05/engine.py:
  * ``vision`` (:157-190): the 14 x 14 patch embedding as one fp16 matmul over the
    reshaped pixels plus position embeddings (torch, as upstream), then per
    SigLIP layer: LayerNorm to FP8, q|k|v projection, rescale + bias to fp16,
    attention over each view's 256 patches, FP8 of its output, o projection,
    residual + LayerNorm, fc1 with GELU and requantization, fc2, residual + the
    next LayerNorm (the post-LayerNorm after the last layer); the projector into
    the float32 prefix rows;
  * ``prefix`` (:192-216): the language rows after the image rows, RMS pre-norm
    to FP8, per layer q|k|v, QKV split with rotary into the K/V cache, attention
    up to the device-side prefix length, o projection, residual + pre-norm,
    gate|up, GeGLU requantization, down, residual + pre-norm; the last layer
    only fills the K/V cache (its o / MLP weights are absent, as the
    reference loads them);
  * the expert's Euler steps over that cache (``Pi05Expert``, :218-245).

The prompt length lives in device memory (``set_prompt``), so one captured graph
per physical row count serves every prompt of that bucket. ``reference_calls``
selects the reference's exact call sequence (raw accumulators rescaled by
``dequant_rows``, GELU / GeGLU requantization of raw accumulators); the default
writes the rescaled q|k|v (fp16) and projector rows (float32) from the GEMM
epilogue, applies GELU / GeGLU in the fc1 / gate|up epilogues, and runs the
expert in its tile layouts (``Pi05Expert``). Weights are random with the published shapes
(no checkpoint here); ``random_pi05_weights`` draws them on the device.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .kernels import E4M3, Fp8Weight, attention, dequant_rows, gated_act_quant, gemm, linear, pack_glu, \
    quant_rows, quantize_weight, qkv_split, residual_norm_quant, rope_inv_freq, row_quant
from .kernels.activation import GELU_TANH
from .pi05 import ACTION_DIM, EX_D, EX_FF, HEAD_DIM, HEADS, QKV_N, ExpertLayer, ExpertWeights, Pi05Expert

#: engines/pi05/engine.py:25-29
VISION_TOKENS = 256
VIS_D, VIS_HEADS, VIS_HD, VIS_FF = 1152, 16, 72, 4304
LM_D, LM_FF = 2048, 16384
PATCH = 14
LN_EPS = 1e-6


@dataclass
class VisionLayer:
    ln1_w: torch.Tensor
    ln1_b: torch.Tensor
    qkv: Fp8Weight       # [3 VIS_D, VIS_D] + bias
    o: Fp8Weight
    ln2_w: torch.Tensor
    ln2_b: torch.Tensor
    fc1: Fp8Weight       # [VIS_FF, VIS_D] + bias
    fc2: Fp8Weight       # [VIS_D, VIS_FF] + bias


@dataclass
class PrefixLayer:
    qkv: Fp8Weight               # [QKV_N, LM_D]
    o: Fp8Weight | None          # None on the last layer (it only fills the K/V cache)
    gate_up: Fp8Weight | None    # [2 LM_FF, LM_D], gate rows then up rows
    down: Fp8Weight | None


@dataclass
class Pi05Weights:
    patch_w: torch.Tensor        # [VIS_D, 3, 14, 14]
    patch_b: torch.Tensor
    pos_emb: torch.Tensor        # [VISION_TOKENS, VIS_D]
    vision: list
    post_ln_w: torch.Tensor
    post_ln_b: torch.Tensor
    projector: Fp8Weight         # [LM_D, VIS_D] + bias
    prefix: list
    expert: ExpertWeights


def random_pi05_weights(device, *, vision_layers=27, prefix_layers=18, expert_layers=18, steps=10,
                        seed=0) -> Pi05Weights:
    """Random weights with pi05's shapes, drawn on the device (the full model has
    ~2.5 G projection parameters): FP8 projections N(0, 0.02) quantized per output
    channel, biases N(0, 0.01), LayerNorm weights 1 + N(0, 0.1)."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)

    def rn(*shape, s=1.0):
        return torch.randn(*shape, generator=g, device=dev) * s

    def lin(n, k, bias=False):
        return quantize_weight(rn(n, k, s=0.02).to(torch.bfloat16), rn(n, s=0.01) if bias else None, dev)

    vision = [VisionLayer(1.0 + rn(VIS_D, s=0.1), rn(VIS_D, s=0.05), lin(3 * VIS_D, VIS_D, True),
                          lin(VIS_D, VIS_D, True), 1.0 + rn(VIS_D, s=0.1), rn(VIS_D, s=0.05),
                          lin(VIS_FF, VIS_D, True), lin(VIS_D, VIS_FF, True)) for _ in range(vision_layers)]
    prefix = [PrefixLayer(lin(QKV_N, LM_D), lin(LM_D, HEADS * HEAD_DIM), lin(2 * LM_FF, LM_D), lin(LM_D, LM_FF))
              for _ in range(prefix_layers - 1)]
    prefix.append(PrefixLayer(lin(QKV_N, LM_D), None, None, None))
    ls = [ExpertLayer(lin(QKV_N, EX_D), lin(EX_D, HEADS * HEAD_DIM), lin(2 * EX_FF, EX_D), lin(EX_D, EX_FF))
          for _ in range(expert_layers)]
    gate = lambda *s: torch.rand(*s, generator=g, device=dev) * 0.5 + 0.5  # noqa: E731
    ma = torch.cat([rn(steps, expert_layers, 2, EX_D, s=0.1), gate(steps, expert_layers, 1, EX_D)], 2).contiguous()
    mf = torch.cat([rn(steps, expert_layers, 2, EX_D, s=0.1), gate(steps, expert_layers, 1, EX_D)], 2).contiguous()
    expert = ExpertWeights(ls, ma, mf, rn(steps, 2, EX_D, s=0.1).contiguous(), rn(EX_D, ACTION_DIM, s=0.2),
                           rn(EX_D, s=0.01), rn(ACTION_DIM, EX_D, s=0.02), rn(ACTION_DIM, s=0.01))
    return Pi05Weights(rn(VIS_D, 3, PATCH, PATCH, s=0.02), rn(VIS_D, s=0.01), rn(VISION_TOKENS, VIS_D, s=0.02),
                       vision, 1.0 + rn(VIS_D, s=0.1), rn(VIS_D, s=0.05), lin(LM_D, VIS_D, True), prefix, expert)


class Pi05Engine:
    """pi05 over ``num_views`` 224 x 224 images, up to ``max_prompt`` language
    rows (in buckets of ``bucket``) and a 50-action chunk. Inputs: ``img``
    [V, 3, 224, 224] float32, the language rows via ``set_prompt`` (token
    embeddings, [n, LM_D]), ``noise`` [chunk, 32]; ``forward(M)`` (M = the
    bucketed prefix row count, ``rows``) leaves the actions in ``x_t``."""

    def __init__(self, weights: Pi05Weights, num_views, device, *, max_prompt=256, chunk=50, bucket=16,
                 reference_calls=False):
        self.w = weights
        self.V = int(num_views)
        self.dev = torch.device(device)
        self.bucket = int(bucket)
        self.max_prompt = int(max_prompt)
        self.reference_calls = bool(reference_calls)
        T = self.T = self.V * VISION_TOKENS
        self.smax = T + -(-self.max_prompt // self.bucket) * self.bucket
        dev, f32, f16, bf16 = self.dev, torch.float32, torch.float16, torch.bfloat16
        rows = max(self.smax, T)
        self.img = torch.zeros(self.V, 3, 224, 224, dtype=f32, device=dev)
        self.lang = torch.zeros(self.max_prompt + self.bucket, LM_D, dtype=f32, device=dev)
        self.q8buf = torch.zeros(rows * LM_FF, dtype=E4M3, device=dev)
        self.rawbuf = torch.zeros(rows * 2 * LM_FF, dtype=bf16, device=dev)
        self.scale = [torch.zeros(rows, dtype=f32, device=dev) for _ in range(2)]
        self.vx = torch.zeros(T, VIS_D, dtype=f32, device=dev)
        self.vqkv = torch.zeros(T, 3 * VIS_D, dtype=f16, device=dev)
        self.vo = torch.zeros(T, VIS_D, dtype=f16, device=dev)
        self.patch_w = weights.patch_w.reshape(VIS_D, -1).t().contiguous().to(f16)  # [588, VIS_D]
        self.px = torch.zeros(self.smax, LM_D, dtype=f32, device=dev)
        self.pq16 = torch.zeros(self.smax, HEADS, HEAD_DIM, dtype=f16, device=dev)
        self.po16 = torch.zeros(self.smax, HEADS * HEAD_DIM, dtype=f16, device=dev)
        self.ph = torch.zeros(self.smax * LM_FF, dtype=bf16, device=dev)
        self.pos_prefix = torch.arange(self.smax, dtype=f32, device=dev)[:, None].contiguous()
        self.inv_freq = rope_inv_freq(HEAD_DIM, 10000.0, dev)
        self.prefix_layers = weights.prefix if self.reference_calls else [
            PrefixLayer(L.qkv, L.o, None if L.gate_up is None else pack_glu(L.gate_up), L.down)
            for L in weights.prefix]
        # the expert owns the K/V cache [layers, smax + chunk, 1, HEAD_DIM] and the
        # device prefix length; the prefix stage fills the cache's first rows
        self.expert = Pi05Expert(weights.expert, dev, smax=self.smax, chunk=chunk, reference_calls=reference_calls)
        if len(weights.prefix) != len(weights.expert.layers):
            raise ValueError("prefix and expert need the same layer count (one K/V cache per layer)")
        self.rows = None

    def q8(self, rows, cols):
        return self.q8buf[: rows * cols].view(rows, cols)

    def raw(self, rows, cols):
        return self.rawbuf[: rows * cols].view(rows, cols)

    @property
    def x_t(self):
        return self.expert.x_t

    def set_prompt(self, lang_rows: torch.Tensor):
        """engines/pi05/engine.py:98-110 after the token-embedding lookup:
        ``lang_rows`` [n, LM_D] (the scaled embeddings). Sets the device prefix
        length (image rows + n) and returns the bucketed row count."""
        n = int(lang_rows.shape[0])
        if not 1 <= n <= self.max_prompt:
            raise ValueError(f"1..{self.max_prompt} prompt rows supported, got {n}")
        self.lang[:n].copy_(lang_rows)
        self.lang[n:].zero_()
        self.expert.set_prefix(self.T + n)
        self.rows = self.T + -(-n // self.bucket) * self.bucket
        return self.rows

    def forward(self, M=None, on_call=None):
        """engines/pi05/engine.py:151-155 (`_forward`); ``on_call`` receives the
        vision stage's calls (for per-call parity tests)."""
        M = self.rows if M is None else int(M)
        if M is None or not self.T < M <= self.smax:
            raise ValueError("set_prompt first (or M out of range)")
        self.vision(on_call)
        self.prefix(M)
        return self.expert.forward()

    def vision(self, on_call=None):
        note = on_call or (lambda name, **t: None)
        w, V, T = self.w, self.V, self.T
        q8, raw = self.q8, self.raw
        s = [v[:T] for v in self.scale]
        pix = self.img.view(V, 3, 16, PATCH, 16, PATCH).permute(0, 2, 4, 1, 3, 5).reshape(T, 3 * PATCH * PATCH)
        self.vx.copy_(torch.mm(pix.to(torch.float16), self.patch_w)).add_(w.patch_b)
        self.vx.view(V, VISION_TOKENS, VIS_D).add_(w.pos_emb)
        L0 = w.vision[0]
        note("pre_res", res=self.vx)
        residual_norm_quant(self.vx, layernorm=True, weight=L0.ln1_w, beta=L0.ln1_b, q=q8(T, VIS_D), q_scale=s[0])
        note("norm", res=self.vx, weight=L0.ln1_w, beta=L0.ln1_b, q=q8(T, VIS_D), s=s[0])
        view = (V, VISION_TOKENS, VIS_HEADS, VIS_HD)
        for i, L in enumerate(w.vision):
            if self.reference_calls:
                gemm(q8(T, VIS_D), L.qkv, raw(T, 3 * VIS_D))
                note("gemm", a=q8(T, VIS_D), w=L.qkv, out=raw(T, 3 * VIS_D))
                dequant_rows(raw(T, 3 * VIS_D), self.vqkv, row=s[0], col=L.qkv.scale, bias=L.qkv.bias)
                note("dequant", x=raw(T, 3 * VIS_D), y=self.vqkv, row=s[0], w=L.qkv)
            else:  # rescaled fp16 rows straight from the epilogue
                linear(q8(T, VIS_D), s[0], L.qkv, out=self.vqkv)
                note("qkv16", a=q8(T, VIS_D), sa=s[0], w=L.qkv, out=self.vqkv)
            qkv = self.vqkv.view(V, VISION_TOKENS, 3, VIS_HEADS, VIS_HD)
            attention(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], out=self.vo.view(view), scale=VIS_HD ** -0.5)
            note("attention", q=qkv[:, :, 0], k=qkv[:, :, 1], v=qkv[:, :, 2], out=self.vo.view(view))
            row_quant(self.vo, q8(T, VIS_D), s[1])
            note("row_quant", x=self.vo, q=q8(T, VIS_D), s=s[1])
            gemm(q8(T, VIS_D), L.o, raw(T, VIS_D))
            note("gemm", a=q8(T, VIS_D), w=L.o, out=raw(T, VIS_D))
            note("pre_res", res=self.vx)
            residual_norm_quant(self.vx, delta=raw(T, VIS_D), delta_row=s[1], delta_col=L.o.scale, bias=L.o.bias,
                                layernorm=True, weight=L.ln2_w, beta=L.ln2_b, q=q8(T, VIS_D), q_scale=s[0])
            note("norm", res=self.vx, delta=raw(T, VIS_D), delta_row=s[1], w=L.o, weight=L.ln2_w, beta=L.ln2_b,
                 q=q8(T, VIS_D), s=s[0])
            if self.reference_calls:
                gemm(q8(T, VIS_D), L.fc1, raw(T, VIS_FF))
                note("gemm", a=q8(T, VIS_D), w=L.fc1, out=raw(T, VIS_FF))
                row_quant(raw(T, VIS_FF), q8(T, VIS_FF), s[1], row=s[0], col=L.fc1.scale, bias=L.fc1.bias, gelu=True)
                note("fc1_quant", x=raw(T, VIS_FF), row=s[0], w=L.fc1, q=q8(T, VIS_FF), s=s[1])
            else:
                h = raw(T, VIS_FF)
                linear(q8(T, VIS_D), s[0], L.fc1, out=h, act="gelu_tanh")
                note("fc1", a=q8(T, VIS_D), sa=s[0], w=L.fc1, out=h)
                quant_rows(h, q8(T, VIS_FF), s[1])
                note("row_quant", x=h, q=q8(T, VIS_FF), s=s[1])
            gemm(q8(T, VIS_FF), L.fc2, raw(T, VIS_D))
            note("gemm", a=q8(T, VIS_FF), w=L.fc2, out=raw(T, VIS_D))
            nxt = w.vision[i + 1] if i + 1 < len(w.vision) else None
            note("pre_res", res=self.vx)
            residual_norm_quant(self.vx, delta=raw(T, VIS_D), delta_row=s[1], delta_col=L.fc2.scale, bias=L.fc2.bias,
                                layernorm=True, weight=nxt.ln1_w if nxt else w.post_ln_w,
                                beta=nxt.ln1_b if nxt else w.post_ln_b, q=q8(T, VIS_D), q_scale=s[0])
            note("norm", res=self.vx, delta=raw(T, VIS_D), delta_row=s[1], w=L.fc2,
                 weight=nxt.ln1_w if nxt else w.post_ln_w, beta=nxt.ln1_b if nxt else w.post_ln_b,
                 q=q8(T, VIS_D), s=s[0])
        if self.reference_calls:
            gemm(q8(T, VIS_D), w.projector, raw(T, LM_D))
            note("gemm", a=q8(T, VIS_D), w=w.projector, out=raw(T, LM_D))
            dequant_rows(raw(T, LM_D), self.px[:T], row=s[0], col=w.projector.scale, bias=w.projector.bias)
            note("dequant", x=raw(T, LM_D), y=self.px[:T], row=s[0], w=w.projector)
        else:  # float32 prefix rows straight from the epilogue
            linear(q8(T, VIS_D), s[0], w.projector, out=self.px[:T])
            note("projector", a=q8(T, VIS_D), sa=s[0], w=w.projector, out=self.px[:T])

    def prefix(self, M):
        """engines/pi05/engine.py:192-216 over M rows (image rows, then the
        bucketed language rows); the K/V cache goes to the expert's ``kc`` / ``vc``."""
        T = self.T
        q8, raw = self.q8, self.raw
        s = [v[:M] for v in self.scale]
        kc, vc = self.expert.kc, self.expert.vc
        self.px[T:M].copy_(self.lang[: M - T])
        residual_norm_quant(self.px[:M], q=q8(M, LM_D), q_scale=s[0])
        qv = self.pq16[:M].view(1, M, HEADS, HEAD_DIM)
        for i, L in enumerate(self.prefix_layers):
            gemm(q8(M, LM_D), L.qkv, raw(M, QKV_N))
            qkv_split(raw(M, QKV_N), self.pq16[:M], kc[i], vc[i], heads_q=HEADS, heads_kv=1, head_dim=HEAD_DIM,
                      inv_freq=self.inv_freq, pos=self.pos_prefix[:M], row=s[0], col=L.qkv.scale)
            if L.o is None:
                break
            attention(qv, kc[i][None], vc[i][None], out=self.po16[:M].view(1, M, HEADS, HEAD_DIM),
                      kv_len=self.expert.prefix_len, scale=HEAD_DIM ** -0.5)
            row_quant(self.po16[:M], q8(M, LM_D), s[1])
            gemm(q8(M, LM_D), L.o, raw(M, LM_D))
            residual_norm_quant(self.px[:M], delta=raw(M, LM_D), delta_row=s[1], delta_col=L.o.scale,
                                q=q8(M, LM_D), q_scale=s[0])
            if self.reference_calls:
                gemm(q8(M, LM_D), L.gate_up, raw(M, 2 * LM_FF))
                gated_act_quant(raw(M, 2 * LM_FF), q8(M, LM_FF), s[1], row=s[0], col=L.gate_up.scale, act=GELU_TANH)
            else:
                h = self.ph[: M * LM_FF].view(M, LM_FF)
                linear(q8(M, LM_D), s[0], L.gate_up, out=h, act="geglu")
                quant_rows(h, q8(M, LM_FF), s[1])
            gemm(q8(M, LM_FF), L.down, raw(M, LM_D))
            residual_norm_quant(self.px[:M], delta=raw(M, LM_D), delta_row=s[1], delta_col=L.down.scale,
                                q=q8(M, LM_D), q_scale=s[0])

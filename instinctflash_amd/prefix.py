"""The prefix (language-model) stacks of the pi05 and LingBot-VLA-4B engines on
the gfx950 kernels: the call sites that define configs C3 (pi05 PaliGemma
prefix MLP, M = 816) and C4 (VLA4 Qwen2.5 decoder layer, M = 1024).

Both reference stages run the same decoder loop (instinctflash/engines/pi05/
engine.py:192-216 `_prefix`, instinctflash/engines/vla4/engine.py:114-139
`_prefix`): RMS pre-norm of the prefix rows to per-token FP8, then per layer
  * the fused q|k|v projection (``gemm``), the QKV split with rotary into the
    K/V cache (``qkv_split``; VLA4 with a q|k|v bias);
  * bidirectional attention of the prefix over itself up to the device-side
    prefix length, the per-token FP8 of its output (``row_quant``), the output
    projection and the residual update + next pre-norm (``residual_norm_quant``);
  * the gate|up projection, GeGLU (pi05) or SwiGLU (VLA4) with the per-token
    requantization (``gated_act_quant``), the down projection and the residual
    update + next pre-norm.
The two models differ only in their shapes, the activation and the q|k|v bias
(``PrefixConfig``).

``reference_calls=True`` makes exactly the reference's calls. The default lays
the MLP out for gfx950: the gate|up weight is GLU-packed and the activation is
applied in the projection's epilogue (half-width bf16 result, ``linear(...,
act=)``), then ``quant_rows`` requantizes it -- the full-width raw accumulator
never goes to HBM. Weights are random (no checkpoint here) with the published
architectures' shapes; ``on_call`` (optional) is called after every kernel with
its name and the buffers it read and wrote, for the per-call parity tests.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .kernels import E4M3, Fp8Weight, attention, gated_act_quant, gemm, linear, pack_glu, qkv_split, quant_rows, \
    quantize_weight, residual_norm_quant, rope_inv_freq, row_quant
from .kernels.activation import GELU_TANH, SILU


@dataclass(frozen=True)
class PrefixConfig:
    name: str
    D: int          # model width
    FF: int         # MLP width (gate|up has 2 * FF rows)
    HQ: int         # query heads
    HKV: int        # key/value heads
    HD: int         # head dim
    act: str        # "geglu" (GELU-tanh gate) or "swiglu" (SiLU gate)
    qkv_bias: bool
    rope_theta: float = 10000.0

    @property
    def qkv_n(self) -> int:
        return (self.HQ + 2 * self.HKV) * self.HD


#: pi05's PaliGemma (Gemma-2B) prefix: engines/pi05/engine.py LM_D / LM_FF / HEADS / HEAD_DIM
PI05_PREFIX = PrefixConfig("pi05 PaliGemma prefix", 2048, 16384, 8, 1, 256, "geglu", False)
#: LingBot-VLA-4B's Qwen2.5 backbone: engines/vla4/engine.py D / FF / HQ / HKV / HD
VLA4_PREFIX = PrefixConfig("LingBot-VLA-4B Qwen2.5 prefix", 2048, 11008, 16, 2, 128, "swiglu", True)


@dataclass
class PrefixLayer:
    qkv: Fp8Weight      # [(HQ + 2 HKV) HD, D] (+ bias for VLA4)
    o: Fp8Weight        # [D, HQ HD]
    gate_up: Fp8Weight  # [2 FF, D], gate rows then up rows (reference layout)
    down: Fp8Weight     # [D, FF]


def random_prefix_weights(cfg: PrefixConfig, layers: int, device, seed=0) -> list:
    """Random weights of the stack (N(0, 0.02) projections, q|k|v bias N(0, 0.01)
    for VLA4), quantized per output channel on the device."""
    g = torch.Generator().manual_seed(seed)

    def lin(n, k, bias=False):
        w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
        b = torch.randn(n, generator=g) * 0.01 if bias else None
        return quantize_weight(w.to(device), b, device)

    return [PrefixLayer(lin(cfg.qkv_n, cfg.D, cfg.qkv_bias), lin(cfg.D, cfg.HQ * cfg.HD), lin(2 * cfg.FF, cfg.D),
                        lin(cfg.D, cfg.FF)) for _ in range(layers)]


class PrefixStack:
    """The prefix stage over ``M`` rows (<= smax): ``forward(x, M)`` runs every
    layer on the fp32 residual stream ``px`` (initialised from x [M, D]) and
    fills the K/V caches ``kc`` / ``vc`` [layers, smax, HKV, HD] (fp16) that the
    action expert reads. The prefix length the attention uses lives in device
    memory (``set_prefix``), so a captured graph follows it."""

    def __init__(self, cfg: PrefixConfig, layers: list, device, *, smax=1024, reference_calls=False):
        self.cfg, self.layers_ref = cfg, layers
        self.reference_calls = bool(reference_calls)
        self.dev = torch.device(device)
        self.smax = int(smax)
        dev, f32, f16, bf16 = self.dev, torch.float32, torch.float16, torch.bfloat16
        L, D, FF = len(layers), cfg.D, cfg.FF
        wide = max(D, cfg.HQ * cfg.HD, FF)
        self.px = torch.zeros(self.smax, D, dtype=f32, device=dev)
        self.q8 = torch.zeros(self.smax * wide, dtype=E4M3, device=dev)
        self.raw = torch.zeros(self.smax * max(2 * FF, cfg.qkv_n), dtype=bf16, device=dev)
        self.h = torch.zeros(self.smax * FF, dtype=bf16, device=dev)
        self.scale = [torch.zeros(self.smax, dtype=f32, device=dev) for _ in range(2)]
        self.q16 = torch.zeros(self.smax, cfg.HQ, cfg.HD, dtype=f16, device=dev)
        self.o16 = torch.zeros(self.smax, cfg.HQ * cfg.HD, dtype=f16, device=dev)
        self.kc = torch.zeros(L, self.smax, cfg.HKV, cfg.HD, dtype=f16, device=dev)
        self.vc = torch.zeros_like(self.kc)
        self.prefix_len = torch.zeros(1, dtype=torch.int32, device=dev)
        self.inv_freq = rope_inv_freq(cfg.HD, cfg.rope_theta, dev)
        self.pos = torch.arange(self.smax, dtype=f32, device=dev)[:, None].contiguous()
        self.layers = layers if self.reference_calls else [
            PrefixLayer(l.qkv, l.o, pack_glu(l.gate_up), l.down) for l in layers]

    def set_prefix(self, n: int):
        if not 1 <= n <= self.smax:
            raise ValueError(f"prefix length must be in [1, {self.smax}]")
        self.prefix_len.fill_(n)

    def q8v(self, rows, cols):
        return self.q8[: rows * cols].view(rows, cols)

    def rawv(self, rows, cols):
        return self.raw[: rows * cols].view(rows, cols)

    def forward(self, x=None, M=None, on_call=None):
        """Reference _prefix (engines/pi05/engine.py:192-216, engines/vla4/
        engine.py:114-139); ``x`` [M, D] (any float dtype) initialises the
        residual stream, else it continues from ``px``."""
        c, M = self.cfg, int(M if M is not None else (x.shape[0] if x is not None else self.smax))
        if not 1 <= M <= self.smax:
            raise ValueError(f"M must be in [1, {self.smax}]")
        if x is not None:
            self.px[:M].copy_(x)
        note = on_call or (lambda name, **t: None)
        q8, raw, s = self.q8v, self.rawv, self.scale
        D, FF, HQ, HKV, HD = c.D, c.FF, c.HQ, c.HKV, c.HD
        act_id = GELU_TANH if c.act == "geglu" else SILU
        px = self.px[:M]
        qv = self.q16[:M].view(1, M, HQ, HD)
        ov = self.o16[:M].view(1, M, HQ, HD)
        residual_norm_quant(px, q=q8(M, D), q_scale=s[0])
        note("norm0", res=px, q=q8(M, D), s=s[0])
        for i, L in enumerate(self.layers):
            gemm(q8(M, D), L.qkv, raw(M, c.qkv_n))
            note("qkv", a=q8(M, D), w=self.layers_ref[i].qkv, out=raw(M, c.qkv_n))
            qkv_split(raw(M, c.qkv_n), self.q16[:M], self.kc[i], self.vc[i], heads_q=HQ, heads_kv=HKV, head_dim=HD,
                      row=s[0], col=L.qkv.scale, bias=L.qkv.bias, inv_freq=self.inv_freq, pos=self.pos[:M])
            note("qkv_split", raw=raw(M, c.qkv_n), row=s[0], w=self.layers_ref[i].qkv, q=self.q16[:M],
                 k=self.kc[i][:M], v=self.vc[i][:M], inv_freq=self.inv_freq, pos=self.pos[:M])
            attention(qv, self.kc[i][None], self.vc[i][None], out=ov, kv_len=self.prefix_len, scale=HD ** -0.5)
            note("attention", q=qv, k=self.kc[i][None], v=self.vc[i][None], out=ov, kv_len=self.prefix_len)
            row_quant(self.o16[:M], q8(M, HQ * HD), s[1])
            note("row_quant", x=self.o16[:M], q=q8(M, HQ * HD), s=s[1])
            gemm(q8(M, HQ * HD), L.o, raw(M, D))
            note("o", a=q8(M, HQ * HD), w=self.layers_ref[i].o, out=raw(M, D))
            note("pre_res", res=px)
            residual_norm_quant(px, delta=raw(M, D), delta_row=s[1], delta_col=L.o.scale, q=q8(M, D), q_scale=s[0])
            note("norm_o", res=px, delta=raw(M, D), delta_row=s[1], w=self.layers_ref[i].o, q=q8(M, D), s=s[0])
            if self.reference_calls:
                gemm(q8(M, D), L.gate_up, raw(M, 2 * FF))
                note("gate_up_raw", a=q8(M, D), w=self.layers_ref[i].gate_up, out=raw(M, 2 * FF))
                gated_act_quant(raw(M, 2 * FF), q8(M, FF), s[1], row=s[0], col=L.gate_up.scale, act=act_id)
                note("gated_act_quant", gu=raw(M, 2 * FF), row=s[0], w=self.layers_ref[i].gate_up, q=q8(M, FF),
                     s=s[1])
            else:
                h = self.h[: M * FF].view(M, FF)
                linear(q8(M, D), s[0], L.gate_up, out=h, act=c.act)
                note("gate_up", a=q8(M, D), sa=s[0], w=self.layers_ref[i].gate_up, out=h, act=c.act)
                quant_rows(h, q8(M, FF), s[1])
                note("quant_h", x=h, q=q8(M, FF), s=s[1])
            gemm(q8(M, FF), L.down, raw(M, D))
            note("down", a=q8(M, FF), w=self.layers_ref[i].down, out=raw(M, D))
            note("pre_res", res=px)
            residual_norm_quant(px, delta=raw(M, D), delta_row=s[1], delta_col=L.down.scale, q=q8(M, D),
                                q_scale=s[0])
            note("norm_down", res=px, delta=raw(M, D), delta_row=s[1], w=self.layers_ref[i].down, q=q8(M, D), s=s[0])
        return px

"""Seeded synthetic workloads for the five benchmark configurations of the FP8
projection path (shapes from the reference engines' FP8 call sites:
instinctflash/engines/pi05/engine.py:211-214,241, engines/groot_n17/engine.py:184-188,
engines/vla4/engine.py:123-137, engines/wan_va/engine.py:214-245).

Inputs are generated on the CPU with torch.Generator (fixed order: activations,
weights, bias, residual, gate) and copied to the device once; weights are
quantized once with this package's quantize_weight. A workload's ``step()`` runs
the whole path for one batch: per-token quantization of every projection input,
each FP8 GEMM with its fused epilogue, and the re-quantization of GLU/GELU
outputs that feed a down projection.

For M <= 64 the weights rotate through a pool larger than the MI355X's 256 MB
Infinity Cache, so consecutive steps stream weights from HBM, as an engine with
many layers does.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .kernels import fp8 as F

INFINITY_CACHE_BYTES = 256 << 20


@dataclass
class Gemm:
    """One projection: shapes, fused epilogue and its algorithmic traffic."""
    name: str
    M: int
    N: int          # weight rows (2F for GLU)
    K: int
    act: str | None = None
    bias: bool = False
    residual: bool = False
    gate: bool = False

    @property
    def n_out(self) -> int:
        return self.N // 2 if self.act in ("geglu", "swiglu") else self.N

    @property
    def flops(self) -> int:
        return 2 * self.M * self.N * self.K

    @property
    def bytes(self) -> int:
        # A + W + sa + sw + bias(f32) + gate(bf16) + residual(bf16) + out(bf16)
        b = self.M * self.K + self.N * self.K + 4 * self.M + 4 * self.N
        b += 4 * self.N if self.bias else 0
        b += 2 * self.n_out if self.gate else 0
        b += 2 * self.M * self.n_out if self.residual else 0
        return b + 2 * self.M * self.n_out


def quant_bytes(M: int, K: int) -> int:
    """bf16 in + e4m3 out + f32 scale."""
    return 3 * M * K + 4 * M


@dataclass
class Call:
    name: str
    kind: str      # "gemm" or "quant"
    work: object   # Gemm, or (M, K) of a quantizer pass
    fn: object     # fn(i): run with weight set i % pool
    io: dict = field(default_factory=dict)
    """The call's operands at weight set 0, for parity checks. quant: x (bf16
    source), q (e4m3 rows or TiledRows), s (scales). gemm: a, sa, w (the weight
    the kernel reads), w_ref (the same weight in the reference layout: gate
    rows then up rows, not tiled), out, residual, gate, act."""

    @property
    def flops(self) -> int:
        return self.work.flops if self.kind == "gemm" else 0

    @property
    def bytes(self) -> int:
        return self.work.bytes if self.kind == "gemm" else quant_bytes(*self.work)


@dataclass
class Workload:
    key: str
    title: str
    bound: str                      # "hbm" or "mfma"
    gemms: list
    quants: list                    # (M, K) of every quantizer pass per step
    steps_per_unit: int = 1         # C2: 4 flow-matching steps per timed unit
    pool: int = 1                   # rotating weight sets
    dominant: str = ""              # name of the kernel the roofline line reports
    tensors: dict = field(default_factory=dict)
    ref: dict = field(default_factory=dict)  # weights in the reference layout, by projection
    _i: int = 0

    @property
    def flops(self) -> int:
        return self.steps_per_unit * sum(g.flops for g in self.gemms)

    @property
    def gemm_bytes(self) -> int:
        return self.steps_per_unit * sum(g.bytes for g in self.gemms)

    @property
    def quant_bytes(self) -> int:
        return self.steps_per_unit * sum(quant_bytes(m, k) for m, k in self.quants)

    @property
    def bytes(self) -> int:
        return self.gemm_bytes + self.quant_bytes

    def step(self):
        """One timed unit: every call of the path, steps_per_unit times."""
        for s in range(self.steps_per_unit):
            i = self._i * self.steps_per_unit + s
            for c in self.calls():
                c.fn(i)
        self._i += 1

    def calls(self) -> list:
        """The path's calls in order, as Call(name, kind, work, fn): fn(i) runs the
        call with weight set i % pool; work is the Gemm or the quantizer's (M, K)."""
        raise NotImplementedError

    def dominant_call(self, i: int):
        """Launch only the dominant kernel (its inputs prepared by an earlier step)."""
        next(c for c in self.calls() if c.name == self.dominant).fn(i)

    @property
    def dominant_gemm(self) -> Gemm:
        return next(g for g in self.gemms if g.name == self.dominant)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _act(g, M, K, outlier_frac=0.0, outlier_std=20.0):
    x = torch.randn((M, K), generator=g)
    if outlier_frac:
        mask = torch.rand((M, K), generator=g) < outlier_frac
        x = torch.where(mask, torch.randn((M, K), generator=g) * outlier_std, x)
    return x


def _weights(g, N, K, dev, bias=False, glu=False, ref=None, name=None):
    """Per-channel e4m3 weight N(0, 0.02) [+ bias N(0, 0.01)]; GLU weights are
    repacked for the fused epilogue. With ``ref`` (a dict), the weight in the
    reference layout is kept there under ``name`` for parity checks."""
    w = torch.randn((N, K), generator=g) * 0.02
    b = torch.randn(N, generator=g) * 0.01 if bias else None
    fw = F.quantize_weight(w, b, device=dev)
    if ref is not None:
        ref[name] = fw
    return F.pack_glu(fw) if glu else fw


def _gemm_io(g: Gemm, a, sa, w, w_ref, out, residual=None, gate=None):
    return dict(a=a, sa=sa, w=w, w_ref=w_ref, out=out, residual=residual, gate=gate, act=g.act)


def _copies(fw, n):
    """fw and n-1 clones: identical numerics, distinct HBM lines."""
    return [fw] + [F.Fp8Weight(fw.w.clone(), fw.scale.clone(), None if fw.bias is None else fw.bias.clone(),
                               glu=fw.glu, tiled=fw.tiled, nk=fw.nk) for _ in range(n - 1)]


def _pool_size(bytes_per_set: int) -> int:
    return max(1, -(-(INFINITY_CACHE_BYTES + (32 << 20)) // bytes_per_set))


class _Buffers:
    def __init__(self, dev):
        self.dev = dev

    def q(self, M, K):
        return (torch.empty((M, K), dtype=F.E4M3, device=self.dev), torch.empty(M, dtype=torch.float32, device=self.dev))


# ---------------------------------------------------------------------------
# C1: pi05 action-expert MLP up-projection, M=50 (HBM-bound)
# ---------------------------------------------------------------------------

class C1(Workload):
    def __init__(self, dev, seed=0, pool=None):
        M, K, N = 50, 1024, 4096
        super().__init__("C1", "pi05 expert up-proj 50x1024->4096 +bias", "hbm",
                         [Gemm("up", M, N, K, bias=True)], [(M, K)], dominant="up")
        g = _gen(seed)
        x = _act(g, M, K, outlier_frac=0.01)
        self.pool = pool or _pool_size(N * K)
        # M <= 64 weights are packed once into the skinny tile layout; rotated
        # copies give identical numerics on distinct HBM lines.
        ws = _copies(F.pack_skinny(_weights(g, N, K, dev, bias=True, ref=self.ref, name="up")), self.pool)
        xb = x.to(torch.bfloat16).to(dev)
        self.tensors = dict(x=xb, w=ws, qa=F.quant_rows_tiled(xb),
                            out=torch.empty((M, N), dtype=torch.bfloat16, device=dev))

    def calls(self):
        t = self.tensors
        qa, sa = t["qa"]
        g = self.gemms[0]
        return [  # M <= 64: activations in the skinny tile layout
            Call("quant x", "quant", (g.M, g.K), lambda i: F.quant_rows_tiled(t["x"], qa, sa),
                 dict(x=t["x"], q=qa, s=sa)),
            Call("up", "gemm", g, lambda i: F.linear(qa, sa, t["w"][i % self.pool], out=t["out"]),
                 _gemm_io(g, qa, sa, t["w"][0], self.ref["up"], t["out"])),
        ]


# ---------------------------------------------------------------------------
# C2: GR00T-style DiT action head, M=16, up(GELU) + down(+residual) x 4 steps
# ---------------------------------------------------------------------------

class C2(Workload):
    def __init__(self, dev, seed=0, pool=None):
        M, D, FF = 16, 1536, 6144
        super().__init__("C2", "GR00T DiT M=16: 1536->6144 GELU, 6144->1536 +res, x4 steps", "hbm",
                         [Gemm("up", M, FF, D, act="gelu_tanh"), Gemm("down", M, D, FF, residual=True)],
                         [(M, D), (M, FF)], steps_per_unit=4, dominant="up")
        g = _gen(seed)
        xs = [_act(g, M, D) for _ in range(4)]  # fresh x per flow-matching step
        w1 = _weights(g, FF, D, dev, ref=self.ref, name="up")
        w2 = _weights(g, D, FF, dev, ref=self.ref, name="down")
        res = torch.randn((M, D), generator=g).to(torch.bfloat16)
        self.pool = pool or _pool_size(2 * FF * D)
        w1s = _copies(F.pack_skinny(w1), self.pool)
        w2s = _copies(F.pack_skinny(w2), self.pool)
        xsd = [x.to(torch.bfloat16).to(dev) for x in xs]
        h = torch.empty((M, FF), dtype=torch.bfloat16, device=dev)
        self.tensors = dict(xs=xsd, w1=w1s, w2=w2s, res=res.to(dev), q1=F.quant_rows_tiled(xsd[0]),
                            q2=F.quant_rows_tiled(h.zero_()), h=h,
                            out=torch.empty((M, D), dtype=torch.bfloat16, device=dev))

    def calls(self):
        # one flow step (the unit runs it 4 times, fresh x each time); one weight set
        # per (unit, flow step): a deep DiT streams each layer's weights; M = 16:
        # activations quantized straight into the skinny tile layout
        t = self.tensors
        q1, s1 = t["q1"]
        q2, s2 = t["q2"]
        up, down = self.gemms
        return [
            Call("quant x", "quant", (up.M, up.K), lambda i: F.quant_rows_tiled(t["xs"][i % 4], q1, s1),
                 dict(x=t["xs"][0], q=q1, s=s1)),
            Call("up", "gemm", up,
                 lambda i: F.linear(q1, s1, t["w1"][i % self.pool], out=t["h"], act="gelu_tanh"),
                 _gemm_io(up, q1, s1, t["w1"][0], self.ref["up"], t["h"])),
            Call("quant h", "quant", (down.M, down.K), lambda i: F.quant_rows_tiled(t["h"], q2, s2),
                 dict(x=t["h"], q=q2, s=s2)),
            Call("down", "gemm", down,
                 lambda i: F.linear(q2, s2, t["w2"][i % self.pool], out=t["out"], residual=t["res"]),
                 _gemm_io(down, q2, s2, t["w2"][0], self.ref["down"], t["out"], residual=t["res"])),
        ]


# ---------------------------------------------------------------------------
# C3: pi05 PaliGemma prefix MLP, M=816, GeGLU + down(+residual)
# ---------------------------------------------------------------------------

class C3(Workload):
    def __init__(self, dev, seed=0):
        M, D, FF = 816, 2048, 16384
        super().__init__("C3", "pi05 prefix MLP M=816: 2048->2x16384 GeGLU, 16384->2048 +res", "mfma",
                         [Gemm("gate_up", M, 2 * FF, D, act="geglu"), Gemm("down", M, D, FF, residual=True)],
                         [(M, D), (M, FF)], dominant="gate_up")
        g = _gen(seed)
        x = torch.randn((M, D), generator=g)
        x = x / x.pow(2).mean(dim=1, keepdim=True).sqrt()  # unit-RMS rows (post-RMSNorm)
        wgu = _weights(g, 2 * FF, D, dev, glu=True, ref=self.ref, name="gate_up")
        wd = _weights(g, D, FF, dev, ref=self.ref, name="down")
        res = torch.randn((M, D), generator=g).to(torch.bfloat16)
        b = _Buffers(dev)
        self.tensors = dict(x=x.to(torch.bfloat16).to(dev), wgu=wgu, wd=wd, res=res.to(dev), q1=b.q(M, D),
                            q2=b.q(M, FF), h=torch.empty((M, FF), dtype=torch.bfloat16, device=dev),
                            out=torch.empty((M, D), dtype=torch.bfloat16, device=dev))

    def calls(self):
        t = self.tensors
        q1, s1 = t["q1"]
        q2, s2 = t["q2"]
        gu, down = self.gemms
        return [
            Call("quant x", "quant", (gu.M, gu.K), lambda i: F.quant_rows(t["x"], q1, s1),
                 dict(x=t["x"], q=q1, s=s1)),
            Call("gate_up", "gemm", gu, lambda i: F.linear(q1, s1, t["wgu"], out=t["h"], act="geglu"),
                 _gemm_io(gu, q1, s1, t["wgu"], self.ref["gate_up"], t["h"])),
            Call("quant h", "quant", (down.M, down.K), lambda i: F.quant_rows(t["h"], q2, s2),
                 dict(x=t["h"], q=q2, s=s2)),
            Call("down", "gemm", down, lambda i: F.linear(q2, s2, t["wd"], out=t["out"], residual=t["res"]),
                 _gemm_io(down, q2, s2, t["wd"], self.ref["down"], t["out"], residual=t["res"])),
        ]


# ---------------------------------------------------------------------------
# C4: Qwen2.5-style decoder layer projections (LingBot-VLA-4B), M=1024
# ---------------------------------------------------------------------------

def _channel_outliers(g, M, K, n=8, factor=30.0):
    x = torch.randn((M, K), generator=g)
    ch = torch.randperm(K, generator=g)[:n]
    x[:, ch] *= factor
    return x


class C4(Workload):
    def __init__(self, dev, seed=0):
        M, D, FF = 1024, 2048, 11008
        qkv_n = 2048 + 256 + 256
        super().__init__("C4", "VLA4 layer M=1024: qkv(+bias), o(+res), gate|up SwiGLU, down(+res)", "mfma",
                         [Gemm("qkv", M, qkv_n, D, bias=True), Gemm("o", M, D, D, residual=True),
                          Gemm("gate_up", M, 2 * FF, D, act="swiglu"), Gemm("down", M, D, FF, residual=True)],
                         [(M, D), (M, D), (M, D), (M, FF)], dominant="gate_up")
        g = _gen(seed)
        x_attn_in = _channel_outliers(g, M, D)
        x_o_in = _channel_outliers(g, M, D)
        x_mlp_in = _channel_outliers(g, M, D)
        wqkv = _weights(g, qkv_n, D, dev, bias=True, ref=self.ref, name="qkv")
        wo = _weights(g, D, D, dev, ref=self.ref, name="o")
        wgu = _weights(g, 2 * FF, D, dev, glu=True, ref=self.ref, name="gate_up")
        wd = _weights(g, D, FF, dev, ref=self.ref, name="down")
        res = torch.randn((M, D), generator=g).to(torch.bfloat16)
        b = _Buffers(dev)
        bf = lambda t: t.to(torch.bfloat16).to(dev)  # noqa: E731
        self.tensors = dict(xa=bf(x_attn_in), xo=bf(x_o_in), xm=bf(x_mlp_in), wqkv=wqkv, wo=wo, wgu=wgu, wd=wd,
                            res=res.to(dev), q=b.q(M, D), qh=b.q(M, FF),
                            qkv=torch.empty((M, qkv_n), dtype=torch.bfloat16, device=dev),
                            h=torch.empty((M, FF), dtype=torch.bfloat16, device=dev),
                            r1=torch.empty((M, D), dtype=torch.bfloat16, device=dev),
                            r2=torch.empty((M, D), dtype=torch.bfloat16, device=dev))

    def calls(self):
        t = self.tensors
        q, s = t["q"]
        qh, sh = t["qh"]
        qkv, o, gu, down = self.gemms
        return [
            Call("quant attn in", "quant", (qkv.M, qkv.K), lambda i: F.quant_rows(t["xa"], q, s),
                 dict(x=t["xa"], q=q, s=s)),
            Call("qkv", "gemm", qkv, lambda i: F.linear(q, s, t["wqkv"], out=t["qkv"]),
                 _gemm_io(qkv, q, s, t["wqkv"], self.ref["qkv"], t["qkv"])),
            Call("quant o in", "quant", (o.M, o.K), lambda i: F.quant_rows(t["xo"], q, s),
                 dict(x=t["xo"], q=q, s=s)),
            Call("o", "gemm", o, lambda i: F.linear(q, s, t["wo"], out=t["r1"], residual=t["res"]),
                 _gemm_io(o, q, s, t["wo"], self.ref["o"], t["r1"], residual=t["res"])),
            Call("quant mlp in", "quant", (gu.M, gu.K), lambda i: F.quant_rows(t["xm"], q, s),
                 dict(x=t["xm"], q=q, s=s)),
            Call("gate_up", "gemm", gu, lambda i: F.linear(q, s, t["wgu"], out=t["h"], act="swiglu"),
                 _gemm_io(gu, q, s, t["wgu"], self.ref["gate_up"], t["h"])),
            Call("quant h", "quant", (down.M, down.K), lambda i: F.quant_rows(t["h"], qh, sh),
                 dict(x=t["h"], q=qh, s=sh)),
            Call("down", "gemm", down, lambda i: F.linear(qh, sh, t["wd"], out=t["r2"], residual=t["r1"]),
                 _gemm_io(down, qh, sh, t["wd"], self.ref["down"], t["r2"], residual=t["r1"])),
        ]


# ---------------------------------------------------------------------------
# C5: Wan-style video DiT block projections (LingBot-VA), M=8192
# ---------------------------------------------------------------------------

class C5(Workload):
    def __init__(self, dev, seed=0):
        M, D, FF = 8192, 3072, 14336
        super().__init__("C5", "Wan DiT block M=8192: qkv, o(gated res), up GELU, down(gated res)", "mfma",
                         [Gemm("qkv", M, 3 * D, D), Gemm("o", M, D, D, residual=True, gate=True),
                          Gemm("up", M, FF, D, act="gelu_tanh"), Gemm("down", M, D, FF, residual=True, gate=True)],
                         [(M, D), (M, D), (M, D), (M, FF)], dominant="up")
        g = _gen(seed)
        mod = torch.rand(D, generator=g) + 0.5  # adaLN modulation scale U(0.5, 1.5) per channel
        xa = torch.randn((M, D), generator=g) * mod
        xo = torch.randn((M, D), generator=g) * mod
        xm = torch.randn((M, D), generator=g) * mod
        wqkv = _weights(g, 3 * D, D, dev, ref=self.ref, name="qkv")
        wo = _weights(g, D, D, dev, ref=self.ref, name="o")
        wu = _weights(g, FF, D, dev, ref=self.ref, name="up")
        wd = _weights(g, D, FF, dev, ref=self.ref, name="down")
        res = torch.randn((M, D), generator=g).to(torch.bfloat16)
        gate_o = torch.rand(D, generator=g).to(torch.bfloat16)
        gate_f = torch.rand(D, generator=g).to(torch.bfloat16)
        b = _Buffers(dev)
        bf = lambda t: t.to(torch.bfloat16).to(dev)  # noqa: E731
        self.tensors = dict(xa=bf(xa), xo=bf(xo), xm=bf(xm), wqkv=wqkv, wo=wo, wu=wu, wd=wd, res=res.to(dev),
                            gate_o=gate_o.to(dev), gate_f=gate_f.to(dev), q=b.q(M, D), qh=b.q(M, FF),
                            qkv=torch.empty((M, 3 * D), dtype=torch.bfloat16, device=dev),
                            h=torch.empty((M, FF), dtype=torch.bfloat16, device=dev),
                            r1=torch.empty((M, D), dtype=torch.bfloat16, device=dev),
                            r2=torch.empty((M, D), dtype=torch.bfloat16, device=dev))

    def calls(self):
        t = self.tensors
        q, s = t["q"]
        qh, sh = t["qh"]
        qkv, o, up, down = self.gemms
        return [
            Call("quant attn in", "quant", (qkv.M, qkv.K), lambda i: F.quant_rows(t["xa"], q, s),
                 dict(x=t["xa"], q=q, s=s)),
            Call("qkv", "gemm", qkv, lambda i: F.linear(q, s, t["wqkv"], out=t["qkv"]),
                 _gemm_io(qkv, q, s, t["wqkv"], self.ref["qkv"], t["qkv"])),
            Call("quant o in", "quant", (o.M, o.K), lambda i: F.quant_rows(t["xo"], q, s),
                 dict(x=t["xo"], q=q, s=s)),
            Call("o", "gemm", o,
                 lambda i: F.linear(q, s, t["wo"], out=t["r1"], residual=t["res"], gate=t["gate_o"]),
                 _gemm_io(o, q, s, t["wo"], self.ref["o"], t["r1"], residual=t["res"], gate=t["gate_o"])),
            Call("quant mlp in", "quant", (up.M, up.K), lambda i: F.quant_rows(t["xm"], q, s),
                 dict(x=t["xm"], q=q, s=s)),
            Call("up", "gemm", up, lambda i: F.linear(q, s, t["wu"], out=t["h"], act="gelu_tanh"),
                 _gemm_io(up, q, s, t["wu"], self.ref["up"], t["h"])),
            Call("quant h", "quant", (down.M, down.K), lambda i: F.quant_rows(t["h"], qh, sh),
                 dict(x=t["h"], q=qh, s=sh)),
            Call("down", "gemm", down,
                 lambda i: F.linear(qh, sh, t["wd"], out=t["r2"], residual=t["r1"], gate=t["gate_f"]),
                 _gemm_io(down, qh, sh, t["wd"], self.ref["down"], t["r2"], residual=t["r1"],
                          gate=t["gate_f"])),
        ]


CONFIGS = {"C1": C1, "C2": C2, "C3": C3, "C4": C4, "C5": C5}


# ---------------------------------------------------------------------------
# Producer: pre-norm residual update + LayerNorm + adaLN + per-token quant
# ---------------------------------------------------------------------------

class NormQuant:
    """``residual_norm_quant`` at a pre-norm site: res (fp32) += (delta (bf16) *
    row * col + bias) * gate, LayerNorm with adaptive scale/shift, per-token E4M3.
    Algorithmic bytes: res read + write (8 B), delta (2 B), q (1 B) per element;
    the [D] vectors once; q_scale and delta_row per row."""

    def __init__(self, dev, M, D, seed=0):
        from .kernels import norm as N
        self.N, self.M, self.D = N, M, D
        g = _gen(seed)
        f = lambda *s: torch.randn(*s, generator=g).to(dev)  # noqa: E731
        self.base = f(M, D)
        self.t = dict(res=self.base.clone(), delta=f(M, D).to(torch.bfloat16), delta_row=f(M).abs(),
                      delta_col=f(D).abs(), bias=f(D), gate=f(D).abs(), mod_scale=f(D) * 0.1, mod_shift=f(D) * 0.1)
        self.q = torch.empty((M, D), dtype=F.E4M3, device=dev)
        self.qs = torch.empty(M, dtype=torch.float32, device=dev)
        self.title = f"residual_norm_quant {M}x{D} (fp32 res += gated bf16 delta, LayerNorm, adaLN, e4m3)"

    @property
    def bytes(self) -> int:
        return 11 * self.M * self.D + 5 * 4 * self.D + 2 * 4 * self.M

    def step(self, i=0):
        self.N.residual_norm_quant(self.t["res"], delta=self.t["delta"], delta_row=self.t["delta_row"],
                                   delta_col=self.t["delta_col"], bias=self.t["bias"], gate=self.t["gate"],
                                   layernorm=True, mod_scale=self.t["mod_scale"], mod_shift=self.t["mod_shift"],
                                   q=self.q, q_scale=self.qs)


class QkvSplit:
    """``qkv_split`` after the C4 qkv projection (Qwen2.5-style: 16 query / 2 KV
    heads of 128, bias, M-RoPE with 3 position sections), writing q and the K/V
    cache rows. Algorithmic bytes: the bf16 accumulator read once, q/k/v written
    once (bf16), the scale/bias vectors and position rows once."""

    def __init__(self, dev, T=1024, HQ=16, HKV=2, HD=128, seed=0):
        from .kernels import rope as R
        self.R, self.T, self.HQ, self.HKV, self.HD = R, T, HQ, HKV, HD
        g = _gen(seed)
        C = (HQ + 2 * HKV) * HD
        self.raw = torch.randn(T, C, generator=g).to(torch.bfloat16).to(dev)
        self.row = (torch.rand(T, generator=g) + 0.5).to(dev)
        self.col = (torch.rand(C, generator=g) + 0.5).to(dev)
        self.bias = torch.randn(C, generator=g).to(dev)
        self.inv = R.rope_inv_freq(HD, 1e6, dev)
        self.pos = torch.stack([torch.arange(T)] * 3, 1).float().to(dev)
        self.sec = (torch.arange(HD // 2) % 3).int().to(dev)
        self.q = torch.empty(T, HQ, HD, dtype=torch.bfloat16, device=dev)
        self.kc = torch.empty(2 * T, HKV, HD, dtype=torch.bfloat16, device=dev)
        self.vc = torch.empty_like(self.kc)
        self.title = f"qkv_split {T} tokens, {HQ}+2x{HKV} heads x {HD} (rescale, bias, M-RoPE, KV-cache store)"

    @property
    def bytes(self) -> int:
        C = (self.HQ + 2 * self.HKV) * self.HD
        return 2 * self.T * C * 2 + 2 * C * 4 + self.T * (4 + 3 * 4) + self.HD // 2 * (4 + 4)

    def step(self, i=0):
        self.R.qkv_split(self.raw, self.q, self.kc, self.vc, heads_q=self.HQ, heads_kv=self.HKV, head_dim=self.HD,
                         row=self.row, col=self.col, bias=self.bias, inv_freq=self.inv, pos=self.pos,
                         sections=self.sec, kv_base=self.T // 2)


class QkvRope:
    """The pi05 expert's QKV projection with the QKV split in its epilogue
    (``linear_qkv_rope``): 50 tokens x 1024 -> 8 query + 1 KV heads of 256,
    rotary on Q and K, Q and the K/V cache rows in fp16, weights and activations
    in the skinny tile layout (weights rotated through a pool larger than the
    MALL, as 18 layers of them are in the engine). Algorithmic bytes: weights,
    activations and scales read once, q/k/v written once."""

    def __init__(self, dev, M=50, K=1024, HQ=8, HKV=1, HD=256, seed=0):
        from .kernels import rope as R
        self.R, self.M, self.K, self.HQ, self.HKV, self.HD = R, M, K, HQ, HKV, HD
        g = _gen(seed)
        N = (HQ + 2 * HKV) * HD
        x = torch.randn(M, K, generator=g).to(dev)
        self.xq, self.sa = F.quant_rows_tiled(x)
        w = F.quantize_weight((torch.randn(N, K, generator=g) * 0.02).to(dev))
        pool = max(1, (300 << 20) // (N * K))
        self.ws = [F.pack_skinny(R.permute_rope_rows(F.Fp8Weight(w.w.clone(), w.scale.clone()), HQ, HKV, HD))
                   for _ in range(pool)]
        self.inv = R.rope_inv_freq(HD, 1e4, dev)
        self.pos = (torch.arange(M, dtype=torch.float32) + 800).reshape(M, 1).to(dev)
        self.base = torch.tensor([800], dtype=torch.int32, device=dev)
        self.q = torch.empty(M, HQ, HD, dtype=torch.float16, device=dev)
        self.kc = torch.empty(832 + M, HKV, HD, dtype=torch.float16, device=dev)
        self.vc = torch.empty_like(self.kc)
        self.title = (f"linear_qkv_rope {M}x{K} -> {HQ}+2x{HKV} heads x {HD} (FP8 projection + rotary + "
                      f"KV-cache store, weight pool of {pool})")

    @property
    def bytes(self) -> int:
        N = (self.HQ + 2 * self.HKV) * self.HD
        return N * self.K + self.M * self.K + 4 * (self.M + N) + 2 * self.M * N

    def step(self, i=0):
        self.R.linear_qkv_rope(self.xq, self.sa, self.ws[i % len(self.ws)], self.q, self.kc, self.vc,
                               inv_freq=self.inv, pos=self.pos, kv_base=self.base)


class WanQkv:
    """``wan_qkv`` after the C5 qkv projection (Wan 5B: 24 heads of 128, bias,
    full-width q/k RMSNorm, 3-section interleaved rotary), Q dense, K/V into
    slot rows of the pools. Algorithmic bytes: the bf16 accumulator read once,
    Q/K/V written once (bf16), vectors once."""

    def __init__(self, dev, rows=8192, H=24, HD=128, seed=0):
        from .kernels import rope as R, wan as W
        self.W, self.rows, self.H, self.HD = W, rows, H, HD
        g = _gen(seed)
        D = H * HD
        self.raw = torch.randn(rows, 3 * D, generator=g).to(torch.bfloat16).to(dev)
        self.row = (torch.rand(rows, generator=g) + 0.5).to(dev)
        self.col = (torch.rand(3 * D, generator=g) + 0.5).to(dev)
        self.bias = torch.randn(3 * D, generator=g).to(dev)
        self.qn = (torch.rand(D, generator=g) + 0.5).to(dev)
        self.kn = (torch.rand(D, generator=g) + 0.5).to(dev)
        self.inv = R.rope_inv_freq(HD, 1e4, dev)
        self.pos = torch.randint(0, 64, (rows, 3), generator=g).float().to(dev)
        self.sec = (torch.arange(HD // 2) % 3).int().to(dev)
        self.slots = torch.arange(rows, dtype=torch.int32, device=dev)
        self.q = torch.empty(rows, D, dtype=torch.bfloat16, device=dev)
        self.kp = torch.empty(1, rows, D, dtype=torch.bfloat16, device=dev)
        self.vp = torch.empty_like(self.kp)
        self.title = f"wan_qkv {rows} rows, {H} heads x {HD} (rescale, bias, q/k RMSNorm, 3D RoPE, KV pools)"

    @property
    def bytes(self) -> int:
        D = self.H * self.HD
        return 3 * self.rows * D * 2 * 2 + 3 * D * 8 + 2 * D * 4 + self.rows * (4 + 12 + 4) + self.HD * 4

    def step(self, i=0):
        self.W.wan_qkv(self.raw, self.q, heads=self.H, head_dim=self.HD, tokens=self.rows, k_pool=self.kp,
                       v_pool=self.vp, slots=self.slots, row=self.row, col=self.col, bias=self.bias, q_norm=self.qn,
                       k_norm=self.kn, pos=self.pos, sections=self.sec, inv_freq=self.inv)


class MoeRoute:
    """The MoE layer's pre-norm with the fused router (``residual_norm_quant``
    with ``router=``) at the vla2 action-expert shape: 51 suffix tokens x 768,
    32 experts, top 4. Algorithmic bytes: res read + write (8 B), bf16 delta
    (2 B), q (1 B) per element, the fp32 router matrix [E, D] once, the routing
    weights [M, E] written, vectors once."""

    def __init__(self, dev, M=51, D=768, E=32, seed=0):
        from .kernels import norm as N
        self.N, self.M, self.D, self.E = N, M, D, E
        g = _gen(seed)
        f = lambda *s: torch.randn(*s, generator=g).to(dev)  # noqa: E731
        self.t = dict(res=f(M, D), delta=f(M, D).to(torch.bfloat16), delta_row=f(M).abs(), delta_col=f(D).abs(),
                      mod_scale=f(D) * 0.1, mod_shift=f(D) * 0.1)
        self.router = (f(E, D) * 0.05, f(E).abs() * 0.01, torch.empty(M, E, device=dev), 4, 4.0)
        self.q = torch.empty((M, D), dtype=F.E4M3, device=dev)
        self.qs = torch.empty(M, dtype=torch.float32, device=dev)
        self.title = f"residual_norm_quant + router {M}x{D}, {E} experts top 4 (vla2 MoE pre-norm)"

    @property
    def bytes(self) -> int:
        return 11 * self.M * self.D + 3 * 4 * self.D + 2 * 4 * self.M + 4 * self.E * self.D + 4 * self.E * (self.M + 1)

    def step(self, i=0):
        self.N.residual_norm_quant(self.t["res"], delta=self.t["delta"], delta_row=self.t["delta_row"],
                                   delta_col=self.t["delta_col"], mod_scale=self.t["mod_scale"],
                                   mod_shift=self.t["mod_shift"], q=self.q, q_scale=self.qs, router=self.router)


class MoeAct:
    """``moe_act_quant`` at the vla2 MoE shape: 51 tokens, 32 routed experts x 512
    + 704 shared columns (F = 17088). Algorithmic bytes: the bf16 gate|up
    accumulator read (4 B per output column), q written (1 B), col [2F] and the
    routing weights once, row and q_scale per row."""

    def __init__(self, dev, M=51, E=32, G=512, S=704, seed=0):
        from .kernels import activation as A
        self.A, self.M, self.E, self.G = A, M, E, G
        self.F = F_ = E * G + S
        g = _gen(seed)
        self.gu = torch.randn(M, 2 * F_, generator=g).to(torch.bfloat16).to(dev)
        self.row = (torch.rand(M, generator=g) + 0.5).to(dev)
        self.col = (torch.rand(2 * F_, generator=g) + 0.5).to(dev)
        self.rw = torch.rand(M, E, generator=g).to(dev)
        self.q = torch.empty((M, F_), dtype=F.E4M3, device=dev)
        self.qs = torch.empty(M, dtype=torch.float32, device=dev)
        self.title = f"moe_act_quant {M}x{F_} ({E} experts x {G} + {S} shared, routed SwiGLU, e4m3)"

    @property
    def bytes(self) -> int:
        return 5 * self.M * self.F + 8 * self.F + 4 * self.M * (self.E + 2)

    def step(self, i=0):
        self.A.moe_act_quant(self.gu, self.q, self.qs, self.rw, row=self.row, col=self.col, experts=self.E,
                             group=self.G, n_routed=self.E * self.G)


class Attn:
    """``attention`` at the pi05 shapes (8 query heads, 1 KV head of 256 dims):
    the 51-token action chunk over an 800-token prefix plus itself, split over
    key ranges (``split_count``) with the fused per-token E4M3 output row (the
    o-projection's A operand), or the 800-token prefix self-attention (keys
    split automatically). Work: 4 * Tq * Hq * Tk * D
    FLOP (bf16 matrix cores); algorithmic bytes: q, k, v read once, the output
    (bf16 row, or e4m3 row + scale) written once."""

    def __init__(self, dev, Tq=51, Tk=851, Hq=8, Hkv=1, D=256, splits=None, q8=True, seed=0):
        from .kernels.attention import SplitWorkspace, attention, split_count
        if splits is None:
            splits = max(2, split_count(1, Tq, Hq, Hkv, Tk)) if q8 else 1
        self.attention, self.Tq, self.Tk, self.Hq, self.Hkv, self.D = attention, Tq, Tk, Hq, Hkv, D
        g = _gen(seed)
        self.q = torch.randn(1, Tq, Hq, D, generator=g).to(torch.bfloat16).to(dev)
        self.k = torch.randn(1, Tk, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
        self.v = torch.randn(1, Tk, Hkv, D, generator=g).to(torch.bfloat16).to(dev)
        self.ws = SplitWorkspace(1, Tq, Hq, Hkv, D, splits, dev) if splits > 1 else None
        self.q8 = torch.empty(Tq, Hq * D, dtype=F.E4M3, device=dev) if q8 else None
        self.qs = torch.empty(Tq, dtype=torch.float32, device=dev) if q8 else None
        self.out = None if q8 else torch.empty_like(self.q)
        kind = f"split {splits}, fused e4m3 row" if q8 else "bf16 out"
        self.title = f"attention {Tq}x{Tk} keys, {Hq}/{Hkv} heads x {D} ({kind})"

    @property
    def flops(self) -> float:
        return 4.0 * self.Tq * self.Hq * self.Tk * self.D

    @property
    def bytes(self) -> int:
        qo = self.Tq * self.Hq * self.D
        out = qo + 4 * self.Tq if self.q8 is not None else 2 * qo
        return 2 * qo + 2 * 2 * self.Tk * self.Hkv * self.D + out

    def step(self, i=0):
        self.attention(self.q, self.k, self.v, out=self.out, split=self.ws, q8=self.q8, q8_scale=self.qs)


class AttnPrefix(Attn):
    def __init__(self, dev):
        super().__init__(dev, Tq=800, Tk=800, splits=1, q8=False)


PRODUCERS = {"C5": (8192, 3072), "C2": (16, 1536)}
CONSUMERS = {"C4": QkvSplit, "C5": WanQkv, "pi05 qkv": QkvRope, "vla2 MoE": MoeRoute, "vla2 MoE act": MoeAct,
             "pi05 chunk": Attn, "pi05 prefix": AttnPrefix}

"""The GR00T N1.7 action head -- config C2's call site -- at the head's widths
(VLSA 2048 wide, 32 heads of 64; DiT 1536 wide, 32 heads of 48, MLP 6144) with
a reduced block count (2 VLSA, 4 DiT blocks: cross-text, self, cross-image,
self) and 2 flow steps, every kernel call checked against the oracle on the
inputs that call actually received (instinctflash_amd/groot.py, reference
engines/groot_n17/engine.py:92-200):

  * LayerNorms: the float32 residual update bit-exact; the e4m3 row within the
    reference test's bar (7% of the row max, tests/test_gi_kernels.py:112) of
    the oracle's float64 LayerNorm (+ affine / AdaLN); float32 y outputs within
    1e-5 of the row max;
  * GEMMs: max|d| <= 2e-2 * rms + one bf16 rounding and cosine >= 0.9999 against
    dequantize-then-fp32-matmul (+ bias, GELU);
  * dequant_rows to fp16 (q|k|v, cross K / V): bit-exact against the float32
    expression in the reference's order;
  * attention (self, cross up to the device-side text / image row counts,
    VLSA up to the sequence length): the reference test's fp16 bar (2e-3);
  * quantizers of kernel-produced rows: bytes and scales bit-exact;
and the captured graph replays the head bit for bit."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _u8(t):
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def _f(t):
    return t.detach().float().cpu().numpy()


def _bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _inputs(n, seed):
    from instinctflash_amd.groot import ACT_DIM, HORIZON, VL_D
    g = torch.Generator().manual_seed(seed)
    feat = torch.randn(n, VL_D, generator=g) * 2.0
    img = torch.rand(n, generator=g) < 0.6
    valid = torch.rand(n, generator=g) < 0.9
    return feat, img, valid, torch.randn(ACT_DIM, generator=g), torch.randn(HORIZON, ACT_DIM, generator=g)


class Checker:
    def __init__(self, oracle, head):
        self.o, self.head = oracle, head
        self.pre = None
        self.seen = []

    def gemm(self, what, a, w, out, sa=None, act=None):
        o = self.o
        rows = np.arange(a.shape[0])
        if rows.size > 64:
            rows = np.sort(np.random.default_rng(rows.size).choice(rows, 64, replace=False))
        ridx = torch.as_tensor(rows, device=out.device)
        ref = o.ref_linear(_u8(a[ridx]), None if sa is None else _f(sa)[rows], _u8(w.w),
                           None if sa is None else _f(w.scale), bias=None if sa is None else _f(w.bias), act=act)
        got = _f(out[ridx])
        _, cos = o.parity_stats(got, ref)
        rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
        excess = np.abs(got - ref) - (2e-2 * rms + 2.0 ** -8 * np.abs(ref))
        assert excess.max() <= 0 and cos >= 0.9999, f"{what}: excess {excess.max():.3e} cos {cos:.7f}"

    def deq(self, what, x, y, row, col, bias):
        f32 = np.float32
        ref = ((_f(x) * _f(row)[:, None]).astype(f32) * _f(col)[None, :]).astype(f32)
        ref = (ref + _f(bias)[None, :]).astype(f32).astype(np.float16)
        got = y.detach().cpu().numpy()
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), f"{what}: fp16 rows differ"

    def norm(self, what, t, eps):
        o = self.o
        kw = dict(eps=eps)
        if what != "res_vl":
            kw["layernorm"] = True
        if "delta" in t:
            w = t["w"]
            kw.update(delta=_f(t["delta"]), delta_row=_f(t["delta_row"]), delta_col=_f(w.scale), bias=_f(w.bias))
        if "weight" in t:
            kw.update(weight=_f(t["weight"]), beta=_f(t["beta"]))
        if "mod" in t:
            kw.update(mod_scale=_f(t["mod"][0]), mod_shift=_f(t["mod"][1]))
        x_ref, y_ref = o.residual_norm(self.pre if "src" not in t else _f(t["src"]), **kw)
        if "res" in t:
            got = _f(t["res"])
            assert np.array_equal(got.view(np.uint32), x_ref.view(np.uint32)), f"{what}: residual not bit-exact"
        if "q" in t:
            deq = o.e4m3_decode(_u8(t["q"])) * _f(t["s"])[:, None]
            err = (np.abs(deq - y_ref).max(axis=1) / np.abs(y_ref).max(axis=1)).max()
            assert err < 0.07, f"{what}: e4m3 row error {err:.3e} of the row max"
        if "y" in t:
            yk = _f(t["y"]).astype(np.float64)
            err = (np.abs(yk - y_ref).max(axis=1) / np.abs(y_ref).max(axis=1)).max()
            assert err <= 1e-5, f"{what}: y rel err {err:.3e}"

    def __call__(self, name, **t):
        torch.cuda.synchronize()
        o = self.o
        self.seen.append(name)
        if name == "pre_res":
            self.pre = _f(t["res"])
        elif name == "vlln":
            self.norm(name, dict(src=t["src"], weight=t["weight"], beta=t["beta"], y=t["y"]), 1e-5)
        elif name in ("norm_vl", "norm_dit", "res_vl"):
            self.norm(name, t, 1e-5)
        elif name == "norm_out":
            self.norm(name, t, 1e-6)
        elif name in ("gemm", "ff1_raw"):
            self.gemm(name, t["a"], t["w"], t["out"])
        elif name == "ff1_quant":
            # row_quant with GELU of the raw accumulator (hardware exp): the quantizer
            # tests' bar -- scales within 8 ulp, >= 99.9% identical bytes, 7% of the row max
            x = _f(t["x"]) * _f(t["row"])[:, None] * _f(t["w"].scale)[None, :]
            hh = o.gelu_tanh((x + _f(t["w"].bias)[None, :]).astype(np.float32))
            eq, es = o.quant_rows(hh.astype(np.float32))
            sg = _f(t["s"])
            assert np.all(np.abs(sg.view(np.int32).astype(np.int64) - es.view(np.int32)) <= 8)
            assert (_u8(t["q"]) == eq).mean() > 0.999
            deq = o.e4m3_decode(_u8(t["q"])) * sg[:, None]
            assert (np.abs(deq - hh) / np.abs(hh).max(axis=1, keepdims=True)).max() < 0.07
        elif name == "ff1":
            self.gemm(name, t["a"], t["w"], t["out"], sa=t["sa"], act=t["act"])
        elif name == "dequant":
            self.deq(name, t["x"], t["y"], t["row"], t["w"].scale, t["w"].bias)
        elif name == "dequant_kv":
            w, x = t["w"], t["x"]
            D = x.shape[1] // 2
            self.deq("cross k", x[:, :D], t["k"], t["row"], w.scale[:D], w.bias[:D])
            self.deq("cross v", x[:, D:], t["v"], t["row"], w.scale[D:], w.bias[D:])
        elif name == "attention":
            q = _f(t["q"])
            n = q.shape[1] if t["kv_len"] is None else int(t["kv_len"].item())
            n = min(n, t["k"].shape[1])
            ref = o.attention(q, _f(t["k"]), _f(t["v"]), np.full(q.shape[1], n), q.shape[3] ** -0.5)
            err = np.abs(_f(t["out"]) - ref).max()
            assert err < 2e-3, f"attention: max |d| {err:.3e}"
        elif name in ("row_quant", "quant_h", "enc_quant"):
            x = t["x"]
            src = _bits(x) if x.dtype == torch.bfloat16 else _f(x)  # fp16 / fp32: exact in float32
            eq, es = o.quant_rows(src)
            assert np.array_equal(_u8(t["q"]), eq), f"{name}: e4m3 bytes"
            assert np.array_equal(_f(t["s"]).view(np.uint32), es.view(np.uint32)), f"{name}: scales"
        else:
            raise AssertionError(f"unchecked call {name}")


def test_groot_head_calls_against_oracle(gpu, oracle_mod):
    from instinctflash_amd.groot import GrootHead, random_groot_weights
    n, M = 90, 96
    print(f"[groot] n={n} M={M}", flush=True)
    w = random_groot_weights(gpu, vlsa_blocks=2, dit_blocks=4, steps=2, seed=3)
    head = GrootHead(w, gpu, max_seq=128, reference_calls=True)
    head.set_inputs(*(t.to(gpu) for t in _inputs(n, 4)))
    chk = Checker(oracle_mod, head)
    a = head.forward(M, on_call=chk)
    assert chk.seen.count("norm_out") == 2 and chk.seen.count("ff1_quant") == 2 + 2 * 4
    assert chk.seen.count("dequant_kv") == 2 and chk.seen.count("enc_quant") == 2
    assert np.isfinite(_f(a)).all()


def test_groot_reference_calls_and_graph(gpu):
    # the reference's MLP calls (raw accumulator + row_quant with GELU) against
    # the GELU-epilogue layout, and the captured graph bit for bit
    from instinctflash_amd.groot import GrootHead, random_groot_weights
    n, M = 90, 96
    w = random_groot_weights(gpu, vlsa_blocks=2, dit_blocks=4, steps=2, seed=5)
    inputs = [t.to(gpu) for t in _inputs(n, 6)]
    ref = GrootHead(w, gpu, max_seq=128, reference_calls=True)
    ref.set_inputs(*inputs)
    a = ref.forward(M).clone()
    head = GrootHead(w, gpu, max_seq=128)
    head.set_inputs(*inputs)
    b = head.forward(M).clone()
    d = (a - b).abs().max() / a.abs().max()
    cos = torch.nn.functional.cosine_similarity(a.flatten(), b.flatten(), dim=0)
    assert d < 0.05 and cos > 0.999, f"reference sequence vs GELU epilogue: {d:.3e} {cos:.6f}"
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # eager first run on the capture stream (its workspaces)
        head.forward(M)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        head.forward(M)
    for _ in range(3):
        head.a_t.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(head.a_t, b), "graph replay differs from the eager forward"
        ref.forward(M)  # eager work between replays

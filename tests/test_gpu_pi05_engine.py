"""The whole pi05 forward (SigLIP vision tower -> Gemma-2B prefix -> action
expert) on the gfx950 kernels, reference instinctflash/engines/pi05/engine.py
(instinctflash_amd/pi05_engine.py). Reduced depth (2 vision, 2 prefix, 2 expert
layers, 2 Euler steps) at full width:

  * every vision-stage call against the oracle on the inputs it received:
    LayerNorm residuals bit-exact (float32) and FP8 rows within the reference
    test's bar (7% of the row max, tests/test_gi_kernels.py:112); GEMMs at the
    north-star bar (max|d| <= 2e-2 rms + one bf16 rounding, cosine >= 0.9999);
    q|k|v (fp16) and the projector rows (float32) from the GEMM epilogue at the
    GEMM bar; attention over each view's 256 patches at the fp16 bar
    (2e-3); requantization bit-exact. The prefix and expert calls are the same
    kernels checked call by call in test_gpu_prefix.py and test_gpu_pi05.py;
  * the reference call sequence against the default layout (GeGLU / GELU
    epilogues, tile layouts);
  * one captured graph replays the eager forward bit for bit, and follows a new
    prompt length inside the same row bucket."""
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


def _engine(gpu, seed, V=2, reference_calls=False, n=40):
    from instinctflash_amd.pi05_engine import LM_D, Pi05Engine, random_pi05_weights
    w = random_pi05_weights(gpu, vision_layers=2, prefix_layers=2, expert_layers=2, steps=2, seed=seed)
    eng = Pi05Engine(w, V, gpu, max_prompt=64, reference_calls=reference_calls)
    g = torch.Generator().manual_seed(seed + 1)
    eng.img.copy_(torch.rand(V, 3, 224, 224, generator=g) * 2 - 1)
    lang = torch.randn(64, LM_D, generator=g)
    eng.expert.noise.copy_(torch.randn(eng.expert.chunk, 32, generator=g))
    return eng, lang


class VisionChecker:
    def __init__(self, oracle):
        self.o, self.pre, self.seen = oracle, None, []

    def __call__(self, name, **t):
        torch.cuda.synchronize()
        o = self.o
        self.seen.append(name)
        if name == "pre_res":
            self.pre = _f(t["res"])
        elif name == "norm":
            kw = dict(layernorm=True, weight=_f(t["weight"]), beta=_f(t["beta"]), eps=1e-6)
            if "delta" in t:
                w = t["w"]
                kw.update(delta=_f(t["delta"]), delta_row=_f(t["delta_row"]), delta_col=_f(w.scale), bias=_f(w.bias))
            x_ref, y_ref = o.residual_norm(self.pre, **kw)
            assert np.array_equal(_f(t["res"]).view(np.uint32), x_ref.view(np.uint32)), "residual not bit-exact"
            deq = o.e4m3_decode(_u8(t["q"])) * _f(t["s"])[:, None]
            assert (np.abs(deq - y_ref).max(axis=1) / np.abs(y_ref).max(axis=1)).max() < 0.07
        elif name in ("gemm", "fc1", "qkv16", "projector"):
            a, w, out = t["a"], t["w"], t["out"]
            rows = np.sort(np.random.default_rng(a.shape[0]).choice(a.shape[0], 64, replace=False))
            ridx = torch.as_tensor(rows, device=out.device)
            sa = t.get("sa")
            ref = o.ref_linear(_u8(a[ridx]), None if sa is None else _f(sa)[rows], _u8(w.w),
                               None if sa is None else _f(w.scale), bias=None if sa is None else _f(w.bias),
                               act="gelu_tanh" if name == "fc1" else None)
            if out.dtype == torch.float16:  # the fp16 epilogue rounds once: one fp16 rounding allowance
                ref = ref.astype(np.float16).astype(np.float32)
            got = _f(out[ridx])
            _, cos = o.parity_stats(got, ref)
            rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
            excess = np.abs(got - ref) - (2e-2 * rms + 2.0 ** -8 * np.abs(ref))
            assert excess.max() <= 0 and cos >= 0.9999, f"{name} {tuple(w.w.shape)}: {excess.max():.3e} {cos:.7f}"
        elif name == "dequant":
            f32 = np.float32
            w, y = t["w"], t["y"]
            ref = ((_f(t["x"]) * _f(t["row"])[:, None]).astype(f32) * _f(w.scale)[None, :]).astype(f32)
            ref = (ref + _f(w.bias)[None, :]).astype(f32)
            got = y.detach().cpu().numpy()
            if y.dtype == torch.float16:
                assert np.array_equal(got.view(np.uint16), ref.astype(np.float16).view(np.uint16)), "fp16 rows"
            else:
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "float32 rows"
        elif name == "attention":
            q = _f(t["q"])
            ref = o.attention(q, _f(t["k"]), _f(t["v"]), np.full(q.shape[1], q.shape[1]), q.shape[3] ** -0.5)
            err = np.abs(_f(t["out"]) - ref).max()
            assert err < 2e-3, f"attention: max |d| {err:.3e}"
        elif name == "row_quant":
            x = t["x"]
            eq, es = o.quant_rows(_bits(x) if x.dtype == torch.bfloat16 else _f(x))
            assert np.array_equal(_u8(t["q"]), eq) and np.array_equal(_f(t["s"]).view(np.uint32), es.view(np.uint32))
        else:
            raise AssertionError(f"unchecked call {name}")


def test_vision_calls_against_oracle(gpu, oracle_mod):
    eng, lang = _engine(gpu, seed=1)
    M = eng.set_prompt(lang[:40])
    print(f"[pi05 engine] V={eng.V} rows={M}", flush=True)
    chk = VisionChecker(oracle_mod)
    x = eng.forward(M, on_call=chk)
    assert chk.seen.count("attention") == 2 and chk.seen.count("qkv16") == 2 and chk.seen.count("projector") == 1
    assert torch.isfinite(x).all() and torch.isfinite(eng.px[:M]).all()


def test_reference_calls_agree(gpu):
    a_eng, lang = _engine(gpu, seed=3, reference_calls=True)
    b_eng, _ = _engine(gpu, seed=3)
    M = a_eng.set_prompt(lang[:40])
    b_eng.set_prompt(lang[:40])
    a = a_eng.forward(M).clone()
    b = b_eng.forward(M).clone()
    pa, pb = a_eng.px[:M], b_eng.px[:M]
    cos = lambda u, v: float(torch.nn.functional.cosine_similarity(u.flatten().double(), v.flatten().double(), dim=0))  # noqa: E731
    # two valid forms of the same math: the reference rounds the raw fc1 / gate|up
    # accumulators to bf16 before GELU / GeGLU, so some requantized e4m3 codes differ
    # and the residual streams drift apart layer by layer (measured: vision stream
    # 0.9995, projected rows 0.9989, prefix rows 0.997 after 2 + 1 layers of random
    # weights; every call of each form is pinned to the oracle separately)
    assert cos(pa, pb) > 0.995 and cos(a, b) > 0.999, (cos(pa, pb), cos(a, b))


def test_graph_replay_and_prompt_length(gpu):
    eng, lang = _engine(gpu, seed=5)
    M = eng.set_prompt(lang[:40])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eng.forward(M)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    eager = eng.x_t.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        eng.forward(M)
    for _ in range(2):
        eng.x_t.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(eng.x_t, eager), "replay differs from the eager forward"
    # a shorter prompt in the same 16-row bucket: the graph follows the device length
    assert eng.set_prompt(lang[:35]) == M
    graph.replay()
    torch.cuda.synchronize()
    replayed = eng.x_t.clone()
    eng.forward(M)
    torch.cuda.synchronize()
    assert torch.equal(replayed, eng.x_t) and not torch.equal(replayed, eager)

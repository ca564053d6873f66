"""GPU parity of ``qkv_split`` (reference instinctflash/kernels/rope.py:89-116)
against the CPU oracle (float64 after the reference's float32 rescale and
float32 rotary angles).

Bar: |out - ref| <= u * |ref| + 2e-5, u = the output format's unit roundoff x2
(bf16 2^-7, fp16 2^-10, fp32 2e-5 -- the fp32 case is bounded by the device's
sqrt / sincos and summation order); K/V cache rows outside [kv_base, kv_base+T)
must stay untouched.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

U = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2e-5}


def _case(T, HQ, HKV, HD, seed, in_dtype=torch.bfloat16, rope=True, norm=True, sections=True, big_pos=False):
    from instinctflash_amd.kernels.rope import rope_inv_freq
    g = torch.Generator().manual_seed(seed)
    C = (HQ + 2 * HKV) * HD
    c = dict(raw=torch.randn(T, C, generator=g).to(in_dtype), row=torch.rand(T, generator=g) + 0.5,
             col=torch.rand(C, generator=g) + 0.5, bias=torch.randn(C, generator=g))
    if norm:
        c["q_norm"], c["k_norm"] = torch.rand(HD, generator=g) + 0.5, torch.rand(HD, generator=g) + 0.5
    if rope:
        c["inv_freq"] = rope_inv_freq(HD, 1e6, "cpu")
        scale = 4099.0 if big_pos else 1.0
        c["pos"] = (torch.stack([torch.arange(T), torch.arange(T) * 2, torch.arange(T) * 3], 1) * scale).float()
        if sections:
            c["sections"] = (torch.arange(HD // 2) % 3).int()
        else:
            c["pos"] = c["pos"][:, :1].contiguous()
    return c


def _run(gpu, c, HQ, HKV, HD, out_dtype, kv_base, S, q_view=False):
    from instinctflash_amd.kernels import qkv_split
    T = c["raw"].shape[0]
    d = {k: v.to(gpu) for k, v in c.items()}
    if q_view:  # a strided view of a wider buffer
        qbuf = torch.zeros(T, HQ + 1, HD + 8, device=gpu, dtype=out_dtype)
        q = qbuf[:, :HQ, :HD]
    else:
        q = torch.empty(T, HQ, HD, device=gpu, dtype=out_dtype)
    kc = torch.full((S, HKV, HD), 7.0, device=gpu, dtype=out_dtype)
    vc = torch.full_like(kc, 7.0)
    qkv_split(d["raw"], q, kc, vc, heads_q=HQ, heads_kv=HKV, head_dim=HD, row=d["row"], col=d["col"],
              bias=d["bias"], inv_freq=d.get("inv_freq"), pos=d.get("pos"), sections=d.get("sections"),
              q_norm=d.get("q_norm"), k_norm=d.get("k_norm"), kv_base=kv_base)
    torch.cuda.synchronize()
    return q, kc, vc


def _ref(oracle_mod, c, HQ, HKV, HD):
    n = lambda k: None if k not in c else c[k].float().numpy() if k != "sections" else c[k].numpy()  # noqa: E731
    return oracle_mod.qkv_split(c["raw"].float().numpy(), HQ, HKV, HD, n("row"), n("col"), n("bias"), n("inv_freq"),
                                n("pos"), n("sections"), n("q_norm"), n("k_norm"))


def _close(got, ref, dt, what):
    g = got.float().cpu().numpy().astype(np.float64)
    err = np.abs(g - ref) - (U[dt] * np.abs(ref) + 2e-5)
    assert err.max() <= 0, f"{what}: worst excess {err.max():.3e}"


def _check(gpu, oracle_mod, c, HQ, HKV, HD, out_dtype, kv_base, S, what, q_view=False):
    T = c["raw"].shape[0]
    base = kv_base.item() if torch.is_tensor(kv_base) else kv_base
    q, kc, vc = _run(gpu, c, HQ, HKV, HD, out_dtype, kv_base if not torch.is_tensor(kv_base) else kv_base.to(gpu),
                     S, q_view)
    rq, rk, rv = _ref(oracle_mod, c, HQ, HKV, HD)
    _close(q, rq, out_dtype, f"{what}: q")
    _close(kc[base:base + T], rk, out_dtype, f"{what}: k")
    _close(vc[base:base + T], rv, out_dtype, f"{what}: v")
    for t in (kc, vc):  # rows outside the written range keep their contents
        assert (t[:base] == 7.0).all() and (t[base + T:] == 7.0).all(), f"{what}: cache rows outside written"


def test_reference_case(gpu, oracle_mod):
    # tests/test_gi_kernels.py:58-90: fp16 outputs, device kv_base 9, cache of 20 rows
    c = _case(7, 4, 2, 128, 2)
    _check(gpu, oracle_mod, c, 4, 2, 128, torch.float16, torch.tensor([9], dtype=torch.int32), 20, "reference case")


@pytest.mark.parametrize("HD", [64, 96, 128, 256])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_head_dims_and_dtypes(gpu, oracle_mod, HD, out_dtype):
    c = _case(11, 8, 2, HD, HD)
    _check(gpu, oracle_mod, c, 8, 2, HD, out_dtype, 5, 32, f"HD={HD} {out_dtype}")


@pytest.mark.parametrize("opts", [dict(rope=False, norm=False), dict(rope=True, norm=False), dict(rope=False, norm=True),
                                  dict(rope=True, norm=True, sections=False), dict(big_pos=True),
                                  dict(in_dtype=torch.float32)])
def test_options(gpu, oracle_mod, opts):
    c = _case(16, 16, 2, 128, 7, **opts)
    _check(gpu, oracle_mod, c, 16, 2, 128, torch.bfloat16, 0, 16, f"options {opts}")


def test_strided_q_and_pi05_shape(gpu, oracle_mod):
    # pi05: 8 query heads, 1 KV head, head_dim 256, qkv width 2560
    c = _case(50, 8, 1, 256, 3)
    _check(gpu, oracle_mod, c, 8, 1, 256, torch.bfloat16, 100, 200, "pi05 shape, strided q", q_view=True)


def test_graph_follows_device_kv_base(gpu, oracle_mod):
    from instinctflash_amd.kernels import qkv_split
    HQ, HKV, HD, T = 4, 2, 64, 5
    c = {k: v.to(gpu) for k, v in _case(T, HQ, HKV, HD, 9).items()}
    q = torch.empty(T, HQ, HD, device=gpu, dtype=torch.bfloat16)
    kc = torch.zeros(40, HKV, HD, device=gpu, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    base = torch.tensor([3], device=gpu, dtype=torch.int32)
    kw = dict(heads_q=HQ, heads_kv=HKV, head_dim=HD, row=c["row"], col=c["col"], bias=c["bias"],
              inv_freq=c["inv_freq"], pos=c["pos"], sections=c["sections"], q_norm=c["q_norm"], k_norm=c["k_norm"],
              kv_base=base)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        qkv_split(c["raw"], q, kc, vc, **kw)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    first = kc[3:3 + T].clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        qkv_split(c["raw"], q, kc, vc, **kw)
    for b in (11, 20, 3):
        kc.zero_()
        base.fill_(b)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(kc[b:b + T], first) and kc[:b].abs().max() == 0 and kc[b + T:].abs().max() == 0


def test_contract_errors(gpu):
    from instinctflash_amd.kernels import qkv_split
    raw = torch.zeros(2, 8 * 64, device=gpu, dtype=torch.bfloat16)
    q = torch.empty(2, 4, 64, device=gpu, dtype=torch.bfloat16)
    kc = torch.empty(4, 2, 64, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="share a dtype"):
        qkv_split(raw, q, kc.half(), kc, heads_q=4, heads_kv=2, head_dim=64)
    with pytest.raises(ValueError, match="position table"):
        qkv_split(raw, q, kc, kc, heads_q=4, heads_kv=2, head_dim=64, inv_freq=torch.ones(32, device=gpu))
    with pytest.raises(ValueError, match="columns"):
        qkv_split(raw, q, kc, kc, heads_q=4, heads_kv=1, head_dim=64)
    with pytest.raises(ValueError, match="rows"):
        qkv_split(raw, q, kc, kc, heads_q=4, heads_kv=2, head_dim=64, kv_base=3)

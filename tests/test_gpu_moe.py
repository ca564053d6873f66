"""GPU parity of the MoE routing kernels (reference
instinctflash/kernels/activation.py:71-137 and the router option of
kernels/norm.py:84-94) against the CPU oracle.

Bars:
  * moe_router: |route_w - oracle| <= 1e-5 (the reference test's bar,
    tests/test_gi_kernels.py:192) on every token whose top_k boundary is not a
    near tie (selection-score gap >= 1e-5 between the k-th and (k+1)-th expert;
    there float32 dot products may legitimately pick either); on exact ties the
    lowest expert index wins, checked bit for bit;
  * the fused router of residual_norm_quant equals moe_router on the float32 y
    bit for bit;
  * moe_act_quant: per-row scale within 8 float32 ulps of the oracle recipe on
    the oracle activation, >= 99.9% identical bytes, and the dequantized rows
    within 0.07 of the row max (tests/test_gi_kernels.py:203).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _router_case(M, D, E, seed, x_dtype=torch.float32, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, D, generator=g).to(x_dtype)
    gw = torch.randn(E, D, generator=g) * (0.05 * (768 / D) ** 0.5)
    eb = torch.rand(E, generator=g) * 0.01 if bias else torch.zeros(E)
    return x, gw, eb


def _check_router(got, x, gw, eb, K, scale, oracle_mod):
    ref, sel = oracle_mod.moe_router(x.float().numpy(), gw.numpy(), eb.numpy(), K, scale)
    got = got.cpu().numpy()
    srt = -np.sort(-sel, axis=1)
    clear = np.ones(len(sel), bool) if K in (0, sel.shape[1]) else (srt[:, K - 1] - srt[:, K]) >= 1e-5
    assert clear.mean() > 0.8, "too many near-tie tokens for a meaningful check"
    err = np.abs(got - ref)[clear].max(initial=0.0)
    assert err < 1e-5, f"max |d| {err:.3e}"
    assert ((got != 0).sum(1) <= K).all()


def test_router_reference_case(gpu, oracle_mod):
    # tests/test_gi_kernels.py:179-192
    from instinctflash_amd.kernels import moe_router
    x, gw, eb = _router_case(51, 768, 32, 7, bias=False)
    rw = torch.empty(51, 32, device=gpu)
    moe_router(x.to(gpu), gw.to(gpu), eb.to(gpu), rw, top_k=4, scale=4.0)
    _check_router(rw, x, gw, eb, 4, 4.0, oracle_mod)


@pytest.mark.parametrize("M,D,E,K,xd", [(1, 768, 32, 4, torch.float32), (64, 2048, 64, 8, torch.bfloat16),
                                        (37, 1024, 100, 6, torch.float32), (8, 16384, 256, 8, torch.bfloat16),
                                        (5, 64, 3, 3, torch.float32), (5, 520, 16, 0, torch.float32)])
def test_router_shapes(gpu, oracle_mod, M, D, E, K, xd):
    from instinctflash_amd.kernels import moe_router
    x, gw, eb = _router_case(M, D, E, M + D + E, xd)
    rw = torch.full((M, E), 9.0, device=gpu)
    moe_router(x.to(gpu), gw.to(gpu), eb.to(gpu), rw, top_k=K, scale=2.5)
    _check_router(rw, x, gw, eb, K, 2.5, oracle_mod)


def test_router_ties_pick_lowest_index(gpu):
    from instinctflash_amd.kernels import moe_router
    E, K = 70, 5
    x = torch.zeros(3, 256, device=gpu)
    gw = torch.randn(E, 256, device=gpu)
    eb = torch.zeros(E, device=gpu)
    eb[[66, 69]] = 1.0  # two clear winners past the first wave lane block, then ties
    rw = torch.empty(3, E, device=gpu)
    moe_router(x, gw, eb, rw, top_k=K, scale=1.0)
    exp = torch.zeros(3, E)
    exp[:, [0, 1, 2, 66, 69]] = 0.2  # all sigmoids are 0.5
    assert torch.equal(rw.cpu(), exp)


def test_router_strided_rows(gpu, oracle_mod):
    from instinctflash_amd.kernels import moe_router
    x, gw, eb = _router_case(20, 512, 24, 4)
    buf = torch.zeros(20, 600, device=gpu)
    buf[:, :512] = x.to(gpu)
    rw = torch.empty(20, 24, device=gpu)
    moe_router(buf[:, :512], gw.to(gpu), eb.to(gpu), rw, top_k=3, scale=1.0)
    _check_router(rw, x, gw, eb, 3, 1.0, oracle_mod)


@pytest.mark.parametrize("res_dtype,y_dtype,E,D", [(torch.float32, torch.float32, 32, 768),
                                                   (torch.bfloat16, torch.bfloat16, 32, 768),
                                                   (torch.float32, None, 32, 768), (torch.float32, None, 48, 768),
                                                   (torch.bfloat16, torch.float32, 16, 2048),
                                                   (torch.float32, None, 16, 4096), (torch.bfloat16, torch.float32, 16, 8192),
                                                   (torch.float32, torch.bfloat16, 8, 12288)])
def test_fused_router_matches_standalone(gpu, res_dtype, y_dtype, E, D):
    # tests/test_gi_kernels.py:206-216, plus bf16 residual / y, no y at all, and
    # shapes outside the prefetched-weights path (E > 32, D > 1024): the fused
    # weights equal moe_router on the float32 normalized row.
    from instinctflash_amd.kernels import E4M3, moe_router, residual_norm_quant
    g = torch.Generator().manual_seed(8)
    M = 51
    res = torch.randn(M, D, generator=g).to(res_dtype).to(gpu)
    delta = torch.randn(M, D, generator=g).to(torch.bfloat16).to(gpu)
    ms, mh = (torch.randn(D, generator=g) * 0.1).to(gpu), (torch.randn(D, generator=g) * 0.1).to(gpu)
    gw, eb = (torch.randn(E, D, generator=g) * 0.05).to(gpu), (torch.rand(E, generator=g) * 0.01).to(gpu)
    kw = dict(delta=delta, mod_scale=ms, mod_shift=mh)
    q = torch.empty(M, D, device=gpu, dtype=E4M3)
    qs = torch.empty(M, device=gpu)
    y = None if y_dtype is None else torch.empty(M, D, device=gpu, dtype=y_dtype)
    rw_fused, rw_ref = torch.empty(M, E, device=gpu), torch.empty(M, E, device=gpu)
    r1 = res.clone()
    residual_norm_quant(r1, q=q, q_scale=qs, y=y, router=(gw, eb, rw_fused, 4, 4.0), **kw)
    # the same producer without the router, y in float32, then the standalone router
    r2 = res.clone()
    y32 = torch.empty(M, D, device=gpu)
    q2, qs2 = torch.empty_like(q), torch.empty_like(qs)
    residual_norm_quant(r2, q=q2, q_scale=qs2, y=y32, **kw)
    moe_router(y32, gw, eb, rw_ref, top_k=4, scale=4.0)
    torch.cuda.synchronize()
    assert torch.equal(rw_fused, rw_ref)
    assert torch.equal(r1, r2) and torch.equal(qs, qs2) and torch.equal(q.view(torch.uint8), q2.view(torch.uint8))
    if y is not None:
        assert torch.equal(y, y32.to(y_dtype))


def _act_case(M, E, G, S, seed):
    g = torch.Generator().manual_seed(seed)
    F = E * G + S
    gu = torch.randn(M, 2 * F, generator=g).to(torch.bfloat16)
    row, col = torch.rand(M, generator=g) + 0.5, torch.rand(2 * F, generator=g) + 0.5
    rw = torch.rand(M, E, generator=g)
    rw[rw < 0.5] = 0.0  # unselected experts contribute exactly zero
    return gu, row, col, rw


def _check_act(gpu, oracle_mod, gu, row, col, rw, E, G, NR):
    from instinctflash_amd.kernels import moe_act_quant
    M, F = gu.shape[0], gu.shape[1] // 2
    q = torch.empty(M, F, device=gpu, dtype=torch.float8_e4m3fn)
    qs = torch.empty(M, device=gpu)
    moe_act_quant(gu.to(gpu), q, qs, rw.to(gpu), row=row.to(gpu), col=None if col is None else col.to(gpu),
                  experts=E, group=G, n_routed=NR)
    torch.cuda.synchronize()
    cn = np.ones(2 * F, np.float32) if col is None else col.numpy()  # no column scale: x 1.0 is exact
    h = oracle_mod.moe_act(gu.float().numpy(), row.numpy(), cn, rw.numpy(), E, G, NR)
    eq, es = oracle_mod.quant_rows(h)
    got_s = qs.cpu().numpy()
    assert np.all(np.abs(got_s.view(np.int32).astype(np.int64) - es.view(np.int32)) <= 8)
    gq = q.cpu().view(torch.uint8).numpy()
    assert (gq == eq).mean() > 0.999
    deq = q.float().cpu().numpy() * got_s[:, None]
    assert (np.abs(deq - h) / np.abs(h).max(axis=1, keepdims=True)).max() < 0.07
    # columns of unselected routed experts quantize to exact zero
    grp = np.minimum(np.arange(F) // G, E - 1)
    dead = (rw.numpy()[:, grp] == 0) & (np.arange(F)[None, :] < NR)
    assert (gq[dead] & 0x7F == 0).all()


def test_act_reference_case(gpu, oracle_mod):
    # tests/test_gi_kernels.py:193-203 (the vla2 engine's MoE: 32 experts x 512 + 704 shared)
    E, G, S = 32, 512, 704
    gu, row, col, rw = _act_case(51, E, G, S, 9)
    _check_act(gpu, oracle_mod, gu, row, col, rw, E, G, E * G)


@pytest.mark.parametrize("M,E,G,S,nr", [(4, 8, 512, 512, None), (300, 8, 128, 64, None), (3, 4, 64, 40, "all"),
                                        (7, 6, 24, 0, None)])
def test_act_shapes(gpu, oracle_mod, M, E, G, S, nr):
    gu, row, col, rw = _act_case(M, E, G, S, M + E)
    F = E * G + S
    _check_act(gpu, oracle_mod, gu, row, col, rw, E, G, F if nr == "all" else E * G)


@pytest.mark.parametrize("M,E,G,S", [(4, 8, 512, 512), (300, 8, 128, 64), (40, 32, 512, 704)])
def test_act_without_column_scale(gpu, oracle_mod, M, E, G, S):
    gu, row, _, rw = _act_case(M, E, G, S, M + G)
    _check_act(gpu, oracle_mod, gu, row, None, rw, E, G, E * G)


def test_contract_errors(gpu):
    from instinctflash_amd.kernels import moe_act_quant, moe_router, residual_norm_quant
    x = torch.zeros(4, 256, device=gpu)
    gw, eb, rw = torch.zeros(8, 256, device=gpu), torch.zeros(8, device=gpu), torch.empty(4, 8, device=gpu)
    with pytest.raises(ValueError, match="top_k"):
        moe_router(x, gw, eb, rw, top_k=9, scale=1.0)
    with pytest.raises(ValueError, match="gate_w"):
        moe_router(x, gw.half(), eb, rw, top_k=2, scale=1.0)
    with pytest.raises(ValueError, match="route_w"):
        moe_router(x, gw, eb, rw[:3], top_k=2, scale=1.0)
    with pytest.raises(ValueError, match="router"):
        residual_norm_quant(x.clone(), router=(gw, eb, rw, 2))
    gu = torch.zeros(4, 2 * 96, device=gpu, dtype=torch.bfloat16)
    q = torch.empty(4, 96, device=gpu, dtype=torch.float8_e4m3fn)
    qs = torch.empty(4, device=gpu)
    with pytest.raises(ValueError, match="n_routed"):
        moe_act_quant(gu, q, qs, rw, row=None, col=None, experts=8, group=8, n_routed=97)

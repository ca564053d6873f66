"""The producers' tile-layout outputs (row stride IFX_LD_TILED): row_quant,
gated_act_quant, moe_act_quant, residual_norm_quant and attention's fused q8
write the same bytes and scales as their row-major outputs, placed in the
skinny tile layout of quant_rows_tiled (zeros in the row and K padding), and
the M <= 64 GEMM reads them bit-identically."""
import numpy as np
import pytest
import torch

from test_gpu_gemm import _tile_rows_np

pytestmark = pytest.mark.gpu


def _tiled(M, K, gpu):
    from instinctflash_amd import _lib
    from instinctflash_amd.kernels import TiledRows
    n = _lib.load().ifx_quant_rows_tiled_bytes(M, K)
    return TiledRows(torch.full((n,), 0x7F, dtype=torch.uint8, device=gpu).view(torch.float8_e4m3fn), M, K)


def _same(tq, q, M, K):
    got = tq.q.view(torch.uint8).cpu().numpy()
    exp = _tile_rows_np(q.view(torch.uint8).cpu().numpy(), M, K).reshape(-1)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("M,K,dtype,gelu", [(50, 2048, torch.float16, False), (16, 6144, torch.bfloat16, True),
                                            (7, 144, torch.bfloat16, False), (64, 1040, torch.float16, True)])
def test_row_quant(gpu, M, K, dtype, gelu):
    from instinctflash_amd.kernels import row_quant
    g = torch.Generator().manual_seed(M + K)
    x = (torch.randn(M, K, generator=g) * 2).to(dtype).to(gpu)
    col = (torch.rand(K, generator=g) + 0.5).to(gpu)
    q = torch.empty(M, K, device=gpu, dtype=torch.float8_e4m3fn)
    s, ts = torch.empty(M, device=gpu), torch.empty(M, device=gpu)
    tq = _tiled(M, K, gpu)
    row_quant(x, q, s, col=col, gelu=gelu)
    row_quant(x, tq, ts, col=col, gelu=gelu)
    assert torch.equal(s, ts)
    _same(tq, q, M, K)


@pytest.mark.parametrize("M,F", [(50, 4096), (16, 3072), (5, 1040)])
def test_gated_and_moe(gpu, M, F):
    from instinctflash_amd.kernels import gated_act_quant, moe_act_quant
    g = torch.Generator().manual_seed(M + F)
    gu = torch.randn(M, 2 * F, generator=g).to(torch.bfloat16).to(gpu)
    row, col = (torch.rand(M, generator=g) + 0.5).to(gpu), (torch.rand(2 * F, generator=g) + 0.5).to(gpu)
    q = torch.empty(M, F, device=gpu, dtype=torch.float8_e4m3fn)
    s, ts = torch.empty(M, device=gpu), torch.empty(M, device=gpu)
    tq = _tiled(M, F, gpu)
    gated_act_quant(gu, q, s, row=row, col=col)
    gated_act_quant(gu, tq, ts, row=row, col=col)
    assert torch.equal(s, ts)
    _same(tq, q, M, F)
    E, G = 4, 8 * (F // 64)  # group % 8 == 0: the vector path, the only one with a tile-layout output
    rw = torch.rand(M, E, generator=g).to(gpu)
    moe_act_quant(gu, q, s, rw, row=row, col=col, experts=E, group=G, n_routed=E * G)
    tq = _tiled(M, F, gpu)
    moe_act_quant(gu, tq, ts, rw, row=row, col=col, experts=E, group=G, n_routed=E * G)
    assert torch.equal(s, ts)
    _same(tq, q, M, F)


@pytest.mark.parametrize("M,D,router", [(50, 1024, False), (16, 1536, True), (3, 208, False)])
def test_residual_norm_quant(gpu, M, D, router):
    from instinctflash_amd.kernels import residual_norm_quant
    g = torch.Generator().manual_seed(M + D)
    res = torch.randn(M, D, generator=g).to(gpu)
    delta = torch.randn(M, D, generator=g).to(torch.bfloat16).to(gpu)
    ms, mh = (torch.randn(D, generator=g) * 0.1).to(gpu), (torch.randn(D, generator=g) * 0.1).to(gpu)
    E = 16
    gw, eb = (torch.randn(E, D, generator=g) * 0.05).to(gpu), torch.zeros(E, device=gpu)
    outs = []
    for tiled in (False, True):
        r = res.clone()
        q = _tiled(M, D, gpu) if tiled else torch.empty(M, D, device=gpu, dtype=torch.float8_e4m3fn)
        s = torch.empty(M, device=gpu)
        rw = torch.empty(M, E, device=gpu)
        residual_norm_quant(r, delta=delta, mod_scale=ms, mod_shift=mh, q=q, q_scale=s,
                            router=(gw, eb, rw, 4, 1.0) if router else None)
        outs.append((r, q, s, rw))
    (r0, q0, s0, w0), (r1, q1, s1, w1) = outs
    assert torch.equal(r0, r1) and torch.equal(s0, s1)
    if router:
        assert torch.equal(w0, w1)
    _same(q1, q0, M, D)


def test_attention_q8(gpu):
    from instinctflash_amd.kernels import SplitWorkspace, attention
    g = torch.Generator().manual_seed(11)
    T, H, D = 50, 8, 256
    q = torch.randn(1, T, H, D, generator=g).to(torch.bfloat16).to(gpu)
    k = torch.randn(1, 300, 1, D, generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn(1, 300, 1, D, generator=g).to(torch.bfloat16).to(gpu)
    ws = SplitWorkspace(1, T, H, 1, D, 4, gpu)
    q8 = torch.empty(T, H * D, device=gpu, dtype=torch.float8_e4m3fn)
    s, ts = torch.empty(T, device=gpu), torch.empty(T, device=gpu)
    tq = _tiled(T, H * D, gpu)
    attention(q, k, v, split=ws, q8=q8, q8_scale=s)
    attention(q, k, v, split=ws, q8=tq, q8_scale=ts)
    assert torch.equal(s, ts)
    _same(tq, q8, T, H * D)

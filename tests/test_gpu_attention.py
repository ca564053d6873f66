"""GPU parity of ``attention`` (reference instinctflash/kernels/attention.py:23-213)
against the float64 CPU oracle.

Bars: max |out - ref| < 2e-3 for fp16 operands (the reference test's bar,
tests/test_gi_kernels.py:41), < 2^-7 for bf16 (probabilities and outputs carry
bf16 rounding, 2^-9 relative each); the fused FP8 row within 0.07 of the row max
(tests/test_gi_kernels.py:176) with its scale within 1% of the recipe applied to
the reference row.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

BAR = {torch.float16: 2e-3, torch.bfloat16: 2.0 ** -7}


def _qkv(B, Tq, Tk, hq, hkv, hd, seed, dtype=torch.float16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Tq, hq, hd, generator=g).to(dtype)
    k = torch.randn(B, Tk, hkv, hd, generator=g).to(dtype)
    v = torch.randn(B, Tk, hkv, hd, generator=g).to(dtype)
    return q, k, v


def _ref(oracle_mod, q, k, v, limits, scale=None, kv_index=None):
    hd = q.shape[-1]
    return oracle_mod.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), np.asarray(limits),
                                hd ** -0.5 if scale is None else scale,
                                None if kv_index is None else kv_index.numpy())


def _close(out, ref, dtype, what=""):
    err = np.abs(out.float().cpu().numpy() - ref).max()
    assert err < BAR[dtype], f"{what} max |d| {err:.3e}"


@pytest.mark.parametrize("hd,hq,hkv", [(256, 8, 1), (72, 16, 16), (128, 16, 2)])
def test_dynamic_length(gpu, oracle_mod, hd, hq, hkv):
    # tests/test_gi_kernels.py:32-41
    from instinctflash_amd.kernels import attention
    q, k, v = _qkv(2, 40, 64, hq, hkv, hd, 0)
    n = torch.tensor([53], device=gpu, dtype=torch.int32)
    out = attention(q.to(gpu), k.to(gpu), v.to(gpu), kv_len=n, config=(32, 32, 4, 2))
    _close(out, _ref(oracle_mod, q, k, v, np.full(40, 53)), torch.float16)


def test_causal_and_extra(gpu, oracle_mod):
    # tests/test_gi_kernels.py:44-55
    from instinctflash_amd.kernels import attention
    q, k, v = _qkv(1, 20, 48, 4, 2, 128, 1)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    out = attention(qd, kd, vd, causal=True, causal_offset=5, config=(16, 16, 4, 1))
    lim = np.minimum(48, np.arange(20) + 6)
    _close(out, _ref(oracle_mod, q, k, v, lim), torch.float16, "causal")
    extra = torch.tensor([1] + [11] * 19, dtype=torch.int32)
    base = torch.tensor([30], device=gpu, dtype=torch.int32)
    out = attention(qd, kd, vd, kv_len=base, kv_extra=extra.to(gpu), max_extra=11, config=(16, 16, 4, 1))
    _close(out, _ref(oracle_mod, q, k, v, 30 + extra.numpy()), torch.float16, "extra")


@pytest.mark.parametrize("hd,hq,hkv,splits", [(256, 8, 1, 3), (128, 16, 2, 2), (72, 16, 16, 4), (128, 40, 8, 5),
                                              (32, 4, 1, 2)])
def test_split_with_fused_quant(gpu, oracle_mod, hd, hq, hkv, splits):
    # combine widths: 1280 / 512 / 288 / 32 four-dim groups per token row
    # tests/test_gi_kernels.py:157-176
    from instinctflash_amd.kernels import SplitWorkspace, attention
    T = 50
    q, k, v = _qkv(1, T, 700, hq, hkv, hd, 6)
    base = torch.tensor([600], device=gpu, dtype=torch.int32)
    extra = torch.tensor([1] + [T] * (T - 1), dtype=torch.int32)
    ws = SplitWorkspace(1, T, hq, hkv, hd, splits, gpu)
    out = torch.empty(1, T, hq, hd, device=gpu, dtype=torch.float16)
    q8 = torch.empty(T, hq * hd, device=gpu, dtype=torch.float8_e4m3fn)
    qs = torch.empty(T, device=gpu)
    attention(q.to(gpu), k.to(gpu), v.to(gpu), out=out, kv_len=base, kv_extra=extra.to(gpu), max_extra=T,
              split=ws, q8=q8, q8_scale=qs, config=(32, 64, 4, 2))
    ref = _ref(oracle_mod, q, k, v, 600 + extra.numpy())
    _close(out, ref, torch.float16, "split out")
    r = ref.reshape(T, -1)
    deq = q8.float().cpu().numpy() * qs.cpu().numpy()[:, None]
    assert (np.abs(deq - r) / np.abs(r).max(axis=1, keepdims=True)).max() < 0.07
    _, es = oracle_mod.quant_rows(r.astype(np.float32))
    assert np.abs(qs.cpu().numpy() / es - 1).max() < 1e-2
    # q8 alone (no out): same bytes
    q8b, qsb = torch.empty_like(q8), torch.empty_like(qs)
    attention(q.to(gpu), k.to(gpu), v.to(gpu), kv_len=base, kv_extra=extra.to(gpu), max_extra=T, split=ws,
              q8=q8b, q8_scale=qsb)
    assert torch.equal(q8b.view(torch.uint8), q8.view(torch.uint8)) and torch.equal(qsb, qs)


@pytest.mark.parametrize("B,Tq,Tk,hq,hkv,hd,splits", [(1, 800, 800, 8, 1, 256, 1), (2, 51, 900, 8, 1, 256, 4),
                                                      (1, 1, 2000, 16, 2, 128, 8), (3, 17, 130, 12, 4, 64, 1),
                                                      (1, 33, 65, 4, 4, 96, 2), (1, 5, 7, 2, 1, 32, 1),
                                                      (1, 40, 300, 4, 2, 160, 3), (1, 33, 129, 2, 1, 200, 1),
                                                      (2, 17, 70, 4, 4, 224, 2), (1, 70, 1, 8, 1, 256, 1)])
def test_shapes_bf16(gpu, oracle_mod, B, Tq, Tk, hq, hkv, hd, splits):
    from instinctflash_amd.kernels import SplitWorkspace, attention
    q, k, v = _qkv(B, Tq, Tk, hq, hkv, hd, Tq + Tk, torch.bfloat16)
    ws = SplitWorkspace(B, Tq, hq, hkv, hd, splits, gpu) if splits > 1 else None
    out = attention(q.to(gpu), k.to(gpu), v.to(gpu), split=ws)
    _close(out, _ref(oracle_mod, q, k, v, np.full(Tq, Tk)), torch.bfloat16, f"B{B} Tq{Tq} Tk{Tk} hd{hd}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hd,hq,hkv,Tq,splits", [(160, 4, 2, 40, 2), (192, 4, 1, 33, 1), (192, 8, 2, 20, 3),
                                                 (224, 2, 2, 17, 2), (256, 16, 2, 9, 2)])
def test_head_dim_forms(gpu, oracle_mod, dtype, hd, hq, hkv, Tq, splits):
    # head dims 160-224 (5-7 32-dim slices per lane group) in both operand types,
    # and the split combine at its widest (16 heads x 256 dims over few tokens)
    from instinctflash_amd.kernels import SplitWorkspace, attention
    Tk = 150
    q, k, v = _qkv(1, Tq, Tk, hq, hkv, hd, hd + hq + Tq, dtype)
    ws = SplitWorkspace(1, Tq, hq, hkv, hd, splits, gpu) if splits > 1 else None
    out = attention(q.to(gpu), k.to(gpu), v.to(gpu), split=ws)
    _close(out, _ref(oracle_mod, q, k, v, np.full(Tq, Tk)), dtype, f"hd{hd} hq{hq} {dtype}")


def test_engine_views_and_pooled_index(gpu, oracle_mod):
    # q/k/v as strided views of one fused buffer (engines/pi05/engine.py:174), a
    # custom scale, and a pooled cache read through kv_index (wan_va/engine.py:218)
    from instinctflash_amd.kernels import attention
    g = torch.Generator().manual_seed(4)
    B, T, H, HD = 2, 37, 4, 128
    qkv = torch.randn(B, T, 3, H, HD, generator=g).to(torch.bfloat16)
    d = qkv.to(gpu)
    out = torch.empty(B, T, H, HD, device=gpu, dtype=torch.bfloat16)
    attention(d[:, :, 0], d[:, :, 1], d[:, :, 2], out=out, scale=0.05)
    _close(out, _ref(oracle_mod, qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], np.full(T, T), scale=0.05),
           torch.bfloat16, "views")
    q, k, v = _qkv(1, 9, 64, 4, 2, 64, 5, torch.bfloat16)
    idx = torch.tensor([63, 2, 5, 5, 40, 0, 17, 33, 8, 9, 60], dtype=torch.int32)
    out = attention(q.to(gpu), k.to(gpu), v.to(gpu), kv_len=11, kv_index=idx.to(gpu))
    _close(out, _ref(oracle_mod, q, k, v, np.full(9, 11), kv_index=idx), torch.bfloat16, "kv_index")


def test_graph_follows_device_kv_len(gpu, oracle_mod):
    from instinctflash_amd.kernels import SplitWorkspace, attention
    q, k, v = _qkv(1, 50, 300, 8, 1, 256, 8, torch.bfloat16)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    n = torch.tensor([100], device=gpu, dtype=torch.int32)
    ws = SplitWorkspace(1, 50, 8, 1, 256, 3, gpu)
    out = torch.empty_like(qd)
    q8 = torch.empty(50, 8 * 256, device=gpu, dtype=torch.float8_e4m3fn)
    qs = torch.empty(50, device=gpu)
    kw = dict(out=out, kv_len=n, split=ws, q8=q8, q8_scale=qs)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        attention(qd, kd, vd, **kw)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        attention(qd, kd, vd, **kw)
    for length in (300, 1, 177, 100):
        n.fill_(length)
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _close(out, _ref(oracle_mod, q, k, v, np.full(50, length)), torch.bfloat16, f"replay len {length}")
        eager_q8, eager_qs = torch.empty_like(q8), torch.empty_like(qs)
        attention(qd, kd, vd, kv_len=n, split=ws, q8=eager_q8, q8_scale=eager_qs)
        torch.cuda.synchronize()
        assert torch.equal(eager_q8.view(torch.uint8), q8.view(torch.uint8)) and torch.equal(eager_qs, qs)


def test_contract_errors(gpu):
    from instinctflash_amd import _lib
    from instinctflash_amd.kernels import SplitWorkspace, attention
    q = torch.zeros(1, 4, 2, 64, device=gpu, dtype=torch.bfloat16)
    k = torch.zeros(1, 8, 1, 64, device=gpu, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="dtype"):
        attention(q, k.half(), k)
    with pytest.raises(ValueError, match="multiple"):
        attention(torch.zeros(1, 4, 3, 64, device=gpu, dtype=torch.bfloat16), torch.zeros(1, 8, 2, 64, device=gpu,
                  dtype=torch.bfloat16), torch.zeros(1, 8, 2, 64, device=gpu, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="split"):
        attention(q, k, k, q8=torch.empty(4, 128, device=gpu, dtype=torch.float8_e4m3fn),
                  q8_scale=torch.empty(4, device=gpu))
    with pytest.raises(ValueError, match="geometry"):
        attention(q, k, k, split=SplitWorkspace(1, 5, 2, 1, 64, 2, gpu))
    with pytest.raises(_lib.IfxError):
        attention(torch.zeros(1, 4, 2, 36, device=gpu, dtype=torch.bfloat16),
                  torch.zeros(1, 8, 1, 36, device=gpu, dtype=torch.bfloat16),
                  torch.zeros(1, 8, 1, 36, device=gpu, dtype=torch.bfloat16))  # D % 8
    with pytest.raises(_lib.IfxError):
        attention(torch.zeros(1, 4, 1, 320, device=gpu, dtype=torch.bfloat16),
                  torch.zeros(1, 8, 1, 320, device=gpu, dtype=torch.bfloat16),
                  torch.zeros(1, 8, 1, 320, device=gpu, dtype=torch.bfloat16))  # D > 256


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_many_splits_long_keys(gpu, oracle_mod, dtype):
    # 16 key splits over ~4000 keys: the partial rows are kept in the operands'
    # 16-bit type (normalized by their own softmax sum); the merged output stays
    # within the same bars as the unsplit kernel
    from instinctflash_amd.kernels import SplitWorkspace, attention
    q, k, v = _qkv(1, 33, 4000, 8, 1, 256, 21, dtype)
    n = torch.tensor([3900], device=gpu, dtype=torch.int32)
    ws = SplitWorkspace(1, 33, 8, 1, 256, 16, gpu)
    out = attention(q.to(gpu), k.to(gpu), v.to(gpu), kv_len=n, split=ws)
    _close(out, _ref(oracle_mod, q, k, v, np.full(33, 3900)), dtype, f"16 splits {dtype}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_split_partials_q8_agreement(gpu, oracle_mod, dtype):
    # The split partial rows are stored normalized in the operands' 16-bit type
    # (the reference keeps fp32 partials, kernels/attention.py:155). What that costs
    # the fused e4m3 row, at the pi05 chunk's shape (51 queries over 851 keys, 8/1
    # heads of 256, 14 splits), against the oracle recipe applied to the exact
    # float64 attention rows -- measured: fp16 1.27% of the codes differ, scale drift
    # 3.1e-4; bf16 7.2% and 2.3e-3; codes more than one step apart (or of opposite
    # sign) only where a value is below 2.2e-3 / 1.6e-2 of its row max; the
    # dequantized rows stay within 3.7% of the row max. Bounds: the reference
    # test's 7% row bar (tests/test_gi_kernels.py:112), differing codes <= 2% / 10%,
    # scale drift <= 2^-11 / 2^-8 (fp16 / bf16), far codes only below 1/32 of the
    # row max
    from instinctflash_amd.kernels import SplitWorkspace, attention
    T, hq, hd = 51, 8, 256
    q, k, v = _qkv(1, T, 851, hq, 1, hd, 77, dtype)
    n = torch.tensor([851], device=gpu, dtype=torch.int32)
    ws = SplitWorkspace(1, T, hq, 1, hd, 14, gpu)
    q8 = torch.empty(T, hq * hd, device=gpu, dtype=torch.float8_e4m3fn)
    qs = torch.empty(T, device=gpu)
    attention(q.to(gpu), k.to(gpu), v.to(gpu), kv_len=n, split=ws, q8=q8, q8_scale=qs)
    r = _ref(oracle_mod, q, k, v, np.full(T, 851)).reshape(T, -1).astype(np.float32)
    eq, es = oracle_mod.quant_rows(r)
    got = q8.view(torch.uint8).cpu().numpy()
    differ = (got != eq).mean()
    drift = np.abs(qs.cpu().numpy() / es - 1).max()
    deq = oracle_mod.e4m3_decode(got) * qs.cpu().numpy()[:, None]
    rowmax = np.abs(r).max(axis=1, keepdims=True)
    rel = (np.abs(deq - r) / rowmax).max()
    # codes more than one step apart: values small against their row max
    far = (np.abs(got.astype(np.int16) - eq.astype(np.int16)) > 1) | ((got & 0x80) != (eq & 0x80))
    small = (np.abs(r) / rowmax)[far].max() if far.any() else 0.0
    print(f"[attn q8 {dtype}] differing codes {differ:.4%}, scale drift {drift:.2e}, err / row max {rel:.3e}, "
          f"largest |value| / row max among far codes {small:.3e}", flush=True)
    bound = {torch.float16: (0.02, 2.0 ** -11), torch.bfloat16: (0.10, 2.0 ** -8)}[dtype]
    assert rel < 0.07 and differ <= bound[0] and drift <= bound[1] and small < 1 / 32, (rel, differ, drift, small)

"""GPU parity of ``linear_qkv_rope`` (the qkv_split work in the skinny FP8 GEMM's
epilogue; replaces gemm + qkv_split, reference instinctflash/kernels/fp8.py:50-53
and kernels/rope.py:89-116).

The fused call must equal, bit for bit, the unfused pair run on the same fp32
values: ``linear`` with an fp32 output on the unpermuted weight (identical K
accumulation per output column, identical epilogue formula), then ``qkv_split``
on that fp32 accumulator with no further scales. qkv_split itself is pinned
against the CPU oracle in test_gpu_rope.py. Cache rows outside
kv_base .. kv_base + T stay untouched; a captured graph follows a device kv_base.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(gpu, M, HQ, HKV, HD, K, bias, seed):
    from instinctflash_amd.kernels import quant_rows, quantize_weight
    g = torch.Generator().manual_seed(seed)
    N = (HQ + 2 * HKV) * HD
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.02
    b = torch.randn(N, generator=g) * 0.1 if bias else None
    fw = quantize_weight(w.to(gpu), None if b is None else b.to(gpu))
    qa, sa = quant_rows(x.to(gpu))
    pos = (torch.arange(M, dtype=torch.float32) * 3 + 11).reshape(M, 1).to(gpu)
    return qa, sa, fw, pos, x.to(gpu)


def _unfused(qa, sa, fw, HQ, HKV, HD, pos, inv_freq, kv_base, rows, dtype, gpu):
    from instinctflash_amd.kernels import linear, qkv_split
    M = qa.shape[0]
    y = linear(qa, sa, fw, out_dtype=torch.float32)
    q = torch.full((M, HQ, HD), 7.0, dtype=dtype, device=gpu)
    k = torch.full((rows, HKV, HD), 7.0, dtype=dtype, device=gpu)
    v = torch.full((rows, HKV, HD), 7.0, dtype=dtype, device=gpu)
    qkv_split(y, q, k, v, heads_q=HQ, heads_kv=HKV, head_dim=HD, inv_freq=inv_freq, pos=pos, kv_base=kv_base)
    return q, k, v


@pytest.mark.parametrize("M,HQ,HKV,HD,K,bias,dtype,tiled", [
    (50, 8, 1, 256, 1024, False, torch.float16, True),    # pi05 action expert
    (50, 8, 1, 256, 1024, False, torch.float16, False),
    (16, 4, 2, 128, 512, True, torch.bfloat16, True),
    (33, 2, 1, 64, 256, True, torch.float32, False),
    (64, 16, 4, 128, 2048, False, torch.bfloat16, True),
])
def test_matches_gemm_plus_qkv_split(gpu, M, HQ, HKV, HD, K, bias, dtype, tiled):
    from instinctflash_amd.kernels import linear_qkv_rope, pack_skinny, permute_rope_rows, rope_inv_freq
    qa, sa, fw, pos, x = _case(gpu, M, HQ, HKV, HD, K, bias, M + HD)
    inv_freq = rope_inv_freq(HD, 10000.0, gpu)
    base, rows = 5, M + 9
    q0, k0, v0 = _unfused(qa, sa, fw, HQ, HKV, HD, pos, inv_freq, base, rows, dtype, gpu)
    pw = permute_rope_rows(fw, HQ, HKV, HD)
    if tiled:
        pw = pack_skinny(pw)
    q = torch.full_like(q0, 7.0)
    k = torch.full_like(k0, 7.0)
    v = torch.full_like(v0, 7.0)
    linear_qkv_rope(qa, sa, pw, q, k, v, inv_freq=inv_freq, pos=pos, kv_base=base)
    torch.cuda.synchronize()
    assert torch.equal(q, q0) and torch.equal(k, k0) and torch.equal(v, v0)
    assert (k[:base] == 7.0).all() and (k[base + M:] == 7.0).all() and (v[:base] == 7.0).all()


def test_no_rotation_and_tiled_activations(gpu):
    from instinctflash_amd.kernels import (linear_qkv_rope, pack_skinny, permute_rope_rows, quant_rows_tiled)
    M, HQ, HKV, HD, K = 20, 4, 1, 128, 768
    qa, sa, fw, pos, x = _case(gpu, M, HQ, HKV, HD, K, True, 3)
    q0, k0, v0 = _unfused(qa, sa, fw, HQ, HKV, HD, None, None, 0, M, torch.bfloat16, gpu)
    x_t, s_t = quant_rows_tiled(x)  # the same bytes and scales as quant_rows, tile layout
    assert torch.equal(s_t, sa)
    pw = pack_skinny(permute_rope_rows(fw, HQ, HKV, HD))
    q, k, v = torch.empty_like(q0), torch.empty_like(k0), torch.empty_like(v0)
    linear_qkv_rope(x_t, s_t, pw, q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(q, q0) and torch.equal(k, k0) and torch.equal(v, v0)


def test_graph_follows_device_kv_base(gpu):
    from instinctflash_amd.kernels import linear_qkv_rope, pack_skinny, permute_rope_rows, rope_inv_freq
    M, HQ, HKV, HD, K = 50, 8, 1, 256, 1024
    qa, sa, fw, pos, x = _case(gpu, M, HQ, HKV, HD, K, False, 8)
    inv_freq = rope_inv_freq(HD, 10000.0, gpu)
    pw = pack_skinny(permute_rope_rows(fw, HQ, HKV, HD))
    base = torch.tensor([0], dtype=torch.int32, device=gpu)
    rows = M + 200
    q = torch.empty(M, HQ, HD, dtype=torch.float16, device=gpu)
    k = torch.zeros(rows, HKV, HD, dtype=torch.float16, device=gpu)
    v = torch.zeros_like(k)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        linear_qkv_rope(qa, sa, pw, q, k, v, inv_freq=inv_freq, pos=pos, kv_base=base)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        linear_qkv_rope(qa, sa, pw, q, k, v, inv_freq=inv_freq, pos=pos, kv_base=base)
    for b in (123, 7, 200):
        base.fill_(b)
        k.zero_()
        v.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        q0, k0, v0 = _unfused(qa, sa, fw, HQ, HKV, HD, pos, inv_freq, b, rows, torch.float16, gpu)
        assert torch.equal(q, q0)
        assert torch.equal(k[b:b + M], k0[b:b + M]) and torch.equal(v[b:b + M], v0[b:b + M])
        assert not k[:b].any() and not k[b + M:].any()


def test_contract_errors(gpu):
    from instinctflash_amd.kernels import linear, linear_qkv_rope, permute_rope_rows
    qa, sa, fw, pos, x = _case(gpu, 8, 2, 1, 64, 256, False, 1)
    q = torch.empty(8, 2, 64, dtype=torch.float16, device=gpu)
    k = torch.empty(8, 1, 64, dtype=torch.float16, device=gpu)
    with pytest.raises(ValueError, match="permute_rope_rows"):
        linear_qkv_rope(qa, sa, fw, q, k, k.clone())
    pw = permute_rope_rows(fw, 2, 1, 64)
    with pytest.raises(ValueError, match="linear_qkv_rope"):
        linear(qa, sa, pw)
    with pytest.raises(ValueError, match="share a dtype"):
        linear_qkv_rope(qa, sa, pw, q, k, k.float())
    with pytest.raises(ValueError):
        permute_rope_rows(fw, 2, 2, 64)  # N mismatch

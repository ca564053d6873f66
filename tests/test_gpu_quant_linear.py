"""GPU parity of the quantize-and-project entry point (ifx_quant_linear).

Its contract is bit-identity with the two-call sequence it packages: per-token
(``quant_rows``) or per-tensor (``quantize_tensor``) E4M3 quantization of the
bf16 activations, then ``linear`` on the result, with the E4M3 copy in the
caller's workspace. Both halves are pinned to the oracle elsewhere (byte-exact
quantizers, GEMM within the north-star tolerance); here every output bit and
every scale bit must match them. Shapes cover both GEMM families, ragged K,
strided rows, GLU, residual and gate epilogues, and rows holding NaN, +-inf,
zeros and subnormals.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _same(a, b, what):
    """Bit equality, except that NaN only has to meet NaN."""
    a, b = a.detach().cpu(), b.detach().cpu()
    assert a.shape == b.shape and a.dtype == b.dtype, what
    nan = torch.isnan(a.float()) & torch.isnan(b.float())
    ia = a.view(torch.int16 if a.dtype == torch.bfloat16 else torch.int32)
    ib = b.view(torch.int16 if b.dtype == torch.bfloat16 else torch.int32)
    bad = (ia != ib) & ~nan
    assert not bad.any(), f"{what}: {int(bad.sum())} differing elements, first at {bad.nonzero()[0].tolist()}"


def _weights(gpu, N, K, seed, bias=True, glu=False, per_tensor_w=False):
    from instinctflash_amd.kernels import Fp8Weight, pack_glu, quantize_tensor, quantize_weight
    g = torch.Generator().manual_seed(seed)
    w = torch.randn((N, K), generator=g) * 0.02
    b = torch.randn(N, generator=g) * 0.01 if bias else None
    if per_tensor_w:
        qw, sw = quantize_tensor(w.to(torch.bfloat16).to(gpu))
        fw = Fp8Weight(qw, sw, None if b is None else b.to(gpu))
    else:
        fw = quantize_weight(w, b, device=gpu)
    return (pack_glu(fw) if glu else fw), g


def _both(gpu, x, fw, per_tensor=False, **kw):
    """(fused, reference sequence) outputs and scales, bf16 and fp32 outputs."""
    from instinctflash_amd.kernels import linear, quant_linear, quant_rows, quantize_tensor
    M = x.shape[0]
    n = 1 if per_tensor else M
    res = []
    for dt in (torch.bfloat16, torch.float32):
        s_fused = torch.full((n,), -1.0, device=gpu)
        o_fused = quant_linear(x, fw, per_tensor=per_tensor, a_scale=s_fused, out_dtype=dt, **kw)
        if per_tensor:
            qa, sa = quantize_tensor(x.contiguous())
        else:
            qa, sa = quant_rows(x)
        o_ref = linear(qa, sa, fw, out_dtype=dt, **kw)
        res.append((o_fused, o_ref, s_fused, sa))
    return res


def _check(gpu, x, fw, what, per_tensor=False, **kw):
    for o_f, o_r, s_f, s_r in _both(gpu, x, fw, per_tensor=per_tensor, **kw):
        _same(s_f, s_r.reshape(-1), f"{what}: scales")
        _same(o_f, o_r, f"{what}: {o_f.dtype} output")


CASES = [
    # M, N, K: skinny GEMM (M <= 64), ragged K
    (1, 16, 128), (16, 6144, 1536), (16, 1536, 6144), (16, 512, 16384), (5, 256, 176),
    (33, 48, 176), (50, 4096, 1024), (64, 256, 2048), (17, 1040, 1040),
    # M > 64: LDS-tiled GEMM families
    (65, 256, 1024), (200, 512, 1024), (816, 2048, 2048),
]


@pytest.mark.parametrize("M,N,K", CASES)
@pytest.mark.parametrize("per_tensor", [False, True])
def test_matches_quantize_then_linear(gpu, M, N, K, per_tensor):
    fw, g = _weights(gpu, N, K, seed=M * 31 + N + K)
    x = (torch.randn((M, K), generator=g) * torch.rand((M, 1), generator=g) * 4).to(torch.bfloat16).to(gpu)
    _check(gpu, x, fw, f"{M}x{N}x{K} {'tensor' if per_tensor else 'token'}", per_tensor=per_tensor)


@pytest.mark.parametrize("M,act", [(16, "gelu_tanh"), (16, "geglu"), (50, "swiglu"), (200, "geglu")])
def test_epilogues(gpu, M, act):
    glu = act in ("geglu", "swiglu")
    N, K = 2048, 1536
    fw, g = _weights(gpu, N, K, seed=M, glu=glu)
    n_out = N // 2 if glu else N
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).to(gpu)
    res = torch.randn((M, n_out), generator=g).to(torch.bfloat16).to(gpu)
    gate = torch.randn(n_out, generator=g).to(torch.bfloat16).to(gpu)
    _check(gpu, x, fw, f"{act} M={M}", act=act, residual=res, gate=gate)


def test_per_tensor_weight_scale(gpu):
    fw, g = _weights(gpu, 1024, 1024, seed=5, per_tensor_w=True)
    x = torch.randn((21, 1024), generator=g).to(torch.bfloat16).to(gpu)
    _check(gpu, x, fw, "per-tensor activations and weights", per_tensor=True)


def test_strided_rows(gpu):
    fw, g = _weights(gpu, 512, 1024, seed=7)
    big = torch.randn((40, 1104), generator=g).to(torch.bfloat16).to(gpu)
    x = big[:, 8:8 + 1024]  # row stride 1104 elements, 16-byte aligned start
    assert x.stride(0) == 1104 and x.data_ptr() % 16 == 0
    _check(gpu, x, fw, "strided x")


@pytest.mark.parametrize("M,K", [(16, 1536), (40, 6144)])
def test_special_values(gpu, M, K):
    fw, g = _weights(gpu, 256, K, seed=M + K)
    x = torch.randn((M, K), generator=g)
    x[1] = 0.0                                    # all-zero row: scale floor 1e-12 * fl32(1/448)
    x[2, 5] = float("nan")                        # NaN row: NaN scale, NaN outputs
    x[3, 7] = float("inf")                        # inf row: inf scale
    x[4, :] = torch.randn(K, generator=g) * 1e-38  # subnormal-sized values
    x[5, 0] = 3.0e38                              # huge amax
    x[6, :] = -x[6, :].abs()
    x = x.to(torch.bfloat16).to(gpu)
    _check(gpu, x, fw, f"special values M={M}")
    _check(gpu, x[7:], fw, f"special values tensor M={M}", per_tensor=True)  # finite rows only
    _check(gpu, x, fw, f"special values tensor with NaN M={M}", per_tensor=True)


def test_scale_matches_oracle(gpu, oracle_mod):
    # the scales the fused kernel reports are the oracle's, bit for bit
    from instinctflash_amd.kernels import quant_linear
    fw, g = _weights(gpu, 256, 6144, seed=11)
    x = (torch.randn((16, 6144), generator=g) * 3).to(torch.bfloat16)
    s = torch.empty(16, device=gpu)
    quant_linear(x.to(gpu), fw, a_scale=s)
    _, ref_s = oracle_mod.quant_rows(x.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(s.cpu().numpy().view(np.uint32), ref_s.view(np.uint32))


def test_graph_replay(gpu):
    from instinctflash_amd.kernels import quant_linear
    fw, g = _weights(gpu, 1536, 6144, seed=3)
    x = torch.randn((16, 6144), generator=g).to(torch.bfloat16).to(gpu)
    res = torch.randn((16, 1536), generator=g).to(torch.bfloat16).to(gpu)
    eager = quant_linear(x, fw, residual=res)
    out = torch.empty_like(eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        quant_linear(x, fw, out=out, residual=res)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        quant_linear(x, fw, out=out, residual=res)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _same(out, eager, "graph replay")


def test_contract_errors(gpu):
    from instinctflash_amd import _lib
    from instinctflash_amd.kernels import quant_linear
    fw, g = _weights(gpu, 256, 512, seed=1)
    with pytest.raises(ValueError, match="bfloat16"):
        quant_linear(torch.zeros((4, 512), device=gpu), fw)
    with pytest.raises(ValueError):
        quant_linear(torch.zeros((4, 256), dtype=torch.bfloat16, device=gpu), fw)
    lib = _lib.load()
    x = torch.zeros((4, 512), dtype=torch.bfloat16, device=gpu)
    out = torch.empty((4, 256), dtype=torch.bfloat16, device=gpu)
    P = lambda t: t.data_ptr()  # noqa: E731
    # unknown scale mode; a caller-supplied scalar activation scale
    assert lib.ifx_quant_linear(P(x), 512, 2, P(fw.w), 512, P(fw.scale), None, None, 0, None, 0, P(out), 256,
                                4, 256, 512, None, None, 0, None) == _lib.ERR_INVALID
    assert lib.ifx_quant_linear(P(x), 512, 0, P(fw.w), 512, P(fw.scale), None, None, 0, None, _lib.EPI_SCALAR_SA,
                                P(out), 256, 4, 256, 512, None, None, 0, None) == _lib.ERR_INVALID
    # misaligned rows; no workspace
    assert lib.ifx_quant_linear(P(x), 500, 0, P(fw.w), 512, P(fw.scale), None, None, 0, None, 0, P(out), 256,
                                1, 256, 496, None, None, 0, None) == _lib.ERR_ALIGN
    assert lib.ifx_quant_linear(P(x), 512, 0, P(fw.w), 512, P(fw.scale), None, None, 0, None, 0, P(out), 256,
                                4, 256, 512, None, None, 0, None) == _lib.ERR_WORKSPACE
    xb = torch.zeros((100, 512), dtype=torch.bfloat16, device=gpu)
    ob = torch.empty((100, 256), dtype=torch.bfloat16, device=gpu)
    assert lib.ifx_quant_linear_workspace_size(100, 256, 512, 0, 0) > 0
    assert lib.ifx_quant_linear(P(xb), 512, 0, P(fw.w), 512, P(fw.scale), None, None, 0, None, 0, P(ob), 256,
                                100, 256, 512, None, None, 0, None) == _lib.ERR_WORKSPACE
    torch.cuda.synchronize()

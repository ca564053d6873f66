"""ifx_quant_linear_noalloc (no workspace argument, library-owned scratch)
against ifx_quant_linear (caller workspace), through the C ABI: bit-identical
outputs and scales on two calls in a row, the second with a smaller input,
for the large-M path (split K with its partials in the scratch), the skinny
path (long K, GLU), and per-tensor scaling; a call that needs more than the
scratch is rejected before anything is launched. The caller workspace is
filled with a nonzero pattern first: no part of it needs initialising."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _weights(gpu, N, K, seed, glu=False):
    from instinctflash_amd.kernels import pack_glu, quantize_weight
    g = torch.Generator().manual_seed(seed)
    w = torch.randn((N, K), generator=g) * 0.02
    b = torch.randn(N, generator=g) * 0.01
    fw = quantize_weight(w, b, device=gpu)
    return pack_glu(fw) if glu else fw, g


def _call(lib, fn, x, fw, out, flags, mode, res, a_scale, ws=None):
    M, K = x.shape
    N = fw.w.shape[0]
    args = [x.data_ptr(), K, mode, fw.w.data_ptr(), K, fw.scale.data_ptr(), fw.bias.data_ptr(),
            None if res is None else res.data_ptr(), 0 if res is None else res.stride(0), None, flags,
            out.data_ptr(), out.stride(0), M, N, K, a_scale.data_ptr()]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    args.append(torch.cuda.current_stream().cuda_stream)
    return getattr(lib, fn)(*args)


@pytest.mark.parametrize("case", [
    # (M1, M2, N, K, flags, scale mode)
    ("large split-K +res", 1024, 300, 2048, 11008, "res", "row"),
    ("large GELU", 512, 129, 4096, 2048, "gelu", "row"),
    ("skinny long K", 16, 8, 1024, 16384, None, "row"),
    ("skinny GeGLU", 50, 16, 4096, 1024, "geglu", "row"),
    ("per tensor", 256, 64, 1536, 1536, None, "tensor"),
])
def test_noalloc_matches_workspace_call(gpu, case):
    from instinctflash_amd import _lib
    lib = _lib.load()
    name, M1, M2, N, K, ep, mode = case
    glu = ep == "geglu"
    fw, g = _weights(gpu, N, K, seed=M1 + N, glu=glu)
    flags = _lib.EPI_BIAS | {None: 0, "res": _lib.EPI_RESIDUAL, "gelu": _lib.EPI_GELU_TANH,
                             "geglu": _lib.EPI_GEGLU}[ep]
    smode = _lib.SCALE_TENSOR if mode == "tensor" else _lib.SCALE_ROW
    n_out = N // 2 if glu else N
    print(f"[noalloc] {name}", flush=True)
    for M in (M1, M2):  # two calls in a row, the second smaller
        x = (torch.randn((M, K), generator=g) * 2).to(torch.bfloat16).to(gpu)
        res = torch.randn((M, n_out), generator=g).to(torch.bfloat16).to(gpu) if ep == "res" else None
        ns = 1 if mode == "tensor" else M
        nbytes = lib.ifx_quant_linear_workspace_size(M, N, K, flags, smode)
        assert 0 < nbytes <= lib.ifx_quant_linear_noalloc_max_bytes()
        ws = torch.full((nbytes,), 0xA5, dtype=torch.uint8, device=gpu)
        o_ref = torch.full((M, n_out), float("nan"), dtype=torch.bfloat16, device=gpu)
        o_na = torch.full_like(o_ref, -1.0)
        s_ref = torch.empty(ns, device=gpu)
        s_na = torch.empty(ns, device=gpu)
        _lib.check(_call(lib, "ifx_quant_linear", x, fw, o_ref, flags, smode, res, s_ref, ws), "ifx_quant_linear")
        _lib.check(_call(lib, "ifx_quant_linear_noalloc", x, fw, o_na, flags, smode, res, s_na),
                   "ifx_quant_linear_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(o_na.view(torch.int16), o_ref.view(torch.int16)), f"{name} M={M}: output differs"
        assert torch.equal(s_na.view(torch.int32), s_ref.view(torch.int32)), f"{name} M={M}: scales differ"
        assert torch.isfinite(o_ref.float()).all()


def test_noalloc_rejects_oversize(gpu):
    from instinctflash_amd import _lib
    lib = _lib.load()
    M, N, K = 8192, 3072, 14336  # ~117 MB of e4m3 activations: beyond the scratch
    assert lib.ifx_quant_linear_workspace_size(M, N, K, 0, _lib.SCALE_ROW) > lib.ifx_quant_linear_noalloc_max_bytes()
    p = ctypes.c_void_p(16)  # never dereferenced: the size check comes first
    rc = lib.ifx_quant_linear_noalloc(p, K, _lib.SCALE_ROW, p, K, p, None, None, 0, None, 0, p, N, M, N, K, None,
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.ERR_SCRATCH

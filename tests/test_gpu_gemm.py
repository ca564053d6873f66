"""GPU parity of the FP8 GEMM + fused epilogue against the dequantize-then-fp32-matmul
oracle (benchmarks/native/fp8_probe.py:36 in the reference).

Acceptance bar of the FP8 path: max|d| <= 2e-2 * rms(ref) and cosine >= 0.9999,
for every epilogue and every kernel family (skinny M <= 64, LDS-staged large-M for
K % 128 == 0, register-staged LDS tiles for other K),
including ragged M/N/K tails, strided operands, in-place residual and determinism.

The tolerance gates the kernel's arithmetic through its fp32-output mode (same
kernel, same code path; only the final store differs). The bf16 output is then
required to be bit-identical to round-to-nearest-even of that fp32 output. The
split matters for heavy-tailed outputs (GeGLU/SwiGLU, max/rms ~ 25): there bf16
rounding alone moves the largest values by up to 2^-8 * 25 rms = 0.1 rms,
which no bf16 result could keep under 2e-2 rms.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL_MAXD = 2e-2   # max|d| / rms(ref)
TOL_COS = 0.9999


def _q(t):
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def _f(t):
    return t.detach().float().cpu().numpy()


def _make(gpu, M, N, K, seed, wscale=0.02, bias=False):
    from instinctflash_amd.kernels import quant_rows, quantize_weight
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    w = torch.randn((N, K), generator=g) * wscale
    b = torch.randn(N, generator=g) * 0.01 if bias else None
    fw = quantize_weight(w, b, device=gpu)
    qa, sa = quant_rows(x.to(gpu))
    return qa, sa, fw, g


def _assert_close(out, ref, what=""):
    from oracle import parity_stats
    d, cos = parity_stats(out, ref)
    assert np.isfinite(out).all(), f"{what}: non-finite output"
    assert d <= TOL_MAXD and cos >= TOL_COS, f"{what}: max|d|/rms={d:.3e} cos={cos:.6f}"


def _ref(oracle_mod, qa, sa, fw, **kw):
    return oracle_mod.ref_linear(_q(qa), _f(sa), _q(fw.w), _f(fw.scale),
                                 bias=None if fw.bias is None else _f(fw.bias), **kw)


def _check(gpu, oracle_mod, qa, sa, fw, what, ref_w=None, act=None, residual=None, gate=None):
    """fp32-output arithmetic within tolerance + bf16 / fp16 outputs == RNE(fp32 output)."""
    from instinctflash_amd.kernels import linear
    r = None if residual is None else residual.to(gpu)
    gt = None if gate is None else gate.to(gpu)
    o32 = linear(qa, sa, fw, act=act, residual=r, gate=gt, out_dtype=torch.float32)
    o16 = linear(qa, sa, fw, act=act, residual=r, gate=gt, out_dtype=torch.bfloat16)
    ref = _ref(oracle_mod, qa, sa, ref_w or fw, act=act,
               residual=None if residual is None else residual.float().numpy(),
               gate=None if gate is None else gate.float().numpy())
    _assert_close(_f(o32), ref, what)
    assert torch.equal(o16.view(torch.int16), o32.to(torch.bfloat16).view(torch.int16)), f"{what}: bf16 store"
    # the fp16 output mode (IFX_EPI_OUT_F16): the same fp32 values, RNE to fp16
    oh = linear(qa, sa, fw, act=act, residual=r, gate=gt, out_dtype=torch.float16)
    assert torch.equal(oh.view(torch.int16), o32.to(torch.float16).view(torch.int16)), f"{what}: fp16 store"
    return o32, o16


SHAPES = [
    (1, 16, 128), (16, 6144, 1536), (16, 1536, 6144), (50, 4096, 1024), (64, 256, 2048),
    (33, 48, 176), (65, 256, 1024), (130, 272, 384), (256, 512, 1024), (300, 1040, 1040),
    (816, 2048, 256), (1024, 2560, 2048),
]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_linear_plain(gpu, oracle_mod, M, N, K):
    qa, sa, fw, _ = _make(gpu, M, N, K, seed=M * 7 + N + K)
    _check(gpu, oracle_mod, qa, sa, fw, f"{M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(50, 4096, 1024), (16, 512, 256), (200, 2560, 2048)])
def test_raw_gemm_unit_scales(gpu, oracle_mod, M, N, K):
    # reference kernels/fp8.py:50-53: raw accumulator in bf16, unit scales.
    from instinctflash_amd.kernels import gemm
    qa, sa, fw, _ = _make(gpu, M, N, K, seed=3)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
    gemm(qa, fw, out)
    ref = oracle_mod.ref_linear(_q(qa), None, _q(fw.w), None)
    _assert_close(_f(out), ref, "raw")
    # Error budget against the exact sum: bf16 rounding of the result (2^-8
    # relative) plus the matrix core's accumulation error. One FP8 MFMA adds its
    # 128 products with an error of at most ~2^-16 of their absolute sum
    # (measured on gfx950; fp32 adds would give 2^-24), so allow 2^-14.
    A = oracle_mod.e4m3_decode(_q(qa)).astype(np.float64)
    W = oracle_mod.e4m3_decode(_q(fw.w)).astype(np.float64)
    exact, absum = A @ W.T, np.abs(A) @ np.abs(W).T
    assert np.all(np.abs(_f(out) - exact) <= 2.0 ** -8 * np.abs(exact) + 2.0 ** -14 * absum)


@pytest.mark.parametrize("M", [16, 50, 300])
def test_bias_gelu(gpu, oracle_mod, M):
    qa, sa, fw, _ = _make(gpu, M, 6144, 1536, seed=M, bias=True)
    _check(gpu, oracle_mod, qa, sa, fw, "gelu", act="gelu_tanh")


@pytest.mark.parametrize("M,act", [(16, "geglu"), (50, "swiglu"), (816, "geglu"), (200, "swiglu")])
def test_glu(gpu, oracle_mod, M, act):
    from instinctflash_amd.kernels import pack_glu
    F, K = 1024, 2048
    qa, sa, fw, _ = _make(gpu, M, 2 * F, K, seed=M + 1, bias=True)
    packed = pack_glu(fw)
    o32, _ = _check(gpu, oracle_mod, qa, sa, packed, act, ref_w=fw, act=act)
    assert o32.shape == (M, F)


@pytest.mark.parametrize("M,res_dtype", [(16, torch.bfloat16), (64, torch.float32), (816, torch.bfloat16),
                                         (200, torch.float32)])
def test_residual_and_gate(gpu, oracle_mod, M, res_dtype):
    from instinctflash_amd.kernels import linear
    N, K = 1536, 6144 if M <= 64 else 2048
    qa, sa, fw, g = _make(gpu, M, N, K, seed=M + 2, bias=True)
    res = torch.randn((M, N), generator=g).to(res_dtype)
    gate = torch.rand(N, generator=g).to(torch.bfloat16)
    # plain residual, separate output
    _check(gpu, oracle_mod, qa, sa, fw, "res", residual=res)
    o32, o16 = _check(gpu, oracle_mod, qa, sa, fw, "gated", residual=res, gate=gate)
    # in place (out aliases residual): same bytes as the out-of-place result
    r = res.to(gpu)
    linear(qa, sa, fw, out=r, residual=r, gate=gate.to(gpu))
    expect = o32 if res_dtype == torch.float32 else o16
    assert torch.equal(r, expect), "in-place residual update differs"


@pytest.mark.parametrize("act,res,gate", [("gelu_tanh", True, False), ("gelu_tanh", True, True), (None, False, True),
                                          ("geglu", True, False), ("swiglu", True, True)])
def test_large_m_epilogue_combinations(gpu, oracle_mod, act, res, gate):
    # large-M kernel: flag sets outside its compile-time modes (activation with a
    # residual, gate without residual, GLU with residual) against the oracle, and
    # the bf16 store equal to the rounded fp32 result of the same call
    from instinctflash_amd.kernels import pack_glu
    M, N, K = 2000, 6144, 512  # >= 192 tiles of 256 x 256: no K split, ragged last token tile
    qa, sa, fw, g = _make(gpu, M, N, K, seed=31, bias=True)
    n_out = N // 2 if act in ("geglu", "swiglu") else N
    r = torch.randn((M, n_out), generator=g).to(torch.bfloat16) if res else None
    gt = torch.rand(n_out, generator=g).to(torch.bfloat16) if gate else None
    w = pack_glu(fw) if act in ("geglu", "swiglu") else fw
    _check(gpu, oracle_mod, qa, sa, w, f"{act} res={res} gate={gate}", ref_w=fw, act=act, residual=r, gate=gt)


@pytest.mark.parametrize("M,N,K,act", [(4112, 12304, 128, None), (4112, 12304, 256, "gelu_tanh"),
                                       (4112, 12304, 384, None), (3000, 16416, 640, "geglu"),
                                       (2100, 24608, 128, "swiglu"), (8192, 6144, 1024, "gelu_tanh"),
                                       (8100, 3056, 128, None), (7900, 3040, 256, "gelu_tanh"),
                                       (5000, 3840, 384, None), (8192, 3072, 640, None),
                                       (1000, 22016, 256, "swiglu"), (777, 21952, 128, "geglu")])
def test_wide_tile_k_loop_edges(gpu, oracle_mod, M, N, K, act):
    # >= 192 tiles of 256 x 256 (or of 256 x 192 for the last six shapes, the
    # last two GLU with 4-row epilogue passes of 12-lane groups): the
    # 4-wave register-pipelined kernel, whose K
    # loop has a prologue of two stages, a main part that issues the stage two
    # ahead and a tail of up to two stages without DMA; K of 1..5 stages and
    # 8 stages exercises every split of the three, ragged M and N clamp the
    # DMA rows of the last tiles, GLU weights included. The ragged last token
    # tiles also run the K-loop forms that skip token fragments past M: half
    # of a wave's fragments (4112, 3000, 2100, 8100, 5000, 777) or none (the
    # second token wave of 4112, 2100, 777)
    from instinctflash_amd.kernels import pack_glu
    qa, sa, fw, g = _make(gpu, M, N, K, seed=M + N + K, bias=True)
    glu = act in ("geglu", "swiglu")
    res = torch.randn((M, N // 2 if glu else N), generator=g).to(torch.bfloat16)
    _check(gpu, oracle_mod, qa, sa, pack_glu(fw) if glu else fw, f"wide {M}x{N}x{K}", ref_w=fw, act=act,
           residual=res)


@pytest.mark.parametrize("K", [1024, 8192])
@pytest.mark.parametrize("act,resgate", [("gelu_tanh", False), (None, True), ("swiglu", False)])
def test_ragged_small_grid_configs(gpu, oracle_mod, K, act, resgate):
    # outputs of fewer than 192 256x256 tiles: 128x64 tiles for K <= 4096, split-K
    # 256x128 tiles above; M and N end inside a tile
    from instinctflash_amd.kernels import pack_glu
    M, N = 333, 1056
    qa, sa, fw, g = _make(gpu, M, N, K, seed=K + M, bias=True)
    glu = act == "swiglu"
    n_out = N // 2 if glu else N
    r = torch.randn((M, n_out), generator=g).to(torch.bfloat16) if resgate else None
    gt = torch.rand(n_out, generator=g).to(torch.bfloat16) if resgate else None
    _check(gpu, oracle_mod, qa, sa, pack_glu(fw) if glu else fw, f"ragged {act} K={K}", ref_w=fw, act=act,
           residual=r, gate=gt)


@pytest.mark.parametrize("M,N,K,act", [(65, 256, 1040, None), (100, 768, 528, "gelu_tanh"), (300, 512, 1552, "geglu"),
                                       (1000, 2112, 1040, None), (2048, 8192, 272, "swiglu"),
                                       (2048, 4096, 272, None)])
def test_unaligned_k_lds_path(gpu, oracle_mod, M, N, K, act):
    # M > 64 with K % 128 != 0 runs the register-staged LDS kernel (everything
    # else past the skinny range runs the large-M kernel): 64x64 tiles under one
    # round of 256x128 tiles, 256x128 tiles above (2048x8192 GLU)
    from instinctflash_amd.kernels import pack_glu
    qa, sa, fw, g = _make(gpu, M, N, K, seed=M + K, bias=True)
    glu = act in ("geglu", "swiglu")
    res = torch.randn((M, N // 2 if glu else N), generator=g).to(torch.bfloat16)
    _check(gpu, oracle_mod, qa, sa, pack_glu(fw) if glu else fw, f"lds {M}x{N}x{K}", ref_w=fw, act=act,
           residual=res)


@pytest.mark.parametrize("M,N,K,act", [(65, 2048, 2048, None), (100, 2560, 2048, "gelu_tanh"), (128, 1024, 4096, None),
                                       (96, 1056, 8192, None), (96, 4096, 1024, "geglu"), (72, 2048, 6144, "swiglu")])
def test_mid_m_large_kernel(gpu, oracle_mod, M, N, K, act):
    # 64 < M <= 128 with K % 128 == 0: the large-M kernel's small-grid tiles
    # (32-token tiles, split K for K > 4096), GLU included
    from instinctflash_amd.kernels import pack_glu
    qa, sa, fw, g = _make(gpu, M, N, K, seed=M + N, bias=True)
    glu = act in ("geglu", "swiglu")
    res = torch.randn((M, N // 2 if glu else N), generator=g).to(torch.bfloat16)
    _check(gpu, oracle_mod, qa, sa, pack_glu(fw) if glu else fw, f"mid {M}x{N}x{K}", ref_w=fw, act=act, residual=res)


def test_fp32_output(gpu, oracle_mod):
    qa, sa, fw, _ = _make(gpu, 100, 512, 512, seed=8, bias=True)
    o32, _ = _check(gpu, oracle_mod, qa, sa, fw, "f32 out")
    assert o32.dtype == torch.float32


def test_strided_operands(gpu, oracle_mod):
    from instinctflash_amd.kernels import linear
    M, N, K = 96, 256, 512
    qa, sa, fw, _ = _make(gpu, M, N, K, seed=9)
    abig = torch.zeros((M, K + 128), dtype=torch.float8_e4m3fn, device=gpu)
    abig[:, 64:64 + K] = qa
    obig = torch.zeros((M, N + 64), dtype=torch.bfloat16, device=gpu)
    out = obig[:, 32:32 + N]
    linear(abig[:, 64:64 + K], sa, fw, out=out)
    _assert_close(_f(out), _ref(oracle_mod, qa, sa, fw), "strided")
    assert not obig[:, :32].any() and not obig[:, 32 + N:].any()


@pytest.mark.parametrize("M,N,K", [(16, 1536, 6144), (50, 4096, 1024), (512, 1024, 2048)])
def test_deterministic(gpu, M, N, K):
    from instinctflash_amd.kernels import linear
    qa, sa, fw, _ = _make(gpu, M, N, K, seed=10)
    a = linear(qa, sa, fw)
    for _ in range(3):
        b = linear(qa, sa, fw)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_edge_rows_untouched(gpu, oracle_mod):
    # M not a multiple of any tile: rows past M must not be written.
    from instinctflash_amd.kernels import linear
    M, N, K = 70, 512, 256
    qa, sa, fw, _ = _make(gpu, M, N, K, seed=12)
    obig = torch.full((M + 8, N), 7.0, dtype=torch.bfloat16, device=gpu)
    linear(qa, sa, fw, out=obig[:M])
    assert (obig[M:] == 7.0).all()


def test_graph_capture_replay(gpu, oracle_mod):
    from instinctflash_amd.kernels import linear, quant_rows
    M, N, K = 16, 1536, 6144
    g = torch.Generator().manual_seed(13)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).to(gpu)
    from instinctflash_amd.kernels import quantize_weight
    fw = quantize_weight(torch.randn((N, K), generator=g) * 0.02, device=gpu)
    qa = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=gpu)
    sa = torch.empty(M, device=gpu)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        for _ in range(2):
            quant_rows(x, qa, sa)
            linear(qa, sa, fw, out=out)
    torch.cuda.current_stream().wait_stream(st)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):
        quant_rows(x, qa, sa)
        linear(qa, sa, fw, out=out)
    for i in range(4):
        x.copy_(torch.randn((M, K), generator=g).to(torch.bfloat16).to(gpu))
        graph.replay()
        torch.cuda.synchronize()
        q2, s2 = quant_rows(x)
        eager = linear(q2, s2, fw)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {i}"


def test_contract_errors(gpu):
    from instinctflash_amd.kernels import linear, pack_glu
    qa, sa, fw, _ = _make(gpu, 16, 64, 128, seed=14)
    with pytest.raises(ValueError):
        linear(qa, sa, fw, act="relu")
    with pytest.raises(ValueError):
        linear(qa, sa, fw, act="geglu")  # not packed
    with pytest.raises(ValueError):
        linear(qa.float(), sa, fw)
    with pytest.raises(ValueError):
        linear(qa[:, :120], sa, fw)
    p = pack_glu(fw)
    with pytest.raises(ValueError):
        linear(qa, sa, p)  # packed weight needs a GLU epilogue


def test_workspace_reuse_across_shapes(gpu, oracle_mod):
    # Regression: calls with different plans share one workspace per stream,
    # whatever an earlier call left in it (large-M split-K calls of 32 and 8
    # slices between skinny calls, which need none).
    seq = [(16, 64, 4096), (100, 256, 16384), (16, 1536, 6144), (300, 512, 4736), (64, 256, 2048),
           (100, 256, 16384), (1, 512, 8192), (50, 96, 4096)]
    for i, (M, N, K) in enumerate(seq):
        qa, sa, fw, _ = _make(gpu, M, N, K, seed=100 + i)
        from instinctflash_amd.kernels import linear
        out = linear(qa, sa, fw, out_dtype=torch.float32)
        _assert_close(_f(out), _ref(oracle_mod, qa, sa, fw), f"seq {i}: {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,act", [(816, 2048, 16384, None), (512, 1024, 2048, None), (300, 1024, 4096, "swiglu"),
                                       (1024, 2048, 11008, None), (257, 512, 2048, "gelu_tanh"),
                                       (128, 4096, 2048, "geglu"), (100, 256, 16384, None), (200, 768, 8192, "gelu_tanh")])
def test_split_k_shapes(gpu, oracle_mod, M, N, K, act):
    # few output tiles: the large-M kernel splits K and a reduce kernel adds the
    # partials in slice order and applies the epilogue (100 x 256 x 16384: one
    # tile, 32 slices)
    from instinctflash_amd import _lib
    from instinctflash_amd.kernels import fp8 as F, pack_glu
    glu = act in ("geglu", "swiglu")
    assert _lib.load().ifx_fp8_linear_workspace_size(M, N, K, _lib.EPI_GEGLU if glu else 0) > 0
    qa, sa, fw, g = _make(gpu, M, N, K, seed=M + N, bias=True)
    res = torch.randn((M, N // 2 if glu else N), generator=g).to(torch.bfloat16)
    w = pack_glu(fw) if glu else fw
    o32, o16 = _check(gpu, oracle_mod, qa, sa, w, f"split {M}x{N}x{K}", ref_w=fw, act=act, residual=res)
    # repeated calls: bit-identical (fixed slice order), the workspace
    # overwritten with a nonzero pattern in between
    for _ in range(3):
        for ws in F._WORKSPACES.values():
            ws.fill_(0xA5)
        again = F.linear(qa, sa, w, act=act, residual=res.to(gpu), out_dtype=torch.float32)
        assert torch.equal(again.view(torch.int32), o32.view(torch.int32))
    # in place: out aliases the residual
    r = res.to(gpu).clone()
    F.linear(qa, sa, w, out=r, act=act, residual=r)
    assert torch.equal(r.view(torch.int16), o16.view(torch.int16))


@pytest.mark.parametrize("M,N,K,act", [
    (100, 256, 128, None), (100, 256, 256, "gelu_tanh"), (100, 256, 384, None),  # 32-token tiles, 4-stage ring
    (600, 2048, 256, None), (1024, 2048, 256, None),  # 3-stage rings with fewer K stages than slots
    (1024, 2048, 384, "swiglu"),
    (300, 512, 4736, None),  # 128 x 256 split tiles: 8 slices of 5 stages, the last of 2
    (300, 512, 5248, "gelu_tanh"),  # 9 slices of 5 stages, the last of 1
])
def test_ring_depth_edges(gpu, oracle_mod, M, N, K, act):
    # K shorter than the operand ring, and split-K slices shorter than the ring,
    # in the 3- and 4-stage rings of the small-grid and split tiles
    from instinctflash_amd.kernels import pack_glu
    glu = act in ("geglu", "swiglu")
    qa, sa, fw, g = _make(gpu, M, N, K, seed=M * 7 + K, bias=True)
    res = torch.randn((M, N // 2 if glu else N), generator=g).to(torch.bfloat16)
    w = pack_glu(fw) if glu else fw
    _check(gpu, oracle_mod, qa, sa, w, f"ring {M}x{N}x{K}", ref_w=fw, act=act, residual=res)


@pytest.mark.parametrize("case", ["wide", "wide_glu", "wide192", "narrow", "narrow_glu"])
def test_operands_past_4gib(gpu, oracle_mod, case):
    # An activation operand spanning >= 4 GiB (the 4-wave loops form 32-bit DMA
    # offsets): the 8-wave forms run -- 256 x 256 tiles (GLU: the 256 x 192 choice
    # falls back to them), and 128 x 256 split-K tiles over a row-strided operand.
    # Sampled rows against the oracle, rows past the 4 GiB offset included.
    from instinctflash_amd.kernels import linear, pack_glu, quantize_weight
    if case in ("narrow", "narrow_glu"):  # 126 tiles of 128 x 256: K split in two (plain)
        M, N, K, lda = 16100, 512 if case == "narrow_glu" else 256, 4224, 268448
    elif case == "wide192":  # 8192 x 3072: 256 x 192 tiles (two full rounds), row-strided operand
        M, N, K, lda = 8192, 3072, 3072, 524400
    else:
        M, N, K, lda = 524544, 512 if case == "wide_glu" else 256, 8192, 8192
    assert M * lda >= 1 << 32 and M < 1 << 24
    print(f"[4gib] {case} {M}x{N}x{K} lda={lda}", flush=True)
    gg = torch.Generator(device=gpu).manual_seed(11)
    buf = torch.randint(0, 256, (M, lda), dtype=torch.uint8, device=gpu, generator=gg)
    buf.bitwise_and_(0xBF)  # exponent field <= 7: |x| <= 1.875, no NaN codes
    a = buf[:, :K].view(torch.float8_e4m3fn)
    sa = torch.rand(M, device=gpu, generator=gg) + 0.5
    g = torch.Generator().manual_seed(12)
    fw = quantize_weight(torch.randn((N, K), generator=g) * 0.02, torch.randn(N, generator=g) * 0.01, device=gpu)
    act = "swiglu" if case.endswith("glu") else None
    w = pack_glu(fw) if act else fw
    out = linear(a, sa, w, act=act, out_dtype=torch.float32)
    ob = linear(a, sa, w, act=act, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    first_past = (1 << 32) // lda + 1  # first row whose bytes start past 4 GiB
    rows = np.unique(np.concatenate([np.array([0, 1, M // 2, first_past - 1, first_past, M - 2, M - 1]),
                                     np.random.default_rng(3).choice(M, 57, replace=False)]))
    ridx = torch.as_tensor(rows, device=gpu)
    ref = oracle_mod.ref_linear(_q(a[ridx]), _f(sa[ridx]), _q(fw.w), _f(fw.scale), bias=_f(fw.bias), act=act)
    _assert_close(_f(out[ridx]), ref, f"4gib {case}")
    assert torch.equal(ob[ridx].view(torch.int16), out[ridx].to(torch.bfloat16).view(torch.int16))
    del buf, a, out, ob
    torch.cuda.empty_cache()


@pytest.mark.parametrize("M,N,K,act", [
    (32, 4096, 1024, None), (32, 4096, 4096, None), (40, 4096, 4096, "gelu_tanh"), (64, 4096, 4096, None),
    (32, 4096, 4096, "swiglu"), (40, 2048, 1024, "geglu"), (64, 16384, 1024, "swiglu"), (48, 8192, 1024, None),
])
def test_skinny_token_block_forms(gpu, oracle_mod, M, N, K, act):
    # 2-4 token blocks per workgroup (256 or more row groups, so no split over
    # the tokens), with 4 or 8 waves, plain and GLU
    from instinctflash_amd.kernels import pack_glu
    glu = act in ("geglu", "swiglu")
    qa, sa, fw, g = _make(gpu, M, N, K, seed=M + N + K, bias=True)
    res = torch.randn((M, N // 2 if glu else N), generator=g).to(torch.bfloat16)
    w = pack_glu(fw) if glu else fw
    o32, _ = _check(gpu, oracle_mod, qa, sa, w, f"skinny blocks {M}x{N}x{K}", ref_w=fw, act=act, residual=res)
    # the tile-layout weights: bit-identical
    from instinctflash_amd.kernels import fp8 as F, pack_skinny
    got = F.linear(qa, sa, pack_skinny(w), act=act, residual=res.to(gpu), out_dtype=torch.float32)
    assert torch.equal(got.view(torch.int32), o32.view(torch.int32)), f"tiled skinny blocks {M}x{N}x{K}"


@pytest.mark.parametrize("M,N,K", [(16, 1536, 6144), (16, 768, 3072), (8, 1024, 4096), (1, 1024, 16384),
                                   (16, 512, 8192)])
def test_skinny_needs_no_workspace(gpu, M, N, K):
    # M <= 64 never splits K across workgroups
    from instinctflash_amd import _lib
    assert _lib.load().ifx_fp8_linear_workspace_size(M, N, K, 0) == 0


@pytest.mark.parametrize("M,N,K", [(16, 1536, 6144), (200, 512, 1024), (1024, 2048, 2048)])
def test_per_tensor_scales(gpu, oracle_mod, M, N, K):
    # per-tensor activation and weight scales (reference runtime/torch_fp8_linear.py:75-78)
    from instinctflash_amd.kernels import Fp8Weight, linear, quantize_tensor
    g = torch.Generator().manual_seed(M)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    w = (torch.randn((N, K), generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.01
    qa, sa = quantize_tensor(x.to(gpu))
    qw, sw = quantize_tensor(w.to(gpu))
    fw = Fp8Weight(qw, sw, b.to(gpu))
    o32 = linear(qa, sa, fw, out_dtype=torch.float32)
    o16 = linear(qa, sa, fw)
    ref = oracle_mod.ref_linear(_q(qa), np.full(M, _f(sa)[0], np.float32), _q(qw), np.full(N, _f(sw)[0], np.float32),
                                bias=b.numpy())
    _assert_close(_f(o32), ref, "per-tensor")
    assert torch.equal(o16.view(torch.int16), o32.to(torch.bfloat16).view(torch.int16))


def test_fp8_linear_module(gpu, oracle_mod):
    # Gfx950FP8Linear mirrors ThorFP8Linear (runtime/torch_fp8_linear.py:10-79)
    from instinctflash_amd.modules import Gfx950FP8Linear
    torch.manual_seed(0)
    lin = torch.nn.Linear(1024, 512, dtype=torch.bfloat16).to(gpu)
    mod = Gfx950FP8Linear(lin)
    x = torch.randn((3, 7, 1024), device=gpu).to(torch.bfloat16)
    y = mod(x)
    assert y.shape == (3, 7, 512) and y.dtype == torch.bfloat16
    # weight recipe: per-tensor, reciprocal scale, bit-exact
    wq, ws = oracle_mod.quant_tensor(lin.weight.detach().cpu().view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(_q(mod.weight_fp8), wq) and _f(mod.weight_scale).view(np.uint32)[0] == ws.view(np.uint32)[0]
    xq, xs = oracle_mod.quant_tensor(x.reshape(-1, 1024).cpu().view(torch.int16).numpy().view(np.uint16))
    ref = oracle_mod.ref_linear(xq, np.full(21, xs[0], np.float32), wq, np.full(512, ws[0], np.float32),
                                bias=lin.bias.detach().float().cpu().numpy())
    d, cos = oracle_mod.parity_stats(_f(y.reshape(-1, 512)), ref)
    assert cos >= TOL_COS and d <= TOL_MAXD + 2.0 ** -8 * np.abs(ref).max() / np.sqrt(np.mean(ref ** 2))
    assert mod(x[:0]).shape == (0, 7, 512)
    with pytest.raises(ValueError):
        mod(x.float())
    with pytest.raises(TypeError):
        Gfx950FP8Linear(torch.nn.Sequential(lin))
    with pytest.raises(ValueError):
        Gfx950FP8Linear(torch.nn.Linear(1000, 512, dtype=torch.bfloat16).to(gpu))


@pytest.mark.parametrize("M,N,K,act", [(16, 1536, 8192, None), (1, 512, 8208, None), (9, 1024, 8336, "gelu_tanh"),
                                       (16, 2048, 8192, "geglu"), (13, 4096, 16384, "swiglu")])
def test_skinny_long_k(gpu, oracle_mod, M, N, K, act):
    # one token block, <= 128 row groups and K >= 64 steps of 128: one
    # workgroup (or two row halves) per group streams the whole of K
    from instinctflash_amd import _lib
    from instinctflash_amd.kernels import fp8 as F, pack_glu
    glu = act in ("geglu", "swiglu")
    assert _lib.load().ifx_fp8_linear_workspace_size(M, N, K, _lib.EPI_GEGLU if glu else 0) == 0
    qa, sa, fw, g = _make(gpu, M, N, K, seed=M + N + K, bias=True)
    n_out = N // 2 if glu else N
    res = torch.randn((M, n_out), generator=g).to(torch.bfloat16)
    w = pack_glu(fw) if glu else fw
    o32, o16 = _check(gpu, oracle_mod, qa, sa, w, f"skinny long K {M}x{N}x{K}", ref_w=fw, act=act, residual=res)
    # repeated calls: bit-identical (fixed slice order), the workspace
    # overwritten with a nonzero pattern in between
    for _ in range(3):
        for ws in F._WORKSPACES.values():
            ws.fill_(0xA5)
        again = F.linear(qa, sa, w, act=act, residual=res.to(gpu), out_dtype=torch.float32)
        assert torch.equal(again.view(torch.int32), o32.view(torch.int32))
    # in place: out aliases the residual
    r = res.to(gpu).clone()
    F.linear(qa, sa, w, out=r, act=act, residual=r)
    assert torch.equal(r.view(torch.int16), o16.view(torch.int16))


def _tile_layout_np(w, K):
    """Numpy restatement of the pack_skinny layout (ifx_fp8.h): tile (b, s) holds, for
    lane l, row 16b + l%16 K bytes [128s + 32(l/16), +16) at 16l and the next 16 at 1024+16l."""
    N = w.shape[0]
    ks = -(-K // 128)
    wp = np.zeros((N, ks * 128), np.uint8)
    wp[:, :K] = w[:, :K]
    out = np.zeros((N // 16, ks, 2, 64, 16), np.uint8)
    for l in range(64):
        rows = np.arange(N // 16) * 16 + (l % 16)
        for half in range(2):
            for s in range(ks):
                k0 = 128 * s + 32 * (l // 16) + 16 * half
                out[:, s, half, l] = wp[rows, k0:k0 + 16]
    return out.reshape(-1)


@pytest.mark.parametrize("M,N,K,act", [(16, 6144, 1536, "gelu_tanh"), (16, 1536, 6144, None), (50, 4096, 1024, None),
                                       (1, 16, 128, None), (33, 48, 176, None), (16, 2048, 1536, "geglu"),
                                       (13, 4096, 16384, "swiglu"), (64, 256, 2064, "gelu_tanh")])
def test_skinny_tiled_weights(gpu, M, N, K, act):
    # pack_skinny: the tile bytes follow the documented layout, and the projection is
    # bit-identical to the row-major weight's (same bytes in the same fragment slots)
    from instinctflash_amd.kernels import fp8 as F, pack_glu, pack_skinny
    glu = act in ("geglu", "swiglu")
    qa, sa, fw, g = _make(gpu, M, N, K, seed=N + K, bias=True)
    w = pack_glu(fw) if glu else fw
    wt = pack_skinny(w)
    assert wt.tiled and wt.shape == (N, K) and wt.glu == glu
    assert np.array_equal(_q(wt.w), _tile_layout_np(_q(w.w), K))
    n_out = N // 2 if glu else N
    res = torch.randn((M, n_out), generator=g).to(torch.bfloat16).to(gpu)
    gate = torch.rand(n_out, generator=g).to(torch.bfloat16).to(gpu)
    for dt in (torch.bfloat16, torch.float32):
        ref = F.linear(qa, sa, w, act=act, residual=res, gate=gate, out_dtype=dt)
        got = F.linear(qa, sa, wt, act=act, residual=res, gate=gate, out_dtype=dt)
        iv = torch.int16 if dt == torch.bfloat16 else torch.int32
        assert torch.equal(got.view(iv), ref.view(iv)), f"tiled {M}x{N}x{K} {act} {dt}"
    if not glu:
        raw_ref = torch.empty((M, N), dtype=torch.bfloat16, device=gpu)
        raw = torch.empty_like(raw_ref)
        F.gemm(qa, fw, raw_ref)
        F.gemm(qa, wt, raw)
        assert torch.equal(raw.view(torch.int16), raw_ref.view(torch.int16))


def test_skinny_tiled_contract(gpu):
    from instinctflash_amd.kernels import fp8 as F, pack_glu, pack_skinny
    qa, sa, fw, g = _make(gpu, 16, 256, 512, seed=1)
    wt = pack_skinny(fw)
    big = torch.zeros((65, 512), dtype=torch.float8_e4m3fn, device=gpu)
    with pytest.raises(ValueError, match="M <= 64"):
        F.linear(big, torch.ones(65, device=gpu), wt)
    with pytest.raises(ValueError, match="before pack_skinny"):
        pack_glu(wt)
    assert pack_skinny(wt) is wt


def _tile_rows_np(q, M, K):
    """Tile layout of an [M, K] e4m3 activation (rows padded to 16, K to 128 with zeros)."""
    mp = -(-M // 16) * 16
    full = np.zeros((mp, K), np.uint8)
    full[:M] = q
    return _tile_layout_np(full, K)


@pytest.mark.parametrize("M,N,K,act", [(16, 6144, 1536, "gelu_tanh"), (16, 1536, 6144, None), (50, 4096, 1024, None),
                                       (1, 16, 128, None), (33, 48, 176, None), (16, 2048, 1536, "geglu"),
                                       (64, 256, 2064, "gelu_tanh")])
def test_tiled_activations(gpu, M, N, K, act):
    # quant_rows_tiled writes quant_rows' bytes in the tile layout (zeros elsewhere), and
    # linear on it is bit-identical to linear on the row-major activations, with row-major
    # or tiled weights
    from instinctflash_amd.kernels import fp8 as F, pack_glu, pack_skinny, quant_rows, quant_rows_tiled
    glu = act in ("geglu", "swiglu")
    g = torch.Generator().manual_seed(M + K)
    x = (torch.randn((M, K), generator=g) * 3).to(torch.bfloat16).to(gpu)
    qa, sa = quant_rows(x)
    ta, ts = quant_rows_tiled(x)
    assert torch.equal(ts.view(torch.int32), sa.view(torch.int32))
    assert np.array_equal(_q(ta.q), _tile_rows_np(_q(qa), M, K))
    _, _, fw, _ = _make(gpu, 1, N, K, seed=N, bias=True)
    w = pack_glu(fw) if glu else fw
    n_out = N // 2 if glu else N
    res = torch.randn((M, n_out), generator=g).to(torch.bfloat16).to(gpu)
    ref = F.linear(qa, sa, w, act=act, residual=res, out_dtype=torch.float32)
    for weight in (w, pack_skinny(w)):
        got = F.linear(ta, ts, weight, act=act, residual=res, out_dtype=torch.float32)
        assert torch.equal(got.view(torch.int32), ref.view(torch.int32)), f"tiled A {M}x{N}x{K} {act}"


@pytest.mark.parametrize("M,N,K,act,resgate", [(4096, 3072, 640, "gelu_tanh", False), (4000, 3008, 512, None, True),
                                               (4096, 3072, 384, None, False)])
def test_wide_192_row_tiles(gpu, oracle_mod, M, N, K, act, resgate):
    # output shapes whose 256-row tiles would leave a partial round on 256 CUs take
    # 192-row weight tiles; ragged N ends inside a tile
    qa, sa, fw, g = _make(gpu, M, N, K, seed=M + N + K, bias=True)
    res = torch.randn((M, N), generator=g).to(torch.bfloat16) if resgate else None
    gate = torch.rand(N, generator=g).to(torch.bfloat16) if resgate else None
    _check(gpu, oracle_mod, qa, sa, fw, f"wide192 {M}x{N}x{K}", act=act, residual=res, gate=gate)


@pytest.mark.parametrize("M,N,K,act,resgate", [(16, 1536, 6144, None, True), (1, 16, 256, "gelu_tanh", False),
                                               (9, 48, 2048, None, True), (16, 2048, 1024, "gelu_tanh", True),
                                               (13, 1024, 3072, None, False)])
def test_skinny_row_halves(gpu, oracle_mod, M, N, K, act, resgate):
    # one token block, unsplit K and <= 128 row groups: two workgroups per group,
    # each streaming 8 of its 16 weight rows and storing their outputs; row-major
    # and tile-layout weights, bit-identical, and repeated calls identical
    from instinctflash_amd.kernels import fp8 as F, pack_skinny
    qa, sa, fw, g = _make(gpu, M, N, K, seed=M * 3 + N + K, bias=True)
    res = torch.randn((M, N), generator=g).to(torch.bfloat16) if resgate else None
    gate = torch.rand(N, generator=g).to(torch.bfloat16) if resgate else None
    o32, _ = _check(gpu, oracle_mod, qa, sa, fw, f"row halves {M}x{N}x{K}", act=act, residual=res, gate=gate)
    kw = dict(act=act, residual=None if res is None else res.to(gpu), gate=None if gate is None else gate.to(gpu),
              out_dtype=torch.float32)
    got = F.linear(qa, sa, pack_skinny(fw), **kw)
    assert torch.equal(got.view(torch.int32), o32.view(torch.int32)), f"tiled row halves {M}x{N}x{K}"
    for _ in range(2):
        assert torch.equal(F.linear(qa, sa, fw, **kw).view(torch.int32), o32.view(torch.int32))

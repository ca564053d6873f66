"""GPU parity of the pre-norm producer ``residual_norm_quant`` (reference
instinctflash/kernels/norm.py:25-123) against the CPU oracle.

Bars:
  * residual update: bit-exact (float32 operations in the reference's order, no
    contraction; bf16 residuals store RNE of the sum);
  * normalized row y (fp32 output): |y - y_oracle| <= 1e-5 * max|y_oracle| per
    row -- the device sums the row in a different order than float64 numpy;
  * quantization: q and q_scale bit-exact against the oracle quantizer applied
    to the kernel's own fp32 y (the recipe is exact given y), and within the
    reference test's bar (tests/test_gi_kernels.py:112, 7% of the row max)
    against the oracle's y.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(M, D, seed, res_dtype=torch.float32, n_tables=0, delta_dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    t = dict(
        res=torch.randn(M, D, generator=g).to(res_dtype),
        delta=(torch.randn(M, D, generator=g) * 4).to(delta_dtype),
        delta_row=torch.rand(M, generator=g), delta_col=torch.rand(D, generator=g),
        bias=torch.randn(D, generator=g), weight=torch.rand(D, generator=g) + 0.5, beta=torch.randn(D, generator=g),
    )
    rows = (n_tables, D) if n_tables else (D,)
    t["gate"] = torch.rand(rows, generator=g)
    t["mod_scale"] = torch.randn(rows, generator=g) * 0.1
    t["mod_shift"] = torch.randn(rows, generator=g) * 0.1
    if n_tables:
        t["mod_index"] = torch.randint(0, n_tables, (M,), generator=g, dtype=torch.int32)
    return t


def _run(gpu, t, use, layernorm, write_res=True, y_dtype=torch.float32, quant=True, eps=1e-6):
    from instinctflash_amd.kernels import E4M3, residual_norm_quant
    M, D = t["res"].shape
    d = {k: v.to(gpu) for k, v in t.items()}
    res = d["res"].clone()
    q = torch.empty(M, D, dtype=E4M3, device=gpu) if quant else None
    qs = torch.full((M,), -1.0, device=gpu) if quant else None
    y = torch.empty(M, D, dtype=y_dtype, device=gpu) if y_dtype is not None else None
    kw = {k: d[k] for k in use}
    residual_norm_quant(res, **kw, write_res=write_res, layernorm=layernorm, q=q, q_scale=qs, y=y, eps=eps)
    torch.cuda.synchronize()
    return res, q, qs, y


def _oracle(oracle_mod, t, use, layernorm, write_res=True, eps=1e-6):
    kw = {k: t[k].float().numpy() if k != "mod_index" else t[k].numpy() for k in use}
    return oracle_mod.residual_norm(t["res"].float().numpy(), **kw, write_res=write_res, layernorm=layernorm,
                                    eps=eps, res_bf16=t["res"].dtype == torch.bfloat16)


def _check(gpu, oracle_mod, t, use, layernorm, what, write_res=True):
    res, q, qs, y = _run(gpu, t, use, layernorm, write_res)
    x_ref, y_ref = _oracle(oracle_mod, t, use, layernorm, write_res)
    # residual
    if write_res and "delta" in use:
        got = res.float().cpu().numpy()
        assert np.array_equal(got.view(np.uint32), x_ref.view(np.uint32)), f"{what}: residual not bit-exact"
    else:
        assert torch.equal(res.cpu(), t["res"]), f"{what}: residual must be untouched"
    # normalized row
    yk = y.cpu().numpy()
    err = np.abs(yk - y_ref).max(axis=1) / np.abs(y_ref).max(axis=1)
    assert err.max() <= 1e-5, f"{what}: y rel err {err.max():.3e}"
    # quantization of the kernel's own y: exact
    qo, so = oracle_mod.quant_rows(yk)
    assert np.array_equal(q.cpu().view(torch.uint8).numpy(), qo), f"{what}: q bytes"
    assert np.array_equal(qs.cpu().numpy().view(np.uint32), so.view(np.uint32)), f"{what}: q_scale"
    # and against the oracle's y, at the reference test's bar
    deq = oracle_mod.e4m3_decode(qo) * so[:, None]
    assert (np.abs(deq - y_ref).max(axis=1) / np.abs(y_ref).max(axis=1)).max() < 0.07
    return res, q, qs, y


ALL = ["delta", "delta_row", "delta_col", "bias", "gate", "weight", "beta", "mod_scale", "mod_shift"]


@pytest.mark.parametrize("layernorm", [False, True])
def test_reference_case(gpu, oracle_mod, layernorm):
    # the reference's own test shape and options (tests/test_gi_kernels.py:93-112)
    _check(gpu, oracle_mod, _inputs(33, 1152, 3), ALL, layernorm, f"reference case ln={layernorm}")


@pytest.mark.parametrize("M,D", [(1, 8), (16, 1536), (50, 1024), (7, 2040), (64, 3072), (5, 4096), (3, 16384),
                                 (816, 2048)])
@pytest.mark.parametrize("layernorm", [False, True])
def test_shapes(gpu, oracle_mod, M, D, layernorm):
    _check(gpu, oracle_mod, _inputs(M, D, M + D), ALL, layernorm, f"{M}x{D} ln={layernorm}")


@pytest.mark.parametrize("D", [1024, 3072, 6144, 12288])  # 1, 2, 4, 8 groups of 8 values per lane
@pytest.mark.parametrize("M", [5, 1030])  # one row per workgroup / the many-rows form (M >= 1024)
@pytest.mark.parametrize("res_dtype,delta_dtype", [(torch.float32, torch.bfloat16), (torch.float32, torch.float32),
                                                   (torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32)])
def test_width_and_dtype_forms(gpu, oracle_mod, D, M, res_dtype, delta_dtype):
    # every compiled form of the producer: lane width x residual dtype x delta dtype x row form
    t = _inputs(M, D, M + D, res_dtype=res_dtype, delta_dtype=delta_dtype)
    _check(gpu, oracle_mod, t, ALL, D % 2048 == 0, f"{M}x{D} res {res_dtype} delta {delta_dtype}")


@pytest.mark.parametrize("use", [[], ["weight"], ["mod_scale", "mod_shift"], ["delta"], ["delta", "delta_col"],
                                 ["delta", "delta_row", "bias"], ["delta", "gate", "weight", "beta"]])
def test_option_subsets(gpu, oracle_mod, use):
    _check(gpu, oracle_mod, _inputs(24, 1536, 11), use, True, f"options {use}")
    _check(gpu, oracle_mod, _inputs(24, 1536, 12), use, False, f"options {use} rms")


def test_per_row_tables(gpu, oracle_mod):
    # Wan-style: gate / modulation tables [n, D] selected per row by int32 mod_index
    t = _inputs(40, 3072, 5, res_dtype=torch.bfloat16, n_tables=3)
    _check(gpu, oracle_mod, t, ALL + ["mod_index"], True, "tables, bf16 residual")


def test_bf16_residual_and_no_write(gpu, oracle_mod):
    t = _inputs(16, 1536, 6, res_dtype=torch.bfloat16)
    _check(gpu, oracle_mod, t, ALL, True, "bf16 residual")
    _check(gpu, oracle_mod, _inputs(16, 1536, 7), ALL, False, "write_res=False", write_res=False)


def test_bf16_y_and_q_only(gpu, oracle_mod):
    t = _inputs(20, 2048, 8)
    res, q, qs, y = _run(gpu, t, ALL, True, y_dtype=torch.bfloat16)
    res2, q2, qs2, _ = _run(gpu, t, ALL, True, y_dtype=None)
    assert torch.equal(q, q2) and torch.equal(qs, qs2) and torch.equal(res, res2)
    _, y_ref = _oracle(oracle_mod, t, ALL, True)
    yb = y.float().cpu().numpy()
    assert (np.abs(yb - y_ref).max(axis=1) / np.abs(y_ref).max(axis=1)).max() < 2 ** -8


def test_nonfinite_propagates(gpu, oracle_mod):
    t = _inputs(4, 1024, 9)
    t["delta"][1, 17] = float("nan")
    t["delta"][2, 3] = float("inf")
    res, q, qs, y = _run(gpu, t, ALL, False)
    qs = qs.cpu()
    assert torch.isnan(qs[1]) and torch.isnan(qs[2]) and torch.isfinite(qs[[0, 3]]).all()
    qo, so = oracle_mod.quant_rows(y.cpu().numpy())
    assert np.array_equal(q.cpu().view(torch.uint8).numpy()[[0, 3]], qo[[0, 3]])


def test_deterministic_and_graph_replay(gpu):
    from instinctflash_amd.kernels import E4M3, residual_norm_quant
    t = {k: v.to(gpu) for k, v in _inputs(64, 3072, 13).items()}
    base = t["res"].clone()
    q = torch.empty(64, 3072, dtype=E4M3, device=gpu)
    qs = torch.empty(64, device=gpu)
    kw = {k: t[k] for k in ALL}
    res = base.clone()
    residual_norm_quant(res, **kw, layernorm=True, q=q, q_scale=qs)
    ref = (res.clone(), q.clone(), qs.clone())
    work = base.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        residual_norm_quant(work, **kw, layernorm=True, q=q, q_scale=qs)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        residual_norm_quant(work, **kw, layernorm=True, q=q, q_scale=qs)
    for _ in range(3):
        work.copy_(base)
        q.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(work, ref[0]) and torch.equal(q.view(torch.uint8), ref[1].view(torch.uint8))
        assert torch.equal(qs, ref[2])


def test_contract_errors(gpu):
    from instinctflash_amd import _lib
    from instinctflash_amd.kernels import E4M3, residual_norm_quant
    res = torch.zeros(4, 1024, device=gpu)
    with pytest.raises(ValueError):
        residual_norm_quant(res, mod_scale=torch.zeros(1024, device=gpu))  # shift missing
    with pytest.raises(ValueError):
        residual_norm_quant(res, router=(None,))
    with pytest.raises(ValueError):
        residual_norm_quant(res, q=torch.empty(4, 1024, dtype=E4M3, device=gpu))  # no q_scale
    with pytest.raises(ValueError):
        residual_norm_quant(res, weight=torch.zeros(1024, device=gpu, dtype=torch.bfloat16))
    with pytest.raises(_lib.IfxError):
        residual_norm_quant(torch.zeros(4, 1020, device=gpu))  # D % 8
    with pytest.raises(_lib.IfxError):
        residual_norm_quant(torch.zeros(2, 16392, device=gpu))  # D > 16384

"""GPU parity of ``wan_qkv`` (reference instinctflash/kernels/wan.py:84-116)
against the CPU oracle. Bar as for qkv_split: |out - ref| <= u * |ref| + 2e-5
with u = 2x the output format's unit roundoff (fp32: 2e-5); pool rows other
than the slots written stay untouched."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

U = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2e-5}


def _close(got, ref, dt, what):
    g = got.float().cpu().numpy().astype(np.float64)
    err = np.abs(g - ref) - (U[dt] * np.abs(ref) + 2e-5)
    assert err.max() <= 0, f"{what}: worst excess {err.max():.3e}"


def _case(B, T, H, HD, parts, seed, rope=True, norm=True):
    from instinctflash_amd.kernels.rope import rope_inv_freq
    g = torch.Generator().manual_seed(seed)
    D = H * HD
    c = dict(raw=torch.randn(B * T, parts * D, generator=g).to(torch.bfloat16),
             row=torch.rand(B * T, generator=g) + 0.5, col=torch.rand(parts * D, generator=g) + 0.5,
             bias=torch.randn(parts * D, generator=g))
    if norm:
        c["q_norm"], c["k_norm"] = torch.rand(D, generator=g) + 0.5, torch.rand(D, generator=g) + 0.5
    if rope:
        c["inv_freq"] = rope_inv_freq(HD, 1e4, "cpu")
        c["pos"] = torch.randint(0, 300, (T, 3), generator=g).float()
        c["sections"] = (torch.arange(HD // 2) % 3).int()
    c["slots"] = torch.randperm(2 * T, generator=g)[:T].int()
    return c


def _run_check(gpu, oracle_mod, B, T, H, HD, k, v, out_dtype, seed, **kw):
    from instinctflash_amd.kernels import wan_qkv
    D = H * HD
    parts = 1 + k + v
    c = _case(B, T, H, HD, parts, seed, **kw)
    d = {n: x.to(gpu) for n, x in c.items()}
    q = torch.empty(B * T, D, device=gpu, dtype=out_dtype)
    kp = torch.full((B, 2 * T, D), 7.0, device=gpu, dtype=out_dtype) if k else None
    vp = torch.full((B, 2 * T, D), 7.0, device=gpu, dtype=out_dtype) if v else None
    wan_qkv(d["raw"], q, heads=H, head_dim=HD, tokens=T, k_pool=kp, v_pool=vp, slots=d["slots"], row=d["row"],
            col=d["col"], bias=d["bias"], q_norm=d.get("q_norm"), k_norm=d.get("k_norm"), pos=d.get("pos"),
            sections=d.get("sections"), inv_freq=d.get("inv_freq"))
    torch.cuda.synchronize()
    n = lambda key: None if key not in c else c[key].float().numpy() if key != "sections" else c[key].numpy()  # noqa
    ref = oracle_mod.wan_qkv(c["raw"].float().numpy(), H, HD, T, parts, n("row"), n("col"), n("bias"), n("q_norm"),
                             n("k_norm"), n("inv_freq"), n("pos"), n("sections"))
    what = f"B{B} T{T} H{H} HD{HD} k{k} v{v} {out_dtype}"
    _close(q, ref[0], out_dtype, what + " q")
    slots = c["slots"].long()
    for p, pool in ((1, kp), (2, vp)):
        if pool is None or p >= parts:
            continue
        want = ref[p].reshape(B, T, D)
        _close(pool[:, slots], want, out_dtype, what + (" k" if p == 1 else " v"))
        others = torch.ones(2 * T, dtype=torch.bool)
        others[slots] = False
        assert (pool[:, others.to(gpu)] == 7.0).all(), what + " pool rows outside the slots"
    return q, kp, vp


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_wan5b_shape(gpu, oracle_mod, out_dtype):
    # Wan 5B: 24 heads x 128 (D = 3072), two batches, slot-permuted KV pools
    _run_check(gpu, oracle_mod, 2, 64, 24, 128, True, True, out_dtype, 1)


@pytest.mark.parametrize("H,HD", [(4, 64), (8, 256), (2, 8), (40, 128), (48, 256)])
def test_shapes(gpu, oracle_mod, H, HD):
    _run_check(gpu, oracle_mod, 1, 33, H, HD, True, True, torch.bfloat16, H + HD)


@pytest.mark.parametrize("k,v,opts", [(False, False, {}), (True, False, {}), (True, True, dict(rope=False)),
                                      (True, True, dict(norm=False)), (True, True, dict(rope=False, norm=False))])
def test_parts_and_options(gpu, oracle_mod, k, v, opts):
    _run_check(gpu, oracle_mod, 2, 16, 12, 128, k, v, torch.float16, 7, **opts)


def test_v_pool_without_k_pool_is_not_written(gpu):
    # the reference launches parts = 2 and part 1 is K (absent): V stays untouched
    from instinctflash_amd.kernels import wan_qkv
    raw = torch.randn(8, 2 * 256, device=gpu).to(torch.bfloat16)
    q = torch.empty(8, 256, device=gpu, dtype=torch.float16)
    vp = torch.full((1, 8, 256), 7.0, device=gpu, dtype=torch.float16)
    wan_qkv(raw, q, heads=2, head_dim=128, tokens=8, v_pool=vp)
    torch.cuda.synchronize()
    assert (vp == 7.0).all()
    assert torch.allclose(q.float(), raw[:, :256].float(), rtol=2 ** -9, atol=0)


def test_contract_errors(gpu):
    from instinctflash_amd.kernels import wan_qkv
    raw = torch.zeros(8, 3 * 256, device=gpu, dtype=torch.bfloat16)
    q = torch.empty(8, 256, device=gpu, dtype=torch.float16)
    with pytest.raises(ValueError, match="position table"):
        wan_qkv(raw, q, heads=2, head_dim=128, tokens=8, inv_freq=torch.ones(64, device=gpu))
    with pytest.raises(ValueError, match="batches"):
        wan_qkv(raw, q, heads=2, head_dim=128, tokens=3)
    with pytest.raises(ValueError, match="parts"):
        wan_qkv(raw[:, :256], q, heads=2, head_dim=128, tokens=8, k_pool=torch.empty(1, 8, 256, device=gpu,
                                                                                      dtype=torch.float16))

"""Host-side logic on the CPU: argument validation before launch, the gfx950
capability gates (with a stand-in torch module, as the reference's
tests/test_engine_available_kernels.py:11-16 does), the kernel declarations,
and the workloads' algorithmic FLOP/byte accounting."""
from types import SimpleNamespace

import pytest
import torch

from instinctflash_amd import backend
from instinctflash_amd.kernels import (Fp8Weight, dequant_rows, gated_act_quant, gemm, linear, pack_glu,
                                       quant_rows, quantize_tensor, row_quant)


# ---------------------------------------------------------------------------
# validation raises before anything is launched
# ---------------------------------------------------------------------------

def test_cpu_tensors_are_rejected_loudly():
    x = torch.randn(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="gfx950 device"):
        quant_rows(x)
    with pytest.raises(ValueError, match="gfx950 device"):
        quantize_tensor(x)
    w = Fp8Weight(torch.zeros(64, 64, dtype=torch.float8_e4m3fn), torch.ones(64))
    a = torch.zeros(4, 64, dtype=torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="gfx950 device"):
        linear(a, torch.ones(4), w)
    with pytest.raises(ValueError, match="gfx950 device"):
        gemm(a, w, torch.empty(4, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        row_quant(x, torch.empty(4, 64, dtype=torch.float8_e4m3fn), torch.empty(4))
    with pytest.raises(ValueError):
        gated_act_quant(x, torch.empty(4, 32, dtype=torch.float8_e4m3fn), torch.empty(4))
    with pytest.raises(ValueError):
        dequant_rows(x, torch.empty(4, 64))
    with pytest.raises(ValueError):
        pack_glu(w)


def test_dtype_and_activation_checks():
    with pytest.raises(ValueError, match="bf16 or fp32"):
        quant_rows(torch.zeros(2, 8, dtype=torch.float16))
    w = Fp8Weight(torch.zeros(64, 64, dtype=torch.float8_e4m3fn), torch.ones(64))
    with pytest.raises(ValueError, match="unknown activation"):
        linear(torch.zeros(4, 64, dtype=torch.float8_e4m3fn), torch.ones(4), w, act="relu")


# ---------------------------------------------------------------------------
# capability gates (reference engine_backend.py:302-333, engine_offload.py:33-100)
# ---------------------------------------------------------------------------

def fake_torch(arch="gfx950:sramecc+:xnack-", available=True):
    props = SimpleNamespace(gcnArchName=arch, major=9, minor=5)
    return SimpleNamespace(cuda=SimpleNamespace(is_available=lambda: available,
                                                get_device_properties=lambda i: props))


@pytest.mark.parametrize("backbone", backend.GI_ENGINE_BACKBONES)
def test_engine_available_on_gfx950(backbone):
    ok, why = backend.engine_available(backbone, torch_mod=fake_torch(), load_library=lambda: None)
    assert ok and "gfx950" in why


def test_engine_available_names_the_missing_piece():
    ok, why = backend.engine_available("pi05", torch_mod=fake_torch(available=False))
    assert not ok and "no GPU" in why
    ok, why = backend.engine_available("pi05", torch_mod=fake_torch(arch="gfx942:sramecc+:xnack-"))
    assert not ok and "gfx942" in why
    ok, why = backend.engine_available("wam", torch_mod=fake_torch(), load_library=lambda: None)
    assert not ok and "no gfx950_fp8 engine" in why

    def missing():
        raise RuntimeError("libifx_fp8.so is not built")
    ok, why = backend.engine_available("pi05", torch_mod=fake_torch(), load_library=missing)
    assert not ok and "libifx_fp8.so" in why


def test_no_triton_or_scaled_mm_needed():
    # The reference gate requires both (engine_backend.py:328-333); this one does not.
    t = fake_torch()
    assert not hasattr(t, "_scaled_mm")
    assert backend.engine_available("groot_n17", torch_mod=t, load_library=lambda: None)[0]


def test_offload_decision():
    d = backend.engine_offload_decision("gfx950:sramecc+:xnack-", "pi05")
    assert d.applies and d.tier == "numeric" and d.params["executor"] == "gfx950_fp8"
    assert d.params["backend"] == "engine"
    assert not backend.engine_offload_decision("gfx942", "pi05").applies
    d = backend.engine_offload_decision("gfx950", "unknown")
    assert not d.applies and "backend" not in d.params


def test_feature_probe_vocabulary():
    f = backend.probe_features(torch_mod=fake_torch())
    assert f == backend.GFX950_FEATURES
    assert not f & {"wgmma", "tma", "triton", "cuda_graphs", "nvfp4"}
    assert backend.probe_features(torch_mod=fake_torch(arch="gfx90a")) == frozenset()


def test_kernel_declarations():
    decl = {k.name: k for k in backend.kernel_declarations()}
    assert decl["ifx_quant_rows"].preserves_intermediate_rounding
    assert not decl["ifx_fp8_linear"].preserves_reduction_order
    assert all(k.requires == {"gfx950_fp8"} for k in decl.values())


# ---------------------------------------------------------------------------
# workload accounting (the per-config FLOP and byte model of the benchmark)
# ---------------------------------------------------------------------------

def test_workload_accounting_matches_published_table():
    from instinctflash_amd.workloads import Gemm, quant_bytes
    C1 = [Gemm("up", 50, 4096, 1024, bias=True)]
    C2 = [Gemm("up", 16, 6144, 1536, act="gelu_tanh"), Gemm("down", 16, 1536, 6144, residual=True)]
    C3 = [Gemm("gu", 816, 32768, 2048, act="geglu"), Gemm("down", 816, 2048, 16384, residual=True)]
    C4 = [Gemm("qkv", 1024, 2560, 2048, bias=True), Gemm("o", 1024, 2048, 2048, residual=True),
          Gemm("gu", 1024, 22016, 2048, act="swiglu"), Gemm("down", 1024, 2048, 11008, residual=True)]
    C5 = [Gemm("qkv", 8192, 9216, 3072), Gemm("o", 8192, 3072, 3072, residual=True, gate=True),
          Gemm("up", 8192, 14336, 3072, act="gelu_tanh"), Gemm("down", 8192, 3072, 14336, residual=True, gate=True)]
    gf = lambda gs, k=1: round(k * sum(g.flops for g in gs) / 1e9, 2)  # noqa: E731
    mb = lambda gs, k=1: round(k * sum(g.bytes for g in gs) / 1e6, 2)  # noqa: E731
    assert (gf(C1), gf(C2, 4), gf(C3), gf(C4), gf(C5)) == (0.42, 2.42, 164.28, 157.84, 2061.58)
    assert abs(mb(C1) - 4.688) < 0.01 and abs(mb(C2, 4) - 77.29) < 0.05
    assert abs(mb(C3) - 149.27) < 0.05 and abs(mb(C4) - 139.34) < 0.05 and abs(mb(C5) - 906.23) < 0.05
    assert abs(4 * (quant_bytes(16, 1536) + quant_bytes(16, 6144)) / 1e6 - 1.475) < 0.002


def test_fp8_linear_module_refuses_cpu_and_non_linear():
    from instinctflash_amd.modules import Gfx950FP8Linear
    lin = torch.nn.Linear(32, 16, dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        Gfx950FP8Linear(torch.nn.Sequential(lin))
    with pytest.raises(ValueError, match="gfx950"):
        Gfx950FP8Linear(lin)  # CPU weights, no gfx950 target


# ---------------------------------------------------------------------------
# row order of linear_qkv_rope's weights (host side, no GPU)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("hd", [16, 64, 128, 256])
def test_rope_row_order_pairs_rotary_partners_per_lane(hd):
    # every head dim appears once, and each 4-row lane group of the skinny
    # GEMM's output fragment holds (d, d + 1, d + hd/2, d + 1 + hd/2)
    from instinctflash_amd.kernels.rope import _rope_row_order
    order = _rope_row_order(hd)
    assert sorted(order) == list(range(hd))
    half = hd // 2
    for p in range(0, hd, 4):
        d = order[p]
        assert d < half and d % 2 == 0
        assert order[p:p + 4] == [d, d + 1, d + half, d + 1 + half]
        # the decoding used by the kernel's epilogue: d = 8 * (p // 16) + 2 * ((p % 16) // 4)
        assert d == 8 * (p // 16) + 2 * ((p % 16) // 4)


def test_permute_rope_rows_on_cpu_tensors():
    import torch
    from instinctflash_amd.kernels.fp8 import Fp8Weight
    from instinctflash_amd.kernels.rope import _rope_row_order, permute_rope_rows
    hq, hkv, hd, K = 2, 1, 32, 16
    N = (hq + 2 * hkv) * hd
    w = torch.arange(N, dtype=torch.float32).repeat(K, 1).t().contiguous().to(torch.float8_e4m3fn)
    scale = torch.arange(N, dtype=torch.float32)
    bias = -torch.arange(N, dtype=torch.float32)
    p = permute_rope_rows(Fp8Weight(w, scale, bias), hq, hkv, hd)
    expect = [h * hd + o for h in range(hq + 2 * hkv) for o in _rope_row_order(hd)]
    assert p.scale.tolist() == [float(i) for i in expect]
    assert p.bias.tolist() == [-float(i) for i in expect]
    assert torch.equal(p.w.view(torch.uint8), w.view(torch.uint8)[expect])
    assert p.rope == (hq, hkv, hd)
    with pytest.raises(ValueError):
        permute_rope_rows(Fp8Weight(w, scale), hq, hkv + 1, hd)


def test_wan_rope_tables_sections_and_ladders():
    # 3-D rotary of the Wan blocks (reference engines/wan_va/weights.py:76-84):
    # 128-dim heads split their 64 channel pairs 22 / 21 / 21 over frame, height
    # and width; each section's ladder starts at 1 and falls by theta^(-2/d)
    from instinctflash_amd.kernels.wan import wan_rope_tables
    inv, sec = wan_rope_tables(128, 10000.0)
    assert inv.dtype == torch.float32 and sec.dtype == torch.int32 and inv.numel() == sec.numel() == 64
    assert [int((sec == s).sum()) for s in range(3)] == [22, 21, 21]
    for s, d in ((0, 44), (1, 42), (2, 42)):
        f = inv[sec == s].double()
        assert f[0] == 1.0
        assert torch.allclose(f[1:] / f[:-1], torch.full_like(f[1:], 10000.0 ** (-2.0 / d)), rtol=1e-6)

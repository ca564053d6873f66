"""Write tests/golden/fp8_golden.npz: input/output vectors of the FP8 recipe.

Run from the repo root:  python tests/golden/make_golden.py

Every vector is computed twice, by the C oracle (oracle/ifx_oracle.c) and by
torch's own CPU implementation of the reference recipe (the formulation of
instinctflash/runtime/torch_fp8_linear.py:39-48 / tests/test_sm89_fp8.py:242-254:
amax.clamp_min(1e-12) * tensor(1/448), (x.float()/scale).clamp(+-448).to(e4m3fn)),
and the script refuses to write unless both agree bit for bit. The reference
itself is not imported: its recipe is plain torch arithmetic, restated here.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent / "fp8_golden.npz"
FIXED_SCALES = (1.0, 1.0 + 2.0 ** -23, 1.0 - 2.0 ** -24, 2.0 ** -16, 1.0 / 448.0)  # qualify_sm89_fp8.py:61


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def torch_quant_rows(x):
    scale = x.float().abs().amax(dim=1).clamp_min(1e-12) * torch.tensor(1.0 / 448.0, dtype=torch.float32)
    q = (x.float() / scale[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).numpy(), scale.numpy()


def all_finite_bf16():
    pat = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    return pat[torch.isfinite(pat)].contiguous()


def rows_case(name, x, out, store_x=True):
    eq, es = oracle.quant_rows(bits(x) if x.dtype == torch.bfloat16 else x.numpy())
    tq, ts = torch_quant_rows(x)
    assert np.array_equal(eq, tq) and np.array_equal(es.view(np.uint32), ts.view(np.uint32)), name
    if store_x:  # the all-pattern inputs are rebuilt by the tests instead
        out[f"{name}_x"] = bits(x) if x.dtype == torch.bfloat16 else x.numpy()
    out[f"{name}_q"] = eq
    out[f"{name}_s"] = es


def main():
    out = {}
    # known answer from the reference's tests (tests/test_sm89_fp8.py:48-56)
    rows_case("kat", torch.full((1, 16), 0.0361328125, dtype=torch.bfloat16), out)
    assert out["kat_s"].view(np.uint32)[0] == 0x38A92493
    # every finite bf16 pattern in one row (tests/test_dynamic_fp8_pack.py:22)
    fin = all_finite_bf16()
    rows_case("allbf16", fin.reshape(1, -1), out, store_x=False)
    # the same patterns as 255 rows of 256 (each row its own scale)
    rows_case("allbf16_rows", fin.reshape(255, 256), out, store_x=False)
    # fixed midpoint scales (scripts/qualify_sm89_fp8.py:58-67)
    for i, s in enumerate(FIXED_SCALES):
        st = torch.tensor([s], dtype=torch.float32)
        tq = (fin.float() / st).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        eq = oracle.pack_fixed(bits(fin), float(st.item()))
        assert np.array_equal(tq, eq), f"fixed scale {s}"
        out[f"fixed{i}_scale"] = st.numpy()
        out[f"fixed{i}_q"] = eq
    # activation rows shaped like the five benchmark configurations (seeded)
    g = torch.Generator().manual_seed(2024)
    for name, K, kind in (("c1", 1024, "outliers"), ("c2", 1536, "normal"), ("c3", 2048, "unit_rms"),
                          ("c4", 2048, "channels"), ("c5", 3072, "modulated"), ("c3h", 16384, "normal"),
                          ("c4h", 11008, "normal"), ("c5h", 14336, "normal")):
        R = 4 if K <= 4096 else 2
        x = torch.randn((R, K), generator=g)
        if kind == "outliers":
            mask = torch.rand((R, K), generator=g) < 0.01
            x = torch.where(mask, torch.randn((R, K), generator=g) * 20, x)
        elif kind == "unit_rms":
            x = x / x.pow(2).mean(dim=1, keepdim=True).sqrt()
        elif kind == "channels":
            x[:, torch.randperm(K, generator=g)[:8]] *= 30
        elif kind == "modulated":
            x = x * (torch.rand(K, generator=g) + 0.5)
        rows_case(f"act_{name}", x.to(torch.bfloat16), out)
    # per-output-channel weight quantization from fp32 (kernels/fp8.py:30-37)
    w = torch.randn((16, 1536), generator=g) * 0.02
    w[3] = 0.0
    rows_case("weight_f32", w, out)
    # a small GEMM with every epilogue, reference = dequantize-then-fp32-matmul
    M, N, K = 8, 64, 256
    qa, sa = oracle.quant_rows(bits(torch.randn((M, K), generator=g).to(torch.bfloat16)))
    qw, sw = oracle.quant_rows((torch.randn((N, K), generator=g) * 0.02).numpy())
    bias = (torch.randn(N, generator=g) * 0.01).numpy()
    res = torch.randn((M, N), generator=g).to(torch.bfloat16)
    gate = torch.rand(N, generator=g).to(torch.bfloat16)
    out.update(gemm_qa=qa, gemm_sa=sa, gemm_qw=qw, gemm_sw=sw, gemm_bias=bias, gemm_res=bits(res),
               gemm_gate=bits(gate))
    out["gemm_plain"] = oracle.ref_linear(qa, sa, qw, sw, bias=bias)
    out["gemm_gelu"] = oracle.ref_linear(qa, sa, qw, sw, bias=bias, act="gelu_tanh")
    out["gemm_geglu"] = oracle.ref_linear(qa, sa, qw, sw, act="geglu")
    out["gemm_swiglu"] = oracle.ref_linear(qa, sa, qw, sw, act="swiglu")
    out["gemm_gated_res"] = oracle.ref_linear(qa, sa, qw, sw, bias=bias, residual=res.float().numpy(),
                                              gate=gate.float().numpy())
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()

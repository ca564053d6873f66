"""The C-ABI library loads and exports exactly what include/ifx_fp8.h declares
(CPU only: no call here reaches the GPU -- only version/status/size queries and
argument checks that return before any launch)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from instinctflash_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "ifx_fp8.h"


def declared():
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(ifx_\w+)\s*\(", text, re.M))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built (run python -m instinctflash_amd.build)")
    return _lib.load()


def test_header_and_binding_agree():
    assert declared() == set(_lib.SIGNATURES), declared() ^ set(_lib.SIGNATURES)


def test_every_declared_symbol_is_exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\s[TW]\s+(ifx_\w+)$", out, re.M))
    assert declared() <= exported, declared() - exported
    for name in declared():
        assert getattr(lib, name)


def test_abi_version_and_status_strings(lib):
    assert lib.ifx_abi_version() == _lib.ABI_VERSION == 3
    for code in (_lib.OK, _lib.ERR_INVALID, _lib.ERR_ALIGN, _lib.ERR_WORKSPACE, _lib.ERR_UNSUPPORTED):
        assert lib.ifx_status_string(code)
    macro = dict(re.findall(r"#define (IFX_(?:ERR_\w+|OK|EPI_\w+|ACT_\w+|DTYPE_\w+|ABI_VERSION))\s+\(?(-?\d+)\)?",
                            HEADER.read_text()))
    assert int(macro["IFX_ERR_INVALID"]) == _lib.ERR_INVALID
    assert int(macro["IFX_EPI_SWIGLU"]) == _lib.EPI_SWIGLU and int(macro["IFX_EPI_RES_F32"]) == _lib.EPI_RES_F32
    assert int(macro["IFX_ACT_SILU"]) == _lib.ACT_SILU and int(macro["IFX_DTYPE_F32"]) == _lib.DTYPE_F32


def test_workspace_queries(lib):
    # enough output tiles (or M <= 64): no split-K, no workspace
    assert lib.ifx_fp8_linear_workspace_size(8192, 3072, 3072, 0) == 0
    assert lib.ifx_fp8_linear_workspace_size(16, 6144, 1536, 0) == 0
    # 816 x 2048 has 32 tiles: fp32 split-K partials, whole M x N slices, no header
    ws = lib.ifx_fp8_linear_workspace_size(816, 2048, 16384, 0)
    assert ws > 0 and ws % (816 * 2048 * 4) == 0
    # skinny (M <= 64) never splits K, whatever K and the row-group count
    assert lib.ifx_fp8_linear_workspace_size(16, 1536, 8192, 0) == 0
    assert lib.ifx_fp8_linear_workspace_size(1, 1024, 16384, 0) == 0
    assert lib.ifx_fp8_linear_workspace_size(16, 1536, 6144, 0) == 0
    # quantize-and-project: the e4m3 copy + scales (+ per-tensor partials) + the GEMM's own
    assert lib.ifx_quant_linear_workspace_size(16, 6144, 1536, 0, _lib.SCALE_ROW) >= 16 * 1536 + 64
    assert (lib.ifx_quant_linear_workspace_size(64, 6144, 1536, 0, _lib.SCALE_TENSOR)
            > lib.ifx_quant_linear_workspace_size(64, 6144, 1536, 0, _lib.SCALE_ROW))
    assert lib.ifx_quant_linear_workspace_size(100, 256, 512, 0, _lib.SCALE_ROW) >= 100 * 512 + 400
    assert (lib.ifx_quant_linear_workspace_size(816, 2048, 16384, 0, _lib.SCALE_ROW)
            >= 816 * 16384 + lib.ifx_fp8_linear_workspace_size(816, 2048, 16384, 0))
    assert lib.ifx_quant_tensor_workspace_size(0) == 0
    assert lib.ifx_quant_tensor_workspace_size(8193) == 8


def test_contract_violations_rejected_before_launch(lib):
    P = ctypes.c_void_p
    fake = P(0x1000)  # never dereferenced: every call below fails its argument check first
    # N % 16 != 0
    assert lib.ifx_fp8_linear(fake, 64, None, fake, 64, None, None, None, 0, None, 0, fake, 64,
                              16, 15, 64, None, 0, None) == _lib.ERR_INVALID
    # GLU with N % 32 != 0
    assert lib.ifx_fp8_linear(fake, 64, None, fake, 64, None, None, None, 0, None, _lib.EPI_GEGLU, fake, 8,
                              16, 48, 64, None, 0, None) == _lib.ERR_INVALID
    # GeGLU and SwiGLU together, unknown flag
    assert lib.ifx_fp8_linear(fake, 64, None, fake, 64, None, None, None, 0, None,
                              _lib.EPI_GEGLU | _lib.EPI_SWIGLU, fake, 32, 16, 64, 64, None, 0, None) == _lib.ERR_INVALID
    assert lib.ifx_fp8_linear(fake, 64, None, fake, 64, None, None, None, 0, None, 1 << 13, fake, 64,
                              16, 64, 64, None, 0, None) == _lib.ERR_INVALID
    # fp16 and fp32 output together
    assert lib.ifx_fp8_linear(fake, 64, None, fake, 64, None, None, None, 0, None,
                              _lib.EPI_OUT_F16 | _lib.EPI_OUT_F32, fake, 64, 16, 64, 64, None, 0, None) == _lib.ERR_INVALID
    # misaligned operand pointer
    assert lib.ifx_fp8_linear(P(0x1001), 64, None, fake, 64, None, None, None, 0, None, 0, fake, 64,
                              16, 64, 64, None, 0, None) == _lib.ERR_ALIGN
    # bias flag without bias, stride shorter than the row
    assert lib.ifx_fp8_linear(fake, 64, None, fake, 64, None, None, None, 0, None, _lib.EPI_BIAS, fake, 64,
                              16, 64, 64, None, 0, None) == _lib.ERR_INVALID
    assert lib.ifx_fp8_linear(fake, 32, None, fake, 64, None, None, None, 0, None, 0, fake, 64,
                              16, 64, 64, None, 0, None) == _lib.ERR_INVALID
    # empty M is a no-op
    assert lib.ifx_fp8_linear(None, 64, None, None, 64, None, None, None, 0, None, 0, None, 64,
                              0, 64, 64, None, 0, None) == _lib.OK
    # quantizers
    assert lib.ifx_quant_rows(fake, 7, 64, 1, 64, fake, 64, fake, None) == _lib.ERR_INVALID
    assert lib.ifx_quant_rows(fake, _lib.DTYPE_BF16, 32, 1, 64, fake, 64, fake, None) == _lib.ERR_INVALID
    assert lib.ifx_quant_rows(None, _lib.DTYPE_BF16, 64, 0, 64, None, 64, None, None) == _lib.OK
    assert lib.ifx_gated_act_quant(fake, 64, 1, 32, None, None, 5, fake, 32, fake, None) == _lib.ERR_INVALID
    assert lib.ifx_quant_tensor_bf16(fake, 100, fake, fake, None, 0, None) == _lib.ERR_WORKSPACE
    assert lib.ifx_fp8_pack_glu(fake, fake, None, 24, 64, fake, fake, None, None) == _lib.ERR_INVALID
    # quantize-and-project: bad scale mode, caller scalar scale, misaligned rows, no workspace
    ql = lambda ldx, mode, epi, M, K, ws=None: lib.ifx_quant_linear(  # noqa: E731
        fake, ldx, mode, fake, 64, fake, None, None, 0, None, epi, fake, 64, M, 64, K, None, ws, 0, None)
    assert ql(64, 2, 0, 16, 64) == _lib.ERR_INVALID
    assert ql(64, _lib.SCALE_ROW, _lib.EPI_SCALAR_SA, 16, 64) == _lib.ERR_INVALID
    assert ql(60, _lib.SCALE_ROW, 0, 16, 48) == _lib.ERR_ALIGN
    assert ql(64, _lib.SCALE_ROW, 0, 100, 64) == _lib.ERR_WORKSPACE
    assert ql(64, _lib.SCALE_ROW, 0, 16, 64) == _lib.ERR_WORKSPACE
    assert ql(64, _lib.SCALE_ROW, 0, 0, 64) == _lib.OK
    # the no-allocation variant runs the same checks before its scratch clear,
    # so a rejected call launches nothing (these return without touching a GPU)
    qn = lambda x, ldx, mode, epi, M, K: lib.ifx_quant_linear_noalloc(  # noqa: E731
        x, ldx, mode, fake, 64, fake, None, None, 0, None, epi, fake, 64, M, 64, K, None, None)
    assert qn(P(0x1001), 64, _lib.SCALE_ROW, 0, 16, 64) == _lib.ERR_ALIGN
    assert qn(fake, 60, _lib.SCALE_ROW, 0, 16, 48) == _lib.ERR_ALIGN
    assert qn(None, 64, _lib.SCALE_ROW, 0, 16, 64) == _lib.ERR_INVALID
    assert qn(fake, 64, 2, 0, 16, 64) == _lib.ERR_INVALID
    assert qn(fake, 64, _lib.SCALE_ROW, 1 << 13, 16, 64) == _lib.ERR_INVALID
    assert qn(fake, 16, _lib.SCALE_TENSOR, 0, 16, 32) == _lib.ERR_INVALID
    assert qn(fake, 128, _lib.SCALE_TENSOR, 0, 16, 64) == _lib.ERR_UNSUPPORTED
    assert lib.ifx_dequant_rows(fake, 0, 64, 1, 64, None, None, None, fake, 9, 64, None) == _lib.ERR_INVALID
    assert lib.ifx_dequant_rows(fake, 7, 64, 1, 64, None, None, None, fake, 0, 64, None) == _lib.ERR_INVALID


def test_loader_rejects_missing_library(tmp_path):
    with pytest.raises(_lib.IfxError, match="not built"):
        _lib.load(tmp_path / "missing.so")

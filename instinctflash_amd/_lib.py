"""ctypes binding of libifx_fp8.so (the C ABI declared in include/ifx_fp8.h).

The loader mirrors the reference's native-library pattern
(instinctflash/backends/sm120_residual.py:25-90): locate the in-tree shared
library, check its ABI version, declare every symbol's signature once. There is
no fallback: if the library is missing or stale the import of a compute entry
point raises, so a GPU run can never silently use another implementation.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

ABI_VERSION = 3
LIB_PATH = Path(os.environ.get("IFX_FP8_LIBRARY", Path(__file__).resolve().parent / "libifx_fp8.so"))

# Status codes (include/ifx_fp8.h)
OK = 0
ERR_INVALID = -1
ERR_ALIGN = -2
ERR_WORKSPACE = -3
ERR_UNSUPPORTED = -4
ERR_SCRATCH = -5

DTYPE_BF16 = 0
DTYPE_F32 = 1
DTYPE_F16 = 2

LD_TILED = 0  # row stride selecting the skinny tile layout of an e4m3 output

RQ_GELU = 1
RQ_F16 = 2
RQ_F32 = 4

ACT_GELU_TANH = 0
ACT_SILU = 1

EPI_NONE = 0
EPI_BIAS = 1
EPI_GELU_TANH = 2
EPI_GEGLU = 4
EPI_SWIGLU = 8
EPI_RESIDUAL = 16
EPI_GATE = 32
EPI_OUT_F32 = 64
EPI_RES_F32 = 128
EPI_SCALAR_SA = 256
EPI_SCALAR_SW = 512
EPI_W_TILED = 1024
EPI_A_TILED = 2048
EPI_OUT_F16 = 4096
RNQ_WRITE_RES = 1
RNQ_LAYERNORM = 2
SCALE_ROW = 0
SCALE_TENSOR = 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); exactly the exports of include/ifx_fp8.h.
SIGNATURES = {
    "ifx_abi_version": (_INT, []),
    "ifx_status_string": (ctypes.c_char_p, [_INT]),
    "ifx_quant_rows": (_INT, [_P, _INT, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "ifx_quant_tensor_workspace_size": (_SZ, [_I64]),
    "ifx_quant_tensor_bf16": (_INT, [_P, _I64, _P, _P, _P, _SZ, _P]),
    "ifx_pack_tensor_bf16": (_INT, [_P, _I64, _P, _P, _P]),
    "ifx_row_quant": (_INT, [_P, _I64, _I64, _I64, _P, _P, _P, _INT, _P, _I64, _P, _P]),
    "ifx_gated_act_quant": (_INT, [_P, _I64, _I64, _I64, _P, _P, _INT, _P, _I64, _P, _P]),
    "ifx_dequant_rows": (_INT, [_P, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _INT, _I64, _P]),
    "ifx_fp8_linear_workspace_size": (_SZ, [_I64, _I64, _I64, _INT]),
    "ifx_quant_linear_workspace_size": (_SZ, [_I64, _I64, _I64, _INT, _INT]),
    "ifx_fp8_skinny_tiled_bytes": (_SZ, [_I64, _I64]),
    "ifx_wan_qkv": (_INT, [_P, _INT, _I64, _P, _P, _P, _P, _P, ctypes.c_float, _P, _P, _I64, _P, _P, _I64, _P, _I64,
                           _I64, _P, _I64, _I64, _P, _INT, _I64, _I64, _I64, _I64, _P]),
    "ifx_qkv_split": (_INT, [_P, _INT, _I64, _P, _P, _P, _P, _P, ctypes.c_float, _P, _P, _I64, _P, _P, _I64, _I64,
                             _P, _I64, _I64, _P, _I64, _I64, _INT, _I64, _P, _I64, _I64, _I64, _I64, _P]),
    "ifx_quant_rows_tiled_bytes": (_SZ, [_I64, _I64]),
    "ifx_quant_rows_tiled": (_INT, [_P, _INT, _I64, _I64, _I64, _P, _P, _P]),
    "ifx_fp8_pack_skinny": (_INT, [_P, _I64, _I64, _I64, _P, _P]),
    "ifx_residual_norm_quant": (_INT, [_P, _INT, _I64, _P, _INT, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _INT,
                                       ctypes.c_float, _P, _I64, _P, _P, _INT, _I64, _P, _P, _P, _I64, _INT,
                                       ctypes.c_float, _I64, _I64, _P]),
    "ifx_attention_workspace_size": (_SZ, [_I64, _I64, _I64, _I64, _I64, _INT]),
    "ifx_attention": (_INT, [_P, _P, _P, _P, _INT, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P, _P,
                             _INT, _I64, _P, _I64, ctypes.c_float, _INT, _P, _SZ, _P, _I64, _P, _P]),
    "ifx_moe_router": (_INT, [_P, _INT, _I64, _I64, _I64, _P, _P, _P, _I64, _INT, ctypes.c_float, _P]),
    "ifx_moe_act_quant": (_INT, [_P, _I64, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "ifx_quant_linear": (_INT, [_P, _I64, _INT, _P, _I64, _P, _P, _P, _I64, _P, _INT, _P, _I64, _I64, _I64, _I64,
                                _P, _P, _SZ, _P]),
    "ifx_quant_linear_noalloc_max_bytes": (_SZ, []),
    "ifx_quant_linear_noalloc": (_INT, [_P, _I64, _INT, _P, _I64, _P, _P, _P, _I64, _P, _INT, _P, _I64, _I64, _I64,
                                        _I64, _P, _P]),
    "ifx_sclk_probe": (_INT, [_P, _I64, _P]),
    "ifx_wall_clock_khz": (_INT, [ctypes.POINTER(_INT)]),
    "ifx_fp8_linear": (_INT, [_P, _I64, _P, _P, _I64, _P, _P, _P, _I64, _P, _INT, _P, _I64, _I64,
                              _I64, _I64, _P, _SZ, _P]),
    "ifx_fp8_pack_glu": (_INT, [_P, _P, _P, _I64, _I64, _P, _P, _P, _P]),
    "ifx_fp8_linear_qkv_rope": (_INT, [_P, _I64, _P, _P, _I64, _P, _P, _INT, _P, _I64, _P, _I64, _I64, _I64,
                                       _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _INT, _I64, _P,
                                       _I64, _I64, _P, _SZ, _P]),
}

_lock = threading.Lock()
_lib = None


class IfxError(RuntimeError):
    """A launch or contract error reported by libifx_fp8.so."""


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is missing or its ABI differs."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise IfxError(f"{p} is not built; run `python -m instinctflash_amd.build` "
                           "(the FP8 path has no non-HIP fallback)")
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.ifx_abi_version()
        if ver != ABI_VERSION:
            raise IfxError(f"{p} has ABI version {ver}, this package expects {ABI_VERSION}; rebuild it")
        if path is None:
            _lib = lib
        return lib


def check(status: int, what: str) -> None:
    if status != OK:
        msg = load().ifx_status_string(status).decode()
        raise IfxError(f"{what} failed: {msg} (status {status})")

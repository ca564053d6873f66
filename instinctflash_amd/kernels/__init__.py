"""HIP (gfx950) kernels of the FP8 projection path.

Mirrors the public surface of the reference package instinctflash/kernels
(fp8.py, norm.py, activation.py, rope.py, wan.py) that the engines import. Importing this
package needs neither a GPU nor the built library; the first compute call
loads libifx_fp8.so and fails loudly if it is absent.
"""
from .attention import SplitWorkspace, attention
from .activation import GELU_TANH, SILU, gated_act_quant, moe_act_quant, moe_router
from .fp8 import (E4M3, FP8_MAX, Fp8Weight, TiledRows, gemm, linear, pack_glu, pack_skinny, pack_tensor,
                  quant_linear, quant_rows, quant_rows_tiled, quantize_tensor, quantize_weight)
from .norm import dequant_rows, residual_norm_quant, row_quant
from .rope import linear_qkv_rope, permute_rope_rows, qkv_split, rope_inv_freq
from .wan import wan_qkv

__all__ = ["E4M3", "FP8_MAX", "Fp8Weight", "quantize_weight", "gemm", "linear", "pack_glu", "pack_skinny", "pack_tensor",
           "quant_linear", "quant_rows", "quant_rows_tiled", "TiledRows", "quantize_tensor", "row_quant", "residual_norm_quant", "dequant_rows", "qkv_split", "rope_inv_freq", "linear_qkv_rope", "permute_rope_rows", "wan_qkv", "gated_act_quant", "attention", "SplitWorkspace", "moe_router", "moe_act_quant", "GELU_TANH", "SILU"]

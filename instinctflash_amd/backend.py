"""gfx950 (MI355X) branch of the reference's FP8 capability gates.

The reference decides whether ``Runtime.from_pretrained(..., precision="fp8")``
may run the FP8 engines at three places, all keyed on CUDA capability tuples
that an MI355X (reported by ROCm torch as capability (9, 5)) never matches:

  * planner: instinctflash/passes/generic/engine_offload.py:33-100
    (``EngineOffloadApplicable.evaluate``; declines every capability it does
    not list, :63-66);
  * runtime: instinctflash/runtime/engine_backend.py:302-333
    (``engine_available``; requires Triton and torch._scaled_mm, :328-333)
    and :458 (``EngineBackend.__init__`` requires (11, 0));
  * device features: instinctflash/passes/contract.py:105,191-197
    (``DeviceProfile.probe`` would label (9, 5) with "wgmma"/"tma").

This module holds the decisions those gates need for a gfx950 device, keyed on
the architecture name (``gcnArchName``), not on a capability tuple, and with the
HIP library as the only requirement (no Triton, no torch._scaled_mm). The
functions take an optional ``torch`` module so the decision logic is testable
on a CPU box with a stand-in module, as the reference's own gate tests do
(tests/test_engine_available_kernels.py:11-16).
"""
from __future__ import annotations

from dataclasses import dataclass, field

EXECUTOR = "gfx950_fp8"
ARCH = "gfx950"

#: Backbones whose engines call the FP8 seam this package implements
#: (reference instinctflash/runtime/engine_backend.py:32).
GI_ENGINE_BACKBONES = ("pi05", "lingbot_vla", "lingbot_vla_v2", "groot_n17", "wan_va")

#: Feature names the gfx950 probe can emit, added to the reference vocabulary
#: (instinctflash/passes/contract.py:105).
GFX950_FEATURES = frozenset({"rocm", "hip_graphs", "fp8", EXECUTOR})


def _torch(torch_mod):
    if torch_mod is not None:
        return torch_mod
    import torch
    return torch


def device_arch(device=None, torch_mod=None) -> str | None:
    """gcnArchName of the device (e.g. 'gfx950:sramecc+:xnack-'), or None off ROCm."""
    t = _torch(torch_mod)
    if not t.cuda.is_available():
        return None
    if isinstance(device, int):
        idx = device
    elif isinstance(device, str):
        idx = int(device.split(":")[1]) if ":" in device else 0
    else:
        idx = 0 if device is None else (getattr(device, "index", None) or 0)
    props = t.cuda.get_device_properties(idx)
    return getattr(props, "gcnArchName", None)


def is_gfx950(device=None, torch_mod=None) -> bool:
    arch = device_arch(device, torch_mod)
    return bool(arch) and arch.split(":")[0] == ARCH


def probe_features(device=None, torch_mod=None) -> frozenset:
    """Features of a gfx950 device in the reference's vocabulary. Never emits
    'wgmma', 'tma', 'triton' or 'cuda_graphs' (NVIDIA-only meanings)."""
    return GFX950_FEATURES if is_gfx950(device, torch_mod) else frozenset()


def engine_available(backbone=None, torch_mod=None, load_library=None) -> "tuple[bool, str]":
    """gfx950 counterpart of instinctflash/runtime/engine_backend.py:302-333:
    (ok, reason), the reason naming the missing piece."""
    try:
        t = _torch(torch_mod)
    except ImportError:
        return False, "no torch in this interpreter"
    if not t.cuda.is_available():
        return False, "no GPU device"
    arch = device_arch(None, t)
    if not arch or arch.split(":")[0] != ARCH:
        return False, f"device is {arch or 'not a ROCm GPU'}; the {EXECUTOR} executor needs {ARCH} (MI355X)"
    if backbone not in GI_ENGINE_BACKBONES:
        return False, f"no {EXECUTOR} engine is registered for backbone {backbone!r}"
    try:
        if load_library is None:
            from . import _lib
            load_library = _lib.load
        load_library()
    except Exception as e:  # noqa: BLE001 - the reason is reported to the caller
        return False, f"the {EXECUTOR} executor needs libifx_fp8.so ({e})"
    return True, f"{ARCH} + {EXECUTOR} HIP kernels (libifx_fp8.so)"


@dataclass
class OffloadDecision:
    """Mirror of the reference PassResult fields the planner reads
    (instinctflash/planners/planner.py PassResult: name, applies, tier, reason, params)."""
    applies: bool
    reason: str
    tier: str = "numeric"
    name: str = "engine_offload"
    params: dict = field(default_factory=dict)


def engine_offload_decision(arch: str | None, backbone: str | None) -> OffloadDecision:
    """gfx950 branch of EngineOffloadApplicable.evaluate
    (instinctflash/passes/generic/engine_offload.py:33-100). An FP8 projection is
    NUMERIC by construction (:82-84): it never claims bit-equality with bf16."""
    if not arch or arch.split(":")[0] != ARCH:
        return OffloadDecision(False, f"device {arch!r} is not {ARCH}: the {EXECUTOR} executor does not apply")
    if backbone not in GI_ENGINE_BACKBONES:
        return OffloadDecision(False, f"No {ARCH} FP8 engine for backbone {backbone!r}")
    return OffloadDecision(
        True, f"{ARCH} FP8 projections (per-token E4M3 activations, per-channel E4M3 weights, fp32 "
              "accumulation, fused bf16 epilogue); task quality requires device qualification",
        params={"backend": "engine", "executor": EXECUTOR, "certification": "uncertified"})


@dataclass(frozen=True)
class KernelDeclaration:
    """The fields the reference's @register_kernel records
    (instinctflash/backends/registry.py:26-55,218-234) for one HIP kernel."""
    name: str
    region: str
    requires: frozenset
    preserves_intermediate_rounding: bool
    preserves_reduction_order: bool
    matches_reference_contraction: bool
    compute_dtype: str
    note: str


def kernel_declarations() -> tuple:
    """Registry entries for this package's kernels. The quantizers are bit-exact
    to the recipe; the GEMM is NUMERIC (matrix-core accumulation order)."""
    req = frozenset({EXECUTOR})
    return (
        KernelDeclaration("ifx_quant_rows", "fp8_row_quant", req, True, True, True, "fp32",
                          "per-row E4M3, scale = max(amax,1e-12)*fl32(1/448), IEEE division"),
        KernelDeclaration("ifx_quant_tensor_bf16", "fp8_tensor_quant", req, True, True, True, "fp32",
                          "per-tensor E4M3, same recipe, NaN-propagating amax"),
        KernelDeclaration("ifx_fp8_linear", "fp8_linear", req, False, False, False, "fp8",
                          "E4M3 x E4M3 MFMA, fp32 accumulation, fused scale/bias/act/gate/residual"),
    )

"""The committed gate patch (integration/gfx950_fp8_gates.patch) against this
package: every instinctflash_amd.backend function the patch calls exists and
answers on a stand-in torch module, and every name the reference engines
import from the kernel seam (instinctflash/engines/*/engine.py and
instinctflash/runtime/*.py import lines, listed here as data) is exported by
the module the patch maps it to."""
import re
import types
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PATCH = ROOT / "integration" / "gfx950_fp8_gates.patch"

# `from instinctflash.kernels.<module> import <names>` in the reference engines and runtime
ENGINE_IMPORTS = {
    "activation": ["GELU_TANH", "SILU", "gated_act_quant", "moe_act_quant"],
    "attention": ["attention"],
    "fp8": ["E4M3", "gemm", "Fp8Weight", "quantize_weight"],
    "norm": ["dequant_rows", "residual_norm_quant", "row_quant"],
    "rope": ["qkv_split", "rope_inv_freq"],
    "wan": ["wan_qkv"],
}


def _added_lines():
    return [l[1:] for l in PATCH.read_text().splitlines() if l.startswith("+") and not l.startswith("+++")]


def test_patch_targets_the_four_gate_files():
    targets = re.findall(r"^\+\+\+ b/(\S+)", PATCH.read_text(), re.M)
    assert targets == ["instinctflash/kernels/__init__.py", "instinctflash/passes/contract.py",
                       "instinctflash/passes/generic/engine_offload.py", "instinctflash/runtime/engine_backend.py"]


def test_patch_calls_existing_backend_functions():
    from instinctflash_amd import backend
    called = set(re.findall(r"gfx950\.(\w+)\(", "\n".join(_added_lines())))
    assert called == {"is_gfx950", "engine_offload_decision", "device_arch", "engine_available", "probe_features"}
    for name in called:
        assert callable(getattr(backend, name)), name


def _fake_torch(arch):
    props = types.SimpleNamespace(gcnArchName=arch, major=9, minor=5, name="AMD Instinct MI355X", total_memory=1)
    cuda = types.SimpleNamespace(is_available=lambda: True, get_device_properties=lambda i: props)
    return types.SimpleNamespace(cuda=cuda)


def test_patched_gates_decide_on_gfx950_stand_in():
    from instinctflash_amd import backend
    t = _fake_torch("gfx950:sramecc+:xnack-")
    for dev in (None, 0, "cuda:0"):
        assert backend.is_gfx950(dev, torch_mod=t)
        assert "wgmma" not in backend.probe_features(dev, torch_mod=t)
    ok, why = backend.engine_available("pi05", torch_mod=t, load_library=lambda: None)
    assert ok, why
    d = backend.engine_offload_decision(backend.device_arch(None, t), "wan_va")
    assert d.applies and d.params["executor"] == backend.EXECUTOR
    assert not backend.is_gfx950(None, torch_mod=_fake_torch("gfx942"))


def test_kernel_seam_modules_export_engine_names():
    import importlib
    mapped = re.search(r'for _name in \(([^)]*)\)', PATCH.read_text()).group(1)
    modules = [m.strip().strip('"') for m in mapped.split(",") if m.strip()]
    assert sorted(modules) == sorted(ENGINE_IMPORTS)
    for mod, names in ENGINE_IMPORTS.items():
        m = importlib.import_module(f"instinctflash_amd.kernels.{mod}")
        missing = [n for n in names if not hasattr(m, n)]
        assert not missing, f"instinctflash_amd.kernels.{mod} lacks {missing}"


REF = Path("/root/reference")
GATE_FILES = ("instinctflash/kernels/__init__.py", "instinctflash/passes/contract.py",
              "instinctflash/passes/generic/engine_offload.py", "instinctflash/runtime/engine_backend.py")


def test_patch_applies_to_the_reference_gate_files(tmp_path):
    # Copies the four gate files out of the reference tree (read only) and
    # dry-runs the patch on the copies, so drift in either side fails here.
    import shutil
    import subprocess

    import pytest
    if not all((REF / f).is_file() for f in GATE_FILES):
        pytest.skip("reference tree not present (only in the build container)")
    for f in GATE_FILES:
        dst = tmp_path / f
        dst.parent.mkdir(parents=True, exist_ok=True)
        shutil.copyfile(REF / f, dst)
    res = subprocess.run(["git", "apply", "--check", "-p1", str(PATCH)], cwd=tmp_path, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    res = subprocess.run(["patch", "--dry-run", "-p1", "-i", str(PATCH)], cwd=tmp_path, capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr

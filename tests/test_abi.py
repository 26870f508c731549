"""The C-ABI library loads and exports every symbol include/t0_gemm.h declares
(no compute calls: these run without a GPU)."""
import os
import re
import subprocess

import pytest

from t0_gpu import _ffi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "t0_gemm.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = set(re.findall(r"\b(t0_[a-z0-9_]+)\s*\(", src))
    return sorted(names)


def test_library_loads():
    L = _ffi.lib()
    assert L.t0_version().decode().startswith("t0-gemm-mi355x")


def test_every_declared_symbol_is_exported():
    out = subprocess.run(["nm", "-D", "--defined-only", _ffi.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\sT\s(t0_[a-z0-9_]+)", out))
    declared = declared_functions()
    assert len(declared) > 60
    missing = [n for n in declared if n not in exported]
    assert not missing, missing


def test_every_declared_symbol_has_ctypes_signature():
    missing = [n for n in declared_functions() if n not in _ffi.SIGNATURES]
    assert not missing, missing


def test_library_embeds_gfx950_code_object():
    import t0_gpu
    ptr, size = t0_gpu.code_object()
    assert size > 100_000
    import ctypes
    head = ctypes.string_at(ptr, 20)
    assert head[:4] == b"\x7fELF"
    # e_machine == EM_AMDGPU (224)
    assert int.from_bytes(head[18:20], "little") == 224


def test_runtime_without_device_fails_loudly():
    import t0_gpu
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is visible")
    except ImportError:
        pass
    with pytest.raises(t0_gpu.T0Error) as e:
        t0_gpu.GpuRuntime(0)
    assert e.value.status == -7   # T0_ERR_NO_DEVICE

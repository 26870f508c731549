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


HSACO = os.path.join(ROOT, "rust-gpu_amd", "build", "t0_kernels.hsaco")
READELF = "/opt/rocm/llvm/bin/llvm-readelf"


def scratch_users(notes: str):
    """(kernel count, [(kernel, field, value)]) from llvm-readelf --notes:
    kernels with VGPR spills or a private (scratch) segment."""
    bad, name, n = [], None, 0
    for line in notes.splitlines():
        m = re.match(r"^    \.name:\s+(\S+)", line)        # kernel level; arguments are deeper
        if m:
            name = m.group(1)
            n += 1
            continue
        m = re.match(r"^    \.(vgpr_spill_count|private_segment_fixed_size):\s+(\d+)", line)
        if m and int(m.group(2)) != 0:
            bad.append((name, m.group(1), int(m.group(2))))
    return n, bad


def test_scratch_parser_flags_a_spill():
    notes = ("  - .args:\n      - .name:           p\n    .name:           k_ok\n"
             "    .private_segment_fixed_size: 0\n    .vgpr_spill_count: 0\n"
             "  - .args:\n      - .name:           p\n    .name:           k_spill\n"
             "    .private_segment_fixed_size: 272\n    .sgpr_spill_count: 5\n    .vgpr_spill_count: 68\n")
    assert scratch_users(notes) == (2, [("k_spill", "private_segment_fixed_size", 272),
                                        ("k_spill", "vgpr_spill_count", 68)])


@pytest.mark.skipif(not (os.path.exists(HSACO) and os.path.exists(READELF)), reason="code object or llvm-readelf absent")
def test_no_kernel_uses_scratch():
    """Every kernel of the gfx950 code object keeps its VGPRs in registers:
    no VGPR spills and no private (scratch) segment. The 8-wave GEMM tiles
    sit at the 256-VGPR budget, where a spill would silently cost most of
    their throughput. SGPR spills go to VGPR lanes and are allowed."""
    notes = subprocess.run([READELF, "--notes", HSACO], capture_output=True, text=True, check=True).stdout
    n, bad = scratch_users(notes)
    assert n > 50, f"only {n} kernels found in the code object metadata"
    assert not bad, bad

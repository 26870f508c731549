"""The Python mirror's ctypes declarations (rust-gpu_amd/t0_gpu/_ffi.py)
against include/t0_gemm.h, on the CPU: every function the header declares
has an entry with as many arguments, each of a ctypes type that passes the
C type unchanged, and the same return type; every ctypes Structure mirrors
its C struct field by field at gcc's offsets and size."""
import ctypes as C

import pytest

from t0_gpu import _ffi
from test_rust_binding import _gcc_facts, parse_header

SCALAR = {"u8": C.c_uint8, "u16": C.c_uint16, "u32": C.c_uint32, "u64": C.c_uint64, "i32": C.c_int32,
          "c_int": C.c_int, "f32": C.c_float, "f64": C.c_double, "usize": C.c_size_t}
STRUCTS = {"t0_gemm_config": _ffi.GemmConfigC, "t0_gemm_geometry": _ffi.GemmGeometryC,
           "t0_tile_gemm": _ffi.TileGemmC, "t0_kernel_load_config": _ffi.KernelLoadConfigC,
           "t0_gemm_desc": _ffi.GemmDescC, "t0_tile_tune_entry": _ffi.TileTuneEntryC,
           "t0_tune_entry": _ffi.TuneEntryC, "t0_gptq_view": _ffi.GptqViewC, "t0_w4a16_desc": _ffi.W4A16DescC,
           "t0_rmsnorm_desc": _ffi.RmsNormDescC}
OPAQUE = {"t0_runtime", "t0_kernel", "t0_buffer", "t0_event", "t0_graph"}


def same_abi(c_type: str, py) -> bool:
    """Whether ctypes type py passes a value of Rust-spelled C type c_type."""
    t = c_type.strip()
    if t in SCALAR:
        return C.sizeof(py) == C.sizeof(SCALAR[t]) and (py in (SCALAR[t],) or
                                                       (t in ("u64", "usize") and py in (C.c_uint64, C.c_size_t)) or
                                                       (t in ("c_int", "i32") and py in (C.c_int, C.c_int32)))
    if not t.startswith("*"):
        return False
    pointee = t.split(" ", 1)[1].strip()
    if py is C.c_void_p:
        return True                       # any pointer
    if py is C.c_char_p:
        return pointee == "c_char"
    if not (isinstance(py, type) and issubclass(py, C._Pointer)):
        return False
    target = py._type_
    if pointee.startswith("*"):           # pointer to pointer
        return target is C.c_void_p or same_abi(pointee, target)
    if pointee.startswith("["):           # pointer to an array: its element
        pointee = pointee[1:].split(";")[0]
    if pointee in OPAQUE:
        return target is C.c_void_p
    if pointee in STRUCTS:
        return target is STRUCTS[pointee]
    return pointee in SCALAR and same_abi(pointee, target)


@pytest.fixture(scope="module")
def header():
    return parse_header()


def test_every_function_has_a_matching_signature(header):
    _, _, funcs, _, _ = header
    assert set(funcs) <= set(_ffi.SIGNATURES), sorted(set(funcs) - set(_ffi.SIGNATURES))
    assert set(_ffi.SIGNATURES) <= set(funcs), sorted(set(_ffi.SIGNATURES) - set(funcs))
    for name, (ret, params) in funcs.items():
        args, res = _ffi.SIGNATURES[name]
        assert len(args) == len(params), (name, len(args), len(params))
        for (pn, pt, alt), py in zip(params, args):
            assert same_abi(pt, py) or (alt is not None and same_abi(alt, py)), (name, pn, pt, py)
        if ret is None:
            assert res is None, name
        else:
            assert same_abi(ret, res), (name, ret, res)


def test_every_structure_matches_gcc(header):
    structs, _, _, _, _ = header
    assert set(STRUCTS) == set(structs), set(structs) ^ set(STRUCTS)
    sizes, offs, _ = _gcc_facts(structs, [])
    for name, py in STRUCTS.items():
        assert [f for f, _ in py._fields_] == [f for f, _ in structs[name]], name
        assert (C.sizeof(py), C.alignment(py)) == sizes[name], name
        for f, _ in structs[name]:
            assert getattr(py, f).offset == offs[(name, f)], (name, f)


def test_the_check_sees_a_wrong_argument_type():
    assert not same_abi("u32", C.c_uint64)
    assert not same_abi("*mut t0_gemm_config", C.POINTER(_ffi.TileGemmC))
    assert same_abi("*mut [u32; 3]", C.POINTER(C.c_uint32))
    assert not same_abi("f32", C.c_double)

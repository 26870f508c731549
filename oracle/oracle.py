"""CPU oracle for the GEMM hot path -- TEST INFRASTRUCTURE ONLY.

This module is the checker, never the thing measured or shipped: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product library (``rust-gpu_amd/``) never
imports, links or calls anything under ``oracle/``.

Arithmetic lives in ``oracle.c`` (built to ``liboracle.so`` by
``oracle/Makefile`` with ``-ffp-contract=off``); this file loads it with
ctypes and adds numpy helpers for byte formats.  Each function names the
reference file:line it restates.  How each function is pinned is listed in
``tests/test_oracle.py``.
"""
from __future__ import annotations

import ctypes
import os
import struct
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    """Compile liboracle.so from oracle.c with the oracle Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_SZ = ctypes.c_size_t


def _declare(L: ctypes.CDLL) -> None:
    L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_bf16_to_f32.restype = ctypes.c_float
    L.orc_bf16_rne.argtypes = [ctypes.c_float]
    L.orc_bf16_rne.restype = ctypes.c_uint16
    L.orc_bf16_trunc.argtypes = [ctypes.c_float]
    L.orc_bf16_trunc.restype = ctypes.c_uint16
    L.orc_bf16_rne_array.argtypes = [_P, _P, _SZ]
    L.orc_bf16_trunc_array.argtypes = [_P, _P, _SZ]
    L.orc_xorshift_bf16.argtypes = [_P, _SZ, ctypes.c_uint64]
    L.orc_gemm_bf16_rows.argtypes = [_P, _SZ, _P, _SZ, _SZ, _P, _SZ, _SZ, _SZ, _SZ, _SZ]
    L.orc_gemm_nt.argtypes = [_P, _P, _P, _SZ, _SZ, _SZ]
    L.orc_gemm_nn.argtypes = [_P, _P, _P, _SZ, _SZ, _SZ]
    L.orc_gemm_f64.argtypes = [_P, _SZ, _P, _SZ, _SZ, _P, _SZ, _SZ, _SZ]
    L.orc_splitk_sum.argtypes = [_P, _P, _SZ, _SZ]
    L.orc_int4_get.argtypes = [_P, _SZ]
    L.orc_int4_get.restype = ctypes.c_uint32
    L.orc_int4_pack.argtypes = [_P, _P, _SZ]
    L.orc_int4_unpack.argtypes = [_P, _P, _SZ]
    L.orc_dequant_int4_f32.argtypes = [_P, _P, _P, _P, _SZ, _SZ, _SZ]
    L.orc_dequant_int4_bf16.argtypes = [_P, _P, _P, _P, _SZ, _SZ, _SZ]
    L.orc_w4a16_rows.argtypes = [_P, _P, _P, _P, ctypes.c_uint32, _P, _SZ, _SZ, _SZ, _SZ, _SZ]
    L.orc_w4a16.argtypes = [_P, _P, _P, _P, ctypes.c_uint32, _P, _SZ, _SZ, _SZ, _SZ]
    L.orc_w4a16_dequant.argtypes = [_P, _P, _P, ctypes.c_uint32, _P, _SZ, _SZ, _SZ]
    L.orc_gemm_bf16_f32w_rows.argtypes = [_P, _P, _P, _SZ, _SZ, _SZ, _SZ]
    L.orc_rmsnorm_rows.argtypes = [_P, _P, _P, _P, _P, _P, _SZ, _SZ, ctypes.c_float]
    L.orc_ffn_fused_rmsnorm_gemm.argtypes = [_P, _P, _P, _P, _P, _SZ, _SZ, ctypes.c_float]


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------- bf16 -----

def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    """Ref: examples/test_gemm_correctness.rs:22-24."""
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 round-to-nearest-even. Ref: examples/test_gemm_correctness.rs:15-20."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_bf16_rne_array(_ptr(x), _ptr(out), x.size)
    return out


def bf16_trunc(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 truncation. Ref: src/t0/tile_ir.rs:4677-4678."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_bf16_trunc_array(_ptr(x), _ptr(out), x.size)
    return out


def xorshift_bf16(n: int, seed: int) -> np.ndarray:
    """The reference's seeded bf16 U(-1,1) generator.
    Ref: examples/test_gemm_correctness.rs:45-58."""
    out = np.empty(n, dtype=np.uint16)
    lib().orc_xorshift_bf16(_ptr(out), n, seed & 0xFFFFFFFFFFFFFFFF)
    return out


# ---------------------------------------------------------------- GEMM -----

def gemm_nt(x: np.ndarray, wt: np.ndarray) -> np.ndarray:
    """Y[M,N] f32 = X[M,K] . WT[N,K]^T, sequential f32, no FMA.
    Ref: examples/test_gemm_correctness.rs:28-42."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    wt = np.ascontiguousarray(wt, dtype=np.uint16)
    m, k = x.shape
    n, k2 = wt.shape
    assert k == k2
    y = np.empty((m, n), dtype=np.float32)
    lib().orc_gemm_nt(_ptr(x), _ptr(wt), _ptr(y), m, k, n)
    return y


def gemm_nn(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Y[M,N] f32 = A[M,K] . B[K,N] with the reference k order."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    y = np.empty((m, n), dtype=np.float32)
    lib().orc_gemm_nn(_ptr(a), _ptr(b), _ptr(y), m, k, n)
    return y


def gemm_rows(a: np.ndarray, b: np.ndarray, layout: str, row0: int, row1: int) -> np.ndarray:
    """Rows [row0,row1) of the reference product (used for the CPU baseline
    on a bounded slice).  layout 'nt' (b = WT[N,K]) or 'nn' (b = B[K,N])."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    m, k = a.shape
    if layout == "nt":
        n = b.shape[0]
        sbk, sbn = 1, k
    else:
        n = b.shape[1]
        sbk, sbn = n, 1
    y = np.zeros((row1 - row0, n), dtype=np.float32)
    # write rows into a view whose row 0 is row0
    base = y.ctypes.data - row0 * n * 4
    lib().orc_gemm_bf16_rows(_ptr(a), k, _ptr(b), sbk, sbn, base, n, row0, row1, n, k)
    return y


def gemm_f64(a: np.ndarray, b: np.ndarray, layout: str) -> np.ndarray:
    """Same products accumulated in double (error reporting only)."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    m, k = a.shape
    if layout == "nt":
        n = b.shape[0]
        sbk, sbn = 1, k
    else:
        n = b.shape[1]
        sbk, sbn = n, 1
    y = np.empty((m, n), dtype=np.float64)
    lib().orc_gemm_f64(_ptr(a), k, _ptr(b), sbk, sbn, _ptr(y), m, n, k)
    return y


def bf16_matmul(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Ignis matmul forward: Y[M,N] = bf16(X[M,K]) . bf16(W[K,N]) in f32.
    Ref: src/ignis/ops/bf16_matmul.rs:162-207 (X converted with RNE at
    :370-373, W converted and transposed at :407-414, NT GEMM).  Zero padding
    of the reference adds exact zeros, so the product is the unpadded one."""
    return gemm_nn(bf16_rne(np.asarray(x, np.float32)), bf16_rne(np.asarray(w, np.float32)))


def bf16_matmul_backward_data(dy: np.ndarray, w: np.ndarray) -> np.ndarray:
    """dX[M,K] = bf16(dY[M,N]) . bf16(W[K,N])^T.
    Ref: src/ignis/ops/bf16_matmul.rs:215-258 (W is the NT operand as stored)."""
    return gemm_nt(bf16_rne(np.asarray(dy, np.float32)), bf16_rne(np.asarray(w, np.float32)))


def bf16_matmul_backward_weight(x: np.ndarray, dy: np.ndarray) -> np.ndarray:
    """dW[K,N] = bf16(X[M,K])^T . bf16(dY[M,N]).
    Ref: src/ignis/ops/bf16_matmul.rs:265-308 (X^T and dY^T built by the CPU
    transpose-convert :389-423, then NT GEMM over the contraction M)."""
    xt = bf16_rne(np.ascontiguousarray(np.asarray(x, np.float32).T))
    return gemm_nn(xt, bf16_rne(np.asarray(dy, np.float32)))


def splitk_sum(planes: np.ndarray) -> np.ndarray:
    """Host split-K plane sum. Ref: examples/hello_gemm_gen.rs:125-136."""
    planes = np.ascontiguousarray(planes, dtype=np.float32)
    sk = planes.shape[0]
    mn = planes[0].size
    y = np.empty(planes.shape[1:], dtype=np.float32)
    lib().orc_splitk_sum(_ptr(planes), _ptr(y), mn, sk)
    return y


# ---------------------------------------------------------------- INT4 -----

def int4_pack(q: np.ndarray) -> np.ndarray:
    """Two nibbles per byte, low nibble = even element.
    Ref: src/t0/quant_kernels.rs:3-10, :381-389."""
    q = np.ascontiguousarray(q, dtype=np.uint8).reshape(-1)
    assert q.size % 2 == 0
    out = np.empty(q.size // 2, dtype=np.uint8)
    lib().orc_int4_pack(_ptr(q), _ptr(out), q.size)
    return out


def int4_unpack(packed: np.ndarray, n: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1)
    out = np.empty(n, dtype=np.uint8)
    lib().orc_int4_unpack(_ptr(packed), _ptr(out), n)
    return out


def dequant_int4_f32(packed, scales, zp, rows, cols, group_size) -> np.ndarray:
    """(q - zp) * scale per [row][group]. Ref: src/t0/quant_kernels.rs:37-40, :365-372."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    zp = np.ascontiguousarray(zp, dtype=np.int32)
    out = np.empty(rows * cols, dtype=np.float32)
    lib().orc_dequant_int4_f32(_ptr(packed), _ptr(scales), _ptr(zp), _ptr(out), rows, cols, group_size)
    return out.reshape(rows, cols)


def dequant_int4_bf16(packed, scales, zp, rows, cols, group_size) -> np.ndarray:
    """bf16 output via truncation (store_bf16). Ref: src/t0/quant_kernels.rs:109-127."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    zp = np.ascontiguousarray(zp, dtype=np.int32)
    out = np.empty(rows * cols, dtype=np.uint16)
    lib().orc_dequant_int4_bf16(_ptr(packed), _ptr(scales), _ptr(zp), _ptr(out), rows, cols, group_size)
    return out.reshape(rows, cols)


def w4a16(a, qw, scales, zeros, zc, m, n, k, gs, row0=0, row1=None) -> np.ndarray:
    """W4A16 reference: exact dequant (q - z) * s then the reference f32 loop.
    Ref: src/t0/quant_kernels.rs:365-372 + examples/test_gemm_correctness.rs:28-42."""
    if row1 is None:
        row1 = m
    a = np.ascontiguousarray(a, dtype=np.uint16)
    qw = np.ascontiguousarray(qw, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    if zeros is not None:
        zeros = np.ascontiguousarray(zeros, dtype=np.uint32)
    y = np.zeros((row1 - row0, n), dtype=np.float32)
    base = y.ctypes.data - row0 * n * 4
    lib().orc_w4a16_rows(_ptr(a), _ptr(qw), _ptr(scales), _ptr(zeros), zc, base, row0, row1, n, k, gs)
    return y


def gemm_bf16_f32w_rows(a: np.ndarray, w: np.ndarray, row0: int, row1: int) -> np.ndarray:
    """Rows [row0, row1) of the reference loop on bf16 a [M][K] and f32 w [N][K]
    (dequantized weights).  Ref: examples/test_gemm_correctness.rs:28-42."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    y = np.zeros((row1 - row0, n), dtype=np.float32)
    base = y.ctypes.data - row0 * n * 4
    lib().orc_gemm_bf16_f32w_rows(_ptr(a), _ptr(w), base, row0, row1, n, k)
    return y


def w4a16_dequant(qw, scales, zeros, zc, n, k, gs) -> np.ndarray:
    qw = np.ascontiguousarray(qw, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.uint16)
    if zeros is not None:
        zeros = np.ascontiguousarray(zeros, dtype=np.uint32)
    w = np.empty((n, k), dtype=np.float32)
    lib().orc_w4a16_dequant(_ptr(qw), _ptr(scales), _ptr(zeros), zc, _ptr(w), n, k, gs)
    return w


# --------------------------------------------------------- GPTQ format -----

def gptq_to_bytes(rows, cols, group_size, packed, scales, zero_points) -> bytes:
    """Serialize in the reference GptqWeight byte format:
    [rows u32][cols u32][group_size u32][packed][scales f32 LE][zero_points i32 LE].
    Ref: src/t0/quant_kernels.rs:249-258."""
    return (struct.pack("<III", rows, cols, group_size)
            + np.asarray(packed, dtype=np.uint8).tobytes()
            + np.asarray(scales, dtype="<f4").tobytes()
            + np.asarray(zero_points, dtype="<i4").tobytes())


def gptq_from_bytes(raw: bytes):
    """Parse the reference GptqWeight byte format.
    Ref: src/t0/quant_kernels.rs:259-287 (asserts on short/truncated data)."""
    if len(raw) < 12:
        raise ValueError("GPTQ data too short (need at least 12 bytes header)")
    rows, cols, gs = struct.unpack_from("<III", raw, 0)
    n_groups = cols // gs
    n_params = n_groups * rows
    packed_len = rows * cols // 2
    total = 12 + packed_len + n_params * 8
    if len(raw) < total:
        raise ValueError(f"GPTQ data truncated: need {total} bytes, got {len(raw)}")
    packed = np.frombuffer(raw, dtype=np.uint8, count=packed_len, offset=12)
    scales = np.frombuffer(raw, dtype="<f4", count=n_params, offset=12 + packed_len)
    zps = np.frombuffer(raw, dtype="<i4", count=n_params, offset=12 + packed_len + 4 * n_params)
    return rows, cols, gs, n_groups, packed, scales, zps


# ------------------------------------------------------- decode neighbours --

def rmsnorm_rows(res: np.ndarray, hid: np.ndarray | None, gamma: np.ndarray, eps: float):
    """(normed, x2, inv_rms) of residual add + RMSNorm, f32 in order.
    Ref: src/t0/rmsnorm_kernels.rs:140-153 on src/t0/ffn_fused_kernels.rs:215-224."""
    res = np.ascontiguousarray(res, dtype=np.float32)
    m, d = res.shape
    h = None if hid is None else np.ascontiguousarray(hid, dtype=np.float32)
    g = np.ascontiguousarray(gamma, dtype=np.float32).reshape(d)
    normed = np.empty((m, d), np.float32)
    x2 = np.empty((m, d), np.float32)
    inv = np.empty(m, np.float32)
    lib().orc_rmsnorm_rows(_ptr(res), _ptr(h), _ptr(g), _ptr(normed), _ptr(x2), _ptr(inv), m, d, eps)
    return normed, x2, inv


def ffn_fused_rmsnorm_gemm(res, hid, gamma, weight, eps: float) -> np.ndarray:
    """out[row] = sum_i (x2[row,i] * inv_rms * gamma[i]) * weight[row,i].
    Ref: src/t0/ffn_fused_kernels.rs:203-237."""
    res = np.ascontiguousarray(res, dtype=np.float32)
    m, d = res.shape
    hid = np.ascontiguousarray(hid, dtype=np.float32)
    g = np.ascontiguousarray(gamma, dtype=np.float32).reshape(d)
    w = np.ascontiguousarray(weight, dtype=np.float32).reshape(m, d)
    out = np.empty(m, np.float32)
    lib().orc_ffn_fused_rmsnorm_gemm(_ptr(res), _ptr(hid), _ptr(g), _ptr(w), _ptr(out), m, d, eps)
    return out

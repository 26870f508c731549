"""Mirror of the decode neighbours of the GEMM path: residual add + RMSNorm in
front of a projection (src/t0/ffn_fused_kernels.rs,
src/ignis/ops/fused_rmsnorm_gemm.rs, src/t0/rmsnorm_kernels.rs:140-153).

  x2      = residual (+ hidden)
  inv_rms = 1 / sqrt(mean(x2^2) + eps)
  normed  = x2 * inv_rms * gamma

  ffn_fused_rmsnorm_gemm        out[r] = normed[r] . weight[r]     ffn_fused_kernels.rs:54-237
  rmsnorm                       normed (bf16 or f32), x2           rmsnorm_kernels.rs:140-153
  fused_rmsnorm_gemm            normed @ W, dense f32 W[k, n]      fused_rmsnorm_gemm.rs:33-63
  fused_residual_rmsnorm_gemm   the same with the residual add     fused_rmsnorm_gemm.rs:120-154
  fused_rmsnorm_w4a16           normed @ W^T, INT4 W (W4A16)       the decode kernel with the norm fused in

Buffers are ``GpuBuffer`` objects with dense row-major f32 data (the INT4
operand as in ``GpuRuntime.w4a16``); every call runs GPU kernels of the
library.
"""
from __future__ import annotations

import ctypes as C

from . import GpuBuffer, GpuRuntime, _check, lib
from ._ffi import RmsNormDescC, W4A16DescC


def _addr(b) -> int:
    return 0 if b is None else (b if isinstance(b, int) else b.gpu_addr())


def _need(buf, nbytes: int, what: str):
    if buf is not None and not isinstance(buf, int) and buf.size() < nbytes:
        raise ValueError(f"{what}: buffer holds {buf.size()} bytes, needs {nbytes}")


def ffn_fused_rmsnorm_gemm(rt: GpuRuntime, residual: GpuBuffer, hidden: GpuBuffer, gamma: GpuBuffer,
                           weight: GpuBuffer, m: int, d: int, eps: float) -> GpuBuffer:
    """The reference kernel: out[r] = sum_i normed[r, i] * weight[r*d + i], r < m."""
    if m <= 0 or d <= 0:
        raise ValueError(f"ffn_fused_rmsnorm_gemm: empty shape m={m} d={d}")
    for b, n, w in ((residual, m * d, "residual"), (hidden, m * d, "hidden"), (gamma, d, "gamma"),
                    (weight, m * d, "weight")):
        _need(b, 4 * n, w)
    out = rt.alloc(4 * m)
    _check(lib().t0_ffn_fused_rmsnorm_gemm(rt.h, _addr(residual), _addr(hidden), _addr(gamma), _addr(weight),
                                           out.gpu_addr(), m, d, eps))
    return out


def rmsnorm(rt: GpuRuntime, residual: GpuBuffer, gamma: GpuBuffer, rows: int, d: int, eps: float,
            hidden: GpuBuffer | None = None, out_bf16: bool = False, x2_out: GpuBuffer | None = None) -> GpuBuffer:
    """normed[rows, d] (bf16 RNE or f32) of residual (+ hidden); x2 into x2_out."""
    if rows <= 0 or d <= 0:
        raise ValueError(f"rmsnorm: empty shape rows={rows} d={d}")
    _need(residual, 4 * rows * d, "residual")
    _need(hidden, 4 * rows * d, "hidden")
    _need(gamma, 4 * d, "gamma")
    _need(x2_out, 4 * rows * d, "x2_out")
    out = rt.alloc((2 if out_bf16 else 4) * rows * d)
    _check(lib().t0_rmsnorm(rt.h, _addr(residual), _addr(hidden), _addr(gamma), out.gpu_addr(), _addr(x2_out),
                            rows, d, d, eps, int(out_bf16)))
    return out


def fused_residual_rmsnorm_gemm(rt: GpuRuntime, residual: GpuBuffer, hidden: GpuBuffer | None, gamma: GpuBuffer,
                                weight: GpuBuffer, x_shape, w_shape, eps: float,
                                x2_out: GpuBuffer | None = None) -> GpuBuffer:
    """Y[m, n] = bf16(normed) @ bf16(W), f32 out; W is f32 [k, n]."""
    if len(x_shape) != 2 or len(w_shape) != 2:
        raise ValueError("fused_rmsnorm_gemm: x and weight must be 2D")
    m, k = x_shape
    if w_shape[0] != k:
        raise ValueError(f"weight dim mismatch: x[{m},{k}] @ W[{w_shape[0]},{w_shape[1]}]")
    n = w_shape[1]
    _need(residual, 4 * m * k, "residual")
    _need(hidden, 4 * m * k, "hidden")
    _need(gamma, 4 * k, "gamma")
    _need(weight, 4 * k * n, "weight")
    y = rt.alloc(4 * m * n)
    _check(lib().t0_rmsnorm_matmul(rt.h, _addr(residual), _addr(hidden), _addr(gamma), _addr(weight), y.gpu_addr(),
                                   _addr(x2_out), m, k, n, eps))
    return y


def fused_rmsnorm_gemm(rt: GpuRuntime, x: GpuBuffer, gamma: GpuBuffer, weight: GpuBuffer, x_shape, w_shape,
                       eps: float) -> GpuBuffer:
    """RMSNorm(x) @ W without a residual add."""
    return fused_residual_rmsnorm_gemm(rt, x, None, gamma, weight, x_shape, w_shape, eps)


def fused_rmsnorm_w4a16(rt: GpuRuntime, residual: GpuBuffer, gamma: GpuBuffer, qweight: GpuBuffer,
                        scales: GpuBuffer, zeros: GpuBuffer | None, m: int, n: int, k: int, eps: float,
                        hidden: GpuBuffer | None = None, x2_out: GpuBuffer | None = None, group_size: int = 128,
                        zero_const: int = 8, scales_f32: bool = False, out_f32: bool = False) -> GpuBuffer:
    """C[m, n] = normed @ W^T with the INT4 operand of GpuRuntime.w4a16; for
    m == 1 one decode kernel does the residual add, the norm and the GEMV."""
    _need(residual, 4 * m * k, "residual")
    _need(hidden, 4 * m * k, "hidden")
    _need(gamma, 4 * k, "gamma")
    c = rt.alloc((4 if out_f32 else 2) * m * n)
    d = W4A16DescC(a=0, qweight=_addr(qweight), scales=_addr(scales), zeros=_addr(zeros), c=c.gpu_addr(), m=m, n=n,
                   k=k, lda=0, ldc=0, group_size=group_size, zero_const=zero_const, scales_f32=int(scales_f32),
                   out_f32=int(out_f32), split_k=0)
    nd = RmsNormDescC(residual=_addr(residual), hidden=_addr(hidden), gamma=_addr(gamma), x2_out=_addr(x2_out),
                      eps=eps)
    _check(lib().t0_rmsnorm_w4a16(rt.h, C.byref(d), C.byref(nd)))
    return c

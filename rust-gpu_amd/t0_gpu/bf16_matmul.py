"""Mirror of the Ignis bf16 matmul operator (src/ignis/ops/bf16_matmul.rs).

The reference computes Y = X @ W for f32 tensors by rounding both operands to
bf16 on the CPU, transposing W on the CPU, padding every dimension to the
tile and running the gemm_gen kernel into a padded f32 output that is then
unpadded.  Here the same four calls go through the C ABI, which converts,
pads (to 8 elements) and, where needed, transposes on the GPU and writes the
dense f32 result directly:

  matmul                 Y[m,n]  = X[m,k] @ W[k,n]        bf16_matmul.rs:33-98, 162-207
  gemm_backward_data     dX[m,k] = dY[m,n] @ W[k,n]^T     bf16_matmul.rs:215-258
  gemm_backward_weight   dW[k,n] = X[m,k]^T @ dY[m,n]     bf16_matmul.rs:265-308
  matmul_with_wt_bf16    Y[m,n]  = X[m,k] @ WT[n,k]^T     bf16_matmul.rs:102-134

``matmul_backward`` is the closure the reference records on its tape
(bf16_matmul.rs:72-92): dX when X needs a gradient, dW when W does.

Buffers are ``GpuBuffer`` objects holding dense row-major data (f32, except
the bf16 ``wt_bf16``); shape mismatches raise ``ValueError`` where the
reference asserts.
"""
from __future__ import annotations

from . import GpuBuffer, GpuRuntime, _check, lib


def _need(buf: GpuBuffer, nbytes: int, what: str):
    if buf.size() < nbytes:
        raise ValueError(f"{what}: buffer holds {buf.size()} bytes, needs {nbytes}")


def _dims(m: int, k: int, n: int):
    if min(m, k, n) <= 0:
        raise ValueError(f"matmul: empty shape m={m} k={k} n={n}")


def matmul(rt: GpuRuntime, x: GpuBuffer, w: GpuBuffer, x_shape, w_shape) -> GpuBuffer:
    """Y = X @ W; x_shape (m, k), w_shape (k, n) as the reference's tensor
    shapes (bf16_matmul.rs:34-42).  Returns a new f32 [m, n] buffer."""
    if len(x_shape) != 2 or len(w_shape) != 2:
        raise ValueError(f"matmul: X and W must be 2D, got {tuple(x_shape)} and {tuple(w_shape)}")
    m, k = x_shape
    k2, n = w_shape
    if k2 != k:
        raise ValueError(f"matmul: K mismatch X[{m},{k}] @ W[{k2},{n}]")
    _dims(m, k, n)
    _need(x, m * k * 4, "matmul X")
    _need(w, k * n * 4, "matmul W")
    y = rt.alloc(m * n * 4)
    _check(lib().t0_bf16_matmul(rt.h, x.gpu_addr(), w.gpu_addr(), y.gpu_addr(), m, k, n))
    return y


def gemm_backward_data(rt: GpuRuntime, grad_y: GpuBuffer, w: GpuBuffer, m: int, k: int, n: int) -> GpuBuffer:
    """dX[m,k] = dY[m,n] @ W[k,n]^T (f32 in, f32 out)."""
    _dims(m, k, n)
    _need(grad_y, m * n * 4, "backward_data dY")
    _need(w, k * n * 4, "backward_data W")
    dx = rt.alloc(m * k * 4)
    _check(lib().t0_bf16_matmul_backward_data(rt.h, grad_y.gpu_addr(), w.gpu_addr(), dx.gpu_addr(), m, k, n))
    return dx


def gemm_backward_weight(rt: GpuRuntime, x: GpuBuffer, grad_y: GpuBuffer, m: int, k: int, n: int) -> GpuBuffer:
    """dW[k,n] = X[m,k]^T @ dY[m,n] (f32 in, f32 out)."""
    _dims(m, k, n)
    _need(x, m * k * 4, "backward_weight X")
    _need(grad_y, m * n * 4, "backward_weight dY")
    dw = rt.alloc(k * n * 4)
    _check(lib().t0_bf16_matmul_backward_weight(rt.h, x.gpu_addr(), grad_y.gpu_addr(), dw.gpu_addr(), m, k, n))
    return dw


def matmul_backward(rt: GpuRuntime, grad_y: GpuBuffer, x: GpuBuffer, w: GpuBuffer, m: int, k: int, n: int,
                    x_needs: bool = True, w_needs: bool = True):
    """The recorded backward of ``matmul``: (dX or None, dW or None)."""
    dx = gemm_backward_data(rt, grad_y, w, m, k, n) if x_needs else None
    dw = gemm_backward_weight(rt, x, grad_y, m, k, n) if w_needs else None
    return dx, dw


def matmul_with_wt_bf16(rt: GpuRuntime, x: GpuBuffer, wt_bf16: GpuBuffer, m: int, k: int, n: int) -> GpuBuffer:
    """Y[m,n] = X[m,k] @ WT[n,k]^T with a pre-transposed bf16 weight."""
    _dims(m, k, n)
    _need(x, m * k * 4, "matmul_with_wt_bf16 X")
    _need(wt_bf16, n * k * 2, "matmul_with_wt_bf16 WT")
    y = rt.alloc(m * n * 4)
    _check(lib().t0_bf16_matmul_with_wt_bf16(rt.h, x.gpu_addr(), wt_bf16.gpu_addr(), y.gpu_addr(), m, k, n))
    return y

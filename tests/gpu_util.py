"""Helpers for the GPU parity tests: data generation through the oracle's
bf16 rounding, device round trips, BASELINE's acceptance tolerance
max|err| <= 1e-2 * sqrt(K) * max|a| * max|b|, and the tight per-element bound
of parity.tight_bound (f32 summation in any order, plus half a bf16 ulp for
bf16 output) with the relative Frobenius error."""
import numpy as np

import t0_gpu as t0
from oracle import oracle as orc


def bf16(x) -> np.ndarray:
    return orc.bf16_rne(np.asarray(x, dtype=np.float32))


def f32(h) -> np.ndarray:
    return orc.bf16_to_f32(h)


def tolerance(a_vals: np.ndarray, b_vals: np.ndarray, k: int) -> float:
    return 1e-2 * np.sqrt(k) * float(np.abs(a_vals).max()) * float(np.abs(b_vals).max()) + 1e-30


def check_tight(got: np.ndarray, ref: np.ndarray, a_vals: np.ndarray, b_vals: np.ndarray, out_bf16: bool,
                what: str = "", layout: str = "nn"):
    """Per-element tight bound (parity.tight_bound) and, for bf16 output,
    relative Frobenius error <= 2^-8; returns (max|err|, rel frob)."""
    from oracle.parity import tight_bound, rel_frobenius
    bound = tight_bound(ref, a_vals, b_vals, out_bf16, layout)
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    frob = rel_frobenius(got, ref)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} outputs over the tight bound, worst excess "
                           f"{float((err - bound).max()):.3e} (max|err| {float(err.max()):.3e}, rel frob {frob:.3e})")
    if out_bf16:
        assert frob <= 2.0 ** -8, f"{what}: rel frob {frob:.3e} > 2^-8"
    return float(err.max()), frob


def check_close(got: np.ndarray, ref: np.ndarray, tol: float, what: str = ""):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    max_err = float(err.max()) if err.size else 0.0
    frob = float(np.linalg.norm(got.astype(np.float64) - ref) / (np.linalg.norm(ref) + 1e-30))
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert max_err <= tol, f"{what}: max|err| {max_err:.3e} > tol {tol:.3e} (rel frob {frob:.3e})"
    return max_err, frob


class Dev:
    """Upload / download through the library's own buffers."""

    def __init__(self, rt: t0.GpuRuntime):
        self.rt = rt
        self.bufs = []

    def up(self, arr) -> int:
        b = self.rt.upload(np.ascontiguousarray(arr))
        self.bufs.append(b)
        return b.gpu_addr()

    def zeros(self, nbytes: int) -> int:
        b = self.rt.alloc(nbytes)
        b.zero()
        self.bufs.append(b)
        return b.gpu_addr()

    def fill(self, arr) -> int:
        return self.up(arr)

    def down(self, addr: int, dtype, count: int) -> np.ndarray:
        self.rt.wait_idle()
        for b in self.bufs:
            if b.gpu_addr() == addr:
                return b.read(dtype, count)
        raise KeyError(addr)

    def free(self):
        for b in self.bufs:
            b.free()
        self.bufs = []

"""Tight parity bounds for the bf16 GEMM and W4A16 paths (test
infrastructure, like the rest of oracle/): used by the GPU parity tests, by
the CPU test that shows they reject what BASELINE's loose bound accepts, and
by bench.py's CPU-baseline leg to report each config's error against the
oracle.

Both the GPU kernels and the CPU oracle sum K products of bf16 values in f32
(the products are exact in f32), in different orders.  Each sum is within
gamma_K * sum_k |a_k b_k| of the exact value, gamma_K = K u / (1 - K u) with
u = 2^-24, so the two differ by at most twice that.  A bf16 output adds the
rounding of the GPU's f32 result: at most half a bf16 ulp (2^-8 relative to
the binade) of the rounded value.  So per element

    |got - ref| <= 2 gamma_K (|A| |B|)_ij  [+ ulp_bf16(max(|got|,|ref|)) / 2]

and, for bf16 output, the relative Frobenius error stays below 2^-8 plus
the accumulation term (asserted as <= 2^-8 on the headline shapes, where
the rounding dominates)."""
import numpy as np

U32 = 2.0 ** -24


def gamma(k: int) -> float:
    return k * U32 / (1.0 - k * U32)


def bf16_half_ulp(x: np.ndarray) -> np.ndarray:
    """Half the bf16 spacing at |x| (8 significant bits): 2^(e - 8) for
    2^e <= |x| < 2^(e+1); the smallest normal spacing below 2^-126."""
    ax = np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -126)
    e = np.floor(np.log2(ax))
    return np.ldexp(1.0, (e - 8).astype(np.int64))


def abs_product(a_vals: np.ndarray, b_vals: np.ndarray, layout: str = "nn") -> np.ndarray:
    """(|A| |B|)_ij in float64; layout 'nt' takes b as WT [N][K]."""
    a = np.abs(np.asarray(a_vals, np.float64))
    b = np.abs(np.asarray(b_vals, np.float64))
    return a @ (b.T if layout == "nt" else b)


def tight_bound(ref: np.ndarray, a_vals: np.ndarray, b_vals: np.ndarray, out_bf16: bool,
                layout: str = "nn") -> np.ndarray:
    k = np.asarray(a_vals).shape[1]
    bound = 2.0 * gamma(k) * abs_product(a_vals, b_vals, layout)
    if out_bf16:
        # rounding of the GPU's f32 value, which is within the first term of ref
        bound = bound + bf16_half_ulp(np.abs(np.asarray(ref, np.float64)) + bound)
    return bound


def rel_frobenius(got: np.ndarray, ref: np.ndarray) -> float:
    d = np.asarray(got, np.float64) - np.asarray(ref, np.float64)
    return float(np.linalg.norm(d) / (np.linalg.norm(np.asarray(ref, np.float64)) + 1e-300))


def w4_tight_bound(ref: np.ndarray, a_vals: np.ndarray, q: np.ndarray, s: np.ndarray, z: np.ndarray, gs: int,
                   out_bf16: bool) -> np.ndarray:
    """Per-element bound for the fused W4A16 GEMM against the oracle's exact
    dequant + f32 loop.  The kernels sum, per quant group g of gs k values,
    T_g = sum a_k (128 + q_k) and the zero-point term (128 + z_g) * sum a_k in
    one f32 accumulation (at most gs + 16 terms in the prefill's extra MFMA
    block), scale by s_g in f32, and add the G group results in f32 in some
    order.  So |got - exact| <= gamma_{gs+32} * sum_k |a_k| s_g (256 + q_k + z_g)
    + gamma_{G+1} * (|A||W|), and the oracle adds gamma_K * (|A||W|).
    q: [N][K] nibbles, s: [G][N] f32 scales, z: [G][N] zero points."""
    a = np.abs(np.asarray(a_vals, np.float64))
    k = a.shape[1]
    G = k // gs
    sk = np.repeat(np.asarray(s, np.float64).T, gs, axis=1)           # [N][K]
    zk = np.repeat(np.asarray(z, np.float64).T, gs, axis=1)
    qf = np.asarray(q, np.float64)
    mag = a @ (sk * (256.0 + qf + zk)).T
    w = np.abs(sk * (qf - zk))
    bound = gamma(gs + 32) * mag + (gamma(G + 1) + gamma(k)) * (a @ w.T)
    if out_bf16:
        bound = bound + bf16_half_ulp(np.abs(np.asarray(ref, np.float64)) + bound)
    return bound

"""CPU-only checks of the tight parity bounds (tests/parity.py): a result
with one 16-k MFMA sub-step (GEMM) or one 128-k quant group (W4A16) left
out passes BASELINE's loose bound 1e-2 * sqrt(K) * max|a| * max|b| but fails
the tight one, while the oracle's own f32 result and its bf16 rounding pass."""
import numpy as np
import pytest

from oracle import oracle as orc
from oracle.parity import gamma, bf16_half_ulp, rel_frobenius, tight_bound, w4_tight_bound


def loose(a, b, k):
    return 1e-2 * np.sqrt(k) * float(np.abs(a).max()) * float(np.abs(b).max())


def test_bf16_half_ulp_known_values():
    assert bf16_half_ulp(np.array([1.0]))[0] == 2.0 ** -8
    assert bf16_half_ulp(np.array([1.99]))[0] == 2.0 ** -8
    assert bf16_half_ulp(np.array([-64.0]))[0] == 2.0 ** -2
    assert bf16_half_ulp(np.array([0.75]))[0] == 2.0 ** -9
    # every bf16 value rounded from an f32 is within half an ulp of it
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 50
    r = orc.bf16_to_f32(orc.bf16_rne(x)).astype(np.float64)
    assert np.all(np.abs(r - x) <= bf16_half_ulp(x))


def test_gamma_matches_definition():
    assert gamma(1) == pytest.approx(2.0 ** -24, rel=1e-6)
    assert gamma(4096) == pytest.approx(4096 * 2.0 ** -24 / (1 - 4096 * 2.0 ** -24))


@pytest.mark.parametrize("out_bf16", [False, True])
def test_gemm_dropped_substep_rejected(out_bf16):
    """The headline's data (4096 x 4096 N(0,1) operands rounded to bf16; the
    loose bound takes max|a| and max|b| over the whole operands, as the
    full-size GPU test does), checked on 16 rows x 256 columns: the exact
    result passes both bounds; the same result with k in [1600, 1616) left
    out passes the loose bound and fails the tight one."""
    rng = np.random.default_rng(5)
    K = 4096
    a_full = orc.bf16_rne(rng.standard_normal((K, K)).astype(np.float32))
    b_full = orc.bf16_rne(rng.standard_normal((K, K)).astype(np.float32))
    tol = loose(orc.bf16_to_f32(a_full), orc.bf16_to_f32(b_full), K)
    a, b = a_full[:16].copy(), b_full[:, :256].copy()
    af, bf = orc.bf16_to_f32(a), orc.bf16_to_f32(b)
    ref = orc.gemm_nn(a, b)
    exact = af.astype(np.float64) @ bf.astype(np.float64)
    good = exact.astype(np.float32)
    dropped = (exact - af[:, 1600:1616].astype(np.float64) @ bf[1600:1616].astype(np.float64)).astype(np.float32)
    if out_bf16:
        good = orc.bf16_to_f32(orc.bf16_rne(good))
        dropped = orc.bf16_to_f32(orc.bf16_rne(dropped))
    bound = tight_bound(ref, af, bf, out_bf16)
    # the correct result passes
    assert np.all(np.abs(good - ref) <= bound)
    # the mutated result: inside the loose bound, far outside the tight one
    assert np.abs(dropped.astype(np.float64) - ref).max() <= tol
    assert np.mean(np.abs(dropped.astype(np.float64) - ref) > bound) > 0.5
    assert rel_frobenius(dropped, ref) > 2.0 ** -8
    if out_bf16:
        assert rel_frobenius(good, ref) <= 2.0 ** -8


def test_w4a16_dropped_group_rejected():
    """The decode headline's data (A ~ N(0,1), z = 8, scales U(0.005, 0.02)):
    the exact result rounded to f32 passes the W4A16 bound (a rigorous
    worst case for the 128 + q accumulation, ~1000x the typical error), and a
    result with one 128-k quant group left out fails it on most outputs.
    Smaller defects such as a zero point off by one stay inside this worst
    case; the GPU tests pin those with exact integer closed forms."""
    rng = np.random.default_rng(6)
    m, n, k, gs = 16, 128, 4096, 128
    G = k // gs
    q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    qw = orc.int4_pack(q.reshape(-1)).view("<u4").reshape(n, k // 8)
    s = orc.bf16_rne(rng.uniform(0.005, 0.02, (G, n)).astype(np.float32))
    a = orc.bf16_rne(rng.standard_normal((m, k)).astype(np.float32))
    w = orc.w4a16_dequant(qw, s, None, 8, n, k, gs)
    ref = orc.w4a16(a, qw, s, None, 8, m, n, k, gs)
    af = orc.bf16_to_f32(a).astype(np.float64)
    exact = af @ w.astype(np.float64).T
    z = np.full((G, n), 8)
    for out_bf16 in (False, True):
        bound = w4_tight_bound(ref, orc.bf16_to_f32(a), q, orc.bf16_to_f32(s), z, gs, out_bf16)
        good = exact.astype(np.float32)
        if out_bf16:
            good = orc.bf16_to_f32(orc.bf16_rne(good))
        assert np.all(np.abs(good - ref) <= bound)
        dropped = (exact - af[:, 640:768] @ w[:, 640:768].astype(np.float64).T).astype(np.float32)
        assert np.mean(np.abs(dropped.astype(np.float64) - ref) > bound) > 0.7

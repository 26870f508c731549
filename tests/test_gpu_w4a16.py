"""INT4 path parity on the GPU: the reference's standalone dequant kernels
(bit-exact), and the fused W4A16 GEMMs (decode / prefill / generic) against
the oracle's exact dequant + reference loop."""
import numpy as np
import pytest

import t0_gpu as t0
from gpu_util import Dev, bf16, check_close, f32, tolerance
from oracle.parity import rel_frobenius, w4_tight_bound
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    r = t0.GpuRuntime(0)
    yield r
    r.close()


@pytest.fixture()
def dev(rt):
    d = Dev(rt)
    yield d
    d.free()


def make_w4(rng, n, k, gs, per_group_zeros, scale_lo=0.005, scale_hi=0.02):
    G = k // gs
    q = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    qw = orc.int4_pack(q.reshape(-1)).view("<u4").reshape(n, k // 8).copy()
    s = bf16(rng.uniform(scale_lo, scale_hi, (G, n)))
    zw = None
    if per_group_zeros:
        z = rng.integers(0, 16, size=(G, n), dtype=np.uint8)
        zw = np.zeros((G, n // 8), np.uint32)
        for j in range(n):
            zw[:, j // 8] |= z[:, j].astype(np.uint32) << (4 * (j % 8))
    return qw, s, zw


def run_w4(rt, dev, a, qw, s, zw, m, n, k, gs, zc=8, out_f32=False, split_k=0, scales_f32=False):
    dc = dev.zeros(m * n * (4 if out_f32 else 2))
    sc = s if not scales_f32 else f32(s)
    rt.w4a16(dev.up(a), dev.up(qw), dev.up(sc), dev.up(zw) if zw is not None else 0, dc, m, n, k,
             group_size=gs, zero_const=zc, out_f32=out_f32, split_k=split_k, scales_f32=scales_f32)
    if out_f32:
        return dev.down(dc, np.float32, m * n).reshape(m, n)
    return f32(dev.down(dc, np.uint16, m * n).reshape(m, n))


def w4_tol(a, qw, s, zw, zc, n, k, gs):
    w = orc.w4a16_dequant(qw, s, zw, zc, n, k, gs)
    return tolerance(f32(a), w, k)


# ------------------------------------------------------- reference dequant --

@pytest.mark.parametrize("rows,cols,gs_log2", [(64, 1024, 7), (48, 96, 5), (7, 30, 1)])
@pytest.mark.parametrize("bf16_out", [False, True])
def test_dequant_int4_bit_exact(rt, dev, rows, cols, gs_log2, bf16_out):
    """build_dequant_int4_f32/_bf16 (src/t0/quant_kernels.rs:53-167), with the
    documented semantics: signed (q - zp) * scale, [row][group] params."""
    rng = np.random.default_rng(rows + cols)
    gs = 1 << gs_log2
    q = rng.integers(0, 16, size=rows * cols, dtype=np.uint8)
    packed = orc.int4_pack(q)
    ng = cols // gs
    scales = rng.uniform(-0.1, 0.1, rows * ng).astype(np.float32)
    zps = rng.integers(-3, 19, size=rows * ng).astype(np.int32)   # any i32 zero point
    out = dev.zeros(rows * cols * (2 if bf16_out else 4))
    rt.dequant_int4(dev.up(packed), dev.up(scales), dev.up(zps), out, rows, cols, gs_log2, bf16_out=bf16_out)
    if bf16_out:
        got = dev.down(out, np.uint16, rows * cols).reshape(rows, cols)
        assert np.array_equal(got, orc.dequant_int4_bf16(packed, scales, zps, rows, cols, gs))
    else:
        got = dev.down(out, np.float32, rows * cols).reshape(rows, cols)
        want = orc.dequant_int4_f32(packed, scales, zps, rows, cols, gs)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_reference_known_answers(rt, dev):
    """0xD7 -> lo 7, hi 13 -> (7-8)*s, (13-8)*s (src/t0/quant_kernels.rs:457-466)."""
    packed = np.array([0xD7, 0xAB], np.uint8)
    out = dev.zeros(16)
    rt.dequant_int4(dev.up(packed), dev.up(np.array([0.5], np.float32)), dev.up(np.array([8], np.int32)), out, 1, 4, 2)
    assert dev.down(out, np.float32, 4).tolist() == [-0.5, 2.5, 1.5, 1.0]


# ------------------------------------------------------------ fused W4A16 --

@pytest.mark.parametrize("m", [1, 5, 16, 32, 64])
def test_w4a16_decode_shapes(rt, dev, m):
    rng = np.random.default_rng(m)
    n, k, gs = 512, 1024, 128
    qw, s, zw = make_w4(rng, n, k, gs, per_group_zeros=False)
    a = bf16(rng.standard_normal((m, k)))
    plan, sk = rt.w4a16_plan(0, 0, 0, 0, 0, m, n, k, group_size=gs)
    assert plan.startswith("t0k_w4a16_decode")
    got = run_w4(rt, dev, a, qw, s, None, m, n, k, gs)
    ref = orc.w4a16(a, qw, s, None, 8, m, n, k, gs)
    check_close(got, ref, w4_tol(a, qw, s, None, 8, n, k, gs), f"decode m={m}")


@pytest.mark.parametrize("split_k", [1, 2, 4, 8])
def test_w4a16_decode_split_k_and_zeros(rt, dev, split_k):
    rng = np.random.default_rng(100 + split_k)
    m, n, k, gs = 16, 1024, 1024, 128
    qw, s, zw = make_w4(rng, n, k, gs, per_group_zeros=True)
    a = bf16(rng.standard_normal((m, k)))
    ref = orc.w4a16(a, qw, s, zw, 0, m, n, k, gs)
    got = run_w4(rt, dev, a, qw, s, zw, m, n, k, gs, split_k=split_k, out_f32=True)
    check_close(got, ref, w4_tol(a, qw, s, zw, 0, n, k, gs), f"sk={split_k}")
    assert np.max(np.abs(got - ref)) < 1e-3
    got2 = run_w4(rt, dev, a, qw, s, zw, m, n, k, gs, split_k=split_k, out_f32=True)
    assert np.array_equal(got.view(np.uint32), got2.view(np.uint32))   # deterministic reduction


def test_w4a16_decode_f32_scales(rt, dev):
    rng = np.random.default_rng(7)
    m, n, k, gs = 16, 256, 512, 128
    qw, s, _ = make_w4(rng, n, k, gs, per_group_zeros=False)
    a = bf16(rng.standard_normal((m, k)))
    got = run_w4(rt, dev, a, qw, s, None, m, n, k, gs, scales_f32=True)
    check_close(got, orc.w4a16(a, qw, s, None, 8, m, n, k, gs), w4_tol(a, qw, s, None, 8, n, k, gs), "f32 scales")


def _w4_parts(qw, s, zw, zc, n, k, gs):
    """[N][K] nibbles, [G][N] f32 scales and [G][N] zero points of a W4A16 operand."""
    q = orc.int4_unpack(qw.view(np.uint8), n * k).reshape(n, k)
    G = k // gs
    if zw is None:
        z = np.full((G, n), zc)
    else:
        z = np.zeros((G, n), np.int64)
        for j in range(8):
            z[:, j::8] = ((zw >> np.uint32(4 * j)) & 0xF).astype(np.int64)
    return q, f32(s), z


def check_w4_tight(got, ref, a, qw, s, zw, zc, n, k, gs, out_bf16, what):
    q, sf, z = _w4_parts(qw, s, zw, zc, n, k, gs)
    bound = w4_tight_bound(ref, f32(a), q, sf, z, gs, out_bf16)
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    frob = rel_frobenius(got, ref)
    assert np.all(err <= bound), (f"{what}: {int((err > bound).sum())} outputs over the tight bound "
                                  f"(max|err| {float(err.max()):.3e}, rel frob {frob:.3e})")
    if out_bf16:
        assert frob <= 2.0 ** -8, f"{what}: rel frob {frob:.3e}"
    print(f"{what}: max|err| {float(err.max()):.4g}, rel frob {frob:.4g}")


def test_w4a16_decode_headline(rt, dev):
    """The decode headline: A[16,4096] ~ N(0,1), W[4096,11008] int4, g=128,
    bf16 scales ~U(0.005,0.02), z = 8; a 1376-column block against the
    oracle under BASELINE's bound and the tight W4A16 bound, with bf16 and f32
    output; and an integer closed form over the whole matrix."""
    rng = np.random.default_rng(44)
    m, n, k, gs = 16, 11008, 4096, 128
    qw, s, _ = make_w4(rng, n, k, gs, per_group_zeros=False)
    a = bf16(rng.standard_normal((m, k)))
    j0, j1 = 4096, 4096 + 1376
    qb, sb = qw[j0:j1].copy(), s[:, j0:j1].copy()
    ref = orc.w4a16(a, qb, sb, None, 8, m, j1 - j0, k, gs)
    for out_f32 in (False, True):
        got = run_w4(rt, dev, a, qw, s, None, m, n, k, gs, out_f32=out_f32)
        check_close(got[:, j0:j1], ref, w4_tol(a, qb, sb, None, 8, j1 - j0, k, gs), "decode 16x4096x11008")
        check_w4_tight(got[:, j0:j1], ref, a, qb, sb, None, 8, j1 - j0, k, gs, not out_f32,
                       f"decode 16x4096x11008 {'f32' if out_f32 else 'bf16'} out")
    # whole-matrix closed form: unit scales, integer activations -> exact integers
    ones = np.full_like(s, 0x3F80)
    ai = rng.integers(-2, 3, size=(m, k))
    got_i = run_w4(rt, dev, bf16(ai), qw, ones, None, m, n, k, gs, out_f32=True)
    q = orc.int4_unpack(qw.view(np.uint8), n * k).reshape(n, k).astype(np.int64)
    want = ai.astype(np.int64) @ (q - 8).T
    assert np.array_equal(got_i.astype(np.int64), want)


@pytest.mark.parametrize("m", [3, 16])
def test_w4a16_decode_wide_n_zero_points(rt, dev, m):
    """N = 14336 gives 56 columns per workgroup: the 4-tile decode instance
    (8 waves, four groups in flight per wave), with per-group zero points;
    integer activations and unit scales make every output an exact integer."""
    rng = np.random.default_rng(45 + m)
    n, k, gs = 14336, 4096, 128
    qw, s, zw = make_w4(rng, n, k, gs, per_group_zeros=True)
    plan, _ = rt.w4a16_plan(0, 0, 0, 0, 0, m, n, k, group_size=gs)
    assert plan.startswith("t0k_w4a16_decode_t4_mb1"), plan
    ones = np.full_like(s, 0x3F80)
    ai = rng.integers(-3, 4, size=(m, k))
    got = run_w4(rt, dev, bf16(ai), qw, ones, zw, m, n, k, gs, out_f32=True)
    q = orc.int4_unpack(qw.view(np.uint8), n * k).reshape(n, k).astype(np.int64)
    z = np.zeros((k // gs, n), np.int64)
    for j in range(8):
        z[:, j::8] = ((zw >> np.uint32(4 * j)) & 0xF).astype(np.int64)
    w = q - np.repeat(z.T, gs, axis=1)                    # [n][k]
    assert np.array_equal(got.astype(np.int64), ai.astype(np.int64) @ w.T)
    # random activations and scales on a column block, against the oracle
    a = bf16(rng.standard_normal((m, k)))
    got = run_w4(rt, dev, a, qw, s, zw, m, n, k, gs)
    j0, j1 = 8192, 8192 + 1024
    ref = orc.w4a16(a, qw[j0:j1].copy(), s[:, j0:j1].copy(), zw[:, j0 // 8:j1 // 8].copy(), 0, m, j1 - j0, k, gs)
    check_close(got[:, j0:j1], ref, w4_tol(a, qw[j0:j1].copy(), s[:, j0:j1].copy(), zw[:, j0 // 8:j1 // 8].copy(),
                                           0, j1 - j0, k, gs), f"decode wide m={m}")


@pytest.mark.parametrize("m,n", [(256, 512), (300, 264), (1024, 256)])
def test_w4a16_prefill(rt, dev, m, n):
    rng = np.random.default_rng(m + n)
    k, gs = 1024, 128
    qw, s, zw = make_w4(rng, n, k, gs, per_group_zeros=True)
    a = bf16(rng.standard_normal((m, k)))
    plan, _ = rt.w4a16_plan(0, 0, 0, 0, 0, m, n, k, group_size=gs)
    assert plan.startswith("t0k_w4a16_prefill")
    got = run_w4(rt, dev, a, qw, s, zw, m, n, k, gs, zc=0)
    ref = orc.w4a16(a, qw, s, zw, 0, m, n, k, gs)
    check_close(got, ref, w4_tol(a, qw, s, zw, 0, n, k, gs), f"prefill {m}x{n}")


@pytest.mark.parametrize("m,n", [(300, 264), (1024, 256)])
def test_w4a16_prefill_f32_scales(rt, dev, m, n):
    """f32 scales reach the prefill kernel as given; bf16 scales are widened
    to f32 by its pre-pass, so the same scale values give the same bits."""
    rng = np.random.default_rng(3 * m + n)
    k, gs = 512, 128
    qw, s, zw = make_w4(rng, n, k, gs, per_group_zeros=True)
    a = bf16(rng.standard_normal((m, k)))
    plan, _ = rt.w4a16_plan(0, 0, 0, 0, 0, m, n, k, group_size=gs, scales_f32=True)
    assert plan.startswith("t0k_w4a16_prefill"), plan
    got32 = run_w4(rt, dev, a, qw, s, zw, m, n, k, gs, zc=0, out_f32=True, scales_f32=True)
    got16 = run_w4(rt, dev, a, qw, s, zw, m, n, k, gs, zc=0, out_f32=True)
    assert np.array_equal(got32.view(np.uint32), got16.view(np.uint32))
    ref = orc.w4a16(a, qw, s, zw, 0, m, n, k, gs)
    check_close(got32, ref, w4_tol(a, qw, s, zw, 0, n, k, gs), f"prefill f32 scales {m}x{n}")


@pytest.mark.parametrize("per_group_zeros,m,k,n", [(True, 320, 512, 256), (False, 320, 512, 256),
                                                   (True, 1024, 128, 256), (True, 1024, 256, 256),
                                                   (False, 1024, 384, 256), (True, 1024, 1152, 256),
                                                   (True, 4096, 256, 4096), (False, 2048, 640, 8192)])
def test_w4a16_prefill_exact_integers(rt, dev, per_group_zeros, m, k, n):
    """Integer activations in [-3, 3] and power-of-two scales: every group's
    sum a*(q - z) is an integer below 2^13 and the scaled sum over groups is
    exact in f32, so the f32 output must equal the exact product bit for bit
    (the zero-point term enters as one more MFMA block of row sums).  M = 320
    runs the two-stage 128x128 tiles; M = 1024 the three-stage 128x256 tiles,
    over 1, 2, 3 and 9 quant groups (the peeled last steps alone, and with
    the loop).  4096x4096 (512 tiles) and 2048x8192 (512 tiles, 5 groups)
    have more tiles than one dispatch round of one per CU: the tiles of odd
    rounds walk the quant groups from the last, and with exact sums the order
    cannot hide a group taken twice or skipped."""
    rng = np.random.default_rng(71 + per_group_zeros + m + k)
    gs = 128
    G = k // gs
    qw, _, zw = make_w4(rng, n, k, gs, per_group_zeros=per_group_zeros)
    s = bf16(2.0 ** rng.integers(-8, -4, (G, n)).astype(np.float32))
    ai = rng.integers(-3, 4, (m, k))
    a = bf16(ai.astype(np.float32))
    zc = 8
    q = ((qw[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(n, k).astype(np.int64)
    if per_group_zeros:
        z = np.stack([(zw[:, j // 8] >> (4 * (j % 8))) & 0xF for j in range(n)], axis=1).astype(np.int64)  # [G, n]
    else:
        z = np.full((G, n), zc, np.int64)
    w = (q - np.repeat(z.T, gs, axis=1)) * np.repeat(f32(s).astype(np.float64).T, gs, axis=1)   # [n, k]
    ref = (ai.astype(np.float64) @ w.T).astype(np.float32)
    plan, _ = rt.w4a16_plan(0, 0, 0, 0, 0, m, n, k, group_size=gs)
    assert plan.startswith("t0k_w4a16_prefill") and ("_s3" in plan) == (m >= 1024), plan
    got = run_w4(rt, dev, a, qw, s, zw, m, n, k, gs, zc=zc, out_f32=True)
    assert np.array_equal(got, ref)


def test_w4a16_prefill_headline_rows(rt, dev):
    """The prefill shape: 4096x4096x14336, per-group zero points; sampled
    rows under BASELINE's bound and the tight W4A16 bound."""
    rng = np.random.default_rng(45)
    m, n, k, gs = 4096, 14336, 4096, 128
    qw, s, zw = make_w4(rng, n, k, gs, per_group_zeros=True)
    a = bf16(rng.standard_normal((m, k)))
    got = run_w4(rt, dev, a, qw, s, zw, m, n, k, gs, zc=0)
    rows = [0, 1, 777, 2048, 4095]
    ref = np.concatenate([orc.w4a16(a, qw, s, zw, 0, m, n, k, gs, r, r + 1) for r in rows])
    check_close(got[rows], ref, w4_tol(a, qw[:2048].copy(), s[:, :2048].copy(), zw[:, :256].copy(), 0, 2048, k, gs),
                "prefill rows")
    check_w4_tight(got[rows], ref, a[rows], qw, s, zw, 0, n, k, gs, True, "prefill 4096x4096x14336 bf16 out")


@pytest.mark.parametrize("m,n,rows,per_group_zeros", [(16, 11008, 16, True), (16, 11008, 16, False),
                                                        (4096, 14336, 32, True)])
def test_w4a16_f32_out_error_vs_float64(rt, dev, m, n, rows, per_group_zeros):
    """f32 output of the fused kernels against the float64 product of the
    exactly dequantized weights, next to the oracle (direct dequant +
    sequential f32 loop): the 128 + q form accumulates T = sum a (128 + q),
    up to ~29x the result, yet loses at most about a bit against the direct
    dequant (measured on MI355X: relative Frobenius 8.1e-7 - 1.2e-6 against
    7.0e-7 - 7.9e-7; worst element 1.1e-7 - 1.5e-7 of (|A||W|) against
    2.4e-7 - 3.3e-7).  Bounds: Frobenius within 2x the oracle's, worst
    element within the oracle's worst."""
    rng = np.random.default_rng(46)
    k, gs = 4096, 128
    zc = 0 if per_group_zeros else 8
    qw, s, zw = make_w4(rng, n, k, gs, per_group_zeros=per_group_zeros)
    a = bf16(rng.standard_normal((m, k)))
    got = run_w4(rt, dev, a, qw, s, zw, m, n, k, gs, zc=zc, out_f32=True)[:rows].astype(np.float64)
    w = orc.w4a16_dequant(qw, s, zw, zc, n, k, gs)                 # (q - z) * s, exact in f32
    av = f32(a[:rows]).astype(np.float64)
    exact = av @ w.astype(np.float64).T
    scale = np.abs(av) @ np.abs(w.astype(np.float64)).T
    ora = orc.gemm_bf16_f32w_rows(a, w, 0, rows).astype(np.float64)
    e_got, e_ora = rel_frobenius(got, exact), rel_frobenius(ora, exact)
    w_got, w_ora = np.max(np.abs(got - exact) / scale), np.max(np.abs(ora - exact) / scale)
    assert e_got <= 2.0 * e_ora and w_got <= w_ora, (e_got, e_ora, w_got, w_ora)


def test_w4a16_generic_group_64(rt, dev):
    rng = np.random.default_rng(9)
    m, n, k, gs = 3, 40, 256, 64
    qw, s, zw = make_w4(rng, n, k, gs, per_group_zeros=True)
    a = bf16(rng.standard_normal((m, k)))
    plan, _ = rt.w4a16_plan(0, 0, 0, 0, 0, m, n, k, group_size=gs)
    assert plan == "t0k_w4a16_generic"
    got = run_w4(rt, dev, a, qw, s, zw, m, n, k, gs, zc=0)
    check_close(got, orc.w4a16(a, qw, s, zw, 0, m, n, k, gs), w4_tol(a, qw, s, zw, 0, n, k, gs), "generic")


def test_gptq_weight_end_to_end(rt, dev):
    """GptqWeight bytes (src/t0/quant_kernels.rs:249-258) -> W4A16 operand -> GEMM."""
    rng = np.random.default_rng(12)
    rows, cols, gs = 256, 512, 128
    ng = cols // gs
    q = rng.integers(0, 16, size=rows * cols, dtype=np.uint8)
    packed = orc.int4_pack(q)
    scales = f32(bf16(rng.uniform(0.005, 0.02, rows * ng)))
    zps = rng.integers(0, 16, size=rows * ng).astype(np.int32)
    w = t0.GptqWeight.from_bytes(orc.gptq_to_bytes(rows, cols, gs, packed, scales, zps))
    qw, sc, zw = w.to_w4a16()
    m = 8
    a = bf16(rng.standard_normal((m, cols)))
    got = run_w4(rt, dev, a, qw, sc, zw, m, rows, cols, gs, zc=0, out_f32=True)
    wdq = orc.dequant_int4_f32(packed, scales, zps, rows, cols, gs)
    ref = (f32(a).astype(np.float64) @ wdq.T.astype(np.float64))
    check_close(got, ref, tolerance(f32(a), wdq, cols), "gptq e2e")

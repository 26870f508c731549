"""Residual add + RMSNorm in front of the projections, on the GPU: the
reference's fused kernel (src/t0/ffn_fused_kernels.rs) through the C ABI and
by raw dispatch, the row RMSNorm, and the Ignis fused ops
(src/ignis/ops/fused_rmsnorm_gemm.rs) on an INT4 weight (the decode kernel
with the norm fused in for one row) and on a dense f32 weight.  Checked
against the oracle: bit-exact where the arithmetic is exact (x2, integer
closed forms), else within the acceptance tolerance
1e-2 * sqrt(K) * max|a| * max|w| or the reference tests' own 1e-4."""
import struct

import numpy as np
import pytest

import t0_gpu as t0
from t0_gpu import fused_rmsnorm as fr
from gpu_util import bf16, check_close, f32, tolerance
from oracle import oracle as orc
from test_gpu_w4a16 import make_w4

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rt():
    r = t0.GpuRuntime(0)
    yield r
    r.close()


def up(rt, a):
    return rt.upload(np.ascontiguousarray(a, dtype=np.float32))


def down(rt, buf, dtype, shape):
    rt.wait_idle()
    v = buf.read(dtype, int(np.prod(shape))).reshape(shape)
    buf.free()
    return v


def _sin(n, f, scale=1.0, op=np.sin):
    return (op(np.arange(n, dtype=np.float32) * np.float32(f)) * np.float32(scale)).astype(np.float32)


def _ref_case(name):
    """The data of the reference's own tests (ffn_fused_kernels.rs:247-427)."""
    if name == "cpu_fused_reference":
        m, d = 2, 64
        return (m, d, _sin(m * d, 0.17).reshape(m, d), _sin(m * d, 0.23, op=np.cos).reshape(m, d),
                (0.8 + np.arange(d) * 0.005).astype(np.float32), _sin(m * d, 0.31, 0.5).reshape(m, d))
    if name == "fused_equals_separate":
        m, d = 4, 128
        return (m, d, _sin(m * d, 0.13, 1.5).reshape(m, d), _sin(m * d, 0.19, 0.8, op=np.cos).reshape(m, d),
                (0.9 + np.arange(d) * 0.002).astype(np.float32), _sin(m * d, 0.41).reshape(m, d))
    m, d = 8, 4096                                                     # test_cpu_fused_large
    return (m, d, _sin(m * d, 0.001).reshape(m, d), _sin(m * d, 0.002, op=np.cos).reshape(m, d),
            (1.0 + np.arange(d) * 0.0001).astype(np.float32), _sin(m * d, 0.003, 0.01).reshape(m, d))


@pytest.mark.parametrize("case", ["cpu_fused_reference", "fused_equals_separate", "cpu_fused_large"])
def test_ffn_fused_kernel_matches_oracle(rt, case):
    m, d, res, hid, gamma, w = _ref_case(case)
    eps = 1e-5
    bufs = [up(rt, x) for x in (res, hid, gamma, w)]
    got = down(rt, fr.ffn_fused_rmsnorm_gemm(rt, *bufs, m, d, eps), np.float32, (m,))
    ref = orc.ffn_fused_rmsnorm_gemm(res, hid, gamma, w, eps)
    normed, _, _ = orc.rmsnorm_rows(res, hid, gamma, eps)
    bound = 1e-4 + 1e-5 * np.abs(normed * w).sum(axis=1)           # the reference tests' 1e-4, plus sum order
    assert np.all(np.isfinite(got)) and np.all(np.abs(got - ref) <= bound), (got, ref)
    for b in bufs:
        b.free()


def test_ffn_fused_raw_dispatch_with_reference_kernargs(rt):
    """The reference's own dispatch: kernel by name, 48-byte kernargs
    [residual, hidden, gamma, weight, output: u64; D: u32; eps: f32],
    grid = M * 128 work-items (ffn_fused_kernels.rs:47-49, 191-199)."""
    m, d, res, hid, gamma, w = _ref_case("fused_equals_separate")
    eps = 1e-5
    bufs = [up(rt, x) for x in (res, hid, gamma, w)]
    out = rt.alloc(4 * m)
    kern = rt.kernel_load(t0.code_object(), "ffn_fused_rmsnorm_gemm", [128], kernarg_size=48)
    ka = struct.pack("<QQQQQIf", *(b.gpu_addr() for b in bufs), out.gpu_addr(), d, eps)
    rt.dispatch(kern, [m * 128, 1, 1], ka)
    got = down(rt, out, np.float32, (m,))
    via_abi = down(rt, fr.ffn_fused_rmsnorm_gemm(rt, *bufs, m, d, eps), np.float32, (m,))
    assert np.array_equal(got.view(np.uint32), via_abi.view(np.uint32))
    for b in bufs:
        b.free()


@pytest.mark.parametrize("rows,d,with_hid,out_bf16", [(1, 4096, True, True), (5, 1000, False, False),
                                                      (3, 64, True, False), (16, 4096, True, True),
                                                      (2, 1001, True, True), (1, 9000, False, False)])
def test_rmsnorm_rows(rt, rows, d, with_hid, out_bf16):
    rng = np.random.default_rng(rows * 10 + d)
    res = rng.standard_normal((rows, d)).astype(np.float32)
    hid = rng.standard_normal((rows, d)).astype(np.float32) if with_hid else None
    gamma = rng.uniform(0.5, 1.5, d).astype(np.float32)
    eps = 1e-5
    br, bg = up(rt, res), up(rt, gamma)
    bh = up(rt, hid) if with_hid else None
    bx2 = rt.alloc(4 * rows * d)
    out = fr.rmsnorm(rt, br, bg, rows, d, eps, hidden=bh, out_bf16=out_bf16, x2_out=bx2)
    normed, x2, _ = orc.rmsnorm_rows(res, hid, gamma, eps)
    assert np.array_equal(down(rt, bx2, np.float32, (rows, d)).view(np.uint32), x2.view(np.uint32))
    if out_bf16:
        got = f32(down(rt, out, np.uint16, (rows, d)))
        assert np.all(np.abs(got - normed) <= np.abs(normed) * 2.0**-8 + 1e-30)       # one bf16 ulp
    else:
        got = down(rt, out, np.float32, (rows, d))
        assert np.all(np.abs(got - normed) <= np.abs(normed) * 1e-5 + 1e-30)
    for b in (br, bg, bh):
        if b is not None:
            b.free()


def _closed_form_inputs(m, k):
    res = np.tile(np.array([3.0, -1.0], np.float32), (m, k // 2))
    hid = np.tile(np.array([-1.0, 3.0], np.float32), (m, k // 2))
    gamma = (np.arange(k) % 5 + 1).astype(np.float32)
    return res, hid, gamma


def test_rmsnorm_closed_form(rt):
    """x2 = 2 everywhere, eps 0: inv_rms = 1/2 and normed = gamma exactly."""
    m, k = 4, 96
    res, hid, gamma = _closed_form_inputs(m, k)
    br, bh, bg = up(rt, res), up(rt, hid), up(rt, gamma)
    got = down(rt, fr.rmsnorm(rt, br, bg, m, k, 0.0, hidden=bh), np.float32, (m, k))
    assert np.array_equal(got, np.tile(gamma, (m, 1)))
    for b in (br, bh, bg):
        b.free()


@pytest.mark.parametrize("m,n,k,zp,with_hid", [(1, 11008, 4096, False, True), (1, 4096, 4096, True, False),
                                                (1, 14336, 4096, False, True), (1, 512, 1024, True, True),
                                                (5, 768, 2048, False, True)])
def test_fused_rmsnorm_w4a16(rt, m, n, k, zp, with_hid):
    """One row: the decode kernel with the residual add and RMSNorm fused in;
    more rows: RMSNorm to bf16, then the W4A16 GEMM.  Against the oracle's
    RMSNorm (f32) times the exactly dequantized weight, in f64."""
    rng = np.random.default_rng(m + n + k)
    gs, eps = 128, 1e-5
    qw, s, zw = make_w4(rng, n, k, gs, per_group_zeros=zp)
    res = rng.standard_normal((m, k)).astype(np.float32)
    hid = rng.standard_normal((m, k)).astype(np.float32) if with_hid else None
    gamma = rng.uniform(0.5, 1.5, k).astype(np.float32)
    bufs = {"res": up(rt, res), "g": up(rt, gamma), "qw": rt.upload(qw), "s": rt.upload(s),
            "z": rt.upload(zw) if zp else None, "h": up(rt, hid) if with_hid else None, "x2": rt.alloc(4 * m * k)}
    out = fr.fused_rmsnorm_w4a16(rt, bufs["res"], bufs["g"], bufs["qw"], bufs["s"], bufs["z"], m, n, k, eps,
                                 hidden=bufs["h"], x2_out=bufs["x2"], out_f32=True, zero_const=8)
    got = down(rt, out, np.float32, (m, n))
    normed, x2, _ = orc.rmsnorm_rows(res, hid, gamma, eps)
    w = orc.w4a16_dequant(qw, s, zw if zp else None, 8, n, k, gs)
    ref = normed.astype(np.float64) @ w.astype(np.float64).T
    check_close(got, ref, tolerance(normed, w, k), f"fused rmsnorm w4a16 {m}x{n}x{k}")
    assert np.array_equal(down(rt, bufs.pop("x2"), np.float32, (m, k)).view(np.uint32), x2.view(np.uint32))
    for b in bufs.values():
        if b is not None:
            b.free()


@pytest.mark.parametrize("zp", [False, True])
def test_fused_rmsnorm_w4a16_closed_form(rt, zp):
    """x2 = 2, eps 0, integer gamma, unit scales: every output is the exact
    integer sum_k gamma_k * (q - z)."""
    m, n, k, gs = 1, 512, 1024, 128
    rng = np.random.default_rng(5 + zp)
    qw, s, zw = make_w4(rng, n, k, gs, per_group_zeros=zp)
    ones = np.full_like(s, 0x3F80)
    res, hid, gamma = _closed_form_inputs(m, k)
    bufs = [up(rt, res), up(rt, hid), up(rt, gamma), rt.upload(qw), rt.upload(ones)] + ([rt.upload(zw)] if zp else [])
    out = fr.fused_rmsnorm_w4a16(rt, bufs[0], bufs[2], bufs[3], bufs[4], bufs[5] if zp else None, m, n, k, 0.0,
                                 hidden=bufs[1], out_f32=True, zero_const=8)
    got = down(rt, out, np.float32, (m, n))
    q = orc.int4_unpack(qw.view(np.uint8), n * k).reshape(n, k).astype(np.int64)
    if zp:
        z = np.zeros((k // gs, n), np.int64)
        for j in range(8):
            z[:, j::8] = ((zw >> np.uint32(4 * j)) & 0xF).astype(np.int64)
        q = q - np.repeat(z.T, gs, axis=1)
    else:
        q = q - 8
    want = gamma.astype(np.int64)[None, :] @ q.T
    assert np.array_equal(got.astype(np.int64), want)
    for b in bufs:
        b.free()


@pytest.mark.parametrize("m,k,n,with_hid", [(1, 301, 130, True), (7, 512, 256, False), (33, 1000, 520, True)])
def test_fused_residual_rmsnorm_gemm_dense(rt, m, k, n, with_hid):
    """Dense f32 weight [k, n]: RMSNorm then the bf16 matmul (the Ignis
    prefill branch), bf16(normed) . bf16(W) in f32; k and n not multiples of 8."""
    rng = np.random.default_rng(m * k + n)
    eps = 1e-6
    res = rng.standard_normal((m, k)).astype(np.float32)
    hid = rng.standard_normal((m, k)).astype(np.float32) if with_hid else None
    gamma = rng.uniform(0.5, 1.5, k).astype(np.float32)
    w = (rng.standard_normal((k, n)) * 0.1).astype(np.float32)
    br, bg, bw = up(rt, res), up(rt, gamma), up(rt, w)
    bh = up(rt, hid) if with_hid else None
    y = fr.fused_residual_rmsnorm_gemm(rt, br, bh, bg, bw, (m, k), (k, n), eps)
    got = down(rt, y, np.float32, (m, n))
    normed, _, _ = orc.rmsnorm_rows(res, hid, gamma, eps)
    ref = orc.gemm_nn(orc.bf16_rne(normed), orc.bf16_rne(w))
    check_close(got, ref, tolerance(normed, w, k), f"dense {m}x{k}x{n}")
    for b in (br, bg, bw, bh):
        if b is not None:
            b.free()


def test_shape_errors(rt):
    b = up(rt, np.zeros((4, 8), np.float32))
    with pytest.raises(ValueError, match="weight dim mismatch"):
        fr.fused_rmsnorm_gemm(rt, b, b, b, (4, 8), (7, 4), 1e-5)
    with pytest.raises(t0.T0Error):
        t0._check(t0.lib().t0_rmsnorm(rt.h, b.gpu_addr(), 0, b.gpu_addr(), b.gpu_addr(), 0, 0, 8, 8, 1e-5, 0))
    b.free()

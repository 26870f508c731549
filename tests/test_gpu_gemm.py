"""bf16 GEMM parity on the GPU: every gfx950 kernel instance against the CPU
oracle (the reference's cpu_gemm_bf16 restated), through every entry point
the reference exposes (gemm_gen dispatch, tile_ir dispatch, raw load +
dispatch, high-level t0_gemm, tuner)."""
import os
import struct

import numpy as np
import pytest

import t0_gpu as t0
from gpu_util import Dev, bf16, check_close, check_tight, f32, tolerance
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


def run_gemm(rt, dev, a, b, m, n, k, layout, out_dtype, cfg=None, **kw):
    da, db = dev.up(a), dev.up(b)
    ob = 2 if out_dtype == t0.OUT_BF16 else 4
    dc = dev.zeros(m * n * ob)
    rt.gemm(da, db, dc, m, n, k, transpose=layout, out_dtype=out_dtype, cfg=cfg, **kw)
    if out_dtype == t0.OUT_BF16:
        return f32(dev.down(dc, np.uint16, m * n).reshape(m, n))
    return dev.down(dc, np.float32, m * n).reshape(m, n)


def instance_configs():
    out = []
    for name in t0.PRESETS:
        c = getattr(t0.GemmConfig, name)()
        if c.is_feasible() and c.n_col_passes == 1 and c.use_lds:
            out.append(c)
    return out


# ---------------------------------------------------------- exact layouts --

@pytest.mark.parametrize("layout", [t0.NT, t0.NN])
def test_integer_pattern_exact(rt, dev, layout):
    """Small integers: every partial sum is exact, so any MFMA operand or
    accumulator layout mistake shows as an exact mismatch."""
    m, n, k = 64, 96, 128
    ai = (np.arange(m * k) % 17 - 8).reshape(m, k)          # src/t0/tile_ir.rs:5056-5057
    bi_nt = (np.arange(n * k) % 13 - 6).reshape(n, k)
    b = bf16(bi_nt if layout == t0.NT else bi_nt.T.copy())
    want = ai.astype(np.int64) @ bi_nt.T.astype(np.int64)
    for cfg in instance_configs():
        got = run_gemm(rt, dev, bf16(ai), b, m, n, k, layout, t0.OUT_F32, cfg=cfg.copy(transpose=layout))
        assert np.array_equal(got.astype(np.int64), want), cfg.name()


def test_smoke_pattern_256(rt, dev):
    """src/t0/auto_gemm.rs:235-269 smoke pattern, every instance, both layouts."""
    s = 256
    ai = (np.arange(s * s) % 7 - 3).reshape(s, s)
    bi = (np.arange(s * s) % 5 - 2).reshape(s, s)          # WT[N,K]
    want = ai.astype(np.int64) @ bi.T.astype(np.int64)
    for cfg in instance_configs():
        for layout, b in ((t0.NT, bf16(bi)), (t0.NN, bf16(bi.T.copy()))):
            got = run_gemm(rt, dev, bf16(ai), b, s, s, s, layout, t0.OUT_F32, cfg=cfg.copy(transpose=layout))
            assert np.array_equal(got.astype(np.int64), want), (cfg.name(), layout)


# ------------------------------------------------------- correctness matrix --

SIZES = [(64, 64, 64), (128, 128, 128), (256, 256, 256), (64, 256, 64), (128, 1024, 256), (256, 512, 512)]


@pytest.mark.parametrize("m,k,n", SIZES)
def test_gemm_correctness_matrix(rt, dev, m, k, n):
    """examples/test_gemm_correctness.rs:66-86: xorshift U(-1,1) bf16 data,
    seeds m*1000+k and n*2000+k; all instances x {NT,NN} x {f32,bf16}."""
    x = orc.xorshift_bf16(m * k, m * 1000 + k).reshape(m, k)
    wt = orc.xorshift_bf16(n * k, n * 2000 + k).reshape(n, k)
    ref = orc.gemm_nt(x, wt)
    tol = tolerance(f32(x), f32(wt), k)
    for cfg in instance_configs():
        for layout, b in ((t0.NT, wt), (t0.NN, wt.T.copy())):
            for od in (t0.OUT_F32, t0.OUT_BF16):
                got = run_gemm(rt, dev, x, b, m, n, k, layout, od, cfg=cfg.copy(transpose=layout, out_dtype=od))
                check_close(got, ref, tol, f"{cfg.name()} layout={layout} out={od}")
                if od == t0.OUT_F32:
                    # f32 accumulation order differs from the sequential loop only by rounding
                    assert np.max(np.abs(got - ref)) <= 2e-5 * k


def test_bf16_output_is_rne_of_f32(rt, dev):
    m = n = k = 512
    rng = np.random.default_rng(5)
    a = bf16(rng.standard_normal((m, k)))
    b = bf16(rng.standard_normal((k, n)))
    cfg = t0.GemmConfig.tile_128x128_k64()
    g32 = run_gemm(rt, dev, a, b, m, n, k, t0.NN, t0.OUT_F32, cfg=cfg.copy(transpose=t0.NN))
    g16 = run_gemm(rt, dev, a, b, m, n, k, t0.NN, t0.OUT_BF16, cfg=cfg.copy(transpose=t0.NN, out_dtype=t0.OUT_BF16))
    assert np.array_equal(f32(orc.bf16_rne(g32)).view(np.uint32), g16.view(np.uint32))


# ---------------------------------------------------------- golden vectors --

def _golden(golden_dir, name, dtype, shape):
    return np.fromfile(os.path.join(golden_dir, name), dtype=dtype).reshape(shape)


@pytest.mark.parametrize("w_name,ref_name,ref16_name", [("w_gate.bin", "h_gate_f32ref.bin", "h_gate_bf16acc.bin"),
                                                        ("w_up.bin", "h_up_f32ref.bin", "h_up_bf16acc.bin")])
def test_torch_fixture_gemm(rt, dev, golden_dir, w_name, ref_name, ref16_name):
    """benchmarks/torch_ref (seed 42): X[64,256] . W_gate[512,256]^T and
    X . W_up^T, f32 output and torch's bf16 output."""
    x = _golden(golden_dir, "x.bin", np.uint16, (64, 256))
    w = _golden(golden_dir, w_name, np.uint16, (512, 256))
    ref32 = _golden(golden_dir, ref_name, np.float32, (64, 512))
    ref16 = _golden(golden_dir, ref16_name, np.float32, (64, 512))
    tol = tolerance(f32(x), f32(w), 256)
    for cfg in (None, t0.GemmConfig.tile_64x64_k64(), t0.GemmConfig.tile_256x256_k64()):
        got = run_gemm(rt, dev, x, w, 64, 512, 256, t0.NT, t0.OUT_F32, cfg=cfg)
        check_close(got, ref32, tol, "h_gate f32")
        assert np.max(np.abs(got - ref32)) < 5e-6
        g16 = run_gemm(rt, dev, x, w, 64, 512, 256, t0.NT, t0.OUT_BF16,
                       cfg=cfg.copy(out_dtype=t0.OUT_BF16) if cfg is not None else None)
        assert np.mean(g16 == ref16) > 0.99
        assert np.all(np.abs(g16 - ref16) <= np.abs(ref16) * 2.0**-7 + 1e-30)


def test_torch_fixture_second_gemm(rt, dev, golden_dir):
    s = _golden(golden_dir, "swiglu_bf16_trunc.bin", np.uint16, (64, 512))
    wd = _golden(golden_dir, "w_down.bin", np.uint16, (256, 512))
    ref = _golden(golden_dir, "y_bf16_f32acc.bin", np.float32, (64, 256))
    got = run_gemm(rt, dev, s, wd, 64, 256, 512, t0.NT, t0.OUT_F32)
    check_close(got, ref, tolerance(f32(s), f32(wd), 512), "y")
    # same product in NN form
    got_nn = run_gemm(rt, dev, s, wd.T.copy(), 64, 256, 512, t0.NN, t0.OUT_F32)
    check_close(got_nn, ref, tolerance(f32(s), f32(wd), 512), "y nn")
    # bf16 output against torch's bf16 chain (benchmarks/gen_torch_ref.py:141)
    ref16 = _golden(golden_dir, "y_bf16chain.bin", np.float32, (64, 256))
    g16 = run_gemm(rt, dev, s, wd, 64, 256, 512, t0.NT, t0.OUT_BF16)
    assert np.mean(g16 == ref16) > 0.99
    assert np.all(np.abs(g16 - ref16) <= np.abs(ref16) * 2.0**-7 + 1e-30)


# ------------------------------------------------- instances beyond presets --

@pytest.mark.parametrize("m,n,k,split", [(64, 4096, 1024, 4), (130, 200, 328, 1), (256, 192, 512, 2), (1, 64, 64, 1)])
def test_64x64_four_wave_tile(rt, dev, m, n, k, split):
    """The 64x64 tile on four waves (two workgroups per CU), reached by an
    explicit config (tile 64x64x64, 256 threads): NN and NT, f32 and bf16
    out, ragged M / N / K and in-kernel split-K."""
    rng = np.random.default_rng(m + n + k)
    a = bf16(rng.uniform(-1, 1, (m, k)))
    b = bf16(rng.uniform(-1, 1, (k, n)))
    ref = orc.gemm_nn(a, b)
    tol = tolerance(f32(a), f32(b), k)
    base = t0.GemmConfig.tile_64x64_k64().copy(wg_size=256, split_k=split if split > 1 else 0)
    for layout, bb in ((t0.NN, b), (t0.NT, b.T.copy())):
        for od in (t0.OUT_F32, t0.OUT_BF16):
            got = run_gemm(rt, dev, a, bb, m, n, k, layout, od, cfg=base.copy(transpose=layout, out_dtype=od))
            check_close(got, ref, tol, f"64x64 w4 {m}x{n}x{k} split {split} layout={layout} out={od}")


@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (300, 260, 128), (100, 700, 40), (256, 512, 200),
                                   (513, 300, 1000), (256, 256, 4160), (64, 96, 24), (260, 300, 96)])
def test_eight_wave_256_tiles(rt, dev, m, n, k):
    """The 8-wave 256x256 instances (BK 64 with two stages: the 4096^3
    kernel; BK 32 with four stages and the ping-pong K loop), reached by
    explicit configs (512 threads): one, two, three and many K steps, K
    tails, ragged M / N, NN and NT, f32 and bf16 out. Small-integer operands
    keep every partial sum exact, so the f32 output must match the integer
    product bit for bit."""
    rng = np.random.default_rng(m * 3 + n + k)
    ai = rng.integers(-8, 9, size=(m, k))
    bi = rng.integers(-6, 7, size=(k, n))
    want = ai.astype(np.int64) @ bi.astype(np.int64)
    a, b = bf16(ai), bf16(bi)
    for base in (t0.GemmConfig.tile_256x256_k64(), t0.GemmConfig.tile_256x256_k32()):
        cfg = base.copy(wg_size=512)
        for layout, bb in ((t0.NN, b), (t0.NT, bf16(bi.T.copy()))):
            got = run_gemm(rt, dev, a, bb, m, n, k, layout, t0.OUT_F32, cfg=cfg.copy(transpose=layout))
            assert np.array_equal(got.astype(np.int64), want), (cfg.name(), m, n, k, layout)
            got16 = run_gemm(rt, dev, a, bb, m, n, k, layout, t0.OUT_BF16,
                             cfg=cfg.copy(transpose=layout, out_dtype=t0.OUT_BF16))
            assert np.array_equal(got16, f32(orc.bf16_rne(want.astype(np.float32)))), (cfg.name(), m, n, k, layout)


@pytest.mark.parametrize("m,n,k,sk", [(128, 512, 1024, 1), (128, 512, 1024, 4), (100, 520, 1024, 2),
                                      (128, 4096, 4096, 4), (64, 256, 256, 2), (64, 256, 128, 2), (128, 512, 1000, 1),
                                      (130, 384, 1536, 8)])
@pytest.mark.parametrize("tile", ["64x128", "128x64"])
def test_register_staged_tiles(rt, dev, m, n, k, sk, tile):
    """The 64x128x64 and 128x64x64 four-wave tiles, whose K loop is staged
    through registers when every split-K partition is a whole number of
    pairs of 64-k steps (K % (128 * split) == 0; for 128x64 also M >= 128;
    else the DMA loop runs): one and many pairs per partition, ragged M / N,
    the skinny shape, partitions of one step and a K tail (DMA loop), NN and
    NT, f32 and bf16 out, in-kernel split-K.  Small-integer operands keep
    every partial sum exact."""
    print(f"register-staged {tile}: m={m} n={n} k={k} split={sk}", flush=True)
    rng = np.random.default_rng(m * 7 + n + k + sk)
    ai = rng.integers(-8, 9, size=(m, k))
    bi = rng.integers(-6, 7, size=(k, n))
    want = ai.astype(np.int64) @ bi.astype(np.int64)
    a, b = bf16(ai), bf16(bi)
    base = t0.GemmConfig.tile_64x128_k64() if tile == "64x128" else t0.GemmConfig.tile_128x64_k64()
    cfg = base.copy(wg_size=256, split_k=sk if sk > 1 else 0)
    for layout, bb in ((t0.NN, b), (t0.NT, bf16(bi.T.copy()))):
        got = run_gemm(rt, dev, a, bb, m, n, k, layout, t0.OUT_F32, cfg=cfg.copy(transpose=layout))
        assert np.array_equal(got.astype(np.int64), want), (cfg.name(), m, n, k, sk, layout)
        got16 = run_gemm(rt, dev, a, bb, m, n, k, layout, t0.OUT_BF16,
                         cfg=cfg.copy(transpose=layout, out_dtype=t0.OUT_BF16))
        assert np.array_equal(got16, f32(orc.bf16_rne(want.astype(np.float32)))), (cfg.name(), m, n, k, sk, layout)


@pytest.mark.parametrize("sk", [1, 2, 4])
def test_eight_wave_256x64_split_k_and_bias(rt, dev, sk):
    """The 8-wave 256x256x64 instance on interior tiles with whole 64-k steps
    per partition (its branch-free K loop) and on edge tiles (the general
    loop) in one launch, bit-exact on small-integer operands: split-K
    reduced in-kernel (bf16 out, NN and NT), f32 planes summed on the host
    through the gemm_gen dispatch, and the bias + ReLU epilogue with integer
    bias values."""
    rng = np.random.default_rng(500 + sk)
    k = 1024                                  # K / split_k = 1024, 512 or 256: whole 64-k steps
    cfg0 = t0.GemmConfig.tile_256x256_k64().copy(wg_size=512)
    for m, n in ((512, 512), (300, 520)):     # all tiles interior / interior and edge tiles
        ai = rng.integers(-8, 9, size=(m, k))
        bi = rng.integers(-6, 7, size=(k, n))
        want = ai.astype(np.int64) @ bi.astype(np.int64)
        a, b = bf16(ai), bf16(bi)
        for layout, bb in ((t0.NN, b), (t0.NT, bf16(bi.T.copy()))):
            cfg = cfg0.copy(transpose=layout, out_dtype=t0.OUT_BF16, split_k=sk if sk > 1 else 0)
            got16 = run_gemm(rt, dev, a, bb, m, n, k, layout, t0.OUT_BF16, cfg=cfg)
            assert np.array_equal(got16, f32(orc.bf16_rne(want.astype(np.float32)))), (sk, m, n, layout)
        if m % 256:
            continue                          # the gemm_gen grid has M / tile_m tiles
        da, db = dev.up(a), dev.up(b)
        if sk > 1:
            cfg = cfg0.copy(transpose=t0.NN, out_dtype=t0.OUT_F32, split_k=sk)
            planes = dev.zeros(sk * m * n * 4)
            kern = rt.ensure_kernel_t0(cfg)
            gx, gy = t0.compute_grid_auto(cfg, m, n)
            rt.dispatch(kern, [gx, gy, 1], t0.build_kernargs(da, db, planes, k, n, m, cfg))
            got = orc.splitk_sum(dev.down(planes, np.float32, sk * m * n).reshape(sk, m, n))
            assert np.array_equal(got.astype(np.int64), want), sk
        else:
            bias = rng.integers(-300, 301, size=n).astype(np.float32)
            cfg = cfg0.copy(transpose=t0.NN, out_dtype=t0.OUT_F32, epilogue=t0.EPI_BIAS_ADD_RELU)
            dy = dev.zeros(m * n * 4)
            kern = rt.ensure_kernel_t0(cfg)
            gx, gy = t0.compute_grid_auto(cfg, m, n)
            rt.dispatch(kern, [gx, gy, 1], t0.build_kernargs_with_bias(da, db, dy, k, n, m, cfg, dev.up(bias)))
            got = dev.down(dy, np.float32, m * n).reshape(m, n)
            assert np.array_equal(got.astype(np.int64), np.maximum(want + bias.astype(np.int64), 0))


# ----------------------------------------------------------------- bounds --

@pytest.mark.parametrize("m,n,k", [(33, 31, 40), (1, 1, 8), (255, 257, 264), (100, 200, 72), (300, 130, 1000)])
def test_boundary_sentinel(rt, dev, m, n, k):
    """src/t0/tile_boundary_tests.rs: rows/cols outside M x N stay untouched
    (sentinel -9999 in a padded C with ldc > N), everything inside matches."""
    rng = np.random.default_rng(m * 7 + n)
    a = bf16(rng.uniform(-1, 1, (m, k)))
    b = bf16(rng.uniform(-1, 1, (k, n)))
    ref = orc.gemm_nn(a, b)
    ldc = n + 12
    for cfg in (t0.GemmConfig.tile_256x256_k64(), t0.GemmConfig.tile_128x64_k16(), t0.GemmConfig.tile_32x64_k64(),
                t0.GemmConfig.tile_128x128_k32()):
        for layout, bb in ((t0.NN, b), (t0.NT, b.T.copy())):
            c = np.full((m + 3, ldc), -9999.0, np.float32)
            dc = dev.up(c)
            rt.gemm(dev.up(a), dev.up(bb), dc, m, n, k, transpose=layout, cfg=cfg.copy(transpose=layout), ldc=ldc)
            out = dev.down(dc, np.float32, c.size).reshape(c.shape)
            check_close(out[:m, :n], ref, tolerance(f32(a), f32(b), k), f"{cfg.name()} {layout}")
            assert np.all(out[:m, n:] == -9999.0) and np.all(out[m:, :] == -9999.0), cfg.name()


def test_generic_fallback_unaligned(rt, dev):
    """K % 8 != 0 and an odd lda: the generic kernel takes it."""
    m, n, k = 37, 45, 37
    rng = np.random.default_rng(3)
    a = bf16(rng.uniform(-1, 1, (m, k + 3)))                 # lda = k + 3
    b = bf16(rng.uniform(-1, 1, (n, k)))
    ref = orc.gemm_nt(a[:, :k].copy(), b)
    da, db = dev.up(a), dev.up(b)
    dc = dev.zeros(m * n * 4)
    rt.gemm(da, db, dc, m, n, k, transpose=t0.NT, lda=k + 3)
    got = dev.down(dc, np.float32, m * n).reshape(m, n)
    check_close(got, ref, tolerance(f32(a), f32(b), k), "generic")


# --------------------------------------------------- reference entry points --

def test_gemm_gen_dispatch_path(rt, dev):
    """ensure_kernel_t0 + build_kernargs (40 B) + compute_grid_auto + dispatch,
    as examples/hello_gemm_gen.rs does, including split-K planes summed on the
    host and the 48-byte bias+ReLU variant."""
    m, n, k = 256, 192, 512
    x = orc.xorshift_bf16(m * k, 11).reshape(m, k)
    wt = orc.xorshift_bf16(n * k, 12).reshape(n, k)
    ref = orc.gemm_nt(x, wt)
    tol = tolerance(f32(x), f32(wt), k)
    dx, dw = dev.up(x), dev.up(wt)
    for cfg in (t0.GemmConfig.tile_128x64_k16(), t0.GemmConfig.tile_64x64_k32().copy(split_k=4),
                t0.GemmConfig.tile_32x64_k16().copy(split_k=2, swap_grid=0)):
        sk = max(1, cfg.split_k)
        kern = rt.ensure_kernel_t0(cfg)
        assert kern.info()["kernarg_size"] == 40
        dy = dev.zeros(m * n * 4 * sk)
        gx, gy = t0.compute_grid_auto(cfg, m, n)
        rt.dispatch(kern, [gx, gy, 1], t0.build_kernargs(dx, dw, dy, k, n, m, cfg))
        planes = dev.down(dy, np.float32, m * n * sk).reshape(sk, m, n)
        got = orc.splitk_sum(planes)
        check_close(got, ref, tol, cfg.name())
    bias = np.linspace(-1, 1, n).astype(np.float32)
    cfg = t0.GemmConfig.tile_64x64_k16().copy(epilogue=t0.EPI_BIAS_ADD_RELU)
    kern = rt.ensure_kernel_t0(cfg)
    dy = dev.zeros(m * n * 4)
    gx, gy = t0.compute_grid_auto(cfg, m, n)
    rt.dispatch(kern, [gx, gy, 1], t0.build_kernargs_with_bias(dx, dw, dy, k, n, m, cfg, dev.up(bias)))
    got = dev.down(dy, np.float32, m * n).reshape(m, n)
    check_close(got, np.maximum(ref + bias, 0), tol, "bias_relu")


def _epi_ref(y, ops, bias, scale, lo, hi):
    y = y.astype(np.float64)
    for op in ops:
        if op == "bias": y = y + bias
        elif op == "scale": y = y * scale
        elif op == "relu": y = np.maximum(y, 0)
        elif op == "silu": y = y / (1 + np.exp(-y))
        elif op == "gelu": y = y / (1 + np.exp(-1.702 * y))
        elif op == "abs": y = np.abs(y)
        elif op == "neg": y = -y
        elif op == "clamp": y = np.clip(y, lo, hi)
    return y


@pytest.mark.parametrize("ops", [["bias", "silu"], ["scale", "gelu"], ["neg", "abs", "clamp"], ["bias", "relu", "scale"]])
def test_tile_ir_dispatch_epilogues(rt, dev, ops):
    """TileGemm + build_kernargs_m (44 B + epilogue args) + dispatch, epilogue
    chain semantics of src/t0/tile_ir.rs:3406-3540 (GELU = x*sigmoid(1.702x))."""
    m, n, k = 192, 256, 320
    rng = np.random.default_rng(len(ops))
    x = bf16(rng.uniform(-1, 1, (m, k)))
    wt = bf16(rng.uniform(-1, 1, (n, k)))
    bias = rng.uniform(-2, 2, n).astype(np.float32)
    ref = _epi_ref(orc.gemm_nt(x, wt), ops, bias, 0.75, -0.5, 1.5)
    spec = t0.TileGemm.make(128, 128, 64, epilogue=ops)
    kern = rt.ensure_tile_kernel(spec)
    dy = dev.zeros(m * n * 4)
    ka = spec.build_kernargs_m(dev.up(x), dev.up(wt), dy, k, n, m, bias=dev.up(bias), scale=0.75, clamp_min=-0.5,
                               clamp_max=1.5)
    assert len(ka) == kern.info()["kernarg_size"]
    rt.dispatch(kern, spec.compute_grid(m, n), ka)
    got = dev.down(dy, np.float32, m * n).reshape(m, n)
    check_close(got, ref, tolerance(f32(x), f32(wt), k) * 2, "+".join(ops))


def test_fixup_split_k_bf16_deterministic(rt, dev):
    """split-K reduced in-kernel (bf16 output, epilogue once), twice, bitwise equal."""
    m, n, k = 128, 512, 4096
    rng = np.random.default_rng(8)
    a = bf16(rng.standard_normal((m, k)) * 0.5)
    b = bf16(rng.standard_normal((k, n)) * 0.5)
    ref = orc.gemm_nn(a, b)
    for sk in (2, 4, 8):
        cfg = t0.GemmConfig.tile_128x128_k64().copy(split_k=sk, transpose=t0.NN, out_dtype=t0.OUT_BF16)
        g1 = run_gemm(rt, dev, a, b, m, n, k, t0.NN, t0.OUT_BF16, cfg=cfg)
        g2 = run_gemm(rt, dev, a, b, m, n, k, t0.NN, t0.OUT_BF16, cfg=cfg)
        assert np.array_equal(g1.view(np.uint32), g2.view(np.uint32))
        check_close(g1, ref, tolerance(f32(a), f32(b), k), f"sk={sk}")


@pytest.mark.parametrize("sk", [2, 4])
def test_pingpong_tile_split_k(rt, dev, sk):
    """The ping-pong 256x256x32 instance under split-K, bit-exact on
    small-integer operands with ragged N and a K tail in each partition:
    the in-kernel reduction (bf16 out, ragged M through t0_gemm), and f32
    planes summed on the host through the gemm_gen dispatch, whose 40-byte
    kernargs carry no M (the grid gives M / tile_m tiles, so M is a
    multiple of 256 there, src/t0/gemm_gen.rs:308-329)."""
    n, k = 520, 1120                          # K / split_k = 560 or 280: a partial last stage
    rng = np.random.default_rng(sk)
    base = t0.GemmConfig.tile_256x256_k32().copy(wg_size=512, split_k=sk)
    for m, planes_path in ((300, False), (512, True)):
        ai = rng.integers(-8, 9, size=(m, k))
        bi = rng.integers(-6, 7, size=(k, n))
        want = ai.astype(np.int64) @ bi.astype(np.int64)
        a, b = bf16(ai), bf16(bi)
        for layout, bb in ((t0.NN, b), (t0.NT, bf16(bi.T.copy()))):
            if not planes_path:
                got16 = run_gemm(rt, dev, a, bb, m, n, k, layout, t0.OUT_BF16,
                                 cfg=base.copy(transpose=layout, out_dtype=t0.OUT_BF16))
                assert np.array_equal(got16, f32(orc.bf16_rne(want.astype(np.float32)))), (sk, layout)
                continue
            cfg = base.copy(transpose=layout, out_dtype=t0.OUT_F32)
            assert m % cfg.tile_m == 0
            da, db = dev.up(a), dev.up(bb)
            planes = dev.zeros(sk * m * n * 4)
            kern = rt.ensure_kernel_t0(cfg)
            gx, gy = t0.compute_grid_auto(cfg, m, n)
            rt.dispatch(kern, [gx, gy, 1], t0.build_kernargs(da, db, planes, k, n, m, cfg))
            p = dev.down(planes, np.float32, sk * m * n).reshape(sk, m, n)
            assert np.array_equal(p.astype(np.int64).sum(axis=0), want), (sk, layout)


def test_raw_kernel_load_and_dispatch(rt, dev):
    """GpuKernel::load of the library's code object + raw kernarg dispatch."""
    n = 4096
    x = np.random.default_rng(2).standard_normal(n).astype(np.float32) * 100
    src, dst = dev.up(x), dev.zeros(n * 2)
    kern = rt.kernel_load(t0.code_object(), "t0k_f32_to_bf16", [256], kernarg_size=56)
    # t0_aux_params: src, dst, m, n, ld_src, ld_dst, planes, flags, plane_stride, rows_pad, pad
    ka = struct.pack("<QQIIIIIIQII", src, dst, 1, n, n, n, 0, 0, 0, 0, 0)
    rt.dispatch(kern, [n, 1, 1], ka)
    got = dev.down(dst, np.uint16, n)
    assert np.array_equal(got, orc.bf16_rne(x))


def test_poisoned_runtime_refuses_dispatch(dev):
    """src/ignis/gpu_context.rs:311-313: a poisoned runtime fails fast."""
    with t0.GpuRuntime(0) as r2:
        cfg = t0.GemmConfig.tile_64x64_k16()
        kern = r2.ensure_kernel_t0(cfg)
        r2.mark_poisoned()
        assert r2.is_poisoned()
        with pytest.raises(t0.T0Error) as e:
            r2.dispatch(kern, [64, 1, 1], bytes(40))
        assert e.value.status == -4


def test_kernarg_length_mismatch_rejected(rt):
    """src/ignis/gpu_context.rs:319-322."""
    kern = rt.ensure_kernel_t0(t0.GemmConfig.tile_64x64_k16())
    with pytest.raises(t0.T0Error) as e:
        rt.dispatch(kern, [64, 1, 1], bytes(44))
    assert e.value.status == -5


# ------------------------------------------------------------ small kernels --

def test_splitk_reduce_f32_to_bf16_unpad(rt, dev):
    rng = np.random.default_rng(4)
    planes = rng.standard_normal((4, 65, 130)).astype(np.float32)
    dp = dev.up(planes)
    do = dev.zeros(65 * 130 * 4)
    rt.splitk_reduce(dp, 65 * 130 * 4, 4, do, 65, 130)
    assert np.array_equal(dev.down(do, np.float32, 65 * 130).reshape(65, 130), orc.splitk_sum(planes))
    dob = dev.zeros(65 * 130 * 2)
    rt.splitk_reduce(dp, 65 * 130 * 4, 4, dob, 65, 130, out_bf16=True)
    assert np.array_equal(dev.down(dob, np.uint16, 65 * 130).reshape(65, 130), orc.bf16_rne(orc.splitk_sum(planes)))
    padded = rng.standard_normal((33, 96)).astype(np.float32)
    dpad, dout = dev.up(padded), dev.zeros(33 * 70 * 4)
    rt.unpad_2d(dpad, dout, 33, 70, 96)
    assert np.array_equal(dev.down(dout, np.float32, 33 * 70).reshape(33, 70), padded[:, :70])


# ----------------------------------------------------- headline-size checks --

def _sampled_rows(m, count=16):
    return sorted(set(np.linspace(0, m - 1, count).astype(int).tolist()))


def test_headline_4096_nn_bf16(rt, dev):
    """The headline shape: 4096^3 NN, N(0,1) bf16 inputs, bf16 output.
    16 rows spread over all 16 tile rows against the oracle, under
    BASELINE's bound and the tight per-element bound with relative Frobenius
    error <= 2^-8; the chosen kernel against a second kernel on the whole
    matrix; and every tile of the 16 x 16 grid (XCD remap, grouped order)
    bit-exact on small-integer operands, whose products and sums are exact."""
    m = n = k = 4096
    rng = np.random.default_rng(42)
    a = bf16(rng.standard_normal((m, k)))
    b = bf16(rng.standard_normal((k, n)))
    got = run_gemm(rt, dev, a, b, m, n, k, t0.NN, t0.OUT_BF16)
    rows = _sampled_rows(m)
    ref = np.stack([orc.gemm_rows(a, b, "nn", r, r + 1)[0] for r in rows])
    check_close(got[rows], ref, tolerance(f32(a), f32(b), k), "4096^3")
    err, frob = check_tight(got[rows], ref, f32(a)[rows], f32(b), True, "4096^3 tight")
    print(f"4096^3 NN bf16: max|err| {err:.4g}, rel frob {frob:.4g}")
    other = run_gemm(rt, dev, a, b, m, n, k, t0.NN, t0.OUT_BF16,
                     cfg=t0.GemmConfig.tile_128x128_k64().copy(transpose=t0.NN, out_dtype=t0.OUT_BF16))
    check_close(got, other, tolerance(f32(a), f32(b), k), "4096^3 vs 128x128")
    ai = rng.integers(-2, 3, size=(m, k)).astype(np.float64)
    bi = rng.integers(-2, 3, size=(k, n)).astype(np.float64)
    want = ai @ bi                                   # |sums| <= 16384: exact in f32 and f64
    got_i = run_gemm(rt, dev, bf16(ai), bf16(bi), m, n, k, t0.NN, t0.OUT_BF16)
    assert np.array_equal(got_i, f32(orc.bf16_rne(want.astype(np.float32))))
    got_f = run_gemm(rt, dev, bf16(ai), bf16(bi), m, n, k, t0.NN, t0.OUT_F32)
    assert np.array_equal(got_f, want.astype(np.float32))


def test_skinny_128x4096x4096(rt, dev):
    """The skinny shape: M=128, N=K=4096, N(0,0.02) inputs, bf16 out (split-K
    reduced in-kernel): sampled rows under both bounds, and the whole output
    bit-exact on small-integer operands."""
    m, n, k = 128, 4096, 4096
    rng = np.random.default_rng(43)
    a = bf16(rng.normal(0, 0.02, (m, k)))
    b = bf16(rng.normal(0, 0.02, (k, n)))
    got = run_gemm(rt, dev, a, b, m, n, k, t0.NN, t0.OUT_BF16)
    rows = _sampled_rows(m, 12)
    ref = np.stack([orc.gemm_rows(a, b, "nn", r, r + 1)[0] for r in rows])
    check_close(got[rows], ref, tolerance(f32(a), f32(b), k), "skinny")
    err, frob = check_tight(got[rows], ref, f32(a)[rows], f32(b), True, "skinny tight")
    print(f"skinny 128x4096x4096 bf16: max|err| {err:.4g}, rel frob {frob:.4g}")
    ai = rng.integers(-3, 4, size=(m, k)).astype(np.float64)
    bi = rng.integers(-3, 4, size=(k, n)).astype(np.float64)
    got_i = run_gemm(rt, dev, bf16(ai), bf16(bi), m, n, k, t0.NN, t0.OUT_BF16)
    assert np.array_equal(got_i, f32(orc.bf16_rne((ai @ bi).astype(np.float32))))


# ------------------------------------------------------------------ tuner --

def test_tuner_and_auto_gemm(rt, dev, tmp_path):
    """src/t0/auto_gemm.rs:82-216, :555-590: tune, JSON cache, cached re-tune,
    auto_gemm result."""
    tuner = t0.GemmTuner(cache_dir=str(tmp_path), max_candidates=4, n_iters=3)
    cfg, tf = tuner.tune(rt, 512, 512, 512)
    assert cfg.is_feasible() or cfg.split_k > 1
    assert tf > 0
    f = tmp_path / "gemm_512x512x512.json"     # the reference's file name for NT / f32
    assert f.exists(), list(tmp_path.iterdir())
    text = f.read_text()
    assert f'"wg_size":{cfg.wg_size}' in text and '"arch":"gfx950"' in text, text
    cfg2, tf2 = tuner.tune(rt, 512, 512, 512)
    assert cfg2.name() == cfg.name() and tf2 == tf
    # GemmTuneResult.all: every timed candidate, fastest first, the pick first
    timed, cached = tuner.results(512, 512, 512)
    assert not cached and 1 <= len(timed) <= 4
    assert [tf_ for _, tf_ in timed] == sorted((tf_ for _, tf_ in timed), reverse=True)
    assert (timed[0][0].name(), timed[0][0].wg_size, timed[0][1]) == (cfg.name(), cfg.wg_size, tf)
    # a fresh tuner state (as in a new process) reads the same pick back from disk
    tuner3 = t0.GemmTuner(cache_dir=str(tmp_path), max_candidates=4, n_iters=3)
    cfg3, tf3 = tuner3.tune(rt, 512, 512, 512)
    assert (cfg3.name(), cfg3.wg_size) == (cfg.name(), cfg.wg_size) and abs(tf3 - tf) < 0.01
    timed3, cached3 = tuner3.results(512, 512, 512)
    assert cached3 and [(c.name(), c.wg_size) for c, _ in timed3] == [(c.name(), c.wg_size) for c, _ in timed]
    m = n = k = 512
    x = orc.xorshift_bf16(m * k, 1).reshape(m, k)
    wt = orc.xorshift_bf16(n * k, 2).reshape(n, k)
    dc = dev.zeros(m * n * 4)
    t0.auto_gemm(rt, dev.up(x), dev.up(wt), dc, m, n, k)
    check_close(dev.down(dc, np.float32, m * n).reshape(m, n), orc.gemm_nt(x, wt), tolerance(f32(x), f32(wt), k),
                "auto_gemm")


def test_empty_and_malformed_calls_fail_before_launch(rt, dev):
    """Empty or malformed problems return an error with a message before
    anything is launched, and the runtime stays usable: the reference's
    Result<_, String> paths (gemm_gen.rs:271-281, quant_kernels.rs:251-287)
    rather than a fault or a poisoned runtime."""
    buf = dev.zeros(64 * 64 * 4)
    for m, n, k in ((0, 64, 64), (64, 0, 64), (64, 64, 0)):
        for tr in (t0.NT, t0.NN):
            with pytest.raises(t0.T0Error, match="empty GEMM"):
                rt.gemm(buf, buf, buf, m, n, k, transpose=tr, out_dtype=t0.OUT_BF16)
    with pytest.raises(t0.T0Error, match="split_k"):
        rt.gemm(buf, buf, buf, 64, 64, 64, cfg=t0.GemmConfig.tile_128x128_k64().copy(split_k=3))
    for k, gs in ((100, 128), (128, 12), (130, 64)):   # K % gs, gs % 8, K % 8
        with pytest.raises(t0.T0Error):
            rt.w4a16(buf, buf, buf, 0, buf, 4, 64, k, group_size=gs)
    assert not rt.is_poisoned()
    a = bf16(np.arange(64 * 64).reshape(64, 64) % 5 - 2)
    got = run_gemm(rt, dev, a, a, 64, 64, 64, t0.NN, t0.OUT_F32)
    assert np.array_equal(got, orc.gemm_nn(a, a))


def test_tune_tile_ir(rt, dev, tmp_path):
    """src/t0/cost_model.rs:855-1150: tune_tile_ir times the reference's
    presets and the cost model's tiles, caches the fastest in
    tile_ir_MxNxK.json with the reference's keys, answers the next call from
    that file, reads a file in the reference's own layout, and the tuned spec
    computes the product through the tile_ir dispatch path."""
    t0.GemmTuner(cache_dir=str(tmp_path), max_candidates=4, n_iters=3)
    m, n, k = 256, 384, 512
    r = t0.tune_tile_ir(rt, m, n, k)
    assert not r.from_cache and r.best_tflops > 0 and len(r.all) >= 5, r
    tfs = [tf for _, tf in r.all]
    assert tfs == sorted(tfs, reverse=True)
    assert r.all[0][0] == r.best.name() and r.all[0][1] == r.best_tflops
    assert {t0.TileGemm.make(128, 128, 64).name(), t0.TileGemm.make(32, 64, 16).name()} <= {nm for nm, _ in r.all}
    text = (tmp_path / f"tile_ir_{m}x{n}x{k}.json").read_text()
    for key in ('"tile_m":', '"tile_n":', '"tile_k":', '"split_k":1', '"wgp":false', '"tflops":', '"all":[["',
                '"arch":"gfx950"'):
        assert key in text, (key, text)
    r2 = t0.tune_tile_ir(rt, m, n, k)
    assert r2.from_cache and r2.all == [] and r2.best.name() == r.best.name()
    assert r2.best.waves_per_wg == r.best.waves_per_wg and abs(r2.best_tflops - r.best_tflops) < 0.01
    # as the reference writes it: no arch, no wave count (the tile's gfx950 kernel is taken)
    (tmp_path / "tile_ir_128x128x256.json").write_text(
        '{"tile_m":64,"tile_n":64,"tile_k":16,"split_k":1,"wgp":false,"tflops":12.50,"all":[["x",12.50]]}')
    r3 = t0.tune_tile_ir(rt, 128, 128, 256)
    assert r3.from_cache and (r3.best.tile_m, r3.best.tile_n, r3.best.tile_k) == (64, 64, 16)
    assert r3.best_tflops == 12.5 and r3.best.waves_per_wg >= 1
    x = orc.xorshift_bf16(m * k, 3).reshape(m, k)
    wt = orc.xorshift_bf16(n * k, 4).reshape(n, k)
    kern = rt.ensure_tile_kernel(r.best)
    dy = dev.zeros(m * n * 4)
    rt.dispatch(kern, r.best.compute_grid(m, n), r.best.build_kernargs_m(dev.up(x), dev.up(wt), dy, k, n, m))
    check_close(dev.down(dy, np.float32, m * n).reshape(m, n), orc.gemm_nt(x, wt), tolerance(f32(x), f32(wt), k),
                r.best.name())


# ------------------------------------------------------------------ graphs --

def test_graph_pins_workspace():
    """A captured split-K GEMM holds the runtime's workspace and semaphore
    addresses: while the graph exists a call that would grow them is refused
    (T0_ERR_INVALID, nothing reallocated), replays stay correct, and after
    the graph is destroyed the larger call runs.  A capture whose first call
    would allocate the workspace is refused too."""
    with t0.GpuRuntime(0) as rt2:
        d = Dev(rt2)
        try:
            m, n, k = 256, 256, 1024
            rng = np.random.default_rng(11)
            a = bf16(rng.integers(-4, 5, size=(m, k)))
            b = bf16(rng.integers(-4, 5, size=(k, n)))
            want = f32(orc.bf16_rne(orc.gemm_nn(a, b)))
            cfg = t0.GemmConfig.tile_128x128_k64().copy(split_k=4, transpose=t0.NN, out_dtype=t0.OUT_BF16)
            # first split-K call inside a capture: the workspace would be allocated there
            da, db, dc = d.up(a), d.up(b), d.zeros(m * n * 2)
            with pytest.raises(t0.T0Error, match="graph capture"):
                rt2.capture(lambda: rt2.gemm(da, db, dc, m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16, cfg=cfg))
            rt2.gemm(da, db, dc, m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16, cfg=cfg)   # sizes the workspace
            assert np.array_equal(f32(d.down(dc, np.uint16, m * n).reshape(m, n)), want)
            g = rt2.capture(lambda: rt2.gemm(da, db, dc, m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16, cfg=cfg))
            # a call needing a larger workspace (4096^2 tiles x split 4 = 256 MiB of partials)
            M2 = N2 = 4096
            a2, b2 = d.zeros(M2 * 256 * 2), d.zeros(256 * N2 * 2)
            c2 = d.zeros(M2 * N2 * 2)
            big = t0.GemmConfig.tile_256x256_k64().copy(wg_size=512, split_k=4, transpose=t0.NN, out_dtype=t0.OUT_BF16)
            with pytest.raises(t0.T0Error, match="captured graph"):
                rt2.gemm(a2, b2, c2, M2, N2, 256, transpose=t0.NN, out_dtype=t0.OUT_BF16, cfg=big)
            for _ in range(3):
                d.rt.memset(dc, 0, m * n * 2)
                rt2.wait_idle()
                g.launch()
                rt2.wait_idle()
                assert np.array_equal(f32(d.down(dc, np.uint16, m * n).reshape(m, n)), want)
            del g
            rt2.gemm(a2, b2, c2, M2, N2, 256, transpose=t0.NN, out_dtype=t0.OUT_BF16, cfg=big)
            rt2.wait_idle()
            assert np.all(d.down(c2, np.uint16, M2 * N2) == 0)
        finally:
            d.free()

"""The entry point that allocates nothing (t0_gemm_noalloc) against t0_gemm,
through the C ABI: split-K GEMMs reduced in-kernel in the library's fixed
scratch array give the same bits as with the runtime's workspace, on two
calls in a row (the second smaller), with no device memory taken by the
calls; sizes past the array's limits are refused."""
import ctypes as C

import numpy as np
import pytest

import t0_gpu as t0
from gpu_util import Dev, bf16, f32

pytestmark = pytest.mark.gpu


def _free_bytes():
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def test_noalloc_matches_t0_gemm_twice_second_smaller():
    print("no-alloc: fresh runtime, split-K GEMMs 128x4096x4096 (split 4) then 64x1024x2048 (split 2)", flush=True)
    with t0.GpuRuntime(0) as rt:
        d = Dev(rt)
        try:
            rng = np.random.default_rng(21)
            cases = [(128, 4096, 4096, t0.GemmConfig.tile_128x64_k64().copy(split_k=4)),
                     (64, 1024, 2048, t0.GemmConfig.tile_64x64_k64().copy(wg_size=256, split_k=2))]
            bufs = []
            for m, n, k, cfg in cases:
                a = bf16(rng.standard_normal((m, k)))
                b = bf16(rng.standard_normal((k, n)))
                bufs.append((d.up(a), d.up(b), d.zeros(m * n * 2), d.zeros(m * n * 2)))
            for (m, n, k, cfg), (da, db, c_ref, c_na) in zip(cases, bufs):
                c = cfg.copy(transpose=t0.NN, out_dtype=t0.OUT_BF16)
                rt.wait_idle()
                free0 = _free_bytes()
                rt.gemm_noalloc(da, db, c_na, m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16, cfg=c)
                rt.wait_idle()
                assert _free_bytes() == free0, "t0_gemm_noalloc took device memory"
                rt.gemm(da, db, c_ref, m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16, cfg=c)
                got = d.down(c_na, np.uint16, m * n)
                want = d.down(c_ref, np.uint16, m * n)
                assert np.array_equal(got, want), (m, n, k)
            # a third call reusing the first case after the smaller one: the
            # array keeps the last call's contents, the counters are cleared
            (m, n, k, cfg), (da, db, c_ref, c_na) = cases[0], bufs[0]
            c = cfg.copy(transpose=t0.NN, out_dtype=t0.OUT_BF16)
            d.rt.memset(c_na, 0, m * n * 2)
            rt.gemm_noalloc(da, db, c_na, m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16, cfg=c)
            assert np.array_equal(d.down(c_na, np.uint16, m * n), d.down(c_ref, np.uint16, m * n))
        finally:
            d.free()


def test_noalloc_refuses_past_its_limits():
    print("no-alloc: limits (4096^3 split 4 needs 256 MiB of partials)", flush=True)
    with t0.GpuRuntime(0) as rt:
        d = Dev(rt)
        try:
            m = n = 4096
            k = 256
            da, db, dc = d.zeros(m * k * 2), d.zeros(k * n * 2), d.zeros(m * n * 2)
            big = t0.GemmConfig.tile_256x256_k64().copy(wg_size=512, split_k=4, transpose=t0.NN,
                                                       out_dtype=t0.OUT_BF16)
            with pytest.raises(t0.T0Error, match="scratch"):
                rt.gemm_noalloc(da, db, dc, m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16, cfg=big)
            # without split-K nothing needs the scratch: the same shape runs
            rt.gemm_noalloc(da, db, dc, m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16,
                            cfg=big.copy(split_k=0))
            rt.wait_idle()
            assert np.all(d.down(dc, np.uint16, m * n) == 0)
        finally:
            d.free()


def test_noalloc_without_config_fits_its_scratch():
    """cfg=None: where the selection's split-K partials exceed the scratch
    (1024x4096x11008 NN bf16: 256x256 split 4 needs 64 MiB), the call takes
    the best-ranked candidate that fits, here without split-K; it equals
    t0_gemm with that config bit for bit, takes no device memory, and
    agrees with t0_gemm's own selection within the tight bound on sampled
    rows against float64."""
    import math
    from oracle.parity import tight_bound
    m, n, k = 1024, 4096, 11008
    scratch, max_tiles = 32 << 20, 16384

    def fits(c):
        sk = max(c.split_k, 1)
        tiles = math.ceil(m / c.tile_m) * math.ceil(n / c.tile_n)
        return sk <= 1 or (tiles <= max_tiles and sk * tiles * c.tile_m * c.tile_n * 4 <= scratch - max_tiles * 4)

    ranked = t0.auto_schedule_gemm(m, n, k, t0.NN, t0.OUT_BF16)
    assert not fits(ranked[0][0]), ranked[0][0].name()
    want_cfg = next(c for c, _ in ranked if fits(c))
    print(f"no-alloc: cfg=None {m}x{n}x{k}, selection {ranked[0][0].name()}, expected {want_cfg.name()}", flush=True)
    with t0.GpuRuntime(0) as rt:
        d = Dev(rt)
        try:
            rng = np.random.default_rng(31)
            a = bf16(rng.standard_normal((m, k)))
            b = bf16(rng.standard_normal((k, n)))
            da, db = d.up(a), d.up(b)
            c_na, c_cfg, c_sel = d.zeros(m * n * 2), d.zeros(m * n * 2), d.zeros(m * n * 2)
            rt.wait_idle()
            free0 = _free_bytes()
            rt.gemm_noalloc(da, db, c_na, m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16)
            rt.wait_idle()
            assert _free_bytes() == free0, "t0_gemm_noalloc took device memory"
            rt.gemm(da, db, c_cfg, m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16,
                    cfg=want_cfg.copy(transpose=t0.NN, out_dtype=t0.OUT_BF16))
            rt.gemm(da, db, c_sel, m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16)
            got = d.down(c_na, np.uint16, m * n).reshape(m, n)
            assert np.array_equal(got, d.down(c_cfg, np.uint16, m * n).reshape(m, n))
            rows = [0, 1, 511, 1023]
            af, bf = f32(a[rows]).astype(np.float64), f32(b).astype(np.float64)
            ref = af @ bf
            bound = tight_bound(ref, f32(a[rows]), f32(b), True, "nn")
            sel = d.down(c_sel, np.uint16, m * n).reshape(m, n)
            for out in (got, sel):
                err = np.abs(f32(out[rows]).astype(np.float64) - ref)
                assert np.all(err <= bound), float((err - bound).max())
        finally:
            d.free()

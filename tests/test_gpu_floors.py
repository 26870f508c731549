"""Measurement aids behind the C-ABI (no counterpart in the reference): the
operand read floor of a GEMM tiling runs on the shapes it documents, refuses
the rest with a message before any launch, and leaves the runtime computing
correctly afterwards."""
import numpy as np
import pytest

import t0_gpu as t0
from gpu_util import Dev, f32

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


@pytest.mark.parametrize("layout", [t0.NN, t0.NT])
@pytest.mark.parametrize("m,n,k", [(128, 4096, 4096), (100, 1000, 1024)])
def test_floor_tile_read_runs(rt, dev, layout, m, n, k):
    """Every mode on the pick's tiling and two explicit ones, ragged M / N included
    (the tails read nothing past the operands)."""
    print(f"floor_tile_read layout={layout} m={m} n={n} k={k}", flush=True)
    da, db = dev.zeros(m * k * 2), dev.zeros(k * n * 2)
    pick = rt.gemm_select(m, n, k, layout, t0.OUT_BF16)
    for cfg in (None, pick.copy(tile_m=128, tile_n=64, split_k=4), pick.copy(tile_m=256, tile_n=256, split_k=1)):
        for mode in (1, 2, 3):
            rt.floor_tile_read(da, db, m, n, k, transpose=layout, mode=mode, cfg=cfg)
    rt.wait_idle()


def test_floor_tile_read_refuses(rt, dev):
    m, n, k = 128, 512, 1024
    da, db = dev.zeros(m * k * 2), dev.zeros(k * n * 2)
    pick = rt.gemm_select(m, n, k, t0.NN, t0.OUT_BF16)
    bad = [dict(mode=0), dict(mode=4),
           dict(mode=3, cfg=pick.copy(tile_m=128, tile_n=64, split_k=32)),      # K not a multiple of 64 * split
           dict(mode=3, cfg=pick.copy(tile_m=512, tile_n=64, split_k=1)),       # tile_m + tile_n > 512
           dict(mode=3, cfg=pick.copy(tile_m=60, tile_n=64, split_k=1))]        # tile_m not a multiple of 8
    for kw in bad:
        with pytest.raises(t0.T0Error):
            rt.floor_tile_read(da, db, m, n, k, transpose=t0.NN, **kw)
    with pytest.raises(t0.T0Error):
        rt.floor_tile_read(da, db, m, n, k, transpose=t0.NN, mode=3, lda=k - 8)
    with pytest.raises(t0.T0Error):
        rt.floor_tile_read(da + 8, db, m, n, k, transpose=t0.NN, mode=3)          # misaligned A
    with pytest.raises(t0.T0Error):
        rt.floor_tile_read(da, db, m, n, k, transpose=t0.NN, mode=3, ldb=n + 4)   # ldb % 8 != 0
    # the runtime still computes: a small integer GEMM is exact
    rng = np.random.default_rng(7)
    a = rng.integers(-3, 4, (64, 256)).astype(np.float32)
    b = rng.integers(-3, 4, (256, 128)).astype(np.float32)
    ua = (a.view(np.uint32) >> 16).astype(np.uint16)
    ub = (b.view(np.uint32) >> 16).astype(np.uint16)
    dc = dev.zeros(64 * 128 * 2)
    rt.gemm(dev.up(ua), dev.up(ub), dc, 64, 128, 256, transpose=t0.NN, out_dtype=t0.OUT_BF16)
    got = f32(dev.down(dc, np.uint16, 64 * 128).reshape(64, 128))
    np.testing.assert_array_equal(got, a @ b)

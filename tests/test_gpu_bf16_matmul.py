"""Ignis bf16 matmul path (src/ignis/ops/bf16_matmul.rs) on the GPU: f32
operands converted, padded and transposed by the library's kernels, checked
against the oracle (bf16 RNE of both operands, then the reference CPU
product) -- bit-exact on integer inputs, within the acceptance tolerance
1e-2 * sqrt(K) * max|a| * max|b| on random inputs."""
import numpy as np
import pytest

import t0_gpu as t0
from t0_gpu import bf16_matmul as bm
from gpu_util import bf16, check_close, f32, tolerance
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

# (m, k, n): aligned, ragged in every dimension, tiny, skinny, tile-crossing
SHAPES = [(1, 1, 1), (3, 5, 7), (16, 64, 64), (17, 33, 65), (64, 128, 96), (100, 300, 260),
          (257, 129, 383), (8, 4096, 1024), (512, 1024, 768), (1031, 515, 777)]


@pytest.fixture(scope="module")
def rt():
    r = t0.GpuRuntime(0)
    yield r
    r.close()


def _rand(rng, shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def _down(rt, buf, shape):
    rt.wait_idle()
    out = buf.read(np.float32, int(np.prod(shape))).reshape(shape)
    buf.free()
    return out


def _tol(a, b, k):
    return tolerance(f32(bf16(a)), f32(bf16(b)), k)


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_forward_matches_oracle(rt, m, k, n):
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    x, w = _rand(rng, (m, k)), _rand(rng, (k, n), 0.5)
    dx_, dw_ = rt.upload(x), rt.upload(w)
    y = _down(rt, bm.matmul(rt, dx_, dw_, (m, k), (k, n)), (m, n))
    check_close(y, orc.bf16_matmul(x, w), _tol(x, w, k), f"forward {m}x{k}x{n}")
    dx_.free(), dw_.free()


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_backward_matches_oracle(rt, m, k, n):
    rng = np.random.default_rng(m * 5 + k * 11 + n)
    x, w, dy = _rand(rng, (m, k)), _rand(rng, (k, n)), _rand(rng, (m, n), 2.0)
    bx, bw, bdy = rt.upload(x), rt.upload(w), rt.upload(dy)
    gdx, gdw = bm.matmul_backward(rt, bdy, bx, bw, m, k, n)
    gdx, gdw = _down(rt, gdx, (m, k)), _down(rt, gdw, (k, n))
    check_close(gdx, orc.bf16_matmul_backward_data(dy, w), _tol(dy, w, n), f"dX {m}x{k}x{n}")
    check_close(gdw, orc.bf16_matmul_backward_weight(x, dy), _tol(x, dy, m), f"dW {m}x{k}x{n}")
    for b in (bx, bw, bdy):
        b.free()


@pytest.mark.parametrize("m,k,n", [(3, 5, 7), (33, 70, 45), (128, 256, 136), (200, 96, 301)])
def test_integer_inputs_exact(rt, m, k, n):
    """Small integers: exact in bf16 and in every f32 partial sum, so all three
    products must equal the int64 products bit for bit (catches a transposed
    operand, a wrong pad or a stale staging row)."""
    rng = np.random.default_rng(m + k + n)
    x = rng.integers(-8, 9, (m, k))
    w = rng.integers(-8, 9, (k, n))
    dy = rng.integers(-8, 9, (m, n))
    bx, bw, bdy = (rt.upload(v.astype(np.float32)) for v in (x, w, dy))
    y = _down(rt, bm.matmul(rt, bx, bw, (m, k), (k, n)), (m, n))
    gdx, gdw = bm.matmul_backward(rt, bdy, bx, bw, m, k, n)
    gdx, gdw = _down(rt, gdx, (m, k)), _down(rt, gdw, (k, n))
    assert np.array_equal(y.astype(np.int64), x @ w)
    assert np.array_equal(gdx.astype(np.int64), dy @ w.T)
    assert np.array_equal(gdw.astype(np.int64), x.T @ dy)
    for b in (bx, bw, bdy):
        b.free()


def test_operands_rounded_rne(rt):
    """Both operands are rounded to nearest even (bf16_matmul.rs:371-372):
    a tie rounds to the even neighbour; the sums are exact."""
    k = 32
    for v, want in [(1 + 2.0**-8, 1.0), (1 + 3 * 2.0**-8, 1 + 2.0**-6), (1 + 2.0**-8 + 2.0**-20, 1 + 2.0**-7)]:
        x = np.full((4, k), v, np.float32)
        w = np.ones((k, 8), np.float32)
        bx, bw = rt.upload(x), rt.upload(w)
        y = _down(rt, bm.matmul(rt, bx, bw, (4, k), (k, 8)), (4, 8))
        assert np.all(y == np.float32(k * want)), (v, y[0, 0])
        bx.free(), bw.free()


def test_backward_flags(rt):
    m, k, n = 40, 24, 56
    rng = np.random.default_rng(9)
    bx, bw, bdy = rt.upload(_rand(rng, (m, k))), rt.upload(_rand(rng, (k, n))), rt.upload(_rand(rng, (m, n)))
    dx, dw = bm.matmul_backward(rt, bdy, bx, bw, m, k, n, x_needs=False)
    assert dx is None and dw is not None
    dw.free()
    dx, dw = bm.matmul_backward(rt, bdy, bx, bw, m, k, n, w_needs=False)
    assert dx is not None and dw is None
    dx.free()
    for b in (bx, bw, bdy):
        b.free()


@pytest.mark.parametrize("m,k,n", [(1, 4096, 4096), (16, 64, 64), (50, 200, 120), (7, 13, 9)])
def test_with_wt_bf16(rt, m, k, n):
    """Pre-transposed bf16 weight WT[n,k] (bf16_matmul.rs:102-134); k % 8 != 0
    runs the generic kernel."""
    rng = np.random.default_rng(m + 3 * k + n)
    x = _rand(rng, (m, k))
    wt = bf16(_rand(rng, (n, k)))
    bx, bwt = rt.upload(x), rt.upload(wt)
    y = _down(rt, bm.matmul_with_wt_bf16(rt, bx, bwt, m, k, n), (m, n))
    check_close(y, orc.gemm_nt(bf16(x), wt), tolerance(f32(bf16(x)), f32(wt), k), f"with_wt {m}x{k}x{n}")
    bx.free(), bwt.free()


def test_repeated_calls_reuse_staging(rt):
    """Back-to-back calls of different sizes share the runtime's staging
    buffer (grown once); each result must still be right."""
    rng = np.random.default_rng(21)
    outs, refs = [], []
    for (m, k, n) in [(300, 700, 500), (40, 50, 60), (300, 700, 500), (1024, 1024, 1024)]:
        x, w = _rand(rng, (m, k)), _rand(rng, (k, n))
        bx, bw = rt.upload(x), rt.upload(w)
        outs.append((bm.matmul(rt, bx, bw, (m, k), (k, n)), (m, n), bx, bw))
        refs.append((orc.bf16_matmul(x, w), _tol(x, w, k)))
    for (y, shape, bx, bw), (ref, tol) in zip(outs, refs):
        check_close(_down(rt, y, shape), ref, tol, f"repeat {shape}")
        bx.free(), bw.free()


def test_shape_errors(rt):
    bx, bw = rt.upload(np.zeros((4, 8), np.float32)), rt.upload(np.zeros((8, 4), np.float32))
    with pytest.raises(ValueError, match="K mismatch"):
        bm.matmul(rt, bx, bw, (4, 8), (7, 4))
    with pytest.raises(ValueError):
        bm.matmul(rt, bx, bw, (4, 8, 1), (8, 4))
    with pytest.raises(ValueError):
        bm.matmul(rt, bx, bw, (40, 8), (8, 4))        # X buffer too small
    with pytest.raises(t0.T0Error, match="empty matmul"):     # the C ABI rejects m = 0 itself
        t0._check(t0.lib().t0_bf16_matmul(rt.h, bx.gpu_addr(), bw.gpu_addr(), bw.gpu_addr(), 0, 8, 4))
    bx.free(), bw.free()


def test_threads_share_one_runtime():
    """Four host threads drive one runtime at once: the staging matmul and the
    in-kernel split-K GEMM, with sizes that grow the runtime's staging buffer
    and split-K workspace while the other threads' calls are in flight.  Every
    result matches the oracle."""
    import threading
    r = t0.GpuRuntime(0)
    errors = []

    def worker(tid):
        try:
            rng = np.random.default_rng(100 + tid)
            for step in range(4):
                m, k, n = 64 * (step + 1) + tid, 256 * (step + 1), 96 * (step + 1) + 8 * tid
                x, w = _rand(rng, (m, k)), _rand(rng, (k, n), 0.5)
                bx, bw = r.upload(x), r.upload(w)
                y = bm.matmul(r, bx, bw, (m, k), (k, n))
                check_close(_down(r, y, (m, n)), orc.bf16_matmul(x, w), _tol(x, w, k), f"t{tid} matmul {m}x{k}x{n}")
                a16, b16 = bf16(x), bf16(w)
                da, db, dc = r.upload(a16), r.upload(b16), r.alloc(m * n * 2)
                cfg = t0.GemmConfig.tile_128x128_k64().copy(split_k=4, transpose=t0.NN, out_dtype=t0.OUT_BF16)
                r.gemm(da.gpu_addr(), db.gpu_addr(), dc.gpu_addr(), m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16,
                       cfg=cfg)
                r.wait_idle()
                got = f32(dc.read(np.uint16, m * n).reshape(m, n))
                check_close(got, orc.gemm_nn(a16, b16), tolerance(f32(a16), f32(b16), k), f"t{tid} split-K {m}x{n}x{k}")
                for b in (bx, bw, da, db, dc):
                    b.free()
        except Exception as e:          # reported by the main thread
            errors.append(f"thread {tid}: {e!r}")

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    r.close()
    assert not errors, errors

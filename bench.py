#!/usr/bin/env python3
"""bench.py -- the GEMM hot path on one MI355X (gfx950).

One JSON line on stdout.  The headline ``value`` is the bf16 GEMM
M = N = K = 4096 (NN, N(0,1) inputs rounded to bf16, fp32 accumulate, bf16
output; the compute-bound headline shape), in TFLOP/s: whole-job throughput of ``--steps``
back-to-back GEMMs with inputs resident in HBM, timed with HIP events on the
library's stream.  ``roofline`` relates the GEMM kernel's average launch
duration to MI355X's dense bf16 MFMA peak (2516.6 TFLOP/s); ``cpu_baseline``
times the reference's CPU matmul (restated in oracle/, single thread) on a
row slice of the same workload.  ``extras`` carries the other workloads
of the path: skinny bf16 GEMM (HBM), W4A16 decode (HBM, the metric's second
half), W4A16 prefill (MFMA), each with its own roofline, and the Ignis
f32 matmul forward / backward at 4096^3 (staging conversions + GEMM); the HBM-bound
shapes rotate 12 weight copies (> 256 MB) so the Infinity Cache cannot
serve them, and are timed as graph replays of 12 launches.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "rust-gpu_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

import t0_gpu as t0  # noqa: E402

METRIC = "bf16 GEMM TFLOPS @4096³ (% MFMA peak); W4A16 decode HBM GB/s (% peak)"
PEAK_TFLOPS = 2516.6    # 256 CU x 2.4 GHz x 4096 dense bf16 FLOP/clk/CU
PEAK_GBS = 8000.0       # HBM3E
ROTATE = 12


def bf16_rne(x: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((b + (((b >> 16) & 1) + 0x7FFF)) >> 16).astype(np.uint16)


class Timer:
    def __init__(self, rt):
        self.rt, self.e0, self.e1 = rt, t0.Event(), t0.Event()

    def run(self, fn, steps: int, warmup: int, warm_ms: float = 250.0) -> float:
        """ms per call of fn over `steps` calls after `warmup` untimed ones
        (repeated until at least warm_ms of GPU work has run, so clocks settle)."""
        t_end = time.perf_counter() + warm_ms / 1e3
        while True:
            for _ in range(max(1, warmup)):
                fn()
            self.rt.wait_idle()
            if time.perf_counter() >= t_end:
                break
        self.e0.record(self.rt)
        for _ in range(steps):
            fn()
        self.e1.record(self.rt)
        self.e1.synchronize()
        self.rt.wait_idle()
        return self.e0.elapsed_ms(self.e1) / steps


USE_GRAPHS = True


def rotate_timed(rt, one, steps, warmup) -> float:
    """ms per launch of one(i) over ROTATE buffer sets: the ROTATE launches are
    captured in a HIP graph and replayed (launch overhead stays off the GPU
    timeline), or issued directly with --no-graph (for tracing tools)."""
    if USE_GRAPHS:
        g = rt.capture(lambda: [one(i) for i in range(ROTATE)])
        return Timer(rt).run(g.launch, steps, warmup) / ROTATE

    def all_sets():
        for i in range(ROTATE):
            one(i)
    return Timer(rt).run(all_sets, steps, warmup) / ROTATE


def bench_copy(rt, steps, warmup, rng, tr):
    """Calibration: t0k_copy_b128 over 256 MiB (bytes known exactly)."""
    nbytes = 256 << 20
    src, dst = rt.alloc(nbytes), rt.alloc(nbytes)
    ms = Timer(rt).run(lambda: rt.copy_device(src.gpu_addr(), dst.gpu_addr(), nbytes), steps, warmup)
    src.free()
    dst.free()
    return {"workload": "copy 256 MiB", "kernel": "t0k_copy_b128", "read_bytes": nbytes, "write_bytes": nbytes,
            "us_per_launch": round(ms * 1e3, 3), "gbs": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}


def load_traffic():
    p = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(p):
        return {}
    with open(p) as f:
        return json.load(f)


def roofline(bound, achieved, peak, unit, traffic=None):
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


def traffic_of(tr, key):
    e = tr.get(key)
    return int(e["traffic_bytes"]) if e and e.get("traffic_bytes") else None


# ------------------------------------------------------------- workloads --

def bench_gemm_4096(rt, steps, warmup, rng, tr):
    m = n = k = 4096
    a = bf16_rne(rng.standard_normal((m, k), dtype=np.float32))
    b = bf16_rne(rng.standard_normal((k, n), dtype=np.float32))
    da, db = rt.upload(a), rt.upload(b)
    dc = rt.alloc(m * n * 2)
    cfg = rt.gemm_select(m, n, k, t0.NN, t0.OUT_BF16)

    def step():
        rt.gemm(da.gpu_addr(), db.gpu_addr(), dc.gpu_addr(), m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16,
                cfg=cfg)

    ms = Timer(rt).run(step, steps, warmup)
    flops = 2.0 * m * n * k
    tflops = flops / (ms * 1e-3) / 1e12
    for buf in (da, db, dc):
        buf.free()
    return {"ms": ms, "tflops": tflops, "kernel": cfg.name(), "a": a, "b": b,
            "roofline": roofline("mfma", tflops, PEAK_TFLOPS, "TFLOP/s", traffic_of(tr, "gemm_4096_nn_bf16"))}


def bench_skinny(rt, steps, warmup, rng, tr):
    m, n, k = 128, 4096, 4096
    a = bf16_rne(rng.normal(0, 0.02, (m, k)).astype(np.float32))
    bs = [rt.upload(bf16_rne(rng.normal(0, 0.02, (k, n)).astype(np.float32))) for _ in range(ROTATE)]
    da = rt.upload(a)
    dc = rt.alloc(m * n * 2)
    cfg = rt.gemm_select(m, n, k, t0.NN, t0.OUT_BF16)

    def one(i):
        rt.gemm(da.gpu_addr(), bs[i].gpu_addr(), dc.gpu_addr(), m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16,
                cfg=cfg)

    one(0)
    rt.wait_idle()
    ms = rotate_timed(rt, one, steps, warmup)
    bytes_alg = m * k * 2 + k * n * 2 + m * n * 2
    gbs = bytes_alg / (ms * 1e-3) / 1e9
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    for buf in bs + [da, dc]:
        buf.free()
    return {"workload": "skinny bf16 GEMM M=128 N=4096 K=4096 NN, bf16 out", "kernel": cfg.name(),
            "us_per_launch": round(ms * 1e3, 3), "tflops": round(tflops, 2), "gbs": round(gbs, 1),
            "roofline": roofline("hbm", gbs, PEAK_GBS, "GB/s", traffic_of(tr, "gemm_skinny_128x4096x4096"))}


def _w4_operands(rng, n, k, gs, per_group_zeros):
    G = k // gs
    q = rng.integers(0, 16, size=(n, k // 8, 8), dtype=np.uint32)
    qw = np.zeros((n, k // 8), np.uint32)
    for i in range(8):
        qw |= q[:, :, i] << np.uint32(4 * i)
    s = bf16_rne(rng.uniform(0.005, 0.02, (G, n)).astype(np.float32))
    zw = None
    if per_group_zeros:
        z = rng.integers(0, 16, size=(G, n // 8, 8), dtype=np.uint32)
        zw = np.zeros((G, n // 8), np.uint32)
        for i in range(8):
            zw |= z[:, :, i] << np.uint32(4 * i)
    return qw, s, zw


def bench_decode(rt, steps, warmup, rng, tr):
    m, n, k, gs = 16, 11008, 4096, 128
    a = rt.upload(bf16_rne(rng.standard_normal((m, k), dtype=np.float32)))
    sets = []
    for _ in range(ROTATE):
        qw, s, _ = _w4_operands(rng, n, k, gs, False)
        sets.append((rt.upload(qw), rt.upload(s)))
    dc = rt.alloc(m * n * 2)

    def one(i):
        rt.w4a16(a.gpu_addr(), sets[i][0].gpu_addr(), sets[i][1].gpu_addr(), 0, dc.gpu_addr(), m, n, k,
                 group_size=gs, zero_const=8)

    plan = rt.w4a16_plan(a.gpu_addr(), sets[0][0].gpu_addr(), sets[0][1].gpu_addr(), 0, dc.gpu_addr(), m, n, k,
                         group_size=gs, zero_const=8)
    one(0)
    rt.wait_idle()
    ms = rotate_timed(rt, one, steps, warmup)
    # algorithmic bytes: W nibbles + bf16 scales + A + C (constant z not stored)
    bytes_alg = n * k // 2 + (k // gs) * n * 2 + m * k * 2 + m * n * 2
    gbs = bytes_alg / (ms * 1e-3) / 1e9
    for s in sets:
        for buf in s:
            buf.free()
    a.free()
    dc.free()
    return {"workload": "W4A16 decode M=16 K=4096 N=11008, g=128, z=8, bf16 out", "kernel": plan[0],
            "split_k": plan[1], "us_per_launch": round(ms * 1e3, 3), "gbs": round(gbs, 1),
            "bytes_per_launch": bytes_alg,
            "roofline": roofline("hbm", gbs, PEAK_GBS, "GB/s", traffic_of(tr, "w4a16_decode_16x4096x11008"))}


def bench_prefill(rt, steps, warmup, rng, tr):
    m, n, k, gs = 4096, 14336, 4096, 128
    a = rt.upload(bf16_rne(rng.standard_normal((m, k), dtype=np.float32)))
    qw, s, zw = _w4_operands(rng, n, k, gs, True)
    dq, ds, dz = rt.upload(qw), rt.upload(s), rt.upload(zw)
    dc = rt.alloc(m * n * 2)

    def step():
        rt.w4a16(a.gpu_addr(), dq.gpu_addr(), ds.gpu_addr(), dz.gpu_addr(), dc.gpu_addr(), m, n, k, group_size=gs,
                 zero_const=0)

    plan = rt.w4a16_plan(a.gpu_addr(), dq.gpu_addr(), ds.gpu_addr(), dz.gpu_addr(), dc.gpu_addr(), m, n, k,
                         group_size=gs, zero_const=0)
    ms = Timer(rt).run(step, max(5, steps // 4), max(2, warmup // 2))
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    for buf in (a, dq, ds, dz, dc):
        buf.free()
    return {"workload": "W4A16 prefill M=4096 K=4096 N=14336, g=128, per-group z, bf16 out", "kernel": plan[0],
            "ms_per_launch": round(ms, 4), "tflops": round(tflops, 2),
            "roofline": roofline("mfma", tflops, PEAK_TFLOPS, "TFLOP/s", traffic_of(tr, "w4a16_prefill_4096x4096x14336"))}


def bench_ignis(rt, steps, warmup, rng, tr):
    """Ignis bf16 matmul (f32 X[M,K], W[K,N] -> f32 Y) at M=N=K=4096: forward
    (two staging conversions + NN GEMM) and backward (dX = dY W^T and
    dW = X^T dY, four conversions + two GEMMs)."""
    m = n = k = 4096
    x = rt.upload(rng.standard_normal((m, k), dtype=np.float32))
    w = rt.upload(rng.standard_normal((k, n), dtype=np.float32))
    dy = rt.upload(rng.standard_normal((m, n), dtype=np.float32))
    y, dx, dw = rt.alloc(m * n * 4), rt.alloc(m * k * 4), rt.alloc(k * n * 4)
    L = t0.lib()

    def fwd():
        t0._check(L.t0_bf16_matmul(rt.h, x.gpu_addr(), w.gpu_addr(), y.gpu_addr(), m, k, n))

    def bwd():
        t0._check(L.t0_bf16_matmul_backward_data(rt.h, dy.gpu_addr(), w.gpu_addr(), dx.gpu_addr(), m, k, n))
        t0._check(L.t0_bf16_matmul_backward_weight(rt.h, x.gpu_addr(), dy.gpu_addr(), dw.gpu_addr(), m, k, n))

    ms_f = Timer(rt).run(fwd, steps, warmup)
    ms_b = Timer(rt).run(bwd, steps, warmup)
    for buf in (x, w, dy, y, dx, dw):
        buf.free()
    fl = 2.0 * m * n * k
    return {"workload": "Ignis bf16 matmul M=N=K=4096, f32 in / f32 out", "us_forward": round(ms_f * 1e3, 2),
            "tflops_forward": round(fl / (ms_f * 1e-3) / 1e12, 1), "us_backward": round(ms_b * 1e3, 2),
            "tflops_backward": round(2 * fl / (ms_b * 1e-3) / 1e12, 1)}


def bench_norm_decode(rt, steps, warmup, rng, tr):
    """One decode token through residual add + RMSNorm + the W4A16 projection
    (M=1, K=4096, N=11008, g=128, z=8): the fused decode kernel against the
    two-kernel path (RMSNorm to bf16, then the decode GEMM), 12 rotated
    weight sets as graph replays."""
    from t0_gpu._ffi import RmsNormDescC, W4A16DescC
    import ctypes as C
    m, n, k, gs = 1, 11008, 4096, 128
    res = rt.upload(rng.standard_normal((m, k), dtype=np.float32))
    hid = rt.upload(rng.standard_normal((m, k), dtype=np.float32))
    gam = rt.upload(rng.uniform(0.5, 1.5, k).astype(np.float32))
    x2 = rt.alloc(4 * k)
    a16 = rt.alloc(2 * k)
    sets = []
    for _ in range(ROTATE):
        qw, s, _ = _w4_operands(rng, n, k, gs, False)
        sets.append((rt.upload(qw), rt.upload(s)))
    dc = rt.alloc(m * n * 2)
    L = t0.lib()
    nd = RmsNormDescC(residual=res.gpu_addr(), hidden=hid.gpu_addr(), gamma=gam.gpu_addr(), x2_out=x2.gpu_addr(),
                      eps=1e-5)

    def fused(i):
        d = W4A16DescC(a=0, qweight=sets[i][0].gpu_addr(), scales=sets[i][1].gpu_addr(), zeros=0, c=dc.gpu_addr(),
                       m=m, n=n, k=k, group_size=gs, zero_const=8)
        t0._check(L.t0_rmsnorm_w4a16(rt.h, C.byref(d), C.byref(nd)))

    def separate(i):
        t0._check(L.t0_rmsnorm(rt.h, res.gpu_addr(), hid.gpu_addr(), gam.gpu_addr(), a16.gpu_addr(), x2.gpu_addr(),
                               1, k, k, 1e-5, 1))
        rt.w4a16(a16.gpu_addr(), sets[i][0].gpu_addr(), sets[i][1].gpu_addr(), 0, dc.gpu_addr(), m, n, k,
                 group_size=gs, zero_const=8)

    fused(0)
    separate(0)
    rt.wait_idle()
    ms_f = rotate_timed(rt, fused, steps, warmup)
    ms_s = rotate_timed(rt, separate, steps, warmup)
    for buf in [res, hid, gam, x2, a16, dc] + [b for st in sets for b in st]:
        buf.free()
    return {"workload": "decode token: residual + RMSNorm + W4A16 M=1 K=4096 N=11008, g=128, z=8",
            "kernel": "t0k_w4a16_decode_norm_t3", "us_fused": round(ms_f * 1e3, 3),
            "us_two_kernels": round(ms_s * 1e3, 3)}


def cpu_baseline(a, b, rows: int):
    """The reference CPU matmul (oracle restatement, one thread) on rows
    [0, rows) of the 4096^3 product, scaled to the whole product."""
    from oracle import oracle as orc   # checker-side code: the CPU baseline leg only
    m, k = a.shape
    n = b.shape[1]
    t = time.perf_counter()
    orc.gemm_rows(a, b, "nn", 0, rows)
    dt = time.perf_counter() - t
    tflops = 2.0 * rows * n * k / dt / 1e12
    return {"value": tflops, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"rows 0-{rows - 1} of the 4096^3 NN GEMM ({2.0 * rows * n * k / 1e9:.2f} GFLOP, "
                      f"{dt:.1f} s), sequential-f32 no-FMA loop of examples/test_gemm_correctness.rs:28-42; "
                      f"the naive loop's cost is linear in rows, so the rate holds for all {m} rows",
            "host": platform.processor() or platform.machine(), "nproc": os.cpu_count()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-rows", type=int, default=256)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="issue rotated launches directly (for tracers)")
    ap.add_argument("--only", choices=["gemm4096", "skinny", "decode", "prefill", "ignis", "norm_decode", "copy"],
                    default=None,
                    help="run one workload (for counter collection)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU; --gpus must be 1 (the path would shard by N or K "
              "across GPUs)", file=sys.stderr)
        sys.exit(2)

    global USE_GRAPHS
    USE_GRAPHS = not args.no_graph
    rng = np.random.default_rng(20261201)
    tr = load_traffic()
    rt = t0.GpuRuntime(0)
    info = rt.device_info()

    if args.only:
        fn = {"gemm4096": bench_gemm_4096, "skinny": bench_skinny, "decode": bench_decode,
              "prefill": bench_prefill, "ignis": bench_ignis, "norm_decode": bench_norm_decode,
              "copy": bench_copy}[args.only]
        r = fn(rt, args.steps, args.warmup, rng, tr)
        r.pop("a", None)
        r.pop("b", None)
        print(json.dumps({"only": args.only, **{k: v for k, v in r.items()}}, default=float), flush=True)
        rt.close()
        return

    head = bench_gemm_4096(rt, args.steps, args.warmup, rng, tr)
    print(f"# gemm 4096^3 NN bf16: {head['ms'] * 1e3:.1f} us/launch, {head['tflops']:.1f} TFLOP/s "
          f"({head['kernel']})", file=sys.stderr, flush=True)
    extras = {}
    if not args.no_extras:
        for name, fn in (("skinny", bench_skinny), ("w4a16_decode", bench_decode), ("w4a16_prefill", bench_prefill),
                         ("ignis_matmul", bench_ignis), ("norm_decode", bench_norm_decode)):
            extras[name] = fn(rt, args.steps, args.warmup, rng, tr)
            print(f"# {name}: {json.dumps(extras[name])}", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(head["a"], head["b"], args.cpu_rows)
    rt.close()

    line = {
        "metric": METRIC,
        "value": round(head["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) rounded to bf16 (numpy seed 20261201), inputs resident in HBM",
        "config": {"workload": "bf16 GEMM M=N=K=4096, A[M,K] . B[K,N] row-major (NN), fp32 accumulate, bf16 out",
                   "m": 4096, "n": 4096, "k": 4096, "layout": "NN", "out": "bf16", "kernel": head["kernel"],
                   "device": info},
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

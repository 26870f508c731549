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
PARITY_ROWS = 64        # output rows of the 4096-row workloads checked against the oracle


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

    def per_call(self, fn, n: int) -> list:
        """ms of each of n calls, an event pair around every call (the GPU is
        already warm from run()); the event records themselves add a little."""
        evs = [t0.Event() for _ in range(n + 1)]
        evs[0].record(self.rt)
        for i in range(n):
            fn()
            evs[i + 1].record(self.rt)
        evs[-1].synchronize()
        return [evs[i].elapsed_ms(evs[i + 1]) for i in range(n)]


USE_GRAPHS = True


def rotate_timed(rt, one, steps, warmup):
    """(mean, median) ms per launch of one(i) over ROTATE buffer sets: the
    ROTATE launches are captured in a HIP graph and replayed (launch overhead
    stays off the GPU timeline), or issued directly with --no-graph (for
    tracing tools).  The median is over per-replay times."""
    if USE_GRAPHS:
        g = rt.capture(lambda: [one(i) for i in range(ROTATE)])
        fn = g.launch
    else:
        def fn():
            for i in range(ROTATE):
                one(i)
    tm = Timer(rt)
    mean = tm.run(fn, steps, warmup) / ROTATE
    med = float(np.median(tm.per_call(fn, max(10, steps)))) / ROTATE
    return mean, med


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def bench_copy(rt, steps, warmup, rng, tr):
    """Calibration: t0k_copy_b128 over 256 MiB (bytes known exactly)."""
    nbytes = 256 << 20
    src, dst = rt.alloc(nbytes), rt.alloc(nbytes)
    ms = Timer(rt).run(lambda: rt.copy_device(src.gpu_addr(), dst.gpu_addr(), nbytes), steps, warmup)
    src.free()
    dst.free()
    return {"workload": "copy 256 MiB", "kernel": "t0k_copy_b128", "read_bytes": nbytes, "write_bytes": nbytes,
            "us_per_launch": round(ms * 1e3, 3), "gbs": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}


def bench_floor(rt, steps, warmup, rng, tr):
    """Floors of the W4A16 decode (16x4096x11008): reading its 22.5 MB weight
    array once (t0k_stream_read, 12 rotated copies so the Infinity Cache
    cannot serve them) and an empty launch, for the decode's launch shape
    (256 x 1024) and smaller workgroups; graph replays like the decode.
    Then the GEMM's ceilings (bench_ceilings)."""
    n, k = 11008, 4096
    wbytes = n * k // 2
    sets = [rt.alloc(wbytes) for _ in range(ROTATE)]
    for b in sets:
        rt.memset(b.gpu_addr(), 0x5A, wbytes)
    sink = rt.alloc(65536 * 4)
    out = {"workload": "decode floors: read 22544384 B once / empty launch", "bytes": wbytes}
    for wgs, thr in ((256, 1024), (256, 512), (256, 256), (512, 256), (1024, 256)):
        ms_r, med_r = rotate_timed(rt, lambda i: rt.floor_stream_read(sets[i].gpu_addr(), wbytes, sink.gpu_addr(),
                                                                       wgs, thr), steps, warmup)
        ms_e, med_e = rotate_timed(rt, lambda i: rt.floor_empty(wgs, thr), steps, warmup)
        out[f"{wgs}x{thr}"] = {"us_read": round(ms_r * 1e3, 3), "us_read_median": round(med_r * 1e3, 3),
                               "gbs_read": round(wbytes / (ms_r * 1e-3) / 1e9, 1), "us_empty": round(ms_e * 1e3, 3),
                               "us_empty_median": round(med_e * 1e3, 3)}
    for b in sets + [sink]:
        b.free()
    out.update(bench_ceilings(rt, steps, warmup, rng))
    return out


def _clock_records(buf, wgs):
    """(median shader MHz, median workgroup span in us, median workgroup
    shader cycles) from the 4-u64 records of the floor kernels."""
    r = buf.read(np.uint64, 4 * wgs).reshape(wgs, 4).astype(np.float64)
    real, shader = r[:, 1] - r[:, 0], r[:, 3] - r[:, 2]
    return float(np.median(shader / real * 100.0)), float(np.median(real / 100.0)), float(np.median(shader))


def bench_ceilings(rt, steps, warmup, rng):
    """Ceilings of the 4096^3 GEMM on this part: MFMA issue alone at the
    8-wave 256x256 tile's count (2048 per wave, 4096 per SIMD = 131072
    shader cycles) with N(0,1) bf16 operands and with zeros (the data sets
    the power the MFMAs draw, hence the clock); and the LDS port rates per
    CU (ds_read_b128, the NN operand's ds_read_b64_tr_b16, global->LDS DMA
    from L2) at 1 and 2 waves per SIMD."""
    wgs = 256
    ops = [rt.upload(bf16_rne(rng.standard_normal(wgs * 512 * 96, dtype=np.float32))), rt.alloc(wgs * 512 * 192)]
    rec = rt.alloc(wgs * (32 + 4096))
    out = {}
    for name, src in (("mfma_issue_normal", ops[0]), ("mfma_issue_zeros", ops[1])):
        f = lambda: rt.floor_mfma(src.gpu_addr(), rec.gpu_addr(), wgs, 2048)
        ms = Timer(rt).run(f, steps, warmup)
        f()
        rt.wait_idle()
        mhz, span, cyc = _clock_records(rec, wgs)
        out[name] = {"us_per_launch": round(ms * 1e3, 2), "sclk_mhz": round(mhz, 1), "workgroup_us": round(span, 2),
                     "workgroup_cycles": round(cyc), "mfma_cycles_per_simd": 4096 * 32}
    src64 = rt.alloc(65536)
    rates = {}
    for mode, name, lane_bytes in ((0, "ds_read_b128", 128), (1, "ds_read_b64_tr_b16", 64), (2, "dma_to_lds", 128)):
        for threads in (256, 512):
            rounds = 2000
            rt.floor_lds(mode, src64.gpu_addr(), rec.gpu_addr(), wgs, threads, rounds)
            rt.wait_idle()
            mhz, span, cyc = _clock_records(rec, wgs)
            rates[f"{name}_{threads // 256}_wave_per_simd"] = round(threads * lane_bytes * rounds / cyc, 1)
    out["lds_bytes_per_clk_per_cu"] = rates
    for b in ops + [rec, src64]:
        b.free()
    out["gemm_4096_zero_operands"] = bench_gemm_zero_operands(rt, steps, warmup)
    out["w4a16_prefill_zero_activations"] = bench_prefill_zero_activations(rt, steps, warmup, rng)
    return out


def bench_prefill_zero_activations(rt, steps, warmup, rng):
    """Not a BASELINE workload: the W4A16 prefill (4096x4096x14336, the
    BASELINE weights, scales and zero points) timed with N(0,1) activations
    and, on the same weights and kernel, with all-zero activations.  Only the
    MFMAs' operand values differ, so the gap is what their data-dependent
    power costs the prefill."""
    m, n, k, gs = 4096, 14336, 4096, 128
    qw, s, zw = _w4_operands(rng, n, k, gs, True)
    dq, ds, dz = rt.upload(qw), rt.upload(s), rt.upload(zw)
    dc = rt.alloc(m * n * 2)
    a_n = rt.upload(bf16_rne(rng.standard_normal((m, k), dtype=np.float32)))
    a_z = rt.alloc(m * k * 2)
    rt.memset(a_z.gpu_addr(), 0, m * k * 2)
    out = {}
    for name, a in (("normal", a_n), ("zeros", a_z)):
        def step():
            rt.w4a16(a.gpu_addr(), dq.gpu_addr(), ds.gpu_addr(), dz.gpu_addr(), dc.gpu_addr(), m, n, k,
                     group_size=gs, zero_const=0)
        ms = Timer(rt).run(step, max(5, steps // 4), max(2, warmup // 2))
        tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        out[name] = {"us_per_launch": round(ms * 1e3, 1), "tflops": round(tflops, 1),
                     "frac_of_peak": round(tflops / PEAK_TFLOPS, 4)}
    for buf in (dq, ds, dz, dc, a_n, a_z):
        buf.free()
    return out


def bench_gemm_zero_operands(rt, steps, warmup):
    """Not a BASELINE workload: the headline GEMM (the same config, kernel and
    schedule) on all-zero A and B.  Only the operand values differ from the
    N(0,1) run, so the gap in clock and time is what the MFMAs' data-dependent
    power costs the GEMM."""
    m = n = k = 4096
    da, db, dc = rt.alloc(m * k * 2), rt.alloc(k * n * 2), rt.alloc(m * n * 2)
    rt.memset(da.gpu_addr(), 0, m * k * 2)
    rt.memset(db.gpu_addr(), 0, k * n * 2)
    cfg = rt.gemm_select(m, n, k, t0.NN, t0.OUT_BF16)

    def step():
        rt.gemm(da.gpu_addr(), db.gpu_addr(), dc.gpu_addr(), m, n, k, transpose=t0.NN, out_dtype=t0.OUT_BF16,
                cfg=cfg)

    ms = Timer(rt).run(step, steps, warmup)
    probes = [rt.gemm_clock_probe(da.gpu_addr(), db.gpu_addr(), dc.gpu_addr(), m, n, k, transpose=t0.NN,
                                  out_dtype=t0.OUT_BF16, cfg=cfg) for _ in range(5)]
    for buf in (da, db, dc):
        buf.free()
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    return {"kernel": cfg.name(), "us_per_launch": round(ms * 1e3, 2), "tflops": round(tflops, 1),
            "frac_of_peak": round(tflops / PEAK_TFLOPS, 4),
            "sclk_mhz": round(float(np.median([p[0] for p in probes])), 1),
            "workgroup_cycles": round(float(np.median([p[2] for p in probes])))}


TILE_SHAPES = [(m, n, k) for m in (32, 128, 512, 1024, 2048, 4096)
               for (n, k) in ((4096, 4096), (11008, 4096), (4096, 11008), (14336, 4096))] + \
              [(4096, 1024, 4096), (3072, 8192, 4096), (384, 4096, 4096), (16, 4096, 4096)] + \
              [(m, n, 4096) for m in (64, 256) for n in (4096, 11008, 14336)] + \
              [(1, 4096, 4096), (1, 11008, 4096), (1, 4096, 14336), (1, 8192, 28672), (16, 4096, 14336),
               (128, 4096, 14336), (1024, 4096, 14336), (256, 8192, 28672)]


def bench_tiles(rt, steps, warmup, rng, tr):
    """Evidence for the tile / split-K selection (t0_auto_schedule_gemm,
    src/t0/cost_model.rs:464-535): on LLM shapes (NN, N(0,1) bf16 operands,
    bf16 out), every ranked candidate is timed with the weight operand B
    rotated through copies that exceed the 256 MB Infinity Cache (read cold
    from HBM, as in inference), as graph replays.  Per shape: the pick
    (rank 0) and the measured best, their predicted and measured times, the
    regret pick / best and the best's rank in the predicted order."""
    rows = []
    for (m, n, k) in TILE_SHAPES:
        cands = t0.auto_schedule_gemm(m, n, k, t0.NN, t0.OUT_BF16)
        rot = max(2, -(-300_000_000 // (k * n * 2)))
        a = rt.upload(bf16_rne(rng.standard_normal((m, k), dtype=np.float32)))
        bsets = [rt.upload(bf16_rne(rng.standard_normal((k, n), dtype=np.float32))) for _ in range(rot)]
        c = rt.alloc(m * n * 2)
        meas = []
        for cfg, est in cands:
            def one(i, cfg=cfg):
                rt.gemm(a.gpu_addr(), bsets[i % rot].gpu_addr(), c.gpu_addr(), m, n, k, transpose=t0.NN,
                        out_dtype=t0.OUT_BF16, cfg=cfg)
            one(0)
            rt.wait_idle()
            g = rt.capture(lambda: [one(i) for i in range(rot)])
            tm = Timer(rt)
            ms = tm.run(g.launch, 5, 2, warm_ms=5.0) / rot
            g.destroy()
            meas.append(ms * 1e3)
        for buf in bsets + [a, c]:
            buf.free()
        best = int(np.argmin(meas))
        order = sorted(range(len(cands)), key=lambda i: cands[i][1])
        rows.append({"shape": [m, n, k], "candidates": len(cands),
                     "pick": f"{cands[0][0].name()} w{cands[0][0].wg_size // 64}",
                     "pick_pred_us": round(cands[0][1], 2), "pick_us": round(meas[0], 2),
                     "best": f"{cands[best][0].name()} w{cands[best][0].wg_size // 64}",
                     "best_pred_us": round(cands[best][1], 2), "best_us": round(meas[best], 2),
                     "regret": round(meas[0] / meas[best], 3), "best_rank_predicted": order.index(best),
                     "median_abs_pred_err": round(float(np.median([abs(cands[i][1] / meas[i] - 1)
                                                                   for i in range(len(cands))])), 3),
                     "all": [[f"{cfg.name()} w{cfg.wg_size // 64}", round(est, 2), round(t, 2)]
                             for (cfg, est), t in zip(cands, meas)]})
        print(f"# tiles {m}x{n}x{k}: pick {rows[-1]['pick']} {meas[0]:.1f} us, best {rows[-1]['best']} "
              f"{meas[best]:.1f} us (regret {rows[-1]['regret']})", file=sys.stderr, flush=True)
    reg = [r["regret"] for r in rows]
    return {"workload": "tile / split-K selection, NN bf16 out, B cold", "shapes": rows,
            "regret_median": round(float(np.median(reg)), 3), "regret_max": round(float(np.max(reg)), 3),
            "picks_within_3pct": sum(r <= 1.03 for r in reg), "shape_count": len(rows)}


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

    tm = Timer(rt)
    ms = tm.run(step, steps, warmup)
    per = tm.per_call(step, max(100, steps))
    # measured shader clock under this load: per-workgroup s_memtime against
    # the 100 MHz real-time clock, median over workgroups, over 5 launches
    probes = [rt.gemm_clock_probe(da.gpu_addr(), db.gpu_addr(), dc.gpu_addr(), m, n, k, transpose=t0.NN,
                                  out_dtype=t0.OUT_BF16, cfg=cfg) for _ in range(5)]
    sclk = float(np.median([p[0] for p in probes]))
    span = float(np.median([p[1] for p in probes]))
    wg_cycles = float(np.median([p[2] for p in probes]))
    flops = 2.0 * m * n * k
    tflops = flops / (ms * 1e-3) / 1e12
    step()
    rt.wait_idle()
    gpu_rows = dc.read(np.uint16, PARITY_ROWS * n).reshape(PARITY_ROWS, n)
    for buf in (da, db, dc):
        buf.free()
    rf = roofline("mfma", tflops, PEAK_TFLOPS, "TFLOP/s", traffic_of(tr, "gemm_4096_nn_bf16"))
    rf["sclk_mhz_measured"] = round(sclk, 1)
    # the shader cycles a workgroup takes (MFMA issue alone: 131072 per SIMD)
    rf["workgroup_cycles_measured"] = round(wg_cycles)
    rf["peak_at_measured_sclk"] = round(PEAK_TFLOPS * sclk / 2400.0, 1)
    rf["frac_at_measured_sclk"] = round(tflops / (PEAK_TFLOPS * sclk / 2400.0), 4)
    return {"ms": ms, "ms_median_per_launch": float(np.median(per)), "tflops": tflops, "kernel": cfg.name(),
            "a": a, "b": b, "gpu_rows": gpu_rows, "sclk_mhz": sclk, "workgroup_span_us": span, "roofline": rf}


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
    b0 = bs[0].read(np.uint16, k * n).reshape(k, n)
    ms, med = rotate_timed(rt, one, steps, warmup)
    bytes_alg = m * k * 2 + k * n * 2 + m * n * 2
    gbs = bytes_alg / (ms * 1e-3) / 1e9
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    one(0)
    rt.wait_idle()
    out0 = dc.read(np.uint16, m * n).reshape(m, n)
    # Operand read floors: the pick's grid (and two other tilings) with only the
    # operand slices moving to LDS -- A, B, both -- on the same rotated B sets,
    # and an empty launch of the pick's grid.
    floors = {}
    for label, c in (("pick", cfg), ("128x64_split4", cfg.copy(tile_m=128, tile_n=64, split_k=4)),
                     ("128x128_split8", cfg.copy(tile_m=128, tile_n=128, split_k=8))):
        row = {"tiling": f"{c.tile_m}x{c.tile_n} split {max(1, c.split_k)}"}
        for mode, key in ((1, "A"), (2, "B"), (3, "A+B")):
            ms_f, _ = rotate_timed(rt, lambda i: rt.floor_tile_read(da.gpu_addr(), bs[i].gpu_addr(), m, n, k,
                                                                     transpose=t0.NN, mode=mode, cfg=c),
                                   steps, warmup)
            row[f"us_{key}"] = round(ms_f * 1e3, 3)
        floors[label] = row
    wgs = (m // cfg.tile_m) * (n // cfg.tile_n) * max(1, cfg.split_k)
    ms_e, _ = rotate_timed(rt, lambda i: rt.floor_empty(wgs, cfg.wg_size), steps, warmup)
    floors["pick"]["us_empty_launch"] = round(ms_e * 1e3, 3)
    for buf in bs + [da, dc]:
        buf.free()
    return {"workload": "skinny bf16 GEMM M=128 N=4096 K=4096 NN, bf16 out", "kernel": cfg.name(),
            "us_per_launch": round(ms * 1e3, 3), "us_median_per_launch": round(med * 1e3, 3),
            "tflops": round(tflops, 2), "gbs": round(gbs, 1), "_host": (a, b0, out0),
            "operand_read_floor": floors,
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
    a_h = bf16_rne(rng.standard_normal((m, k), dtype=np.float32))
    a = rt.upload(a_h)
    sets, host0 = [], None
    for _ in range(ROTATE):
        qw, s, _ = _w4_operands(rng, n, k, gs, False)
        host0 = host0 or (qw, s)
        sets.append((rt.upload(qw), rt.upload(s)))
    dc = rt.alloc(m * n * 2)

    def one(i):
        rt.w4a16(a.gpu_addr(), sets[i][0].gpu_addr(), sets[i][1].gpu_addr(), 0, dc.gpu_addr(), m, n, k,
                 group_size=gs, zero_const=8)

    plan = rt.w4a16_plan(a.gpu_addr(), sets[0][0].gpu_addr(), sets[0][1].gpu_addr(), 0, dc.gpu_addr(), m, n, k,
                         group_size=gs, zero_const=8)
    one(0)
    rt.wait_idle()
    ms, med = rotate_timed(rt, one, steps, warmup)
    # algorithmic bytes: W nibbles + bf16 scales + A + C (constant z not stored)
    bytes_alg = n * k // 2 + (k // gs) * n * 2 + m * k * 2 + m * n * 2
    gbs = bytes_alg / (ms * 1e-3) / 1e9
    one(0)
    rt.wait_idle()
    out0 = dc.read(np.uint16, m * n).reshape(m, n)
    for s in sets:
        for buf in s:
            buf.free()
    a.free()
    dc.free()
    return {"workload": "W4A16 decode M=16 K=4096 N=11008, g=128, z=8, bf16 out",
            "weight_layout": "GPTQ: qweight [N][K/8] u32, 8 nibbles along K; scales [K/128][N] bf16",
            "kernel": plan[0],
            "split_k": plan[1], "us_per_launch": round(ms * 1e3, 3), "us_median_per_launch": round(med * 1e3, 3),
            "gbs": round(gbs, 1), "bytes_per_launch": bytes_alg, "_host": (a_h, host0[0], host0[1], out0),
            "roofline": roofline("hbm", gbs, PEAK_GBS, "GB/s", traffic_of(tr, "w4a16_decode_16x4096x11008"))}


def bench_prefill(rt, steps, warmup, rng, tr):
    m, n, k, gs = 4096, 14336, 4096, 128
    a_h = bf16_rne(rng.standard_normal((m, k), dtype=np.float32))
    a = rt.upload(a_h)
    qw, s, zw = _w4_operands(rng, n, k, gs, True)
    dq, ds, dz = rt.upload(qw), rt.upload(s), rt.upload(zw)
    dc = rt.alloc(m * n * 2)

    def step():
        rt.w4a16(a.gpu_addr(), dq.gpu_addr(), ds.gpu_addr(), dz.gpu_addr(), dc.gpu_addr(), m, n, k, group_size=gs,
                 zero_const=0)

    plan = rt.w4a16_plan(a.gpu_addr(), dq.gpu_addr(), ds.gpu_addr(), dz.gpu_addr(), dc.gpu_addr(), m, n, k,
                         group_size=gs, zero_const=0)
    tm = Timer(rt)
    ms = tm.run(step, max(5, steps // 4), max(2, warmup // 2))
    med = float(np.median(tm.per_call(step, 20)))
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    rows0 = dc.read(np.uint16, PARITY_ROWS * n).reshape(PARITY_ROWS, n)
    for buf in (a, dq, ds, dz, dc):
        buf.free()
    return {"workload": "W4A16 prefill M=4096 K=4096 N=14336, g=128, per-group z, bf16 out", "kernel": plan[0],
            "ms_per_launch": round(ms, 4), "ms_median_per_launch": round(med, 4), "tflops": round(tflops, 2),
            "_host": (a_h, qw, s, zw, rows0),
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
    ms_f, _ = rotate_timed(rt, fused, steps, warmup)
    ms_s, _ = rotate_timed(rt, separate, steps, warmup)
    for buf in [res, hid, gam, x2, a16, dc] + [b for st in sets for b in st]:
        buf.free()
    return {"workload": "decode token: residual + RMSNorm + W4A16 M=1 K=4096 N=11008, g=128, z=8",
            "kernel": "t0k_w4a16_decode_norm_t3", "us_fused": round(ms_f * 1e3, 3),
            "us_two_kernels": round(ms_s * 1e3, 3)}


def _cpu_entry(value, unit, sample, secs, extra=None):
    d = {"value": value, "unit": unit, "cores": 1, "kind": "port", "sample": sample, "seconds": round(secs, 2),
         "host": cpu_model(), "nproc": os.cpu_count()}
    if extra:
        d.update(extra)
    return d


LOOP = "sequential-f32 no-FMA loop of examples/test_gemm_correctness.rs:28-42 (oracle restatement, one thread)"


def cpu_baselines(head, extras, rows_big: int, gpu_256=None):
    """The reference's CPU path on every BASELINE config (the same seeded
    inputs as the GPU run, in this process): C1 256^3 and C3 skinny in full;
    C4 decode in full as dequant (src/t0/quant_kernels.rs:365-372) then the
    same loop; C2 4096^3 and C5 prefill on a contiguous slice of rows_big M
    rows, scaled by M / rows_big (the naive loop's cost is linear in M).
    Each config's GPU output is checked against the oracle result on the
    same inputs (the first PARITY_ROWS rows of the 4096-row workloads):
    max |err|, relative Frobenius error and the tight per-element bound of
    oracle/parity.py."""
    from oracle import oracle as orc   # checker-side code: the CPU baseline leg only
    from oracle import parity
    out = {}

    def f32(u16):
        return orc.bf16_to_f32(u16)

    def check(got, ref, bound, rows):
        """The GPU output against the oracle on the same inputs: max |err|,
        relative Frobenius error, and the tight per-element bound."""
        err = np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))
        return {"outputs": int(err.size), "rows": rows, "max_abs_err": float(f"{err.max():.4g}"),
                "rel_frobenius": float(f"{parity.rel_frobenius(got, ref):.4g}"),
                "within_tight_bound": bool(np.all(err <= bound))}

    def w4_parts(qw, sc, zw, zc, nn_, kk):
        q = orc.int4_unpack(qw.view(np.uint8), nn_ * kk).reshape(nn_, kk)
        G = kk // 128
        if zw is None:
            z = np.full((G, nn_), zc)
        else:
            z = np.zeros((G, nn_), np.int64)
            for j in range(8):
                z[:, j::8] = ((zw >> np.uint32(4 * j)) & 0xF).astype(np.int64)
        return q, f32(sc), z

    # C2: 4096^3 NN, bf16 inputs N(0,1)
    a, b = head["a"], head["b"]
    m, k = a.shape
    n = b.shape[1]
    t = time.perf_counter()
    ref = orc.gemm_rows(a, b, "nn", 0, rows_big)
    dt = time.perf_counter() - t
    pr = min(rows_big, PARITY_ROWS)
    got = f32(head["gpu_rows"][:pr])
    parity_head = check(got, ref[:pr], parity.tight_bound(ref[:pr], f32(a[:pr]), f32(b), True), f"0-{pr - 1}")
    out["gemm_4096"] = _cpu_entry(2.0 * rows_big * n * k / dt / 1e12, "TFLOP/s",
                                  f"rows 0-{rows_big - 1} of the 4096^3 NN GEMM ({2.0 * rows_big * n * k / 1e9:.2f} "
                                  f"GFLOP), {LOOP}; scaled to all {m} rows (cost linear in rows): "
                                  f"{dt * m / rows_big:.0f} s for the whole GEMM", dt)
    out["parity_gemm_4096"] = parity_head
    # C1: 256^3, U(-1,1) inputs, f32 out, in full
    rng = np.random.default_rng(256)
    a1 = bf16_rne(rng.uniform(-1, 1, (256, 256)).astype(np.float32))
    b1 = bf16_rne(rng.uniform(-1, 1, (256, 256)).astype(np.float32))
    t = time.perf_counter()
    ref1 = orc.gemm_nn(a1, b1)
    dt = time.perf_counter() - t
    out["gemm_256"] = _cpu_entry(2.0 * 256 ** 3 / dt / 1e12, "TFLOP/s", f"whole 256^3 GEMM (U(-1,1) seed 256), {LOOP}",
                                 dt)
    if gpu_256 is not None:
        out["parity_gemm_256"] = check(gpu_256(a1, b1), ref1, parity.tight_bound(ref1, f32(a1), f32(b1), False),
                                       "all (f32 out)")
    # C3: skinny 128x4096x4096, in full
    if "skinny" in extras:
        a3, b3, g3 = extras["skinny"]["_host"]
        t = time.perf_counter()
        ref3 = orc.gemm_nn(a3, b3)
        dt = time.perf_counter() - t
        extras["skinny"]["parity"] = check(f32(g3), ref3, parity.tight_bound(ref3, f32(a3), f32(b3), True), "all")
        fl = 2.0 * 128 * 4096 * 4096
        by = 128 * 4096 * 2 + 4096 * 4096 * 2 + 128 * 4096 * 2
        out["skinny"] = _cpu_entry(fl / dt / 1e12, "TFLOP/s", f"whole 128x4096x4096 GEMM (weight set 0), {LOOP}", dt,
                                   {"gbs": round(by / dt / 1e9, 4)})
    # C4: decode, dequant + loop, in full
    if "w4a16_decode" in extras:
        a4, qw, sc, g4 = extras["w4a16_decode"]["_host"]
        mm, kk, nn_ = a4.shape[0], a4.shape[1], qw.shape[0]
        t = time.perf_counter()
        w = orc.w4a16_dequant(qw, sc, None, 8, nn_, kk, 128)
        ref4 = orc.gemm_bf16_f32w_rows(a4, w, 0, mm)
        dt = time.perf_counter() - t
        q, sf, z = w4_parts(qw, sc, None, 8, nn_, kk)
        extras["w4a16_decode"]["parity"] = check(f32(g4), ref4,
                                                 parity.w4_tight_bound(ref4, f32(a4), q, sf, z, 128, True), "all")
        by = extras["w4a16_decode"]["bytes_per_launch"]
        out["w4a16_decode"] = _cpu_entry(by / dt / 1e9, "GB/s",
                                         f"whole 16x4096x11008 decode (weight set 0): dequant (q - 8) * s to f32, then "
                                         f"{LOOP}; GB/s of the same algorithmic bytes ({by})", dt,
                                         {"tflops": round(2.0 * mm * nn_ * kk / dt / 1e12, 6)})
    # C5: prefill, dequant + a row slice of the loop
    if "w4a16_prefill" in extras:
        a5, qw, sc, zw, g5 = extras["w4a16_prefill"]["_host"]
        mm, kk, nn_ = a5.shape[0], a5.shape[1], qw.shape[0]
        t = time.perf_counter()
        w = orc.w4a16_dequant(qw, sc, zw, 0, nn_, kk, 128)
        t_dq = time.perf_counter() - t
        ref5 = orc.gemm_bf16_f32w_rows(a5, w, 0, rows_big)
        t_loop = time.perf_counter() - t - t_dq
        q, sf, z = w4_parts(qw, sc, zw, 0, nn_, kk)
        extras["w4a16_prefill"]["parity"] = check(f32(g5[:pr]), ref5[:pr],
                                                  parity.w4_tight_bound(ref5[:pr], f32(a5[:pr]), q, sf, z, 128, True),
                                                  f"0-{pr - 1}")
        total = t_dq + t_loop * mm / rows_big
        out["w4a16_prefill"] = _cpu_entry(2.0 * mm * nn_ * kk / total / 1e12, "TFLOP/s",
                                          f"dequant of the whole 14336x4096 weight ({t_dq:.1f} s) + rows 0-{rows_big - 1}"
                                          f" of {LOOP} ({t_loop:.1f} s), the loop scaled to all {mm} rows: "
                                          f"{total:.0f} s for the whole prefill", t_dq + t_loop)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-rows", type=int, default=64, help="M rows of the 4096^3 and prefill CPU samples")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="issue rotated launches directly (for tracers)")
    ap.add_argument("--only", choices=["gemm4096", "skinny", "decode", "prefill", "ignis", "norm_decode", "copy",
                                       "floor", "tiles"],
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
              "copy": bench_copy, "floor": bench_floor, "tiles": bench_tiles}[args.only]
        r = fn(rt, args.steps, args.warmup, rng, tr)
        for key in ("a", "b", "gpu_rows", "_host"):
            r.pop(key, None)
        print(json.dumps({"only": args.only, **{k: v for k, v in r.items()}}, default=float), flush=True)
        rt.close()
        return

    head = bench_gemm_4096(rt, args.steps, args.warmup, rng, tr)
    print(f"# gemm 4096^3 NN bf16: {head['ms'] * 1e3:.1f} us/launch, {head['tflops']:.1f} TFLOP/s "
          f"({head['kernel']})", file=sys.stderr, flush=True)
    extras = {}
    if not args.no_extras:
        for name, fn in (("skinny", bench_skinny), ("w4a16_decode", bench_decode), ("decode_floor", bench_floor),
                         ("w4a16_prefill", bench_prefill), ("ignis_matmul", bench_ignis),
                         ("norm_decode", bench_norm_decode)):
            extras[name] = fn(rt, args.steps, args.warmup, rng, tr)
            shown = {k: v for k, v in extras[name].items() if k != "_host"}
            print(f"# {name}: {json.dumps(shown)}", file=sys.stderr, flush=True)
    cpu = None
    parity_head = None
    if not args.no_cpu_baseline:
        def gpu_256(a1, b1):
            """The CPU config (256^3, U(-1,1), f32 out) on the GPU, for its parity entry."""
            d1, e1, c1 = rt.upload(a1), rt.upload(b1), rt.alloc(256 * 256 * 4)
            rt.gemm(d1.gpu_addr(), e1.gpu_addr(), c1.gpu_addr(), 256, 256, 256, transpose=t0.NN, out_dtype=t0.OUT_F32)
            rt.wait_idle()
            r1 = c1.read(np.float32, 256 * 256).reshape(256, 256)
            for x in (d1, e1, c1):
                x.free()
            return r1
        cpus = cpu_baselines(head, extras, args.cpu_rows, gpu_256)
        cpu = cpus.pop("gemm_4096")
        parity_head = cpus.pop("parity_gemm_4096")
        extras["cpu_gemm_256"] = {"workload": "bf16 GEMM M=N=K=256, U(-1,1), f32 out (CPU-only config)",
                                  "cpu_baseline": cpus.pop("gemm_256"), "parity": cpus.pop("parity_gemm_256", None)}
        for key, v in cpus.items():
            extras[key]["cpu_baseline"] = v
    for e in extras.values():
        e.pop("_host", None)
    rt.close()

    line = {
        "metric": METRIC,
        "value": round(head["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 5),
        "ms_median_per_launch": round(head["ms_median_per_launch"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) rounded to bf16 (numpy seed 20261201), inputs resident in HBM",
        "config": {"workload": "bf16 GEMM M=N=K=4096, A[M,K] . B[K,N] row-major (NN), fp32 accumulate, bf16 out",
                   "m": 4096, "n": 4096, "k": 4096, "layout": "NN", "out": "bf16", "kernel": head["kernel"],
                   "device": info, "sclk_mhz_measured": round(head["sclk_mhz"], 1),
                   "workgroup_span_us": round(head["workgroup_span_us"], 2)},
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "parity": parity_head,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

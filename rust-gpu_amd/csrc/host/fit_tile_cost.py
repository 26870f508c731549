"""Fits the per-tile cost table of rank_candidates (csrc/host/config.cpp,
kTileCost and the constants beside it) to the measurements that
``python bench.py --only tiles`` prints: every ranked tile x split-K
candidate timed on LLM shapes (NN, bf16 out, weight operand read cold).

    python rust-gpu_amd/csrc/host/fit_tile_cost.py tiles.json [tiles2.json ...]
    python rust-gpu_amd/csrc/host/fit_tile_cost.py --timings profiles/tile_timings.json
    python rust-gpu_amd/csrc/host/fit_tile_cost.py --table profiles/tile_timings.json

Several runs are averaged per candidate (geometric mean of the times).

The model is the one rank_candidates evaluates: per workgroup a + b * k_len
/ 1000 us while a round of workgroups (CUs x workgroups per CU, by LDS) is
resident, a partly filled last round costing DISC + (1 - DISC) * fill of a
round; co-resident workgroups at most 1 / CO as fast each; no faster than
A + B + C plus the split-K partial tiles (written and read back) over HBM,
nor the operand re-reads over L2; split-K adding FIX + FIX_MB per MB of
partial tiles.  (The library's ranking then moves near-ties, within 1 %,
to the fewest partial bytes and the smallest tile: ``pick``.)  Least squares on log time from several
starts, then a ranking refinement: per shape, the measured log regret of
the candidates weighted by a soft minimum of the predicted times (what the
pick costs), plus W_ERR x the mean squared log error (so the predicted
times stay meaningful), minimised by Powell's method from the least-squares
fit.  Prints the fitted constants, the pick's regret (pick / measured best)
per shape, and the same with each shape left out of the fit."""
import json
import math
import re
import sys

import numpy as np
from scipy.optimize import least_squares, minimize

CUS, LDS = 256.0, 160 * 1024.0
NAME = re.compile(r"t0_gemm_(\d+)x(\d+)_k(\d+)_ldsdb(?:_sk(\d+))?_nn_bf16 w(\d+)")
# LDS bytes of each instance (stages x stage bytes, or the epilogue staging)
STAGES = {(256, 256, 64, 8): 2, (256, 128, 64, 4): 3, (128, 256, 64, 4): 3, (128, 128, 64, 4): 4,
          (128, 64, 64, 4): 4, (64, 128, 64, 4): 4, (64, 64, 64, 1): 4, (32, 128, 64, 2): 4, (32, 64, 64, 1): 6}
WAVES = {(256, 256, 64, 8): (2, 4), (256, 128, 64, 4): (2, 2), (128, 256, 64, 4): (2, 2),
         (128, 128, 64, 4): (2, 2), (128, 64, 64, 4): (2, 2), (64, 128, 64, 4): (2, 2), (64, 64, 64, 1): (1, 1),
         (32, 128, 64, 2): (1, 2), (32, 64, 64, 1): (1, 1)}
TILES = list(STAGES)


def lds_bytes(t):
    bm, bn, bk, nw = t
    wm, wn = WAVES[t]
    return max((bm + bn) * bk * 2 * STAGES[t], nw * 32 * (bn // wn + 4) * 4)


def predict(params, t, sk, m, n, k):
    ti = TILES.index(t)
    a, b = params[2 * ti], params[2 * ti + 1]
    disc, fix, fix_mb, hbm, l2, co = params[2 * len(TILES):]
    bm, bn = t[0], t[1]
    slots = CUS * max(1.0, min(math.floor(LDS / lds_bytes(t)), 8.0))
    tiles = math.ceil(m / bm) * math.ceil(n / bn)
    wgs = tiles * sk
    full = math.floor(wgs / slots)
    fill = wgs / slots - full
    rounds = full + (disc + (1 - disc) * fill if fill > 0 else 0.0)
    t_wg = a + b * (k / sk) / 1000.0
    tm = rounds * t_wg
    if slots > CUS:
        tm = max(tm, math.ceil(wgs / CUS) * t_wg * co)
    hb = k * n * 2.0 + m * k * 2.0 + m * n * 2.0 + (2.0 * wgs * bm * bn * 4 if sk > 1 else 0.0)
    l2b = m * k * 2.0 * math.ceil(n / bn) + n * k * 2.0 * math.ceil(m / bm)
    tm = max(tm, hb / (hbm * 1e6), l2b / (l2 * 1e6))
    if sk > 1:
        tm += fix + fix_mb * wgs * bm * bn * 4 / 1e6
    return tm


def _last_json(path):
    with open(path) as f:
        return json.loads(f.read().strip().splitlines()[-1])


def load(*paths):
    """Shapes and their candidates' times; with several runs, per shape the
    geometric mean of each candidate's times over the runs that timed the
    shape (candidates every such run timed)."""
    per_shape = {}
    for p in paths:
        for s in _last_json(p)["shapes"]:
            per_shape.setdefault(tuple(s["shape"]), []).append(s["all"])
    data = []
    for (m, n, k), runs in per_shape.items():
        times = {}
        for cands in runs:
            for name, _est, meas in cands:
                times.setdefault(name, []).append(meas)
        cands = []
        for name, ts in times.items():
            if len(ts) != len(runs):
                continue
            g = NAME.fullmatch(name)
            bm, bn, bk, sk, w = int(g[1]), int(g[2]), int(g[3]), int(g[4] or 1), int(g[5])
            cands.append(((bm, bn, bk, w), sk, float(np.exp(np.mean(np.log(ts))))))
        data.append(((m, n, k), cands))
    return data


CAND = re.compile(r"(\d+)x(\d+)x(\d+)_sk(\d+)_w(\d+)")


def load_timings(path, runs=None):
    """The same from the committed measurements (profiles/tile_timings.json):
    the runs named (default: the runs the cost table was fitted to)."""
    with open(path) as f:
        doc = json.load(f)
    runs = doc["fit_runs"] if runs is None else runs
    data = []
    for s in doc["shapes"]:
        rs = [r for r in runs if r in s["us"]]
        if not rs:
            continue
        cands = []
        for i, name in enumerate(s["candidates"]):
            ts = [s["us"][r][i] for r in rs]
            if any(t is None for t in ts):
                continue
            g = CAND.fullmatch(name)
            cands.append(((int(g[1]), int(g[2]), int(g[3]), int(g[5])), int(g[4]),
                          float(np.exp(np.mean(np.log(ts))))))
        data.append((tuple(s["shape"]), cands))
    return data


def _arrays(data):
    """Per-candidate arrays of the model's inputs (tile index, workgroups,
    rounds structure, bytes) so that a prediction is a few numpy operations."""
    rows = []
    for (m, n, k), cands in data:
        for t, sk, meas in cands:
            bm, bn = t[0], t[1]
            slots = CUS * max(1.0, min(math.floor(LDS / lds_bytes(t)), 8.0))
            wgs = math.ceil(m / bm) * math.ceil(n / bn) * sk
            hb = k * n * 2.0 + m * k * 2.0 + m * n * 2.0 + (2.0 * wgs * bm * bn * 4 if sk > 1 else 0.0)
            l2b = m * k * 2.0 * math.ceil(n / bn) + n * k * 2.0 * math.ceil(m / bm)
            rows.append((TILES.index(t), wgs / slots, slots > CUS, math.ceil(wgs / CUS), k / sk / 1000.0, hb, l2b,
                         sk > 1, wgs * bm * bn * 4 / 1e6, meas))
    a = np.array(rows, dtype=np.float64)
    return {"ti": a[:, 0].astype(int), "q": a[:, 1], "co": a[:, 2] > 0, "qc": a[:, 3], "kl": a[:, 4],
            "hb": a[:, 5], "l2": a[:, 6], "sk": a[:, 7] > 0, "mb": a[:, 8], "meas": a[:, 9]}


def predict_all(p, A):
    nt = len(TILES)
    a, b = p[0:2 * nt:2][A["ti"]], p[1:2 * nt:2][A["ti"]]
    disc, fix, fix_mb, hbm, l2, co = p[2 * nt:]
    full = np.floor(A["q"])
    fill = A["q"] - full
    rounds = full + np.where(fill > 0, disc + (1 - disc) * fill, 0.0)
    t_wg = a + b * A["kl"]
    tm = rounds * t_wg
    tm = np.where(A["co"], np.maximum(tm, A["qc"] * t_wg * co), tm)
    tm = np.maximum(tm, np.maximum(A["hb"] / (hbm * 1e6), A["l2"] / (l2 * 1e6)))
    return tm + np.where(A["sk"], fix + fix_mb * A["mb"], 0.0)


def fit(data, starts=8, seed=0):
    rng = np.random.default_rng(seed)
    A = _arrays(data)

    def resid(p):
        return np.log(np.maximum(predict_all(p, A), 1e-3) / A["meas"])

    lo, hi = LO, HI
    best = None
    for _ in range(starts):
        x0 = [rng.uniform(l, h) for l, h in zip(lo, hi)]
        r = least_squares(resid, x0, bounds=(lo, hi))
        if best is None or r.cost < best.cost:
            best = r
    return best.x, float(np.median(np.abs(np.exp(best.fun) - 1)))


W_ERR, TAU = 3.0, 0.05
LO = [0.1, 0.1] * len(TILES) + [0.5, 0.0, 0.0, 1.0, 2.0, 0.2]
HI = [60.0, 60.0] * len(TILES) + [1.0, 20.0, 5.0, 8.0, 40.0, 1.0]


def fit_rank(data, p0):
    """The least-squares fit p0 refined for the picks (see the module doc)."""
    shapes = []
    for shape, cands in data:
        A = _arrays([(shape, cands)])
        shapes.append((A, np.log(A["meas"] / A["meas"].min())))
    A_all = _arrays(data)
    lo, hi = np.array(LO), np.array(HI)

    def obj(x):
        p = np.clip(x, lo, hi)
        tot = 0.0
        for A, lr in shapes:
            pr = np.log(np.maximum(predict_all(p, A), 1e-3))
            w = np.exp(-(pr - pr.min()) / TAU)
            tot += float((w * lr).sum() / w.sum())
        err = np.log(np.maximum(predict_all(p, A_all), 1e-3) / A_all["meas"])
        return tot + W_ERR * float(np.mean(err ** 2))

    r = minimize(obj, p0, method="Powell", options={"maxiter": 20000, "xtol": 1e-3, "ftol": 1e-6})
    return np.clip(r.x, lo, hi)


def pick(params, cands, m, n, k):
    """Index of the candidate the library ranks first: the least predicted
    time, near-ties (within 1 %) to the fewest partial-tile bytes, then the
    smallest tile (rank_candidates, csrc/host/config.cpp)."""
    pr = [predict(params, t, sk, m, n, k) for t, sk, _ in cands]
    # stable in the library's candidate order: the tile table, then split-K up
    order = sorted(range(len(cands)), key=lambda i: (pr[i], TILES.index(cands[i][0]), cands[i][1]))

    def part(i):
        (bm, bn, _, _), sk, _ = cands[i]
        return math.ceil(m / bm) * math.ceil(n / bn) * sk * bm * bn * 4.0 if sk > 1 else 0.0

    best = order[0]
    for i in order[1:]:
        if pr[i] > pr[order[0]] * 1.01:
            break
        if part(i) < part(best) or (part(i) == part(best) and
                                    cands[i][0][0] * cands[i][0][1] < cands[best][0][0] * cands[best][0][1]):
            best = i
    return best


def regrets(params, data):
    out = []
    for (m, n, k), cands in data:
        best = min(c[2] for c in cands)
        out.append(cands[pick(params, cands, m, n, k)][2] / best)
    return out


def table(path):
    """Markdown tables of the library's pick (t0_auto_schedule_gemm's rank 0)
    against the measured best per shape: the fitted runs averaged, then each
    held-out run."""
    import os
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
    import t0_gpu as t0
    with open(path) as f:
        doc = json.load(f)
    short = lambda t, sk: f"{t[0]}x{t[1]}_k{t[2]}{f'_sk{sk}' if sk > 1 else ''} w{t[3]}"
    for label, runs in [("fitted runs, averaged", None)] + [(f"held-out run {r}", [r]) for r in doc["held_out_runs"]]:
        data = load_timings(path, runs)
        print(f"\n{label}:\n")
        print("| M x N x K | candidates | pick | pick us | measured best | best us | pick / best | best's predicted rank |")
        print("|---|---|---|---|---|---|---|---|")
        reg = []
        for (m, n, k), cands in data:
            ranked = t0.auto_schedule_gemm(m, n, k, t0.NN, t0.OUT_BF16)
            keys = [((c.tile_m, c.tile_n, c.tile_k, c.wg_size // 64), max(c.split_k, 1)) for c, _ in ranked]
            where = {(t, sk): i for i, (t, sk, _) in enumerate(cands)}
            ip = where[keys[0]]
            ib = min(range(len(cands)), key=lambda i: cands[i][2])
            rank = keys.index((cands[ib][0], cands[ib][1]))
            reg.append(cands[ip][2] / cands[ib][2])
            print(f"| {m} x {n} x {k} | {len(cands)} | {short(*cands[ip][:2])} | {cands[ip][2]:.1f} | "
                  f"{short(*cands[ib][:2])} | {cands[ib][2]:.1f} | {reg[-1]:.3f} | {rank} |")
        print(f"\npick / best: median {np.median(reg):.3f}, max {max(reg):.3f}, "
              f"within 3 % on {sum(r <= 1.03 for r in reg)} of {len(reg)}")


def main():
    if sys.argv[1:2] == ["--table"]:
        table(sys.argv[2])
        return
    if sys.argv[1:2] == ["--timings"]:
        data = load_timings(sys.argv[2])
    else:
        data = load(*sys.argv[1:])
    params = fit_rank(data, fit(data)[0])
    A = _arrays(data)
    med_err = float(np.median(np.abs(predict_all(params, A) / A["meas"] - 1)))
    reg = regrets(params, data)
    print(f"fit: median |pred/meas - 1| {med_err:.3f}; pick regret median {np.median(reg):.3f}, "
          f"max {max(reg):.3f}, within 3% on {sum(r <= 1.03 for r in reg)} of {len(reg)}")
    for t, i in zip(TILES, range(len(TILES))):
        print(f"    {{{t[0]}, {t[1]}, {t[2]}, {t[3]}, {params[2 * i]:.2f}, {params[2 * i + 1]:.2f}}},")
    disc, fix, fix_mb, hbm, l2, co = params[2 * len(TILES):]
    print(f"constexpr double kDisc = {disc:.3f}, kFixUs = {fix:.3f}, kFixUsPerMB = {fix_mb:.3f};")
    print(f"constexpr double kHbmTBs = {hbm:.3f}, kL2TBs = {l2:.3f}, kCoResident = {co:.3f};")
    loo = []
    for j in range(len(data)):
        sub = data[:j] + data[j + 1:]
        p = fit_rank(sub, fit(sub, starts=3, seed=j + 1)[0])
        loo.append(regrets(p, [data[j]])[0])
    print(f"leave-one-shape-out regret: median {np.median(loo):.3f}, max {max(loo):.3f}, "
          f"within 3% on {sum(r <= 1.03 for r in loo)} of {len(loo)}")
    for (shape, _), r, rl in zip(data, reg, loo):
        print(f"    {shape}: regret {r:.3f} (left out: {rl:.3f})")


if __name__ == "__main__":
    main()

"""The library's tile / split-K pick (t0_auto_schedule_gemm's rank 0, the
ranking of csrc/host/config.cpp) against the measured times committed in
profiles/tile_timings.json (bench.py --only tiles on MI355X), recomputed
here on the CPU: the regret pick / measured best on the runs the cost table
was fitted to (averaged) and on the run held out from the fit.  Then the
ranking's rules on shapes no run covers, and pinned picks there."""
import math
import os
import sys

import numpy as np
import pytest

import t0_gpu as t0

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "rust-gpu_amd", "csrc", "host"))
import fit_tile_cost as F  # noqa: E402
from test_fit_tile_cost import committed_params  # noqa: E402

TIMINGS = os.path.join(ROOT, "profiles", "tile_timings.json")


def key(cfg):
    return (cfg.tile_m, cfg.tile_n, cfg.tile_k, cfg.wg_size // 64), max(cfg.split_k, 1)


def part_bytes(m, n, cfg):
    sk = max(cfg.split_k, 1)
    return math.ceil(m / cfg.tile_m) * math.ceil(n / cfg.tile_n) * sk * cfg.tile_m * cfg.tile_n * 4 if sk > 1 else 0


def library_regrets(runs):
    out = []
    for (m, n, k), cands in F.load_timings(TIMINGS, runs):
        ranked = t0.auto_schedule_gemm(m, n, k, t0.NN, t0.OUT_BF16)
        where = {(t, sk): i for i, (t, sk, _) in enumerate(cands)}
        assert key(ranked[0][0]) in where, f"{m}x{n}x{k}: pick {ranked[0][0].name()} was not timed"
        pick = cands[where[key(ranked[0][0])]][2]
        best = min(c[2] for c in cands)
        out.append(((m, n, k), pick / best))
    return out


def test_picks_on_the_fitted_runs():
    """34 shapes, the six fitted runs averaged per candidate: every pick
    within 3 % of the measured best."""
    reg = library_regrets(None)
    assert len(reg) == 34
    worst = max(reg, key=lambda x: x[1])
    assert all(r <= 1.03 for _, r in reg), worst
    assert np.median([r for _, r in reg]) == pytest.approx(1.0)


def test_picks_on_the_held_out_run():
    """The run on a fourth box, after the fit: within 3 % on 26 of 34
    shapes, at worst 1.183 (512 x 14336 x 4096)."""
    reg = library_regrets(["c"])
    assert len(reg) == 34
    assert sum(r <= 1.03 for _, r in reg) >= 26
    assert max(r for _, r in reg) <= 1.19


def test_python_pick_rule_is_the_library_ranking():
    """fit_tile_cost.pick (the model and the near-tie rule) picks what the
    library picks on every measured shape."""
    p = committed_params()
    for (m, n, k), cands in F.load_timings(TIMINGS):
        lib = key(t0.auto_schedule_gemm(m, n, k, t0.NN, t0.OUT_BF16)[0][0])
        i = F.pick(p, cands, m, n, k)
        assert (cands[i][0], cands[i][1]) == lib, (m, n, k)


UNMEASURED = [(1, 4096, 4096), (1, 11008, 4096), (1, 4096, 14336), (1, 8192, 28672), (1, 57344, 8192),
              (16, 4096, 14336), (128, 4096, 14336), (128, 8192, 28672), (1024, 4096, 14336), (256, 8192, 28672)]


@pytest.mark.parametrize("m,n,k", UNMEASURED)
def test_split_k_partials_bound_every_candidate(m, n, k):
    """No candidate is predicted faster than its whole HBM traffic allows:
    A + B + C plus the partial tiles written and read back, at 8 TB/s."""
    for cfg, est in t0.auto_schedule_gemm(m, n, k, t0.NN, t0.OUT_BF16):
        traffic = 2.0 * (m * k + k * n + m * n) + 2 * part_bytes(m, n, cfg)
        assert est >= traffic / 8e6 * (1 - 1e-12), (cfg.name(), est, traffic / 8e6)


@pytest.mark.parametrize("m,n,k", UNMEASURED)
def test_near_ties_go_to_fewer_partials_then_smaller_tiles(m, n, k):
    ranked = t0.auto_schedule_gemm(m, n, k, t0.NN, t0.OUT_BF16)
    best_est = min(e for _, e in ranked)
    near = [c for c, e in ranked if e <= best_est * 1.01]
    pick = ranked[0][0]
    assert ranked[0][1] <= best_est * 1.01
    rank_key = lambda c: (part_bytes(m, n, c), c.tile_m * c.tile_n)
    assert rank_key(pick) == min(rank_key(c) for c in near), [c.name() for c in near]


PINNED = {(1, 4096, 4096): "t0_gemm_32x64_k64_ldsdb_sk4_nn_bf16",
          (1, 11008, 4096): "t0_gemm_32x128_k64_ldsdb_sk2_nn_bf16",
          (1, 4096, 14336): "t0_gemm_32x128_k64_ldsdb_sk8_nn_bf16",
          (1, 8192, 28672): "t0_gemm_32x128_k64_ldsdb_sk4_nn_bf16",
          (1, 57344, 8192): "t0_gemm_32x128_k64_ldsdb_nn_bf16",
          (16, 4096, 14336): "t0_gemm_32x128_k64_ldsdb_sk8_nn_bf16",
          (128, 4096, 14336): "t0_gemm_128x128_k64_ldsdb_sk8_nn_bf16",
          (128, 8192, 28672): "t0_gemm_128x128_k64_ldsdb_sk4_nn_bf16",
          (1024, 4096, 14336): "t0_gemm_256x256_k64_ldsdb_sk4_nn_bf16",
          (256, 8192, 28672): "t0_gemm_256x256_k64_ldsdb_sk8_nn_bf16"}


@pytest.mark.parametrize("shape", sorted(PINNED))
def test_pinned_picks_outside_the_measured_shapes(shape):
    """Picks no measurement covers yet, pinned so that a change to the
    ranking shows up here; one row (M = 1) takes the narrowest tile."""
    m, n, k = shape
    pick = t0.auto_schedule_gemm(m, n, k, t0.NN, t0.OUT_BF16)[0][0]
    assert pick.name() == PINNED[shape]
    if m == 1:
        assert pick.tile_m == 32


@pytest.mark.parametrize("runs,top", [(None, 3), (["c"], 6)])
def test_measured_best_is_among_the_best_predicted(runs, top):
    """The tuner times the 8 best-predicted candidates: on every measured
    shape the measured best is among the first 3 of the library's order on
    the fitted runs, and the first 6 on the held-out run."""
    for (m, n, k), cands in F.load_timings(TIMINGS, runs):
        order = [key(c) for c, _ in t0.auto_schedule_gemm(m, n, k, t0.NN, t0.OUT_BF16)]
        best = min(cands, key=lambda c: c[2])
        assert order.index((best[0], best[1])) < top, (m, n, k)

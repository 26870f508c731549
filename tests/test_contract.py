"""CPU contract tests of the drop-in boundary, restating the reference's own
CPU-only contracts (tests/tile_gemm_contract.rs, src/t0/gemm_gen.rs:572-662,
src/t0/quant_kernels.rs:346-491) against the gfx950 library.  No GPU."""
import struct

import numpy as np
import pytest

import t0_gpu as t0
from oracle import oracle as orc


def feasible_presets():
    return [getattr(t0.GemmConfig, n)() for n in t0.PRESETS if getattr(t0.GemmConfig, n)().is_feasible()]


def test_presets_exist_and_keep_reference_values():
    # src/t0/gemm_gen.rs:86-145
    c = t0.GemmConfig.tile_128x64_k16()
    assert (c.tile_m, c.tile_n, c.tile_k, c.wg_size) == (128, 64, 16, 128)
    assert c.use_lds and c.double_buffer and c.swap_grid and c.wgp_mode and c.split_k == 0
    c = t0.GemmConfig.tile_128x128_2pass()
    assert (c.tile_m, c.tile_n, c.n_col_passes) == (128, 64, 2)
    assert t0.GemmConfig.tile_32x64_direct().use_lds == 0


def test_preset_16x64_is_not_a_gfx950_kernel():
    # a 32-lane workgroup cannot hold a wave64 MFMA tile; reported, not panicked
    c = t0.GemmConfig.tile_16x64_k16()
    assert not c.is_feasible()
    with pytest.raises(t0.T0Error) as e:
        t0.generate(c)
    assert e.value.status == -2


def test_preset_dimension_identities():
    """tests/tile_gemm_contract.rs:43-58, restated for wave64 / 32x32 MFMA blocks."""
    presets = feasible_presets()
    assert len(presets) >= 20
    for c in presets:
        g = c.geometry()
        assert c.wg_size == g.n_waves * 64, c.name()
        assert g.waves_m * g.waves_n == g.n_waves
        assert g.rows_per_wave * g.waves_m == c.tile_m
        assert g.cols_per_wave * g.waves_n == c.tile_n
        assert g.n_row_blocks == g.rows_per_wave // 32 and g.rows_per_wave % 32 == 0
        assert g.n_col_tiles == g.cols_per_wave // 32
        assert g.k_sub_steps == c.tile_k // 16
        assert g.mfma_per_k_tile == g.n_row_blocks * g.n_col_tiles * g.k_sub_steps


def test_lds_total_self_consistent():
    """tests/tile_gemm_contract.rs:62-69: LDS = stages x (X + WT) (or the epilogue
    staging area when larger), within gfx950's 160 KiB."""
    for c in feasible_presets():
        g = c.geometry()
        assert g.lds_per_buffer == (c.tile_m + c.tile_n) * c.tile_k * 2
        stage_total = g.stages * g.lds_per_buffer
        epi = g.n_waves * 32 * (g.cols_per_wave + 4) * 4
        assert g.lds_total == max(stage_total, epi)
        assert g.lds_total <= 160 * 1024


def test_grid_coverage_enumeration():
    """tests/tile_gemm_contract.rs:73-93."""
    configs = [t0.GemmConfig.tile_128x64_k16(), t0.GemmConfig.tile_128x64_k32(), t0.GemmConfig.tile_64x64_k32(),
               t0.GemmConfig.tile_256x256_k64()]
    dims = [1, 31, 32, 33, 63, 64, 127, 128, 255, 256, 4095, 4096]
    for cfg in configs:
        for m in dims:
            for n in dims:
                gx, gy = t0.compute_grid_auto(cfg, m, n)
                assert gx % cfg.wg_size == 0
                tiles_m = (m + cfg.tile_m - 1) // cfg.tile_m
                tiles_n = (n + cfg.tile_n - 1) // cfg.tile_n
                assert gy == tiles_m
                assert gx // cfg.wg_size == tiles_n
                assert (gx // cfg.wg_size) * cfg.tile_n >= n and tiles_m * cfg.tile_m >= m


def test_grid_split_k_and_mg():
    c = t0.GemmConfig.tile_64x64_k16().copy(split_k=4)
    assert t0.compute_grid_auto(c, 256, 128) == (2 * 64, 4 * 4)
    c2 = c.copy(swap_grid=0)
    assert t0.compute_grid_auto(c2, 256, 128) == (4 * 64, 2 * 4)
    with pytest.raises(t0.T0Error):
        t0.compute_grid_split_k(c, 64, 64, 3)


def test_build_kernargs_m_field_layout():
    """tests/tile_gemm_contract.rs:98-115: 44 bytes, X@0 WT@8 Y@16 K@24 N@28
    split_k_shift@32 y_split_stride@36 M@40."""
    spec = t0.TileGemm.make(64, 64, 16, split_k=4)
    ka = spec.build_kernargs_m(0xA000, 0xB000, 0xC000, 64, 128, 32)
    assert len(ka) == 44
    x, wt, y, k, n, sh, ys, m = struct.unpack("<QQQIIIII", ka)
    assert (x, wt, y, k, n, sh, ys, m) == (0xA000, 0xB000, 0xC000, 64, 128, 2, 0, 32)


def test_tile_kernargs_with_epilogue_args():
    """Epilogue arguments follow M at 8-byte-aligned offsets in lower_gemm's
    declaration order (src/t0/tile_ir.rs:1014-1026): bias u64, scale f32,
    clamp_min f32, clamp_max f32."""
    spec = t0.TileGemm.make(128, 128, 64, epilogue=["bias", "scale", "relu", "clamp"])
    ka = spec.build_kernargs_m(1, 2, 3, 64, 64, 64, bias=0xBEEF, scale=0.5, clamp_min=-1.0, clamp_max=2.0)
    assert len(ka) == 68
    assert struct.unpack_from("<Q", ka, 48)[0] == 0xBEEF
    assert struct.unpack_from("<fff", ka, 56) == (0.5, -1.0, 2.0)
    spec2 = t0.TileGemm.make(128, 128, 64, persistent=True)
    assert len(spec2.build_kernargs_m(1, 2, 3, 64, 64, 64)) == 64     # src/t0/tile_ir.rs:4604-4639
    spec3 = t0.TileGemm.make(128, 128, 64, persistent=True, epilogue=["bias", "scale", "clamp"])
    assert len(spec3.build_kernargs_m(1, 2, 3, 64, 64, 64)) == 84


def test_gemm_build_kernargs_split_stride_semantics():
    """tests/tile_gemm_contract.rs:119-131."""
    no_sk = t0.GemmConfig.tile_128x64_k16().copy(split_k=0)
    ka1 = t0.build_kernargs(1, 2, 3, 64, 64, 64, no_sk)
    assert len(ka1) == 40 and struct.unpack_from("<I", ka1, 36)[0] == 0
    sk2 = t0.GemmConfig.tile_128x64_k16().copy(split_k=2)
    ka2 = t0.build_kernargs(1, 2, 3, 64, 64, 256, sk2)
    assert struct.unpack_from("<I", ka2, 36)[0] == 256 * 64 * 4
    x, wt, y, k, n, shift = struct.unpack_from("<QQQIII", ka2, 0)
    assert (x, wt, y, k, n, shift) == (1, 2, 3, 64, 64, 0)


def test_kernargs_with_bias_layout():
    """src/t0/gemm_gen.rs:650-661."""
    cfg = t0.GemmConfig.tile_32x64_k16()
    ka = t0.build_kernargs_with_bias(0x1000, 0x2000, 0x3000, 64, 64, 128, cfg, 0x4000)
    assert len(ka) == 48 and struct.unpack_from("<Q", ka, 40)[0] == 0x4000


def test_backward_kernargs():
    """src/t0/gemm_gen.rs:523-531, :557-565: argument routing."""
    cfg = t0.GemmConfig.tile_64x64_k32()
    ka = t0.build_kernargs_backward_data(10, 20, 30, m=128, n_orig=256, k_orig=512, cfg=cfg)
    assert struct.unpack_from("<QQQII", ka) == (10, 20, 30, 256, 512)
    ka = t0.build_kernargs_backward_weight(10, 20, 30, m=128, n_orig=256, k_orig=512, cfg=cfg)
    assert struct.unpack_from("<QQQII", ka) == (10, 20, 30, 128, 512)


def test_epilogue_name_tags():
    """src/t0/gemm_gen.rs:622-633."""
    cfg = t0.GemmConfig.tile_32x64_k16()
    assert "t0_gemm_32x64_k16" in cfg.name() and "_bias" not in cfg.name()
    assert cfg.copy(epilogue=t0.EPI_BIAS_ADD).name().endswith("_bias")
    assert cfg.copy(epilogue=t0.EPI_BIAS_ADD_RELU).name().endswith("_bias_relu")


def test_name_roundtrip():
    variants = []
    for c in feasible_presets():
        variants += [c, c.copy(transpose=t0.NN), c.copy(out_dtype=t0.OUT_BF16), c.copy(split_k=4, swap_grid=0),
                     c.copy(epilogue=t0.EPI_BIAS_ADD_RELU)]
    for c in variants:
        back = t0.GemmConfig.from_name(c.name())
        for f, _ in t0.GemmConfig._fields_:
            if f in ("reserved",):
                continue
            a, b = getattr(c, f), getattr(back, f)
            if f == "split_k":
                a, b = max(a, 1), max(b, 1)
            assert a == b, (c.name(), f, a, b)


def test_auto_select_sizes():
    """src/t0/gemm_gen.rs:576-603, properties restated for gfx950 tiles."""
    c = t0.auto_select(256, 256, 256)
    assert 16 <= c.tile_m <= 256 and c.tile_n >= 32 and c.wg_size >= 64
    # the reference's "1024^3 -> tile_m >= 64" is an RDNA cost-model outcome;
    # on gfx950 the measured per-tile cost table decides, and the tuner measures
    c = t0.auto_select(1024, 1024, 1024)
    assert c.is_feasible() and c.tile_k in (16, 32, 64)
    c = t0.auto_select(8192, 8192, 8192)
    assert c.tile_m >= 64
    c = t0.auto_select(128, 4096, 4096)
    assert 128 % c.tile_m == 0
    # the compute-bound headline shape takes the largest gfx950 tile
    c = t0.auto_select(4096, 4096, 4096)
    assert (c.tile_m, c.tile_n) == (256, 256)


def test_auto_select_takes_measured_best_on_llm_shapes():
    """Shapes whose every tile x split candidate was timed on MI355X (NN,
    bf16 out, B read cold from HBM): where the calibrated model's pick is the
    measured fastest, it stays so, and it splits K only where one partition
    per tile cannot fill the 256 CUs.  (M, N, K) -> (tile_m, tile_n, split, threads)."""
    cases = {(4096, 11008, 4096): (256, 256, 1, 512), (4096, 4096, 11008): (256, 256, 1, 512),
             (2048, 11008, 4096): (256, 256, 1, 512), (1024, 11008, 4096): (256, 256, 1, 512),
             (1024, 4096, 4096): (128, 128, 1, 256), (4096, 1024, 4096): (128, 128, 1, 256),
             (256, 11008, 4096): (128, 128, 1, 256), (4096, 4096, 1024): (256, 256, 1, 512)}
    for (m, n, k), want in cases.items():
        c = t0.auto_select(m, k, n)
        assert (c.tile_m, c.tile_n, max(c.split_k, 1), c.wg_size) == want, ((m, n, k), c.name())
    # skinny shapes: a split-K tile no taller than needed (within 3 % of the best there)
    c = t0.auto_select(128, 4096, 4096)
    assert c.tile_m <= 128 and c.split_k == 4


def test_auto_schedule_gemm_ranked_list():
    """src/t0/cost_model.rs:464-535: the ranked candidate list is sorted by
    predicted time, every entry is a feasible kernel of the requested layout
    and output type, its head is what auto_select picks (NT, f32), and the
    bf16-output list may split K (reduced in-kernel)."""
    for (m, n, k) in ((4096, 4096, 4096), (128, 4096, 4096), (16, 11008, 4096), (1000, 3000, 200)):
        lst = t0.auto_schedule_gemm(m, n, k, t0.NT, t0.OUT_F32)
        assert lst and all(a[1] <= b[1] for a, b in zip(lst, lst[1:]))
        assert all(c.transpose == t0.NT and c.out_dtype == t0.OUT_F32 for c, _ in lst)
        assert lst[0][0].name() == t0.auto_select(m, k, n).name()
        assert all(c.is_feasible() for c, _ in lst)
    sk = [c for c, _ in t0.auto_schedule_gemm(128, 4096, 4096, t0.NN, t0.OUT_BF16) if c.split_k > 1]
    assert sk and all(c.transpose == t0.NN and c.out_dtype == t0.OUT_BF16 for c in sk)


def test_auto_select_legacy_preserved():
    """src/t0/gemm_gen.rs:606-617."""
    c = t0.auto_select_legacy(256, 256, 256)
    assert c.split_k > 1 and c.tile_m == 64
    c = t0.auto_select_legacy(1024, 1024, 1024)
    assert c.tile_m == 128 and c.wgp_mode


def test_auto_select_domain_sample_feasible():
    """tests/tile_gemm_contract.rs:166-180."""
    n_checked = 0
    for m in (16, 31, 64, 128, 256, 1024, 4096):
        for n in (32, 64, 128, 256, 4096):
            for k in (16, 32, 64, 256, 4096):
                cfg = t0.auto_select(m, k, n)
                assert cfg.is_feasible(), (m, k, n, cfg.name())
                assert t0.cached_auto_select(m, k, n).name() == cfg.name()
                n_checked += 1
    assert n_checked >= 100


def test_backward_select_argument_order():
    """src/t0/gemm_gen.rs:510-549."""
    assert t0.auto_select_backward_data(64, 512, 256).name() == t0.auto_select(64, 512, 256).name()
    assert t0.auto_select_backward_weight(64, 512, 256).name() == t0.auto_select(512, 64, 256).name()


def test_sweep_and_standard_configs():
    sw = t0.sweep_configs()
    st = t0.standard_configs()
    assert len(st) == 16                       # src/t0/gemm_gen.rs:407-427
    assert sum(c.split_k > 1 for c in st) == 8
    assert all(c.is_feasible() for c in sw if c.wg_size >= 64)


def test_tile_auto_select_and_names():
    s = t0.tile_auto_select(4096, 4096, 4096)
    assert s.split_k == 1                      # auto split-K disabled (src/t0/tile_ir.rs:859)
    assert s.name().startswith(f"tile_gemm_{s.tile_m}x{s.tile_n}_k{s.tile_k}_db")
    s2 = t0.TileGemm.make(128, 64, 16, epilogue=["bias", "silu"])
    assert s2.name() == "tile_gemm_128x64_k16_db_bias_silu"
    g = s2.compute_grid(256, 128)
    assert g[0] % 64 == 0 and g[2] == 1


# ----------------------------------------------------------- GptqWeight --

def _gptq_fixture(rows=16, cols=16, gs=16, byte=0xAB, scale=1.0, zp=8):
    ng = cols // gs
    return (struct.pack("<III", rows, cols, gs) + bytes([byte]) * (rows * cols // 2)
            + struct.pack(f"<{rows * ng}f", *([scale] * rows * ng))
            + struct.pack(f"<{rows * ng}i", *([zp] * rows * ng)))


def test_gptq_from_bytes():
    """src/t0/quant_kernels.rs:384-422."""
    w = t0.GptqWeight.from_bytes(_gptq_fixture())
    assert (w.rows, w.cols, w.group_size, w.n_groups) == (16, 16, 16, 1)
    assert w.packed_weights.size == 128 and np.all(w.scales == 1.0) and np.all(w.zero_points == 8)
    assert w.gpu_buffer_size() == 256             # :480-490
    with pytest.raises(t0.T0Error):
        t0.GptqWeight.from_bytes(b"\x00" * 11)
    with pytest.raises(t0.T0Error):
        t0.GptqWeight.from_bytes(_gptq_fixture()[:-1])


def test_gptq_to_w4a16_matches_reference_dequant():
    rng = np.random.default_rng(9)
    rows, cols, gs = 64, 512, 128
    ng = cols // gs
    q = rng.integers(0, 16, size=rows * cols, dtype=np.uint8)
    packed = orc.int4_pack(q)
    # bf16-representable f32 scales, so the bf16 conversion is exact
    scales = orc.bf16_to_f32(orc.bf16_rne(rng.uniform(0.005, 0.02, rows * ng).astype(np.float32)))
    zps = rng.integers(0, 16, size=rows * ng).astype(np.int32)
    raw = orc.gptq_to_bytes(rows, cols, gs, packed, scales, zps)
    w = t0.GptqWeight.from_bytes(raw)
    qw, sc, zw = w.to_w4a16()
    assert qw.tobytes() == packed.tobytes()           # same bytes: [N][K/8] u32 view
    ref = orc.dequant_int4_f32(packed, scales, zps, rows, cols, gs)
    ours = orc.w4a16_dequant(qw, sc, zw, 0, rows, cols, gs)
    assert np.array_equal(ref.view(np.uint32), ours.view(np.uint32))
    qw2, sc2, _ = w.to_w4a16(scales_f32=True, with_zeros=False)
    assert np.array_equal(sc2, scales.reshape(rows, ng).T)


def test_gptq_rejects_out_of_range_zero_point():
    raw = _gptq_fixture(zp=16)
    with pytest.raises(t0.T0Error):
        t0.GptqWeight.from_bytes(raw).to_w4a16()


# ----------------------------------------------------- tuning cache on disk --

def _cfg_fields(c):
    return {f: getattr(c, f) for f, _ in t0.GemmConfig._fields_ if f != "reserved"}


def test_tuner_cache_roundtrip_keeps_wave_count(tmp_path):
    """A pick saved to disk and loaded back (a new process reads only the
    file) runs the same kernel: the 8-wave 256x256 instance that wins at
    4096^3 shares its name with the 4-wave one, so the file carries wg_size
    (src/t0/auto_gemm.rs:474-501 writes it too)."""
    t0.lib().t0_tuner_set_cache_dir(str(tmp_path).encode())
    try:
        pick = t0.auto_select(4096, 4096, 4096)
        assert pick.wg_size == 512
        assert t0.GemmConfig.from_name(pick.name()).wg_size != pick.wg_size   # the name alone loses it
        for tr, od in ((t0.NT, t0.OUT_F32), (t0.NN, t0.OUT_BF16)):
            c = pick.copy(transpose=tr, out_dtype=od)
            t0.GemmTuner.save_cache(4096, 4096, 4096, c, 1234.5, transpose=tr, out_dtype=od)
            back, tf = t0.GemmTuner.load_cache(4096, 4096, 4096, transpose=tr, out_dtype=od)
            assert _cfg_fields(back) == _cfg_fields(c) and tf == 1234.5
        # the reference's file name for NT / f32, a suffixed one otherwise
        assert (tmp_path / "gemm_4096x4096x4096.json").exists()
        assert (tmp_path / "gemm_4096x4096x4096_nn_bf16.json").exists()
        # a split-K pick round-trips too
        sk = t0.auto_select(128, 4096, 4096)
        t0.GemmTuner.save_cache(128, 4096, 4096, sk, 200.0)
        back, _ = t0.GemmTuner.load_cache(128, 4096, 4096)
        assert _cfg_fields(back) == _cfg_fields(sk)
        t0.GemmTuner.invalidate(128, 4096, 4096)
        assert t0.GemmTuner.load_cache(128, 4096, 4096) is None
    finally:
        t0.lib().t0_tuner_set_cache_dir(b"")


def test_tuner_cache_reads_reference_files_and_rejects_unusable(tmp_path):
    """A file in the reference's own format (no arch field) loads as an NT /
    f32 config; a split_k the kernels cannot run, a tile without a gfx950
    kernel, or another architecture's file is ignored (NOT_FOUND), so the
    tuner ranks afresh instead of failing every later call."""
    t0.lib().t0_tuner_set_cache_dir(str(tmp_path).encode())
    try:
        ref = ('{"tile_m":128,"tile_n":64,"tile_k":32,"wg_size":128,"split_k":2,"lds_pad":0,'
               '"n_col_passes":1,"wgp":true,"swap":false,"tflops":79.20,"all":[["t0_gemm_128x64_k32_ldsdb",79.2]]}')
        (tmp_path / "gemm_1024x1024x1024.json").write_text(ref)
        c, tf = t0.GemmTuner.load_cache(1024, 1024, 1024)
        assert (c.tile_m, c.tile_n, c.tile_k, c.wg_size, c.split_k, c.wgp_mode, c.swap_grid) == (128, 64, 32, 128, 2, 1, 0)
        assert tf == pytest.approx(79.2) and c.transpose == t0.NT and c.out_dtype == t0.OUT_F32
        for bad in (ref.replace('"split_k":2', '"split_k":3'), ref.replace('"split_k":2', '"split_k":32'),
                    ref.replace('"tile_m":128', '"tile_m":96'), ref.replace('"wg_size":128', '"wg_size":192'),
                    ref.replace('"tflops":79.20', '"tflops":"x"'), ref[:-1] + ',"arch":"gfx1100"}', "{}"):
            (tmp_path / "gemm_1024x1024x1024.json").write_text(bad)
            assert t0.GemmTuner.load_cache(1024, 1024, 1024) is None, bad
        # storing a config no kernel runs is refused
        with pytest.raises(t0.T0Error):
            t0.GemmTuner.save_cache(64, 64, 64, t0.GemmConfig.tile_128x64_k16().copy(wg_size=192), 1.0)
    finally:
        t0.lib().t0_tuner_set_cache_dir(b"")


def test_tuner_all_list_on_disk(tmp_path):
    """GemmTuneResult.all (src/t0/auto_gemm.rs:30-42, written at :480-494):
    the cache file's "all" list comes back through t0_tune_results, fastest
    first with each entry's wave count; entries in the reference's two-element
    form load with the name's instance; entries no gfx950 kernel runs are
    skipped; another architecture's file, or none, is NOT_FOUND."""
    t0.lib().t0_tuner_set_cache_dir(str(tmp_path).encode())
    try:
        assert t0.GemmTuner.results(512, 512, 512) is None
        pick = t0.auto_select(4096, 4096, 4096)
        t0.GemmTuner.save_cache(4096, 4096, 4096, pick, 1234.5)
        text = (tmp_path / "gemm_4096x4096x4096.json").read_text()
        assert f'"all":[["{pick.name()}",1234.50,{pick.wg_size}]]' in text, text
        lst, cached = t0.GemmTuner.results(4096, 4096, 4096)
        assert cached and len(lst) == 1
        assert _cfg_fields(lst[0][0]) == _cfg_fields(pick) and lst[0][1] == pytest.approx(1234.5)
        # a file as a tuning run writes it: several entries, fastest first
        a = t0.GemmConfig.tile_128x128_k64()
        b = t0.auto_select(128, 4096, 4096)
        doc = ('{"tile_m":%d,"tile_n":%d,"tile_k":%d,"wg_size":%d,"split_k":%d,"lds_pad":0,"n_col_passes":1,'
               '"wgp":false,"swap":true,"tflops":900.00,"all":[["%s",900.00,%d],["%s",800.50],'
               '["t0_gemm_96x64_k64_ldsdb",700.0,256],["%s",650.0,192]],"arch":"gfx950"}'
               % (a.tile_m, a.tile_n, a.tile_k, a.wg_size, max(a.split_k, 1), a.name(), a.wg_size, b.name(),
                  a.name()))
        (tmp_path / "gemm_2048x2048x2048.json").write_text(doc)
        lst, cached = t0.GemmTuner.results(2048, 2048, 2048)
        assert cached
        assert [(c.name(), c.wg_size, tf) for c, tf in lst] == \
            [(a.name(), a.wg_size, 900.0), (b.name(), t0.GemmConfig.from_name(b.name()).wg_size, 800.5)]
        (tmp_path / "gemm_2048x2048x2048.json").write_text(doc.replace('"gfx950"', '"gfx1100"'))
        assert t0.GemmTuner.results(2048, 2048, 2048) is None
        t0.GemmTuner.invalidate(4096, 4096, 4096)
        assert t0.GemmTuner.results(4096, 4096, 4096) is None
    finally:
        t0.lib().t0_tuner_set_cache_dir(b"")


def test_tuner_default_directory_is_not_the_references(tmp_path, monkeypatch):
    """Without a directory set, the cache lives in ~/.t0_autotune_gfx950: the
    reference's loader (src/t0/auto_gemm.rs:439-472) ignores "arch" and would
    take gfx950-only configs from its own ~/.t0_autotune."""
    monkeypatch.setenv("HOME", str(tmp_path))
    monkeypatch.delenv("T0_AUTOTUNE_DIR", raising=False)
    t0.lib().t0_tuner_set_cache_dir(b"")
    try:
        t0.GemmTuner.save_cache(256, 256, 256, t0.auto_select(256, 256, 256), 1.0)
        assert (tmp_path / ".t0_autotune_gfx950" / "gemm_256x256x256.json").exists()
        assert not (tmp_path / ".t0_autotune").exists()
    finally:
        t0.lib().t0_tuner_set_cache_dir(b"")

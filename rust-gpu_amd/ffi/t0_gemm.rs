//! Rust FFI for `libt0gpu.so`: every type, constant and function that
//! `include/t0_gemm.h` declares, field for field and argument for argument.
//!
//! Drop it into the reference crate as `src/t0/ffi.rs` (`pub mod ffi;` in
//! `src/t0/mod.rs`) and link the library from `build.rs`
//! (`cargo:rustc-link-lib=dylib=t0gpu`).  The reference items each call
//! replaces are cited on the declarations; the reference's public surface
//! (`src/prelude.rs:11-19`, `src/t0/mod.rs:76-83`) keeps its signatures and
//! calls through these.  Edition 2021; `unsafe extern` as in the reference's
//! own `src/kfd/ioctl.rs`.
//!
//! Every function returns `T0_OK` (0) or a negative status; `check` turns a
//! status into the reference's `Result<_, String>` with the message of
//! `t0_last_error`.  Device pointers are `u64` addresses, bf16 data raw
//! little-endian `u16`, grids in work-items.

#![allow(non_camel_case_types, non_upper_case_globals, dead_code)]

use std::os::raw::{c_char, c_int, c_void};

// ----------------------------------------------------------------- status
pub type t0_status = c_int;
pub const T0_OK: c_int = 0;
pub const T0_ERR_INVALID: c_int = -1;
pub const T0_ERR_INFEASIBLE: c_int = -2;
pub const T0_ERR_HIP: c_int = -3;
pub const T0_ERR_POISONED: c_int = -4;
pub const T0_ERR_KERNARG: c_int = -5;
pub const T0_ERR_NOT_FOUND: c_int = -6;
pub const T0_ERR_NO_DEVICE: c_int = -7;

// ------------------------------------------------------------- GemmConfig
/// gemm_gen::GemmTranspose (src/t0/gemm_gen.rs:22-29).
pub const T0_NT: u32 = 0;
pub const T0_NN: u32 = 1;
/// gemm_gen::EpilogueOp (src/t0/gemm_gen.rs:39-49).
pub const T0_EPI_STORE_F32: u32 = 0;
pub const T0_EPI_BIAS_ADD: u32 = 1;
pub const T0_EPI_BIAS_ADD_RELU: u32 = 2;
/// Output element type (the reference always stores f32).
pub const T0_OUT_F32: u32 = 0;
pub const T0_OUT_BF16: u32 = 1;

/// gemm_gen::GemmConfig (src/t0/gemm_gen.rs:55-84).  `split_k` 0 or 1 is no
/// split; `wg_size` counts 64-lane waves times 64.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct t0_gemm_config {
    pub tile_m: u32,
    pub tile_n: u32,
    pub tile_k: u32,
    pub wg_size: u32,
    pub split_k: u32,
    pub lds_pad: u32,
    pub n_col_passes: u32,
    pub use_lds: u8,
    pub double_buffer: u8,
    pub swap_grid: u8,
    pub wgp_mode: u8,
    pub transpose: u8,
    pub epilogue: u8,
    pub out_dtype: u8,
    pub reserved: u8,
}

/// GemmConfig::tile_* presets (src/t0/gemm_gen.rs:86-145) and the gfx950 tiles.
pub type t0_preset = c_int;
pub const T0_PRESET_16x64_K16: c_int = 0;
pub const T0_PRESET_32x64_DIRECT: c_int = 1;
pub const T0_PRESET_32x64_K16: c_int = 2;
pub const T0_PRESET_32x64_K32: c_int = 3;
pub const T0_PRESET_32x128_K16: c_int = 4;
pub const T0_PRESET_64x64_K16: c_int = 5;
pub const T0_PRESET_64x64_K32: c_int = 6;
pub const T0_PRESET_128x64_K16: c_int = 7;
pub const T0_PRESET_64x128_K16: c_int = 8;
pub const T0_PRESET_128x64_K32: c_int = 9;
pub const T0_PRESET_128x128_K16: c_int = 10;
pub const T0_PRESET_64x64_K64: c_int = 11;
pub const T0_PRESET_128x128_2PASS: c_int = 12;
pub const T0_PRESET_64x128_2PASS: c_int = 13;
pub const T0_PRESET_256x256_K64: c_int = 14;
pub const T0_PRESET_256x128_K64: c_int = 15;
pub const T0_PRESET_128x256_K64: c_int = 16;
pub const T0_PRESET_128x128_K64: c_int = 17;
pub const T0_PRESET_128x128_K32: c_int = 18;
pub const T0_PRESET_128x64_K64: c_int = 19;
pub const T0_PRESET_64x128_K64: c_int = 20;
pub const T0_PRESET_32x64_K64: c_int = 21;
pub const T0_PRESET_32x128_K64: c_int = 22;
pub const T0_PRESET_256x256_K32: c_int = 23;
pub const T0_PRESET_COUNT: c_int = 24;

/// GemmConfig's derived geometry (src/t0/gemm_gen.rs:147-213), for wave64
/// and 32x32x16 MFMA blocks.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct t0_gemm_geometry {
    pub n_waves: u32,
    pub waves_m: u32,
    pub waves_n: u32,
    pub rows_per_wave: u32,
    pub cols_per_wave: u32,
    pub n_row_blocks: u32,
    pub n_col_tiles: u32,
    pub k_sub_steps: u32,
    pub stages: u32,
    pub lds_per_buffer: u32,
    pub lds_total: u32,
    pub x_bytes_per_thread: u32,
    pub wt_bytes_per_thread: u32,
    pub mfma_per_k_tile: u32,
    pub estimated_vgprs: u32,
}

// ------------------------------------------------------ TileGemm (tile_ir)
/// tile_ir::EpilogueOp (src/t0/tile_ir.rs:41-62).
pub const T0_TEPI_BIAS: u8 = 1;
pub const T0_TEPI_SCALE: u8 = 2;
pub const T0_TEPI_RELU: u8 = 3;
pub const T0_TEPI_SILU: u8 = 4;
pub const T0_TEPI_GELU: u8 = 5;
pub const T0_TEPI_ABS: u8 = 6;
pub const T0_TEPI_NEG: u8 = 7;
pub const T0_TEPI_CLAMP: u8 = 8;

/// tile_ir::TileGemm (src/t0/tile_ir.rs:109-152); `waves_per_wg` 0 = default.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct t0_tile_gemm {
    pub tile_m: u32,
    pub tile_n: u32,
    pub tile_k: u32,
    pub split_k: u32,
    pub waves_per_wg: u32,
    pub wgp_mode: u8,
    pub double_buffer: u8,
    pub triple_buffer: u8,
    pub swap_grid: u8,
    pub transpose: u8,
    pub acc_swap: u8,
    pub persistent: u8,
    pub out_dtype: u8,
    pub n_epilogue: u8,
    pub epilogue: [u8; 8],
    pub reserved: [u8; 3],
}

// ---------------------------------------------------------------- runtime
/// GpuRuntime (src/ignis/gpu_context.rs:99-119), opaque.
#[repr(C)]
pub struct t0_runtime {
    _private: [u8; 0],
    _marker: core::marker::PhantomData<(*mut u8, core::marker::PhantomPinned)>,
}
/// GpuKernel (src/kfd/kernel.rs:8-19), opaque.
#[repr(C)]
pub struct t0_kernel {
    _private: [u8; 0],
    _marker: core::marker::PhantomData<(*mut u8, core::marker::PhantomPinned)>,
}
/// GpuBuffer, opaque.
#[repr(C)]
pub struct t0_buffer {
    _private: [u8; 0],
    _marker: core::marker::PhantomData<(*mut u8, core::marker::PhantomPinned)>,
}
/// A HIP event on the runtime's stream, opaque.
#[repr(C)]
pub struct t0_event {
    _private: [u8; 0],
    _marker: core::marker::PhantomData<(*mut u8, core::marker::PhantomPinned)>,
}
/// A captured HIP graph, opaque.
#[repr(C)]
pub struct t0_graph {
    _private: [u8; 0],
    _marker: core::marker::PhantomData<(*mut u8, core::marker::PhantomPinned)>,
}

/// KernelLoadConfig (src/kfd/kernel.rs:26-141).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct t0_kernel_load_config {
    pub workgroup_size: [u32; 3],
    pub lds_size: u32,
    pub kernarg_size: u32,
}

// -------------------------------------------------------- high-level GEMM
/// One GEMM, C = epilogue(A . B) (auto_gemm, src/t0/auto_gemm.rs:555-590).
/// A bf16 [M, lda]; B: NT -> WT [N, ldb], NN -> B [K, ldb]; C [M, ldc];
/// leading dimensions 0 = dense.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq)]
pub struct t0_gemm_desc {
    pub a: u64,
    pub b: u64,
    pub c: u64,
    pub bias: u64,
    pub m: u32,
    pub n: u32,
    pub k: u32,
    pub lda: u32,
    pub ldb: u32,
    pub ldc: u32,
    pub transpose: u32,
    pub out_dtype: u32,
    pub n_epilogue: u32,
    pub epilogue: [u8; 8],
    pub scale: f32,
    pub clamp_min: f32,
    pub clamp_max: f32,
}

/// Size of the per-device scratch array of `t0_gemm_noalloc`.
pub const T0_NOALLOC_SCRATCH_BYTES: u32 = 32 << 20;
/// Most output tiles one `t0_gemm_noalloc` call may have.
pub const T0_NOALLOC_MAX_TILES: u32 = 16384;

/// One timed candidate of `t0_tune` (GemmTuneResult.all, src/t0/auto_gemm.rs:30-42).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq)]
pub struct t0_tune_entry {
    pub cfg: t0_gemm_config,
    pub tflops: f64,
}

/// One timed candidate of `t0_tile_tune` (TileIrTuneResult, src/t0/cost_model.rs:824-860).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq)]
pub struct t0_tile_tune_entry {
    pub spec: t0_tile_gemm,
    pub tflops: f64,
}

// ------------------------------------------------------------------- INT4
/// GptqWeight viewed in place (src/t0/quant_kernels.rs:188-296).
#[repr(C)]
#[derive(Clone, Copy, Debug, PartialEq)]
pub struct t0_gptq_view {
    pub rows: u32,
    pub cols: u32,
    pub group_size: u32,
    pub n_groups: u32,
    pub packed: *const u8,
    pub scales: *const f32,
    pub zero_points: *const i32,
}

impl Default for t0_gptq_view {
    fn default() -> Self {
        t0_gptq_view {
            rows: 0,
            cols: 0,
            group_size: 0,
            n_groups: 0,
            packed: core::ptr::null(),
            scales: core::ptr::null(),
            zero_points: core::ptr::null(),
        }
    }
}

/// W4A16 GEMM (no counterpart in the reference): C = A . ((q - z) * s)^T.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub struct t0_w4a16_desc {
    pub a: u64,
    pub qweight: u64,
    pub scales: u64,
    pub zeros: u64,
    pub c: u64,
    pub m: u32,
    pub n: u32,
    pub k: u32,
    pub lda: u32,
    pub ldc: u32,
    pub group_size: u32,
    pub zero_const: u32,
    pub scales_f32: u32,
    pub out_f32: u32,
    pub split_k: u32,
}

// ------------------------------------------- residual add + RMSNorm ------
/// The norm in front of an INT4 projection (src/ignis/ops/fused_rmsnorm_gemm.rs:33-154).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq)]
pub struct t0_rmsnorm_desc {
    pub residual: u64,
    pub hidden: u64,
    pub gamma: u64,
    pub x2_out: u64,
    pub eps: f32,
    pub pad_: u32,
}

unsafe extern "C" {
    pub fn t0_last_error() -> *const c_char;
    pub fn t0_version() -> *const c_char;

    // GemmConfig presets, geometry, feasibility, names (src/t0/gemm_gen.rs:86-250, :407-427)
    pub fn t0_config_preset(preset: c_int, out: *mut t0_gemm_config) -> c_int;
    pub fn t0_config_geometry(cfg: *const t0_gemm_config, out: *mut t0_gemm_geometry) -> c_int;
    pub fn t0_config_is_feasible(cfg: *const t0_gemm_config) -> c_int;
    pub fn t0_config_name(cfg: *const t0_gemm_config, buf: *mut c_char, len: usize) -> c_int;
    pub fn t0_config_from_name(name: *const c_char, out: *mut t0_gemm_config) -> c_int;
    pub fn t0_sweep_configs(out: *mut t0_gemm_config, cap: usize) -> c_int;
    pub fn t0_standard_configs(out: *mut t0_gemm_config, cap: usize) -> c_int;

    // grids and kernargs (src/t0/gemm_gen.rs:308-329, :430-484, :510-570)
    pub fn t0_compute_grid(cfg: *const t0_gemm_config, m: u32, n: u32, gx: *mut u32, gy: *mut u32) -> c_int;
    pub fn t0_compute_grid_split_k(cfg: *const t0_gemm_config, m: u32, n: u32, split_k: u32, gx: *mut u32,
                                   gy: *mut u32) -> c_int;
    pub fn t0_compute_grid_auto(cfg: *const t0_gemm_config, m: u32, n: u32, gx: *mut u32, gy: *mut u32) -> c_int;
    pub fn t0_build_kernargs(x: u64, wt: u64, y: u64, k: u32, n: u32, m: u32, cfg: *const t0_gemm_config,
                             out: *mut [u8; 40]) -> c_int;
    pub fn t0_build_kernargs_with_bias(x: u64, wt: u64, y: u64, k: u32, n: u32, m: u32,
                                       cfg: *const t0_gemm_config, bias: u64, out: *mut [u8; 48]) -> c_int;
    pub fn t0_auto_select_backward_data(m: u32, n_orig: u32, k_orig: u32, out: *mut t0_gemm_config) -> c_int;
    pub fn t0_auto_select_backward_weight(m: u32, n_orig: u32, k_orig: u32, out: *mut t0_gemm_config) -> c_int;
    pub fn t0_build_kernargs_backward_data(dy: u64, w: u64, dx: u64, m: u32, n_orig: u32, k_orig: u32,
                                           cfg: *const t0_gemm_config, out: *mut [u8; 40]) -> c_int;
    pub fn t0_build_kernargs_backward_weight(dy_t: u64, x_t: u64, dw: u64, m: u32, n_orig: u32, k_orig: u32,
                                             cfg: *const t0_gemm_config, out: *mut [u8; 40]) -> c_int;

    // auto-selection (src/t0/gemm_gen.rs:340-404, src/t0/cost_model.rs:464-668,
    // src/t0/prefill_spec_cache.rs:55-129); note the argument order (m, k, n)
    pub fn t0_auto_select(m: u32, k: u32, n: u32, out: *mut t0_gemm_config) -> c_int;
    pub fn t0_auto_select_legacy(m: u32, k: u32, n: u32, out: *mut t0_gemm_config) -> c_int;
    pub fn t0_auto_schedule_gemm(m: u32, n: u32, k: u32, transpose: u32, out_dtype: u32, out: *mut t0_gemm_config,
                                 est_us: *mut f64, cap: u32) -> c_int;
    pub fn t0_cached_auto_select(m: u32, k: u32, n: u32, out: *mut t0_gemm_config) -> c_int;
    pub fn t0_prewarm_cache(mkn_triples: *const u32, count: usize) -> c_int;

    // tile_ir (src/t0/tile_ir.rs:697-870, :4595-4667)
    pub fn t0_tile_name(spec: *const t0_tile_gemm, buf: *mut c_char, len: usize) -> c_int;
    pub fn t0_tile_auto_select(m: u32, k: u32, n: u32, transpose: c_int, out: *mut t0_tile_gemm) -> c_int;
    pub fn t0_tile_build_kernargs_m(x: u64, wt: u64, y: u64, k: u32, n: u32, m: u32, spec: *const t0_tile_gemm,
                                    y_split_stride: u32, bias: u64, scale: f32, clamp_min: f32, clamp_max: f32,
                                    out: *mut u8, len: *mut usize) -> c_int;
    pub fn t0_tile_compute_grid(spec: *const t0_tile_gemm, m: u32, n: u32, grid: *mut [u32; 3]) -> c_int;

    // runtime (src/ignis/gpu_context.rs:151-210)
    pub fn t0_runtime_create(device_ordinal: c_int, out: *mut *mut t0_runtime) -> c_int;
    pub fn t0_runtime_destroy(rt: *mut t0_runtime) -> c_int;
    pub fn t0_runtime_set_stream(rt: *mut t0_runtime, hip_stream: *mut c_void) -> c_int;
    pub fn t0_runtime_stream(rt: *mut t0_runtime) -> *mut c_void;
    pub fn t0_runtime_is_poisoned(rt: *const t0_runtime) -> c_int;
    pub fn t0_runtime_mark_poisoned(rt: *mut t0_runtime) -> c_int;
    pub fn t0_runtime_device_info(rt: *const t0_runtime, arch: *mut c_char, arch_len: usize, cu_count: *mut c_int,
                                  clock_khz: *mut c_int) -> c_int;

    // code object and kernel loading (src/t0/gemm_gen.rs:261-297, src/t0/compile.rs:1398-1455,
    // src/kfd/kernel.rs:26-141, src/ignis/gpu_context.rs:200-259)
    pub fn t0_code_object(data: *mut *const c_void, size: *mut usize) -> c_int;
    pub fn t0_generate(cfg: *const t0_gemm_config, symbol: *mut c_char, symbol_len: usize) -> c_int;
    pub fn t0_kernel_load(rt: *mut t0_runtime, code_object: *const c_void, size: usize, symbol: *const c_char,
                          cfg: *const t0_kernel_load_config, out: *mut *mut t0_kernel) -> c_int;
    pub fn t0_ensure_kernel(rt: *mut t0_runtime, cfg: *const t0_gemm_config, out: *mut *mut t0_kernel) -> c_int;
    pub fn t0_ensure_tile_kernel(rt: *mut t0_runtime, spec: *const t0_tile_gemm, out: *mut *mut t0_kernel) -> c_int;
    pub fn t0_get_kernel(rt: *mut t0_runtime, name: *const c_char, out: *mut *mut t0_kernel) -> c_int;
    pub fn t0_kernel_info(k: *const t0_kernel, wg: *mut [u32; 3], lds: *mut u32, kernarg_size: *mut u32,
                          name: *mut c_char, name_len: usize) -> c_int;

    // dispatch (src/ignis/gpu_context.rs:305-452)
    pub fn t0_dispatch(rt: *mut t0_runtime, k: *const t0_kernel, grid: *const [u32; 3], kernargs: *const c_void,
                       len: usize) -> c_int;
    pub fn t0_dispatch_async(rt: *mut t0_runtime, k: *const t0_kernel, grid: *const [u32; 3],
                             kernargs: *const c_void, len: usize) -> c_int;
    pub fn t0_wait_idle(rt: *mut t0_runtime) -> c_int;
    pub fn t0_synchronize(rt: *mut t0_runtime) -> c_int;

    // memory (src/ignis/gpu_context.rs:31-92, :508-542)
    pub fn t0_alloc(rt: *mut t0_runtime, bytes: usize, out: *mut *mut t0_buffer) -> c_int;
    pub fn t0_recycle(rt: *mut t0_runtime, buf: *mut t0_buffer) -> c_int;
    pub fn t0_buffer_free(buf: *mut t0_buffer) -> c_int;
    pub fn t0_buffer_addr(buf: *const t0_buffer) -> u64;
    pub fn t0_buffer_size(buf: *const t0_buffer) -> usize;
    pub fn t0_buffer_write(buf: *mut t0_buffer, offset: usize, src: *const c_void, len: usize) -> c_int;
    pub fn t0_buffer_read(buf: *const t0_buffer, offset: usize, dst: *mut c_void, len: usize) -> c_int;
    pub fn t0_buffer_zero(buf: *mut t0_buffer) -> c_int;
    pub fn t0_read_f32(buf: *const t0_buffer, dst: *mut f32, count: usize) -> c_int;
    pub fn t0_memcpy_h2d(rt: *mut t0_runtime, dst: u64, src: *const c_void, len: usize) -> c_int;
    pub fn t0_memcpy_d2h(rt: *mut t0_runtime, dst: *mut c_void, src: u64, len: usize) -> c_int;
    pub fn t0_memset_d(rt: *mut t0_runtime, dst: u64, value: c_int, len: usize) -> c_int;

    // events and graphs (timing; no counterpart in the reference)
    pub fn t0_event_create(out: *mut *mut t0_event) -> c_int;
    pub fn t0_event_destroy(ev: *mut t0_event) -> c_int;
    pub fn t0_event_record(rt: *mut t0_runtime, ev: *mut t0_event) -> c_int;
    pub fn t0_event_synchronize(ev: *mut t0_event) -> c_int;
    pub fn t0_event_elapsed_ms(start: *const t0_event, stop: *const t0_event, ms: *mut f32) -> c_int;
    pub fn t0_graph_begin(rt: *mut t0_runtime) -> c_int;
    pub fn t0_graph_end(rt: *mut t0_runtime, out: *mut *mut t0_graph) -> c_int;
    pub fn t0_graph_launch(rt: *mut t0_runtime, g: *const t0_graph) -> c_int;
    pub fn t0_graph_destroy(g: *mut t0_graph) -> c_int;

    // one GEMM (src/t0/auto_gemm.rs:555-590)
    pub fn t0_gemm(rt: *mut t0_runtime, cfg: *const t0_gemm_config, d: *const t0_gemm_desc) -> c_int;
    pub fn t0_gemm_select(rt: *mut t0_runtime, d: *const t0_gemm_desc, out: *mut t0_gemm_config) -> c_int;
    pub fn t0_gemm_clock_probe(rt: *mut t0_runtime, cfg: *const t0_gemm_config, d: *const t0_gemm_desc,
                               sclk_mhz: *mut f64, span_us: *mut f64, wg_cycles: *mut f64) -> c_int;
    pub fn t0_gemm_noalloc(rt: *mut t0_runtime, cfg: *const t0_gemm_config, d: *const t0_gemm_desc) -> c_int;

    // tuner (src/t0/auto_gemm.rs:82-590, src/t0/cost_model.rs:824-1080)
    pub fn t0_tune(rt: *mut t0_runtime, m: u32, n: u32, k: u32, transpose: u32, out_dtype: u32,
                   cfg_out: *mut t0_gemm_config, tflops_out: *mut f64) -> c_int;
    pub fn t0_tuner_set_cache_dir(dir: *const c_char) -> c_int;
    pub fn t0_tuner_set_params(max_candidates: u32, n_iters: u32) -> c_int;
    pub fn t0_tuner_cache_store(m: u32, n: u32, k: u32, transpose: u32, out_dtype: u32, cfg: *const t0_gemm_config,
                                tflops: f64) -> c_int;
    pub fn t0_tuner_cache_load(m: u32, n: u32, k: u32, transpose: u32, out_dtype: u32, cfg: *mut t0_gemm_config,
                               tflops: *mut f64) -> c_int;
    pub fn t0_tuner_invalidate(m: u32, n: u32, k: u32, transpose: u32, out_dtype: u32) -> c_int;
    pub fn t0_tune_results(m: u32, n: u32, k: u32, transpose: u32, out_dtype: u32, all: *mut t0_tune_entry, cap: u32,
                           n_all: *mut u32, from_cache: *mut c_int) -> c_int;
    pub fn t0_auto_gemm(rt: *mut t0_runtime, a: u64, b: u64, c: u64, m: u32, n: u32, k: u32,
                        tflops_out: *mut f64) -> c_int;
    pub fn t0_tile_tune(rt: *mut t0_runtime, m: u32, n: u32, k: u32, best: *mut t0_tile_gemm, best_tflops: *mut f64,
                        all: *mut t0_tile_tune_entry, cap: u32, n_all: *mut u32, from_cache: *mut c_int) -> c_int;

    // INT4 (src/t0/quant_kernels.rs:53-296) and the fused W4A16 GEMM (new)
    pub fn t0_gptq_from_bytes(raw: *const c_void, len: usize, out: *mut t0_gptq_view) -> c_int;
    pub fn t0_gptq_gpu_buffer_size(w: *const t0_gptq_view) -> usize;
    pub fn t0_gptq_to_w4a16(w: *const t0_gptq_view, qweight: *mut u32, scales: *mut c_void, scales_f32: c_int,
                            zeros: *mut u32) -> c_int;
    pub fn t0_dequant_int4(rt: *mut t0_runtime, packed: u64, scales: u64, zero_points: u64, output: u64, rows: u32,
                           cols: u32, group_size_log2: u32, bf16_out: c_int) -> c_int;
    pub fn t0_w4a16_gemm(rt: *mut t0_runtime, d: *const t0_w4a16_desc) -> c_int;
    pub fn t0_w4a16_plan(rt: *mut t0_runtime, d: *const t0_w4a16_desc, kernel: *mut c_char, len: usize,
                         split_k: *mut u32) -> c_int;

    // small kernels (examples/hello_gemm_gen.rs:125-136, src/ignis/ops/bf16_matmul.rs:356-383,
    // src/t0/math.rs) and measurement aids (no counterpart in the reference)
    pub fn t0_splitk_reduce(rt: *mut t0_runtime, src: u64, plane_stride: u64, planes: u32, dst: u64, m: u32, n: u32,
                            out_bf16: c_int) -> c_int;
    pub fn t0_f32_to_bf16(rt: *mut t0_runtime, src: u64, dst: u64, count: u64) -> c_int;
    pub fn t0_copy_device(rt: *mut t0_runtime, src: u64, dst: u64, bytes: u64) -> c_int;
    pub fn t0_floor_stream_read(rt: *mut t0_runtime, src: u64, bytes: u64, sink: u64, workgroups: u32,
                                threads: u32) -> c_int;
    pub fn t0_floor_empty(rt: *mut t0_runtime, workgroups: u32, threads: u32) -> c_int;
    pub fn t0_floor_tile_read(rt: *mut t0_runtime, cfg: *const t0_gemm_config, d: *const t0_gemm_desc,
                              mode: c_int) -> c_int;
    pub fn t0_floor_mfma(rt: *mut t0_runtime, operands: u64, out: u64, workgroups: u32, mfma_per_wave: u32) -> c_int;
    pub fn t0_floor_lds(rt: *mut t0_runtime, mode: c_int, src: u64, out: u64, workgroups: u32, threads: u32,
                        rounds: u32) -> c_int;
    pub fn t0_unpad_2d(rt: *mut t0_runtime, padded: u64, out: u64, m: u32, n: u32, n_pad: u32) -> c_int;

    // Ignis bf16 matmul (src/ignis/ops/bf16_matmul.rs:33-423): f32 device buffers, f32 out
    pub fn t0_bf16_matmul(rt: *mut t0_runtime, x: u64, w: u64, y: u64, m: u32, k: u32, n: u32) -> c_int;
    pub fn t0_bf16_matmul_backward_data(rt: *mut t0_runtime, dy: u64, w: u64, dx: u64, m: u32, k: u32,
                                        n: u32) -> c_int;
    pub fn t0_bf16_matmul_backward_weight(rt: *mut t0_runtime, x: u64, dy: u64, dw: u64, m: u32, k: u32,
                                          n: u32) -> c_int;
    pub fn t0_bf16_matmul_with_wt_bf16(rt: *mut t0_runtime, x: u64, wt: u64, y: u64, m: u32, k: u32,
                                       n: u32) -> c_int;

    // residual add + RMSNorm (src/t0/ffn_fused_kernels.rs:54-237, src/t0/rmsnorm_kernels.rs:140-153,
    // src/ignis/ops/fused_rmsnorm_gemm.rs:33-154)
    pub fn t0_ffn_fused_rmsnorm_gemm(rt: *mut t0_runtime, residual: u64, hidden: u64, gamma: u64, weight: u64,
                                     output: u64, m: u32, d: u32, eps: f32) -> c_int;
    pub fn t0_rmsnorm(rt: *mut t0_runtime, residual: u64, hidden: u64, gamma: u64, out: u64, x2_out: u64, rows: u32,
                      d: u32, ld_out: u32, eps: f32, out_bf16: c_int) -> c_int;
    pub fn t0_rmsnorm_w4a16(rt: *mut t0_runtime, d: *const t0_w4a16_desc, nd: *const t0_rmsnorm_desc) -> c_int;
    pub fn t0_rmsnorm_matmul(rt: *mut t0_runtime, residual: u64, hidden: u64, gamma: u64, w: u64, y: u64,
                             x2_out: u64, m: u32, k: u32, n: u32, eps: f32) -> c_int;
}

/// A status as the reference's `Result<_, String>`: negative statuses carry
/// the message of the calling thread's last failure.
pub fn check(rc: c_int) -> Result<c_int, String> {
    if rc >= 0 {
        return Ok(rc);
    }
    // SAFETY: t0_last_error returns a NUL-terminated string owned by the
    // library's thread-local storage, valid until the next call on this thread.
    let msg = unsafe { std::ffi::CStr::from_ptr(t0_last_error()) };
    Err(format!("t0 error {}: {}", rc, msg.to_string_lossy()))
}

/// A NUL-terminated name written by one of the `*_name` / `t0_generate`
/// calls into `buf`, as a `String`.
pub fn name_from(buf: &[u8]) -> String {
    let end = buf.iter().position(|&b| b == 0).unwrap_or(buf.len());
    String::from_utf8_lossy(&buf[..end]).into_owned()
}

/// tile_ir::tile_auto_select (src/t0/tile_ir.rs:740-870) through the library.
pub fn tile_auto_select(m: u32, k: u32, n: u32, transpose: bool) -> Result<t0_tile_gemm, String> {
    let mut spec = t0_tile_gemm::default();
    // SAFETY: `spec` is a valid, writable t0_tile_gemm.
    check(unsafe { t0_tile_auto_select(m, k, n, transpose as c_int, &mut spec) })?;
    Ok(spec)
}

/// tile_ir::TileGemm::name (src/t0/tile_ir.rs:697-728).
pub fn tile_name(spec: &t0_tile_gemm) -> Result<String, String> {
    let mut buf = [0u8; 128];
    // SAFETY: `buf` holds `buf.len()` writable bytes.
    check(unsafe { t0_tile_name(spec, buf.as_mut_ptr() as *mut c_char, buf.len()) })?;
    Ok(name_from(&buf))
}

/// tile_ir::build_kernargs_m (src/t0/tile_ir.rs:4595-4602) with the
/// epilogue arguments that follow it: the kernarg bytes, 44 to 84 of them.
pub fn tile_build_kernargs_m(x: u64, wt: u64, y: u64, k: u32, n: u32, m: u32, spec: &t0_tile_gemm,
                             y_split_stride: u32, bias: u64, scale: f32, clamp: (f32, f32))
                             -> Result<Vec<u8>, String> {
    let mut out = [0u8; 96];
    let mut len: usize = 0;
    // SAFETY: `out` holds the 96 bytes the call may write; `len` is writable.
    check(unsafe {
        t0_tile_build_kernargs_m(x, wt, y, k, n, m, spec, y_split_stride, bias, scale, clamp.0, clamp.1,
                                 out.as_mut_ptr(), &mut len)
    })?;
    Ok(out[..len].to_vec())
}

/// tile_ir::compute_grid (src/t0/tile_ir.rs:4645-4667), in work-items.
pub fn tile_compute_grid(spec: &t0_tile_gemm, m: u32, n: u32) -> Result<[u32; 3], String> {
    let mut grid = [0u32; 3];
    // SAFETY: `grid` is a valid [u32; 3].
    check(unsafe { t0_tile_compute_grid(spec, m, n, &mut grid) })?;
    Ok(grid)
}

/// The config `t0_gemm` would run for `d` when given none.
pub fn gemm_select(rt: *mut t0_runtime, d: &t0_gemm_desc) -> Result<t0_gemm_config, String> {
    let mut cfg = t0_gemm_config::default();
    // SAFETY: `rt` comes from t0_runtime_create; `cfg` is writable.
    check(unsafe { t0_gemm_select(rt, d, &mut cfg) })?;
    Ok(cfg)
}

/// One GEMM with `cfg` (None: the library's selection).
pub fn gemm(rt: *mut t0_runtime, cfg: Option<&t0_gemm_config>, d: &t0_gemm_desc) -> Result<(), String> {
    let cfg_ptr = cfg.map_or(core::ptr::null(), |c| c as *const t0_gemm_config);
    // SAFETY: `rt` comes from t0_runtime_create; the device addresses in `d`
    // are the caller's live allocations of the sizes `d` describes.
    check(unsafe { t0_gemm(rt, cfg_ptr, d) }).map(|_| ())
}

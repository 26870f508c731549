/*
 * t0_gemm.h -- C ABI of the MI355X (gfx950) GEMM hot path.
 *
 * Drop-in boundary for the reference crate t0-gpu ("T0-GPU"): every entry
 * point below replaces one Rust item on the reference's GEMM path, cited as
 * file:line into the reference tree.  Rust callers bind these through an
 * extern "C" block with the same signatures.
 *
 * Conventions
 *  - Every function returns T0_OK (0) or a negative t0_status; the message of
 *    the last failure on the calling thread is t0_last_error().  Nothing
 *    aborts the process (the reference panics on infeasible configs,
 *    src/t0/gemm_gen.rs:271-281; here that is T0_ERR_INFEASIBLE).
 *  - bf16 data is raw little-endian uint16; device pointers are uint64_t
 *    addresses as in the reference's kernarg builders.
 *  - Grids are in work-items (HSA convention), as compute_grid returns them.
 *  - Kernarg byte layouts are exactly the reference's (40 / 44 / 48 bytes).
 */
#ifndef T0_GEMM_H
#define T0_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ status */
typedef enum t0_status {
    T0_OK = 0,
    T0_ERR_INVALID = -1,      /* bad argument / layout / size */
    T0_ERR_INFEASIBLE = -2,   /* config has no gfx950 kernel */
    T0_ERR_HIP = -3,          /* HIP runtime error */
    T0_ERR_POISONED = -4,     /* runtime refused: earlier GPU failure */
    T0_ERR_KERNARG = -5,      /* kernarg length != kernel's declared size */
    T0_ERR_NOT_FOUND = -6,    /* kernel symbol not in code object */
    T0_ERR_NO_DEVICE = -7,
} t0_status;

/* Message of the last error on this thread ("" if none). */
const char* t0_last_error(void);
/* Library version string. */
const char* t0_version(void);

/* ------------------------------------------------------------- GemmConfig */
/* Replaces gemm_gen::GemmTranspose (src/t0/gemm_gen.rs:22-29). */
enum { T0_NT = 0, T0_NN = 1 };
/* Replaces gemm_gen::EpilogueOp (src/t0/gemm_gen.rs:39-49). */
enum { T0_EPI_STORE_F32 = 0, T0_EPI_BIAS_ADD = 1, T0_EPI_BIAS_ADD_RELU = 2 };
/* New: output element type (the reference always stores f32). */
enum { T0_OUT_F32 = 0, T0_OUT_BF16 = 1 };

/* Replaces gemm_gen::GemmConfig (src/t0/gemm_gen.rs:55-84).  split_k 0 or 1
 * means no split (Option<u32> None / Some(1)).  On gfx950 wg_size counts
 * 64-lane waves (n_waves = wg_size / 64); lds_pad, use_lds, double_buffer
 * and wgp_mode are accepted for layout compatibility and do not change the
 * kernel (LDS is always used, swizzled, with >= 2 stages; CDNA has no WGP). */
typedef struct t0_gemm_config {
    uint32_t tile_m, tile_n, tile_k, wg_size;
    uint32_t split_k;
    uint32_t lds_pad;
    uint32_t n_col_passes;
    uint8_t use_lds, double_buffer, swap_grid, wgp_mode;
    uint8_t transpose;   /* T0_NT / T0_NN */
    uint8_t epilogue;    /* T0_EPI_* */
    uint8_t out_dtype;   /* T0_OUT_F32 / T0_OUT_BF16 (new) */
    uint8_t reserved;
} t0_gemm_config;

/* Presets: replaces GemmConfig::tile_* (src/t0/gemm_gen.rs:86-145) plus the
 * gfx950-native tiles used by auto-selection. */
typedef enum t0_preset {
    T0_PRESET_16x64_K16 = 0, T0_PRESET_32x64_DIRECT, T0_PRESET_32x64_K16, T0_PRESET_32x64_K32,
    T0_PRESET_32x128_K16, T0_PRESET_64x64_K16, T0_PRESET_64x64_K32, T0_PRESET_128x64_K16,
    T0_PRESET_64x128_K16, T0_PRESET_128x64_K32, T0_PRESET_128x128_K16, T0_PRESET_64x64_K64,
    T0_PRESET_128x128_2PASS, T0_PRESET_64x128_2PASS,
    /* gfx950-native */
    T0_PRESET_256x256_K64, T0_PRESET_256x128_K64, T0_PRESET_128x256_K64, T0_PRESET_128x128_K64,
    T0_PRESET_128x128_K32, T0_PRESET_128x64_K64, T0_PRESET_64x128_K64, T0_PRESET_32x64_K64,
    T0_PRESET_32x128_K64, T0_PRESET_256x256_K32,
    T0_PRESET_COUNT
} t0_preset;

int t0_config_preset(int preset, t0_gemm_config* out);

/* Derived geometry: replaces GemmConfig::{n_col_tiles, n_row_blocks, n_waves,
 * rows_per_wave, k_sub_steps, lds_per_buffer, lds_total, x/wt_bytes_per_thread,
 * wmma_per_k_tile, estimated_vgprs} (src/t0/gemm_gen.rs:147-213), restated
 * for wave64 and 32x32x16 MFMA blocks. */
typedef struct t0_gemm_geometry {
    uint32_t n_waves, waves_m, waves_n;
    uint32_t rows_per_wave, cols_per_wave;
    uint32_t n_row_blocks, n_col_tiles;     /* 32x32 MFMA blocks per wave */
    uint32_t k_sub_steps;                   /* tile_k / 16 */
    uint32_t stages;
    uint32_t lds_per_buffer, lds_total;
    uint32_t x_bytes_per_thread, wt_bytes_per_thread;
    uint32_t mfma_per_k_tile;
    uint32_t estimated_vgprs;               /* accumulators + operands + addresses, of 512 */
} t0_gemm_geometry;

int t0_config_geometry(const t0_gemm_config* cfg, t0_gemm_geometry* out);
/* Replaces GemmConfig::is_feasible (src/t0/gemm_gen.rs:193-213): 1 if a
 * gfx950 kernel exists for this config, else 0. */
int t0_config_is_feasible(const t0_gemm_config* cfg);
/* Replaces GemmConfig::name (src/t0/gemm_gen.rs:215-235); "_bf16" is appended
 * for out_dtype = T0_OUT_BF16.  Returns the full length (snprintf style). */
int t0_config_name(const t0_gemm_config* cfg, char* buf, size_t len);
/* Inverse of t0_config_name. */
int t0_config_from_name(const char* name, t0_gemm_config* out);
/* Replaces sweep_configs / standard_configs (src/t0/gemm_gen.rs:239-250, :407-427).
 * Writes up to cap configs, returns the total count. */
int t0_sweep_configs(t0_gemm_config* out, size_t cap);
int t0_standard_configs(t0_gemm_config* out, size_t cap);

/* ----------------------------------------------------------- grid / args */
/* Replaces compute_grid / compute_grid_split_k / compute_grid_auto
 * (src/t0/gemm_gen.rs:308-329, :430-437).  Work-items. */
int t0_compute_grid(const t0_gemm_config* cfg, uint32_t m, uint32_t n, uint32_t* gx, uint32_t* gy);
int t0_compute_grid_split_k(const t0_gemm_config* cfg, uint32_t m, uint32_t n, uint32_t split_k,
                            uint32_t* gx, uint32_t* gy);
int t0_compute_grid_auto(const t0_gemm_config* cfg, uint32_t m, uint32_t n, uint32_t* gx, uint32_t* gy);

/* Replaces build_kernargs (src/t0/gemm_gen.rs:442-458): 40 bytes
 * [X u64 | WT u64 | Y u64 | K u32 | N u32 | split_k_shift u32 (=0) | y_split_stride u32]. */
int t0_build_kernargs(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                      const t0_gemm_config* cfg, uint8_t out[40]);
/* Replaces build_kernargs_with_bias (src/t0/gemm_gen.rs:466-484): 48 bytes, bias u64 @40. */
int t0_build_kernargs_with_bias(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                                const t0_gemm_config* cfg, uint64_t bias, uint8_t out[48]);

/* Backward helpers: replace auto_select_backward_data/_weight,
 * build_kernargs_backward_*, compute_grid_backward_* (src/t0/gemm_gen.rs:510-570). */
int t0_auto_select_backward_data(uint32_t m, uint32_t n_orig, uint32_t k_orig, t0_gemm_config* out);
int t0_auto_select_backward_weight(uint32_t m, uint32_t n_orig, uint32_t k_orig, t0_gemm_config* out);
int t0_build_kernargs_backward_data(uint64_t dy, uint64_t w, uint64_t dx, uint32_t m, uint32_t n_orig,
                                    uint32_t k_orig, const t0_gemm_config* cfg, uint8_t out[40]);
int t0_build_kernargs_backward_weight(uint64_t dy_t, uint64_t x_t, uint64_t dw, uint32_t m, uint32_t n_orig,
                                      uint32_t k_orig, const t0_gemm_config* cfg, uint8_t out[40]);

/* --------------------------------------------------------- auto-selection */
/* Replaces auto_select (src/t0/gemm_gen.rs:340-342 -> cost_model::predict_best,
 * src/t0/cost_model.rs:660-668) with a per-tile cost table measured on MI355X
 * (tile x split-K ranked by predicted time).  Note argument order (m, k, n). */
int t0_auto_select(uint32_t m, uint32_t k, uint32_t n, t0_gemm_config* out);
/* Replaces auto_select_legacy (src/t0/gemm_gen.rs:351-404): the reference's
 * decision tree over the shapes, mapped onto gfx950 tiles. */
int t0_auto_select_legacy(uint32_t m, uint32_t k, uint32_t n, t0_gemm_config* out);
/* Replaces auto_schedule_gemm (src/t0/cost_model.rs:464-535): every
 * feasible candidate for an m x n x k GEMM of this layout and output type,
 * best first, with its predicted time in microseconds (the score).  Writes
 * at most `cap` configs to out (and times to est_us, if not NULL); returns
 * the number of candidates, or a negative status.  Its first entry is what
 * t0_gemm selects when no tuning cache entry exists. */
int t0_auto_schedule_gemm(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype,
                          t0_gemm_config* out, double* est_us, uint32_t cap);
/* Replaces prefill_spec_cache::cached_auto_select (src/t0/prefill_spec_cache.rs:55-76). */
int t0_cached_auto_select(uint32_t m, uint32_t k, uint32_t n, t0_gemm_config* out);
/* Replaces prefill_spec_cache::prewarm_cache (src/t0/prefill_spec_cache.rs:125-129). */
int t0_prewarm_cache(const uint32_t* mkn_triples, size_t count);

/* ------------------------------------------------------- TileGemm (tile_ir) */
/* Replaces tile_ir::EpilogueOp (src/t0/tile_ir.rs:41-62). */
enum { T0_TEPI_BIAS = 1, T0_TEPI_SCALE = 2, T0_TEPI_RELU = 3, T0_TEPI_SILU = 4, T0_TEPI_GELU = 5,
       T0_TEPI_ABS = 6, T0_TEPI_NEG = 7, T0_TEPI_CLAMP = 8 };
/* Replaces tile_ir::TileGemm (src/t0/tile_ir.rs:109-152); waves_per_wg 0 = default. */
typedef struct t0_tile_gemm {
    uint32_t tile_m, tile_n, tile_k;
    uint32_t split_k;
    uint32_t waves_per_wg;
    uint8_t wgp_mode, double_buffer, triple_buffer, swap_grid;
    uint8_t transpose, acc_swap, persistent, out_dtype;
    uint8_t n_epilogue;
    uint8_t epilogue[8];
    uint8_t reserved[3];
} t0_tile_gemm;

/* tile_ir::TileGemm::name (src/t0/tile_ir.rs:697-728). */
int t0_tile_name(const t0_tile_gemm* spec, char* buf, size_t len);
/* tile_ir::tile_auto_select (src/t0/tile_ir.rs:740-870), gfx950 tiles. */
int t0_tile_auto_select(uint32_t m, uint32_t k, uint32_t n, int transpose, t0_tile_gemm* out);
/* Replaces tile_ir::build_kernargs_m (src/t0/tile_ir.rs:4595-4602): 44 bytes,
 * M @40; split_k_shift = log2(split_k); y_split_stride written as given.
 * Epilogue arguments follow at 8-byte-aligned offsets: bias u64, scale f32,
 * clamp_min f32, clamp_max f32 (src/t0/tile_ir.rs:1014-1026).  *len receives
 * the byte count (at most 84); out must hold 96 bytes. */
int t0_tile_build_kernargs_m(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                             const t0_tile_gemm* spec, uint32_t y_split_stride, uint64_t bias,
                             float scale, float clamp_min, float clamp_max, uint8_t* out, size_t* len);
/* tile_ir::compute_grid (src/t0/tile_ir.rs:4645-4667); persistent kernels get
 * the full tile grid (the gfx950 kernels do not loop over tiles). */
int t0_tile_compute_grid(const t0_tile_gemm* spec, uint32_t m, uint32_t n, uint32_t grid[3]);

/* --------------------------------------------------------------- runtime */
typedef struct t0_runtime t0_runtime;   /* GpuRuntime (src/ignis/gpu_context.rs:99-119) */
typedef struct t0_kernel t0_kernel;     /* GpuKernel  (src/kfd/kernel.rs:8-19) */
typedef struct t0_buffer t0_buffer;     /* GpuBuffer  */

/* GpuRuntime::new / with_device (src/ignis/gpu_context.rs:151-189). */
int t0_runtime_create(int device_ordinal, t0_runtime** out);
int t0_runtime_destroy(t0_runtime* rt);
/* Use the caller's HIP stream (hipStream_t) for every launch; NULL = runtime's own. */
int t0_runtime_set_stream(t0_runtime* rt, void* hip_stream);
void* t0_runtime_stream(t0_runtime* rt);
/* is_poisoned / mark_poisoned (src/ignis/gpu_context.rs:191-198). */
int t0_runtime_is_poisoned(const t0_runtime* rt);
int t0_runtime_mark_poisoned(t0_runtime* rt);
/* Device facts: gfx name, CU count, clock (kHz). */
int t0_runtime_device_info(const t0_runtime* rt, char* arch, size_t arch_len, int* cu_count, int* clock_khz);

/* The gfx950 code object holding every kernel of this library: replaces
 * gemm_gen::generate + T0Kernel::compile (src/t0/gemm_gen.rs:261-297,
 * src/t0/compile.rs:1398-1455): "generate" selects a precompiled kernel by
 * name.  Writes the code object span and the kernel's symbol name. */
int t0_code_object(const void** data, size_t* size);
int t0_generate(const t0_gemm_config* cfg, char* symbol, size_t symbol_len);

/* Replaces KernelLoadConfig + GpuKernel::load (src/kfd/kernel.rs:26-141):
 * load a code object (hipModuleLoadData) and resolve `symbol`.  A kernel
 * loaded this way is dispatched with its raw kernarg bytes. */
typedef struct t0_kernel_load_config {
    uint32_t workgroup_size[3];
    uint32_t lds_size;
    uint32_t kernarg_size;   /* declared kernarg bytes (dispatch checks it) */
} t0_kernel_load_config;
int t0_kernel_load(t0_runtime* rt, const void* code_object, size_t size, const char* symbol,
                   const t0_kernel_load_config* cfg, t0_kernel** out);
/* Replaces GpuRuntime::ensure_kernel_t0 (src/ignis/gpu_context.rs:212-259):
 * name-keyed cache of GEMM kernels; dispatch takes the reference's 40-byte
 * (or 48-byte, bias epilogues) gemm_gen kernargs. */
int t0_ensure_kernel(t0_runtime* rt, const t0_gemm_config* cfg, t0_kernel** out);
/* Same for tile_ir kernels (44-byte kernargs + epilogue arguments). */
int t0_ensure_tile_kernel(t0_runtime* rt, const t0_tile_gemm* spec, t0_kernel** out);
/* Replaces GpuRuntime::get_kernel (src/ignis/gpu_context.rs:200-204). */
int t0_get_kernel(t0_runtime* rt, const char* name, t0_kernel** out);
int t0_kernel_info(const t0_kernel* k, uint32_t wg[3], uint32_t* lds, uint32_t* kernarg_size,
                   char* name, size_t name_len);

/* Replaces GpuRuntime::dispatch (src/ignis/gpu_context.rs:305-356): checks
 * poison and kernarg length, launches, waits.  Returns T0_ERR_HIP and poisons
 * the runtime if the wait fails. */
int t0_dispatch(t0_runtime* rt, const t0_kernel* k, const uint32_t grid[3], const void* kernargs, size_t len);
/* Replaces GpuRuntime::dispatch_async (src/ignis/gpu_context.rs:400-410):
 * returns the slot index (>= 0) or a negative status. */
int t0_dispatch_async(t0_runtime* rt, const t0_kernel* k, const uint32_t grid[3], const void* kernargs, size_t len);
/* GpuRuntime::wait_idle / synchronize (src/ignis/gpu_context.rs:445-452). */
int t0_wait_idle(t0_runtime* rt);
int t0_synchronize(t0_runtime* rt);

/* Memory: GpuRuntime::alloc / recycle / read_f32 (src/ignis/gpu_context.rs:508-542),
 * BufferPool (src/ignis/gpu_context.rs:31-92): recycled buffers are keyed by
 * 4 KiB-rounded size and zeroed on reuse. */
int t0_alloc(t0_runtime* rt, size_t bytes, t0_buffer** out);
int t0_recycle(t0_runtime* rt, t0_buffer* buf);
int t0_buffer_free(t0_buffer* buf);
uint64_t t0_buffer_addr(const t0_buffer* buf);
size_t t0_buffer_size(const t0_buffer* buf);
int t0_buffer_write(t0_buffer* buf, size_t offset, const void* src, size_t len);
int t0_buffer_read(const t0_buffer* buf, size_t offset, void* dst, size_t len);
int t0_buffer_zero(t0_buffer* buf);
int t0_read_f32(const t0_buffer* buf, float* dst, size_t count);
/* Raw copies between host memory and device addresses. */
int t0_memcpy_h2d(t0_runtime* rt, uint64_t dst, const void* src, size_t len);
int t0_memcpy_d2h(t0_runtime* rt, void* dst, uint64_t src, size_t len);
int t0_memset_d(t0_runtime* rt, uint64_t dst, int value, size_t len);

/* Events on the runtime's stream (timing). */
typedef struct t0_event t0_event;
int t0_event_create(t0_event** out);
int t0_event_destroy(t0_event* ev);
int t0_event_record(t0_runtime* rt, t0_event* ev);
int t0_event_synchronize(t0_event* ev);
int t0_event_elapsed_ms(const t0_event* start, const t0_event* stop, float* ms);

/* Stream capture into a HIP graph (no counterpart in the reference, whose
 * DispatchQueue batches AQL packets, src/t0/prefill_dispatch.rs:61-130):
 * everything launched on the runtime's stream between begin and end is
 * recorded, then replayed with one launch.  Workspaces must already exist
 * (run the same calls once before capturing): a call that would grow the
 * runtime's split-K workspace, semaphore array or operand staging buffer
 * fails with T0_ERR_INVALID during capture, and also while any graph made
 * from this runtime exists, since the graph's kernels hold those addresses
 * (a graph pins the workspace size until t0_graph_destroy).  Destroy graphs
 * before their runtime; one that outlives it can still be destroyed. */
typedef struct t0_graph t0_graph;
int t0_graph_begin(t0_runtime* rt);
int t0_graph_end(t0_runtime* rt, t0_graph** out);
int t0_graph_launch(t0_runtime* rt, const t0_graph* g);
int t0_graph_destroy(t0_graph* g);

/* ------------------------------------------------------ high-level GEMM */
/* One GEMM through the tuned kernel family, the way auto_gemm
 * (src/t0/auto_gemm.rs:555-590) runs one: C = epilogue(A . B).
 *   A bf16 [M, lda]; B: NT -> WT [N, ldb], NN -> B [K, ldb]; C [M, ldc].
 *   cfg NULL selects (tuning cache, then t0_auto_select).
 *   split_k > 1 with out_dtype bf16 or an epilogue is reduced in-kernel. */
typedef struct t0_gemm_desc {
    uint64_t a, b, c, bias;
    uint32_t m, n, k;
    uint32_t lda, ldb, ldc;     /* 0 = dense */
    uint32_t transpose;         /* T0_NT / T0_NN */
    uint32_t out_dtype;         /* T0_OUT_F32 / T0_OUT_BF16 */
    uint32_t n_epilogue;
    uint8_t epilogue[8];        /* T0_TEPI_* chain */
    float scale, clamp_min, clamp_max;
} t0_gemm_desc;
int t0_gemm(t0_runtime* rt, const t0_gemm_config* cfg, const t0_gemm_desc* d);
/* The config t0_gemm would use for d (NULL cfg). */
int t0_gemm_select(t0_runtime* rt, const t0_gemm_desc* d, t0_gemm_config* out);
/* Measurement aid with no counterpart in the reference (its README quotes
 * the nominal clock only): runs t0_gemm once with per-workgroup timestamps
 * (shader clock and the 100 MHz real-time clock at each workgroup's start and
 * end), waits, and returns the median shader clock over workgroups in MHz,
 * the span from the first start to the last end in microseconds and (when
 * wg_cycles is not NULL) the median shader cycles per workgroup.  Tiled
 * kernels without split-K only (else T0_ERR_INVALID); at most 65536
 * workgroups.  Synchronous. */
int t0_gemm_clock_probe(t0_runtime* rt, const t0_gemm_config* cfg, const t0_gemm_desc* d, double* sclk_mhz,
                        double* span_us, double* wg_cycles);
/* No counterpart in the reference: t0_gemm for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments and results as t0_gemm; the
 * in-kernel split-K keeps its counters and partial tiles in a fixed
 * per-device scratch array of T0_NOALLOC_SCRATCH_BYTES that the library holds
 * until the process ends, instead of the runtime's growable workspace, and
 * the call allocates and frees nothing.  Limits: at most
 * T0_NOALLOC_MAX_TILES output tiles and split_k * tiles * tile_m * tile_n * 4
 * <= T0_NOALLOC_SCRATCH_BYTES - 4 * T0_NOALLOC_MAX_TILES bytes of partials,
 * else T0_ERR_INVALID (nothing launched).  With cfg NULL the call takes
 * t0_gemm's selection if its split-K fits those limits, else the best-ranked
 * candidate of t0_auto_schedule_gemm that fits (one without split-K always
 * does), so its output can then differ from t0_gemm's in rounding (the same
 * bound).  The counters used are cleared at each call.  Every call on one GPU shares that GPU's array, so calls that
 * overlap on one GPU (other streams, other threads) race. */
#define T0_NOALLOC_SCRATCH_BYTES (32u << 20)
#define T0_NOALLOC_MAX_TILES 16384u
int t0_gemm_noalloc(t0_runtime* rt, const t0_gemm_config* cfg, const t0_gemm_desc* d);

/* Replaces auto_gemm::GemmTuner::tune (src/t0/auto_gemm.rs:82-216) and the
 * JSON cache (src/t0/auto_gemm.rs:435-501): after a 256^3 correctness smoke
 * test, each of the best-ranked candidate configs is timed on seeded N(0,1)
 * bf16 operands with the weight operand B rotated through copies that
 * together exceed the 256 MB Infinity Cache (read from HBM, as in
 * inference), the launches over all copies captured as one HIP graph and
 * replayed (hipEvent timing, median of n_iters replays).  The fastest is
 * cached in memory and on disk in the reference's JSON layout (tile_m,
 * tile_n, tile_k, wg_size, split_k, lds_pad, n_col_passes, wgp, swap,
 * tflops, all; plus arch, transpose, out_dtype, name), "all" holding every
 * timed candidate fastest first as ["name", tflops, wg_size].  NT with f32
 * output keeps the reference's file name <cache_dir>/gemm_<M>x<N>x<K>.json;
 * other layouts add _<nn|nt>_<bf16|f32>.  The cache directory is the one
 * set by t0_tuner_set_cache_dir, else $T0_AUTOTUNE_DIR, else
 * ~/.t0_autotune_gfx950 (not the reference's ~/.t0_autotune, whose loader
 * would take gfx950-only configs; set it there to read the reference's
 * files).  A file is used only if a gfx950 kernel runs its config (tile and
 * wave count, split_k a power of two <= 16) and it names no other
 * architecture; otherwise the candidates are ranked afresh.  cfg_out and
 * tflops_out may be NULL. */
int t0_tune(t0_runtime* rt, uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype,
            t0_gemm_config* cfg_out, double* tflops_out);
int t0_tuner_set_cache_dir(const char* dir);
int t0_tuner_set_params(uint32_t max_candidates, uint32_t n_iters);
/* The on-disk cache without a runtime (gfx950 entries), after
 * GemmTuner::save_cache / load_cache / invalidate (src/t0/auto_gemm.rs:439-507):
 * store writes cfg (T0_ERR_INFEASIBLE if no gfx950 kernel runs it); load
 * returns T0_ERR_NOT_FOUND for a missing or unusable file; invalidate drops
 * the file and the in-memory entry. */
int t0_tuner_cache_store(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype,
                         const t0_gemm_config* cfg, double tflops);
int t0_tuner_cache_load(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype,
                        t0_gemm_config* cfg, double* tflops);
int t0_tuner_invalidate(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype);
/* One timed candidate of t0_tune. */
typedef struct t0_tune_entry {
    t0_gemm_config cfg;
    double tflops;
} t0_tune_entry;
/* GemmTuneResult.all (src/t0/auto_gemm.rs:30-42): every candidate the last
 * t0_tune of this problem timed, fastest first -- from this process's tune
 * (*from_cache = 0) or else from the cache file's "all" list (*from_cache =
 * 1; the reference's own loader leaves it empty).  Up to cap entries into
 * all (may be NULL with cap 0), the count to *n_all; T0_ERR_NOT_FOUND if
 * neither holds the problem. */
int t0_tune_results(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype, t0_tune_entry* all,
                    uint32_t cap, uint32_t* n_all, int* from_cache);
/* Replaces auto_gemm::auto_gemm (src/t0/auto_gemm.rs:555-590): tune then run
 * (NT, f32 out, like the reference). */
int t0_auto_gemm(t0_runtime* rt, uint64_t a, uint64_t b, uint64_t c, uint32_t m, uint32_t n, uint32_t k,
                 double* tflops_out);
/* One timed candidate of t0_tile_tune. */
typedef struct t0_tile_tune_entry {
    t0_tile_gemm spec;
    double tflops;
} t0_tile_tune_entry;
/* Replaces cost_model::tune_tile_ir and TileIrTuneResult
 * (src/t0/cost_model.rs:824-1080): for an NT tile_ir GEMM (bf16 in, f32
 * out), the tile_ir_MxNxK.json cache in the tuner's directory if it holds a
 * usable gfx950 tile; otherwise the reference's presets, then the cost
 * model's tiles, each timed through the tile_ir dispatch path on seeded
 * N(0,1) operands (median of the tuner's n_iters launches), the fastest
 * cached.  Writes the best spec and its TFLOP/s, up to `cap` timed
 * candidates fastest first to all (may be NULL), their count to *n_all
 * (0 from the cache, whose file keeps only names) and whether the result
 * came from the cache to *from_cache. */
int t0_tile_tune(t0_runtime* rt, uint32_t m, uint32_t n, uint32_t k, t0_tile_gemm* best, double* best_tflops,
                 t0_tile_tune_entry* all, uint32_t cap, uint32_t* n_all, int* from_cache);

/* ------------------------------------------------------------------ INT4 */
/* Replaces GptqWeight (src/t0/quant_kernels.rs:188-296): parse / measure the
 * reference byte format [rows u32][cols u32][group_size u32][packed]
 * [scales f32 x rows*n_groups][zero_points i32 x rows*n_groups]. */
typedef struct t0_gptq_view {
    uint32_t rows, cols, group_size, n_groups;
    const uint8_t* packed;        /* rows*cols/2 bytes */
    const float* scales;          /* [row][group] */
    const int32_t* zero_points;   /* [row][group] */
} t0_gptq_view;
int t0_gptq_from_bytes(const void* raw, size_t len, t0_gptq_view* out);
size_t t0_gptq_gpu_buffer_size(const t0_gptq_view* w);
/* Convert a GptqWeight to the W4A16 operand layout (host memory):
 * qweight [rows][cols/8] u32 (same bytes), scales [G][rows] bf16 (RNE of the
 * f32 scale, or f32 copy if scales_f32 != 0), zeros [G][rows/8] u32 packed
 * nibbles (zero points must be 0..15). */
int t0_gptq_to_w4a16(const t0_gptq_view* w, uint32_t* qweight, void* scales, int scales_f32, uint32_t* zeros);

/* Replaces build_dequant_int4_f32 / _bf16 (src/t0/quant_kernels.rs:53-167)
 * with the documented semantics: out[e] = (q(e) - zp[g]) * scale[g], g over
 * [row][cols >> gs_log2]; bf16 output truncates (store_bf16).  Kernarg order
 * as the reference: packed, scales, zero_points, output, rows, cols. */
int t0_dequant_int4(t0_runtime* rt, uint64_t packed, uint64_t scales, uint64_t zero_points, uint64_t output,
                    uint32_t rows, uint32_t cols, uint32_t group_size_log2, int bf16_out);

/* W4A16 GEMM (new; the reference has no fused INT4 GEMM):
 * C[M,N] = A[M,K] (bf16) . W^T with W = (q - z) * s, dequantized exactly
 * inside the K loop.  qweight [N][K/8] u32; scales [G][N] bf16 (or f32);
 * zeros [G][N/8] u32 packed or 0 with zero_const.  split_k 0 = auto. */
typedef struct t0_w4a16_desc {
    uint64_t a, qweight, scales, zeros, c;
    uint32_t m, n, k;
    uint32_t lda, ldc;          /* 0 = dense */
    uint32_t group_size;
    uint32_t zero_const;
    uint32_t scales_f32;        /* 1: f32 scales */
    uint32_t out_f32;           /* 1: f32 output, else bf16 (RNE) */
    uint32_t split_k;           /* decode path K partitions, 0 = auto */
} t0_w4a16_desc;
int t0_w4a16_gemm(t0_runtime* rt, const t0_w4a16_desc* d);
/* Name of the kernel t0_w4a16_gemm would launch for d, and its split_k. */
int t0_w4a16_plan(t0_runtime* rt, const t0_w4a16_desc* d, char* kernel, size_t len, uint32_t* split_k);

/* --------------------------------------------------------- small kernels */
/* Sum split-K planes (plane p at src + p*plane_stride bytes, f32 [m][n])
 * into dst f32 or bf16 (RNE), in plane order: the host reduction of
 * examples/hello_gemm_gen.rs:125-136 on the GPU. */
int t0_splitk_reduce(t0_runtime* rt, uint64_t src, uint64_t plane_stride, uint32_t planes, uint64_t dst,
                     uint32_t m, uint32_t n, int out_bf16);
/* f32 -> bf16 RNE (src/ignis/ops/bf16_matmul.rs:356-383 does this on the CPU). */
int t0_f32_to_bf16(t0_runtime* rt, uint64_t src, uint64_t dst, uint64_t count);
/* Device-to-device copy through a plain 16-byte-per-lane kernel (no
 * counterpart in the reference): the calibration kernel for HBM byte counters. */
int t0_copy_device(t0_runtime* rt, uint64_t src, uint64_t dst, uint64_t bytes);
/* Floors of the HBM-bound shapes (measurement aids, no reference
 * counterpart): t0_floor_stream_read only reads `bytes` (16-byte aligned,
 * < 4 GiB) with 16-byte loads on a grid of `workgroups` x `threads` (a
 * multiple of 64, <= 1024) -- the time to stream a weight array once; sink
 * takes at most workgroups * 4 bytes.  t0_floor_empty launches an empty
 * kernel of that shape: the per-launch cost alone.  Asynchronous. */
int t0_floor_stream_read(t0_runtime* rt, uint64_t src, uint64_t bytes, uint64_t sink, uint32_t workgroups,
                         uint32_t threads);
int t0_floor_empty(t0_runtime* rt, uint32_t workgroups, uint32_t threads);
/* Operand read floor of a GEMM tiling (measurement aid, no reference
 * counterpart): one launch with the grid t0_gemm would use for cfg (NULL:
 * t0_gemm_select's pick) on d's shape, in which every workgroup only moves
 * its operand slices -- the A rows of its tile (mode 1), the B columns
 * (mode 2) or both (mode 3) over its split-K partition -- from d->a / d->b to
 * LDS, 64 k per step, as the GEMM stages them: no MFMAs, no partial sums, no
 * stores.  The time the tiling's operand traffic takes on its own.  Tiled
 * configs with tile_m, tile_n multiples of 8, tile_m + tile_n <= 512, K a
 * multiple of 64 * split_k, 16-byte aligned operands under 4 GiB with lda
 * and ldb multiples of 8.  Asynchronous. */
int t0_floor_tile_read(t0_runtime* rt, const t0_gemm_config* cfg, const t0_gemm_desc* d, int mode);
/* Ceilings of the compute-bound GEMM (measurement aids, no reference
 * counterpart).  t0_floor_mfma issues mfma_per_wave (a multiple of 16)
 * v_mfma_f32_32x32x16_bf16 per wave from registers on `workgroups` 512-thread
 * workgroups, the 8-wave 256x256 tile's accumulators and operand
 * fragments, nothing else in the loop; the fragments come from `operands`
 * (workgroups * 512 * 192 bytes, 16-byte aligned), whose values set the
 * power the MFMAs draw.  t0_floor_lds has every wave read its LDS window in
 * rounds of 8 ds_read_b128 (mode 0) or ds_read_b64_tr_b16 (mode 1), or issue
 * 8 one-KiB global->LDS DMAs from the 64 KiB `src` (mode 2), `rounds` times.
 * Both write 4 u64 per workgroup to `out` -- the 100 MHz clock and the
 * shader clock at start and end -- and need out to hold workgroups * 32
 * bytes, plus workgroups * 2048 (t0_floor_mfma) or 4096 (t0_floor_lds) bytes
 * that are written only on an impossible result.  Asynchronous. */
int t0_floor_mfma(t0_runtime* rt, uint64_t operands, uint64_t out, uint32_t workgroups, uint32_t mfma_per_wave);
int t0_floor_lds(t0_runtime* rt, int mode, uint64_t src, uint64_t out, uint32_t workgroups, uint32_t threads,
                 uint32_t rounds);
/* t0_unpad_2d (src/t0/math.rs): out[m][n] = padded[m][n_pad]. */
int t0_unpad_2d(t0_runtime* rt, uint64_t padded, uint64_t out, uint32_t m, uint32_t n, uint32_t n_pad);

/* ----------------------------------------------------- Ignis bf16 matmul */
/* The GEMM calls of src/ignis/ops/bf16_matmul.rs on dense row-major f32
 * device buffers, f32 output, operands rounded to bf16 (RNE) on the GPU.
 * Any m, k, n >= 1.  The bf16 operands are staged in a buffer the runtime
 * owns and grows on demand (hipMalloc on growth only); calls on one runtime
 * run in its stream order and share that buffer.
 *
 * Y[m,n] = X[m,k] . W[k,n]  -- matmul forward, bf16_matmul.rs:33-47 with
 * dispatch_gemm_forward :162-207 (W is read as the NN operand, not transposed). */
int t0_bf16_matmul(t0_runtime* rt, uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t k, uint32_t n);
/* dX[m,k] = dY[m,n] . W[k,n]^T  -- gemm_backward_data, bf16_matmul.rs:215-258. */
int t0_bf16_matmul_backward_data(t0_runtime* rt, uint64_t dy, uint64_t w, uint64_t dx, uint32_t m, uint32_t k,
                                 uint32_t n);
/* dW[k,n] = X[m,k]^T . dY[m,n]  -- gemm_backward_weight, bf16_matmul.rs:265-308
 * (X^T is produced by the converting kernel; dY is not transposed). */
int t0_bf16_matmul_backward_weight(t0_runtime* rt, uint64_t x, uint64_t dy, uint64_t dw, uint32_t m, uint32_t k,
                                   uint32_t n);
/* Y[m,n] = X[m,k] . WT[n,k]^T with WT dense bf16  -- matmul_with_wt_bf16,
 * bf16_matmul.rs:102-134. */
int t0_bf16_matmul_with_wt_bf16(t0_runtime* rt, uint64_t x, uint64_t wt, uint64_t y, uint32_t m, uint32_t k,
                                uint32_t n);

/* ------------------------------------------- residual add + RMSNorm ---- */
/* x2 = residual (+ hidden); inv_rms = 1 / sqrt(sum(x2^2)/d + eps);
 * normed = x2 * inv_rms * gamma.  f32 device buffers, dense rows.          */

/* Replaces the reference kernel build_ffn_fused_rmsnorm_gemm and its CPU form
 * (src/t0/ffn_fused_kernels.rs:54-237): output[r] = sum_i normed[r,i] *
 * weight[r*d + i] for rows r < m.  The code object also exports the kernel
 * itself as "ffn_fused_rmsnorm_gemm" (128-lane workgroups, one per row, the
 * reference's 48-byte kernargs) for raw t0_kernel_load + t0_dispatch. */
int t0_ffn_fused_rmsnorm_gemm(t0_runtime* rt, uint64_t residual, uint64_t hidden, uint64_t gamma, uint64_t weight,
                              uint64_t output, uint32_t m, uint32_t d, float eps);
/* Residual add + RMSNorm over rows (src/t0/rmsnorm_kernels.rs:140-153 on the
 * residual sum of ffn_fused_kernels.rs:215-224): out[r][0..d) = normed as
 * bf16 (RNE, out_bf16 != 0) or f32, zeros in [d, ld_out) (0 = d); x2_out
 * (may be 0) receives x2.  hidden may be 0. */
int t0_rmsnorm(t0_runtime* rt, uint64_t residual, uint64_t hidden, uint64_t gamma, uint64_t out, uint64_t x2_out,
               uint32_t rows, uint32_t d, uint32_t ld_out, float eps, int out_bf16);
typedef struct t0_rmsnorm_desc {
    uint64_t residual, hidden, gamma;  /* f32 [m][k], [m][k] or 0, [k] */
    uint64_t x2_out;                   /* f32 [m][k] or 0 */
    float eps;
    uint32_t pad_;
} t0_rmsnorm_desc;
/* fused_rmsnorm_gemm / fused_residual_rmsnorm_gemm
 * (src/ignis/ops/fused_rmsnorm_gemm.rs:33-154) on an INT4 weight:
 * C[m,n] = normed[m,:] . W^T with W as in t0_w4a16_desc (d->a and d->lda are
 * ignored).  m == 1: one decode kernel with the residual add and RMSNorm in
 * front (the per-row 1/rms is applied after the k sum); other m: t0_rmsnorm
 * to bf16 in the runtime's staging buffer, then t0_w4a16_gemm. */
int t0_rmsnorm_w4a16(t0_runtime* rt, const t0_w4a16_desc* d, const t0_rmsnorm_desc* nd);
/* The same with a dense f32 weight W[k,n] (the Ignis prefill path:
 * rmsnorm, then bf16_matmul): Y[m,n] = bf16(normed) . bf16(W), f32 out. */
int t0_rmsnorm_matmul(t0_runtime* rt, uint64_t residual, uint64_t hidden, uint64_t gamma, uint64_t w, uint64_t y,
                      uint64_t x2_out, uint32_t m, uint32_t k, uint32_t n, float eps);

#ifdef __cplusplus
}
#endif
#endif /* T0_GEMM_H */

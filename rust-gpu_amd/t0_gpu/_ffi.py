"""ctypes declarations for libt0gpu.so (include/t0_gemm.h)."""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libt0gpu.so")

u8, u32, u64, i32, f32, f64 = C.c_uint8, C.c_uint32, C.c_uint64, C.c_int32, C.c_float, C.c_double
sz, vp, cp = C.c_size_t, C.c_void_p, C.c_char_p

T0_OK = 0
STATUS = {0: "T0_OK", -1: "T0_ERR_INVALID", -2: "T0_ERR_INFEASIBLE", -3: "T0_ERR_HIP", -4: "T0_ERR_POISONED",
          -5: "T0_ERR_KERNARG", -6: "T0_ERR_NOT_FOUND", -7: "T0_ERR_NO_DEVICE"}


class GemmConfigC(C.Structure):
    _fields_ = [("tile_m", u32), ("tile_n", u32), ("tile_k", u32), ("wg_size", u32), ("split_k", u32),
                ("lds_pad", u32), ("n_col_passes", u32), ("use_lds", u8), ("double_buffer", u8),
                ("swap_grid", u8), ("wgp_mode", u8), ("transpose", u8), ("epilogue", u8), ("out_dtype", u8),
                ("reserved", u8)]


class GemmGeometryC(C.Structure):
    _fields_ = [(n, u32) for n in ("n_waves", "waves_m", "waves_n", "rows_per_wave", "cols_per_wave",
                                   "n_row_blocks", "n_col_tiles", "k_sub_steps", "stages", "lds_per_buffer",
                                   "lds_total", "x_bytes_per_thread", "wt_bytes_per_thread", "mfma_per_k_tile",
                                   "estimated_vgprs")]


class TileGemmC(C.Structure):
    _fields_ = [("tile_m", u32), ("tile_n", u32), ("tile_k", u32), ("split_k", u32), ("waves_per_wg", u32),
                ("wgp_mode", u8), ("double_buffer", u8), ("triple_buffer", u8), ("swap_grid", u8),
                ("transpose", u8), ("acc_swap", u8), ("persistent", u8), ("out_dtype", u8),
                ("n_epilogue", u8), ("epilogue", u8 * 8), ("reserved", u8 * 3)]


class TileTuneEntryC(C.Structure):
    _fields_ = [("spec", TileGemmC), ("tflops", C.c_double)]


class TuneEntryC(C.Structure):
    _fields_ = [("cfg", GemmConfigC), ("tflops", C.c_double)]


class KernelLoadConfigC(C.Structure):
    _fields_ = [("workgroup_size", u32 * 3), ("lds_size", u32), ("kernarg_size", u32)]


class GemmDescC(C.Structure):
    _fields_ = [("a", u64), ("b", u64), ("c", u64), ("bias", u64), ("m", u32), ("n", u32), ("k", u32),
                ("lda", u32), ("ldb", u32), ("ldc", u32), ("transpose", u32), ("out_dtype", u32),
                ("n_epilogue", u32), ("epilogue", u8 * 8), ("scale", f32), ("clamp_min", f32), ("clamp_max", f32)]


class GptqViewC(C.Structure):
    _fields_ = [("rows", u32), ("cols", u32), ("group_size", u32), ("n_groups", u32), ("packed", vp),
                ("scales", vp), ("zero_points", vp)]


class W4A16DescC(C.Structure):
    _fields_ = [("a", u64), ("qweight", u64), ("scales", u64), ("zeros", u64), ("c", u64), ("m", u32),
                ("n", u32), ("k", u32), ("lda", u32), ("ldc", u32), ("group_size", u32), ("zero_const", u32),
                ("scales_f32", u32), ("out_f32", u32), ("split_k", u32)]


class RmsNormDescC(C.Structure):
    _fields_ = [("residual", u64), ("hidden", u64), ("gamma", u64), ("x2_out", u64), ("eps", C.c_float),
                ("pad_", u32)]


P = C.POINTER
SIGNATURES = {
    "t0_last_error": ([], cp), "t0_version": ([], cp),
    "t0_config_preset": ([C.c_int, P(GemmConfigC)], C.c_int),
    "t0_config_geometry": ([P(GemmConfigC), P(GemmGeometryC)], C.c_int),
    "t0_config_is_feasible": ([P(GemmConfigC)], C.c_int),
    "t0_config_name": ([P(GemmConfigC), cp, sz], C.c_int),
    "t0_config_from_name": ([cp, P(GemmConfigC)], C.c_int),
    "t0_sweep_configs": ([P(GemmConfigC), sz], C.c_int),
    "t0_standard_configs": ([P(GemmConfigC), sz], C.c_int),
    "t0_compute_grid": ([P(GemmConfigC), u32, u32, P(u32), P(u32)], C.c_int),
    "t0_compute_grid_split_k": ([P(GemmConfigC), u32, u32, u32, P(u32), P(u32)], C.c_int),
    "t0_compute_grid_auto": ([P(GemmConfigC), u32, u32, P(u32), P(u32)], C.c_int),
    "t0_build_kernargs": ([u64, u64, u64, u32, u32, u32, P(GemmConfigC), vp], C.c_int),
    "t0_build_kernargs_with_bias": ([u64, u64, u64, u32, u32, u32, P(GemmConfigC), u64, vp], C.c_int),
    "t0_auto_select_backward_data": ([u32, u32, u32, P(GemmConfigC)], C.c_int),
    "t0_auto_select_backward_weight": ([u32, u32, u32, P(GemmConfigC)], C.c_int),
    "t0_build_kernargs_backward_data": ([u64, u64, u64, u32, u32, u32, P(GemmConfigC), vp], C.c_int),
    "t0_build_kernargs_backward_weight": ([u64, u64, u64, u32, u32, u32, P(GemmConfigC), vp], C.c_int),
    "t0_auto_select": ([u32, u32, u32, P(GemmConfigC)], C.c_int),
    "t0_auto_schedule_gemm": ([u32, u32, u32, u32, u32, P(GemmConfigC), P(C.c_double), u32], C.c_int),
    "t0_auto_select_legacy": ([u32, u32, u32, P(GemmConfigC)], C.c_int),
    "t0_cached_auto_select": ([u32, u32, u32, P(GemmConfigC)], C.c_int),
    "t0_prewarm_cache": ([P(u32), sz], C.c_int),
    "t0_tile_name": ([P(TileGemmC), cp, sz], C.c_int),
    "t0_tile_auto_select": ([u32, u32, u32, C.c_int, P(TileGemmC)], C.c_int),
    "t0_tile_build_kernargs_m": ([u64, u64, u64, u32, u32, u32, P(TileGemmC), u32, u64, f32, f32, f32, vp, P(sz)],
                                 C.c_int),
    "t0_tile_compute_grid": ([P(TileGemmC), u32, u32, P(u32)], C.c_int),
    "t0_runtime_create": ([C.c_int, P(vp)], C.c_int),
    "t0_runtime_destroy": ([vp], C.c_int),
    "t0_runtime_set_stream": ([vp, vp], C.c_int),
    "t0_runtime_stream": ([vp], vp),
    "t0_runtime_is_poisoned": ([vp], C.c_int),
    "t0_runtime_mark_poisoned": ([vp], C.c_int),
    "t0_runtime_device_info": ([vp, cp, sz, P(C.c_int), P(C.c_int)], C.c_int),
    "t0_code_object": ([P(vp), P(sz)], C.c_int),
    "t0_generate": ([P(GemmConfigC), cp, sz], C.c_int),
    "t0_kernel_load": ([vp, vp, sz, cp, P(KernelLoadConfigC), P(vp)], C.c_int),
    "t0_ensure_kernel": ([vp, P(GemmConfigC), P(vp)], C.c_int),
    "t0_ensure_tile_kernel": ([vp, P(TileGemmC), P(vp)], C.c_int),
    "t0_get_kernel": ([vp, cp, P(vp)], C.c_int),
    "t0_kernel_info": ([vp, P(u32), P(u32), P(u32), cp, sz], C.c_int),
    "t0_dispatch": ([vp, vp, P(u32), vp, sz], C.c_int),
    "t0_dispatch_async": ([vp, vp, P(u32), vp, sz], C.c_int),
    "t0_wait_idle": ([vp], C.c_int),
    "t0_synchronize": ([vp], C.c_int),
    "t0_alloc": ([vp, sz, P(vp)], C.c_int),
    "t0_recycle": ([vp, vp], C.c_int),
    "t0_buffer_free": ([vp], C.c_int),
    "t0_buffer_addr": ([vp], u64),
    "t0_buffer_size": ([vp], sz),
    "t0_buffer_write": ([vp, sz, vp, sz], C.c_int),
    "t0_buffer_read": ([vp, sz, vp, sz], C.c_int),
    "t0_buffer_zero": ([vp], C.c_int),
    "t0_read_f32": ([vp, vp, sz], C.c_int),
    "t0_memcpy_h2d": ([vp, u64, vp, sz], C.c_int),
    "t0_memcpy_d2h": ([vp, vp, u64, sz], C.c_int),
    "t0_memset_d": ([vp, u64, C.c_int, sz], C.c_int),
    "t0_event_create": ([P(vp)], C.c_int),
    "t0_event_destroy": ([vp], C.c_int),
    "t0_event_record": ([vp, vp], C.c_int),
    "t0_event_synchronize": ([vp], C.c_int),
    "t0_event_elapsed_ms": ([vp, vp, P(f32)], C.c_int),
    "t0_gemm": ([vp, P(GemmConfigC), P(GemmDescC)], C.c_int),
    "t0_tuner_cache_store": ([u32, u32, u32, u32, u32, P(GemmConfigC), f64], C.c_int),
    "t0_tuner_cache_load": ([u32, u32, u32, u32, u32, P(GemmConfigC), P(f64)], C.c_int),
    "t0_tuner_invalidate": ([u32, u32, u32, u32, u32], C.c_int),
    "t0_tune_results": ([u32, u32, u32, u32, u32, P(TuneEntryC), u32, P(u32), P(C.c_int)], C.c_int),
    "t0_gemm_noalloc": ([vp, P(GemmConfigC), P(GemmDescC)], C.c_int),
    "t0_gemm_clock_probe": ([vp, P(GemmConfigC), P(GemmDescC), P(f64), P(f64), P(f64)], C.c_int),
    "t0_gemm_select": ([vp, P(GemmDescC), P(GemmConfigC)], C.c_int),
    "t0_tune": ([vp, u32, u32, u32, u32, u32, P(GemmConfigC), P(f64)], C.c_int),
    "t0_tuner_set_cache_dir": ([cp], C.c_int),
    "t0_tuner_set_params": ([u32, u32], C.c_int),
    "t0_tile_tune": ([vp, u32, u32, u32, P(TileGemmC), P(f64), P(TileTuneEntryC), u32, P(u32), P(C.c_int)], C.c_int),
    "t0_auto_gemm": ([vp, u64, u64, u64, u32, u32, u32, P(f64)], C.c_int),
    "t0_gptq_from_bytes": ([vp, sz, P(GptqViewC)], C.c_int),
    "t0_gptq_gpu_buffer_size": ([P(GptqViewC)], sz),
    "t0_gptq_to_w4a16": ([P(GptqViewC), vp, vp, C.c_int, vp], C.c_int),
    "t0_dequant_int4": ([vp, u64, u64, u64, u64, u32, u32, u32, C.c_int], C.c_int),
    "t0_w4a16_gemm": ([vp, P(W4A16DescC)], C.c_int),
    "t0_w4a16_plan": ([vp, P(W4A16DescC), cp, sz, P(u32)], C.c_int),
    "t0_splitk_reduce": ([vp, u64, u64, u32, u64, u32, u32, C.c_int], C.c_int),
    "t0_f32_to_bf16": ([vp, u64, u64, u64], C.c_int),
    "t0_unpad_2d": ([vp, u64, u64, u32, u32, u32], C.c_int),
    "t0_copy_device": ([vp, u64, u64, u64], C.c_int),
    "t0_floor_stream_read": ([vp, u64, u64, u64, u32, u32], C.c_int),
    "t0_floor_tile_read": ([vp, P(GemmConfigC), P(GemmDescC), C.c_int], C.c_int),
    "t0_floor_empty": ([vp, u32, u32], C.c_int),
    "t0_floor_mfma": ([vp, u64, u64, u32, u32], C.c_int),
    "t0_floor_lds": ([vp, C.c_int, u64, u64, u32, u32, u32], C.c_int),
    "t0_bf16_matmul": ([vp, u64, u64, u64, u32, u32, u32], C.c_int),
    "t0_bf16_matmul_backward_data": ([vp, u64, u64, u64, u32, u32, u32], C.c_int),
    "t0_bf16_matmul_backward_weight": ([vp, u64, u64, u64, u32, u32, u32], C.c_int),
    "t0_bf16_matmul_with_wt_bf16": ([vp, u64, u64, u64, u32, u32, u32], C.c_int),
    "t0_ffn_fused_rmsnorm_gemm": ([vp, u64, u64, u64, u64, u64, u32, u32, C.c_float], C.c_int),
    "t0_rmsnorm": ([vp, u64, u64, u64, u64, u64, u32, u32, u32, C.c_float, C.c_int], C.c_int),
    "t0_rmsnorm_w4a16": ([vp, P(W4A16DescC), P(RmsNormDescC)], C.c_int),
    "t0_rmsnorm_matmul": ([vp, u64, u64, u64, u64, u64, u64, u32, u32, u32, C.c_float], C.c_int),
    "t0_graph_begin": ([vp], C.c_int),
    "t0_graph_end": ([vp, P(vp)], C.c_int),
    "t0_graph_launch": ([vp, vp], C.c_int),
    "t0_graph_destroy": ([vp], C.c_int),
}

_lib = None


def lib() -> C.CDLL:
    """Load libt0gpu.so.  There is no fallback: a missing library is an error."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python __graft_entry__.py build` "
                              "(make -C rust-gpu_amd)")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib

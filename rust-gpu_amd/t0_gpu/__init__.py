"""t0_gpu -- Python mirror of the reference's GEMM-path API over libt0gpu.so.

The names follow the reference crate (t0-gpu) so callers and tests read like
the reference's own: ``GemmConfig`` and its presets (src/t0/gemm_gen.rs:55-145),
``auto_select`` / ``cached_auto_select`` / ``compute_grid_auto`` /
``build_kernargs`` (src/t0/gemm_gen.rs:308-484), ``TileGemm`` and
``build_kernargs_m`` (src/t0/tile_ir.rs), ``GpuRuntime`` with
``ensure_kernel_t0`` / ``dispatch`` / ``dispatch_async`` / ``wait_idle`` /
``alloc`` / ``recycle`` / ``read_f32`` (src/ignis/gpu_context.rs),
``GemmTuner`` / ``auto_gemm`` (src/t0/auto_gemm.rs) and ``GptqWeight``
(src/t0/quant_kernels.rs).  All work happens in the C ABI (include/t0_gemm.h);
every GPU call runs a gfx950 kernel of the library and there is no CPU path.
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass

import numpy as np

from . import _ffi
from ._ffi import (GemmConfigC, GemmDescC, GemmGeometryC, GptqViewC, KernelLoadConfigC, TileGemmC, TileTuneEntryC,
                   TuneEntryC, W4A16DescC, lib)

NT, NN = 0, 1
EPI_STORE_F32, EPI_BIAS_ADD, EPI_BIAS_ADD_RELU = 0, 1, 2
OUT_F32, OUT_BF16 = 0, 1
TEPI = {"bias": 1, "scale": 2, "relu": 3, "silu": 4, "gelu": 5, "abs": 6, "neg": 7, "clamp": 8}

PRESETS = ["tile_16x64_k16", "tile_32x64_direct", "tile_32x64_k16", "tile_32x64_k32", "tile_32x128_k16",
           "tile_64x64_k16", "tile_64x64_k32", "tile_128x64_k16", "tile_64x128_k16", "tile_128x64_k32",
           "tile_128x128_k16", "tile_64x64_k64", "tile_128x128_2pass", "tile_64x128_2pass",
           "tile_256x256_k64", "tile_256x128_k64", "tile_128x256_k64", "tile_128x128_k64", "tile_128x128_k32",
           "tile_128x64_k64", "tile_64x128_k64", "tile_32x64_k64", "tile_32x128_k64", "tile_256x256_k32"]


class T0Error(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{_ffi.STATUS.get(status, status)}: {msg}")
        self.status = status


def _check(rc: int) -> int:
    if rc < 0:
        raise T0Error(rc, lib().t0_last_error().decode())
    return rc


# ------------------------------------------------------------------ GemmConfig --

class GemmConfig(GemmConfigC):
    """src/t0/gemm_gen.rs:55-84 (fields), with ``out_dtype`` added."""

    def copy(self, **kw) -> "GemmConfig":
        c = GemmConfig()
        C.pointer(c)[0] = self
        for k, v in kw.items():
            setattr(c, k, 0 if v is None else v)
        return c

    def name(self) -> str:
        buf = C.create_string_buffer(160)
        _check(lib().t0_config_name(C.byref(self), buf, 160))
        return buf.value.decode()

    @staticmethod
    def from_name(name: str) -> "GemmConfig":
        c = GemmConfig()
        _check(lib().t0_config_from_name(name.encode(), C.byref(c)))
        return c

    def is_feasible(self) -> bool:
        return bool(lib().t0_config_is_feasible(C.byref(self)))

    def geometry(self) -> GemmGeometryC:
        g = GemmGeometryC()
        _check(lib().t0_config_geometry(C.byref(self), C.byref(g)))
        return g

    # geometry accessors, src/t0/gemm_gen.rs:147-213 (wave64 / 32x32 MFMA blocks)
    def n_waves(self): return self.wg_size // 64
    def n_col_tiles(self): return self.geometry().n_col_tiles
    def n_row_blocks(self): return self.geometry().n_row_blocks
    def rows_per_wave(self): return self.geometry().rows_per_wave
    def k_sub_steps(self): return self.tile_k // 16
    def lds_per_buffer(self): return (self.tile_m + self.tile_n) * self.tile_k * 2
    def lds_total(self): return self.geometry().lds_total
    def x_bytes_per_thread(self): return self.tile_m * self.tile_k * 2 // self.wg_size
    def wt_bytes_per_thread(self): return self.tile_n * self.tile_k * 2 // self.wg_size
    def mfma_per_k_tile(self): return self.geometry().mfma_per_k_tile
    def estimated_vgprs(self): return self.geometry().estimated_vgprs

    def __repr__(self):
        return f"GemmConfig({self.name()})"


def _preset(i: int) -> GemmConfig:
    c = GemmConfig()
    _check(lib().t0_config_preset(i, C.byref(c)))
    return c


for _i, _n in enumerate(PRESETS):
    setattr(GemmConfig, _n, staticmethod(lambda _i=_i: _preset(_i)))


def _config_list(fn) -> list:
    n = fn(None, 0)
    arr = (GemmConfig * n)()
    fn(arr, n)
    return list(arr)


def sweep_configs() -> list:
    return _config_list(lib().t0_sweep_configs)


def standard_configs() -> list:
    return _config_list(lib().t0_standard_configs)


def _sel(fn, a, b, c) -> GemmConfig:
    out = GemmConfig()
    _check(fn(a, b, c, C.byref(out)))
    return out


def auto_select(m: int, k: int, n: int) -> GemmConfig:
    """src/t0/gemm_gen.rs:340 (argument order m, k, n)."""
    return _sel(lib().t0_auto_select, m, k, n)


def auto_schedule_gemm(m: int, n: int, k: int, transpose=NT, out_dtype=OUT_F32) -> list:
    """src/t0/cost_model.rs:464-535: every feasible candidate, best first, as
    (GemmConfig, predicted microseconds)."""
    count = _check(lib().t0_auto_schedule_gemm(m, n, k, transpose, out_dtype, None, None, 0))
    raw = (GemmConfigC * count)()
    est = (C.c_double * count)()
    _check(lib().t0_auto_schedule_gemm(m, n, k, transpose, out_dtype, raw, est, count))
    out = []
    for i in range(count):
        c = GemmConfig()
        C.memmove(C.addressof(c), C.addressof(raw[i]), C.sizeof(GemmConfigC))
        out.append((c, float(est[i])))
    return out


def auto_select_legacy(m: int, k: int, n: int) -> GemmConfig:
    return _sel(lib().t0_auto_select_legacy, m, k, n)


def cached_auto_select(m: int, k: int, n: int) -> GemmConfig:
    return _sel(lib().t0_cached_auto_select, m, k, n)


def auto_select_backward_data(m, n_orig, k_orig) -> GemmConfig:
    return _sel(lib().t0_auto_select_backward_data, m, n_orig, k_orig)


def auto_select_backward_weight(m, n_orig, k_orig) -> GemmConfig:
    return _sel(lib().t0_auto_select_backward_weight, m, n_orig, k_orig)


def compute_grid(cfg: GemmConfig, m: int, n: int):
    gx, gy = C.c_uint32(), C.c_uint32()
    _check(lib().t0_compute_grid(C.byref(cfg), m, n, C.byref(gx), C.byref(gy)))
    return gx.value, gy.value


def compute_grid_split_k(cfg: GemmConfig, m: int, n: int, split_k: int):
    gx, gy = C.c_uint32(), C.c_uint32()
    _check(lib().t0_compute_grid_split_k(C.byref(cfg), m, n, split_k, C.byref(gx), C.byref(gy)))
    return gx.value, gy.value


def compute_grid_auto(cfg: GemmConfig, m: int, n: int):
    gx, gy = C.c_uint32(), C.c_uint32()
    _check(lib().t0_compute_grid_auto(C.byref(cfg), m, n, C.byref(gx), C.byref(gy)))
    return gx.value, gy.value


def build_kernargs(x, wt, y, k, n, m, cfg: GemmConfig) -> bytes:
    out = (C.c_uint8 * 40)()
    _check(lib().t0_build_kernargs(x, wt, y, k, n, m, C.byref(cfg), out))
    return bytes(out)


def build_kernargs_with_bias(x, wt, y, k, n, m, cfg: GemmConfig, bias) -> bytes:
    out = (C.c_uint8 * 48)()
    _check(lib().t0_build_kernargs_with_bias(x, wt, y, k, n, m, C.byref(cfg), bias, out))
    return bytes(out)


def build_kernargs_backward_data(dy, w, dx, m, n_orig, k_orig, cfg) -> bytes:
    out = (C.c_uint8 * 40)()
    _check(lib().t0_build_kernargs_backward_data(dy, w, dx, m, n_orig, k_orig, C.byref(cfg), out))
    return bytes(out)


def build_kernargs_backward_weight(dy_t, x_t, dw, m, n_orig, k_orig, cfg) -> bytes:
    out = (C.c_uint8 * 40)()
    _check(lib().t0_build_kernargs_backward_weight(dy_t, x_t, dw, m, n_orig, k_orig, C.byref(cfg), out))
    return bytes(out)


# -------------------------------------------------------------------- TileGemm --

class TileGemm(TileGemmC):
    """src/t0/tile_ir.rs:109-152."""

    @staticmethod
    def make(tile_m, tile_n, tile_k, waves_per_wg=0, split_k=1, transpose=NT, epilogue=(), out_dtype=OUT_F32,
             swap_grid=True, persistent=False) -> "TileGemm":
        s = TileGemm()
        s.tile_m, s.tile_n, s.tile_k = tile_m, tile_n, tile_k
        s.waves_per_wg, s.split_k, s.transpose = waves_per_wg, split_k, transpose
        s.double_buffer, s.swap_grid, s.persistent, s.out_dtype = 1, int(swap_grid), int(persistent), out_dtype
        s.n_epilogue = len(epilogue)
        for i, op in enumerate(epilogue):
            s.epilogue[i] = TEPI[op] if isinstance(op, str) else op
        return s

    def name(self) -> str:
        buf = C.create_string_buffer(200)
        _check(lib().t0_tile_name(C.byref(self), buf, 200))
        return buf.value.decode()

    def build_kernargs_m(self, x, wt, y, k, n, m, y_split_stride=0, bias=0, scale=1.0, clamp_min=0.0,
                         clamp_max=0.0) -> bytes:
        out = (C.c_uint8 * 96)()
        ln = C.c_size_t()
        _check(lib().t0_tile_build_kernargs_m(x, wt, y, k, n, m, C.byref(self), y_split_stride, bias, scale,
                                              clamp_min, clamp_max, out, C.byref(ln)))
        return bytes(out)[:ln.value]

    def compute_grid(self, m, n):
        g = (C.c_uint32 * 3)()
        _check(lib().t0_tile_compute_grid(C.byref(self), m, n, g))
        return list(g)


def tile_auto_select(m, k, n, transpose=NT) -> TileGemm:
    s = TileGemm()
    _check(lib().t0_tile_auto_select(m, k, n, transpose, C.byref(s)))
    return s


# --------------------------------------------------------------------- runtime --

class GpuBuffer:
    def __init__(self, rt: "GpuRuntime", handle):
        self.rt, self.h = rt, handle

    def gpu_addr(self) -> int:
        return lib().t0_buffer_addr(self.h)

    def size(self) -> int:
        return lib().t0_buffer_size(self.h)

    def write(self, data, offset: int = 0):
        arr = np.ascontiguousarray(data)
        _check(lib().t0_buffer_write(self.h, offset, arr.ctypes.data, arr.nbytes))

    def zero(self):
        _check(lib().t0_buffer_zero(self.h))

    def read(self, dtype, count, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        _check(lib().t0_buffer_read(self.h, offset, out.ctypes.data, out.nbytes))
        return out

    def free(self):
        if self.h:
            lib().t0_buffer_free(self.h)
            self.h = None


class GpuKernel:
    def __init__(self, handle):
        self.h = handle

    def info(self):
        wg = (C.c_uint32 * 3)()
        lds, ka = C.c_uint32(), C.c_uint32()
        name = C.create_string_buffer(200)
        _check(lib().t0_kernel_info(self.h, wg, C.byref(lds), C.byref(ka), name, 200))
        return {"workgroup_size": list(wg), "lds_size": lds.value, "kernarg_size": ka.value,
                "name": name.value.decode()}


class GpuRuntime:
    """src/ignis/gpu_context.rs:99-119 (device + stream + kernel cache + pool + poison flag)."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        _check(lib().t0_runtime_create(device, C.byref(h)))
        self.h = h

    @classmethod
    def new(cls, device: int = 0) -> "GpuRuntime":
        return cls(device)

    def close(self):
        if self.h:
            lib().t0_runtime_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def device_info(self):
        arch = C.create_string_buffer(64)
        cu, clk = C.c_int(), C.c_int()
        _check(lib().t0_runtime_device_info(self.h, arch, 64, C.byref(cu), C.byref(clk)))
        return {"arch": arch.value.decode(), "cu_count": cu.value, "clock_khz": clk.value}

    def set_stream(self, stream_handle):
        _check(lib().t0_runtime_set_stream(self.h, stream_handle))

    def is_poisoned(self) -> bool:
        return bool(lib().t0_runtime_is_poisoned(self.h))

    def mark_poisoned(self):
        _check(lib().t0_runtime_mark_poisoned(self.h))

    # kernels
    def ensure_kernel_t0(self, cfg: GemmConfig) -> GpuKernel:
        k = C.c_void_p()
        _check(lib().t0_ensure_kernel(self.h, C.byref(cfg), C.byref(k)))
        return GpuKernel(k)

    def ensure_tile_kernel(self, spec: TileGemm) -> GpuKernel:
        k = C.c_void_p()
        _check(lib().t0_ensure_tile_kernel(self.h, C.byref(spec), C.byref(k)))
        return GpuKernel(k)

    def get_kernel(self, name: str) -> GpuKernel:
        k = C.c_void_p()
        _check(lib().t0_get_kernel(self.h, name.encode(), C.byref(k)))
        return GpuKernel(k)

    def kernel_load(self, code_object: tuple, symbol: str, workgroup_size, lds_size=0, kernarg_size=0) -> GpuKernel:
        """GpuKernel::load (src/kfd/kernel.rs:26-134): code_object = (pointer, size)."""
        cfg = KernelLoadConfigC()
        for i, w in enumerate(list(workgroup_size) + [1] * (3 - len(workgroup_size))):
            cfg.workgroup_size[i] = w
        cfg.lds_size, cfg.kernarg_size = lds_size, kernarg_size
        k = C.c_void_p()
        _check(lib().t0_kernel_load(self.h, code_object[0], code_object[1], symbol.encode(), C.byref(cfg),
                                    C.byref(k)))
        return GpuKernel(k)

    def _grid(self, grid):
        g = list(grid) + [1] * (3 - len(grid))
        return (C.c_uint32 * 3)(*g)

    def dispatch(self, kernel: GpuKernel, grid, kernargs: bytes):
        buf = C.create_string_buffer(bytes(kernargs), len(kernargs))
        _check(lib().t0_dispatch(self.h, kernel.h, self._grid(grid), buf, len(kernargs)))

    def dispatch_async(self, kernel: GpuKernel, grid, kernargs: bytes) -> int:
        buf = C.create_string_buffer(bytes(kernargs), len(kernargs))
        return _check(lib().t0_dispatch_async(self.h, kernel.h, self._grid(grid), buf, len(kernargs)))

    def wait_idle(self):
        _check(lib().t0_wait_idle(self.h))

    synchronize = wait_idle

    # memory
    def alloc(self, nbytes: int) -> GpuBuffer:
        b = C.c_void_p()
        _check(lib().t0_alloc(self.h, nbytes, C.byref(b)))
        return GpuBuffer(self, b)

    def upload(self, arr: np.ndarray) -> GpuBuffer:
        arr = np.ascontiguousarray(arr)
        b = self.alloc(max(arr.nbytes, 1))
        if arr.nbytes:
            _check(lib().t0_buffer_write(b.h, 0, arr.ctypes.data, arr.nbytes))
        return b

    def recycle(self, buf: GpuBuffer):
        _check(lib().t0_recycle(self.h, buf.h))
        buf.h = None

    def read_f32(self, buf: GpuBuffer, count: int) -> np.ndarray:
        return buf.read(np.float32, count)

    def memset(self, addr: int, value: int, nbytes: int):
        _check(lib().t0_memset_d(self.h, addr, value, nbytes))

    # high level
    def gemm(self, a: int, b: int, c: int, m: int, n: int, k: int, transpose=NT, out_dtype=OUT_F32,
             cfg: GemmConfig | None = None, lda=0, ldb=0, ldc=0, bias=0, epilogue=(), scale=1.0,
             clamp_min=0.0, clamp_max=0.0):
        d = GemmDescC(a=a, b=b, c=c, bias=bias, m=m, n=n, k=k, lda=lda, ldb=ldb, ldc=ldc, transpose=transpose,
                      out_dtype=out_dtype, n_epilogue=len(epilogue), scale=scale, clamp_min=clamp_min,
                      clamp_max=clamp_max)
        for i, op in enumerate(epilogue):
            d.epilogue[i] = TEPI[op] if isinstance(op, str) else op
        _check(lib().t0_gemm(self.h, C.byref(cfg) if cfg is not None else None, C.byref(d)))

    def gemm_noalloc(self, a: int, b: int, c: int, m: int, n: int, k: int, transpose=NT, out_dtype=OUT_F32,
                     cfg: GemmConfig | None = None, lda=0, ldb=0, ldc=0):
        """t0_gemm without device allocation: split-K partials and counters in
        the library's fixed per-device scratch array (see t0_gemm_noalloc)."""
        d = GemmDescC(a=a, b=b, c=c, m=m, n=n, k=k, lda=lda, ldb=ldb, ldc=ldc, transpose=transpose,
                      out_dtype=out_dtype)
        _check(lib().t0_gemm_noalloc(self.h, C.byref(cfg) if cfg is not None else None, C.byref(d)))

    def gemm_clock_probe(self, a: int, b: int, c: int, m: int, n: int, k: int, transpose=NT, out_dtype=OUT_F32,
                         cfg: GemmConfig | None = None):
        """One GEMM with per-workgroup timestamps: (median shader clock in MHz,
        first-start to last-end span in us, median shader cycles per workgroup)."""
        d = GemmDescC(a=a, b=b, c=c, m=m, n=n, k=k, transpose=transpose, out_dtype=out_dtype)
        mhz, span, cyc = C.c_double(), C.c_double(), C.c_double()
        _check(lib().t0_gemm_clock_probe(self.h, C.byref(cfg) if cfg is not None else None, C.byref(d),
                                         C.byref(mhz), C.byref(span), C.byref(cyc)))
        return mhz.value, span.value, cyc.value

    def gemm_select(self, m, n, k, transpose=NT, out_dtype=OUT_F32) -> GemmConfig:
        d = GemmDescC(m=m, n=n, k=k, transpose=transpose, out_dtype=out_dtype)
        c = GemmConfig()
        _check(lib().t0_gemm_select(self.h, C.byref(d), C.byref(c)))
        return c

    def _w4desc(self, a, qweight, scales, zeros, c, m, n, k, group_size=128, zero_const=8, scales_f32=False,
                out_f32=False, split_k=0, lda=0, ldc=0):
        return W4A16DescC(a=a, qweight=qweight, scales=scales, zeros=zeros or 0, c=c, m=m, n=n, k=k, lda=lda,
                          ldc=ldc, group_size=group_size, zero_const=zero_const, scales_f32=int(scales_f32),
                          out_f32=int(out_f32), split_k=split_k)

    def w4a16(self, *args, **kw):
        d = self._w4desc(*args, **kw)
        _check(lib().t0_w4a16_gemm(self.h, C.byref(d)))

    def w4a16_plan(self, *args, **kw):
        d = self._w4desc(*args, **kw)
        name = C.create_string_buffer(96)
        sk = C.c_uint32()
        _check(lib().t0_w4a16_plan(self.h, C.byref(d), name, 96, C.byref(sk)))
        return name.value.decode(), sk.value

    def dequant_int4(self, packed, scales, zero_points, output, rows, cols, group_size_log2, bf16_out=False):
        _check(lib().t0_dequant_int4(self.h, packed, scales, zero_points, output, rows, cols, group_size_log2,
                                     int(bf16_out)))

    def splitk_reduce(self, src, plane_stride, planes, dst, m, n, out_bf16=False):
        _check(lib().t0_splitk_reduce(self.h, src, plane_stride, planes, dst, m, n, int(out_bf16)))

    def f32_to_bf16(self, src, dst, count):
        _check(lib().t0_f32_to_bf16(self.h, src, dst, count))

    def capture(self, fn) -> "Graph":
        """Record everything fn() launches on this runtime's stream into a graph."""
        _check(lib().t0_graph_begin(self.h))
        try:
            fn()
        except Exception:
            g = C.c_void_p()
            lib().t0_graph_end(self.h, C.byref(g))
            if g:
                lib().t0_graph_destroy(g)
            raise
        g = C.c_void_p()
        _check(lib().t0_graph_end(self.h, C.byref(g)))
        return Graph(self, g)

    def floor_stream_read(self, src, nbytes, sink, workgroups=256, threads=1024):
        _check(lib().t0_floor_stream_read(self.h, src, nbytes, sink, workgroups, threads))

    def floor_tile_read(self, a, b, m, n, k, transpose=NT, mode=3, cfg: GemmConfig | None = None, lda=0, ldb=0):
        """Only the operand slices of the GEMM tiling cfg (None: the pick) move
        to LDS: mode 1 the A slices, 2 the B slices, 3 both.  Asynchronous."""
        d = GemmDescC(a=a, b=b, m=m, n=n, k=k, lda=lda, ldb=ldb, transpose=transpose)
        _check(lib().t0_floor_tile_read(self.h, C.byref(cfg) if cfg is not None else None, C.byref(d), mode))

    def floor_empty(self, workgroups=256, threads=1024):
        _check(lib().t0_floor_empty(self.h, workgroups, threads))

    def floor_mfma(self, operands, out, workgroups=256, mfma_per_wave=2048):
        _check(lib().t0_floor_mfma(self.h, operands, out, workgroups, mfma_per_wave))

    def floor_lds(self, mode, src, out, workgroups=256, threads=512, rounds=2000):
        _check(lib().t0_floor_lds(self.h, mode, src, out, workgroups, threads, rounds))

    def copy_device(self, src, dst, nbytes):
        _check(lib().t0_copy_device(self.h, src, dst, nbytes))

    def unpad_2d(self, padded, out, m, n, n_pad):
        _check(lib().t0_unpad_2d(self.h, padded, out, m, n, n_pad))


class Graph:
    def __init__(self, rt: GpuRuntime, handle):
        self.rt, self.h = rt, handle

    def launch(self):
        _check(lib().t0_graph_launch(self.rt.h, self.h))

    def destroy(self):
        """Releases the graph (and its pin on the runtime's shared buffers)."""
        if self.h:
            lib().t0_graph_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Event:
    def __init__(self):
        h = C.c_void_p()
        _check(lib().t0_event_create(C.byref(h)))
        self.h = h

    def record(self, rt: GpuRuntime):
        _check(lib().t0_event_record(rt.h, self.h))

    def synchronize(self):
        _check(lib().t0_event_synchronize(self.h))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        _check(lib().t0_event_elapsed_ms(self.h, end.h, C.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self.h:
                lib().t0_event_destroy(self.h)
        except Exception:
            pass


def code_object():
    """The library's gfx950 code object as (pointer, size)."""
    p, n = C.c_void_p(), C.c_size_t()
    _check(lib().t0_code_object(C.byref(p), C.byref(n)))
    return p.value, n.value


def generate(cfg: GemmConfig) -> str:
    """gemm_gen::generate + compile: the symbol of the precompiled kernel."""
    buf = C.create_string_buffer(128)
    _check(lib().t0_generate(C.byref(cfg), buf, 128))
    return buf.value.decode()


# ---------------------------------------------------------------------- tuner --

class GemmTuner:
    """src/t0/auto_gemm.rs:46-216."""

    def __init__(self, cache_dir: str | None = None, max_candidates: int = 8, n_iters: int = 10):
        if cache_dir is not None:
            _check(lib().t0_tuner_set_cache_dir(cache_dir.encode()))
        _check(lib().t0_tuner_set_params(max_candidates, n_iters))

    def tune(self, rt: GpuRuntime, m: int, n: int, k: int, transpose=NT, out_dtype=OUT_F32):
        c = GemmConfig()
        tf = C.c_double()
        _check(lib().t0_tune(rt.h, m, n, k, transpose, out_dtype, C.byref(c), C.byref(tf)))
        return c, tf.value

    @staticmethod
    def save_cache(m: int, n: int, k: int, cfg: GemmConfig, tflops: float, transpose=NT, out_dtype=OUT_F32):
        """GemmTuner::save_cache (src/t0/auto_gemm.rs:474-501)."""
        _check(lib().t0_tuner_cache_store(m, n, k, transpose, out_dtype, C.byref(cfg), tflops))

    @staticmethod
    def load_cache(m: int, n: int, k: int, transpose=NT, out_dtype=OUT_F32):
        """GemmTuner::load_cache (src/t0/auto_gemm.rs:439-472): (config, tflops) or None."""
        c, tf = GemmConfig(), C.c_double()
        rc = lib().t0_tuner_cache_load(m, n, k, transpose, out_dtype, C.byref(c), C.byref(tf))
        if rc == -6:   # T0_ERR_NOT_FOUND
            return None
        _check(rc)
        return c, tf.value

    @staticmethod
    def invalidate(m: int, n: int, k: int, transpose=NT, out_dtype=OUT_F32):
        """GemmTuner::invalidate (src/t0/auto_gemm.rs:503-507)."""
        _check(lib().t0_tuner_invalidate(m, n, k, transpose, out_dtype))

    @staticmethod
    def results(m: int, n: int, k: int, transpose=NT, out_dtype=OUT_F32):
        """GemmTuneResult.all (src/t0/auto_gemm.rs:30-42): every candidate the
        last tune of this problem timed, fastest first, as (GemmConfig,
        tflops), and whether the list came from the cache file; None if the
        problem was never tuned here and has no cache file."""
        n_all, cached = C.c_uint32(), C.c_int()
        rc = lib().t0_tune_results(m, n, k, transpose, out_dtype, None, 0, C.byref(n_all), C.byref(cached))
        if rc == -6:   # T0_ERR_NOT_FOUND
            return None
        _check(rc)
        cap = n_all.value
        entries = (TuneEntryC * max(cap, 1))()
        _check(lib().t0_tune_results(m, n, k, transpose, out_dtype, entries, cap, C.byref(n_all), C.byref(cached)))
        out = []
        for e in entries[:min(n_all.value, cap)]:
            c = GemmConfig()
            C.memmove(C.addressof(c), C.addressof(e.cfg), C.sizeof(GemmConfigC))
            out.append((c, e.tflops))
        return out, bool(cached.value)


@dataclass
class TileIrTuneResult:
    """src/t0/cost_model.rs:824-833: the best tile_ir spec, its TFLOP/s, every
    timed candidate as (name, tflops) fastest first (empty from the cache)."""
    best: TileGemm
    best_tflops: float
    all: list
    from_cache: bool


def tune_tile_ir(rt: GpuRuntime, m: int, n: int, k: int) -> TileIrTuneResult:
    """cost_model::tune_tile_ir (src/t0/cost_model.rs:855-1080); the cache
    directory and the number of timed launches are GemmTuner's."""
    best, tf = TileGemm(), C.c_double()
    cap = 64
    entries = (TileTuneEntryC * cap)()
    n_all, cached = C.c_uint32(), C.c_int()
    _check(lib().t0_tile_tune(rt.h, m, n, k, C.byref(best), C.byref(tf), entries, cap, C.byref(n_all),
                              C.byref(cached)))
    timed = []
    for e in entries[:min(n_all.value, cap)]:
        s = TileGemm()
        C.memmove(C.byref(s), C.byref(e.spec), C.sizeof(TileGemmC))
        timed.append((s.name(), e.tflops))
    return TileIrTuneResult(best, tf.value, timed, bool(cached.value))


def auto_gemm(rt: GpuRuntime, a: int, b: int, c: int, m: int, n: int, k: int) -> float:
    tf = C.c_double()
    _check(lib().t0_auto_gemm(rt.h, a, b, c, m, n, k, C.byref(tf)))
    return tf.value


# ----------------------------------------------------------------------- INT4 --

@dataclass
class GptqWeight:
    """src/t0/quant_kernels.rs:188-296."""
    rows: int
    cols: int
    group_size: int
    n_groups: int
    packed_weights: np.ndarray
    scales: np.ndarray
    zero_points: np.ndarray
    _raw: bytes = b""

    @staticmethod
    def from_bytes(raw: bytes) -> "GptqWeight":
        v = GptqViewC()
        buf = C.create_string_buffer(raw, len(raw))
        _check(lib().t0_gptq_from_bytes(buf, len(raw), C.byref(v)))
        pk = v.rows * v.cols // 2
        npar = v.rows * v.n_groups
        packed = np.frombuffer(raw, np.uint8, pk, 12).copy()
        scales = np.frombuffer(raw, "<f4", npar, 12 + pk).copy()
        zps = np.frombuffer(raw, "<i4", npar, 12 + pk + 4 * npar).copy()
        return GptqWeight(v.rows, v.cols, v.group_size, v.n_groups, packed, scales, zps, raw)

    def to_bytes(self) -> bytes:
        return (struct.pack("<III", self.rows, self.cols, self.group_size) + self.packed_weights.tobytes()
                + self.scales.astype("<f4").tobytes() + self.zero_points.astype("<i4").tobytes())

    def _view(self):
        raw = self._raw or self.to_bytes()
        self._keep = C.create_string_buffer(raw, len(raw))
        v = GptqViewC()
        _check(lib().t0_gptq_from_bytes(self._keep, len(raw), C.byref(v)))
        return v

    def gpu_buffer_size(self) -> int:
        v = self._view()
        return lib().t0_gptq_gpu_buffer_size(C.byref(v))

    def to_w4a16(self, scales_f32=False, with_zeros=True):
        """-> (qweight [N][K/8] u32, scales [G][N], zeros [G][N/8] u32 or None)."""
        v = self._view()
        qw = np.empty((self.rows, self.cols // 8), np.uint32)
        sc = np.empty((self.n_groups, self.rows), np.float32 if scales_f32 else np.uint16)
        zw = np.empty((self.n_groups, self.rows // 8), np.uint32) if with_zeros else None
        _check(lib().t0_gptq_to_w4a16(C.byref(v), qw.ctypes.data, sc.ctypes.data, int(scales_f32),
                                      zw.ctypes.data if zw is not None else None))
        return qw, sc, zw

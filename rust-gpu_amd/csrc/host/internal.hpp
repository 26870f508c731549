// internal.hpp -- shared declarations of the host side of libt0gpu.
#pragma once
#include <cstdarg>
#include <cstdint>
#include <string>
#include <vector>

#include "../../../include/t0_gemm.h"
#include "../kernel_params.h"

namespace t0h {

// ---- errors (thread-local last error) ----------------------------------------
int fail(int status, const char* fmt, ...);
void clear_error();

// ---- compiled GEMM kernel instances -------------------------------------------
// One entry per extern "C" kernel of csrc/kernels/gemm_bf16.hip (both layouts).
struct GemmInstance {
    uint32_t bm, bn, bk, wm, wn, stages;
    uint32_t nw() const { return wm * wn; }
    uint32_t threads() const { return wm * wn * 64; }
    std::string symbol(bool nn) const;
    uint32_t lds_bytes() const;   // static LDS of the kernel
};
const std::vector<GemmInstance>& gemm_instances();
const GemmInstance* find_instance(uint32_t bm, uint32_t bn, uint32_t bk, uint32_t nw);
const GemmInstance* instance_for(const t0_gemm_config& c);

// Config checks shared with the runtime.
bool config_valid(const t0_gemm_config& c, std::string* why);
std::string config_name(const t0_gemm_config& c);
uint32_t split_of(const t0_gemm_config& c);

// ---- tile_ir specs ---------------------------------------------------------------
std::string tile_name(const t0_tile_gemm& s);
const GemmInstance* tile_instance(const t0_tile_gemm& s);
uint32_t tile_epi_ops(const t0_tile_gemm& s);
// kernarg layout of a tile_ir spec: offsets of optional arguments, total size
struct TileArgLayout {
    uint32_t bias_off = 0, scale_off = 0, clamp_off = 0, size = 44;
    bool has_bias = false, has_scale = false, has_clamp = false;
};
TileArgLayout tile_arg_layout(const t0_tile_gemm& s);

// ---- analytical gfx950 model used by auto_select and to rank tuner candidates ---
struct Candidate {
    t0_gemm_config cfg;
    double est_us;
};
std::vector<Candidate> rank_candidates(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose,
                                       uint32_t out_dtype, bool allow_fixup);

// ---- GEMM on caller-provided scratch (the no-allocation entry point) -----------
// Runs t0_gemm with the in-kernel split-K using `scratch` (device memory of
// `bytes`): counters for up to T0_NOALLOC_MAX_TILES tiles first, partial tiles
// after them.  Allocates nothing; clears the counters it uses with a kernel.
int gemm_with_scratch(t0_runtime* rt, const t0_gemm_config* cfg, const t0_gemm_desc* d, void* scratch,
                      size_t bytes);
int runtime_device(const t0_runtime* rt);

}  // namespace t0h

// Implemented in csrc/host/noalloc.hip (compiled by hipcc with its device
// array): resolves that array's address on the current device.
extern "C" int t0h_noalloc_setup(int device);

// config.cpp -- GemmConfig / TileGemm value logic: presets, geometry,
// feasibility, names, grids, kernarg layouts and shape-based selection.
// No HIP calls: everything here runs (and is tested) without a GPU.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>

#include "internal.hpp"

namespace t0h {

// ------------------------------------------------------------------ errors --
static thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}
void clear_error() { g_last_error.clear(); }
const char* last_error() { return g_last_error.c_str(); }

// ------------------------------------------------------ kernel instances --
// Must list exactly the T0_GEMM_BOTH(...) instances of gemm_bf16.hip.
const std::vector<GemmInstance>& gemm_instances() {
    static const std::vector<GemmInstance> v = {
        {256, 256, 64, 2, 2, 2}, {256, 256, 64, 2, 4, 2}, {256, 256, 64, 4, 2, 2}, {256, 256, 32, 2, 2, 4},
        {256, 256, 32, 2, 4, 4}, {256, 128, 64, 2, 2, 3}, {128, 256, 64, 2, 2, 3},
        {128, 128, 64, 2, 2, 4}, {128, 128, 32, 2, 2, 4}, {128, 64, 64, 2, 2, 4},  {64, 128, 64, 2, 2, 4}, {64, 64, 64, 2, 2, 4},
        {64, 64, 64, 1, 1, 4},   {32, 64, 64, 1, 1, 6},   {32, 128, 64, 1, 2, 4},
        {32, 64, 16, 1, 1, 4},   {32, 64, 32, 1, 1, 4},   {32, 128, 16, 1, 1, 4},
        {64, 64, 16, 1, 1, 4},   {64, 64, 32, 1, 1, 4},   {128, 64, 16, 2, 1, 4},
        {128, 64, 32, 2, 1, 4},  {64, 128, 16, 1, 1, 4},  {128, 128, 16, 2, 1, 4},
    };
    return v;
}

std::string GemmInstance::symbol(bool nn) const {
    char b[96];
    snprintf(b, sizeof b, "t0k_gemm_%ux%ux%u_w%ux%u_s%u_%s", bm, bn, bk, wm, wn, stages, nn ? "nn" : "nt");
    return b;
}

uint32_t GemmInstance::lds_bytes() const {
    const uint32_t stage = (bm + bn) * bk * 2;
    const uint32_t epi = nw() * 32 * (bn / wn + 4) * 4;
    return std::max(stage * stages, epi);
}

const GemmInstance* find_instance(uint32_t bm, uint32_t bn, uint32_t bk, uint32_t nw) {
    for (const auto& g : gemm_instances())
        if (g.bm == bm && g.bn == bn && g.bk == bk && (nw == 0 || g.nw() == nw)) return &g;
    return nullptr;
}

const GemmInstance* instance_for(const t0_gemm_config& c) {
    if (c.wg_size == 0 || c.wg_size % 64) return nullptr;
    return find_instance(c.tile_m, c.tile_n, c.tile_k, c.wg_size / 64);
}

uint32_t split_of(const t0_gemm_config& c) { return c.split_k > 1 ? c.split_k : 1; }

bool config_valid(const t0_gemm_config& c, std::string* why) {
    auto no = [&](const char* w) { if (why) *why = w; return false; };
    if (!instance_for(c)) return no("no gfx950 kernel for this tile_m x tile_n x tile_k / wg_size (wave64)");
    const uint32_t sk = split_of(c);
    if (sk > 16 || (sk & (sk - 1))) return no("split_k must be a power of two <= 16");
    if (c.transpose > T0_NN) return no("transpose must be NT or NN");
    if (c.epilogue > T0_EPI_BIAS_ADD_RELU) return no("unknown epilogue");
    if (c.out_dtype > T0_OUT_BF16) return no("unknown out_dtype");
    if (sk > 1 && c.out_dtype == T0_OUT_BF16)
        return no("split_k planes are f32 partial sums: out_dtype must be f32 (t0_gemm reduces bf16 in-kernel)");
    if (sk > 1 && c.epilogue != T0_EPI_STORE_F32)
        return no("an epilogue on split_k planes would be applied once per plane");
    return true;
}

std::string config_name(const t0_gemm_config& c) {
    // format of GemmConfig::name (src/t0/gemm_gen.rs:215-235)
    std::string s = "t0_gemm_" + std::to_string(c.tile_m) + "x" + std::to_string(c.tile_n) + "_k" +
                    std::to_string(c.tile_k);
    s += c.use_lds ? (c.double_buffer ? "_ldsdb" : "_lds") : "_direct";
    if (split_of(c) > 1) s += "_sk" + std::to_string(c.split_k);
    if (c.n_col_passes > 1) s += "_" + std::to_string(c.n_col_passes) + "p";
    if (!c.swap_grid) s += "_mg";
    if (c.wgp_mode) s += "_wgp";
    if (c.transpose == T0_NN) s += "_nn";
    if (c.epilogue == T0_EPI_BIAS_ADD) s += "_bias";
    else if (c.epilogue == T0_EPI_BIAS_ADD_RELU) s += "_bias_relu";
    if (c.out_dtype == T0_OUT_BF16) s += "_bf16";
    return s;
}

static t0_gemm_config mk(uint32_t tm, uint32_t tn, uint32_t tk, uint32_t wg, bool lds, bool db, uint32_t passes,
                         bool wgp) {
    t0_gemm_config c;
    memset(&c, 0, sizeof c);
    c.tile_m = tm; c.tile_n = tn; c.tile_k = tk; c.wg_size = wg;
    c.use_lds = lds; c.double_buffer = db; c.split_k = 0; c.lds_pad = 0; c.n_col_passes = passes;
    c.swap_grid = 1; c.wgp_mode = wgp; c.transpose = T0_NT; c.epilogue = T0_EPI_STORE_F32; c.out_dtype = T0_OUT_F32;
    return c;
}

static bool preset(int id, t0_gemm_config* o) {
    switch (id) {
    // src/t0/gemm_gen.rs:86-145 (values kept; wg_size counts wave64 lanes on gfx950)
    case T0_PRESET_16x64_K16: *o = mk(16, 64, 16, 32, true, true, 1, true); return true;
    case T0_PRESET_32x64_DIRECT: *o = mk(32, 64, 16, 64, false, false, 1, true); return true;
    case T0_PRESET_32x64_K16: *o = mk(32, 64, 16, 64, true, true, 1, true); return true;
    case T0_PRESET_32x64_K32: *o = mk(32, 64, 32, 64, true, true, 1, true); return true;
    case T0_PRESET_32x128_K16: *o = mk(32, 128, 16, 64, true, true, 1, true); return true;
    case T0_PRESET_64x64_K16: *o = mk(64, 64, 16, 64, true, true, 1, true); return true;
    case T0_PRESET_64x64_K32: *o = mk(64, 64, 32, 64, true, true, 1, true); return true;
    case T0_PRESET_128x64_K16: *o = mk(128, 64, 16, 128, true, true, 1, true); return true;
    case T0_PRESET_64x128_K16: *o = mk(64, 128, 16, 64, true, true, 1, true); return true;
    case T0_PRESET_128x64_K32: *o = mk(128, 64, 32, 128, true, true, 1, true); return true;
    case T0_PRESET_128x128_K16: *o = mk(128, 128, 16, 128, true, true, 1, true); return true;
    case T0_PRESET_64x64_K64: *o = mk(64, 64, 64, 64, true, true, 1, true); return true;
    case T0_PRESET_128x128_2PASS: *o = mk(128, 64, 16, 128, true, true, 2, true); return true;
    case T0_PRESET_64x128_2PASS: *o = mk(64, 64, 16, 64, true, true, 2, true); return true;
    // gfx950-native
    case T0_PRESET_256x256_K64: *o = mk(256, 256, 64, 256, true, true, 1, false); return true;
    case T0_PRESET_256x128_K64: *o = mk(256, 128, 64, 256, true, true, 1, false); return true;
    case T0_PRESET_128x256_K64: *o = mk(128, 256, 64, 256, true, true, 1, false); return true;
    case T0_PRESET_128x128_K64: *o = mk(128, 128, 64, 256, true, true, 1, false); return true;
    case T0_PRESET_128x128_K32: *o = mk(128, 128, 32, 256, true, true, 1, false); return true;
    case T0_PRESET_128x64_K64: *o = mk(128, 64, 64, 256, true, true, 1, false); return true;
    case T0_PRESET_64x128_K64: *o = mk(64, 128, 64, 256, true, true, 1, false); return true;
    case T0_PRESET_32x64_K64: *o = mk(32, 64, 64, 64, true, true, 1, false); return true;
    case T0_PRESET_32x128_K64: *o = mk(32, 128, 64, 128, true, true, 1, false); return true;
    case T0_PRESET_256x256_K32: *o = mk(256, 256, 32, 256, true, true, 1, false); return true;
    default: return false;
    }
}

// -------------------------------------------------------- selection model --
// gfx950 (MI355X): 256 CUs, 4 SIMDs each, 1024 bf16 FLOP/cycle/SIMD dense,
// 2.4 GHz, 160 KiB LDS/CU, 512 VGPRs per lane at one wave per SIMD.
namespace hw {
constexpr double CUS = 256;
constexpr double LDS = 160 * 1024;
}

static uint32_t est_vgprs(const GemmInstance& g) {
    const uint32_t fm = g.bm / g.wm / 32, fn = g.bn / g.wn / 32;
    return fm * fn * 16 + (fm + fn) * 8 + 48;
}

// Per-tile cost, fitted (fit_tile_cost.py, beside this file) to every ranked tile x
// split-K candidate timed on MI355X by `bench.py --only tiles`: 28 LLM
// shapes (NN, bf16 out, M = 16..4096, N = 1024..14336, K = 4096 or 11008),
// the weight operand B rotated through more copies than the 256 MB MALL
// holds (read cold from HBM, as in inference).  Predicted time:
//   per workgroup  a + b * k_len / 1000 us while a round of workgroups
//                  (CUs x workgroups per CU, by LDS) is resident; a partly
//                  filled last round costs DISC + (1 - DISC) * fill of a round;
//   co-resident workgroups (2+ per CU) run at most 1/CO_RESIDENT as fast,
//                  so ceil(workgroups / CUs) of them queue on one CU;
//   memory         no faster than A + B + C, plus the split-K partial
//                  tiles written and read back, over HBM_TBS, nor the
//                  operand re-reads (A once per column tile, B once per row
//                  tile) over L2_TBS;
//   split-K        + FIX us + FIX_MB us per MB of partial tiles;
//   near-ties      within 1 % of the best predicted time (several tiles at
//                  the memory bound, shapes outside the fitted range) go to
//                  the fewest partial-tile bytes, then the smallest tile.
// Fitted to the geometric mean of six runs on three boxes (a candidate's
// time moves by a median 1 %, up to ~15 % run to run), 34 shapes: least
// squares on log time, then refined for the picks (the measured regret
// under a soft minimum of the predicted times, plus 3 x the squared log
// error).  The fit drives several constants to their bounds (no split-K
// term, an HBM bound that never binds on the fitted shapes): the
// per-workgroup a and b carry it, and the predicted times rank the
// candidates (median error 14 %) rather than forecast them.  The partial
// tiles in the HBM bound and the near-tie rule came after the fit; they
// change no pick on the fitted shapes.  The pick is within 3 % of the measured best
// on all 34 shapes of that data (33 with each shape left out of the fit,
// at most 8 % slower), 26 of 34 re-measured on a fourth box (at most
// 18 %), and the measured best is among the 4 best-predicted candidates
// on every shape, so the tuner's candidates (t0_tune, top 8) include it.
struct TileCost {
    uint32_t bm, bn, bk, nw;
    double a_us, b_us;
};
constexpr TileCost kTileCost[] = {
    {256, 256, 64, 8, 45.46, 7.71}, {256, 128, 64, 4, 27.50, 12.11}, {128, 256, 64, 4, 28.30, 11.53},
    {128, 128, 64, 4, 18.31, 4.56}, {128, 64, 64, 4, 8.26, 6.64},    {64, 128, 64, 4, 7.17, 5.96},
    {64, 64, 64, 1, 2.97, 6.02},    {32, 128, 64, 2, 5.97, 4.84},    {32, 64, 64, 1, 2.38, 4.43},
};
constexpr double kDisc = 1.000, kFixUs = 0.000, kFixUsPerMB = 0.000;
constexpr double kHbmTBs = 8.000, kL2TBs = 18.896, kCoResident = 1.000;

std::vector<Candidate> rank_candidates(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype,
                                       bool allow_fixup) {
    std::vector<Candidate> out;
    for (const auto& tc : kTileCost) {
        const GemmInstance* g = find_instance(tc.bm, tc.bn, tc.bk, tc.nw);
        if (!g) continue;
        const double slots = hw::CUS * std::max(1.0, std::min(std::floor(hw::LDS / g->lds_bytes()), 8.0));
        const double tiles = std::ceil((double)m / g->bm) * std::ceil((double)n / g->bn);
        for (uint32_t sk = 1; sk <= 16; sk *= 2) {
            if (sk > 1) {
                if (k % (8 * sk)) continue;
                if (k / sk < g->bk * 2) continue;
                if (!allow_fixup && out_dtype == T0_OUT_BF16) continue;
            }
            const double wgs = tiles * sk;
            const double full = std::floor(wgs / slots), fill = wgs / slots - full;
            const double rounds = full + (fill > 0 ? kDisc + (1 - kDisc) * fill : 0.0);
            const double t_wg = tc.a_us + tc.b_us * (k / (double)sk) / 1000.0;
            double t = rounds * t_wg;
            if (slots > hw::CUS) t = std::max(t, std::ceil(wgs / hw::CUS) * t_wg * kCoResident);
            const double part = sk > 1 ? wgs * g->bm * g->bn * 4.0 : 0.0;   // f32 partial tiles
            const double hbm = (double)k * n * 2 + (double)m * k * 2 + (double)m * n * 2 + 2 * part;
            const double l2 = (double)m * k * 2 * std::ceil((double)n / g->bn) + (double)n * k * 2 * std::ceil((double)m / g->bm);
            t = std::max({t, hbm / (kHbmTBs * 1e6), l2 / (kL2TBs * 1e6)});
            if (sk > 1) t += kFixUs + kFixUsPerMB * wgs * g->bm * g->bn * 4 / 1e6;
            t0_gemm_config c = mk(g->bm, g->bn, g->bk, g->threads(), true, true, 1, false);
            c.split_k = sk > 1 ? sk : 0;
            c.transpose = (uint8_t)transpose;
            c.out_dtype = (uint8_t)out_dtype;
            out.push_back({c, t});
        }
    }
    std::stable_sort(out.begin(), out.end(), [](const Candidate& a, const Candidate& b) { return a.est_us < b.est_us; });
    // near-ties: the fewest partial-tile bytes, then the smallest tile, moves to the front
    auto part_bytes = [&](const t0_gemm_config& c) {
        return c.split_k > 1 ? std::ceil((double)m / c.tile_m) * std::ceil((double)n / c.tile_n) * c.split_k *
                                   c.tile_m * c.tile_n * 4.0
                             : 0.0;
    };
    size_t best = 0;
    for (size_t i = 1; i < out.size() && out[i].est_us <= out[0].est_us * 1.01; i++) {
        const double pi = part_bytes(out[i].cfg), pb = part_bytes(out[best].cfg);
        if (pi < pb || (pi == pb && out[i].cfg.tile_m * out[i].cfg.tile_n < out[best].cfg.tile_m * out[best].cfg.tile_n))
            best = i;
    }
    std::rotate(out.begin(), out.begin() + best, out.begin() + best + 1);
    return out;
}

// ----------------------------------------------------------------- tile_ir --
std::string tile_name(const t0_tile_gemm& s) {
    // format of TileGemm::name (src/t0/tile_ir.rs:697-728)
    std::string r = "tile_gemm_" + std::to_string(s.tile_m) + "x" + std::to_string(s.tile_n) + "_k" +
                    std::to_string(s.tile_k);
    if (s.double_buffer) r += "_db";
    if (s.split_k > 1) r += "_sk" + std::to_string(s.split_k);
    if (!s.swap_grid) r += "_mg";
    if (s.wgp_mode) r += "_wgp";
    if (s.transpose == T0_NN) r += "_nn";
    if (s.acc_swap) r += "_swap";
    if (s.persistent) r += "_persistent";
    static const char* names[] = {"", "bias", "scale", "relu", "silu", "gelu", "abs", "neg", "clamp"};
    if (s.n_epilogue) {
        r += "_";
        for (uint32_t i = 0; i < s.n_epilogue && i < 8; i++) {
            if (i) r += "_";
            r += s.epilogue[i] <= 8 ? names[s.epilogue[i]] : "?";
        }
    }
    if (s.out_dtype == T0_OUT_BF16) r += "_bf16";
    return r;
}

const GemmInstance* tile_instance(const t0_tile_gemm& s) {
    return find_instance(s.tile_m, s.tile_n, s.tile_k, s.waves_per_wg);
}

uint32_t tile_epi_ops(const t0_tile_gemm& s) {
    uint32_t ops = 0;
    for (uint32_t i = 0; i < s.n_epilogue && i < T0_MAX_EPI_OPS; i++) ops |= (uint32_t)(s.epilogue[i] & 0xF) << (4 * i);
    return ops;
}

TileArgLayout tile_arg_layout(const t0_tile_gemm& s) {
    // argument order of lower_gemm (src/t0/tile_ir.rs:993-1026): X WT Y K N
    // split_k_shift y_split_stride M [counter n_tiles_n_shift tiles_per_wg]
    // [bias] [scale] [clamp_min clamp_max]
    TileArgLayout L;
    uint32_t off = 44;
    if (s.persistent) off = 64;   // counter@48 shift@56 tiles_per_wg@60 (src/t0/tile_ir.rs:4604-4639)
    for (uint32_t i = 0; i < s.n_epilogue && i < 8; i++) {
        if (s.epilogue[i] == T0_TEPI_BIAS) L.has_bias = true;
        if (s.epilogue[i] == T0_TEPI_SCALE) L.has_scale = true;
        if (s.epilogue[i] == T0_TEPI_CLAMP) L.has_clamp = true;
    }
    if (L.has_bias) { off = (off + 7) & ~7u; L.bias_off = off; off += 8; }
    if (L.has_scale) { L.scale_off = off; off += 4; }
    if (L.has_clamp) { L.clamp_off = off; off += 8; }
    L.size = off;
    return L;
}

}  // namespace t0h

using namespace t0h;

// =============================================================== C ABI ==
extern "C" {

const char* t0_last_error(void) { return t0h::last_error(); }
const char* t0_version(void) { return "t0-gemm-mi355x 0.1.0 (gfx950)"; }

int t0_config_preset(int id, t0_gemm_config* out) {
    if (!out) return fail(T0_ERR_INVALID, "null output");
    if (!preset(id, out)) return fail(T0_ERR_INVALID, "unknown preset %d", id);
    return T0_OK;
}

int t0_config_geometry(const t0_gemm_config* c, t0_gemm_geometry* o) {
    if (!c || !o) return fail(T0_ERR_INVALID, "null argument");
    const GemmInstance* g = instance_for(*c);
    memset(o, 0, sizeof *o);
    o->n_waves = c->wg_size / 64;
    o->k_sub_steps = c->tile_k / 16;
    o->lds_per_buffer = (c->tile_m + c->tile_n) * c->tile_k * 2;
    o->x_bytes_per_thread = c->wg_size ? c->tile_m * c->tile_k * 2 / c->wg_size : 0;
    o->wt_bytes_per_thread = c->wg_size ? c->tile_n * c->tile_k * 2 / c->wg_size : 0;
    if (!g) {
        o->lds_total = o->lds_per_buffer * 2;
        return fail(T0_ERR_INFEASIBLE, "%s: no gfx950 kernel", config_name(*c).c_str());
    }
    o->waves_m = g->wm;
    o->waves_n = g->wn;
    o->rows_per_wave = g->bm / g->wm;
    o->cols_per_wave = g->bn / g->wn;
    o->n_row_blocks = o->rows_per_wave / 32;
    o->n_col_tiles = o->cols_per_wave / 32;
    o->stages = g->stages;
    o->lds_total = g->lds_bytes();
    o->mfma_per_k_tile = o->n_row_blocks * o->n_col_tiles * o->k_sub_steps;
    o->estimated_vgprs = est_vgprs(*g);
    return T0_OK;
}

int t0_config_is_feasible(const t0_gemm_config* c) { return c && config_valid(*c, nullptr) ? 1 : 0; }

int t0_config_name(const t0_gemm_config* c, char* buf, size_t len) {
    if (!c) return fail(T0_ERR_INVALID, "null config");
    const std::string s = config_name(*c);
    if (buf && len) snprintf(buf, len, "%s", s.c_str());
    return (int)s.size();
}

int t0_config_from_name(const char* name, t0_gemm_config* out) {
    if (!name || !out) return fail(T0_ERR_INVALID, "null argument");
    unsigned tm, tn, tk;
    int used = 0;
    if (sscanf(name, "t0_gemm_%ux%u_k%u%n", &tm, &tn, &tk, &used) != 3) return fail(T0_ERR_INVALID, "not a t0_gemm name: %s", name);
    t0_gemm_config c = mk(tm, tn, tk, 0, true, true, 1, false);
    c.swap_grid = 1;
    std::string rest = name + used;
    auto eat = [&](const char* tag) {
        size_t L = strlen(tag);
        if (rest.compare(0, L, tag) == 0 && (rest.size() == L || rest[L] == '_')) { rest.erase(0, L); return true; }
        return false;
    };
    if (eat("_ldsdb")) { c.use_lds = 1; c.double_buffer = 1; }
    else if (eat("_lds")) { c.use_lds = 1; c.double_buffer = 0; }
    else if (eat("_direct")) { c.use_lds = 0; c.double_buffer = 0; }
    unsigned v;
    int u2 = 0;
    if (sscanf(rest.c_str(), "_sk%u%n", &v, &u2) == 1) { c.split_k = v; rest.erase(0, u2); }
    if (sscanf(rest.c_str(), "_%up%n", &v, &u2) == 1 && rest.c_str()[u2 - 1] == 'p') { c.n_col_passes = v; rest.erase(0, u2); }
    if (eat("_mg")) c.swap_grid = 0;
    if (eat("_wgp")) c.wgp_mode = 1;
    if (eat("_nn")) c.transpose = T0_NN;
    if (eat("_bias_relu")) c.epilogue = T0_EPI_BIAS_ADD_RELU;
    else if (eat("_bias")) c.epilogue = T0_EPI_BIAS_ADD;
    if (eat("_bf16")) c.out_dtype = T0_OUT_BF16;
    if (!rest.empty()) return fail(T0_ERR_INVALID, "unparsed suffix '%s' in %s", rest.c_str(), name);
    // wg_size: the one gfx950 instance with this tile (reference presets keep their wg)
    const GemmInstance* g = find_instance(tm, tn, tk, 0);
    c.wg_size = g ? g->threads() : 64;
    for (int p = 0; p < T0_PRESET_COUNT; p++) {
        t0_gemm_config q;
        preset(p, &q);
        if (q.tile_m == tm && q.tile_n == tn && q.tile_k == tk && instance_for(q)) { c.wg_size = q.wg_size; break; }
    }
    *out = c;
    return T0_OK;
}

static int fill_list(const std::vector<t0_gemm_config>& v, t0_gemm_config* out, size_t cap) {
    for (size_t i = 0; i < v.size() && i < cap && out; i++) out[i] = v[i];
    return (int)v.size();
}

int t0_sweep_configs(t0_gemm_config* out, size_t cap) {
    // src/t0/gemm_gen.rs:239-250 plus the gfx950-native tiles
    std::vector<t0_gemm_config> v;
    const int ids[] = {T0_PRESET_16x64_K16, T0_PRESET_32x64_K16, T0_PRESET_32x64_K32, T0_PRESET_32x128_K16,
                       T0_PRESET_64x64_K16, T0_PRESET_64x64_K32, T0_PRESET_128x64_K16, T0_PRESET_64x128_K16,
                       T0_PRESET_128x64_K32, T0_PRESET_256x256_K64, T0_PRESET_256x128_K64, T0_PRESET_128x256_K64,
                       T0_PRESET_128x128_K64, T0_PRESET_128x128_K32, T0_PRESET_128x64_K64, T0_PRESET_64x128_K64,
                       T0_PRESET_32x64_K64, T0_PRESET_32x128_K64, T0_PRESET_256x256_K32};
    for (int id : ids) { t0_gemm_config c; preset(id, &c); v.push_back(c); }
    return fill_list(v, out, cap);
}

int t0_standard_configs(t0_gemm_config* out, size_t cap) {
    // src/t0/gemm_gen.rs:407-427
    std::vector<t0_gemm_config> v;
    const int ids[] = {T0_PRESET_16x64_K16, T0_PRESET_32x64_K16, T0_PRESET_32x64_K32, T0_PRESET_32x128_K16,
                       T0_PRESET_64x64_K16, T0_PRESET_64x64_K32, T0_PRESET_128x64_K16, T0_PRESET_128x64_K32};
    for (int id : ids) { t0_gemm_config c; preset(id, &c); v.push_back(c); }
    const struct { int id; uint32_t sk; } sks[] = {
        {T0_PRESET_32x64_K32, 2}, {T0_PRESET_16x64_K16, 4}, {T0_PRESET_64x64_K32, 2}, {T0_PRESET_64x64_K16, 4},
        {T0_PRESET_64x64_K32, 4}, {T0_PRESET_64x64_K16, 8}, {T0_PRESET_128x64_K16, 2}, {T0_PRESET_128x64_K32, 2}};
    for (auto s : sks) { t0_gemm_config c; preset(s.id, &c); c.split_k = s.sk; v.push_back(c); }
    return fill_list(v, out, cap);
}

int t0_compute_grid(const t0_gemm_config* c, uint32_t m, uint32_t n, uint32_t* gx, uint32_t* gy) {
    // src/t0/gemm_gen.rs:308-316
    if (!c || !gx || !gy || !c->tile_m || !c->tile_n) return fail(T0_ERR_INVALID, "bad arguments");
    const uint32_t tm = (m + c->tile_m - 1) / c->tile_m, tn = (n + c->tile_n - 1) / c->tile_n;
    if (c->swap_grid) { *gx = tn * c->wg_size; *gy = tm; }
    else { *gx = tm * c->wg_size; *gy = tn; }
    return T0_OK;
}

int t0_compute_grid_split_k(const t0_gemm_config* c, uint32_t m, uint32_t n, uint32_t sk, uint32_t* gx, uint32_t* gy) {
    // src/t0/gemm_gen.rs:319-329 (asserts power of two)
    if (sk == 0 || (sk & (sk - 1))) return fail(T0_ERR_INVALID, "split_k=%u must be power of 2", sk);
    int r = t0_compute_grid(c, m, n, gx, gy);
    if (r) return r;
    *gy *= sk;
    return T0_OK;
}

int t0_compute_grid_auto(const t0_gemm_config* c, uint32_t m, uint32_t n, uint32_t* gx, uint32_t* gy) {
    // src/t0/gemm_gen.rs:430-437
    if (!c) return fail(T0_ERR_INVALID, "null config");
    const uint32_t sk = split_of(*c);
    return sk > 1 ? t0_compute_grid_split_k(c, m, n, sk, gx, gy) : t0_compute_grid(c, m, n, gx, gy);
}

static void put64(uint8_t* p, uint64_t v) { memcpy(p, &v, 8); }
static void put32(uint8_t* p, uint32_t v) { memcpy(p, &v, 4); }

int t0_build_kernargs(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                      const t0_gemm_config* c, uint8_t out[40]) {
    // src/t0/gemm_gen.rs:442-458
    if (!c || !out) return fail(T0_ERR_INVALID, "null argument");
    const uint32_t sk = split_of(*c);
    put64(out, x); put64(out + 8, wt); put64(out + 16, y);
    put32(out + 24, k); put32(out + 28, n); put32(out + 32, 0);
    put32(out + 36, sk > 1 ? m * n * 4 : 0);
    return T0_OK;
}

int t0_build_kernargs_with_bias(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                                const t0_gemm_config* c, uint64_t bias, uint8_t out[48]) {
    // src/t0/gemm_gen.rs:466-484
    int r = t0_build_kernargs(x, wt, y, k, n, m, c, out);
    if (r) return r;
    put64(out + 40, bias);
    return T0_OK;
}

int t0_auto_select(uint32_t m, uint32_t k, uint32_t n, t0_gemm_config* out) {
    if (!out || !m || !n || !k) return fail(T0_ERR_INVALID, "bad arguments");
    auto c = rank_candidates(m, n, k, T0_NT, T0_OUT_F32, false);
    if (c.empty()) return t0_auto_select_legacy(m, k, n, out);
    *out = c.front().cfg;
    return T0_OK;
}

int t0_auto_schedule_gemm(uint32_t m, uint32_t n, uint32_t k, uint32_t transpose, uint32_t out_dtype,
                          t0_gemm_config* out, double* est_us, uint32_t cap) {
    if (!m || !n || !k || transpose > T0_NN || out_dtype > T0_OUT_BF16) return fail(T0_ERR_INVALID, "bad arguments");
    if (cap && !out) return fail(T0_ERR_INVALID, "null output");
    const auto c = rank_candidates(m, n, k, transpose, out_dtype, true);
    for (uint32_t i = 0; i < cap && i < c.size(); i++) {
        out[i] = c[i].cfg;
        if (est_us) est_us[i] = c[i].est_us;
    }
    return (int)c.size();
}

int t0_auto_select_legacy(uint32_t m, uint32_t k, uint32_t n, t0_gemm_config* out) {
    // decision tree of auto_select_legacy (src/t0/gemm_gen.rs:351-404)
    if (!out) return fail(T0_ERR_INVALID, "null output");
    const uint64_t mn = (uint64_t)m * n;
    auto clamp_sk = [&](uint32_t tk, uint32_t desired) -> uint32_t {
        uint32_t max_sk = k / tk, sk = std::min(desired, max_sk);
        while (sk > 1 && k % (tk * sk) != 0) sk /= 2;
        return sk > 1 ? sk : 0;
    };
    const bool use_128m = m % 128 == 0 && m >= 128, use_64m = m % 64 == 0;
    t0_gemm_config c;
    if (m <= 256 && k >= 512 && n >= 1024 && use_128m) {
        preset(T0_PRESET_128x64_K16, &c); c.swap_grid = 0; c.wgp_mode = 1; c.split_k = clamp_sk(16, 4);
    } else if (m <= 512 && k >= 512 && n >= 1024 && use_128m) {
        preset(T0_PRESET_128x64_K16, &c); c.swap_grid = 0; c.wgp_mode = 1; c.split_k = clamp_sk(16, 8);
    } else if (mn <= 512ull * 512) {
        preset(T0_PRESET_64x64_K16, &c); c.swap_grid = 0; c.split_k = clamp_sk(16, 8);
    } else if (mn <= 1024ull * 1024 && use_128m) {
        preset(T0_PRESET_128x64_K16, &c); c.swap_grid = 0; c.wgp_mode = 1; c.split_k = clamp_sk(16, 2);
    } else if (use_128m && mn >= 2048ull * 2048) {
        preset(T0_PRESET_128x64_K32, &c); c.wgp_mode = 1; c.split_k = clamp_sk(32, 2);
    } else if (use_128m) {
        preset(T0_PRESET_128x64_K16, &c); c.wgp_mode = 1; c.split_k = clamp_sk(16, 8);
    } else if (use_64m) {
        preset(T0_PRESET_64x64_K16, &c); c.wgp_mode = 1; c.split_k = clamp_sk(16, 4);
    } else {
        preset(T0_PRESET_32x64_K16, &c); c.split_k = clamp_sk(16, 4);
    }
    *out = c;
    return T0_OK;
}

int t0_cached_auto_select(uint32_t m, uint32_t k, uint32_t n, t0_gemm_config* out) {
    // src/t0/prefill_spec_cache.rs:55-76: process-global memo
    static std::mutex mu;
    static std::map<uint64_t, t0_gemm_config> memo;
    if (!out) return fail(T0_ERR_INVALID, "null output");
    const uint64_t key = ((uint64_t)m << 42) ^ ((uint64_t)k << 21) ^ n;
    {
        std::lock_guard<std::mutex> g(mu);
        auto it = memo.find(key);
        if (it != memo.end()) { *out = it->second; return T0_OK; }
    }
    int r = t0_auto_select(m, k, n, out);
    if (r) return r;
    std::lock_guard<std::mutex> g(mu);
    memo[key] = *out;
    return T0_OK;
}

int t0_prewarm_cache(const uint32_t* mkn, size_t count) {
    if (!mkn && count) return fail(T0_ERR_INVALID, "null shapes");
    for (size_t i = 0; i < count; i++) {
        t0_gemm_config c;
        int r = t0_cached_auto_select(mkn[3 * i], mkn[3 * i + 1], mkn[3 * i + 2], &c);
        if (r) return r;
    }
    return T0_OK;
}

int t0_auto_select_backward_data(uint32_t m, uint32_t n_orig, uint32_t k_orig, t0_gemm_config* out) {
    return t0_auto_select(m, n_orig, k_orig, out);          // src/t0/gemm_gen.rs:510-514
}
int t0_auto_select_backward_weight(uint32_t m, uint32_t n_orig, uint32_t k_orig, t0_gemm_config* out) {
    return t0_auto_select(n_orig, m, k_orig, out);          // src/t0/gemm_gen.rs:545-549
}
int t0_build_kernargs_backward_data(uint64_t dy, uint64_t w, uint64_t dx, uint32_t m, uint32_t n_orig,
                                    uint32_t k_orig, const t0_gemm_config* c, uint8_t out[40]) {
    return t0_build_kernargs(dy, w, dx, n_orig, k_orig, m, c, out);    // src/t0/gemm_gen.rs:523-531
}
int t0_build_kernargs_backward_weight(uint64_t dy_t, uint64_t x_t, uint64_t dw, uint32_t m, uint32_t n_orig,
                                      uint32_t k_orig, const t0_gemm_config* c, uint8_t out[40]) {
    return t0_build_kernargs(dy_t, x_t, dw, m, k_orig, n_orig, c, out);  // src/t0/gemm_gen.rs:557-565
}

int t0_tile_name(const t0_tile_gemm* s, char* buf, size_t len) {
    if (!s) return fail(T0_ERR_INVALID, "null spec");
    const std::string n = tile_name(*s);
    if (buf && len) snprintf(buf, len, "%s", n.c_str());
    return (int)n.size();
}

int t0_tile_auto_select(uint32_t m, uint32_t k, uint32_t n, int transpose, t0_tile_gemm* out) {
    // tile_auto_select (src/t0/tile_ir.rs:740-870) keeps split_k = 1 (auto
    // split-K disabled there, :859); the gfx950 model picks the tile.
    if (!out) return fail(T0_ERR_INVALID, "null output");
    auto c = rank_candidates(m, n, k, (uint32_t)transpose, T0_OUT_F32, false);
    memset(out, 0, sizeof *out);
    for (const auto& cand : c) {
        if (split_of(cand.cfg) != 1) continue;
        const GemmInstance* g = instance_for(cand.cfg);
        out->tile_m = g->bm; out->tile_n = g->bn; out->tile_k = g->bk;
        out->split_k = 1; out->waves_per_wg = g->nw();
        out->double_buffer = 1; out->swap_grid = 1; out->transpose = (uint8_t)transpose;
        return T0_OK;
    }
    return fail(T0_ERR_INFEASIBLE, "no tile for %ux%ux%u", m, n, k);
}

int t0_tile_build_kernargs_m(uint64_t x, uint64_t wt, uint64_t y, uint32_t k, uint32_t n, uint32_t m,
                             const t0_tile_gemm* s, uint32_t y_split_stride, uint64_t bias, float scale,
                             float cmin, float cmax, uint8_t* out, size_t* len) {
    if (!s || !out || !len) return fail(T0_ERR_INVALID, "null argument");
    uint32_t shift = 0;
    switch (s->split_k) {   // src/t0/tile_ir.rs:4614
    case 0: case 1: shift = 0; break;
    case 2: shift = 1; break;
    case 4: shift = 2; break;
    case 8: shift = 3; break;
    case 16: shift = 4; break;
    default: shift = 0;
    }
    const TileArgLayout L = tile_arg_layout(*s);
    memset(out, 0, L.size);
    put64(out, x); put64(out + 8, wt); put64(out + 16, y);
    put32(out + 24, k); put32(out + 28, n); put32(out + 32, shift); put32(out + 36, y_split_stride);
    put32(out + 40, m);
    if (L.has_bias) put64(out + L.bias_off, bias);
    if (L.has_scale) memcpy(out + L.scale_off, &scale, 4);
    if (L.has_clamp) { memcpy(out + L.clamp_off, &cmin, 4); memcpy(out + L.clamp_off + 4, &cmax, 4); }
    *len = L.size;
    return T0_OK;
}

int t0_tile_compute_grid(const t0_tile_gemm* s, uint32_t m, uint32_t n, uint32_t grid[3]) {
    // src/t0/tile_ir.rs:4645-4667
    if (!s || !grid || !s->tile_m || !s->tile_n) return fail(T0_ERR_INVALID, "bad arguments");
    const GemmInstance* g = tile_instance(*s);
    const uint32_t wg = g ? g->threads() : (s->waves_per_wg ? s->waves_per_wg : s->tile_m / 32) * 64;
    const uint32_t sk = s->split_k > 1 ? s->split_k : 1;
    const uint32_t wn = (n + s->tile_n - 1) / s->tile_n, wm = (m + s->tile_m - 1) / s->tile_m;
    if (s->swap_grid) { grid[0] = wn * wg; grid[1] = wm * sk; }
    else { grid[0] = wm * wg; grid[1] = wn * sk; }
    grid[2] = 1;
    return T0_OK;
}

}  // extern "C"

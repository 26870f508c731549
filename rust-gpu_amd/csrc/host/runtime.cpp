// runtime.cpp -- HIP runtime side of libt0gpu: device/stream, code-object
// loading, kernarg decoding and dispatch, buffers, events, the high-level GEMM
// and W4A16 entry points and the measured tuner.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <mutex>
#include <set>
#include <sstream>
#include <string>
#include <sys/stat.h>
#include <vector>

#include "internal.hpp"

using namespace t0h;

// The gfx950 code object with every kernel of the library (embed.S).
extern "C" const unsigned char t0_hsaco_start[];
extern "C" const unsigned char t0_hsaco_end[];

enum KernelKind { KK_RAW = 0, KK_GEMM_GEN = 1, KK_TILE = 2 };

struct t0_kernel {
    KernelKind kind = KK_RAW;
    hipFunction_t fn = nullptr;
    hipModule_t own_module = nullptr;   // RAW kernels loaded from a caller's code object
    uint32_t wg[3] = {64, 1, 1};
    uint32_t lds = 0;
    uint32_t kernarg_size = 0;
    std::string name;
    const GemmInstance* inst = nullptr;
    t0_gemm_config cfg{};
    t0_tile_gemm tile{};
    TileArgLayout layout;
};

struct t0_buffer {
    struct t0_runtime* rt = nullptr;
    void* ptr = nullptr;
    size_t size = 0, alloc_size = 0;
};

struct t0_event {
    hipEvent_t ev = nullptr;
};

struct t0_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    t0_runtime* rt = nullptr;   // cleared when the runtime goes first
};

struct t0_runtime {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    hipModule_t module = nullptr;
    std::mutex mu;
    std::map<std::string, t0_kernel*> cache;
    std::map<std::string, hipFunction_t> fns;
    std::mutex fn_mu;               // guards fns
    std::atomic<bool> poisoned{false};
    std::map<size_t, std::vector<t0_buffer*>> pool;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    void* stage = nullptr;          // bf16 operand staging of the matmul path
    size_t stage_bytes = 0;
    uint32_t* sem = nullptr;
    size_t sem_count = 0;
    void* probe = nullptr;          // t0_gemm_clock_probe timestamps
    // Graphs instantiated from this runtime's stream (their kernel arguments
    // hold ws / stage / sem, so those buffers must not move while any exists).
    std::set<struct t0_graph*> graphs;
    // Held for the host side of every call that uses ws / stage / sem, so
    // that threads sharing the runtime never resize a buffer another call
    // has just put into its kernel arguments (recursive: calls nest).
    std::recursive_mutex call_mu;
    std::atomic<uint32_t> slot{0};  // t0_dispatch_async's completion slots
    std::string arch;
    int cu_count = 0, clock_khz = 0;
};

#define HIPCHK(expr)                                                                          \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess) return fail(T0_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

namespace {

int set_dev(t0_runtime* rt) {
    HIPCHK(hipSetDevice(rt->device));
    return T0_OK;
}

int get_fn(t0_runtime* rt, const std::string& sym, hipFunction_t* out) {
    std::lock_guard<std::mutex> g(rt->fn_mu);
    auto it = rt->fns.find(sym);
    if (it != rt->fns.end()) { *out = it->second; return T0_OK; }
    hipFunction_t f;
    hipError_t e = hipModuleGetFunction(&f, rt->module, sym.c_str());
    if (e != hipSuccess) return fail(T0_ERR_NOT_FOUND, "kernel %s not in code object: %s", sym.c_str(), hipGetErrorString(e));
    rt->fns[sym] = f;
    *out = f;
    return T0_OK;
}

template <class P>
int launch(t0_runtime* rt, hipFunction_t f, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t threads, const P& p) {
    if (rt->poisoned.load()) return fail(T0_ERR_POISONED, "runtime poisoned after an earlier GPU failure; refusing dispatch");
    if (gx == 0 || gy == 0 || gz == 0) return T0_OK;
    P copy = p;
    void* args[] = {&copy};
    HIPCHK(hipModuleLaunchKernel(f, gx, gy, gz, threads, 1, 1, 0, rt->stream, args, nullptr));
    return T0_OK;
}

// A shared buffer may grow only outside graph capture (growing syncs the
// stream, and the semaphores are cleared by a memset) and, once it exists,
// only while no captured graph holds its address.
int may_grow(t0_runtime* rt, const void* cur, const char* what) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(rt->stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone)
        return fail(T0_ERR_INVALID, "the %s would grow during graph capture: run the same call once before capturing",
                    what);
    if (cur && !rt->graphs.empty())
        return fail(T0_ERR_INVALID, "the %s would grow while %zu captured graph(s) hold its address: destroy them "
                    "first, or run the largest call once before capturing", what, rt->graphs.size());
    return T0_OK;
}

int ensure_ws(t0_runtime* rt, size_t bytes) {
    if (bytes <= rt->ws_bytes) return T0_OK;
    int r = may_grow(rt, rt->ws, "split-K workspace");
    if (r) return r;
    if (rt->ws) { HIPCHK(hipStreamSynchronize(rt->stream)); HIPCHK(hipFree(rt->ws)); rt->ws = nullptr; rt->ws_bytes = 0; }
    size_t want = std::max<size_t>(bytes + 4096, 64u << 20);
    HIPCHK(hipMalloc(&rt->ws, want));
    rt->ws_bytes = want;
    return T0_OK;
}

int ensure_stage(t0_runtime* rt, size_t bytes) {
    if (bytes <= rt->stage_bytes) return T0_OK;
    int r = may_grow(rt, rt->stage, "operand staging buffer");
    if (r) return r;
    if (rt->stage) { HIPCHK(hipStreamSynchronize(rt->stream)); HIPCHK(hipFree(rt->stage)); rt->stage = nullptr; rt->stage_bytes = 0; }
    size_t want = std::max<size_t>(bytes + 4096, 16u << 20);
    HIPCHK(hipMalloc(&rt->stage, want));
    rt->stage_bytes = want;
    return T0_OK;
}

int ensure_sem(t0_runtime* rt, size_t count) {
    if (count <= rt->sem_count) return T0_OK;
    int r = may_grow(rt, rt->sem, "split-K semaphore array");
    if (r) return r;
    if (rt->sem) { HIPCHK(hipStreamSynchronize(rt->stream)); HIPCHK(hipFree(rt->sem)); rt->sem = nullptr; rt->sem_count = 0; }
    size_t want = std::max<size_t>(count, 65536);
    HIPCHK(hipMalloc(&rt->sem, want * 4));
    HIPCHK(hipMemsetAsync(rt->sem, 0, want * 4, rt->stream));
    HIPCHK(hipStreamSynchronize(rt->stream));
    rt->sem_count = want;
    return T0_OK;
}

bool aligned16(uint64_t p) { return (p & 15) == 0; }
bool aligned8(uint64_t p) { return (p & 7) == 0; }

// Fast tiled kernels need 16-byte operand rows; anything else takes the
// generic kernel.  NN reads B in 8-column chunks: with N % 8 != 0 the last
// chunk of a row runs past column N, which stays inside the row only when the
// caller guarantees ldb >= round_up(N, 8) allocated columns (b_cols_padded).
bool fast_ok(const t0_gemm_params& p, bool nn, bool b_cols_padded = false) {
    if (!aligned16((uint64_t)p.A) || !aligned16((uint64_t)p.B) || !aligned16((uint64_t)p.C)) return false;
    if (p.lda % 8 || p.ldb % 8) return false;
    if (p.K % (8 * p.split_k)) return false;
    if (nn && p.N % 8 && !(b_cols_padded && p.ldb >= (p.N + 7) / 8 * 8)) return false;
    return true;
}

// Caller-provided split-K scratch (no allocation): counters then partials.
struct Scratch {
    void* base = nullptr;
    size_t bytes = 0;
};

// The register-staged K loop (t0k_gemm_*_vg2_*) where it measured faster
// than the DMA loop (graph replays, B cold, the pick on each shape): the
// 64x128 four-wave tile (128x4096x4096 0.97x) and the 128x64 one with no
// fully masked rows (M 128-512: 0.93-1.00x; at M = 32 it lost 7 %).  The
// 128x128, 64x64 and 32-row tiles lost 2-13 % and keep the DMA loop.
bool use_vg_variant(const GemmInstance& g, const t0_gemm_params& p) {
    if (g.bk != 64 || g.wm != 2 || g.wn != 2 || g.stages != 4) return false;
    if (g.bm == 64 && g.bn == 128) return true;
    return g.bm == 128 && g.bn == 64 && p.M >= 128;
}

int run_gemm_params(t0_runtime* rt, const GemmInstance* g, bool nn, t0_gemm_params& p, uint32_t threads_override = 0,
                    bool b_cols_padded = false, const Scratch* sc = nullptr) {
    hipFunction_t f;
    if (!g || !fast_ok(p, nn, b_cols_padded)) {
        if (p.flags & T0_GEMM_FIXUP) {   // generic kernel writes planes; reduce separately
            return fail(T0_ERR_INVALID, "in-kernel split-K needs the tiled path (16-byte aligned rows)");
        }
        int r = get_fn(rt, nn ? "t0k_gemm_generic_nn" : "t0k_gemm_generic_nt", &f);
        if (r) return r;
        const uint32_t tiles = ((p.M + 63) / 64) * ((p.N + 63) / 64) * p.split_k;
        return launch(rt, f, tiles, 1, 1, 256, p);
    }
    std::string sym = g->symbol(nn);
    // the register-staged variant when every split-K partition is a whole
    // number of pairs of 64-k steps (bit-identical)
    if (use_vg_variant(*g, p) && p.split_k && p.K % (128u * p.split_k) == 0)
        sym.insert(sym.size() - 3, "_vg2");
    int r = get_fn(rt, sym, &f);
    if (r) return r;
    const uint32_t tiles = ((p.M + g->bm - 1) / g->bm) * ((p.N + g->bn - 1) / g->bn);
    if ((p.flags & T0_GEMM_FIXUP) && sc) {
        const size_t partials = (size_t)p.split_k * tiles * g->bm * g->bn * 4;
        if (tiles > T0_NOALLOC_MAX_TILES || partials > sc->bytes - T0_NOALLOC_MAX_TILES * 4)
            return fail(T0_ERR_INVALID, "split-K scratch: %u tiles (at most %u) and %zu bytes of partial tiles "
                        "(at most %zu) for %ux%ux%u split %u", tiles, (unsigned)T0_NOALLOC_MAX_TILES, partials,
                        sc->bytes - T0_NOALLOC_MAX_TILES * 4, p.M, p.N, p.K, p.split_k);
        hipFunction_t fill;
        r = get_fn(rt, "t0k_fill_u32", &fill);
        if (r) return r;
        t0_aux_params z;
        memset(&z, 0, sizeof z);
        z.dst = sc->base;
        z.m = tiles;
        r = launch(rt, fill, (tiles + 255) / 256, 1, 1, 256, z);   // counters start at zero
        if (r) return r;
        p.semaphores = (uint32_t*)sc->base;
        p.workspace = (float*)((uint8_t*)sc->base + T0_NOALLOC_MAX_TILES * 4);
    } else if (p.flags & T0_GEMM_FIXUP) {
        r = ensure_ws(rt, (size_t)p.split_k * tiles * g->bm * g->bn * 4);
        if (r) return r;
        r = ensure_sem(rt, tiles);
        if (r) return r;
        p.workspace = (float*)rt->ws;
        p.semaphores = rt->sem;
    }
    // grid x = tiles, y = split (the kernel linearises and remaps to XCDs)
    return launch(rt, f, tiles, p.split_k, 1, threads_override ? threads_override : g->threads(), p);
}

uint32_t epi_ops_from_gemm_gen(uint8_t epi) {
    if (epi == T0_EPI_BIAS_ADD) return T0_EPI_BIAS;
    if (epi == T0_EPI_BIAS_ADD_RELU) return T0_EPI_BIAS | (T0_EPI_RELU << 4);
    return 0;
}

uint64_t rd64(const uint8_t* p) { uint64_t v; memcpy(&v, p, 8); return v; }
uint32_t rd32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }
float rdf(const uint8_t* p) { float v; memcpy(&v, p, 4); return v; }

// ---------------------------------------------------------------- tuner --
using TuneList = std::vector<std::pair<t0_gemm_config, double>>;   // (config, TFLOP/s), fastest first
struct TunerState {
    std::mutex mu;
    std::map<std::string, std::pair<t0_gemm_config, double>> mem;
    std::map<std::string, TuneList> all;   // every timed candidate of the tunes run in this process
    std::string dir;
    uint32_t max_candidates = 8, n_iters = 10;
};
TunerState& tuner() {
    static TunerState s;
    return s;
}

std::string cache_dir() {
    auto& T = tuner();
    if (!T.dir.empty()) return T.dir;
    if (const char* e = getenv("T0_AUTOTUNE_DIR")) return e;
    // not the reference's ~/.t0_autotune (src/t0/auto_gemm.rs:594-600): its
    // loader ignores "arch" and would take gfx950-only configs written here;
    // point the tuner there (t0_tuner_set_cache_dir, T0_AUTOTUNE_DIR) to read
    // the reference's files
    const char* home = getenv("HOME");
    return std::string(home ? home : "/tmp") + "/.t0_autotune_gfx950";
}

std::string tune_key_arch(const char* arch, uint32_t m, uint32_t n, uint32_t k, uint32_t tr, uint32_t od) {
    char b[160];
    snprintf(b, sizeof b, "%s_%ux%ux%u_%s_%s", arch, m, n, k, tr == T0_NN ? "nn" : "nt",
             od == T0_OUT_BF16 ? "bf16" : "f32");
    return b;
}
std::string tune_key(const t0_runtime* rt, uint32_t m, uint32_t n, uint32_t k, uint32_t tr, uint32_t od) {
    return tune_key_arch(rt->arch.c_str(), m, n, k, tr, od);
}

// Tuned configs on disk, one JSON file per problem in the reference's layout
// (src/t0/auto_gemm.rs:435-501): tile_m, tile_n, tile_k, wg_size, split_k,
// lds_pad, n_col_passes, wgp, swap, tflops, all.  NT with f32 output (the
// reference's only form) keeps its file name gemm_MxNxK.json, so reference
// cache files load; NN or bf16 output add a _nn / _nt and _bf16 / _f32
// suffix.  Files written here also name the architecture ("arch") and the
// layout; a file for another architecture is ignored.
std::string cache_file(uint32_t m, uint32_t n, uint32_t k, uint32_t tr, uint32_t od) {
    std::string f = "gemm_" + std::to_string(m) + "x" + std::to_string(n) + "x" + std::to_string(k);
    if (tr != T0_NT || od != T0_OUT_F32)
        f += std::string(tr == T0_NN ? "_nn" : "_nt") + (od == T0_OUT_BF16 ? "_bf16" : "_f32");
    return cache_dir() + "/" + f + ".json";
}

// n values ~ N(0,1) rounded to bf16 (RNE): xorshift64* uniforms, Box-Muller
void fill_normal_bf16(uint16_t* out, size_t n, uint64_t seed) {
    uint64_t x = seed ? seed : 1;
    auto uni = [&]() {   // (0, 1]
        x ^= x >> 12; x ^= x << 25; x ^= x >> 27;
        return ((x * 0x2545F4914F6CDD1Dull) >> 11) * (1.0 / 9007199254740992.0) + 1.0 / 18014398509481984.0;
    };
    auto rne = [](float f) {
        uint32_t u;
        memcpy(&u, &f, 4);
        return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
    };
    for (size_t i = 0; i < n; i += 2) {
        const double r = std::sqrt(-2.0 * std::log(uni())), t = 6.283185307179586 * uni();
        out[i] = rne((float)(r * std::cos(t)));
        if (i + 1 < n) out[i + 1] = rne((float)(r * std::sin(t)));
    }
}

// a config read back from disk is used only if a gfx950 kernel runs it
bool tuned_config_ok(const t0_gemm_config& c) {
    const uint32_t sk = split_of(c);
    return instance_for(c) != nullptr && sk <= 16 && (sk & (sk - 1)) == 0 && c.transpose <= T0_NN &&
           c.out_dtype <= T0_OUT_BF16;
}

// Flat JSON objects as the tuners write them: the text of one field's value
// (quotes dropped), or a number.
bool read_text(const std::string& path, std::string* s) {
    std::ifstream f(path);
    if (!f) return false;
    std::stringstream ss;
    ss << f.rdbuf();
    *s = ss.str();
    return true;
}
bool json_raw(const std::string& s, const char* name, std::string* out) {
    const std::string pat = std::string("\"") + name + "\":";
    size_t p = s.find(pat);
    if (p == std::string::npos) return false;
    p += pat.size();
    while (p < s.size() && (s[p] == ' ' || s[p] == '"')) p++;
    size_t e = p;
    while (e < s.size() && s[e] != '"' && s[e] != ',' && s[e] != '}') e++;
    *out = s.substr(p, e - p);
    return true;
}
bool json_num(const std::string& s, const char* name, double* v) {
    std::string t;
    if (!json_raw(s, name, &t) || t.empty()) return false;
    char* end = nullptr;
    *v = strtod(t.c_str(), &end);
    return end && *end == 0;
}

bool load_cache_file(uint32_t m, uint32_t n, uint32_t k, uint32_t tr, uint32_t od, const char* arch,
                     t0_gemm_config* cfg, double* tf) {
    std::string s;
    if (!read_text(cache_file(m, n, k, tr, od), &s)) return false;
    auto raw = [&](const char* name, std::string* out) { return json_raw(s, name, out); };
    auto num = [&](const char* name, double* v) { return json_num(s, name, v); };
    std::string a;
    if (raw("arch", &a) && a != arch) return false;
    double tm, tn, tk, wg, t;
    if (!num("tile_m", &tm) || !num("tile_n", &tn) || !num("tile_k", &tk) || !num("wg_size", &wg) || !num("tflops", &t))
        return false;
    double sk = 1, pad = 0, passes = 1;
    num("split_k", &sk);
    num("lds_pad", &pad);
    num("n_col_passes", &passes);
    t0_gemm_config c;
    memset(&c, 0, sizeof c);
    c.tile_m = (uint32_t)tm; c.tile_n = (uint32_t)tn; c.tile_k = (uint32_t)tk; c.wg_size = (uint32_t)wg;
    c.split_k = sk > 1 ? (uint32_t)sk : 0;
    c.lds_pad = (uint32_t)pad;
    c.n_col_passes = passes >= 1 ? (uint32_t)passes : 1;
    c.use_lds = 1; c.double_buffer = 1;
    c.wgp_mode = s.find("\"wgp\":true") != std::string::npos;
    c.swap_grid = s.find("\"swap\":true") != std::string::npos;
    c.transpose = (uint8_t)tr;
    c.out_dtype = (uint8_t)od;
    c.epilogue = T0_EPI_STORE_F32;
    if (!tuned_config_ok(c)) return false;
    *cfg = c;
    *tf = t;
    return true;
}

// "all" holds every timed candidate, fastest first, as the reference writes
// it (["name", tflops], src/t0/auto_gemm.rs:480-494) plus a third element,
// the workgroup size, which the name does not carry.
bool save_cache_file(uint32_t m, uint32_t n, uint32_t k, uint32_t tr, uint32_t od, const char* arch,
                     const t0_gemm_config& c, double tf, const TuneList& all) {
    const std::string d = cache_dir();
    mkdir(d.c_str(), 0755);
    std::ofstream f(cache_file(m, n, k, tr, od));
    if (!f) return false;
    char num[32];
    snprintf(num, sizeof num, "%.2f", tf);
    f << "{\"tile_m\":" << c.tile_m << ",\"tile_n\":" << c.tile_n << ",\"tile_k\":" << c.tile_k
      << ",\"wg_size\":" << c.wg_size << ",\"split_k\":" << split_of(c) << ",\"lds_pad\":" << c.lds_pad
      << ",\"n_col_passes\":" << (c.n_col_passes ? c.n_col_passes : 1) << ",\"wgp\":" << (c.wgp_mode ? "true" : "false")
      << ",\"swap\":" << (c.swap_grid ? "true" : "false") << ",\"tflops\":" << num << ",\"all\":[";
    for (size_t i = 0; i < all.size(); i++) {
        snprintf(num, sizeof num, "%.2f", all[i].second);
        f << (i ? "," : "") << "[\"" << config_name(all[i].first) << "\"," << num << "," << all[i].first.wg_size << "]";
    }
    f << "],\"arch\":\"" << arch << "\",\"transpose\":\"" << (tr == T0_NN ? "nn" : "nt") << "\",\"out_dtype\":\""
      << (od == T0_OUT_BF16 ? "bf16" : "f32") << "\",\"name\":\"" << config_name(c) << "\"}\n";
    return (bool)f;
}

// The "all" list of a cache file: entries ["name", tflops] or
// ["name", tflops, wg_size] whose name parses and runs on gfx950, in file
// order.  False if the file is missing or names another architecture.
bool load_cache_all(uint32_t m, uint32_t n, uint32_t k, uint32_t tr, uint32_t od, const char* arch, TuneList* out) {
    std::string s, a;
    if (!read_text(cache_file(m, n, k, tr, od), &s)) return false;
    if (json_raw(s, "arch", &a) && a != arch) return false;
    out->clear();
    size_t p = s.find("\"all\":[");
    if (p == std::string::npos) return true;
    p += 7;
    while (p < s.size()) {
        while (p < s.size() && (s[p] == ' ' || s[p] == ',')) p++;
        if (p >= s.size() || s[p] != '[') break;
        const size_t e = s.find(']', p);
        if (e == std::string::npos) break;
        const std::string item = s.substr(p + 1, e - p - 1);   // "name",tf[,wg]
        p = e + 1;
        const size_t q0 = item.find('"'), q1 = item.find('"', q0 + 1);
        if (q0 == std::string::npos || q1 == std::string::npos) continue;
        t0_gemm_config c;
        if (t0_config_from_name(item.substr(q0 + 1, q1 - q0 - 1).c_str(), &c) != T0_OK) continue;
        double tf = 0, wg = 0;
        if (sscanf(item.c_str() + q1 + 1, " ,%lf ,%lf", &tf, &wg) < 1) continue;
        if (wg > 0) c.wg_size = (uint32_t)wg;
        c.transpose = (uint8_t)tr;
        c.out_dtype = (uint8_t)od;
        if (!tuned_config_ok(c)) continue;
        out->push_back({c, tf});
    }
    return true;
}

// tile_ir tuning results, tile_ir_MxNxK.json beside the GEMM tuner's files in
// the reference's layout (src/t0/cost_model.rs:1083-1150: tile_m, tile_n,
// tile_k, split_k, wgp, tflops, all); files written here add "arch" and
// "waves".  A file for another architecture, or a tile no gfx950 kernel
// runs, is ignored.
std::string tile_cache_file(uint32_t m, uint32_t n, uint32_t k) {
    return cache_dir() + "/tile_ir_" + std::to_string(m) + "x" + std::to_string(n) + "x" + std::to_string(k) + ".json";
}

t0_tile_gemm tile_spec(uint32_t bm, uint32_t bn, uint32_t bk, uint32_t waves, uint32_t split_k) {
    t0_tile_gemm s;
    memset(&s, 0, sizeof s);
    s.tile_m = bm; s.tile_n = bn; s.tile_k = bk;
    s.waves_per_wg = waves;
    s.split_k = split_k;
    s.double_buffer = 1; s.swap_grid = 1;   // the reference's defaults (src/t0/cost_model.rs:1107-1120)
    s.transpose = T0_NT;
    s.out_dtype = T0_OUT_F32;
    return s;
}

bool load_tile_cache(uint32_t m, uint32_t n, uint32_t k, const char* arch, t0_tile_gemm* spec, double* tf) {
    std::string s, a;
    if (!read_text(tile_cache_file(m, n, k), &s)) return false;
    if (json_raw(s, "arch", &a) && a != arch) return false;
    double tm, tn, tk, t, sk = 1, w = 0;
    if (!json_num(s, "tile_m", &tm) || !json_num(s, "tile_n", &tn) || !json_num(s, "tile_k", &tk) ||
        !json_num(s, "tflops", &t))
        return false;
    json_num(s, "split_k", &sk);
    json_num(s, "waves", &w);
    t0_tile_gemm c = tile_spec((uint32_t)tm, (uint32_t)tn, (uint32_t)tk, (uint32_t)w, sk > 1 ? (uint32_t)sk : 1);
    c.wgp_mode = s.find("\"wgp\":true") != std::string::npos;
    const uint32_t q = c.split_k;
    if (!tile_instance(c) || q > 16 || (q & (q - 1))) return false;
    if (!w) c.waves_per_wg = tile_instance(c)->nw();
    *spec = c;
    *tf = t;
    return true;
}

bool save_tile_cache(uint32_t m, uint32_t n, uint32_t k, const char* arch, const t0_tile_gemm& c, double tf,
                     const std::vector<std::pair<t0_tile_gemm, double>>& all) {
    const std::string d = cache_dir();
    mkdir(d.c_str(), 0755);
    std::ofstream f(tile_cache_file(m, n, k));
    if (!f) return false;
    char num[32];
    snprintf(num, sizeof num, "%.2f", tf);
    f << "{\"tile_m\":" << c.tile_m << ",\"tile_n\":" << c.tile_n << ",\"tile_k\":" << c.tile_k
      << ",\"split_k\":" << (c.split_k > 1 ? c.split_k : 1) << ",\"wgp\":" << (c.wgp_mode ? "true" : "false")
      << ",\"tflops\":" << num << ",\"all\":[";
    for (size_t i = 0; i < all.size(); i++) {
        snprintf(num, sizeof num, "%.2f", all[i].second);
        f << (i ? "," : "") << "[\"" << tile_name(all[i].first) << "\"," << num << "]";
    }
    f << "],\"arch\":\"" << arch << "\",\"waves\":" << c.waves_per_wg << "}\n";
    return (bool)f;
}

}  // namespace

// ================================================================= C ABI ==
extern "C" {

int t0_runtime_create(int device_ordinal, t0_runtime** out) {
    if (!out) return fail(T0_ERR_INVALID, "null output");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(T0_ERR_NO_DEVICE, "no HIP device visible");
    if (device_ordinal < 0 || device_ordinal >= n) return fail(T0_ERR_NO_DEVICE, "device %d of %d", device_ordinal, n);
    HIPCHK(hipSetDevice(device_ordinal));
    hipDeviceProp_t prop;
    HIPCHK(hipGetDeviceProperties(&prop, device_ordinal));
    const std::string arch = prop.gcnArchName;
    if (arch.compare(0, 6, "gfx950") != 0)
        return fail(T0_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950 only", device_ordinal, arch.c_str());
    auto* rt = new t0_runtime();
    rt->device = device_ordinal;
    rt->arch = "gfx950";
    rt->cu_count = prop.multiProcessorCount;
    rt->clock_khz = prop.clockRate;
    hipError_t e = hipStreamCreateWithFlags(&rt->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) { delete rt; return fail(T0_ERR_HIP, "hipStreamCreate: %s", hipGetErrorString(e)); }
    rt->stream = rt->own_stream;
    e = hipModuleLoadData(&rt->module, t0_hsaco_start);
    if (e != hipSuccess) {
        hipStreamDestroy(rt->own_stream);
        delete rt;
        return fail(T0_ERR_HIP, "hipModuleLoadData(embedded gfx950 code object): %s", hipGetErrorString(e));
    }
    int r = t0h_noalloc_setup(device_ordinal);   // the no-allocation entry's scratch on this device
    if (r) {
        hipModuleUnload(rt->module);
        hipStreamDestroy(rt->own_stream);
        delete rt;
        return r;
    }
    *out = rt;
    return T0_OK;
}

int t0_runtime_destroy(t0_runtime* rt) {
    if (!rt) return T0_OK;
    hipSetDevice(rt->device);
    hipStreamSynchronize(rt->stream);
    for (auto* g : rt->graphs) g->rt = nullptr;   // graphs outliving the runtime no longer point at it
    for (auto& kv : rt->cache) {
        if (kv.second->own_module) hipModuleUnload(kv.second->own_module);
        delete kv.second;
    }
    for (auto& kv : rt->pool)
        for (auto* b : kv.second) { hipFree(b->ptr); delete b; }
    if (rt->ws) hipFree(rt->ws);
    if (rt->stage) hipFree(rt->stage);
    if (rt->sem) hipFree(rt->sem);
    if (rt->probe) hipFree(rt->probe);
    if (rt->module) hipModuleUnload(rt->module);
    if (rt->own_stream) hipStreamDestroy(rt->own_stream);
    delete rt;
    return T0_OK;
}

int t0_runtime_set_stream(t0_runtime* rt, void* s) {
    if (!rt) return fail(T0_ERR_INVALID, "null runtime");
    rt->stream = s ? (hipStream_t)s : rt->own_stream;
    return T0_OK;
}
void* t0_runtime_stream(t0_runtime* rt) { return rt ? (void*)rt->stream : nullptr; }
int t0_runtime_is_poisoned(const t0_runtime* rt) { return rt && rt->poisoned.load() ? 1 : 0; }
int t0_runtime_mark_poisoned(t0_runtime* rt) {
    if (!rt) return fail(T0_ERR_INVALID, "null runtime");
    rt->poisoned.store(true);
    fprintf(stderr, "[t0] runtime POISONED -- all subsequent dispatches fail fast\n");
    return T0_OK;
}

int t0_runtime_device_info(const t0_runtime* rt, char* arch, size_t arch_len, int* cu, int* clk) {
    if (!rt) return fail(T0_ERR_INVALID, "null runtime");
    if (arch && arch_len) snprintf(arch, arch_len, "%s", rt->arch.c_str());
    if (cu) *cu = rt->cu_count;
    if (clk) *clk = rt->clock_khz;
    return T0_OK;
}

int t0_code_object(const void** data, size_t* size) {
    if (!data || !size) return fail(T0_ERR_INVALID, "null argument");
    *data = t0_hsaco_start;
    *size = (size_t)(t0_hsaco_end - t0_hsaco_start);
    return T0_OK;
}

int t0_generate(const t0_gemm_config* cfg, char* symbol, size_t len) {
    if (!cfg) return fail(T0_ERR_INVALID, "null config");
    std::string why;
    if (!config_valid(*cfg, &why)) return fail(T0_ERR_INFEASIBLE, "%s: %s", config_name(*cfg).c_str(), why.c_str());
    const std::string s = instance_for(*cfg)->symbol(cfg->transpose == T0_NN);
    if (symbol && len) snprintf(symbol, len, "%s", s.c_str());
    return T0_OK;
}

int t0_kernel_load(t0_runtime* rt, const void* co, size_t size, const char* symbol, const t0_kernel_load_config* cfg,
                   t0_kernel** out) {
    if (!rt || !co || !symbol || !out || !cfg) return fail(T0_ERR_INVALID, "null argument");
    (void)size;
    int r = set_dev(rt);
    if (r) return r;
    auto* k = new t0_kernel();
    k->kind = KK_RAW;
    if (co == (const void*)t0_hsaco_start) {
        r = get_fn(rt, symbol, &k->fn);
        if (r) { delete k; return r; }
    } else {
        hipError_t e = hipModuleLoadData(&k->own_module, co);
        if (e != hipSuccess) { delete k; return fail(T0_ERR_HIP, "hipModuleLoadData: %s", hipGetErrorString(e)); }
        e = hipModuleGetFunction(&k->fn, k->own_module, symbol);
        if (e != hipSuccess) {
            hipModuleUnload(k->own_module);
            delete k;
            return fail(T0_ERR_NOT_FOUND, "kernel %s not in code object", symbol);
        }
    }
    memcpy(k->wg, cfg->workgroup_size, sizeof k->wg);
    for (auto& w : k->wg) if (!w) w = 1;
    k->lds = cfg->lds_size;
    k->kernarg_size = cfg->kernarg_size;
    k->name = symbol;
    std::lock_guard<std::mutex> g(rt->mu);
    std::string key = "raw:" + k->name + ":" + std::to_string((uintptr_t)co);
    auto it = rt->cache.find(key);
    if (it != rt->cache.end()) {   // cached kernels live until runtime destroy
        if (k->own_module) hipModuleUnload(k->own_module);
        delete k;
        *out = it->second;
        return T0_OK;
    }
    rt->cache[key] = k;
    *out = k;
    return T0_OK;
}

int t0_ensure_kernel(t0_runtime* rt, const t0_gemm_config* cfg, t0_kernel** out) {
    if (!rt || !cfg || !out) return fail(T0_ERR_INVALID, "null argument");
    const std::string name = config_name(*cfg);
    // the name format carries no wave count; tiles with several wave layouts
    // (256x256x64 on 4 or 8 waves) are distinct kernels
    const std::string key = name + "#w" + std::to_string(cfg->wg_size / 64);
    {
        std::lock_guard<std::mutex> g(rt->mu);
        auto it = rt->cache.find(key);
        if (it != rt->cache.end()) { *out = it->second; return T0_OK; }
    }
    std::string why;
    if (!config_valid(*cfg, &why)) return fail(T0_ERR_INFEASIBLE, "%s: %s", name.c_str(), why.c_str());
    int r = set_dev(rt);
    if (r) return r;
    auto* k = new t0_kernel();
    k->kind = KK_GEMM_GEN;
    k->inst = instance_for(*cfg);
    k->cfg = *cfg;
    k->name = name;
    k->wg[0] = cfg->wg_size;
    k->lds = k->inst->lds_bytes();
    k->kernarg_size = cfg->epilogue == T0_EPI_STORE_F32 ? 40 : 48;
    r = get_fn(rt, k->inst->symbol(cfg->transpose == T0_NN), &k->fn);
    if (r) { delete k; return r; }
    std::lock_guard<std::mutex> g(rt->mu);
    auto it = rt->cache.find(key);
    if (it != rt->cache.end()) { delete k; *out = it->second; return T0_OK; }   // another thread won
    rt->cache[key] = k;
    *out = k;
    return T0_OK;
}

int t0_ensure_tile_kernel(t0_runtime* rt, const t0_tile_gemm* spec, t0_kernel** out) {
    if (!rt || !spec || !out) return fail(T0_ERR_INVALID, "null argument");
    const std::string name = tile_name(*spec);
    const GemmInstance* inst = tile_instance(*spec);
    if (!inst) return fail(T0_ERR_INFEASIBLE, "%s: no gfx950 kernel for this tile", name.c_str());
    const std::string key = name + "#w" + std::to_string(inst->nw());
    {
        std::lock_guard<std::mutex> g(rt->mu);
        auto it = rt->cache.find(key);
        if (it != rt->cache.end()) { *out = it->second; return T0_OK; }
    }
    if (spec->split_k > 1 && (spec->out_dtype == T0_OUT_BF16 || spec->n_epilogue))
        return fail(T0_ERR_INFEASIBLE, "%s: split-K planes must be f32 without epilogue", name.c_str());
    int r = set_dev(rt);
    if (r) return r;
    auto* k = new t0_kernel();
    k->kind = KK_TILE;
    k->inst = inst;
    k->tile = *spec;
    k->layout = tile_arg_layout(*spec);
    k->name = name;
    k->wg[0] = inst->threads();
    k->lds = inst->lds_bytes();
    k->kernarg_size = k->layout.size;
    r = get_fn(rt, inst->symbol(spec->transpose == T0_NN), &k->fn);
    if (r) { delete k; return r; }
    std::lock_guard<std::mutex> g(rt->mu);
    auto it = rt->cache.find(key);
    if (it != rt->cache.end()) { delete k; *out = it->second; return T0_OK; }
    rt->cache[key] = k;
    *out = k;
    return T0_OK;
}

int t0_get_kernel(t0_runtime* rt, const char* name, t0_kernel** out) {
    if (!rt || !name || !out) return fail(T0_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> g(rt->mu);
    auto it = rt->cache.find(name);
    if (it == rt->cache.end()) {
        // GEMM kernels are cached as "<name>#w<waves>": the lowest wave count loaded under this name
        const std::string pre = std::string(name) + "#w";
        it = rt->cache.lower_bound(pre);
        if (it == rt->cache.end() || it->first.compare(0, pre.size(), pre) != 0)
            return fail(T0_ERR_NOT_FOUND, "kernel %s not loaded", name);
    }
    *out = it->second;
    return T0_OK;
}

int t0_kernel_info(const t0_kernel* k, uint32_t wg[3], uint32_t* lds, uint32_t* ka, char* name, size_t len) {
    if (!k) return fail(T0_ERR_INVALID, "null kernel");
    if (wg) memcpy(wg, k->wg, sizeof k->wg);
    if (lds) *lds = k->lds;
    if (ka) *ka = k->kernarg_size;
    if (name && len) snprintf(name, len, "%s", k->name.c_str());
    return T0_OK;
}

static int dispatch_impl(t0_runtime* rt, const t0_kernel* k, const uint32_t grid[3], const void* ka, size_t len) {
    if (!rt || !k || !grid) return fail(T0_ERR_INVALID, "null argument");
    if (rt->poisoned.load())
        return fail(T0_ERR_POISONED, "queue poisoned after GPU failure -- refusing dispatch");   // gpu_context.rs:311-313
    if (k->kernarg_size && len != k->kernarg_size)                                               // gpu_context.rs:319-322
        return fail(T0_ERR_KERNARG, "kernarg mismatch: builder produced %zuB, kernel %s declares %uB", len,
                    k->name.c_str(), k->kernarg_size);
    if (len && !ka) return fail(T0_ERR_INVALID, "null kernargs");
    int r = set_dev(rt);
    if (r) return r;
    const uint8_t* b = (const uint8_t*)ka;
    for (int d = 0; d < 3; d++)
        if (grid[d] % k->wg[d]) return fail(T0_ERR_INVALID, "grid[%d]=%u is not a multiple of the workgroup size %u", d, grid[d], k->wg[d]);
    const uint32_t bx = grid[0] / k->wg[0], by = grid[1] / k->wg[1], bz = grid[2] / k->wg[2];

    if (k->kind == KK_RAW) {
        if (rt->poisoned.load()) return fail(T0_ERR_POISONED, "poisoned");
        size_t sz = len;
        void* cfgv[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(ka), HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz,
                        HIP_LAUNCH_PARAM_END};
        HIPCHK(hipModuleLaunchKernel(k->fn, bx, by, bz, k->wg[0], k->wg[1], k->wg[2], 0, rt->stream, nullptr, cfgv));
        return T0_OK;
    }
    t0_gemm_params p;
    memset(&p, 0, sizeof p);
    p.A = (const void*)rd64(b);
    p.B = (const void*)rd64(b + 8);
    p.C = (void*)rd64(b + 16);
    p.K = rd32(b + 24);
    p.N = rd32(b + 28);
    p.y_split_stride = rd32(b + 36);
    bool nn;
    if (k->kind == KK_GEMM_GEN) {
        const t0_gemm_config& c = k->cfg;
        const uint32_t sk = split_of(c);
        // gemm_gen kernels carry no M: the grid gives the M tiles
        // (src/t0/gemm_gen.rs:308-329; M % tile_m == 0 there).
        const uint32_t tiles_m = c.swap_grid ? by / sk : bx;
        p.M = tiles_m * c.tile_m;
        p.split_k = sk;
        p.flags = c.out_dtype == T0_OUT_BF16 ? T0_GEMM_OUT_BF16 : 0;
        p.epi_ops = epi_ops_from_gemm_gen(c.epilogue);
        if (len >= 48) p.bias = (const float*)rd64(b + 40);
        nn = c.transpose == T0_NN;
    } else {
        const t0_tile_gemm& s = k->tile;
        const uint32_t shift = rd32(b + 32);
        p.M = rd32(b + 40);
        p.split_k = 1u << std::min(shift, 4u);
        p.flags = s.out_dtype == T0_OUT_BF16 ? T0_GEMM_OUT_BF16 : 0;
        p.epi_ops = tile_epi_ops(s);
        if (k->layout.has_bias) p.bias = (const float*)rd64(b + k->layout.bias_off);
        if (k->layout.has_scale) p.epi_scale = rdf(b + k->layout.scale_off);
        if (k->layout.has_clamp) { p.clamp_lo = rdf(b + k->layout.clamp_off); p.clamp_hi = rdf(b + k->layout.clamp_off + 4); }
        nn = s.transpose == T0_NN;
    }
    p.lda = p.K;
    p.ldb = nn ? p.N : p.K;
    p.ldc = p.N;
    if (p.split_k > 1 && p.K % p.split_k) return fail(T0_ERR_INVALID, "K=%u not divisible by split_k=%u", p.K, p.split_k);
    return run_gemm_params(rt, k->inst, nn, p);
}

int t0_dispatch(t0_runtime* rt, const t0_kernel* k, const uint32_t grid[3], const void* ka, size_t len) {
    int r = dispatch_impl(rt, k, grid, ka, len);
    if (r) return r;
    hipError_t e = hipStreamSynchronize(rt->stream);
    if (e != hipSuccess) {   // src/ignis/gpu_context.rs:352-355
        t0_runtime_mark_poisoned(rt);
        return fail(T0_ERR_HIP, "wait failed: %s", hipGetErrorString(e));
    }
    return T0_OK;
}

int t0_dispatch_async(t0_runtime* rt, const t0_kernel* k, const uint32_t grid[3], const void* ka, size_t len) {
    int r = dispatch_impl(rt, k, grid, ka, len);
    if (r) return r;
    return (int)(rt->slot.fetch_add(1) % 256);
}

int t0_wait_idle(t0_runtime* rt) {
    if (!rt) return fail(T0_ERR_INVALID, "null runtime");
    hipError_t e = hipStreamSynchronize(rt->stream);
    if (e != hipSuccess) { t0_runtime_mark_poisoned(rt); return fail(T0_ERR_HIP, "%s", hipGetErrorString(e)); }
    return T0_OK;
}
int t0_synchronize(t0_runtime* rt) { return t0_wait_idle(rt); }

// ---------------------------------------------------------------- memory --
int t0_alloc(t0_runtime* rt, size_t bytes, t0_buffer** out) {
    if (!rt || !out) return fail(T0_ERR_INVALID, "null argument");
    int r = set_dev(rt);
    if (r) return r;
    const size_t rounded = std::max<size_t>(4096, (bytes + 4095) & ~(size_t)4095);
    {
        std::lock_guard<std::mutex> g(rt->mu);
        auto it = rt->pool.find(rounded);
        if (it != rt->pool.end() && !it->second.empty()) {
            t0_buffer* b = it->second.back();
            it->second.pop_back();
            b->size = bytes;
            HIPCHK(hipMemsetAsync(b->ptr, 0, b->alloc_size, rt->stream));   // zeroed on reuse
            HIPCHK(hipStreamSynchronize(rt->stream));
            *out = b;
            return T0_OK;
        }
    }
    auto* b = new t0_buffer();
    b->rt = rt;
    b->size = bytes;
    b->alloc_size = rounded;
    hipError_t e = hipMalloc(&b->ptr, rounded);
    if (e != hipSuccess) { delete b; return fail(T0_ERR_HIP, "hipMalloc(%zu): %s", rounded, hipGetErrorString(e)); }
    *out = b;
    return T0_OK;
}

int t0_recycle(t0_runtime* rt, t0_buffer* b) {
    if (!rt || !b) return fail(T0_ERR_INVALID, "null argument");
    std::lock_guard<std::mutex> g(rt->mu);
    rt->pool[b->alloc_size].push_back(b);
    return T0_OK;
}

int t0_buffer_free(t0_buffer* b) {
    if (!b) return T0_OK;
    hipFree(b->ptr);
    delete b;
    return T0_OK;
}

uint64_t t0_buffer_addr(const t0_buffer* b) { return b ? (uint64_t)b->ptr : 0; }
size_t t0_buffer_size(const t0_buffer* b) { return b ? b->size : 0; }

int t0_buffer_write(t0_buffer* b, size_t off, const void* src, size_t len) {
    if (!b || (!src && len) || off + len > b->alloc_size) return fail(T0_ERR_INVALID, "write out of range");
    HIPCHK(hipMemcpy((char*)b->ptr + off, src, len, hipMemcpyHostToDevice));
    return T0_OK;
}

int t0_buffer_read(const t0_buffer* b, size_t off, void* dst, size_t len) {
    if (!b || (!dst && len) || off + len > b->alloc_size) return fail(T0_ERR_INVALID, "read out of range");
    HIPCHK(hipStreamSynchronize(b->rt->stream));
    HIPCHK(hipMemcpy(dst, (const char*)b->ptr + off, len, hipMemcpyDeviceToHost));
    return T0_OK;
}

int t0_buffer_zero(t0_buffer* b) {
    if (!b) return fail(T0_ERR_INVALID, "null buffer");
    HIPCHK(hipMemsetAsync(b->ptr, 0, b->alloc_size, b->rt->stream));
    HIPCHK(hipStreamSynchronize(b->rt->stream));
    return T0_OK;
}

int t0_read_f32(const t0_buffer* b, float* dst, size_t count) { return t0_buffer_read(b, 0, dst, count * 4); }

int t0_memcpy_h2d(t0_runtime* rt, uint64_t dst, const void* src, size_t len) {
    if (!rt) return fail(T0_ERR_INVALID, "null runtime");
    HIPCHK(hipStreamSynchronize(rt->stream));
    HIPCHK(hipMemcpy((void*)dst, src, len, hipMemcpyHostToDevice));
    return T0_OK;
}

int t0_memcpy_d2h(t0_runtime* rt, void* dst, uint64_t src, size_t len) {
    if (!rt) return fail(T0_ERR_INVALID, "null runtime");
    HIPCHK(hipStreamSynchronize(rt->stream));
    HIPCHK(hipMemcpy(dst, (const void*)src, len, hipMemcpyDeviceToHost));
    return T0_OK;
}

int t0_memset_d(t0_runtime* rt, uint64_t dst, int value, size_t len) {
    if (!rt) return fail(T0_ERR_INVALID, "null runtime");
    HIPCHK(hipMemsetAsync((void*)dst, value, len, rt->stream));
    return T0_OK;
}

int t0_event_create(t0_event** out) {
    if (!out) return fail(T0_ERR_INVALID, "null output");
    auto* e = new t0_event();
    hipError_t r = hipEventCreate(&e->ev);
    if (r != hipSuccess) { delete e; return fail(T0_ERR_HIP, "hipEventCreate: %s", hipGetErrorString(r)); }
    *out = e;
    return T0_OK;
}
int t0_event_destroy(t0_event* e) {
    if (e) { hipEventDestroy(e->ev); delete e; }
    return T0_OK;
}
int t0_event_record(t0_runtime* rt, t0_event* e) {
    if (!rt || !e) return fail(T0_ERR_INVALID, "null argument");
    HIPCHK(hipEventRecord(e->ev, rt->stream));
    return T0_OK;
}
int t0_event_synchronize(t0_event* e) {
    if (!e) return fail(T0_ERR_INVALID, "null event");
    HIPCHK(hipEventSynchronize(e->ev));
    return T0_OK;
}
int t0_event_elapsed_ms(const t0_event* a, const t0_event* b, float* ms) {
    if (!a || !b || !ms) return fail(T0_ERR_INVALID, "null argument");
    HIPCHK(hipEventElapsedTime(ms, a->ev, b->ev));
    return T0_OK;
}

// ----------------------------------------------------------------- graphs --

int t0_graph_begin(t0_runtime* rt) {
    if (!rt) return fail(T0_ERR_INVALID, "null runtime");
    int r = set_dev(rt);
    if (r) return r;
    HIPCHK(hipStreamBeginCapture(rt->stream, hipStreamCaptureModeThreadLocal));
    return T0_OK;
}

int t0_graph_end(t0_runtime* rt, t0_graph** out) {
    if (!rt || !out) return fail(T0_ERR_INVALID, "null argument");
    auto* g = new t0_graph();
    hipError_t e = hipStreamEndCapture(rt->stream, &g->graph);
    if (e != hipSuccess) { delete g; return fail(T0_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e)); }
    e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        hipGraphDestroy(g->graph);
        delete g;
        return fail(T0_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    {
        std::lock_guard<std::recursive_mutex> lk(rt->call_mu);
        g->rt = rt;
        rt->graphs.insert(g);
    }
    *out = g;
    return T0_OK;
}

int t0_graph_launch(t0_runtime* rt, const t0_graph* g) {
    if (!rt || !g) return fail(T0_ERR_INVALID, "null argument");
    if (rt->poisoned.load()) return fail(T0_ERR_POISONED, "runtime poisoned; refusing graph launch");
    HIPCHK(hipGraphLaunch(g->exec, rt->stream));
    return T0_OK;
}

int t0_graph_destroy(t0_graph* g) {
    if (!g) return T0_OK;
    if (g->rt) {
        std::lock_guard<std::recursive_mutex> lk(g->rt->call_mu);
        g->rt->graphs.erase(g);
    }
    if (g->exec) hipGraphExecDestroy(g->exec);
    if (g->graph) hipGraphDestroy(g->graph);
    delete g;
    return T0_OK;
}

// ------------------------------------------------------------ high level --
static int desc_to_params(const t0_gemm_desc* d, const t0_gemm_config& c, t0_gemm_params& p) {
    memset(&p, 0, sizeof p);
    p.A = (const void*)d->a;
    p.B = (const void*)d->b;
    p.C = (void*)d->c;
    p.bias = (const float*)d->bias;
    p.M = d->m; p.N = d->n; p.K = d->k;
    const bool nn = d->transpose == T0_NN;
    p.lda = d->lda ? d->lda : d->k;
    p.ldb = d->ldb ? d->ldb : (nn ? d->n : d->k);
    p.ldc = d->ldc ? d->ldc : d->n;
    p.split_k = split_of(c);
    p.flags = d->out_dtype == T0_OUT_BF16 ? T0_GEMM_OUT_BF16 : 0;
    uint32_t ops = 0;
    for (uint32_t i = 0; i < d->n_epilogue && i < 8; i++) {
        if (d->epilogue[i] == 0 || d->epilogue[i] > 8) return fail(T0_ERR_INVALID, "bad epilogue op %u", d->epilogue[i]);
        ops |= (uint32_t)d->epilogue[i] << (4 * i);
    }
    p.epi_ops = ops;
    p.epi_scale = d->scale;
    p.clamp_lo = d->clamp_min;
    p.clamp_hi = d->clamp_max;
    // split-K in t0_gemm always reduces in-kernel (one output, epilogue once)
    if (p.split_k > 1) p.flags |= T0_GEMM_FIXUP;
    if (p.lda < p.K || p.ldc < p.N || p.ldb < (nn ? p.N : p.K)) return fail(T0_ERR_INVALID, "leading dimension too small");
    return T0_OK;
}

int t0_gemm_select(t0_runtime* rt, const t0_gemm_desc* d, t0_gemm_config* out) {
    if (!rt || !d || !out) return fail(T0_ERR_INVALID, "null argument");
    auto& T = tuner();
    const std::string key = tune_key(rt, d->m, d->n, d->k, d->transpose, d->out_dtype);
    {
        std::lock_guard<std::mutex> g(T.mu);
        auto it = T.mem.find(key);
        if (it != T.mem.end()) { *out = it->second.first; return T0_OK; }
    }
    double tf;
    if (load_cache_file(d->m, d->n, d->k, d->transpose, d->out_dtype, rt->arch.c_str(), out, &tf)) {
        std::lock_guard<std::mutex> g(T.mu);
        T.mem[key] = {*out, tf};
        return T0_OK;
    }
    auto c = rank_candidates(d->m, d->n, d->k, d->transpose, d->out_dtype, true);
    if (c.empty()) return fail(T0_ERR_INFEASIBLE, "no candidate for %ux%ux%u", d->m, d->n, d->k);
    *out = c.front().cfg;
    return T0_OK;
}

// Whether config c's in-kernel split-K fits the caller's scratch array (its
// counters and partial tiles, as run_gemm_params lays them out there); a
// config without split-K needs none.
static bool scratch_fits(const t0_gemm_config& c, const t0_gemm_desc* d, const Scratch& sc) {
    const uint32_t sk = split_of(c);
    if (sk <= 1) return true;
    const uint64_t tiles = (uint64_t)((d->m + c.tile_m - 1) / c.tile_m) * ((d->n + c.tile_n - 1) / c.tile_n);
    return tiles <= T0_NOALLOC_MAX_TILES &&
           sk * tiles * c.tile_m * c.tile_n * 4 <= sc.bytes - (uint64_t)T0_NOALLOC_MAX_TILES * 4;
}

static int gemm_impl(t0_runtime* rt, const t0_gemm_config* cfg, const t0_gemm_desc* d, uint64_t* clock_probe,
                     uint32_t* workgroups, const Scratch* sc = nullptr) {
    if (!rt || !d) return fail(T0_ERR_INVALID, "null argument");
    std::lock_guard<std::recursive_mutex> call_lock(rt->call_mu);
    if (!d->m || !d->n || !d->k) return fail(T0_ERR_INVALID, "empty GEMM %ux%ux%u", d->m, d->n, d->k);
    if (d->transpose > T0_NN || d->out_dtype > T0_OUT_BF16) return fail(T0_ERR_INVALID, "bad layout / out_dtype");
    t0_gemm_config c;
    if (cfg) c = *cfg;
    else {
        int r = t0_gemm_select(rt, d, &c);
        if (r) return r;
        if (sc && !scratch_fits(c, d, *sc)) {
            // the caller's scratch is too small for the selected split: the
            // best-ranked candidate that fits it, else the selection unsplit
            t0_gemm_config fit = c;
            fit.split_k = 0;
            for (const auto& cand : rank_candidates(d->m, d->n, d->k, d->transpose, d->out_dtype, true))
                if (scratch_fits(cand.cfg, d, *sc)) {
                    fit = cand.cfg;
                    break;
                }
            c = fit;
        }
    }
    const GemmInstance* g = instance_for(c);
    if (!g) return fail(T0_ERR_INFEASIBLE, "%s: no gfx950 kernel", config_name(c).c_str());
    const uint32_t sk = split_of(c);
    if (sk > 16 || (sk & (sk - 1))) return fail(T0_ERR_INVALID, "split_k must be a power of two <= 16");
    t0_gemm_params p;
    int r = desc_to_params(d, c, p);
    if (r) return r;
    r = set_dev(rt);
    if (r) return r;
    if (p.split_k > 1 && !fast_ok(p, d->transpose == T0_NN)) p.split_k = 1, p.flags &= ~T0_GEMM_FIXUP;
    if (clock_probe) {
        if (p.split_k > 1 || !fast_ok(p, d->transpose == T0_NN))
            return fail(T0_ERR_INVALID, "the clock probe needs a tiled kernel without split-K");
        const uint32_t wgs = ((p.M + g->bm - 1) / g->bm) * ((p.N + g->bn - 1) / g->bn);
        if (wgs > *workgroups) return fail(T0_ERR_INVALID, "clock probe: %u workgroups, at most %u", wgs, *workgroups);
        p.clock_probe = clock_probe;
        *workgroups = wgs;
    }
    return run_gemm_params(rt, g, d->transpose == T0_NN, p, 0, false, sc);
}

}  // extern "C"

int t0h::gemm_with_scratch(t0_runtime* rt, const t0_gemm_config* cfg, const t0_gemm_desc* d, void* scratch,
                           size_t bytes) {
    if (!scratch || bytes <= T0_NOALLOC_MAX_TILES * 4) return fail(T0_ERR_INVALID, "no scratch");
    Scratch sc;
    sc.base = scratch;
    sc.bytes = bytes;
    return gemm_impl(rt, cfg, d, nullptr, nullptr, &sc);
}

int t0h::runtime_device(const t0_runtime* rt) { return rt ? rt->device : -1; }

extern "C" {

int t0_gemm(t0_runtime* rt, const t0_gemm_config* cfg, const t0_gemm_desc* d) {
    return gemm_impl(rt, cfg, d, nullptr, nullptr);
}

int t0_gemm_clock_probe(t0_runtime* rt, const t0_gemm_config* cfg, const t0_gemm_desc* d, double* sclk_mhz,
                        double* span_us, double* wg_cycles) {
    if (!rt || !d || !sclk_mhz || !span_us) return fail(T0_ERR_INVALID, "null argument");
    std::lock_guard<std::recursive_mutex> call_lock(rt->call_mu);
    const size_t max_wg = 65536;
    if (!rt->probe) {
        int r = set_dev(rt);
        if (r) return r;
        HIPCHK(hipMalloc(&rt->probe, max_wg * 32));
    }
    uint32_t wgs = (uint32_t)max_wg;   // in: capacity of the timestamp buffer, out: workgroups launched
    int r = gemm_impl(rt, cfg, d, (uint64_t*)rt->probe, &wgs);
    if (r) return r;
    std::vector<uint64_t> ts((size_t)wgs * 4);
    HIPCHK(hipStreamSynchronize(rt->stream));
    HIPCHK(hipMemcpy(ts.data(), rt->probe, ts.size() * 8, hipMemcpyDeviceToHost));
    std::vector<double> mhz, cyc;
    uint64_t first = ~0ull, last = 0;
    for (uint32_t w = 0; w < wgs; w++) {
        const uint64_t rt0 = ts[4 * w], rt1 = ts[4 * w + 1], c0 = ts[4 * w + 2], c1 = ts[4 * w + 3];
        if (rt1 <= rt0) continue;
        mhz.push_back((double)(c1 - c0) / (double)(rt1 - rt0) * 100.0);   // s_memrealtime counts at 100 MHz
        cyc.push_back((double)(c1 - c0));
        first = std::min(first, rt0);
        last = std::max(last, rt1);
    }
    if (mhz.empty()) return fail(T0_ERR_HIP, "clock probe: no workgroup recorded its timestamps");
    std::sort(mhz.begin(), mhz.end());
    std::sort(cyc.begin(), cyc.end());
    *sclk_mhz = mhz[mhz.size() / 2];
    *span_us = (double)(last - first) / 100.0;
    if (wg_cycles) *wg_cycles = cyc[cyc.size() / 2];
    return T0_OK;
}

// ------------------------------------------------------------------ tuner --
int t0_tuner_set_cache_dir(const char* dir) {
    std::lock_guard<std::mutex> g(tuner().mu);
    tuner().dir = dir ? dir : "";
    tuner().mem.clear();
    tuner().all.clear();
    return T0_OK;
}

int t0_tuner_set_params(uint32_t max_candidates, uint32_t n_iters) {
    std::lock_guard<std::mutex> g(tuner().mu);
    if (max_candidates) tuner().max_candidates = max_candidates;
    if (n_iters) tuner().n_iters = n_iters;
    return T0_OK;
}

// The tuning cache on disk without a runtime (gfx950 entries): warm-start a
// tuner with known picks, read one back, or drop one
// (src/t0/auto_gemm.rs:439-507: load_cache, save_cache, invalidate).
int t0_tuner_cache_store(uint32_t m, uint32_t n, uint32_t k, uint32_t tr, uint32_t od, const t0_gemm_config* cfg,
                         double tflops) {
    if (!cfg || !m || !n || !k || tr > T0_NN || od > T0_OUT_BF16) return fail(T0_ERR_INVALID, "bad arguments");
    if (!tuned_config_ok(*cfg)) return fail(T0_ERR_INFEASIBLE, "%s: no gfx950 kernel", config_name(*cfg).c_str());
    std::lock_guard<std::mutex> g(tuner().mu);
    if (!save_cache_file(m, n, k, tr, od, "gfx950", *cfg, tflops, TuneList{{*cfg, tflops}}))
        return fail(T0_ERR_INVALID, "cannot write %s", cache_file(m, n, k, tr, od).c_str());
    tuner().mem.erase(tune_key_arch("gfx950", m, n, k, tr, od));
    tuner().all.erase(tune_key_arch("gfx950", m, n, k, tr, od));
    return T0_OK;
}

int t0_tuner_cache_load(uint32_t m, uint32_t n, uint32_t k, uint32_t tr, uint32_t od, t0_gemm_config* cfg,
                        double* tflops) {
    if (!cfg || !tflops) return fail(T0_ERR_INVALID, "null output");
    std::lock_guard<std::mutex> g(tuner().mu);
    if (!load_cache_file(m, n, k, tr, od, "gfx950", cfg, tflops))
        return fail(T0_ERR_NOT_FOUND, "no usable tuned config in %s", cache_file(m, n, k, tr, od).c_str());
    return T0_OK;
}

int t0_tuner_invalidate(uint32_t m, uint32_t n, uint32_t k, uint32_t tr, uint32_t od) {
    std::lock_guard<std::mutex> g(tuner().mu);
    tuner().mem.erase(tune_key_arch("gfx950", m, n, k, tr, od));
    tuner().all.erase(tune_key_arch("gfx950", m, n, k, tr, od));
    remove(cache_file(m, n, k, tr, od).c_str());
    return T0_OK;
}

int t0_tune_results(uint32_t m, uint32_t n, uint32_t k, uint32_t tr, uint32_t od, t0_tune_entry* all, uint32_t cap,
                    uint32_t* n_all, int* from_cache) {
    if (!n_all || (cap && !all)) return fail(T0_ERR_INVALID, "null output");
    if (tr > T0_NN || od > T0_OUT_BF16) return fail(T0_ERR_INVALID, "bad layout / out_dtype");
    std::lock_guard<std::mutex> g(tuner().mu);
    TuneList list;
    int cached = 0;
    auto it = tuner().all.find(tune_key_arch("gfx950", m, n, k, tr, od));
    if (it != tuner().all.end()) {
        list = it->second;
    } else if (load_cache_all(m, n, k, tr, od, "gfx950", &list)) {
        cached = 1;
    } else {
        return fail(T0_ERR_NOT_FOUND, "%ux%ux%u was not tuned here and %s holds no usable entry", m, n, k,
                    cache_file(m, n, k, tr, od).c_str());
    }
    for (uint32_t i = 0; i < cap && i < list.size(); i++) all[i] = {list[i].first, list[i].second};
    *n_all = (uint32_t)list.size();
    if (from_cache) *from_cache = cached;
    return T0_OK;
}

// 256^3 smoke test of one candidate (src/t0/auto_gemm.rs:223-272): small
// integer data (exact in bf16 and in the f32 sums) checked at sampled points
// against the exact integer product.
static int smoke_256(t0_runtime* rt, const t0_gemm_config& c, uint32_t tr, uint32_t od, bool* ok) {
    const uint32_t S = 256;
    std::vector<uint16_t> a(S * S), b(S * S);
    auto bf = [](int v) { float f = (float)v; uint32_t u; memcpy(&u, &f, 4); return (uint16_t)(u >> 16); };
    for (uint32_t i = 0; i < S * S; i++) { a[i] = bf((int)(i % 7) - 3); b[i] = bf((int)(i % 5) - 2); }
    void *da, *db, *dc;
    HIPCHK(hipMalloc(&da, S * S * 2));
    HIPCHK(hipMalloc(&db, S * S * 2));
    HIPCHK(hipMalloc(&dc, S * S * 4));
    HIPCHK(hipMemcpy(da, a.data(), S * S * 2, hipMemcpyHostToDevice));
    HIPCHK(hipMemcpy(db, b.data(), S * S * 2, hipMemcpyHostToDevice));
    HIPCHK(hipMemset(dc, 0, S * S * 4));
    t0_gemm_desc d;
    memset(&d, 0, sizeof d);
    d.a = (uint64_t)da; d.b = (uint64_t)db; d.c = (uint64_t)dc;
    d.m = d.n = d.k = S;
    d.transpose = tr;
    d.out_dtype = od;
    int r = t0_gemm(rt, &c, &d);
    std::vector<float> cf(S * S);
    std::vector<uint16_t> ch(S * S);
    if (!r) {
        hipStreamSynchronize(rt->stream);
        if (od == T0_OUT_BF16) hipMemcpy(ch.data(), dc, S * S * 2, hipMemcpyDeviceToHost);
        else hipMemcpy(cf.data(), dc, S * S * 4, hipMemcpyDeviceToHost);
    }
    hipFree(da); hipFree(db); hipFree(dc);
    if (r) { *ok = false; return T0_OK; }
    *ok = true;
    auto av = [&](uint32_t i, uint32_t kk) { return (int)((i * S + kk) % 7) - 3; };
    auto bv = [&](uint32_t j, uint32_t kk) {   // B element for output column j
        const uint32_t idx = tr == T0_NN ? kk * S + j : j * S + kk;
        return (int)(idx % 5) - 2;
    };
    for (uint32_t t = 0; t < 72; t++) {
        const uint32_t idx = t < 16 ? t * S + t : ((t - 16) * 331 + 97) % (S * S);
        const uint32_t i = idx / S, j = idx % S;
        long exact = 0;
        for (uint32_t kk = 0; kk < S; kk++) exact += (long)av(i, kk) * bv(j, kk);
        float got;
        if (od == T0_OUT_BF16) { uint32_t u = (uint32_t)ch[idx] << 16; memcpy(&got, &u, 4); }
        else got = cf[idx];
        if (std::fabs(got - (float)exact) > (od == T0_OUT_BF16 ? std::fabs((float)exact) / 128.0f + 0.5f : 0.0f)) {
            *ok = false;
            break;
        }
    }
    return T0_OK;
}

int t0_tune(t0_runtime* rt, uint32_t m, uint32_t n, uint32_t k, uint32_t tr, uint32_t od, t0_gemm_config* cfg_out,
            double* tflops_out) {
    if (!rt || !m || !n || !k) return fail(T0_ERR_INVALID, "bad arguments");
    auto& T = tuner();
    const std::string key = tune_key(rt, m, n, k, tr, od);
    {
        std::lock_guard<std::mutex> g(T.mu);
        auto it = T.mem.find(key);
        if (it != T.mem.end()) {
            if (cfg_out) *cfg_out = it->second.first;
            if (tflops_out) *tflops_out = it->second.second;
            return T0_OK;
        }
    }
    t0_gemm_config cached;
    double tf = 0;
    if (load_cache_file(m, n, k, tr, od, rt->arch.c_str(), &cached, &tf)) {
        std::lock_guard<std::mutex> g(T.mu);
        T.mem[key] = {cached, tf};
        if (cfg_out) *cfg_out = cached;
        if (tflops_out) *tflops_out = tf;
        return T0_OK;
    }
    int r = set_dev(rt);
    if (r) return r;
    auto ranked = rank_candidates(m, n, k, tr, od, true);
    // candidate list: best-ranked, at most two split factors per tile
    std::vector<t0_gemm_config> cands;
    std::map<std::string, int> per_tile;
    for (const auto& c : ranked) {
        if (cands.size() >= T.max_candidates) break;
        const std::string tile = std::to_string(c.cfg.tile_m) + "x" + std::to_string(c.cfg.tile_n) + "x" + std::to_string(c.cfg.tile_k);
        if (per_tile[tile]++ >= 2) continue;
        cands.push_back(c.cfg);
    }
    // Operands: seeded N(0,1) values rounded to bf16 (the MFMA clock under
    // load depends on the data, and constant operands run faster; the
    // reference zero-fills them, src/t0/auto_gemm.rs:311-314).  The weight
    // operand B is rotated through copies that together exceed the 256 MB
    // Infinity Cache, so every launch reads it from HBM as inference does;
    // the launches over all copies are one HIP graph, replayed and timed.
    const size_t ob = od == T0_OUT_BF16 ? 2 : 4;
    const size_t b_bytes = (size_t)n * k * 2;
    const uint32_t rot = (uint32_t)std::min<size_t>(64, std::max<size_t>(2, (300ull << 20) / b_bytes + 1));
    void *da = nullptr, *dc = nullptr;
    std::vector<void*> db(rot, nullptr);
    auto free_all = [&]() {
        hipFree(da);
        hipFree(dc);
        for (void* p : db) hipFree(p);
    };
    hipError_t he = hipMalloc(&da, (size_t)m * k * 2);
    if (he == hipSuccess) he = hipMalloc(&dc, (size_t)m * n * ob);
    for (uint32_t i = 0; i < rot && he == hipSuccess; i++) he = hipMalloc(&db[i], b_bytes);
    if (he == hipSuccess) {
        std::vector<uint16_t> h(std::max((size_t)m * k, (size_t)n * k));
        fill_normal_bf16(h.data(), (size_t)m * k, 0x9E3779B97F4A7C15ull);
        he = hipMemcpy(da, h.data(), (size_t)m * k * 2, hipMemcpyHostToDevice);
        fill_normal_bf16(h.data(), (size_t)n * k, 0xD1B54A32D192ED03ull);
        for (uint32_t i = 0; i < rot && he == hipSuccess; i++) he = hipMemcpy(db[i], h.data(), b_bytes, hipMemcpyHostToDevice);
    }
    if (he != hipSuccess) {
        free_all();
        return fail(T0_ERR_HIP, "tuner operands (%u copies of B): %s", rot, hipGetErrorString(he));
    }
    t0_gemm_desc d;
    memset(&d, 0, sizeof d);
    d.a = (uint64_t)da; d.c = (uint64_t)dc;
    d.m = m; d.n = n; d.k = k;
    d.transpose = tr;
    d.out_dtype = od;
    hipEvent_t e0, e1;
    hipEventCreate(&e0);
    hipEventCreate(&e1);
    TuneList results;
    for (const auto& c : cands) {
        bool ok = false;
        if (smoke_256(rt, c, tr, od, &ok) || !ok) {
            fprintf(stderr, "[autotune] %s -> SKIP (256^3 check failed)\n", config_name(c).c_str());
            continue;
        }
        // one eager launch per copy of B: sizes the runtime's workspace
        // before the capture and warms the code
        bool bad = false;
        for (uint32_t i = 0; i < rot && !bad; i++) {
            d.b = (uint64_t)db[i];
            bad = t0_gemm(rt, &c, &d) != T0_OK;
        }
        if (bad || hipStreamSynchronize(rt->stream) != hipSuccess) continue;
        t0_graph* gr = nullptr;
        int ge;
        {
            // the runtime's call lock across the capture: a call from another
            // thread on this runtime would otherwise land in the graph
            std::lock_guard<std::recursive_mutex> capture_lock(rt->call_mu);
            if (t0_graph_begin(rt) != T0_OK) continue;
            for (uint32_t i = 0; i < rot; i++) {
                d.b = (uint64_t)db[i];
                if (t0_gemm(rt, &c, &d) != T0_OK) bad = true;
            }
            ge = t0_graph_end(rt, &gr);
        }
        if (ge != T0_OK || bad) {
            t0_graph_destroy(gr);
            continue;
        }
        std::vector<float> times;
        if (t0_graph_launch(rt, gr) == T0_OK && hipStreamSynchronize(rt->stream) == hipSuccess) {   // warm
            for (uint32_t it = 0; it < T.n_iters; it++) {
                hipEventRecord(e0, rt->stream);
                if (t0_graph_launch(rt, gr) != T0_OK) break;
                hipEventRecord(e1, rt->stream);
                hipEventSynchronize(e1);
                float ms = 0;
                hipEventElapsedTime(&ms, e0, e1);
                times.push_back(ms / rot);
            }
        }
        t0_graph_destroy(gr);
        if (times.empty()) continue;
        std::sort(times.begin(), times.end());
        const double us = times[times.size() / 2] * 1e3;
        results.push_back({c, 2.0 * m * n * k / (us * 1e-6) / 1e12});
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipStreamSynchronize(rt->stream);
    free_all();
    std::stable_sort(results.begin(), results.end(),
                     [](const std::pair<t0_gemm_config, double>& x, const std::pair<t0_gemm_config, double>& y) {
                         return x.second > y.second;
                     });
    t0_gemm_config best;
    if (results.empty()) {   // src/t0/auto_gemm.rs:125-167: fall back to the static choice
        int rr = t0_auto_select_legacy(m, k, n, &best);
        if (rr) return rr;
        tf = 0;
    } else {
        best = results[0].first;
        tf = results[0].second;
        save_cache_file(m, n, k, tr, od, rt->arch.c_str(), best, tf, results);
    }
    {
        std::lock_guard<std::mutex> g(T.mu);
        T.mem[key] = {best, tf};
        T.all[key] = results;
    }
    if (cfg_out) *cfg_out = best;
    if (tflops_out) *tflops_out = tf;
    return T0_OK;
}

int t0_auto_gemm(t0_runtime* rt, uint64_t a, uint64_t b, uint64_t c, uint32_t m, uint32_t n, uint32_t k, double* tflops) {
    t0_gemm_config cfg;
    int r = t0_tune(rt, m, n, k, T0_NT, T0_OUT_F32, &cfg, tflops);
    if (r) return r;
    t0_gemm_desc d;
    memset(&d, 0, sizeof d);
    d.a = a; d.b = b; d.c = c;
    d.m = m; d.n = n; d.k = k;
    r = t0_gemm(rt, &cfg, &d);
    if (r) return r;
    return t0_wait_idle(rt);
}

int t0_tile_tune(t0_runtime* rt, uint32_t m, uint32_t n, uint32_t k, t0_tile_gemm* best_out, double* tflops_out,
                 t0_tile_tune_entry* all_out, uint32_t cap, uint32_t* n_all, int* from_cache) {
    // src/t0/cost_model.rs:855-1080
    if (!rt || !m || !n || !k || !best_out) return fail(T0_ERR_INVALID, "bad arguments");
    if (n_all) *n_all = 0;
    if (from_cache) *from_cache = 0;
    t0_tile_gemm spec;
    double tf = 0;
    {
        std::lock_guard<std::mutex> g(tuner().mu);
        if (load_tile_cache(m, n, k, rt->arch.c_str(), &spec, &tf)) {   // 1. the cache file
            *best_out = spec;
            if (tflops_out) *tflops_out = tf;
            if (from_cache) *from_cache = 1;
            return T0_OK;
        }
    }
    int r = set_dev(rt);
    if (r) return r;
    // 2a. the reference's proven presets (:877-896), with its filters, mapped
    //     to the gfx950 kernel of each geometry
    std::vector<t0_tile_gemm> cands;
    std::set<std::string> seen;
    auto add = [&](const t0_tile_gemm& c) {
        const GemmInstance* g = tile_instance(c);
        if (!g) return;
        t0_tile_gemm x = c;
        x.waves_per_wg = g->nw();
        if (seen.insert(tile_name(x) + "#w" + std::to_string(g->nw())).second) cands.push_back(x);
    };
    static const uint32_t presets[][3] = {{128, 128, 64}, {128, 128, 32}, {128, 128, 16}, {128, 64, 32},
                                          {128, 64, 16},  {64, 64, 16},   {32, 64, 16}};
    for (const auto& q : presets) {
        if (k % q[2]) continue;
        if (q[0] > m && m >= 32) continue;
        if (q[1] > n && n >= 32) continue;
        add(tile_spec(q[0], q[1], q[2], 0, 1));
    }
    // 2b. the cost model's tiles (split 1, as tile_auto_select), best first
    uint32_t from_model = 0;
    for (const auto& c : rank_candidates(m, n, k, T0_NT, T0_OUT_F32, false)) {
        if (split_of(c.cfg) != 1 || from_model >= tuner().max_candidates) continue;
        const GemmInstance* g = instance_for(c.cfg);
        add(tile_spec(g->bm, g->bn, g->bk, g->nw(), 1));
        from_model++;
    }
    if (cands.empty()) return fail(T0_ERR_INFEASIBLE, "tile_tune: no candidates for %ux%ux%u", m, n, k);
    // 3. seeded N(0,1) bf16 operands (the reference zero-fills them,
    //    :1004-1009; constant data runs the MFMAs at a higher clock)
    void *da, *db, *dc;
    HIPCHK(hipMalloc(&da, (size_t)m * k * 2));
    HIPCHK(hipMalloc(&db, (size_t)n * k * 2));
    HIPCHK(hipMalloc(&dc, (size_t)m * n * 4));
    {
        std::vector<uint16_t> h(std::max((size_t)m * k, (size_t)n * k));
        fill_normal_bf16(h.data(), (size_t)m * k, 0x9E3779B97F4A7C15ull);
        HIPCHK(hipMemcpy(da, h.data(), (size_t)m * k * 2, hipMemcpyHostToDevice));
        fill_normal_bf16(h.data(), (size_t)n * k, 0xD1B54A32D192ED03ull);
        HIPCHK(hipMemcpy(db, h.data(), (size_t)n * k * 2, hipMemcpyHostToDevice));
    }
    // 4. each candidate through the tile_ir dispatch path: warm-up, then the
    //    median of per-launch event timings
    hipEvent_t e0, e1;
    hipEventCreate(&e0);
    hipEventCreate(&e1);
    std::vector<std::pair<t0_tile_gemm, double>> res;
    for (const auto& c : cands) {
        t0_kernel* kern = nullptr;
        uint8_t ka[96];
        size_t len = 0;
        uint32_t grid[3];
        if (t0_ensure_tile_kernel(rt, &c, &kern) ||
            t0_tile_build_kernargs_m((uint64_t)da, (uint64_t)db, (uint64_t)dc, k, n, m, &c, 0, 0, 1.0f, 0.0f, 0.0f,
                                     ka, &len) ||
            t0_tile_compute_grid(&c, m, n, grid))
            continue;
        bool ok = true;
        for (int w = 0; w < 3 && ok; w++) ok = t0_dispatch_async(rt, kern, grid, ka, len) >= 0;
        std::vector<float> times;
        for (uint32_t it = 0; ok && it < tuner().n_iters; it++) {
            hipEventRecord(e0, rt->stream);
            if (t0_dispatch_async(rt, kern, grid, ka, len) < 0) { ok = false; break; }
            hipEventRecord(e1, rt->stream);
            hipEventSynchronize(e1);
            float ms = 0;
            hipEventElapsedTime(&ms, e0, e1);
            times.push_back(ms);
        }
        if (!ok || times.empty()) {
            if (rt->poisoned.load()) break;   // :1037-1041
            continue;
        }
        std::sort(times.begin(), times.end());
        const double us = times[times.size() / 2] * 1e3;
        res.push_back({c, 2.0 * m * n * k / (us * 1e-6) / 1e12});
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipStreamSynchronize(rt->stream);
    hipFree(da); hipFree(db); hipFree(dc);
    if (res.empty()) return fail(T0_ERR_HIP, "tile_tune: every candidate failed");
    // 5. fastest first; the best is cached
    std::stable_sort(res.begin(), res.end(), [](const auto& a, const auto& b) { return a.second > b.second; });
    {
        std::lock_guard<std::mutex> g(tuner().mu);
        save_tile_cache(m, n, k, rt->arch.c_str(), res[0].first, res[0].second, res);
    }
    *best_out = res[0].first;
    if (tflops_out) *tflops_out = res[0].second;
    for (size_t i = 0; all_out && i < res.size() && i < cap; i++) {
        all_out[i].spec = res[i].first;
        all_out[i].tflops = res[i].second;
    }
    if (n_all) *n_all = (uint32_t)res.size();
    return T0_OK;
}

// ------------------------------------------------------------------- INT4 --
int t0_gptq_from_bytes(const void* raw, size_t len, t0_gptq_view* o) {
    // src/t0/quant_kernels.rs:251-287
    if (!raw || !o) return fail(T0_ERR_INVALID, "null argument");
    if (len < 12) return fail(T0_ERR_INVALID, "GPTQ data too short (need at least 12 bytes header)");
    const uint8_t* b = (const uint8_t*)raw;
    o->rows = rd32(b);
    o->cols = rd32(b + 4);
    o->group_size = rd32(b + 8);
    if (!o->group_size) return fail(T0_ERR_INVALID, "group_size 0");
    o->n_groups = o->cols / o->group_size;
    const size_t n_params = (size_t)o->n_groups * o->rows;
    const size_t packed = (size_t)o->rows * o->cols / 2;
    const size_t need = 12 + packed + n_params * 8;
    if (len < need) return fail(T0_ERR_INVALID, "GPTQ data truncated: need %zu bytes, got %zu", need, len);
    o->packed = b + 12;
    o->scales = (const float*)(b + 12 + packed);
    o->zero_points = (const int32_t*)(b + 12 + packed + n_params * 4);
    return T0_OK;
}

size_t t0_gptq_gpu_buffer_size(const t0_gptq_view* w) {
    // src/t0/quant_kernels.rs:289-296
    if (!w) return 0;
    return (size_t)w->rows * w->cols / 2 + (size_t)w->n_groups * w->rows * 8;
}

int t0_gptq_to_w4a16(const t0_gptq_view* w, uint32_t* qweight, void* scales, int scales_f32, uint32_t* zeros) {
    if (!w || !qweight || !scales) return fail(T0_ERR_INVALID, "null argument");
    if (w->cols % 8 || (zeros && w->rows % 8)) return fail(T0_ERR_INVALID, "cols %% 8 (and rows %% 8 for zeros) required");
    memcpy(qweight, w->packed, (size_t)w->rows * w->cols / 2);
    const uint32_t G = w->n_groups, N = w->rows;
    if (zeros) memset(zeros, 0, (size_t)G * (N / 8) * 4);
    for (uint32_t n = 0; n < N; n++)
        for (uint32_t g = 0; g < G; g++) {
            const float s = w->scales[(size_t)n * G + g];
            if (scales_f32) ((float*)scales)[(size_t)g * N + n] = s;
            else {
                uint32_t u;
                memcpy(&u, &s, 4);
                uint16_t h;
                if ((u & 0x7FFFFFFFu) > 0x7F800000u) h = (uint16_t)((u >> 16) | 0x40);
                else h = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1)) >> 16);
                ((uint16_t*)scales)[(size_t)g * N + n] = h;
            }
            if (zeros) {
                const int32_t z = w->zero_points[(size_t)n * G + g];
                if (z < 0 || z > 15) return fail(T0_ERR_INVALID, "zero point %d at row %u group %u not in 0..15", z, n, g);
                zeros[(size_t)g * (N / 8) + n / 8] |= (uint32_t)z << (4 * (n % 8));
            }
        }
    return T0_OK;
}

int t0_dequant_int4(t0_runtime* rt, uint64_t packed, uint64_t scales, uint64_t zp, uint64_t output, uint32_t rows,
                    uint32_t cols, uint32_t gs_log2, int bf16_out) {
    if (!rt || !packed || !scales || !zp || !output) return fail(T0_ERR_INVALID, "null argument");
    if (gs_log2 > 16 || ((uint64_t)rows * cols) % 2) return fail(T0_ERR_INVALID, "bad shape");
    int r = set_dev(rt);
    if (r) return r;
    hipFunction_t f;
    r = get_fn(rt, bf16_out ? "dequant_int4_bf16" : "dequant_int4_f32", &f);
    if (r) return r;
    t0_dequant_params p;
    memset(&p, 0, sizeof p);
    p.packed = (const uint8_t*)packed;
    p.scales = (const float*)scales;
    p.zero_points = (const int32_t*)zp;
    p.output = (void*)output;
    p.rows = rows;
    p.cols = cols;
    p.group_size_log2 = gs_log2;
    const uint64_t total = (uint64_t)rows * cols;
    return launch(rt, f, (uint32_t)((total + 255) / 256), 1, 1, 256, p);
}

struct W4Plan {
    std::string sym;
    uint32_t gx = 1, gy = 1, threads = 256, split = 1;
    int kind = 0;   // 0 generic, 1 decode, 2 prefill
    uint32_t bm = 0, bn = 0;
};

static int w4_plan(t0_runtime* rt, const t0_w4a16_desc* d, W4Plan& pl) {
    const uint32_t M = d->m, N = d->n, K = d->k, gs = d->group_size;
    if (!M || !N || !K || !gs) return fail(T0_ERR_INVALID, "empty W4A16 problem");
    if (K % 8 || gs % 8 || K % gs) return fail(T0_ERR_INVALID, "K %% 8, gs %% 8 and K %% gs must be 0");
    if (d->zeros && N % 8) return fail(T0_ERR_INVALID, "packed zero points need N %% 8 == 0");
    const uint32_t lda = d->lda ? d->lda : K, ldc = d->ldc ? d->ldc : N;
    const bool align_ok = aligned16(d->a) && aligned16(d->qweight) && lda % 8 == 0 && aligned16(d->c) && ldc % 4 == 0 &&
                          (d->scales % 8) == 0;
    const bool fast = gs == 128 && K % 128 == 0 && align_ok;
    pl = W4Plan();
    if (fast && M <= 64 && N % 8 == 0 && d->scales % 16 == 0 && d->zeros % 4 == 0) {
        const uint32_t mb = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
        const uint32_t kg = 4 / mb;                  // quant groups per pipeline stage
        const uint32_t cus = rt && rt->cu_count > 0 ? (uint32_t)rt->cu_count : 256;
        const uint32_t units = N / 4, G = K / 128;
        // one workgroup per CU, each streaming an even share of the 4-column
        // units (at least a 16-column tile's worth) over the whole K ...
        uint32_t wgs = std::min<uint32_t>(cus, (N + 15) / 16);
        uint32_t tiles = (4 * ((units + wgs - 1) / wgs) + 15) / 16;
        if (tiles > 4) {                             // ... or 64-column ranges
            wgs = (units + 15) / 16;
            tiles = 4;
        }
        uint32_t sk = d->split_k;
        if (!sk) {
            // narrow N: split K over otherwise idle CUs, a stage or more each
            sk = 1;
            while ((uint64_t)wgs * sk * 2 <= cus && G % (2 * sk) == 0 && G / (2 * sk) >= kg) sk *= 2;
        }
        if (G % sk)
            return fail(T0_ERR_INVALID, "split_k %u must divide the %u quant groups of K", sk, G);
        char b[64];
        snprintf(b, sizeof b, "t0k_w4a16_decode_t%u_mb%u", tiles, mb);
        pl.sym = b;
        pl.gx = wgs;
        pl.gy = sk;
        pl.threads = 64 * t0_w4_decode_waves((int)tiles, (int)mb);
        pl.split = sk;
        pl.kind = 1;
        pl.bm = 16 * mb;
        pl.bn = 16 * tiles;
        return T0_OK;
    }
    if (fast && M > 64 && N % 8 == 0 && (!d->scales_f32 || d->scales % 16 == 0)) {
        const bool big = M >= 1024;
        pl.bm = 128;
        pl.bn = big ? 256 : 128;
        char b[64];
        // 128x256 tiles on 8 waves with three stages in LDS, 128x128 on 4
        snprintf(b, sizeof b, big ? "t0k_w4a16_prefill_%ux%u_w1x8_s3" : "t0k_w4a16_prefill_%ux%u_w2x2_s2", pl.bm,
                 pl.bn);
        pl.sym = b;
        pl.gx = ((M + pl.bm - 1) / pl.bm) * ((N + pl.bn - 1) / pl.bn);
        pl.threads = big ? 512 : 256;
        pl.kind = 2;
        return T0_OK;
    }
    pl.sym = "t0k_w4a16_generic";
    pl.gx = (N + 255) / 256;
    pl.gy = M;
    pl.threads = 256;
    pl.kind = 0;
    return T0_OK;
}

int t0_w4a16_plan(t0_runtime* rt, const t0_w4a16_desc* d, char* kernel, size_t len, uint32_t* split_k) {
    if (!d) return fail(T0_ERR_INVALID, "null desc");
    W4Plan pl;
    int r = w4_plan(rt, d, pl);
    if (r) return r;
    if (kernel && len) snprintf(kernel, len, "%s", pl.sym.c_str());
    if (split_k) *split_k = pl.split;
    return T0_OK;
}

int t0_w4a16_gemm(t0_runtime* rt, const t0_w4a16_desc* d) {
    if (!rt || !d || !d->a || !d->qweight || !d->scales || !d->c) return fail(T0_ERR_INVALID, "null argument");
    std::lock_guard<std::recursive_mutex> call_lock(rt->call_mu);
    W4Plan pl;
    int r = w4_plan(rt, d, pl);
    if (r) return r;
    r = set_dev(rt);
    if (r) return r;
    t0_w4a16_params p;
    memset(&p, 0, sizeof p);
    p.A = (const void*)d->a;
    p.qweight = (const uint32_t*)d->qweight;
    p.scales = (const void*)d->scales;
    p.zeros = (const uint32_t*)d->zeros;
    p.C = (void*)d->c;
    p.M = d->m; p.N = d->n; p.K = d->k;
    p.lda = d->lda ? d->lda : d->k;
    p.ldc = d->ldc ? d->ldc : d->n;
    p.group_size = d->group_size;
    p.zero_const = d->zero_const;
    p.flags = (d->scales_f32 ? T0_W4_SCALE_F32 : 0) | (d->out_f32 ? T0_W4_OUT_F32 : 0);
    p.split_k = pl.split;
    p.round_wgs = rt->cu_count > 0 ? (uint32_t)rt->cu_count : 256;
    if (!d->zeros && d->zero_const > 15) return fail(T0_ERR_INVALID, "zero_const must be 0..15");
    hipFunction_t f;
    if (pl.kind == 1 && pl.split > 1) {
        r = ensure_ws(rt, (size_t)pl.split * pl.gx * pl.bm * pl.bn * 4);   // [column block][split][tile]
        if (r) return r;
        r = ensure_sem(rt, pl.gx);
        if (r) return r;
        p.workspace = (float*)rt->ws;
        p.semaphores = rt->sem;
    }
    if (pl.kind == 2) {
        // workspace: [G][M] x 16 B, the group row sums of A as the
        // prefill's correction operand; bf16 scales widened to f32 [G][N]
        // (the prefill reads f32 scales); a 2 KiB tail
        const uint32_t G = p.K / 128;
        const size_t r_bytes = ((size_t)G * p.M * 16 + 255) & ~(size_t)255;
        const bool widen = !d->scales_f32;
        r = ensure_ws(rt, r_bytes + (widen ? (size_t)G * p.N * 4 : 0) + 2048);
        if (r) return r;
        p.workspace = (float*)rt->ws;
        if (widen) p.scales_f32 = (float*)((uint8_t*)rt->ws + r_bytes);
        hipFunction_t fr;
        r = get_fn(rt, "t0k_w4a16_rowsum", &fr);
        if (r) return r;
        const uint32_t sum_blocks = (p.M * ((G + 7) / 8) + 3) / 4;
        const uint32_t widen_blocks = widen ? (uint32_t)(((uint64_t)G * p.N / 4 + 255) / 256) : 0;
        r = launch(rt, fr, sum_blocks + widen_blocks, 1, 1, 256, p);
        if (r) return r;
        if (widen) p.scales = p.scales_f32;
        p.flags |= T0_W4_SCALE_F32;
    }
    r = get_fn(rt, pl.sym, &f);
    if (r) return r;
    return launch(rt, f, pl.gx, pl.gy, 1, pl.threads, p);
}

// --------------------------------------------------------- small kernels --
int t0_splitk_reduce(t0_runtime* rt, uint64_t src, uint64_t stride, uint32_t planes, uint64_t dst, uint32_t m,
                     uint32_t n, int out_bf16) {
    if (!rt || !src || !dst) return fail(T0_ERR_INVALID, "null argument");
    int r = set_dev(rt);
    if (r) return r;
    hipFunction_t f;
    r = get_fn(rt, "t0k_splitk_reduce", &f);
    if (r) return r;
    t0_aux_params p;
    memset(&p, 0, sizeof p);
    p.src = (const void*)src; p.dst = (void*)dst;
    p.m = m; p.n = n; p.ld_src = n; p.ld_dst = n;
    p.planes = planes; p.plane_stride = stride;
    p.flags = out_bf16 ? T0_GEMM_OUT_BF16 : 0;
    return launch(rt, f, (uint32_t)(((uint64_t)m * n + 255) / 256), 1, 1, 256, p);
}

int t0_f32_to_bf16(t0_runtime* rt, uint64_t src, uint64_t dst, uint64_t count) {
    if (!rt || !src || !dst) return fail(T0_ERR_INVALID, "null argument");
    if (count > 0xFFFFFFFFull) return fail(T0_ERR_INVALID, "count too large");
    int r = set_dev(rt);
    if (r) return r;
    hipFunction_t f;
    r = get_fn(rt, "t0k_f32_to_bf16", &f);
    if (r) return r;
    t0_aux_params p;
    memset(&p, 0, sizeof p);
    p.src = (const void*)src; p.dst = (void*)dst;
    p.m = 1; p.n = (uint32_t)count; p.ld_src = p.n; p.ld_dst = p.n;
    return launch(rt, f, (uint32_t)((count + 255) / 256), 1, 1, 256, p);
}

int t0_copy_device(t0_runtime* rt, uint64_t src, uint64_t dst, uint64_t bytes) {
    if (!rt || !src || !dst || bytes % 16 || (src | dst) % 16) return fail(T0_ERR_INVALID, "16-byte aligned copy only");
    int r = set_dev(rt);
    if (r) return r;
    hipFunction_t f;
    r = get_fn(rt, "t0k_copy_b128", &f);
    if (r) return r;
    t0_aux_params p;
    memset(&p, 0, sizeof p);
    p.src = (const void*)src; p.dst = (void*)dst;
    p.plane_stride = bytes / 16;
    return launch(rt, f, (uint32_t)((bytes / 16 + 255) / 256), 1, 1, 256, p);
}

int t0_floor_stream_read(t0_runtime* rt, uint64_t src, uint64_t bytes, uint64_t sink, uint32_t workgroups,
                         uint32_t threads) {
    if (!rt || !src || !sink || bytes % 16 || src % 16 || bytes >= (1ull << 32))
        return fail(T0_ERR_INVALID, "16-byte aligned source under 4 GiB and a sink of workgroups * 4 bytes");
    if (!workgroups || !threads || threads % 64 || threads > 1024) return fail(T0_ERR_INVALID, "bad launch shape");
    int r = set_dev(rt);
    if (r) return r;
    hipFunction_t f;
    r = get_fn(rt, "t0k_stream_read", &f);
    if (r) return r;
    t0_aux_params p;
    memset(&p, 0, sizeof p);
    p.src = (const void*)src;
    p.dst = (void*)sink;
    p.plane_stride = bytes / 16;
    p.m = 0x9E3779B9u;
    return launch(rt, f, workgroups, 1, 1, threads, p);
}

int t0_floor_empty(t0_runtime* rt, uint32_t workgroups, uint32_t threads) {
    if (!rt || !workgroups || !threads || threads % 64 || threads > 1024) return fail(T0_ERR_INVALID, "bad launch shape");
    int r = set_dev(rt);
    if (r) return r;
    hipFunction_t f;
    r = get_fn(rt, "t0k_empty", &f);
    if (r) return r;
    t0_aux_params p;
    memset(&p, 0, sizeof p);
    return launch(rt, f, workgroups, 1, 1, threads, p);
}

int t0_floor_tile_read(t0_runtime* rt, const t0_gemm_config* cfg, const t0_gemm_desc* d, int mode) {
    if (!rt || !d || !d->a || !d->b) return fail(T0_ERR_INVALID, "null argument");
    if (mode < 1 || mode > 3) return fail(T0_ERR_INVALID, "mode 1 (A slices), 2 (B slices) or 3 (both)");
    if (!d->m || !d->n || !d->k || d->transpose > T0_NN) return fail(T0_ERR_INVALID, "bad shape or layout");
    t0_gemm_config c;
    if (cfg) c = *cfg;
    else {
        int r = t0_gemm_select(rt, d, &c);
        if (r) return r;
    }
    const uint32_t sk = split_of(c);
    if (c.tile_m % 8 || c.tile_n % 8 || !c.tile_m || !c.tile_n || c.tile_m + c.tile_n > 512)
        return fail(T0_ERR_INVALID, "tile_m and tile_n multiples of 8 with tile_m + tile_n <= 512");
    if (d->k % (64 * sk)) return fail(T0_ERR_INVALID, "K must be a multiple of 64 * split_k");
    const bool nt = d->transpose == T0_NT;
    const uint64_t lda = d->lda ? d->lda : d->k, ldb = d->ldb ? d->ldb : (nt ? d->k : d->n);
    if (lda < d->k || ldb < (nt ? d->k : d->n)) return fail(T0_ERR_INVALID, "leading dimension below the row length");
    if (!aligned16(d->a) || !aligned16(d->b) || lda % 8 || ldb % 8)
        return fail(T0_ERR_INVALID, "16-byte aligned operands with lda %% 8 == 0 and ldb %% 8 == 0");
    if ((uint64_t)d->m * lda * 2 >= (1ull << 32) || (uint64_t)(nt ? d->n : d->k) * ldb * 2 >= (1ull << 32))
        return fail(T0_ERR_INVALID, "operands must stay under 4 GiB");
    const uint64_t tiles = (uint64_t)((d->m + c.tile_m - 1) / c.tile_m) * ((d->n + c.tile_n - 1) / c.tile_n);
    if (tiles * sk > 0x7FFFFFFFu) return fail(T0_ERR_INVALID, "too many workgroups");
    int r = set_dev(rt);
    if (r) return r;
    hipFunction_t f;
    r = get_fn(rt, "t0k_tile_read", &f);
    if (r) return r;
    t0_tile_read_params p;
    memset(&p, 0, sizeof p);
    p.A = (const void*)d->a;
    p.B = (const void*)d->b;
    p.M = d->m; p.N = d->n; p.K = d->k;
    p.lda = (uint32_t)lda; p.ldb = (uint32_t)ldb;
    p.tile_m = c.tile_m; p.tile_n = c.tile_n; p.split_k = sk;
    p.b_nt = nt;
    p.mode = (uint32_t)mode;
    return launch(rt, f, (uint32_t)(tiles * sk), 1, 1, 256, p);
}

int t0_floor_mfma(t0_runtime* rt, uint64_t operands, uint64_t out, uint32_t workgroups, uint32_t mfma_per_wave) {
    if (!rt || !operands || !out || operands % 16 || out % 8) return fail(T0_ERR_INVALID, "null or misaligned buffer");
    if (!workgroups || !mfma_per_wave || mfma_per_wave % 16)
        return fail(T0_ERR_INVALID, "workgroups > 0 and mfma_per_wave a positive multiple of 16");
    int r = set_dev(rt);
    if (r) return r;
    hipFunction_t f;
    r = get_fn(rt, "t0k_mfma_issue", &f);
    if (r) return r;
    t0_aux_params p;
    memset(&p, 0, sizeof p);
    p.src = (const void*)operands;
    p.dst = (void*)out;
    p.m = mfma_per_wave / 8;
    p.n = 0x7FBADBADu;   // a signalling-NaN pattern no f32 sum produces
    return launch(rt, f, workgroups, 1, 1, 512, p);
}

int t0_floor_lds(t0_runtime* rt, int mode, uint64_t src, uint64_t out, uint32_t workgroups, uint32_t threads,
                 uint32_t rounds) {
    static const char* const syms[] = {"t0k_lds_read_b128", "t0k_lds_read_tr16", "t0k_lds_dma"};
    if (!rt || !out || out % 8 || mode < 0 || mode > 2 || (mode == 2 && (!src || src % 16)))
        return fail(T0_ERR_INVALID, "bad arguments (mode 2 needs a 16-byte aligned 64 KiB source)");
    if (!workgroups || !threads || threads % 64 || threads > 1024 || !rounds)
        return fail(T0_ERR_INVALID, "bad launch shape");
    int r = set_dev(rt);
    if (r) return r;
    hipFunction_t f;
    r = get_fn(rt, syms[mode], &f);
    if (r) return r;
    t0_aux_params p;
    memset(&p, 0, sizeof p);
    p.src = (const void*)src;
    p.dst = (void*)out;
    p.m = rounds;
    p.n = 0xDEADBEEFu;   // never equal to the xor of the LDS contents
    return launch(rt, f, workgroups, 1, 1, threads, p);
}

int t0_unpad_2d(t0_runtime* rt, uint64_t padded, uint64_t out, uint32_t m, uint32_t n, uint32_t n_pad) {
    if (!rt || !padded || !out || n_pad < n) return fail(T0_ERR_INVALID, "bad arguments");
    int r = set_dev(rt);
    if (r) return r;
    hipFunction_t f;
    r = get_fn(rt, "t0_unpad_2d", &f);
    if (r) return r;
    t0_aux_params p;
    memset(&p, 0, sizeof p);
    p.src = (const void*)padded; p.dst = (void*)out;
    p.m = m; p.n = n; p.ld_src = n_pad; p.ld_dst = n;
    return launch(rt, f, (uint32_t)(((uint64_t)m * n + 255) / 256), 1, 1, 256, p);
}

}  // extern "C"

// ------------------------------------------------------ bf16 matmul path --
// src/ignis/ops/bf16_matmul.rs converts f32 operands to bf16 on the CPU,
// transposes W / X / dY on the CPU and pads every dimension to the tile.
// Here each operand is converted once by a GPU kernel into the runtime's
// staging buffer, with rows padded to 8 elements (zeros) so that the tiled
// kernels apply at any m / k / n; the output is written straight into the
// caller's dense f32 buffer (no padded output, no unpad pass).
namespace {

uint32_t round8(uint32_t x) { return (x + 7u) & ~7u; }
size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// dst[rows_pad][ld_dst] bf16 = RNE(src[m][n] f32, row stride ld_src), zero padded.
int stage_cvt(t0_runtime* rt, uint64_t src, uint32_t ld_src, uint32_t m, uint32_t n, uint64_t dst, uint32_t ld_dst,
              uint32_t rows_pad) {
    hipFunction_t f;
    int r = get_fn(rt, "t0k_cvt_pad_bf16", &f);
    if (r) return r;
    t0_aux_params p;
    memset(&p, 0, sizeof p);
    p.src = (const void*)src; p.dst = (void*)dst;
    p.m = m; p.n = n; p.ld_src = ld_src; p.ld_dst = ld_dst; p.rows_pad = rows_pad;
    p.flags = (aligned16(src) && ld_src % 4 == 0) ? T0_AUX_SRC_VEC4 : 0;
    const uint64_t chunks = (uint64_t)rows_pad * (ld_dst / 8);
    return launch(rt, f, (uint32_t)((chunks + 255) / 256), 1, 1, 256, p);
}

// dst[rows_pad][ld_dst] bf16 = RNE(src[m][n] f32)^T, zero padded.
int stage_cvt_t(t0_runtime* rt, uint64_t src, uint32_t ld_src, uint32_t m, uint32_t n, uint64_t dst, uint32_t ld_dst,
                uint32_t rows_pad) {
    hipFunction_t f;
    int r = get_fn(rt, "t0k_cvt_t_bf16", &f);
    if (r) return r;
    t0_aux_params p;
    memset(&p, 0, sizeof p);
    p.src = (const void*)src; p.dst = (void*)dst;
    p.m = m; p.n = n; p.ld_src = ld_src; p.ld_dst = ld_dst; p.rows_pad = rows_pad;
    p.flags = (aligned16(src) && ld_src % 4 == 0) ? T0_AUX_SRC_VEC4 : 0;
    const uint64_t tiles = (uint64_t)((ld_dst + 63) / 64) * ((rows_pad + 63) / 64);
    return launch(rt, f, (uint32_t)tiles, 1, 1, 256, p);
}

// One f32-out GEMM on staged operands, with the config t0_gemm would pick.
int staged_gemm(t0_runtime* rt, uint64_t a, uint32_t lda, uint64_t b, uint32_t ldb, uint64_t c, uint32_t ldc,
                uint32_t m, uint32_t n, uint32_t k, bool nn) {
    t0_gemm_desc d;
    memset(&d, 0, sizeof d);
    d.a = a; d.b = b; d.c = c;
    d.m = m; d.n = n; d.k = k;
    d.lda = lda; d.ldb = ldb; d.ldc = ldc;
    d.transpose = nn ? T0_NN : T0_NT;
    d.out_dtype = T0_OUT_F32;
    t0_gemm_config cfg;
    int r = t0_gemm_select(rt, &d, &cfg);
    if (r) return r;
    const GemmInstance* g = instance_for(cfg);
    if (!g) return fail(T0_ERR_INFEASIBLE, "%s: no gfx950 kernel", config_name(cfg).c_str());
    t0_gemm_params p;
    r = desc_to_params(&d, cfg, p);
    if (r) return r;
    if (p.split_k > 1 && !fast_ok(p, nn, true)) p.split_k = 1, p.flags &= ~T0_GEMM_FIXUP;
    return run_gemm_params(rt, g, nn, p, 0, true);
}

int matmul_args(t0_runtime* rt, uint64_t p0, uint64_t p1, uint64_t p2, uint32_t m, uint32_t k, uint32_t n) {
    if (!rt || !p0 || !p1 || !p2) return fail(T0_ERR_INVALID, "null argument");
    if (!m || !k || !n) return fail(T0_ERR_INVALID, "empty matmul m=%u k=%u n=%u", m, k, n);
    if (m > 0x7FFFFFF8u || k > 0x7FFFFFF8u || n > 0x7FFFFFF8u) return fail(T0_ERR_INVALID, "dimension too large");
    return set_dev(rt);
}

}  // namespace

extern "C" {

int t0_bf16_matmul(t0_runtime* rt, uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t k, uint32_t n) {
    int r = matmul_args(rt, x, w, y, m, k, n);
    if (r) return r;
    std::lock_guard<std::recursive_mutex> call_lock(rt->call_mu);
    const uint32_t k8 = round8(k), n8 = round8(n);
    const size_t a_bytes = align256((size_t)m * k8 * 2), b_bytes = align256((size_t)k8 * n8 * 2);
    r = ensure_stage(rt, a_bytes + b_bytes);
    if (r) return r;
    const uint64_t sa = (uint64_t)rt->stage, sb = sa + a_bytes;
    if ((r = stage_cvt(rt, x, k, m, k, sa, k8, m))) return r;        // X  -> [m][k8]
    if ((r = stage_cvt(rt, w, n, k, n, sb, n8, k8))) return r;       // W  -> [k8][n8], rows k.. zero
    return staged_gemm(rt, sa, k8, sb, n8, y, n, m, n, k8, true);    // NN: no transpose of W
}

int t0_bf16_matmul_backward_data(t0_runtime* rt, uint64_t dy, uint64_t w, uint64_t dx, uint32_t m, uint32_t k,
                                 uint32_t n) {
    int r = matmul_args(rt, dy, w, dx, m, k, n);
    if (r) return r;
    std::lock_guard<std::recursive_mutex> call_lock(rt->call_mu);
    const uint32_t n8 = round8(n);
    const size_t a_bytes = align256((size_t)m * n8 * 2), b_bytes = align256((size_t)k * n8 * 2);
    r = ensure_stage(rt, a_bytes + b_bytes);
    if (r) return r;
    const uint64_t sa = (uint64_t)rt->stage, sb = sa + a_bytes;
    if ((r = stage_cvt(rt, dy, n, m, n, sa, n8, m))) return r;       // dY -> [m][n8]
    if ((r = stage_cvt(rt, w, n, k, n, sb, n8, k))) return r;        // W  -> [k][n8]: the NT operand as is
    return staged_gemm(rt, sa, n8, sb, n8, dx, k, m, k, n8, false);
}

int t0_bf16_matmul_backward_weight(t0_runtime* rt, uint64_t x, uint64_t dy, uint64_t dw, uint32_t m, uint32_t k,
                                   uint32_t n) {
    int r = matmul_args(rt, x, dy, dw, m, k, n);
    if (r) return r;
    std::lock_guard<std::recursive_mutex> call_lock(rt->call_mu);
    const uint32_t m8 = round8(m), n8 = round8(n);
    const size_t a_bytes = align256((size_t)k * m8 * 2), b_bytes = align256((size_t)m8 * n8 * 2);
    r = ensure_stage(rt, a_bytes + b_bytes);
    if (r) return r;
    const uint64_t sa = (uint64_t)rt->stage, sb = sa + a_bytes;
    if ((r = stage_cvt_t(rt, x, k, m, k, sa, m8, k))) return r;      // X^T -> [k][m8]
    if ((r = stage_cvt(rt, dy, n, m, n, sb, n8, m8))) return r;      // dY  -> [m8][n8], rows m.. zero
    return staged_gemm(rt, sa, m8, sb, n8, dw, n, k, n, m8, true);
}

int t0_bf16_matmul_with_wt_bf16(t0_runtime* rt, uint64_t x, uint64_t wt, uint64_t y, uint32_t m, uint32_t k,
                                uint32_t n) {
    int r = matmul_args(rt, x, wt, y, m, k, n);
    if (r) return r;
    std::lock_guard<std::recursive_mutex> call_lock(rt->call_mu);
    const uint32_t k8 = round8(k);
    const size_t a_bytes = align256((size_t)m * k8 * 2);
    r = ensure_stage(rt, a_bytes);
    if (r) return r;
    const uint64_t sa = (uint64_t)rt->stage;
    if ((r = stage_cvt(rt, x, k, m, k, sa, k8, m))) return r;        // X -> [m][k8]
    // WT is the caller's dense [n][k] bf16: the contraction stays k (a k that
    // is not a multiple of 8 takes the generic kernel).
    return staged_gemm(rt, sa, k8, wt, k, y, n, m, n, k, false);
}

}  // extern "C"

// ------------------------------------------------- decode neighbours ----
// Residual add + RMSNorm in front of the projections: the reference's fused
// kernel (src/t0/ffn_fused_kernels.rs), the Ignis ops built on it
// (src/ignis/ops/fused_rmsnorm_gemm.rs) with an INT4 or a dense weight.
namespace {

int launch_rmsnorm(t0_runtime* rt, uint64_t res, uint64_t hid, uint64_t gamma, uint64_t out, uint64_t x2_out,
                   uint32_t rows, uint32_t d, uint32_t ld_out, float eps, bool out_bf16) {
    hipFunction_t f;
    int r = get_fn(rt, "t0k_rmsnorm", &f);
    if (r) return r;
    t0_rmsnorm_params p;
    memset(&p, 0, sizeof p);
    p.res = (const float*)res; p.hid = (const float*)hid; p.gamma = (const float*)gamma;
    p.out = (void*)out; p.x2_out = (float*)x2_out;
    p.rows = rows; p.d = d; p.ld_out = ld_out; p.out_bf16 = out_bf16; p.eps = eps;
    // 16-byte chunks: rows of a multiple of 4 elements, every row start 16-byte
    // aligned on the inputs and 8/16-byte aligned on the output
    const bool vec = d % 4 == 0 && ld_out % 4 == 0 && aligned16(res) && aligned16(hid) && aligned16(gamma) &&
                     aligned16(x2_out) && (out_bf16 ? aligned8(out) : aligned16(out));
    p.flags = vec ? T0_RMSNORM_VEC4 : 0;
    return launch(rt, f, rows, 1, 1, 256, p);
}

}  // namespace

extern "C" {

int t0_ffn_fused_rmsnorm_gemm(t0_runtime* rt, uint64_t residual, uint64_t hidden, uint64_t gamma, uint64_t weight,
                              uint64_t output, uint32_t m, uint32_t d, float eps) {
    if (!rt || !residual || !hidden || !gamma || !weight || !output) return fail(T0_ERR_INVALID, "null argument");
    if (!m || !d) return fail(T0_ERR_INVALID, "empty problem m=%u d=%u", m, d);
    int r = set_dev(rt);
    if (r) return r;
    hipFunction_t f;
    r = get_fn(rt, "ffn_fused_rmsnorm_gemm", &f);
    if (r) return r;
    t0_ffn_params p;
    p.residual = (const float*)residual; p.hidden = (const float*)hidden; p.gamma = (const float*)gamma;
    p.weight = (const float*)weight; p.output = (float*)output; p.D = d; p.eps = eps;
    return launch(rt, f, m, 1, 1, 128, p);
}

int t0_rmsnorm(t0_runtime* rt, uint64_t residual, uint64_t hidden, uint64_t gamma, uint64_t out, uint64_t x2_out,
               uint32_t rows, uint32_t d, uint32_t ld_out, float eps, int out_bf16) {
    if (!rt || !residual || !gamma || !out) return fail(T0_ERR_INVALID, "null argument");
    if (!rows || !d) return fail(T0_ERR_INVALID, "empty problem rows=%u d=%u", rows, d);
    if (ld_out == 0) ld_out = d;
    if (ld_out < d) return fail(T0_ERR_INVALID, "ld_out %u < d %u", ld_out, d);
    int r = set_dev(rt);
    if (r) return r;
    return launch_rmsnorm(rt, residual, hidden, gamma, out, x2_out, rows, d, ld_out, eps, out_bf16 != 0);
}

int t0_rmsnorm_w4a16(t0_runtime* rt, const t0_w4a16_desc* d, const t0_rmsnorm_desc* nd) {
    if (!rt || !d || !nd || !nd->residual || !nd->gamma || !d->qweight || !d->scales || !d->c)
        return fail(T0_ERR_INVALID, "null argument");
    std::lock_guard<std::recursive_mutex> call_lock(rt->call_mu);
    if (!d->m || !d->k) return fail(T0_ERR_INVALID, "empty problem");
    int r = set_dev(rt);
    if (r) return r;
    const bool vec_ok = aligned8(nd->residual) && aligned8(nd->hidden) && aligned8(nd->gamma) && aligned8(nd->x2_out);
    if (d->m == 1 && vec_ok) {
        t0_w4a16_desc d1 = *d;
        d1.a = 0; d1.lda = 0; d1.split_k = 1;        // one partition: every workgroup sees the whole row
        W4Plan pl;
        r = w4_plan(rt, &d1, pl);
        if (r) return r;
        if (pl.kind == 1) {
            if (!d->zeros && d->zero_const > 15) return fail(T0_ERR_INVALID, "zero_const must be 0..15");
            const uint32_t tiles = pl.bn / 16;
            char sym[64];
            snprintf(sym, sizeof sym, "t0k_w4a16_decode_norm_t%u", tiles);
            hipFunction_t f;
            r = get_fn(rt, sym, &f);
            if (r) return r;
            t0_w4a16_params p;
            memset(&p, 0, sizeof p);
            p.qweight = (const uint32_t*)d->qweight;
            p.scales = (const void*)d->scales;
            p.zeros = (const uint32_t*)d->zeros;
            p.C = (void*)d->c;
            p.M = 1; p.N = d->n; p.K = d->k;
            p.lda = d->k;
            p.ldc = d->ldc ? d->ldc : d->n;
            p.group_size = d->group_size;
            p.zero_const = d->zero_const;
            p.flags = (d->scales_f32 ? T0_W4_SCALE_F32 : 0) | (d->out_f32 ? T0_W4_OUT_F32 : 0);
            p.split_k = 1;
            p.norm_res = (const float*)nd->residual;
            p.norm_hid = (const float*)nd->hidden;
            p.norm_gamma = (const float*)nd->gamma;
            p.norm_x2 = (float*)nd->x2_out;
            p.norm_eps = nd->eps;
            return launch(rt, f, pl.gx, 1, 1, 64 * t0_w4_decode_norm_waves((int)tiles), p);
        }
    }
    // any other shape: normalised bf16 activations into the staging buffer,
    // then the W4A16 GEMM on them
    const size_t a_bytes = align256((size_t)d->m * d->k * 2);
    r = ensure_stage(rt, a_bytes);
    if (r) return r;
    const uint64_t sa = (uint64_t)rt->stage;
    r = launch_rmsnorm(rt, nd->residual, nd->hidden, nd->gamma, sa, nd->x2_out, d->m, d->k, d->k, nd->eps, true);
    if (r) return r;
    t0_w4a16_desc d2 = *d;
    d2.a = sa;
    d2.lda = d->k;
    return t0_w4a16_gemm(rt, &d2);
}

int t0_rmsnorm_matmul(t0_runtime* rt, uint64_t residual, uint64_t hidden, uint64_t gamma, uint64_t w, uint64_t y,
                      uint64_t x2_out, uint32_t m, uint32_t k, uint32_t n, float eps) {
    int r = matmul_args(rt, residual, w, y, m, k, n);
    if (r) return r;
    std::lock_guard<std::recursive_mutex> call_lock(rt->call_mu);
    if (!gamma) return fail(T0_ERR_INVALID, "null gamma");
    const uint32_t k8 = round8(k), n8 = round8(n);
    const size_t a_bytes = align256((size_t)m * k8 * 2), b_bytes = align256((size_t)k8 * n8 * 2);
    r = ensure_stage(rt, a_bytes + b_bytes);
    if (r) return r;
    const uint64_t sa = (uint64_t)rt->stage, sb = sa + a_bytes;
    if ((r = launch_rmsnorm(rt, residual, hidden, gamma, sa, x2_out, m, k, k8, eps, true))) return r;   // -> [m][k8]
    if ((r = stage_cvt(rt, w, n, k, n, sb, n8, k8))) return r;                                         // W -> [k8][n8]
    return staged_gemm(rt, sa, k8, sb, n8, y, n, m, n, k8, true);
}

}  // extern "C"

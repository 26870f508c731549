// w4a16.hip -- INT4-weight x bf16-activation GEMMs for gfx950, and the
// reference's standalone INT4 dequant kernels.
//
// Weight operand (W4):
//   qweight [N][K/8] u32   -- the reference's GPTQ packing (src/t0/quant_kernels.rs:3-20,
//                             :191-199): row n holds k at bits 4*(k%8) of word k/8.
//   scales  [G][N]         -- bf16 (or f32), G = K / group_size, n contiguous.
//   zeros   [G][N/8] u32   -- 4-bit zero points, column n at bits 4*(n%8);
//                             or none, with a constant zero point.
//   w(n,k) = (q(n,k) - z(n,g)) * s(n,g)      (src/t0/quant_kernels.rs:365-372)
//
// Fused dequant, exact: a nibble pair becomes two bf16 of value 128 + q (an
// integer in [128,143], exact in bf16) with one v_perm and one v_and_or; MFMA
// accumulates T = sum a*(128 + q) - (128 + z) * sum a over a quant group (the
// zero-point term from the activations' row sums: per decode tile, or as one
// more MFMA block in the prefill); the group's result s * T is applied in f32.
// So the weight value the GEMM uses is exactly (q - z) * s and the weights
// cross HBM once, at 4 bits.
#include "common.h"

namespace t0 {

T0_DEV uint32_t zero_of(const t0_w4a16_params& p, uint32_t g, uint32_t n) {
    if (!p.zeros) return p.zero_const;
    return (p.zeros[(size_t)g * (p.N / 8) + n / 8] >> (4 * (n % 8))) & 0xFu;
}

T0_DEV float scale_of(const t0_w4a16_params& p, uint32_t g, uint32_t n) {
    const size_t i = (size_t)g * p.N + n;
    if (p.flags & T0_W4_SCALE_F32) return ((const float*)p.scales)[i];
    return bf16_bits_to_f32(((const uint16_t*)p.scales)[i]);
}

T0_DEV void store_out4(const t0_w4a16_params& p, uint32_t m, uint32_t n, f32x4_t v) {
    if (m >= p.M) return;
    if (p.flags & T0_W4_OUT_F32) {
        float* dst = (float*)p.C + (size_t)m * p.ldc + n;
        if (n + 3 < p.N) *(f32x4_t*)dst = v;
        else for (int e = 0; e < 4; e++) if (n + e < p.N) dst[e] = v[e];
    } else {
        uint16_t* dst = (uint16_t*)p.C + (size_t)m * p.ldc + n;
        if (n + 3 < p.N) *(u32x2_t*)dst = u32x2_t{pack2_bf16_rne(v[0], v[1]), pack2_bf16_rne(v[2], v[3])};
        else for (int e = 0; e < 4; e++) if (n + e < p.N) dst[e] = (uint16_t)(pack2_bf16_rne(v[e], 0.f) & 0xFFFFu);
    }
}

// ---------------------------------------------------------------------------
// Decode: small M (<= 16*MB), HBM bound.
//   grid = (WG, split_k), block = 64*WAVES; the host sizes WG to the CU count,
//   so each workgroup (alone on its CU) streams one contiguous column range
//   over its whole K slice and, with split_k == 1, no partial sums leave the
//   CU.  Workgroup i owns columns [c0, c1): the 4-column units of N split
//   evenly over gridDim.x, at most 16*TILES columns.
//   Wave w owns the quant groups w, w + WAVES, w + 2*WAVES, ... of the
//   workgroup's K slice and loads everything a group needs by itself, so no
//   wave waits for another until the final sum:
//     A  [16*MB rows][256 B] of the group -> the wave's own LDS slot by
//        buffer_load ... lds (rows past M read zeros), 16-B chunks
//        XOR-swizzled by row
//     W  -> VGPRs: lane l (c = l%16, h = l/16) loads, per tile t, the 16 bytes
//        of column c0 + 16t + c holding k = 128g + 32h + [0, 32)
//     S, Z -> the same slot by 4-byte DMAs: the group's scales of columns
//        [c0, c1) and the zero-point words holding them
//   Groups go in rounds of SLOTS (up to 4, as LDS and registers allow): every load of the
//   round is issued before the first group is consumed, the weight loads of
//   all the round's groups first (they come from HBM; the activations, read
//   by every workgroup, from L2), then group by group the LDS loads.
//   Each group issues a fixed number of loads, so an explicit vmcnt wait
//   lets a group's LDS data be read while the later groups' loads are still
//   in flight; the DMAs are compiler-visible (buffer-load-to-LDS builtin), so
//   the compiler's own waits for the weight registers count them too and
//   group j computes while group j + 1 is still arriving.
//   Per group, v_mfma_f32_16x16x32_bf16(W, A) with W = bf16(128 + q) gives
//   lane l T = sum_k a*(128 + q) for outputs (m = 16mb + c,
//   n = c0 + 16t + 4h + r), r = 0..3; a ones-MFMA gives sum_k a, and
//   acc += s * (T - (128 + z) * sum a).  The waves are summed in wave order
//   through LDS at the end.
//   split_k > 1 (narrow N): partition blockIdx.y covers G/split_k groups; the
//   workgroup's tile goes to the workspace [i][split][tile] and the last
//   partition to arrive adds them in split order.
// Requires: group_size == 128, K % 128 == 0, (K/128) % split_k == 0,
//           N % 8 == 0, lda % 8 == 0, 16-byte aligned A / qweight / scales.
// ---------------------------------------------------------------------------

// 8 nibbles of one u32 (k = 0..7) -> 8 bf16 of value 128 + q, in k order:
// dword i = bytes (w.byte_i, -, (w >> 4).byte_i, -) masked to the low nibbles
// and or-ed into 0x4300 (= 128.0).
// The mask-and-insert is one v_and_or_b32: a VOP3 here cannot take a
// literal, so both constants come in registers, the mask in an SGPR
// (m000f = sgpr_const(0x000F000F)) and 0x43004300 in a VGPR.  It is plain C,
// not inline asm: an MFMA that reads a VALU result needs two wait states,
// which the compiler inserts only after instructions it emitted itself.
T0_DEV bf16x8_t unpack8_128(uint32_t w, uint32_t bits4300, uint32_t m000f) {
    const uint32_t t = w >> 4;
    u32x4_t r;
#pragma unroll
    for (int i = 0; i < 4; i++)
        r[i] = (__builtin_amdgcn_perm(t, w, 0x0C000C00u | ((4u + i) << 16) | (uint32_t)i) & m000f) | bits4300;
    return __builtin_bit_cast(bf16x8_t, r);
}

template <int TILES, int MB, bool NORM = false>
struct W4DecCfg {
    // as many waves as the per-group registers allow (16 waves: <= 128 VGPRs)
    static constexpr int WAVES = NORM ? t0_w4_decode_norm_waves(TILES) : t0_w4_decode_waves(TILES, MB);
    static constexpr int NT = 64 * WAVES;
    static constexpr int GROUP_A = 16 * MB * 256;         // A bytes of one group
    static constexpr int A_DMA = GROUP_A / 1024;          // 4-row DMA blocks per group
    // a wave's slot: A, then the group's scales (<= 256 B) and zero-point words (<= 64 B)
    static constexpr int S_OFF = GROUP_A, Z_OFF = GROUP_A + 256, WAVE_SLOT = GROUP_A + 512;
    static constexpr int SLOT_BYTES = WAVES * WAVE_SLOT;  // one group per wave
    // groups in flight per wave: as many as LDS holds, at most 2 under the
    // 128-VGPR budget of 16 waves, else 4
    static constexpr int SLOTS_LDS = 156 * 1024 / SLOT_BYTES;
    static constexpr int SLOTS = SLOTS_LDS < (WAVES >= 16 ? 2 : 4) ? SLOTS_LDS : (WAVES >= 16 ? 2 : 4);
    static constexpr int OUT_SLOTS = TILES * MB * 64;     // 16-byte outputs per workgroup
    static constexpr int MAX_GROUP_LOADS = A_DMA + 2 + TILES;   // VMEM ops per group: A, S, Z, W
    static_assert(SLOTS * MAX_GROUP_LOADS < 64, "vmcnt range");
    static_assert(SLOTS >= 1 && SLOTS * SLOT_BYTES <= 156 * 1024, "LDS");
    static_assert(TILES <= 4, "scale / zero-point DMA covers 64 columns");
    static_assert(OUT_SLOTS * 16 + 4 <= WAVE_SLOT && WAVE_SLOT % 16 == 0,
                  "a wave's partials and sum of squares fit its own slot-0 area");
};

template <int TILES, int MB, bool ZP, bool SF32, bool NORM>
__device__ __forceinline__ void w4_decode_body(const t0_w4a16_params& p, LDS_AS uint8_t* const (&slot)[4],
                                               uint32_t* s_last) {
    using G = W4DecCfg<TILES, MB, NORM>;
    static_assert(!NORM || MB == 1, "the fused RMSNorm decode takes one activation row");
    typedef __attribute__((address_space(3))) void lds_void;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t K = p.K, N = p.N, M = p.M, sk = p.split_k;
    const uint32_t wg = blockIdx.x, part = blockIdx.y;
    const uint32_t units = N / 4;
    const uint32_t c0 = 4 * (uint32_t)((uint64_t)wg * units / gridDim.x);
    const uint32_t c1 = 4 * (uint32_t)((uint64_t)(wg + 1) * units / gridDim.x);
    const uint32_t GP = K / 128 / sk;                   // groups in this partition
    const uint32_t g_begin = part * GP;
    const uint32_t c = lane & 15, h = lane >> 4;
    constexpr uint32_t ES = SF32 ? 4 : 2;               // scale bytes
    // VMEM ops per group: A (DMA blocks, or residual / hidden / gamma pairs), S, Z, W
    // Without the norm, every weight load of the round goes out first (the
    // weights come from HBM, the activations from L2), so between two groups'
    // LDS loads there are only LDS loads: A, S, Z.
    constexpr int GROUP_LOADS = (NORM ? 3 : G::A_DMA) + 1 + (ZP ? 1 : 0) + (NORM ? TILES : 0);

    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.scales);
    const __amdgpu_buffer_rsrc_t rz = make_rsrc(ZP ? (const void*)p.zeros : p.scales);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.qweight + (size_t)c0 * (K / 8));

    // ---- loop-invariant per-lane offsets (OOB_OFFSET: the lane reads zeros)
    // A DMA block i of a group: rows 4i + h' (h' = lane / 16), LDS chunk c,
    // global chunk c ^ (row & 15) of the group's 256 bytes.
    uint32_t a_off[G::A_DMA];
#pragma unroll
    for (int i = 0; i < G::A_DMA; i++) {
        const uint32_t row = 4 * i + h;
        a_off[i] = row < M ? row * p.lda * 2 + ((c ^ (row & 15)) * 16) : OOB_OFFSET;
    }
    uint32_t w_row[TILES];
#pragma unroll
    for (int t = 0; t < TILES; t++) w_row[t] = c0 + 16 * t + c < c1 ? (16 * t + c) * (K / 2) + 16 * h : OOB_OFFSET;
    // scales: lane l DMAs the 4 bytes of columns c0 + 2l, +1 (bf16) or c0 + l (f32);
    // zero points: lane l the word c0/8 + l
    const uint32_t zb = c0 / 8;
    const uint32_t s_lane = (SF32 ? c0 + lane : c0 + 2 * lane) < c1 ? (SF32 ? c0 + lane : c0 + 2 * lane) * ES : OOB_OFFSET;
    const uint32_t z_lane = (ZP && lane < 9 && (zb + lane) * 8 < c1) ? (zb + lane) * 4 : OOB_OFFSET;
    // fused RMSNorm: lane l owns k = 128g + 2l, 2l+1 of each group; rows 1..15
    // of the activation slots stay zero, row 0 is written per group
    const __amdgpu_buffer_rsrc_t rn_res = make_rsrc(p.norm_res), rn_hid = make_rsrc(p.norm_hid);
    const __amdgpu_buffer_rsrc_t rn_gam = make_rsrc(p.norm_gamma);
    const uint32_t hid_ok = p.norm_hid != nullptr;
    const bool store_x2 = NORM && p.norm_x2 != nullptr && wg == 0 && part == 0;
    float ssq = 0.0f;                                   // this lane's share of sum(x2^2)
    if constexpr (NORM) {
#pragma unroll
        for (int s = 0; s < G::SLOTS; s++)
#pragma unroll
            for (int q = 0; q < G::GROUP_A / 1024; q++)
                *(LDS_AS u32x4_t*)(slot[s] + wave * G::WAVE_SLOT + q * 1024 + lane * 16) = u32x4_t{0u, 0u, 0u, 0u};
    }
    const float zc_const = 128.0f + (float)p.zero_const;
    const uint32_t bits4300 = __builtin_amdgcn_mov_dpp(0x43004300u, 0xE4, 0xF, 0xF, false);  // in a VGPR
    const uint32_t m000f = sgpr_const(0x000F000Fu);
    const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4_t{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
    f32x4_t acc[TILES][MB];
#pragma unroll
    for (int t = 0; t < TILES; t++)
#pragma unroll
        for (int mb = 0; mb < MB; mb++) acc[t][mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // groups of this wave: g_begin + wave + WAVES * j, j < nj
    const uint32_t nj = GP > wave ? (GP - wave + G::WAVES - 1) / G::WAVES : 0;
#pragma unroll 1
    for (uint32_t j0 = 0; j0 < nj; j0 += G::SLOTS) {
        // ---- 1. every load of the round: the weights of all its groups, then
        // each group's activations, scales and zero points --------------------
        u32x4_t wq[G::SLOTS][TILES];
        u32x2_t nr[G::SLOTS], nh[G::SLOTS], ng[G::SLOTS];   // NORM: residual, hidden, gamma pairs
        if constexpr (!NORM) {
#pragma unroll
            for (int s = 0; s < G::SLOTS; s++) {
                const bool ok = j0 + s < nj;      // wave-uniform; a group past nj reads zeros and adds 0
                const uint32_t g = g_begin + wave + G::WAVES * (j0 + s);
#pragma unroll
                for (int t = 0; t < TILES; t++)
                    wq[s][t] = buffer_load_x4(rw, ok && w_row[t] != OOB_OFFSET ? w_row[t] + g * 64 : OOB_OFFSET);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int s = 0; s < G::SLOTS; s++) {
            const bool ok = j0 + s < nj;
            const uint32_t g = g_begin + wave + G::WAVES * (j0 + s);
            LDS_AS uint8_t* dst = slot[s] + wave * G::WAVE_SLOT;
            if constexpr (NORM) {
                const uint32_t ko = ok ? (g * 128 + 2 * lane) * 4 : OOB_OFFSET;
                nr[s] = buffer_load_x2(rn_res, ko);
                nh[s] = buffer_load_x2(rn_hid, hid_ok ? ko : OOB_OFFSET);
                ng[s] = buffer_load_x2(rn_gam, ko);
            } else {
#pragma unroll
                for (int i = 0; i < G::A_DMA; i++)       // every block, so the count per group is fixed
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(dst + i * 1024), 16,
                                                            ok && a_off[i] != OOB_OFFSET ? a_off[i] + g * 256 : OOB_OFFSET,
                                                            0, 0, 0);
            }
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(dst + G::S_OFF), 4,
                                                    ok && s_lane != OOB_OFFSET ? s_lane + g * N * ES : OOB_OFFSET, 0, 0, 0);
            if (ZP)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rz, (lds_void*)(dst + G::Z_OFF), 4,
                                                        ok && z_lane != OOB_OFFSET ? z_lane + g * (N / 8) * 4 : OOB_OFFSET,
                                                        0, 0, 0);
            if constexpr (NORM) {
#pragma unroll
                for (int t = 0; t < TILES; t++)
                    wq[s][t] = buffer_load_x4(rw, ok && w_row[t] != OOB_OFFSET ? w_row[t] + g * 64 : OOB_OFFSET);
            }
            __builtin_amdgcn_sched_barrier(0);   // keep the groups' loads in consumption order
        }
        // ---- 2. consume the groups in order: a group's LDS data is complete
        // once only the later groups' loads are outstanding (explicit wait,
        // also a compiler fence); its weight registers the compiler waits for --
#pragma unroll
        for (int s = 0; s < G::SLOTS; s++) {
            if (s == 0) wait_vmcnt_fence<(G::SLOTS - 1) * GROUP_LOADS>();
            else if (s == 1) wait_vmcnt_fence<(G::SLOTS - 2 > 0 ? G::SLOTS - 2 : 0) * GROUP_LOADS>();
            else if (s == 2) wait_vmcnt_fence<(G::SLOTS - 3 > 0 ? G::SLOTS - 3 : 0) * GROUP_LOADS>();
            else wait_vmcnt_fence<0>();
            const LDS_AS uint8_t* sp = slot[s] + wave * G::WAVE_SLOT;
            if constexpr (NORM) {
                // x2 = res + hid; row 0 of the slot = bf16(x2 * gamma); the
                // per-row 1/rms is a common factor applied after the sum
                const float x0 = __uint_as_float(nr[s][0]) + __uint_as_float(nh[s][0]);
                const float x1 = __uint_as_float(nr[s][1]) + __uint_as_float(nh[s][1]);
                ssq += x0 * x0;
                ssq += x1 * x1;
                if (store_x2 && j0 + s < nj) {
                    const uint32_t g = g_begin + wave + G::WAVES * (j0 + s);
                    *(u32x2_t*)(p.norm_x2 + g * 128 + 2 * lane) = u32x2_t{__float_as_uint(x0), __float_as_uint(x1)};
                }
                *(LDS_AS uint32_t*)(slot[s] + wave * G::WAVE_SLOT + lane * 4) =
                    pack2_bf16_rne(x0 * __uint_as_float(ng[s][0]), x1 * __uint_as_float(ng[s][1]));
            }
            // activation fragments and sums of every row block, then one tile
            // at a time: unpack its weights once, use them for every row block
            bf16x8_t av[MB][4];
            f32x4_t sa[MB];
#pragma unroll
            for (int mb = 0; mb < MB; mb++) {
                const uint32_t row = 16 * mb + c;
#pragma unroll
                for (int w = 0; w < 4; w++)
                    av[mb][w] = *(const LDS_AS bf16x8_t*)(sp + row * 256 + (((4 * h + w) ^ c) * 16));
                sa[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int w = 0; w < 4; w++) sa[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, av[mb][w], sa[mb], 0, 0, 0);
            }
#pragma unroll
            for (int t = 0; t < TILES; t++) {
                const uint32_t n4 = c0 + 16 * t + 4 * h;     // this lane's columns n4 .. n4+3
                f32x4_t s4, zc;
                if (SF32) {
                    const u32x4_t v = *(const LDS_AS u32x4_t*)(sp + G::S_OFF + (16 * t + 4 * h) * 4);
                    s4 = f32x4_t{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
                } else {
                    const u32x2_t v = *(const LDS_AS u32x2_t*)(sp + G::S_OFF + (16 * t + 4 * h) * 2);
                    s4 = f32x4_t{bf16_bits_to_f32(v[0] & 0xFFFFu), bf16_bits_to_f32(v[0] >> 16),
                                 bf16_bits_to_f32(v[1] & 0xFFFFu), bf16_bits_to_f32(v[1] >> 16)};
                }
                if (ZP) {
                    const uint32_t zw = *(const LDS_AS uint32_t*)(sp + G::Z_OFF + (n4 / 8 - zb) * 4) >> (4 * (n4 % 8));
#pragma unroll
                    for (int r = 0; r < 4; r++) zc[r] = 128.0f + (float)((zw >> (4 * r)) & 0xFu);
                } else {
                    zc = f32x4_t{zc_const, zc_const, zc_const, zc_const};
                }
                bf16x8_t wv[4];
#pragma unroll
                for (int w = 0; w < 4; w++) wv[w] = unpack8_128(wq[s][t][w], bits4300, m000f);
#pragma unroll
                for (int mb = 0; mb < MB; mb++) {
                    f32x4_t tt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int w = 0; w < 4; w++) tt = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv[w], av[mb][w], tt, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[t][mb][r] = fmaf(s4[r], fmaf(-zc[r], sa[mb][r], tt[r]), acc[t][mb][r]);
                }
            }
        }
    }

    // ---- sum the waves, in wave order ----------------------------------------
    if constexpr (NORM) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ssq += __shfl_xor(ssq, o, 64);
    }
    // Each wave parks its partials (and its sum of squares) in its own slot-0
    // area, which only it has used, so no barrier is needed before the writes.
    constexpr uint32_t RED_STRIDE = G::WAVE_SLOT / 16;   // f32x4 per wave area
    LDS_AS f32x4_t* red = (LDS_AS f32x4_t*)slot[0];
#pragma unroll
    for (int t = 0; t < TILES; t++)
#pragma unroll
        for (int mb = 0; mb < MB; mb++) red[wave * RED_STRIDE + (t * MB + mb) * 64 + lane] = acc[t][mb];
    if (NORM && lane == 0) *(LDS_AS float*)(slot[0] + wave * G::WAVE_SLOT + G::OUT_SLOTS * 16) = ssq;
    __syncthreads();
    float inv_rms = 1.0f;
    if constexpr (NORM) {
        float t = *(const LDS_AS float*)(slot[0] + G::OUT_SLOTS * 16);
#pragma unroll
        for (int q = 1; q < G::WAVES; q++)   // in wave order
            t += *(const LDS_AS float*)(slot[0] + q * G::WAVE_SLOT + G::OUT_SLOTS * 16);
        inv_rms = 1.0f / sqrtf(t / (float)K + p.norm_eps);
    }
    constexpr uint32_t TILE_BYTES = G::OUT_SLOTS * 16;
    constexpr int NE = (G::OUT_SLOTS + G::NT - 1) / G::NT;
    const __amdgpu_buffer_rsrc_t rws = make_rsrc((const uint8_t*)p.workspace + (size_t)wg * sk * TILE_BYTES);
    f32x4_t v[NE];
#pragma unroll
    for (int e = 0; e < NE; e++) {
        const uint32_t slot = e * G::NT + tid;          // (t, mb, lane)
        v[e] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        if (slot < (uint32_t)G::OUT_SLOTS) {
            f32x4_t pw[G::WAVES];                        // every wave's partial in flight at once
#pragma unroll
            for (int q = 0; q < G::WAVES; q++) pw[q] = red[q * RED_STRIDE + slot];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < G::WAVES; q++) v[e] += pw[q];   // in wave order
            if (NORM) v[e] *= inv_rms;
            if (sk > 1) st_agent_x4(rws, part * TILE_BYTES + slot * 16, v[e]);
        }
    }
    if (sk > 1) {
        if (!publish_and_count(&p.semaphores[wg], sk, s_last)) return;
#pragma unroll
        for (int e = 0; e < NE; e++) {
            const uint32_t slot = e * G::NT + tid;
            if (slot < (uint32_t)G::OUT_SLOTS) v[e] = sum_partials_x4(rws, slot * 16, TILE_BYTES, sk);
        }
    }
#pragma unroll
    for (int e = 0; e < NE; e++) {
        const uint32_t slot = e * G::NT + tid;
        if (slot >= (uint32_t)G::OUT_SLOTS) continue;
        const uint32_t t = slot / (MB * 64), mb = (slot / 64) % MB, l = slot % 64;
        const uint32_t n = c0 + 16 * t + 4 * (l >> 4);
        if (n < c1) store_out4(p, 16 * mb + (l & 15), n, v[e]);
    }
    if (sk > 1) reset_counter(&p.semaphores[wg]);
}

template <int TILES, int MB, bool NORM = false>
__device__ __forceinline__ void w4_decode(const t0_w4a16_params& p) {
    using G = W4DecCfg<TILES, MB, NORM>;
    // distinct objects, so that the compiler tells the slots' DMAs apart
    __shared__ __attribute__((aligned(1024))) uint8_t slot0[G::SLOT_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t slot1[G::SLOTS > 1 ? G::SLOT_BYTES : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t slot2[G::SLOTS > 2 ? G::SLOT_BYTES : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t slot3[G::SLOTS > 3 ? G::SLOT_BYTES : 16];
    __shared__ uint32_t s_last;
    LDS_AS uint8_t* const sl[4] = {(LDS_AS uint8_t*)slot0, (LDS_AS uint8_t*)slot1, (LDS_AS uint8_t*)slot2,
                                   (LDS_AS uint8_t*)slot3};
    // zero points and scale type are uniform: one straight-line body each
    const bool zp = p.zeros != nullptr, sf32 = p.flags & T0_W4_SCALE_F32;
    if (zp) {
        if (sf32) w4_decode_body<TILES, MB, true, true, NORM>(p, sl, &s_last);
        else w4_decode_body<TILES, MB, true, false, NORM>(p, sl, &s_last);
    } else {
        if (sf32) w4_decode_body<TILES, MB, false, true, NORM>(p, sl, &s_last);
        else w4_decode_body<TILES, MB, false, false, NORM>(p, sl, &s_last);
    }
}

// ---------------------------------------------------------------------------
// Prefill: large M, MFMA bound.  One 128-k quant group per K step.
//   Tile BM x BN, WM x WN waves, v_mfma_f32_32x32x16_bf16.
//   Stage (LDS, filled by buffer_load ... lds):
//     A  [BM][128] bf16, 16-B chunks swizzled by row         BM*256 B
//     W  [BN][16 words] packed nibbles, chunk-swizzled         BN*64 B
//     S  [BN] f32 scales of this group                         BN*4 B (1 KB slot)
//     R  [BM] x 16 B: the correction block's A operand of row m BM*16 B
//        (R_m = sum_k a[m][k] over this group, split by w4_rowsum)
//   MFMA step kk (0..7) takes, in lane half h, the 8 k of word h*8 + kk, so a
//   lane reads its W column as two 16-B LDS loads per group.
//   Per group T = sum_k a[m][k] * (q[k][n] - z_n), exactly as MFMA products:
//     - the nibbles unpack to bf16 128 + q (exact);
//     - one more 16-deep MFMA block per group holds the correction
//       -(128 + z_n) * R_m: its A rows are R_m split into three bf16 pieces
//       (hi + mid + lo == R_m exactly), its B columns -(128 + z_n) three
//       times (an exact bf16 integer), the other 13 k zero;
//   then acc += s_n * T, one FMA per output per group.
// Requires: group_size == 128, K % 128 == 0, lda % 8 == 0, N % 8 == 0,
//           R precomputed by w4_rowsum into workspace [G][M] x 16 B, f32 scales
//           (bf16 scales are widened by the same pre-pass).
// ---------------------------------------------------------------------------
template <int CH>
T0_DEV uint32_t swz16(uint32_t r) { return r & (CH - 1) & 15; }

template <int BM, int BN, int WM, int WN, int STAGES>
struct W4Cfg {
    static constexpr int NW = WM * WN, NT = NW * 64;
    static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    static constexpr int A_BYTES = BM * 256;
    static constexpr int W_BYTES = BN * 64;
    // The scale DMA writes all 64 lanes x 16 B (1 KB, lanes past BN*4 bytes
    // write zeros), the zero-point DMA 64 x 4 B: separate slots.
    static constexpr int S_BYTES = 2048;                 // scales [0, 1024), zero-point words [1024, 1280)
    static constexpr int Z_OFF = 1024;
    static constexpr int X_BYTES = BM * 16;
    static constexpr int X_LOADS = X_BYTES / 1024;    // 1-KB row-sum DMAs per stage
    static constexpr int XW = NW - 2;                  // issued by waves 2.., at most two each
    static constexpr int STAGE = A_BYTES + W_BYTES + S_BYTES + X_BYTES;
    static constexpr int A_LOADS = A_BYTES / (1024 * NW);
    static constexpr int W_LOADS = W_BYTES / (1024 * NW);
    static constexpr int EPI_LD = TN + 4;
    static constexpr int SMEM = (STAGE * STAGES > NW * 32 * EPI_LD * 4) ? STAGE * STAGES : NW * 32 * EPI_LD * 4;
    static_assert(A_LOADS >= 1 && A_LOADS * 1024 * NW == A_BYTES, "A split");
    static_assert(W_LOADS >= 1 && W_LOADS * 1024 * NW == W_BYTES, "W split");
    static_assert(BN * 4 <= Z_OFF && BM % 64 == 0, "S/Z/X slots");
    static_assert(NW >= 3 && X_LOADS <= 2 * XW, "S, Z and X DMAs: waves 0, 1 and 2..");
    static_assert(SMEM <= 160 * 1024, "LDS");
    static_assert(STAGES == 2 || STAGES == 3, "stage waits below");
    // loads every wave issues per stage; waves 0, 1 and 2.. add the scale,
    // zero-point and row-sum DMAs, so a wait for MIN_LOADS outstanding covers
    // one stage in flight on every wave (a wave with extras waits slightly longer)
    static constexpr int MIN_LOADS = A_LOADS + W_LOADS;
};

template <int BM, int BN, int WM, int WN, int STAGES>
__device__ __forceinline__ void w4_prefill(const t0_w4a16_params& p) {
    using G = W4Cfg<BM, BN, WM, WN, STAGES>;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[G::SMEM];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wave_s = __builtin_amdgcn_readfirstlane(wave);    // the same, in an SGPR (DMA targets, branches)
    const uint32_t wm = wave / WN, wn = wave % WN;
    const uint32_t M = p.M, N = p.N, K = p.K;
    const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const uint32_t tiles = tiles_m * tiles_n;
    const uint32_t bid = blockIdx.y * gridDim.x + blockIdx.x;
    if (bid >= tiles) return;
    uint32_t tm, tn;
    grouped_tile(xcd_remap(bid, tiles), tiles_m, tiles_n, 4, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t nk = K / 128;
    const uint32_t lda = p.lda;
    const uint8_t* A0 = (const uint8_t*)p.A + (size_t)m0 * lda * 2;
    const uint8_t* W0 = (const uint8_t*)p.qweight + (size_t)n0 * (K / 2);
    const uint8_t* S0 = (const uint8_t*)p.scales + (size_t)n0 * 4;   // f32
    const uint8_t* X = (const uint8_t*)p.workspace;   // [G][M] x 16 B

    // per-lane DMA offsets
    uint32_t a_off[G::A_LOADS], w_off[G::W_LOADS];
#pragma unroll
    for (int j = 0; j < G::A_LOADS; j++) {
        const uint32_t pos = (wave * G::A_LOADS + j) * 1024 + lane * 16;
        const uint32_t r = pos / 256, c = (pos % 256) / 16;
        const uint32_t lc = c ^ swz16<16>(r);
        a_off[j] = (m0 + r < M) ? r * lda * 2 + lc * 16 : OOB_OFFSET;
    }
#pragma unroll
    for (int j = 0; j < G::W_LOADS; j++) {
        const uint32_t pos = (wave * G::W_LOADS + j) * 1024 + lane * 16;
        const uint32_t r = pos / 64, c = (pos % 64) / 16;
        const uint32_t lc = c ^ (((r >> 1) ^ (r >> 3)) & 3);
        w_off[j] = (n0 + r < N) ? r * (K / 2) + lc * 16 : OOB_OFFSET;
    }
    const uint32_t s_off = (lane * 16 < BN * 4 && n0 + lane * 4 < N) ? lane * 16 : OOB_OFFSET;
    const uint32_t z_off = (lane < BN / 8 && n0 + lane * 8 < N) ? lane * 4 : OOB_OFFSET;   // zero-point word per lane
    // row-sum DMA x (one row per lane) goes out from wave 2 + x % XW as its
    // extra load x / XW
    uint32_t x_off[2];
#pragma unroll
    for (int xq = 0; xq < 2; xq++) {
        const uint32_t x = wave - 2 + xq * G::XW, row = x * 64 + lane;
        x_off[xq] = (wave >= 2 && x < (uint32_t)G::X_LOADS && m0 + row < M) ? row * 16 : OOB_OFFSET;
    }
    const uint32_t lds_base = (uint32_t)(uintptr_t)(LDS_AS uint8_t*)smem;

    // The q-th load of this wave for stage t: its A chunks, its W chunks,
    // then (one wave each) the scales, the zero-point words and the row sums.
    constexpr int NQ = G::A_LOADS + G::W_LOADS + 2;
    // Workgroups of odd dispatch rounds (p.round_wgs = the CU count per
    // round) walk the quant groups from the last: a CU's next tile shares the
    // previous one's A row band, whose last groups are then still in the
    // XCD's L2.  Their sum over the groups runs in the reverse order, so a
    // tile's bits depend on its dispatch round (both within the same bound).
    const bool krev = p.round_wgs && ((bid / p.round_wgs) & 1);
    auto issue_q = [&](uint32_t t, int q) {
        const uint32_t st = lds_base + __builtin_amdgcn_readfirstlane((t % STAGES) * G::STAGE);
        t = krev ? nk - 1 - t : t;                       // the quant group of step t
        if (q < G::A_LOADS) {
            dma_x4(make_rsrc(A0 + (size_t)t * 256), __builtin_amdgcn_readfirstlane(st + (wave_s * G::A_LOADS + q) * 1024),
                   a_off[q]);
            return;
        }
        q -= G::A_LOADS;
        if (q < G::W_LOADS) {
            dma_x4(make_rsrc(W0 + (size_t)t * 64),
                   __builtin_amdgcn_readfirstlane(st + G::A_BYTES + (wave_s * G::W_LOADS + q) * 1024), w_off[q]);
            return;
        }
        q -= G::W_LOADS;
        if (wave_s == 0) {
            if (q == 0)
                dma_x4(make_rsrc(S0 + (size_t)t * N * 4), __builtin_amdgcn_readfirstlane(st + G::A_BYTES + G::W_BYTES),
                       s_off);
        } else if (wave_s == 1) {
            if (q == 0 && p.zeros)
                dma_x1(make_rsrc(p.zeros + (size_t)t * (N / 8) + n0 / 8),
                       __builtin_amdgcn_readfirstlane(st + G::A_BYTES + G::W_BYTES + G::Z_OFF), z_off);
        } else {
            const uint32_t x = wave_s - 2 + q * G::XW;
            if (x < (uint32_t)G::X_LOADS)
                dma_x4(make_rsrc(X + ((size_t)t * M + m0) * 16),
                       __builtin_amdgcn_readfirstlane(st + G::A_BYTES + G::W_BYTES + G::S_BYTES + x * 1024), x_off[q]);
        }
    };
    auto issue = [&](uint32_t t) {
#pragma unroll
        for (int q = 0; q < NQ; q++) issue_q(t, q);
    };
    f32x16_t acc[G::FM][G::FN];
#pragma unroll
    for (int i = 0; i < G::FM; i++)
#pragma unroll
        for (int j = 0; j < G::FN; j++) acc[i][j] = f32x16_t{};

    const uint32_t l32 = lane & 31, h = lane >> 5;
    // A operand: row (wm*TM + i*32 + l32), chunk h*8 + kk
    const uint32_t a_row0 = (wm * G::TM + l32) * 256;
    const uint32_t a_sw = swz16<16>(l32);
    // W operand: column wn*TN + j*32 + l32, words h*8..h*8+7 = chunks 2h, 2h+1
    const uint32_t w_sw = ((l32 >> 1) ^ (l32 >> 3)) & 3;
    const uint32_t w_c0 = ((2 * h) ^ w_sw) * 16, w_c1 = ((2 * h + 1) ^ w_sw) * 16;
    const uint32_t bits4300 = __builtin_amdgcn_mov_dpp(0x43004300u, 0xE4, 0xF, 0xF, false);  // in a VGPR
    const uint32_t m000f = sgpr_const(0x000F000Fu);

    // acc += s_n * T for the group whose products are in tmp; sv holds its
    // scales for (j, q4) = columns wn*TN + j*32 + 8*q4 + 4*h .. +3
    f32x16_t tmp[G::FM][G::FN];
    f32x4_t sv[G::FN][4];
    auto scale_add = [&]() {
#pragma unroll
        for (int j = 0; j < G::FN; j++)
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++)
#pragma unroll
                for (int i = 0; i < G::FM; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc[i][j][4 * q4 + r] = fmaf(sv[j][q4][r], tmp[i][j][4 * q4 + r], acc[i][j][4 * q4 + r]);
    };
    // With two waves per SIMD (waves w and w + 4), the barrier of every step
    // starts both in the same phase, so one's MFMAs cannot hide the other's
    // scale FMAs.  The second half of the waves therefore applies a group's
    // scales at the start of the next step, under the first half's MFMAs.
    const bool late = G::NW >= 8 && ((wave >> 2) & 1);

    // The correction block's B operand from this lane's zero-point word:
    // column -(128 + z) in k 0..2 of lane half 0, zero elsewhere (the A
    // operand, R split hi/mid/lo with hi + mid + lo == R exactly, comes
    // ready-made from w4_rowsum).
    const uint32_t z_sh = 4 * (l32 % 8);   // wn*TN + j*32 is a multiple of 8
    auto zcol_of = [&](uint32_t zw) {
        const uint32_t z = p.zeros ? (zw >> z_sh) & 0xFu : p.zero_const;
        const uint32_t zb = h ? 0u : 0xC300u + z;                     // bf16 -(128 + z)
        return __builtin_bit_cast(bf16x8_t, u32x4_t{zb | (zb << 16), zb, 0u, 0u});
    };

    if constexpr (STAGES == 3) {
        // One barrier per step, after its fourth 16-k sub-step: there every
        // wave has finished step t - 1 (so stage t + 2 may go into its
        // buffer, over sub-steps 4-7) and waits for its own loads of stage
        // t + 1, which the barrier makes visible to all.  Sub-step 7 then
        // reads step t + 1's first operands (A fragments, W words, zero-point
        // word, row sums), so the step boundary has no barrier and no LDS
        // wait, and the two waves of a SIMD drift apart instead of starting
        // every step in the same phase.
        constexpr int PER = (NQ + 3) / 4;
        // This lane's LDS byte offsets within a stage, fixed for the loop: a
        // read adds the stage's offset (one SGPR) to one of these, the tile
        // row/column block goes into the instruction's immediate offset.
        uint32_t a_lo[8];
#pragma unroll
        for (int kk = 0; kk < 8; kk++) a_lo[kk] = a_row0 + ((h * 8 + kk) ^ a_sw) * 16;
        const uint32_t col0 = wn * G::TN + l32;
        const uint32_t w_lo0 = G::A_BYTES + col0 * 64 + w_c0, w_lo1 = G::A_BYTES + col0 * 64 + w_c1;
        const uint32_t z_lo = G::A_BYTES + G::W_BYTES + G::Z_OFF + (col0 / 8) * 4;
        const uint32_t s_lo = G::A_BYTES + G::W_BYTES + (wn * G::TN + 4 * h) * 4;
        const uint32_t x_lo = G::A_BYTES + G::W_BYTES + G::S_BYTES + (wm * G::TM + l32) * 16;
        auto stage_at = [&](uint32_t u) {
            return (const LDS_AS uint8_t*)smem + __builtin_amdgcn_readfirstlane((u % STAGES) * G::STAGE);
        };
        issue(0);
        if (nk > 1) issue(1);
        if (nk > 1) wait_vmcnt<G::MIN_LOADS>();
        else wait_vmcnt<0>();
        __syncthreads();
        bf16x8_t af[2][G::FM];
        u32x4_t wlo[G::FN], whi[G::FN], wlo_n[G::FN], whi_n[G::FN];
        uint32_t zw[G::FN], zw_n[G::FN];
        bf16x8_t xr[G::FM], xr_n[G::FM];
        // a step's first operands, from its stage's buffer st
        auto read_first = [&](const LDS_AS uint8_t* st, bf16x8_t* a0, u32x4_t* wl, u32x4_t* wh, uint32_t* z,
                              bf16x8_t* x) {
#pragma unroll
            for (int i = 0; i < G::FM; i++) {
                a0[i] = *(const LDS_AS bf16x8_t*)(st + a_lo[0] + i * 32 * 256);
                x[i] = *(const LDS_AS bf16x8_t*)(st + x_lo + i * 32 * 16);
            }
#pragma unroll
            for (int j = 0; j < G::FN; j++) {
                wl[j] = *(const LDS_AS u32x4_t*)(st + w_lo0 + j * 32 * 64);
                wh[j] = *(const LDS_AS u32x4_t*)(st + w_lo1 + j * 32 * 64);
                z[j] = p.zeros ? *(const LDS_AS uint32_t*)(st + z_lo + j * 32 / 8 * 4) : 0u;
            }
        };
        // tmp[i][j] = the group's correction block, then its 8 sub-steps
        auto correction = [&](int i) {
#pragma unroll
            for (int j = 0; j < G::FN; j++)
                tmp[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(zcol_of(zw[j]), xr[i], f32x16_t{}, 0, 0, 0);
        };
        if (nk) {
            read_first(stage_at(0), af[0], wlo, whi, zw, xr);
#pragma unroll
            for (int i = 0; i < G::FM; i++) correction(i);
        }
        // One step; N2 / N1: stage t + 2 is to be loaded / step t + 1 exists.
        // The last two steps are peeled, so the loop body has no such branch.
        auto step = [&](uint32_t t, auto N2c, auto N1c) {
            constexpr bool has2 = decltype(N2c)::value != 0, has1 = decltype(N1c)::value != 0;
            const LDS_AS uint8_t* sa = stage_at(t);
#pragma unroll
            for (int kk = 0; kk < 8; kk++) {
                const int cur = kk & 1;
                if (kk == 4) {
                    // A plain barrier: the LDS reads still in flight here are
                    // of stage t, and every read of stage t - 1 (whose buffer
                    // the DMA below refills) was consumed before this point.
                    wait_vmcnt_fence<0>();   // this wave's loads of stage t + 1
                    __builtin_amdgcn_sched_barrier(0);
                    __builtin_amdgcn_s_barrier();
                    __builtin_amdgcn_sched_barrier(0);
                    asm volatile("" ::: "memory");
                }
                if constexpr (has2) {
                    if (kk >= 4) {
#pragma unroll
                        for (int q = (kk - 4) * PER; q < (kk - 3) * PER && q < NQ; q++) issue_q(t + 2, q);
                    }
                }
                if (kk + 1 < 8) {
#pragma unroll
                    for (int i = 0; i < G::FM; i++)
                        af[cur ^ 1][i] = *(const LDS_AS bf16x8_t*)(sa + a_lo[kk + 1] + i * 32 * 256);
                } else if constexpr (has1) {
                    read_first(stage_at(t + 1), af[cur ^ 1], wlo_n, whi_n, zw_n, xr_n);
                }
                // the next sub-step's reads stay ahead of this one's MFMAs
                // (the scheduler would sink them next to their uses, into
                // the same registers, and every sub-step would wait on them)
                __builtin_amdgcn_sched_barrier(0);
                bf16x8_t bw[G::FN];
#pragma unroll
                for (int j = 0; j < G::FN; j++) bw[j] = unpack8_128(kk < 4 ? wlo[j][kk] : whi[j][kk - 4], bits4300, m000f);
#pragma unroll
                for (int i = 0; i < G::FM; i++)
#pragma unroll
                    for (int j = 0; j < G::FN; j++)
                        tmp[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw[j], af[cur][i], tmp[i][j], 0, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < G::FN; j++) {
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++)
                    sv[j][q4] = *(const LDS_AS f32x4_t*)(sa + s_lo + (j * 32 + 8 * q4) * 4);
                wlo[j] = wlo_n[j];
                whi[j] = whi_n[j];
                zw[j] = zw_n[j];
            }
#pragma unroll
            for (int i = 0; i < G::FM; i++) xr[i] = xr_n[i];
            // Per row block: this group's scale FMAs, then the next group's
            // correction block into the same tmp.  Block i's FMAs run while
            // the MFMAs of the blocks after it are still in flight, instead
            // of all 64 waiting for the last MFMA and holding back the next
            // group's first MFMA.
#pragma unroll
            for (int i = 0; i < G::FM; i++) {
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < G::FN; j++)
#pragma unroll
                    for (int e = 0; e < 16; e++) acc[i][j][e] = fmaf(sv[j][e / 4][e % 4], tmp[i][j][e], acc[i][j][e]);
                __builtin_amdgcn_sched_barrier(0);
                correction(i);   // after the last group: unused, on the last group's operands
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        uint32_t t = 0;
        for (; t + 2 < nk; t++) step(t, Idx<1>{}, Idx<1>{});
        if (t + 1 < nk) step(t++, Idx<0>{}, Idx<1>{});
        if (t < nk) step(t, Idx<0>{}, Idx<0>{});
    } else {
#pragma unroll
    for (int s = 0; s < STAGES - 1; s++)
        if ((uint32_t)s < nk) issue(s);

    for (uint32_t t = 0; t < nk; t++) {
        // stage t has landed once at most the next stage's loads are in flight
        if (STAGES == 3 && t + 1 < nk) wait_vmcnt<G::MIN_LOADS>();
        else wait_vmcnt<0>();
        __syncthreads();
        if (t + STAGES - 1 < nk) issue(t + STAGES - 1);
        if (late && t > 0) scale_add();
        __builtin_amdgcn_sched_barrier(0);

        const LDS_AS uint8_t* st = (const LDS_AS uint8_t*)smem + (t % STAGES) * G::STAGE;
        const LDS_AS uint8_t* sa = st;
        const LDS_AS uint8_t* sw = st + G::A_BYTES;
        const LDS_AS float* ss = (const LDS_AS float*)(st + G::A_BYTES + G::W_BYTES);
        const LDS_AS uint32_t* sz = (const LDS_AS uint32_t*)(st + G::A_BYTES + G::W_BYTES + G::Z_OFF);
        const LDS_AS uint8_t* sx = st + G::A_BYTES + G::W_BYTES + G::S_BYTES;

        // this lane's W words, and the correction block's operands
        bf16x8_t af[2][G::FM];
#pragma unroll
        for (int i = 0; i < G::FM; i++)
            af[0][i] = *(const LDS_AS bf16x8_t*)(sa + a_row0 + i * 32 * 256 + ((h * 8) ^ a_sw) * 16);
        u32x4_t wlo[G::FN], whi[G::FN];
        bf16x8_t zcol[G::FN], rrow[G::FM];
#pragma unroll
        for (int j = 0; j < G::FN; j++) {
            const uint32_t col = wn * G::TN + j * 32 + l32;
            const LDS_AS uint8_t* wr = sw + col * 64;
            wlo[j] = *(const LDS_AS u32x4_t*)(wr + w_c0);
            whi[j] = *(const LDS_AS u32x4_t*)(wr + w_c1);
            zcol[j] = zcol_of(p.zeros ? sz[col / 8] : 0u);
        }
#pragma unroll
        for (int i = 0; i < G::FM; i++)
            rrow[i] = *(const LDS_AS bf16x8_t*)(sx + (wm * G::TM + i * 32 + l32) * 16);
#pragma unroll
        for (int i = 0; i < G::FM; i++)
#pragma unroll
            for (int j = 0; j < G::FN; j++)
                tmp[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(zcol[j], rrow[i], f32x16_t{}, 0, 0, 0);
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            const int cur = kk & 1;
            if (kk + 1 < 8) {
#pragma unroll
                for (int i = 0; i < G::FM; i++) {
                    const uint32_t c = (h * 8 + kk + 1) ^ a_sw;
                    af[cur ^ 1][i] = *(const LDS_AS bf16x8_t*)(sa + a_row0 + i * 32 * 256 + c * 16);
                }
            }
            bf16x8_t bw[G::FN];
#pragma unroll
            for (int j = 0; j < G::FN; j++) bw[j] = unpack8_128(kk < 4 ? wlo[j][kk] : whi[j][kk - 4], bits4300, m000f);
#pragma unroll
            for (int i = 0; i < G::FM; i++)
#pragma unroll
                for (int j = 0; j < G::FN; j++)
                    tmp[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw[j], af[cur][i], tmp[i][j], 0, 0, 0);
        }
        // this group's scales (the buffer is refilled after the next barrier)
#pragma unroll
        for (int j = 0; j < G::FN; j++)
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++)
                sv[j][q4] = *(const LDS_AS f32x4_t*)(ss + wn * G::TN + j * 32 + 8 * q4 + 4 * h);
        if (!late) scale_add();
    }
    if (late && nk) scale_add();
    }

    // epilogue: stage 32-row blocks through LDS, store rows
    __syncthreads();
    float* wreg = (float*)smem + wave * 32 * G::EPI_LD;
#pragma unroll
    for (int i = 0; i < G::FM; i++) {
#pragma unroll
        for (int j = 0; j < G::FN; j++)
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                f32x4_t v = {acc[i][j][4 * q4], acc[i][j][4 * q4 + 1], acc[i][j][4 * q4 + 2], acc[i][j][4 * q4 + 3]};
                *(LDS_AS f32x4_t*)(wreg + l32 * G::EPI_LD + j * 32 + 8 * q4 + 4 * h) = v;
            }
        constexpr uint32_t QPR = G::TN / 4;
#pragma unroll 1
        for (uint32_t q = lane; q < 32 * QPR; q += 64) {
            const uint32_t r = q / QPR, c4 = q % QPR;
            const f32x4_t v = *(const LDS_AS f32x4_t*)(wreg + r * G::EPI_LD + c4 * 4);
            store_out4(p, m0 + wm * G::TM + i * 32 + r, n0 + wn * G::TN + c4 * 4, v);
        }
    }
}

// Prefill pre-pass (group 128), 256 threads per block:
//   R = sum_{k in group g} a[m][k], written to workspace [G][M] x 16 B as
//   the prefill's correction A operand: bf16 k0..k2 = hi, mid, lo with
//   hi + mid + lo == R exactly (each piece holds the next 8 significant
//   bits; f32 has 24), k3..k7 zero;
//   with bf16 scales, the blocks past the row sums widen them to f32 into
//   p.scales_f32 [G][N] (four per thread).
__device__ __forceinline__ void w4_rowsum(const t0_w4a16_params& p) {
    const uint32_t G = p.K / 128;
    const uint32_t sum_blocks = (p.M * ((G + 7) / 8) + 3) / 4;
    if (blockIdx.x >= sum_blocks) {
        const uint32_t q = (blockIdx.x - sum_blocks) * 256 + threadIdx.x;   // 4 scales
        if (q < G * p.N / 4) {
            const u32x2_t v = ((const u32x2_t*)p.scales)[q];
            ((f32x4_t*)p.scales_f32)[q] = f32x4_t{__uint_as_float(v[0] << 16), __uint_as_float(v[0] & 0xFFFF0000u),
                                                  __uint_as_float(v[1] << 16), __uint_as_float(v[1] & 0xFFFF0000u)};
        }
        return;
    }
    // one wave per (m, 8 groups): lane covers 16 k of a group
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wid = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    const uint32_t m = wid / ((G + 7) / 8);
    const uint32_t g8 = wid % ((G + 7) / 8);
    if (m >= p.M) return;
    const uint32_t g = g8 * 8 + lane / 8;          // 8 lanes per group
    float s = 0.0f;
    if (g < G) {
        const uint16_t* a = (const uint16_t*)p.A + (size_t)m * p.lda + g * 128 + (lane % 8) * 16;
        const u32x4_t v0 = *(const u32x4_t*)a, v1 = *(const u32x4_t*)(a + 8);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            s += __uint_as_float(v0[e] << 16) + __uint_as_float(v0[e] & 0xFFFF0000u);
            s += __uint_as_float(v1[e] << 16) + __uint_as_float(v1[e] & 0xFFFF0000u);
        }
    }
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if (g < G && (lane % 8) == 0) {
        const uint32_t hi = __float_as_uint(s) & 0xFFFF0000u;
        const float r1 = s - __uint_as_float(hi);                       // exact
        const uint32_t mid = __float_as_uint(r1) & 0xFFFF0000u;
        const uint32_t lo = __float_as_uint(r1 - __uint_as_float(mid)); // <= 8 significant bits: exact in bf16
        ((u32x4_t*)p.workspace)[(size_t)g * p.M + m] = u32x4_t{(hi >> 16) | mid, lo >> 16, 0u, 0u};
    }
}

// Generic W4A16 (any M, N, group size dividing K): one thread per output,
// sequential over k.  Correctness fallback for shapes the tiled kernels do
// not take.
__device__ __forceinline__ void w4_generic(const t0_w4a16_params& p) {
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t m = blockIdx.y;
    if (n >= p.N || m >= p.M) return;
    const uint32_t K = p.K, gs = p.group_size;
    const uint32_t* wr = p.qweight + (size_t)n * (K / 8);
    const uint16_t* ar = (const uint16_t*)p.A + (size_t)m * p.lda;
    float acc = 0.0f;
    for (uint32_t g = 0; g < K / gs; g++) {
        const float s = scale_of(p, g, n);
        const int z = (int)zero_of(p, g, n);
        float part = 0.0f;
        for (uint32_t k = g * gs; k < (g + 1) * gs; k++) {
            const int q = (int)((wr[k / 8] >> (4 * (k % 8))) & 0xFu);
            part = fmaf(bf16_bits_to_f32(ar[k]), (float)(q - z), part);
        }
        acc = fmaf(s, part, acc);
    }
    if (p.flags & T0_W4_OUT_F32) ((float*)p.C)[(size_t)m * p.ldc + n] = acc;
    else ((uint16_t*)p.C)[(size_t)m * p.ldc + n] = (uint16_t)(pack2_bf16_rne(acc, 0.f) & 0xFFFFu);
}

// ---------------------------------------------------------------------------
// The reference's standalone dequant kernels, restated to the documented
// format (src/t0/quant_kernels.rs:1-24, :37-47): one work-item per element e
// of [rows x cols]; byte e/2, low nibble for even e; group g = col >> log2(gs)
// indexes f32 scales / i32 zero points laid out [row][group];
// out = (q - zp) * scale as f32, or truncated to bf16 (store_bf16).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void dequant_int4(const t0_dequant_params& p, bool bf16_out) {
    const uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t total = (uint64_t)p.rows * p.cols;
    if (e >= total) return;
    const uint32_t row = (uint32_t)(e / p.cols), col = (uint32_t)(e % p.cols);
    const uint32_t n_groups = p.cols >> p.group_size_log2;
    const uint8_t byte = p.packed[e >> 1];
    const int32_t q = (e & 1) ? (byte >> 4) : (byte & 0xF);
    const uint32_t gi = row * n_groups + (col >> p.group_size_log2);
    const float v = (float)(q - p.zero_points[gi]) * p.scales[gi];
    if (bf16_out) ((uint16_t*)p.output)[e] = (uint16_t)(__float_as_uint(v) >> 16);
    else ((float*)p.output)[e] = v;
}

}  // namespace t0

// t0k_w4a16_decode_t<TILES>_mb<MB>: at most 16*TILES columns per workgroup,
// M <= 16*MB.
#define T0_W4_DECODE(TILES, MB)                                                                  \
    extern "C" __global__ void __launch_bounds__(64 * t0_w4_decode_waves(TILES, MB))              \
        t0k_w4a16_decode_t##TILES##_mb##MB(const t0_w4a16_params p) {                             \
        t0::w4_decode<TILES, MB>(p);                                                             \
    }
T0_W4_DECODE(1, 1)
T0_W4_DECODE(2, 1)
T0_W4_DECODE(3, 1)
T0_W4_DECODE(4, 1)
T0_W4_DECODE(1, 2)
T0_W4_DECODE(2, 2)
T0_W4_DECODE(3, 2)
T0_W4_DECODE(4, 2)
T0_W4_DECODE(1, 4)
T0_W4_DECODE(2, 4)
T0_W4_DECODE(3, 4)
T0_W4_DECODE(4, 4)

// t0k_w4a16_decode_norm_t<TILES>: the M == 1 decode with residual add +
// RMSNorm fused in front (activations from t0_w4a16_params.norm_*).
#define T0_W4_DECODE_NORM(TILES)                                                                 \
    extern "C" __global__ void __launch_bounds__(64 * t0_w4_decode_norm_waves(TILES))             \
        t0k_w4a16_decode_norm_t##TILES(const t0_w4a16_params p) {                                 \
        t0::w4_decode<TILES, 1, true>(p);                                                        \
    }
T0_W4_DECODE_NORM(1)
T0_W4_DECODE_NORM(2)
T0_W4_DECODE_NORM(3)
T0_W4_DECODE_NORM(4)

#define T0_W4_PREFILL(BM, BN, WM, WN, ST)                                                        \
    extern "C" __global__ void __launch_bounds__(WM * WN * 64)                                    \
        t0k_w4a16_prefill_##BM##x##BN##_w##WM##x##WN##_s##ST(const t0_w4a16_params p) {          \
        t0::w4_prefill<BM, BN, WM, WN, ST>(p);                                                   \
    }
T0_W4_PREFILL(256, 128, 2, 2, 2)
T0_W4_PREFILL(256, 128, 4, 2, 2)
T0_W4_PREFILL(128, 128, 2, 2, 2)
T0_W4_PREFILL(128, 256, 2, 4, 3)
T0_W4_PREFILL(128, 256, 1, 8, 3)

extern "C" __global__ void __launch_bounds__(256) t0k_w4a16_rowsum(const t0_w4a16_params p) { t0::w4_rowsum(p); }
extern "C" __global__ void __launch_bounds__(256) t0k_w4a16_generic(const t0_w4a16_params p) { t0::w4_generic(p); }
extern "C" __global__ void __launch_bounds__(256) dequant_int4_f32(const t0_dequant_params p) { t0::dequant_int4(p, false); }
extern "C" __global__ void __launch_bounds__(256) dequant_int4_bf16(const t0_dequant_params p) { t0::dequant_int4(p, true); }

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
// Fused dequant, exact: a nibble pair becomes two bf16 of value
// 144 + q - z (an integer in [129,159], exact in bf16) with one v_perm and one
// integer add; MFMA accumulates T = sum a*(144 + q - z) over a quant group;
// the group's result is s * (T - 144 * sum a), applied in f32.  So the weight
// value the GEMM uses is exactly (q - z) * s and the weights cross HBM once, at
// 4 bits.
#include "common.h"

namespace t0 {

// 8 nibbles of one u32 (k = 0..7) -> 8 bf16 of (144 + q - z), as 4 u32 pairs.
// kadd = 0x43004300 + (16 - z) * 0x00010001.
T0_DEV bf16x8_t unpack8(uint32_t w, uint32_t kadd) {
    const uint32_t lo = w & 0x0F0F0F0Fu;          // bytes q0 q2 q4 q6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // bytes q1 q3 q5 q7
    u32x4_t r;
    r[0] = __builtin_amdgcn_perm(hi, lo, 0x0C040C00u) + kadd;   // q0 | q1<<16
    r[1] = __builtin_amdgcn_perm(hi, lo, 0x0C050C01u) + kadd;   // q2 | q3<<16
    r[2] = __builtin_amdgcn_perm(hi, lo, 0x0C060C02u) + kadd;   // q4 | q5<<16
    r[3] = __builtin_amdgcn_perm(hi, lo, 0x0C070C03u) + kadd;   // q6 | q7<<16
    return __builtin_bit_cast(bf16x8_t, r);
}

T0_DEV uint32_t zero_of(const t0_w4a16_params& p, uint32_t g, uint32_t n) {
    if (!p.zeros) return p.zero_const;
    return (p.zeros[(size_t)g * (p.N / 8) + n / 8] >> (4 * (n % 8))) & 0xFu;
}

T0_DEV uint32_t kadd_of(uint32_t z) { return 0x43004300u + (16u - z) * 0x00010001u; }

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
// Decode: small M (<= 16*MB), memory bound.
//   grid = (N / (16*WAVES), split_k), block = 64*WAVES.
//   Workgroup: 16*WAVES columns x K-slice of K/split_k (multiple of 128).
//   Wave: 16 columns; lane l streams column n0 + l%16, 32 k per 16-byte load
//   (lane group l/16 picks which 32 of each 128).  The activation slice sits
//   in LDS; v_mfma_f32_16x16x32_bf16 with W as the first operand gives lane l
//   the outputs (m = l%16, n = n0 + 4*(l/16) + r).
//   split_k > 1: partial tiles go to the workspace [column block][split][tile]
//   and the last workgroup of each column block adds them in split order.
// Requires: group_size == 128, K % (128*split_k) == 0, N % 16 == 0, lda % 8 == 0.
// ---------------------------------------------------------------------------
template <int WAVES, int MB>
__device__ __forceinline__ void w4_decode(const t0_w4a16_params& p) {
    constexpr int NCW = 16 * WAVES;
    constexpr int ROWS = 16 * MB;
    constexpr int NT = WAVES * 64;
    constexpr int KC_MAX = 1024 / MB;          // K slice per workgroup (host keeps K/split_k <= this)
    constexpr int SP_MAX = KC_MAX / 128;       // quant groups (spans) per slice
    constexpr int LDA_S = KC_MAX + 8;          // LDS row stride (elements), +16 B staggers banks
    constexpr int ACH = ROWS * KC_MAX / 8 / NT;                  // 16-B activation chunks per thread
    constexpr int SCH = (SP_MAX * NCW + NT - 1) / NT;            // scale / zero entries per thread
    static_assert(ACH >= 1 && ACH * NT * 8 == ROWS * KC_MAX, "activation staging split");
    __shared__ __attribute__((aligned(16))) uint16_t a_s[ROWS * LDA_S];
    __shared__ __attribute__((aligned(16))) float s_s[SP_MAX * NCW];
    __shared__ uint32_t z_s[SP_MAX * NCW];
    __shared__ uint32_t s_last;

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t K = p.K, N = p.N, M = p.M;
    const uint32_t sk = p.split_k;
    const uint32_t KC = K / sk;
    const uint32_t nb = blockIdx.x, part = blockIdx.y;
    const uint32_t k0 = part * KC;
    const uint32_t spans = KC / 128;
    const uint32_t g0 = k0 / 128;
    const uint32_t l16 = lane & 15, g4 = lane >> 4;

    // Every load below is unconditional (lanes with nothing to fetch get an
    // out-of-range offset, which reads zero), issued in this order: the
    // activation slice, scales and zero points first, then the whole weight
    // slice.  The LDS staging then waits only for the first group while the
    // weight bytes stay in flight.
    // ---- 1. activation slice (rows >= M read as zero) ------------------------
    const uint32_t chunks_row = KC / 8;
    __amdgpu_buffer_rsrc_t ra = make_rsrc((const uint16_t*)p.A + k0);
    u32x4_t areg[ACH];
#pragma unroll
    for (int i = 0; i < ACH; i++) {
        const uint32_t c = tid + i * NT;
        const uint32_t r = c / chunks_row, kc = (c % chunks_row) * 8;
        const bool ok = r < M && c < ROWS * chunks_row;
        areg[i] = buffer_load_x4(ra, ok ? (r * p.lda + kc) * 2 : OOB_OFFSET);
    }
    // ---- 2. scales and zero points of the block's spans ---------------------
    __amdgpu_buffer_rsrc_t rs = make_rsrc(p.scales);
    __amdgpu_buffer_rsrc_t rz = make_rsrc(p.zeros ? (const void*)p.zeros : (const void*)p.scales);
    const bool sf32 = p.flags & T0_W4_SCALE_F32;
    uint32_t sraw[SCH], zraw[SCH];
#pragma unroll
    for (int i = 0; i < SCH; i++) {
        const uint32_t e = tid + i * NT;
        const uint32_t sp = e / NCW, n = nb * NCW + e % NCW;
        const bool ok = e < spans * NCW;
        const uint32_t gi = (g0 + sp) * N + n;
        sraw[i] = sf32 ? buffer_load_x1(rs, ok ? gi * 4 : OOB_OFFSET)
                       : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, ok ? gi * 2 : OOB_OFFSET, 0, 0);
        zraw[i] = p.zeros ? buffer_load_x1(rz, ok ? ((g0 + sp) * (N / 8) + n / 8) * 4 : OOB_OFFSET) : 0u;
    }
    // ---- 3. weight slice: one 16-B load per lane per 128-k span --------------
    // The resource base is the wave's first column (wave-uniform: a per-lane
    // base would make the compiler serialise each load over the distinct
    // bases); lane l streams column +l%16 at byte offset (l%16)*K/2.
    const uint32_t n_wave = __builtin_amdgcn_readfirstlane(nb * NCW + wave * 16);
    __amdgpu_buffer_rsrc_t rw = make_rsrc(p.qweight + (size_t)n_wave * (K / 8) + k0 / 8);
    const uint32_t w_off = l16 * (K / 2) + g4 * 16;
    u32x4_t wbuf[SP_MAX];
#pragma unroll
    for (int s = 0; s < SP_MAX; s++) wbuf[s] = buffer_load_x4(rw, (uint32_t)s < spans ? w_off + s * 64 : OOB_OFFSET);

    // ---- 4. stage activations / scales / zero adders into LDS ---------------
#pragma unroll
    for (int i = 0; i < ACH; i++) {
        const uint32_t c = tid + i * NT;
        const uint32_t r = c / chunks_row, kc = (c % chunks_row) * 8;
        if (c < ROWS * chunks_row) *(LDS_AS u32x4_t*)((LDS_AS uint16_t*)a_s + r * LDA_S + kc) = areg[i];
    }
#pragma unroll
    for (int i = 0; i < SCH; i++) {
        const uint32_t e = tid + i * NT;
        if (e < SP_MAX * NCW) {
            const uint32_t n = nb * NCW + e % NCW;
            s_s[e] = sf32 ? __uint_as_float(sraw[i]) : bf16_bits_to_f32(sraw[i] & 0xFFFFu);
            const uint32_t z = p.zeros ? (zraw[i] >> (4 * (n % 8))) & 0xFu : p.zero_const;
            z_s[e] = kadd_of(z);
        }
    }
    __syncthreads();

    // bf16 1.0 x 8 for the activation-sum MFMA
    const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4_t{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
    f32x4_t acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) acc[mb] = f32x4_t{0, 0, 0, 0};
    const uint32_t n_out = nb * NCW + wave * 16 + g4 * 4;        // first of this lane's 4 outputs

#pragma unroll
    for (int s = 0; s < SP_MAX; s++) {
        if ((uint32_t)s >= spans) break;
        const u32x4_t wq = wbuf[s];
        const uint32_t kadd = z_s[s * NCW + wave * 16 + l16];
        const f32x4_t sc = *(const LDS_AS f32x4_t*)((const LDS_AS float*)s_s + s * NCW + wave * 16 + g4 * 4);
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            f32x4_t t = {0, 0, 0, 0}, sa = {0, 0, 0, 0};
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const bf16x8_t wv = unpack8(wq[w], kadd);
                const bf16x8_t av = *(const LDS_AS bf16x8_t*)(
                    (const LDS_AS uint16_t*)a_s + (mb * 16 + l16) * LDA_S + s * 128 + g4 * 32 + w * 8);
                t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv, av, t, 0, 0, 0);
                sa = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, av, sa, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) acc[mb][r] = fmaf(sc[r], t[r] - 144.0f * sa[r], acc[mb][r]);
        }
    }

    if (sk == 1) {
#pragma unroll
        for (int mb = 0; mb < MB; mb++) store_out4(p, mb * 16 + l16, n_out, acc[mb]);
        return;
    }
    // split-K: park the partial tile in the workspace in register order
    // (tile (part, nb) is ROWS*NCW floats; thread t's 16 bytes of row block mb
    // at (mb*NT + t)*16), so each wave stores whole lines; the last workgroup
    // of the column block sums the partitions in partition order.
    constexpr uint32_t TILE_BYTES = ROWS * NCW * 4;
    __amdgpu_buffer_rsrc_t rws = make_rsrc((const uint8_t*)p.workspace + (size_t)nb * sk * TILE_BYTES);
#pragma unroll
    for (int mb = 0; mb < MB; mb++) st_agent_x4(rws, part * TILE_BYTES + (mb * NT + tid) * 16, acc[mb]);
    if (!publish_and_count(&p.semaphores[nb], sk, &s_last)) return;
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
        store_out4(p, mb * 16 + l16, n_out, sum_partials_x4(rws, (mb * NT + tid) * 16, TILE_BYTES, sk));
    reset_counter(&p.semaphores[nb]);
}

// ---------------------------------------------------------------------------
// Prefill: large M, MFMA bound.  One 128-k quant group per K step.
//   Tile BM x BN, WM x WN waves, v_mfma_f32_32x32x16_bf16.
//   Stage (LDS, filled by buffer_load ... lds):
//     A  [BM][128] bf16, 16-B chunks swizzled by row         BM*256 B
//     W  [BN][16 words] packed nibbles, chunk-swizzled         BN*64 B
//     S  [BN] bf16 scales of this group                        BN*2 B (padded to 1 KB slot)
//     X  [BM] f32: -144 * sum_k a[m][k] over this group        BM*4 B
//   MFMA step kk (0..7) takes, in lane half h, the 8 k of word h*8 + kk, so a
//   lane reads its W column as two 16-B LDS loads per group.
//   Per group: T = sum_kk mfma(unpack(W), A);  acc += s_n * (T + X_m).
// Requires: group_size == 128, K % 128 == 0, lda % 8 == 0, N % 8 == 0,
//           X precomputed by w4_rowsum into workspace [G][M].
// ---------------------------------------------------------------------------
template <int CH>
T0_DEV uint32_t swz16(uint32_t r) { return r & (CH - 1) & 15; }

template <int BM, int BN, int WM, int WN, int STAGES>
struct W4Cfg {
    static constexpr int NW = WM * WN, NT = NW * 64;
    static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    static constexpr int A_BYTES = BM * 256;
    static constexpr int W_BYTES = BN * 64;
    static constexpr int S_BYTES = 1024;                 // BN*2 <= 1024
    static constexpr int X_BYTES = (BM * 4 + 1023) / 1024 * 1024;
    static constexpr int STAGE = A_BYTES + W_BYTES + S_BYTES + X_BYTES;
    static constexpr int A_LOADS = A_BYTES / (1024 * NW);
    static constexpr int W_LOADS = W_BYTES / (1024 * NW);
    static constexpr int EPI_LD = TN + 4;
    static constexpr int SMEM = (STAGE * STAGES > NW * 32 * EPI_LD * 4) ? STAGE * STAGES : NW * 32 * EPI_LD * 4;
    static_assert(A_LOADS >= 1 && A_LOADS * 1024 * NW == A_BYTES, "A split");
    static_assert(W_LOADS >= 1 && W_LOADS * 1024 * NW == W_BYTES, "W split");
    static_assert(BN * 2 <= 1024 && BM * 4 <= 1024 * 2, "S/X slots");
    static_assert(SMEM <= 160 * 1024, "LDS");
    static_assert(NW >= 2 && STAGES == 2, "scale/X DMA split over two waves; vmcnt(0) per stage");
};

template <int N_>
T0_DEV void w4_wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N_ & 0xF) | (0x7 << 4) | (0xF << 8) | ((N_ >> 4) << 14));
}

T0_DEV void w4_dma(__amdgpu_buffer_rsrc_t r, uint32_t lds_addr, uint32_t voffset) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :: "s"(lds_addr), "v"(voffset), "s"(r) : "memory");
}

template <int BM, int BN, int WM, int WN, int STAGES>
__device__ __forceinline__ void w4_prefill(const t0_w4a16_params& p) {
    using G = W4Cfg<BM, BN, WM, WN, STAGES>;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[G::SMEM];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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
    const uint8_t* S0 = (const uint8_t*)p.scales + (size_t)n0 * 2;
    const float* X = p.workspace;   // [G][M]

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
    const uint32_t s_off = (lane * 16 < BN * 2 && n0 + lane * 8 < N) ? lane * 16 : OOB_OFFSET;
    const uint32_t x_off = (lane * 16 < BM * 4 && m0 + lane * 4 < M) ? lane * 16 : OOB_OFFSET;
    const uint32_t x_off2 = (1024 + lane * 16 < BM * 4 && m0 + 256 + lane * 4 < M) ? 1024 + lane * 16 : OOB_OFFSET;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(LDS_AS uint8_t*)smem;

    auto issue = [&](uint32_t t) {
        const uint32_t st = lds_base + (t % STAGES) * G::STAGE;
        __amdgpu_buffer_rsrc_t ra = make_rsrc(A0 + (size_t)t * 256);
        __amdgpu_buffer_rsrc_t rw = make_rsrc(W0 + (size_t)t * 64);
#pragma unroll
        for (int j = 0; j < G::A_LOADS; j++)
            w4_dma(ra, __builtin_amdgcn_readfirstlane(st + (wave * G::A_LOADS + j) * 1024), a_off[j]);
#pragma unroll
        for (int j = 0; j < G::W_LOADS; j++)
            w4_dma(rw, __builtin_amdgcn_readfirstlane(st + G::A_BYTES + (wave * G::W_LOADS + j) * 1024), w_off[j]);
        if (wave == 0) {
            __amdgpu_buffer_rsrc_t rs = make_rsrc(S0 + (size_t)t * N * 2);
            w4_dma(rs, __builtin_amdgcn_readfirstlane(st + G::A_BYTES + G::W_BYTES), s_off);
        } else if (wave == G::NW - 1) {
            __amdgpu_buffer_rsrc_t rx = make_rsrc(X + (size_t)t * M + m0);
            w4_dma(rx, __builtin_amdgcn_readfirstlane(st + G::A_BYTES + G::W_BYTES + G::S_BYTES), x_off);
            if constexpr (BM * 4 > 1024)
                w4_dma(rx, __builtin_amdgcn_readfirstlane(st + G::A_BYTES + G::W_BYTES + G::S_BYTES + 1024), x_off2);
        }
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

#pragma unroll
    for (int s = 0; s < STAGES - 1; s++)
        if ((uint32_t)s < nk) issue(s);

    for (uint32_t t = 0; t < nk; t++) {
        w4_wait_vmcnt<0>();   // two stages: everything issued so far is this stage
        __syncthreads();
        if (t + STAGES - 1 < nk) issue(t + STAGES - 1);

        const LDS_AS uint8_t* st = (const LDS_AS uint8_t*)smem + (t % STAGES) * G::STAGE;
        const LDS_AS uint8_t* sa = st;
        const LDS_AS uint8_t* sw = st + G::A_BYTES;
        const LDS_AS uint16_t* ss = (const LDS_AS uint16_t*)(st + G::A_BYTES + G::W_BYTES);
        const LDS_AS float* sx = (const LDS_AS float*)(st + G::A_BYTES + G::W_BYTES + G::S_BYTES);

        // this lane's W words and zero-point adders for the group
        u32x4_t wlo[G::FN], whi[G::FN];
        uint32_t kadd[G::FN];
#pragma unroll
        for (int j = 0; j < G::FN; j++) {
            const uint32_t col = wn * G::TN + j * 32 + l32;
            const LDS_AS uint8_t* wr = sw + col * 64;
            wlo[j] = *(const LDS_AS u32x4_t*)(wr + w_c0);
            whi[j] = *(const LDS_AS u32x4_t*)(wr + w_c1);
            kadd[j] = kadd_of(zero_of(p, t, n0 + col < N ? n0 + col : 0));
        }
        f32x16_t tmp[G::FM][G::FN];
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
            bf16x8_t af[G::FM], bw[G::FN];
#pragma unroll
            for (int i = 0; i < G::FM; i++) {
                const uint32_t c = (h * 8 + kk) ^ a_sw;
                af[i] = *(const LDS_AS bf16x8_t*)(sa + a_row0 + i * 32 * 256 + c * 16);
            }
#pragma unroll
            for (int j = 0; j < G::FN; j++) bw[j] = unpack8(kk < 4 ? wlo[j][kk] : whi[j][kk - 4], kadd[j]);
#pragma unroll
            for (int i = 0; i < G::FM; i++)
#pragma unroll
                for (int j = 0; j < G::FN; j++)
                    tmp[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw[j], af[i], kk == 0 ? f32x16_t{} : tmp[i][j], 0, 0, 0);
        }
        // acc += s_n * (T + X_m)
        float xm[G::FM];
#pragma unroll
        for (int i = 0; i < G::FM; i++) xm[i] = sx[wm * G::TM + i * 32 + l32];
#pragma unroll
        for (int j = 0; j < G::FN; j++) {
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const uint32_t ncol = wn * G::TN + j * 32 + 8 * q4 + 4 * h;
                const u32x2_t sv = *(const LDS_AS u32x2_t*)(ss + ncol);
                const float s0 = __uint_as_float(sv[0] << 16), s1 = __uint_as_float(sv[0] & 0xFFFF0000u);
                const float s2 = __uint_as_float(sv[1] << 16), s3 = __uint_as_float(sv[1] & 0xFFFF0000u);
#pragma unroll
                for (int i = 0; i < G::FM; i++) {
                    acc[i][j][4 * q4 + 0] = fmaf(s0, tmp[i][j][4 * q4 + 0] + xm[i], acc[i][j][4 * q4 + 0]);
                    acc[i][j][4 * q4 + 1] = fmaf(s1, tmp[i][j][4 * q4 + 1] + xm[i], acc[i][j][4 * q4 + 1]);
                    acc[i][j][4 * q4 + 2] = fmaf(s2, tmp[i][j][4 * q4 + 2] + xm[i], acc[i][j][4 * q4 + 2]);
                    acc[i][j][4 * q4 + 3] = fmaf(s3, tmp[i][j][4 * q4 + 3] + xm[i], acc[i][j][4 * q4 + 3]);
                }
            }
        }
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

// X[g][m] = -144 * sum_{k in group g} a[m][k]   (prefill pre-pass, group 128)
__device__ __forceinline__ void w4_rowsum(const t0_w4a16_params& p) {
    // one wave per (m, 8 groups): lane covers 16 k of a group
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wid = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
    const uint32_t G = p.K / 128;
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
    if (g < G && (lane % 8) == 0) p.workspace[(size_t)g * p.M + m] = -144.0f * s;
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

#define T0_W4_DECODE(WAVES, MB)                                                                  \
    extern "C" __global__ void __launch_bounds__(WAVES * 64)                                      \
        t0k_w4a16_decode_w##WAVES##_mb##MB(const t0_w4a16_params p) {                             \
        t0::w4_decode<WAVES, MB>(p);                                                             \
    }
T0_W4_DECODE(4, 1)
T0_W4_DECODE(8, 1)
T0_W4_DECODE(4, 2)
T0_W4_DECODE(4, 4)

#define T0_W4_PREFILL(BM, BN, WM, WN, ST)                                                        \
    extern "C" __global__ void __launch_bounds__(WM * WN * 64)                                    \
        t0k_w4a16_prefill_##BM##x##BN##_w##WM##x##WN##_s##ST(const t0_w4a16_params p) {          \
        t0::w4_prefill<BM, BN, WM, WN, ST>(p);                                                   \
    }
T0_W4_PREFILL(256, 128, 2, 2, 2)
T0_W4_PREFILL(128, 128, 2, 2, 2)

extern "C" __global__ void __launch_bounds__(256) t0k_w4a16_rowsum(const t0_w4a16_params p) { t0::w4_rowsum(p); }
extern "C" __global__ void __launch_bounds__(256) t0k_w4a16_generic(const t0_w4a16_params p) { t0::w4_generic(p); }
extern "C" __global__ void __launch_bounds__(256) dequant_int4_f32(const t0_dequant_params p) { t0::dequant_int4(p, false); }
extern "C" __global__ void __launch_bounds__(256) dequant_int4_bf16(const t0_dequant_params p) { t0::dequant_int4(p, true); }

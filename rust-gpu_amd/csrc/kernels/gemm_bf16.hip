// gemm_bf16.hip -- tiled bf16 GEMM for gfx950 (MI355X).
//
//   C[M,N] = epilogue( A[M,K] . B )    bf16 in, f32 accumulate, f32 or bf16 out
//   NT: B = WT[N,K] (k contiguous)     -- the reference's only form
//       (src/t0/gemm_gen.rs:51-54, src/t0/tile_ir.rs:106-107)
//   NN: B = B[K,N]  (n contiguous)     -- new; read through ds_read_b64_tr_b16
//
// One workgroup owns a BM x BN output tile, WM x WN waves each own a
// (BM/WM) x (BN/WN) sub-tile built from 32x32 blocks of
// v_mfma_f32_32x32x16_bf16.  A and B tiles move HBM -> LDS with
// buffer_load_dwordx4 ... lds (no VGPR staging) through STAGES LDS buffers;
// 16-byte chunks are XOR-swizzled per row so the MFMA operand reads are
// bank-conflict free.  Rows/columns past M/N and k past K are read as zero
// through buffer out-of-range masking, so any M, N and K (K % 8 == 0,
// 16-byte aligned rows) is handled without host padding -- the bounds
// behaviour of src/t0/tile_ir.rs:1142-1185 rather than gemm_gen's
// divisibility requirement (src/t0/cost_model.rs:499-500).
//
// Split-K follows the reference: partition p of split_k covers
// K-range [p*Kp, (p+1)*Kp) with Kp = K / split_k and writes a full f32 plane
// at C + p*y_split_stride (src/t0/gemm_gen.rs:769-793).  With T0_GEMM_FIXUP
// the partitions are instead reduced in-kernel, in plane order, by the last
// partition to finish (deterministic), and the epilogue runs once.
#include "common.h"

namespace t0 {

template <int BM, int BN, int BK, int WM, int WN, bool NN, int STAGES>
struct GemmCfg {
    static constexpr int NW = WM * WN;
    static constexpr int NT = NW * 64;
    static constexpr int TM = BM / WM, TN = BN / WN;
    static constexpr int FM = TM / 32, FN = TN / 32;
    static constexpr int A_BYTES = BM * BK * 2;
    static constexpr int B_BYTES = BN * BK * 2;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    static constexpr int A_LOADS = A_BYTES / (1024 * NW);  // per wave per stage
    static constexpr int B_LOADS = B_BYTES / (1024 * NW);
    static constexpr int LOADS = A_LOADS + B_LOADS;
    static constexpr int CHA = BK / 8;          // 16-B chunks per A (and NT-B) row
    static constexpr int CHB = BN / 8;          // 16-B chunks per NN-B row
    static constexpr int EPI_LD = TN + 4;       // staged epilogue row stride (floats)
    static constexpr int EPI_WAVE_FLOATS = 32 * EPI_LD;
    static constexpr int SMEM_BYTES = (STAGE_BYTES * STAGES > NW * EPI_WAVE_FLOATS * 4)
                                          ? STAGE_BYTES * STAGES : NW * EPI_WAVE_FLOATS * 4;
    static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be 32x32 blocks");
    static_assert(BK % 16 == 0, "BK must be a multiple of 16");
    static_assert(A_LOADS >= 1 && A_LOADS * 1024 * NW == A_BYTES, "A tile / load split");
    static_assert(B_LOADS >= 1 && B_LOADS * 1024 * NW == B_BYTES, "B tile / load split");
    static_assert(STAGES >= 2, "at least double buffering");
    static_assert(STAGE_BYTES * STAGES <= 160 * 1024, "LDS");
};

template <class G>
struct TileLoader {
    // per-lane byte offsets relative to the stage's tile base, or OOB
    uint32_t a_off[G::A_LOADS];
    uint32_t b_off[G::B_LOADS];
    uint32_t a_kchunk[G::A_LOADS];  // k offset (elements) of the lane's chunk within the stage
    uint32_t b_krow[G::B_LOADS];    // NN: k row within the stage; NT: k chunk offset
};

// Epilogue + bounds-checked store of 4 consecutive columns n..n+3 of row m.
T0_DEV void store_quad(const t0_gemm_params& p, uint8_t* Cb, uint32_t m, uint32_t n, f32x4_t v) {
    if (m >= p.M || n >= p.N) return;
    const uint32_t N = p.N;
    const uint32_t ops = p.epi_ops;
    if (ops) {
        const bool has_bias = epi_has_bias(ops);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float bv = (has_bias && n + e < N) ? p.bias[n + e] : 0.0f;
            v[e] = apply_epilogue(v[e], ops, bv, p.epi_scale, p.clamp_lo, p.clamp_hi);
        }
    }
    // n is a multiple of 4: a quad is 8/16-byte aligned when ldc is a multiple of 4
    const bool vec = n + 3 < N && (p.ldc & 3u) == 0;
    if (p.flags & T0_GEMM_OUT_BF16) {
        uint16_t* dst = (uint16_t*)Cb + (size_t)m * p.ldc + n;
        if (vec) {
            *(u32x2_t*)dst = u32x2_t{pack2_bf16_rne(v[0], v[1]), pack2_bf16_rne(v[2], v[3])};
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (n + e < N) dst[e] = (uint16_t)(pack2_bf16_rne(v[e], 0.0f) & 0xFFFFu);
        }
    } else {
        float* dst = (float*)Cb + (size_t)m * p.ldc + n;
        if (vec) {
            *(f32x4_t*)dst = v;
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (n + e < N) dst[e] = v[e];
        }
    }
}

// Write one staged 32 x TN block (wave-private LDS, row stride EPI_LD floats)
// to C rows [row0, row0+32), columns [col0, col0+TN), row-major, one 4-column
// quad per lane per step.
template <class G>
T0_DEV void emit_rowblock(const t0_gemm_params& p, uint8_t* Cb, const float* wreg,
                          uint32_t row0, uint32_t col0, uint32_t lane) {
    // Interior block, no epilogue chain, 16-byte aligned rows: 8 columns per
    // lane, one 16-byte bf16 store (or two f32 stores), fully unrolled.
    const bool bf16_out = p.flags & T0_GEMM_OUT_BF16;
    if (p.epi_ops == 0 && row0 + 32 <= p.M && col0 + G::TN <= p.N && (p.ldc & (bf16_out ? 7u : 3u)) == 0) {
        constexpr uint32_t LPR = G::TN / 8;            // lanes per row
        constexpr uint32_t RPI = 64 / LPR;             // rows per iteration
        const uint32_t rr = lane / LPR, c8 = (lane % LPR) * 8;
#pragma unroll
        for (uint32_t r = rr; r < 32; r += RPI) {
            const LDS_AS float* src = (const LDS_AS float*)wreg + r * G::EPI_LD + c8;
            const f32x4_t v0 = *(const LDS_AS f32x4_t*)src;
            const f32x4_t v1 = *(const LDS_AS f32x4_t*)(src + 4);
            const size_t idx = (size_t)(row0 + r) * p.ldc + col0 + c8;
            if (bf16_out) {
                *(u32x4_t*)((uint16_t*)Cb + idx) = u32x4_t{pack2_bf16_rne(v0[0], v0[1]), pack2_bf16_rne(v0[2], v0[3]),
                                                           pack2_bf16_rne(v1[0], v1[1]), pack2_bf16_rne(v1[2], v1[3])};
            } else {
                *(f32x4_t*)((float*)Cb + idx) = v0;
                *(f32x4_t*)((float*)Cb + idx + 4) = v1;
            }
        }
        return;
    }
    constexpr uint32_t QPR = G::TN / 4;  // quads per row
#pragma unroll 1
    for (uint32_t q = lane; q < 32 * QPR; q += 64) {
        const uint32_t r = q / QPR, c4 = q % QPR;
        f32x4_t v = *(const LDS_AS f32x4_t*)(wreg + r * G::EPI_LD + c4 * 4);
        store_quad(p, Cb, row0 + r, col0 + c4 * 4, v);
    }
}

template <int BM, int BN, int BK, int WM, int WN, bool NN, int STAGES, int VGD = 0>
__device__ __forceinline__ void gemm_tile_kernel(const t0_gemm_params& p) {
    using G = GemmCfg<BM, BN, BK, WM, WN, NN, STAGES>;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[G::SMEM_BYTES];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: DMA targets in SGPRs
    const uint32_t wm = wave / WN, wn = wave % WN;

    // ---- tile assignment -------------------------------------------------
    const uint32_t M = p.M, N = p.N, K = p.K;
    const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const uint32_t tiles = tiles_m * tiles_n;
    const uint32_t sk = p.split_k;
    const uint32_t total = tiles * sk;
    const uint32_t bid = blockIdx.y * gridDim.x + blockIdx.x;
    if (bid >= total) return;
    uint64_t* const probe = p.clock_probe;
    if (probe && tid == 0) {
        probe[4 * bid] = __builtin_amdgcn_s_memrealtime();
        probe[4 * bid + 2] = __builtin_amdgcn_s_memtime();
    }
    const uint32_t lid = xcd_remap(bid, total);
    const uint32_t part = lid / tiles;
    const uint32_t tile_id = lid % tiles;
    uint32_t tm, tn;
    grouped_tile(tile_id, tiles_m, tiles_n, 4, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const uint32_t k_per = K / sk;                 // reference: k_end = K >> shift
    const uint32_t k_begin = part * k_per;
    const uint32_t k_end = (part + 1 == sk) ? K : k_begin + k_per;
    const uint32_t k_len = k_end - k_begin;
    const uint32_t nk = (k_len + BK - 1) / BK;

    const uint32_t lda = p.lda, ldb = p.ldb;
    const uint8_t* A0 = (const uint8_t*)p.A + ((size_t)m0 * lda + k_begin) * 2;
    const uint8_t* B0 = NN ? (const uint8_t*)p.B + ((size_t)k_begin * ldb + n0) * 2
                           : (const uint8_t*)p.B + ((size_t)n0 * ldb + k_begin) * 2;

    // ---- per-lane load offsets (constant over the K loop) ------------------
    TileLoader<G> ld;
#pragma unroll
    for (int j = 0; j < G::A_LOADS; j++) {
        uint32_t pos = (wave * G::A_LOADS + j) * 1024 + lane * 16;
        uint32_t r = pos / (BK * 2), s = (pos % (BK * 2)) / 16;
        uint32_t c = s ^ swz_rows<G::CHA>(r);
        bool ok = (m0 + r) < M;
        ld.a_off[j] = ok ? r * lda * 2 + c * 16 : OOB_OFFSET;
        ld.a_kchunk[j] = c * 8;
    }
#pragma unroll
    for (int j = 0; j < G::B_LOADS; j++) {
        uint32_t pos = (wave * G::B_LOADS + j) * 1024 + lane * 16;
        if constexpr (NN) {
            uint32_t r = pos / (BN * 2), s = (pos % (BN * 2)) / 16;
            uint32_t c = s ^ swz_nn<G::CHB>(r);
            bool ok = (n0 + c * 8) < N;
            ld.b_off[j] = ok ? r * ldb * 2 + c * 16 : OOB_OFFSET;
            ld.b_krow[j] = r;
        } else {
            uint32_t r = pos / (BK * 2), s = (pos % (BK * 2)) / 16;
            uint32_t c = s ^ swz_rows<G::CHA>(r);
            bool ok = (n0 + r) < N;
            ld.b_off[j] = ok ? r * ldb * 2 + c * 16 : OOB_OFFSET;
            ld.b_krow[j] = c * 8;
        }
    }

    const uint32_t lds_base = (uint32_t)(uintptr_t)(LDS_AS uint8_t*)smem;
    // With two waves per SIMD (8 waves, two stages), only waves 0..NW/2-1
    // issue the DMAs of a full stage of an interior tile: theirs and those of
    // wave + NW/2, whose chunks sit BM/2 rows of A and BK/2 k-rows (NN) or
    // BN/2 rows (NT) of B further on, at the same per-lane offsets.  An LDS-DMA
    // instruction holds its wave for tens of cycles at issue; this way the
    // other wave on each SIMD keeps the MFMA pipe busy meanwhile.
    constexpr bool PAIR_DMA = G::NW == 8 && STAGES == 2;
    const bool pair_dma = PAIR_DMA && m0 + BM <= M && n0 + BN <= N;
    // Issues the loads q of stage t with q % nparts == part (A loads first,
    // then B), so a stage can go out in slices between MFMA groups.
    auto issue_stage = [&](uint32_t t, int part, int nparts) {
        const uint32_t kt = t * BK;                 // k offset within the partition
        const uint32_t st = lds_base + (t % STAGES) * G::STAGE_BYTES;
        const bool tail = kt + BK > k_len;
        __amdgpu_buffer_rsrc_t ra = make_rsrc(A0 + (size_t)kt * 2);
        __amdgpu_buffer_rsrc_t rb = make_rsrc(NN ? B0 + (size_t)kt * ldb * 2 : B0 + (size_t)kt * 2);
        if (PAIR_DMA && pair_dma && !tail && nparts == 1) {
            if (wave < G::NW / 2) {
                constexpr uint32_t HA = G::NW / 2 * G::A_LOADS * 1024, HB = G::NW / 2 * G::B_LOADS * 1024;
                __amdgpu_buffer_rsrc_t ra2 = make_rsrc(A0 + (size_t)kt * 2 + (size_t)(BM / 2) * lda * 2);
                __amdgpu_buffer_rsrc_t rb2 = make_rsrc(NN ? B0 + (size_t)(kt + BK / 2) * ldb * 2
                                                          : B0 + (size_t)kt * 2 + (size_t)(BN / 2) * ldb * 2);
#pragma unroll
                for (int j = 0; j < G::A_LOADS; j++) {
                    dma_x4(ra, __builtin_amdgcn_readfirstlane(st + (wave * G::A_LOADS + j) * 1024), ld.a_off[j]);
                    dma_x4(ra2, __builtin_amdgcn_readfirstlane(st + HA + (wave * G::A_LOADS + j) * 1024), ld.a_off[j]);
                }
#pragma unroll
                for (int j = 0; j < G::B_LOADS; j++) {
                    dma_x4(rb, __builtin_amdgcn_readfirstlane(st + G::A_BYTES + (wave * G::B_LOADS + j) * 1024),
                           ld.b_off[j]);
                    dma_x4(rb2, __builtin_amdgcn_readfirstlane(st + G::A_BYTES + HB + (wave * G::B_LOADS + j) * 1024),
                           ld.b_off[j]);
                }
            }
            return;
        }
        // a full stage takes the precomputed offsets as they are; only the
        // K tail masks per chunk (a uniform branch, so no selects otherwise)
        if (!tail) {
#pragma unroll
            for (int j = 0; j < G::A_LOADS; j++)
                if (j % nparts == part)
                    dma_x4(ra, __builtin_amdgcn_readfirstlane(st + (wave * G::A_LOADS + j) * 1024), ld.a_off[j]);
#pragma unroll
            for (int j = 0; j < G::B_LOADS; j++)
                if ((G::A_LOADS + j) % nparts == part)
                    dma_x4(rb, __builtin_amdgcn_readfirstlane(st + G::A_BYTES + (wave * G::B_LOADS + j) * 1024),
                           ld.b_off[j]);
            return;
        }
#pragma unroll
        for (int j = 0; j < G::A_LOADS; j++) {
            if (j % nparts != part) continue;
            uint32_t off = ld.a_off[j];
            if (kt + ld.a_kchunk[j] >= k_len) off = OOB_OFFSET;
            dma_x4(ra, __builtin_amdgcn_readfirstlane(st + (wave * G::A_LOADS + j) * 1024), off);
        }
#pragma unroll
        for (int j = 0; j < G::B_LOADS; j++) {
            if ((G::A_LOADS + j) % nparts != part) continue;
            uint32_t off = ld.b_off[j];
            if (kt + ld.b_krow[j] >= k_len) off = OOB_OFFSET;
            dma_x4(rb, __builtin_amdgcn_readfirstlane(st + G::A_BYTES + (wave * G::B_LOADS + j) * 1024), off);
        }
    };

    f32x16_t acc[G::FM][G::FN];
#pragma unroll
    for (int i = 0; i < G::FM; i++)
#pragma unroll
        for (int j = 0; j < G::FN; j++) acc[i][j] = f32x16_t{};

    // ---- per-lane operand read offsets (constant over the K loop) ------------
    // The swizzle of every row a lane reads depends only on the lane, so each
    // operand address is lane_base + per-kk chunk term + compile-time offset.
    const uint32_t l32 = lane & 31, hi = lane >> 5;
    const uint32_t a_lane = (wm * G::TM + l32) * (BK * 2);
    const uint32_t a_swz = swz_rows<G::CHA>(l32);
    uint32_t a_kk[BK / 16];
#pragma unroll
    for (int kk = 0; kk < BK / 16; kk++) a_kk[kk] = a_lane + (((kk * 2 + hi) ^ a_swz) * 16);
    uint32_t b_kk[BK / 16];      // NT
    uint32_t b_col[G::FN];       // NN
    uint32_t b_row = 0;          // NN
    if constexpr (NN) {
        const uint32_t g = lane >> 4, i16 = lane & 15;
        const uint32_t s = swz_nn<G::CHB>(i16 >> 2);
        b_row = ((g >> 1) * 8 + (i16 >> 2)) * (BN * 2);
#pragma unroll
        for (int j = 0; j < G::FN; j++) {
            const uint32_t c16 = (wn * G::TN + j * 32) / 8 + (g & 1) * 2 + (i16 & 3) / 2;
            b_col[j] = b_row + ((c16 ^ s) * 16) + (i16 & 1) * 8;
        }
    } else {
        const uint32_t b_lane = (wn * G::TN + l32) * (BK * 2);
#pragma unroll
        for (int kk = 0; kk < BK / 16; kk++) b_kk[kk] = b_lane + (((kk * 2 + hi) ^ a_swz) * 16);
    }

    // ---- K loop -------------------------------------------------------------
    // Every buffer is filled up front.  Step t computes from buffer
    // t % STAGES in BK/16 sub-steps whose operand fragments are
    // double-buffered in registers.  In the last sub-step of step t, once its
    // fragments are in registers, the workgroup waits for stage t+1,
    // synchronises, refills buffer t % STAGES with stage t+STAGES and reads
    // the first fragments of step t+1, so the barrier and the first LDS reads
    // of a step run under the MFMAs of the previous one.
    constexpr int KK = BK / 16;
    auto stage_ptr = [&](uint32_t t) { return (const LDS_AS uint8_t*)smem + (t % STAGES) * G::STAGE_BYTES; };
    auto load_frags = [&](const LDS_AS uint8_t* sa, int kk, bf16x8_t* af, bf16x8_t* bfr) {
        const LDS_AS uint8_t* sb = sa + G::A_BYTES;
#pragma unroll
        for (int i = 0; i < G::FM; i++)
            af[i] = *(const LDS_AS bf16x8_t*)(sa + a_kk[kk] + i * 32 * (BK * 2));
#pragma unroll
        for (int j = 0; j < G::FN; j++) {
            if constexpr (NN) {
                const LDS_AS uint8_t* p0 = sb + b_col[j] + kk * 16 * (BN * 2);
                bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((LDS_AS bf16x4_t*)p0);
                bf16x4_t hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((LDS_AS bf16x4_t*)(p0 + 4 * (BN * 2)));
                bfr[j] = __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
            } else {
                bfr[j] = *(const LDS_AS bf16x8_t*)(sb + b_kk[kk] + j * 32 * (BK * 2));
            }
        }
    };
    auto mfmas = [&](const bf16x8_t* af, const bf16x8_t* bfr) {
#pragma unroll
        for (int i = 0; i < G::FM; i++)
#pragma unroll
            for (int j = 0; j < G::FN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    };
    // keeps this sub-step's LDS reads (and DMA) ahead of its MFMAs: all of
    // them first with one wave per SIMD (the scheduler would otherwise sink
    // them next to their uses), one read per MFMA with two waves per SIMD
    auto order_substep = [&]() {
        if constexpr (G::NW < 8) {
            __builtin_amdgcn_sched_barrier(0);
        } else {
            constexpr int NR = G::FM + (NN ? 2 : 1) * G::FN;
            constexpr int REST = G::FM * G::FN - NR;
#pragma unroll
            for (int q = 0; q < NR; q++) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
            }
            if constexpr (REST > 0) __builtin_amdgcn_sched_group_barrier(0x008, REST, 0);
        }
    };

    // ---- ping-pong K loop (256 x 256 x 32, 8 waves, 4 stages) ---------------
    // Waves 0-3 (rows 0-127) and 4-7 (rows 128-255) share the SIMDs in pairs
    // (wave s and s + 4 on SIMD s) and run in opposite phases: in every
    // phase one wave of each pair issues the 16 MFMAs of a 32-k stage from
    // registers while the other reads its fragments of the next stage from
    // LDS and issues its half of a later stage's DMA (waves 0-3 the A
    // chunks, waves 4-7 the B chunks).  A barrier ends every phase, so no
    // barrier ever finds both waves of a SIMD without MFMA work.
    //   waves 0-3: LOAD(0) | COMPUTE(0) | LOAD(1) | COMPUTE(1) | ...
    //   waves 4-7:   idle  |  LOAD(0)   | COMPUTE(0) | LOAD(1)  | ...
    // Stage t lives in buffer t % 4; LOAD(i) issues stage i + 3 into the
    // buffer of stage i - 1, which every wave finished reading (and waited
    // for) before the barrier that precedes it.
    // Measured at 4096^3: 112-117 us against 101-102 us for the two-stage
    // 256 x 256 x 64 schedule on the same box.  With one reading wave per
    // SIMD a LOAD phase takes ~700 cycles (16 fragment reads ~350, since the
    // CU's LDS read rate drops to ~180 B/clk for b128 and ~105 B/clk for the
    // transposing reads; 4 DMAs ~250 at the CU's 64 B/clk global->LDS rate)
    // against the 16 MFMAs' ~520, so the MFMA pipes wait on the loads.
    constexpr bool PP = BM == 256 && BN == 256 && BK == 32 && G::NW == 8 && STAGES == 4 && WM == 2;
    uint64_t y_split_stride = 0;
    if constexpr (PP) {
        const bool is_y = wave >= 4;     // SGPR: uniform branches
        constexpr int PPL = 4;           // DMA chunks per wave per stage (16 KB of A or of B over 4 waves)
        static_assert(G::A_BYTES == PPL * 4 * 1024 && G::B_BYTES == PPL * 4 * 1024, "ping-pong DMA split");
        uint32_t d_off[PPL], d_k[PPL], d_lds[PPL];
#pragma unroll
        for (int j = 0; j < PPL; j++) {
            const uint32_t q = (wave & 3) * PPL + j;             // 1 KB chunk of the A or B tile
            const uint32_t pos = q * 1024 + lane * 16;
            if (!is_y) {
                const uint32_t r = pos / (BK * 2), s = (pos % (BK * 2)) / 16;
                const uint32_t c = s ^ swz_rows<G::CHA>(r);
                d_off[j] = (m0 + r) < M ? r * lda * 2 + c * 16 : OOB_OFFSET;
                d_k[j] = c * 8;
                d_lds[j] = q * 1024;
            } else if constexpr (NN) {
                const uint32_t r = pos / (BN * 2), s = (pos % (BN * 2)) / 16;
                const uint32_t c = s ^ swz_nn<G::CHB>(r);
                d_off[j] = (n0 + c * 8) < N ? r * ldb * 2 + c * 16 : OOB_OFFSET;
                d_k[j] = r;
                d_lds[j] = G::A_BYTES + q * 1024;
            } else {
                const uint32_t r = pos / (BK * 2), s = (pos % (BK * 2)) / 16;
                const uint32_t c = s ^ swz_rows<G::CHA>(r);
                d_off[j] = (n0 + r) < N ? r * ldb * 2 + c * 16 : OOB_OFFSET;
                d_k[j] = c * 8;
                d_lds[j] = G::A_BYTES + q * 1024;
            }
        }
        // this wave's PPL chunks of stage t (a K-tail stage masks per chunk,
        // so every stage issues the same number of loads)
        auto pp_issue = [&](uint32_t t) {
            const uint32_t kt = t * BK;
            const uint32_t st = lds_base + (t % STAGES) * G::STAGE_BYTES;
            const bool tail = kt + BK > k_len;
            const uint8_t* src = is_y ? (NN ? B0 + (size_t)kt * ldb * 2 : B0 + (size_t)kt * 2) : A0 + (size_t)kt * 2;
            __amdgpu_buffer_rsrc_t r = make_rsrc(src);
            if (!tail) {
#pragma unroll
                for (int j = 0; j < PPL; j++) dma_x4(r, __builtin_amdgcn_readfirstlane(st + d_lds[j]), d_off[j]);
            } else {
#pragma unroll
                for (int j = 0; j < PPL; j++)
                    dma_x4(r, __builtin_amdgcn_readfirstlane(st + d_lds[j]), kt + d_k[j] >= k_len ? OOB_OFFSET : d_off[j]);
            }
        };
        // at most `ahead` later stages of this wave's DMAs still in flight
        auto pp_wait = [&](uint32_t ahead) {
            if (ahead >= 2) wait_vmcnt_fence<2 * PPL>();
            else if (ahead == 1) wait_vmcnt_fence<PPL>();
            else wait_vmcnt_fence<0>();
        };
        auto pp_barrier = [&]() {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        };
        const uint32_t nh = nk;                          // 32-k stages
#pragma unroll
        for (uint32_t s = 0; s < 3; s++)
            if (s < nh) pp_issue(s);
        pp_wait(nh > 0 ? (nh - 1 < 2 ? nh - 1 : 2) : 0);   // stage 0 landed
        y_split_stride = p.y_split_stride;
        asm volatile("" : "+s"(y_split_stride));
        pp_barrier();
        if (is_y) pp_barrier();                          // waves 4-7 start one phase later
        bf16x8_t pa[2][G::FM], pb[2][G::FN];
        for (uint32_t i = 0; i < nh; i++) {
            // LOAD(i): fragments of stage i, then this wave's share of stage i + 3
            const LDS_AS uint8_t* sa = stage_ptr(i);
            load_frags(sa, 0, pa[0], pb[0]);
            load_frags(sa, 1, pa[1], pb[1]);
            if (i + 3 < nh) pp_issue(i + 3);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            // stage i + 1 must have landed in every wave before the barrier
            // that ends the phase after which waves 0-3 read it
            const uint32_t ahead = nh - 1 > i + 1 ? (nh - 2 - i < 2 ? nh - 2 - i : 2) : 0;
            if (is_y) pp_wait(ahead);
            pp_barrier();
            // COMPUTE(i)
            mfmas(pa[0], pb[0]);
            mfmas(pa[1], pb[1]);
            if (!is_y) pp_wait(ahead);
            if (!(is_y && i + 1 == nh)) pp_barrier();
        }
    }

    // ---- lean K loop (8 waves, two stages, interior tile, whole 64-k steps) ---
    // The schedule of the loop below without its edge cases: waves 0-3 issue
    // every DMA of a stage right after the step's barrier, each sub-step reads
    // the next sub-step's fragments one per MFMA, the last step is peeled.
    // With no K-tail or bounds branch in the body, the operand registers keep
    // one assignment across the loop back-edge (no register copies), which
    // takes ~8 % of the shader cycles off 4096^3 (147.7k against 160.5k per
    // workgroup on one box).  Bit-identical to the general loop: the same
    // MFMAs accumulate in the same order.
    constexpr bool LEAN = PAIR_DMA && !PP && KK == 4;
    bool lean = false;
    if constexpr (LEAN) lean = pair_dma && k_len % BK == 0 && nk >= 2;
    if constexpr (LEAN) {
        if (lean) {
            constexpr uint32_t HA = G::NW / 2 * G::A_LOADS * 1024, HB = G::NW / 2 * G::B_LOADS * 1024;
            // waves 0-3: their chunks of stage t and those of wave + 4
            auto lean_issue = [&](uint32_t t) {
                if (wave < G::NW / 2) {
                    const uint32_t kt = t * BK;
                    const uint32_t st = lds_base + (t & 1) * G::STAGE_BYTES;
                    const __amdgpu_buffer_rsrc_t ra = make_rsrc(A0 + (size_t)kt * 2);
                    const __amdgpu_buffer_rsrc_t ra2 = make_rsrc(A0 + (size_t)kt * 2 + (size_t)(BM / 2) * lda * 2);
                    const __amdgpu_buffer_rsrc_t rb = make_rsrc(NN ? B0 + (size_t)kt * ldb * 2 : B0 + (size_t)kt * 2);
                    const __amdgpu_buffer_rsrc_t rb2 = make_rsrc(NN ? B0 + (size_t)(kt + BK / 2) * ldb * 2
                                                                    : B0 + (size_t)kt * 2 + (size_t)(BN / 2) * ldb * 2);
#pragma unroll
                    for (int j = 0; j < G::A_LOADS; j++) {
                        dma_x4(ra, __builtin_amdgcn_readfirstlane(st + (wave * G::A_LOADS + j) * 1024), ld.a_off[j]);
                        dma_x4(ra2, __builtin_amdgcn_readfirstlane(st + HA + (wave * G::A_LOADS + j) * 1024), ld.a_off[j]);
                    }
#pragma unroll
                    for (int j = 0; j < G::B_LOADS; j++) {
                        dma_x4(rb, __builtin_amdgcn_readfirstlane(st + G::A_BYTES + (wave * G::B_LOADS + j) * 1024),
                               ld.b_off[j]);
                        dma_x4(rb2, __builtin_amdgcn_readfirstlane(st + G::A_BYTES + HB + (wave * G::B_LOADS + j) * 1024),
                               ld.b_off[j]);
                    }
                }
            };
            constexpr int BH = NN ? 2 : 1;                   // LDS reads per B fragment
            constexpr int NQ = G::FM * G::FN;                // MFMAs per sub-step
            constexpr int NR = G::FM + BH * G::FN;           // fragment reads per sub-step
            bf16x8_t la[2][G::FM];
            bf16x4_t lb[2][G::FN][2];                        // NN: the two transposing halves
            bf16x8_t lbt[2][G::FN];                          // NT
            // read q of sub-step KK_'s fragments into buffer BUF
            auto lean_read = [&](const LDS_AS uint8_t* sa, auto KKc, auto BUFc, auto Qc) {
                constexpr int kk = decltype(KKc)::value, buf = decltype(BUFc)::value, q = decltype(Qc)::value;
                const LDS_AS uint8_t* sb = sa + G::A_BYTES;
                if constexpr (q < G::FM) {
                    la[buf][q] = *(const LDS_AS bf16x8_t*)(sa + a_kk[kk] + q * 32 * (BK * 2));
                } else if constexpr (NN) {
                    constexpr int j = (q - G::FM) / 2, h = (q - G::FM) % 2;
                    lb[buf][j][h] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
                        (LDS_AS bf16x4_t*)(sb + b_col[j] + kk * 16 * (BN * 2) + h * 4 * (BN * 2)));
                } else {
                    constexpr int j = q - G::FM;
                    lbt[buf][j] = *(const LDS_AS bf16x8_t*)(sb + b_kk[kk] + j * 32 * (BK * 2));
                }
            };
            auto lean_mfma = [&](auto BUFc, auto Qc) {
                constexpr int buf = decltype(BUFc)::value, q = decltype(Qc)::value;
                constexpr int i = q / G::FN, j = q % G::FN;
                bf16x8_t b;
                if constexpr (NN) b = __builtin_shufflevector(lb[buf][j][0], lb[buf][j][1], 0, 1, 2, 3, 4, 5, 6, 7);
                else b = lbt[buf][j];
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, la[buf][i], acc[i][j], 0, 0, 0);
            };
            // NQ MFMAs from buffer CUR, the reads of (sa_next, KKN) into CUR ^ 1 one per MFMA
            auto lean_sub = [&](auto CURc, const LDS_AS uint8_t* sa_next, auto KKNc, auto READc) {
                constexpr int cur = decltype(CURc)::value;
                constexpr bool rd = decltype(READc)::value != 0;
                static_for<0, (NR > NQ ? NR : NQ)>([&](auto Q) {
                    constexpr int q = decltype(Q)::value;
                    if constexpr (rd && q < NR) lean_read(sa_next, KKNc, Idx<cur ^ 1>{}, Q);
                    if constexpr (q < NQ) lean_mfma(CURc, Q);
                });
                static_for<0, (NR < NQ ? NR : NQ)>([&](auto) {
                    if constexpr (rd) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                    // MFMA
                });
            };
            lean_issue(0);
            lean_issue(1);
            wait_vmcnt<G::A_LOADS * 2 + G::B_LOADS * 2>();   // stage 0 landed (waves 0-3)
            y_split_stride = p.y_split_stride;
            asm volatile("" : "+s"(y_split_stride));
            __syncthreads();
            static_for<0, NR>([&](auto Q) { lean_read(stage_ptr(0), Idx<0>{}, Idx<0>{}, Q); });
            for (uint32_t t = 0; t + 1 < nk; t++) {
                const LDS_AS uint8_t* sa = stage_ptr(t);
                lean_sub(Idx<0>{}, sa, Idx<1>{}, Idx<1>{});
                lean_sub(Idx<1>{}, sa, Idx<2>{}, Idx<1>{});
                lean_sub(Idx<0>{}, sa, Idx<3>{}, Idx<1>{});
                // stage t + 1 landed in every wave, buffer t % 2 read by all
                wait_vmcnt<0>();
                __syncthreads();
                if (t + 2 < nk) lean_issue(t + 2);
                lean_sub(Idx<1>{}, stage_ptr(t + 1), Idx<0>{}, Idx<1>{});
            }
            const LDS_AS uint8_t* sa = stage_ptr(nk - 1);
            lean_sub(Idx<0>{}, sa, Idx<1>{}, Idx<1>{});
            lean_sub(Idx<1>{}, sa, Idx<2>{}, Idx<1>{});
            lean_sub(Idx<0>{}, sa, Idx<3>{}, Idx<1>{});
            lean_sub(Idx<1>{}, sa, Idx<0>{}, Idx<0>{});
        }
    }

    // ---- register-staged K loop (VGD > 0; whole 64-k steps) -----------------
    // For the memory-bound small tiles: every lane loads its 16-byte chunks of
    // a stage into registers, VGD stages ahead, and writes them with
    // ds_write_b128 to the position its global->LDS DMA would have filled
    // (same swizzle, so the fragment reads are unchanged), into one of two
    // LDS buffers.  Step t computes from buffer t % 2; in its first sub-step
    // every wave writes stage t + 1 (its loads issued VGD - 1 steps earlier)
    // to the other buffer, which step t - 1's barrier freed, and refills
    // those registers with stage t + 1 + VGD; one barrier (LDS writes
    // complete, no load wait) at the last sub-step.  The same MFMAs in the
    // same order as the DMA loop: bit-identical.  On the skinny GEMM
    // (128x4096x4096, 64x128 split 4) VGD = 2 takes 16.8-16.9 us against
    // 17.3-17.4 by DMA (VGD 1: 19.0, 4: 17.2, 8: 17.2); a stage-read floor
    // of that tiling moves its operand slices 13 % faster this way.
    bool vg = false;
    if constexpr (VGD > 0) vg = k_len % BK == 0 && nk % VGD == 0 && nk >= VGD;
    if constexpr (VGD > 0) {
        static_assert(KK >= 2 && KK % 2 == 0 && !PP && !LEAN, "register staging: the two-buffer loop");
        if (vg) {
            u32x4_t rg[VGD][G::LOADS];
            // stage t into register set S; a stage past the last reads zeros
            // without touching memory.  Branch-free (the offset is raised to
            // OOB_OFFSET by a max with an opaque scalar), so every step issues
            // the same loads and the compiler's load counting stays exact.
            auto vg_issue = [&](auto Sc, uint32_t t) {
                constexpr int S = decltype(Sc)::value;
                const bool live = t < nk;
                uint32_t lim = live ? 0u : OOB_OFFSET;
                asm volatile("" : "+s"(lim));
                const uint32_t kt = live ? t * BK : 0;
                const __amdgpu_buffer_rsrc_t ra = make_rsrc(A0 + (size_t)kt * 2);
                const __amdgpu_buffer_rsrc_t rb = make_rsrc(NN ? B0 + (size_t)kt * ldb * 2 : B0 + (size_t)kt * 2);
#pragma unroll
                for (int j = 0; j < G::A_LOADS; j++)
                    rg[S][j] = buffer_load_x4(ra, ld.a_off[j] > lim ? ld.a_off[j] : lim);
#pragma unroll
                for (int j = 0; j < G::B_LOADS; j++)
                    rg[S][G::A_LOADS + j] = buffer_load_x4(rb, ld.b_off[j] > lim ? ld.b_off[j] : lim);
            };
            auto vg_write = [&](auto Sc, uint32_t t) {
                constexpr int S = decltype(Sc)::value;
                LDS_AS uint8_t* st = (LDS_AS uint8_t*)smem + (t & 1) * G::STAGE_BYTES;
#pragma unroll
                for (int j = 0; j < G::A_LOADS; j++)
                    *(LDS_AS u32x4_t*)(st + (wave * G::A_LOADS + j) * 1024 + lane * 16) = rg[S][j];
#pragma unroll
                for (int j = 0; j < G::B_LOADS; j++)
                    *(LDS_AS u32x4_t*)(st + G::A_BYTES + (wave * G::B_LOADS + j) * 1024 + lane * 16) =
                        rg[S][G::A_LOADS + j];
            };
            // LDS writes complete, then every wave at the barrier; loads stay in flight
            auto vg_barrier = [&]() {
                __builtin_amdgcn_sched_barrier(0);
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
            };
            auto buf = [&](uint32_t t) { return (const LDS_AS uint8_t*)smem + (t & 1) * G::STAGE_BYTES; };
            static_for<0, VGD>([&](auto U) { vg_issue(U, decltype(U)::value); });
            y_split_stride = p.y_split_stride;
            asm volatile("" : "+s"(y_split_stride));
            vg_write(Idx<0>{}, 0);
            vg_issue(Idx<0>{}, VGD);
            vg_barrier();
            bf16x8_t af[2][G::FM], bfr[2][G::FN];
            load_frags(buf(0), 0, af[0], bfr[0]);
            // step t; NS = the register set of stage t + 1; MORE = t + 1 < nk
            auto vg_step = [&](uint32_t t, auto NSc, auto MOREc) {
                constexpr bool MORE = decltype(MOREc)::value != 0;
                const LDS_AS uint8_t* sa = buf(t);
#pragma unroll
                for (int kk = 0; kk < KK; kk++) {
                    const int cur = kk & 1;
                    if (kk + 1 < KK) {
                        load_frags(sa, kk + 1, af[cur ^ 1], bfr[cur ^ 1]);
                    } else if constexpr (MORE) {
                        vg_barrier();
                        load_frags(buf(t + 1), 0, af[cur ^ 1], bfr[cur ^ 1]);
                    }
                    mfmas(af[cur], bfr[cur]);
                    if constexpr (MORE) {
                        if (kk == 0) {
                            vg_write(NSc, t + 1);
                            vg_issue(NSc, t + 1 + VGD);
                        }
                    }
                    order_substep();
                }
            };
            // whole groups of VGD steps (nk % VGD == 0), the last one peeled
            uint32_t t0 = 0;
            for (; t0 + VGD < nk; t0 += VGD)
                static_for<0, VGD>([&](auto U) {
                    constexpr int u = decltype(U)::value;
                    vg_step(t0 + u, Idx<(u + 1) % VGD>{}, Idx<1>{});
                });
            static_for<0, VGD>([&](auto U) {
                constexpr int u = decltype(U)::value;
                vg_step(t0 + u, Idx<(u + 1) % VGD>{}, Idx<(u + 1 < VGD ? 1 : 0)>{});
            });
        }
    }

    if constexpr (!PP) { if (!lean && !vg) {
    // prologue: every buffer, then stage 0 visible and its first fragments
#pragma unroll
    for (int s = 0; s < STAGES; s++)
        if ((uint32_t)s < nk) issue_stage(s, 0, 1);
    if (nk >= STAGES) wait_vmcnt<G::LOADS * (STAGES - 1)>();
    else wait_vmcnt<0>();
    // The epilogue's plane stride is loaded here, under the prologue
    // barrier's wait: a scalar load still in flight at the K loop's entry
    // (the compiler hoists it there) turns the first LDS wait of every step
    // into a full one, since scalar loads complete out of order.
    y_split_stride = p.y_split_stride;
    asm volatile("" : "+s"(y_split_stride));
    __syncthreads();
    bf16x8_t af[2][G::FM], bfr[2][G::FN];
    if (nk) load_frags(stage_ptr(0), 0, af[0], bfr[0]);

    if constexpr (KK % 2 == 0) {
        // Steps with a successor take the barrier path unconditionally and
        // the last step is peeled: with both paths in one loop body, the
        // compiler's LDS wait at their join made every step's last MFMAs
        // wait for the next step's fragment reads.
        for (uint32_t t = 0; t + 1 < nk; t++) {
            const LDS_AS uint8_t* sa = stage_ptr(t);
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                const int cur = kk & 1;
                if (kk + 1 < KK) {
                    load_frags(sa, kk + 1, af[cur ^ 1], bfr[cur ^ 1]);
                } else {
                    // stage t+1 has landed once only the stages issued after
                    // it (t+2 .. t+STAGES-1) may still be in flight
                    if (t + STAGES - 1 < nk) wait_vmcnt<G::LOADS * (STAGES - 2)>();
                    else wait_vmcnt<0>();
                    __syncthreads();   // all waves are done reading buffer t % STAGES
                    if (t + STAGES < nk) issue_stage(t + STAGES, 0, 1);
                    load_frags(stage_ptr(t + 1), 0, af[cur ^ 1], bfr[cur ^ 1]);
                }
                mfmas(af[cur], bfr[cur]);
                order_substep();
            }
        }
        if (nk) {
            const LDS_AS uint8_t* sa = stage_ptr(nk - 1);
#pragma unroll
            for (int kk = 0; kk < KK; kk++) {
                const int cur = kk & 1;
                if (kk + 1 < KK) load_frags(sa, kk + 1, af[cur ^ 1], bfr[cur ^ 1]);
                mfmas(af[cur], bfr[cur]);
                order_substep();
            }
        }
    } else {
        // one sub-step per stage (BK == 16): the fragment buffer parity
        // alternates with the step, so steps go in pairs
        for (uint32_t t = 0; t < nk; t += 2) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t tt = t + h;
                if (tt >= nk) break;
                if (tt + 1 < nk) {
                    if (tt + STAGES - 1 < nk) wait_vmcnt<G::LOADS * (STAGES - 2)>();
                    else wait_vmcnt<0>();
                    __syncthreads();
                    if (tt + STAGES < nk) issue_stage(tt + STAGES, 0, 1);
                    load_frags(stage_ptr(tt + 1), 0, af[h ^ 1], bfr[h ^ 1]);
                }
                mfmas(af[h], bfr[h]);
                order_substep();
            }
        }
    }
    } }   // !PP, !lean, !vg

    // ---- epilogue -----------------------------------------------------------
    // acc[i][j][r] holds C[m0 + wm*TM + i*32 + lane%32][n0 + wn*TN + j*32 + 8*(r/4) + 4*(lane/32) + r%4].
    // Each 32-row block of the wave's sub-tile is staged through a
    // wave-private LDS region [32][TN + 4] f32 and written back row-major, so
    // global stores are full contiguous rows and the epilogue chain runs from
    // a compact loop.
    // all waves are done reading the stage buffers (the ping-pong loop's
    // last barrier already ensures it: waves 0-3 stage their results while
    // waves 4-7 issue their last MFMAs from registers)
    if constexpr (!PP) __syncthreads();
    float* wreg = (float*)(smem) + wave * G::EPI_WAVE_FLOATS;
    uint8_t* Cb = (uint8_t*)p.C;
    const bool fixup = (p.flags & T0_GEMM_FIXUP) && sk > 1;
    const uint32_t row_base = m0 + wm * G::TM, col_base = n0 + wn * G::TN;

    if (!fixup) {
        Cb += (size_t)part * y_split_stride;
#pragma unroll
        for (int i = 0; i < G::FM; i++) {
#pragma unroll
            for (int j = 0; j < G::FN; j++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    f32x4_t v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                    *(LDS_AS f32x4_t*)(wreg + l32 * G::EPI_LD + j * 32 + 8 * g + 4 * hi) = v;
                }
            emit_rowblock<G>(p, Cb, wreg, row_base + i * 32, col_base, lane);
        }
        if (probe && tid == 0) {
            probe[4 * bid + 1] = __builtin_amdgcn_s_memrealtime();
            probe[4 * bid + 3] = __builtin_amdgcn_s_memtime();
        }
        return;
    }

    // Split-K fixup: every partition parks its partial tile in the workspace
    // (register order, coalesced); the last partition to arrive sums the
    // planes in plane order and runs the epilogue once.
    // Workspace layout [tile][split][BM*BN f32], register order within a tile.
    constexpr uint32_t TILE_BYTES = BM * BN * 4;
    __amdgpu_buffer_rsrc_t rws = make_rsrc((const uint8_t*)p.workspace + (size_t)tile_id * sk * TILE_BYTES);
#pragma unroll
    for (int i = 0; i < G::FM; i++)
#pragma unroll
        for (int j = 0; j < G::FN; j++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint32_t idx = ((i * G::FN + j) * 4 + g) * G::NT + tid;
                st_agent_x4(rws, part * TILE_BYTES + idx * 16,
                            f32x4_t{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]});
            }
    __shared__ uint32_t s_last;
    if (!publish_and_count(&p.semaphores[tile_id], sk, &s_last)) return;
    // The lane's NOUT 16-byte outputs are summed over the planes in plane
    // order; the loads of up to 32 (output, plane) pairs go out before any is
    // consumed (planes past split_k are not loaded).  With few outputs per
    // lane (registers to spare) this partition's own plane comes from its
    // registers, the values it stored, instead of being reloaded.
    constexpr int NJ = G::FN * 4, NOUT = G::FM * NJ;
    constexpr int QB = NOUT >= 32 ? 1 : 32 / NOUT;   // planes per batch
    f32x4_t v[NOUT];
#pragma unroll
    for (int o = 0; o < NOUT; o++) v[o] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (uint32_t q0 = 0; q0 < sk; q0 += QB) {
        f32x4_t t[NOUT][QB];
#pragma unroll
        for (int qq = 0; qq < QB; qq++) {
            if (q0 + qq >= sk) break;                    // uniform
            if (NOUT <= 8 && q0 + qq == part) {          // uniform
#pragma unroll
                for (int o = 0; o < NOUT; o++) {
                    const int i = o / NJ, j = (o % NJ) / 4, g = o % 4;
                    t[o][qq] = f32x4_t{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                }
                continue;
            }
#pragma unroll
            for (int o = 0; o < NOUT; o++)
                t[o][qq] = ld_agent_x4(rws, ((uint32_t)o * G::NT + tid) * 16 + (q0 + qq) * TILE_BYTES);
        }
#pragma unroll
        for (int qq = 0; qq < QB; qq++) {
            if (q0 + qq >= sk) break;
#pragma unroll
            for (int o = 0; o < NOUT; o++) v[o] += t[o][qq];
        }
    }
#pragma unroll
    for (int i = 0; i < G::FM; i++) {
#pragma unroll
        for (int jg = 0; jg < NJ; jg++)
            *(LDS_AS f32x4_t*)(wreg + l32 * G::EPI_LD + (jg / 4) * 32 + 8 * (jg % 4) + 4 * hi) = v[i * NJ + jg];
        emit_rowblock<G>(p, Cb, wreg, row_base + i * 32, col_base, lane);
    }
    reset_counter(&p.semaphores[tile_id]);
}

}  // namespace t0

// ---------------------------------------------------------------------------
// Instances.  Symbol: t0k_gemm_<BM>x<BN>x<BK>_w<WM>x<WN>_s<STAGES>_<nt|nn>
// ---------------------------------------------------------------------------
#define T0_GEMM_INSTANCE(BM, BN, BK, WM, WN, ST, NNF, TAG)                                          \
    extern "C" __global__ void __launch_bounds__(WM * WN * 64)                                      \
        t0k_gemm_##BM##x##BN##x##BK##_w##WM##x##WN##_s##ST##_##TAG(const t0_gemm_params p) {        \
        t0::gemm_tile_kernel<BM, BN, BK, WM, WN, NNF, ST>(p);                                       \
    }

#define T0_GEMM_BOTH(BM, BN, BK, WM, WN, ST)          \
    T0_GEMM_INSTANCE(BM, BN, BK, WM, WN, ST, false, nt) \
    T0_GEMM_INSTANCE(BM, BN, BK, WM, WN, ST, true, nn)

// Register-staged variants (suffix _vg<D>): the same tile with the K loop
// staged through registers D stages ahead; the host takes them when every
// split-K partition is a whole number of D 64-k steps.
#define T0_GEMM_VG_INSTANCE(BM, BN, BK, WM, WN, ST, D, NNF, TAG)                                    \
    extern "C" __global__ void __launch_bounds__(WM * WN * 64)                                      \
        t0k_gemm_##BM##x##BN##x##BK##_w##WM##x##WN##_s##ST##_vg##D##_##TAG(const t0_gemm_params p) { \
        t0::gemm_tile_kernel<BM, BN, BK, WM, WN, NNF, ST, D>(p);                                    \
    }
#define T0_GEMM_VG_BOTH(BM, BN, BK, WM, WN, ST, D)             \
    T0_GEMM_VG_INSTANCE(BM, BN, BK, WM, WN, ST, D, false, nt) \
    T0_GEMM_VG_INSTANCE(BM, BN, BK, WM, WN, ST, D, true, nn)

// gfx950-native tiles (auto-selection targets); stages = LDS buffers in flight
T0_GEMM_BOTH(256, 256, 64, 2, 2, 2)
T0_GEMM_BOTH(256, 256, 64, 2, 4, 2)
T0_GEMM_BOTH(256, 256, 64, 4, 2, 2)
T0_GEMM_BOTH(256, 256, 32, 2, 2, 4)
T0_GEMM_BOTH(256, 256, 32, 2, 4, 4)
T0_GEMM_BOTH(256, 128, 64, 2, 2, 3)
T0_GEMM_BOTH(128, 256, 64, 2, 2, 3)
T0_GEMM_BOTH(128, 128, 64, 2, 2, 4)
T0_GEMM_BOTH(128, 128, 32, 2, 2, 4)
T0_GEMM_BOTH(128, 64, 64, 2, 2, 4)
T0_GEMM_BOTH(64, 128, 64, 2, 2, 4)
T0_GEMM_VG_BOTH(64, 128, 64, 2, 2, 4, 2)
T0_GEMM_VG_BOTH(128, 64, 64, 2, 2, 4, 2)
T0_GEMM_BOTH(64, 64, 64, 2, 2, 4)
T0_GEMM_BOTH(64, 64, 64, 1, 1, 4)
T0_GEMM_BOTH(32, 64, 64, 1, 1, 6)
T0_GEMM_BOTH(32, 128, 64, 1, 2, 4)
// the reference's preset geometries (src/t0/gemm_gen.rs:86-145), wave64
T0_GEMM_BOTH(32, 64, 16, 1, 1, 4)
T0_GEMM_BOTH(32, 64, 32, 1, 1, 4)
T0_GEMM_BOTH(32, 128, 16, 1, 1, 4)
T0_GEMM_BOTH(64, 64, 16, 1, 1, 4)
T0_GEMM_BOTH(64, 64, 32, 1, 1, 4)
T0_GEMM_BOTH(128, 64, 16, 2, 1, 4)
T0_GEMM_BOTH(128, 64, 32, 2, 1, 4)
T0_GEMM_BOTH(64, 128, 16, 1, 1, 4)
T0_GEMM_BOTH(128, 128, 16, 2, 1, 4)

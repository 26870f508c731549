// kernel_params.h -- argument blocks shared by the host runtime and the gfx950
// kernels.  Every kernel in the code object takes exactly one of these structs
// by value; the host runtime decodes the reference's kernarg byte layouts
// (40/44/48-byte GEMM layouts, 40-byte dequant layout) into them.
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// Epilogue chain opcodes (one 4-bit slot each, applied low slot first).
// Semantics follow src/t0/tile_ir.rs:41-62 / :3406-3540 of the reference.
enum t0_epi_op {
    T0_EPI_NONE = 0,
    T0_EPI_BIAS = 1,   // y += bias[col]           (f32 bias vector [N])
    T0_EPI_SCALE = 2,  // y *= scale
    T0_EPI_RELU = 3,   // y = max(y, 0)
    T0_EPI_SILU = 4,   // y = y * sigmoid(y)
    T0_EPI_GELU = 5,   // y = y * sigmoid(1.702 y)  (the reference's GELU form)
    T0_EPI_ABS = 6,    // y = |y|
    T0_EPI_NEG = 7,    // y = -y
    T0_EPI_CLAMP = 8,  // y = min(max(y, lo), hi)
};

#define T0_MAX_EPI_OPS 8

// flags
#define T0_GEMM_OUT_BF16 0x1u   // store bf16 (RNE) instead of f32
#define T0_GEMM_FIXUP 0x2u      // split-K reduced in-kernel into C (workspace + semaphores)

typedef struct t0_gemm_params {
    const void* A;        // bf16 [M, lda]  row-major, k contiguous
    const void* B;        // NT: bf16 [N, ldb] (k contiguous); NN: bf16 [K, ldb] (n contiguous)
    void* C;              // f32 or bf16 [M, ldc] (split-K planes at C + p*y_split_stride)
    const float* bias;    // [N] f32 (T0_EPI_BIAS)
    float* workspace;     // fixup planes [split_k][tiles][BM*BN] f32
    uint32_t* semaphores; // fixup counters [tiles]
    uint64_t* clock_probe;    // NULL, or [workgroups][4]: 100 MHz clock at start / end,
                              // shader clock at start / end (workgroup's thread 0)
    uint32_t M, N, K;
    uint32_t lda, ldb, ldc;
    uint32_t split_k;          // >= 1
    uint32_t flags;
    uint64_t y_split_stride;   // bytes between split-K output planes
    uint32_t epi_ops;          // packed 4-bit opcodes, 0 terminates
    float epi_scale, clamp_lo, clamp_hi;
} t0_gemm_params;

// W4A16: C[M,N] = A[M,K] (bf16) . W^T, W given as GPTQ-packed int4
// [N][K/8] u32 words (k at bits 4*(k%8)), scales [G][N] (bf16 or f32,
// G = K/group_size), zero points either the constant zero_const
// (zeros == NULL) or packed 4-bit [G][N/8] u32 words (column n at bits
// 4*(n%8)).
#define T0_W4_SCALE_F32 0x1u   // scales are f32 (else bf16)
#define T0_W4_OUT_F32 0x2u     // store f32 (else bf16 RNE)

typedef struct t0_w4a16_params {
    const void* A;            // bf16 [M, lda]
    const uint32_t* qweight;  // [N][K/8]
    const void* scales;       // [G][N]
    const uint32_t* zeros;    // [G][N/8] or NULL
    void* C;                  // [M, ldc]
    float* workspace;         // decode split-K partial tiles; prefill group sums
    uint32_t* semaphores;     // decode split-K counters
    uint32_t M, N, K;
    uint32_t lda, ldc;
    uint32_t group_size;      // multiple of 32 (fast kernels: 128)
    uint32_t zero_const;
    uint32_t flags;
    uint32_t split_k;         // decode: K partitions (>= 1)
    uint32_t round_wgs;       // prefill: workgroups per dispatch round (the CU count)
    // fused residual add + RMSNorm in front of the decode (t0k_w4a16_decode_norm_*,
    // M == 1): the activations are x2 * inv_rms * gamma with x2 = res (+ hid)
    const float* norm_res;    // [K]
    const float* norm_hid;    // [K] or NULL
    const float* norm_gamma;  // [K]
    float* norm_x2;           // [K] or NULL: x2, written by workgroup 0
    float norm_eps;
    uint32_t pad2_;
    float* scales_f32;        // prefill pre-pass: bf16 scales widened to f32 [G][N]
} t0_w4a16_params;

// The reference's fused residual add + RMSNorm + row projection kernel,
// byte for byte its kernarg layout (src/t0/ffn_fused_kernels.rs:47-49):
// [residual, hidden, gamma, weight, output: u64; D: u32; eps: f32].
typedef struct t0_ffn_params {
    const float* residual;
    const float* hidden;
    const float* gamma;
    const float* weight;
    float* output;
    uint32_t D;
    float eps;
} t0_ffn_params;

// Residual add + RMSNorm over rows: out = x2 * inv_rms * gamma (bf16 RNE or
// f32), x2 = res (+ hid), optionally written back.
typedef struct t0_rmsnorm_params {
    const float* res;
    const float* hid;         // or NULL
    const float* gamma;
    void* out;
    float* x2_out;            // or NULL
    uint32_t rows, d;
    uint32_t ld_out;          // elements
    uint32_t out_bf16;
    float eps;
    uint32_t flags;           // T0_RMSNORM_VEC4: 16-byte rows and pointers
} t0_rmsnorm_params;
#define T0_RMSNORM_VEC4 0x1u

// Reference dequant kernel arguments (src/t0/quant_kernels.rs:45-47):
// [packed_weights, scales(f32), zero_points(i32), output; rows, cols]
typedef struct t0_dequant_params {
    const uint8_t* packed;
    const float* scales;
    const int32_t* zero_points;
    void* output;
    uint32_t rows, cols;
    uint32_t group_size_log2;
    uint32_t pad_;
} t0_dequant_params;

typedef struct t0_aux_params {
    const void* src;
    void* dst;
    uint32_t m, n;        // logical rows / cols
    uint32_t ld_src, ld_dst;
    uint32_t planes;      // split-K plane count (reduce)
    uint32_t flags;       // T0_GEMM_OUT_BF16 for reduce output
    uint64_t plane_stride;  // bytes
    uint32_t rows_pad;    // conversion: rows of dst written (zero past m / n)
    uint32_t aux_pad_;
} t0_aux_params;

// t0k_tile_read: the operand traffic of one GEMM tiling on its own (measurement aid).
typedef struct t0_tile_read_params {
    const void* A;        // bf16 [M, lda]
    const void* B;        // bf16 [N, ldb] (b_nt) or [K, ldb]
    uint32_t M, N, K;
    uint32_t lda, ldb;
    uint32_t tile_m, tile_n, split_k;
    uint32_t b_nt;
    uint32_t mode;        // bit 0: the A slices, bit 1: the B slices
} t0_tile_read_params;

// t0_aux_params.flags bit for the conversions: src 16-byte aligned, ld_src % 4 == 0.
#define T0_AUX_SRC_VEC4 0x100u

#ifdef __cplusplus
}

// Waves per workgroup of t0k_w4a16_decode_t<tiles>_mb<mb>: 16 (4 per SIMD,
// <= 128 VGPRs each) when a wave's per-group registers allow, else 8 or 4.
constexpr int t0_w4_decode_waves(int tiles, int mb) {
    return (tiles * mb <= 3 && 32 / mb >= 16) ? 16 : (tiles * mb <= 8 ? 8 : 4);
}
// The same for t0k_w4a16_decode_norm_t<tiles> (M == 1 with the fused RMSNorm,
// whose residual / hidden / gamma registers leave 16 waves room for 2 tiles).
constexpr int t0_w4_decode_norm_waves(int tiles) { return tiles <= 2 ? 16 : 8; }
#endif

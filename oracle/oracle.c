/*
 * oracle.c -- CPU restatement of the reference's GEMM-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the gfx950
 * kernels in rust-gpu_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never links,
 * loads or calls it.
 *
 * Build with -O2 -ffp-contract=off and WITHOUT -ffast-math: the reference is
 * Rust, which never contracts `acc + a*b` into an FMA, so a bit-faithful
 * restatement must not either (oracle/Makefile sets the flags).
 *
 * Every function cites the reference file:line it restates.  Pinning of each
 * function (golden vectors, known answers, closed forms) lives in
 * tests/test_oracle.py.
 */
#include <stdint.h>
#include <stddef.h>
#include <string.h>
#include <math.h>

#if defined(__FP_FAST_FMAF) && !defined(ORACLE_ALLOW_FMA)
/* -ffp-contract=off is what matters; this only documents intent. */
#endif

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* bf16 helpers                                                              */
/* ------------------------------------------------------------------------ */

/* bf16 -> f32: place the 16 bits in the high half.
 * Ref: examples/test_gemm_correctness.rs:22-24, src/t0/tile_ir.rs:4681-4683 */
float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* f32 -> bf16, round to nearest even.
 * Ref: examples/test_gemm_correctness.rs:15-20 (bits + 0x7FFF + lsb) >> 16,
 *      src/ignis/ops/bf16_matmul.rs:371-372.
 * The reference formula is applied verbatim to every non-NaN input (it rounds
 * overflow to +-inf as IEEE RNE does).  For NaN the reference formula can
 * carry into the exponent and return an infinity; the restatement returns the
 * quiet NaN with the same sign instead, which is what gfx950's
 * v_cvt_pk_bf16_f32 produces. */
uint16_t orc_bf16_rne(float x)
{
    uint32_t b = f2u(x);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u)
        return (uint16_t)((b >> 16) | 0x0040u);
    uint32_t round = ((b >> 16) & 1u) + 0x7FFFu;
    return (uint16_t)((b + round) >> 16);
}

/* f32 -> bf16 by truncation (drop the low 16 bits).
 * Ref: src/t0/tile_ir.rs:4677-4678, src/t0/block_dsl.rs:855-866 (store_bf16). */
uint16_t orc_bf16_trunc(float x) { return (uint16_t)(f2u(x) >> 16); }

void orc_bf16_rne_array(const float* x, uint16_t* out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = orc_bf16_rne(x[i]);
}

void orc_bf16_trunc_array(const float* x, uint16_t* out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = orc_bf16_trunc(x[i]);
}

/* ------------------------------------------------------------------------ */
/* Seeded data: the reference's xorshift64 bf16 generator                    */
/* ------------------------------------------------------------------------ */

/* Ref: examples/test_gemm_correctness.rs:45-58.  state = seed ^ 0xDEADBEEFCAFEBABE;
 * per element: xorshift64 (13, 7, 17), f = (hi32 as f32 / u32::MAX as f32)*2 - 1,
 * then RNE to bf16.  `u32::MAX as f32` rounds to 2^32 in Rust. */
void orc_xorshift_bf16(uint16_t* out, size_t n, uint64_t seed)
{
    uint64_t state = seed ^ 0xDEADBEEFCAFEBABEull;
    const float denom = (float)4294967295u; /* == 4294967296.0f after rounding */
    for (size_t i = 0; i < n; i++) {
        state ^= state << 13;
        state ^= state >> 7;
        state ^= state << 17;
        float q = (float)(uint32_t)(state >> 32) / denom;
        float f = q * 2.0f - 1.0f;
        out[i] = orc_bf16_rne(f);
    }
}

/* ------------------------------------------------------------------------ */
/* CPU reference GEMM                                                        */
/* ------------------------------------------------------------------------ */

/* General strided form of the reference CPU matmul:
 *   y[i*ldy + j] = sum_{kk=0..K-1} bf16(a[i*lda + kk]) * bf16(b[kk*sbk + j*sbn])
 * with a single f32 accumulator updated `acc += a*b` in increasing kk order,
 * no FMA.  Rows [row0, row1) only (the CPU baseline times a row slice).
 * Ref: examples/test_gemm_correctness.rs:28-42 (NT: sbk=1, sbn=K);
 *      identical loops at src/t0/tile_ir.rs:5021-5040,
 *      src/t0/tile_boundary_tests.rs:27-38, src/t0/test_tile_gemm_suite.rs:26-35.
 * NN (B[K,N] row-major: sbk=N, sbn=1) keeps the same kk order, so it equals
 * the NT loop on B^T bit for bit. */
void orc_gemm_bf16_rows(const uint16_t* a, size_t lda,
                        const uint16_t* b, size_t sbk, size_t sbn,
                        float* y, size_t ldy,
                        size_t row0, size_t row1, size_t n, size_t k)
{
    for (size_t i = row0; i < row1; i++) {
        const uint16_t* ar = a + i * lda;
        for (size_t j = 0; j < n; j++) {
            const uint16_t* bc = b + j * sbn;
            float acc = 0.0f;
            for (size_t kk = 0; kk < k; kk++) {
                float av = orc_bf16_to_f32(ar[kk]);
                float bv = orc_bf16_to_f32(bc[kk * sbk]);
                float p = av * bv;
                acc = acc + p;
            }
            y[i * ldy + j] = acc;
        }
    }
}

/* Y[M,N] = X[M,K] . WT[N,K]^T  (reference cpu_gemm_bf16, NT). */
void orc_gemm_nt(const uint16_t* x, const uint16_t* wt, float* y,
                 size_t m, size_t k, size_t n)
{
    orc_gemm_bf16_rows(x, k, wt, 1, k, y, n, 0, m, n, k);
}

/* Y[M,N] = A[M,K] . B[K,N]  (NN; same k order as NT). */
void orc_gemm_nn(const uint16_t* a, const uint16_t* b, float* y,
                 size_t m, size_t k, size_t n)
{
    orc_gemm_bf16_rows(a, k, b, n, 1, y, n, 0, m, n, k);
}

/* Same products accumulated in double: not the reference order; used only to
 * report how far the f32 results (CPU and GPU) sit from the exact sum. */
void orc_gemm_f64(const uint16_t* a, size_t lda, const uint16_t* b,
                  size_t sbk, size_t sbn, double* y, size_t m, size_t n, size_t k)
{
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            double acc = 0.0;
            for (size_t kk = 0; kk < k; kk++)
                acc += (double)orc_bf16_to_f32(a[i * lda + kk]) *
                       (double)orc_bf16_to_f32(b[kk * sbk + j * sbn]);
            y[i * n + j] = acc;
        }
}

/* Split-K plane reduction as the host does it: planes summed in plane order
 * into a zero-initialised f32 output.
 * Ref: examples/hello_gemm_gen.rs:125-136, examples/test_gemm_correctness.rs:188-199. */
void orc_splitk_sum(const float* planes, float* y, size_t mn, size_t sk)
{
    for (size_t i = 0; i < mn; i++) y[i] = 0.0f;
    for (size_t s = 0; s < sk; s++)
        for (size_t i = 0; i < mn; i++) y[i] = y[i] + planes[s * mn + i];
}

/* ------------------------------------------------------------------------ */
/* INT4 (GPTQ-style) format and dequant                                      */
/* ------------------------------------------------------------------------ */

/* Element e of a packed INT4 array: byte e/2, low nibble for even e, high
 * nibble for odd e.  Ref: src/t0/quant_kernels.rs:3-10, :191-199, tests
 * :350-357 (0xAB -> lo 11, hi 10), :457-466 (0xD7 -> lo 7, hi 13). */
uint32_t orc_int4_get(const uint8_t* packed, size_t e)
{
    uint8_t byte = packed[e >> 1];
    return (e & 1) ? (uint32_t)(byte >> 4) : (uint32_t)(byte & 0x0F);
}

/* Pack 4-bit values (0..15) two per byte, low nibble = even element.
 * Viewed as little-endian u32 this is 8 nibbles per word, nibble i at bits
 * 4i.  Ref: src/t0/quant_kernels.rs:381-389 (packing round trip). */
void orc_int4_pack(const uint8_t* q, uint8_t* packed, size_t n)
{
    for (size_t i = 0; i < n / 2; i++)
        packed[i] = (uint8_t)((q[2 * i] & 0x0F) | ((q[2 * i + 1] & 0x0F) << 4));
}

void orc_int4_unpack(const uint8_t* packed, uint8_t* q, size_t n)
{
    for (size_t e = 0; e < n; e++) q[e] = (uint8_t)orc_int4_get(packed, e);
}

/* GPTQ dequant to f32:
 *   out[r*cols + c] = (float)(q(r,c) - zp[r*n_groups + g]) * scale[r*n_groups + g],
 *   g = c / group_size.
 * Ref: formula src/t0/quant_kernels.rs:37-40, :365-372 (test_dequant_formula),
 *      format :188-206 (scale/zero_point laid out [row][group]),
 *      group index :469-479.  The subtraction is signed (:441-455), which the
 *      reference GPU kernel gets wrong; this restates the documented format. */
void orc_dequant_int4_f32(const uint8_t* packed, const float* scales,
                          const int32_t* zp, float* out,
                          size_t rows, size_t cols, size_t group_size)
{
    size_t n_groups = cols / group_size;
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) {
            size_t e = r * cols + c;
            size_t g = c / group_size;
            int32_t q = (int32_t)orc_int4_get(packed, e);
            float d = (float)(q - zp[r * n_groups + g]);
            out[e] = d * scales[r * n_groups + g];
        }
}

/* bf16 variant: the f32 value truncated to bf16 (store_bf16 semantics).
 * Ref: src/t0/quant_kernels.rs:109-127 (dequant_int4_bf16 "via store_bf16"),
 *      src/t0/block_dsl.rs:855-866 (store_bf16 truncates). */
void orc_dequant_int4_bf16(const uint8_t* packed, const float* scales,
                           const int32_t* zp, uint16_t* out,
                           size_t rows, size_t cols, size_t group_size)
{
    size_t n_groups = cols / group_size;
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) {
            size_t e = r * cols + c;
            size_t g = c / group_size;
            int32_t q = (int32_t)orc_int4_get(packed, e);
            float d = (float)(q - zp[r * n_groups + g]);
            out[e] = orc_bf16_trunc(d * scales[r * n_groups + g]);
        }
}

/* ------------------------------------------------------------------------ */
/* W4A16 GEMM reference (dequant, then the reference matmul loop)            */
/* ------------------------------------------------------------------------ */

/* Weight W for output column n is row n of the GPTQ packed matrix
 * [rows=N][cols=K] (quant_kernels.rs:191-199), i.e. qw[n*(K/8) + k/8] as a
 * little-endian u32 holds k at bits 4*(k%8).  Scales are bf16 [G][N]
 * (G = K/gs, n contiguous); zero points are either the constant zc
 * (zeros == NULL) or packed 4-bit [G][N/8] words, column n of group g at bits
 * 4*(n%8) of word g*(N/8) + n/8 (the GPTQ qzeros packing).
 *
 * y[i,n] = sum_k bf16(a[i,k]) * w(n,k) with w = (q - z) * s in f32 (exact:
 * |q - z| <= 15 and s has 8 significant bits), accumulated in f32 in k order
 * without FMA -- the reference CPU loop (examples/test_gemm_correctness.rs:28-42)
 * applied to the dequantized weights (src/t0/quant_kernels.rs:365-372). */
static inline float w4_weight(const uint32_t* qw, const uint16_t* scales,
                              const uint32_t* zeros, uint32_t zc,
                              size_t j, size_t kk, size_t n, size_t k, size_t gs)
{
    size_t kw = k / 8, nw = n / 8;
    uint32_t q = (qw[j * kw + kk / 8] >> (4 * (kk % 8))) & 0xF;
    size_t g = kk / gs;
    uint32_t z = zeros ? ((zeros[g * nw + j / 8] >> (4 * (j % 8))) & 0xF) : zc;
    float s = orc_bf16_to_f32(scales[g * n + j]);
    return (float)((int32_t)q - (int32_t)z) * s;
}

void orc_w4a16_rows(const uint16_t* a, const uint32_t* qw, const uint16_t* scales,
                    const uint32_t* zeros, uint32_t zc, float* y,
                    size_t row0, size_t row1, size_t n, size_t k, size_t gs)
{
    for (size_t i = row0; i < row1; i++)
        for (size_t j = 0; j < n; j++) {
            float acc = 0.0f;
            for (size_t kk = 0; kk < k; kk++) {
                float w = w4_weight(qw, scales, zeros, zc, j, kk, n, k, gs);
                float p = orc_bf16_to_f32(a[i * k + kk]) * w;
                acc = acc + p;
            }
            y[i * n + j] = acc;
        }
}

void orc_w4a16(const uint16_t* a, const uint32_t* qw, const uint16_t* scales,
               const uint32_t* zeros, uint32_t zc, float* y,
               size_t m, size_t n, size_t k, size_t gs)
{
    orc_w4a16_rows(a, qw, scales, zeros, zc, y, 0, m, n, k, gs);
}

/* The reference CPU loop on bf16 activations and already dequantized f32
 * weights w [N][K]: y[i,j] = sum_k bf16(a[i,k]) * w[j,k], f32 in k order, no
 * FMA.  With w from orc_w4a16_dequant this is "dequant, then the same loop"
 * (src/t0/quant_kernels.rs:365-372 + examples/test_gemm_correctness.rs:28-42)
 * and equals orc_w4a16_rows bit for bit (same products, same order). */
void orc_gemm_bf16_f32w_rows(const uint16_t* a, const float* w, float* y,
                             size_t row0, size_t row1, size_t n, size_t k)
{
    for (size_t i = row0; i < row1; i++)
        for (size_t j = 0; j < n; j++) {
            float acc = 0.0f;
            const float* wr = w + j * k;
            for (size_t kk = 0; kk < k; kk++) {
                float p = orc_bf16_to_f32(a[i * k + kk]) * wr[kk];
                acc = acc + p;
            }
            y[i * n + j] = acc;
        }
}

/* Dequantize the W4A16 operand to an f32 [N][K] matrix (exact). */
void orc_w4a16_dequant(const uint32_t* qw, const uint16_t* scales,
                       const uint32_t* zeros, uint32_t zc, float* w,
                       size_t n, size_t k, size_t gs)
{
    for (size_t j = 0; j < n; j++)
        for (size_t kk = 0; kk < k; kk++)
            w[j * k + kk] = w4_weight(qw, scales, zeros, zc, j, kk, n, k, gs);
}

/* ------------------------------------------------------------------------ */
/* Decode neighbours: residual add + RMSNorm (+ projection)                 */
/* ------------------------------------------------------------------------ */

/* x2 = residual + hidden (hidden may be NULL: x2 = residual);
 * inv_rms = 1 / sqrt(sum(x2^2) / d + eps), the square sum taken in order;
 * normed[i] = x2[i] * inv_rms * gamma[i], multiplied left to right.
 * Ref: src/t0/rmsnorm_kernels.rs:140-153 (cpu_rmsnorm_forward) on the
 *      residual sum of src/t0/ffn_fused_kernels.rs:215-224.
 * x2_out and inv_rms_out may be NULL. */
void orc_rmsnorm_rows(const float* res, const float* hid, const float* gamma,
                      float* normed, float* x2_out, float* inv_rms_out,
                      size_t m, size_t d, float eps)
{
    for (size_t r = 0; r < m; r++) {
        float sum_sq = 0.0f;
        for (size_t i = 0; i < d; i++) {
            float x2 = hid ? res[r * d + i] + hid[r * d + i] : res[r * d + i];
            if (x2_out) x2_out[r * d + i] = x2;
            float sq = x2 * x2;
            sum_sq = sum_sq + sq;
        }
        float mean_sq = sum_sq / (float)d;
        float inv_rms = 1.0f / sqrtf(mean_sq + eps);
        if (inv_rms_out) inv_rms_out[r] = inv_rms;
        for (size_t i = 0; i < d; i++) {
            float x2 = hid ? res[r * d + i] + hid[r * d + i] : res[r * d + i];
            float t = x2 * inv_rms;
            normed[r * d + i] = t * gamma[i];
        }
    }
}

/* The reference's fused residual add + RMSNorm + per-row projection:
 *   out[row] = sum_i (x2[row,i] * inv_rms_row * gamma[i]) * weight[row*d + i]
 * with the products and the running sum in f32, in order, no FMA.
 * Ref: src/t0/ffn_fused_kernels.rs:203-237 (cpu_ffn_fused_rmsnorm_gemm),
 *      the GPU kernel's semantics at :54-189. */
void orc_ffn_fused_rmsnorm_gemm(const float* res, const float* hid, const float* gamma,
                                const float* weight, float* out, size_t m, size_t d, float eps)
{
    for (size_t r = 0; r < m; r++) {
        float sum_sq = 0.0f;
        for (size_t i = 0; i < d; i++) {
            float x2 = res[r * d + i] + hid[r * d + i];
            float sq = x2 * x2;
            sum_sq = sum_sq + sq;
        }
        float mean_sq = sum_sq / (float)d;
        float inv_rms = 1.0f / sqrtf(mean_sq + eps);
        float acc = 0.0f;
        for (size_t i = 0; i < d; i++) {
            float x2 = res[r * d + i] + hid[r * d + i];
            float t = x2 * inv_rms;
            float normed = t * gamma[i];
            float p = normed * weight[r * d + i];
            acc = acc + p;
        }
        out[r] = acc;
    }
}

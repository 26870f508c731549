// common.h -- gfx950 device helpers shared by the GEMM kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../kernel_params.h"
#include "tile_map.h"

#define T0_DEV __device__ __forceinline__
#define LDS_AS __attribute__((address_space(3)))

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

namespace t0 {

// Compile-time loop: f(Idx<B>{}), ..., f(Idx<E-1>{}).  Register arrays
// indexed through it stay in registers (a runtime index, even one an unrolled
// loop makes constant, can leave them in scratch once lambdas are involved).
template <int I> struct Idx { static constexpr int value = I; };
template <int B, int E, class F>
T0_DEV void static_for(F&& f) {
    if constexpr (B < E) {
        f(Idx<B>{});
        static_for<B + 1, E>(f);
    }
}

// ---------------------------------------------------------------- buffers --
// Raw buffer resource (gfx9 word3 = 0x00020000).  Out-of-range offsets
// (>= num_records) read as zero; kernels use OOB_OFFSET to mask lanes.
constexpr uint32_t OOB_OFFSET = 0x7FFFFFF0u;

// A constant in an SGPR (s_mov_b32), opaque to constant folding: expressions
// with it select the VOP3 forms that take one scalar operand and no literal
// (v_and_or_b32 v, v, s, v).  Only the SGPR write is inline asm: the VALU
// instructions reading it are the compiler's own, so it inserts the wait
// states an MFMA needs after them.
T0_DEV uint32_t sgpr_const(uint32_t v) {
    uint32_t r;
    asm("s_mov_b32 %0, %1" : "=s"(r) : "i"(v));
    return r;
}

T0_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                             (int)OOB_OFFSET, 0x00020000);
}

// 16 bytes per lane from global (base + voffset) straight into LDS at
// lds_wave_base + lane*16.  lds_wave_base must be wave-uniform.
T0_DEV void load_lds_x4(__amdgpu_buffer_rsrc_t r, LDS_AS void* lds_wave_base, uint32_t voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_wave_base, 16, voffset, 0, 0, 0);
}

// s_waitcnt vmcnt(N) alone.  gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt_hi[15:14]; the other counters are left at their max.
template <int N>
T0_DEV void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}
// The same wait as a compiler memory barrier: no memory access (LDS reads of
// DMA'd data in particular) moves across it.
template <int N>
T0_DEV void wait_vmcnt_fence() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

// Global (rsrc + voffset) -> LDS (m0 + lane*16, resp. m0 + lane*4) without
// VGPR staging.  Issued as inline asm: the compiler cannot see which LDS
// buffer the DMA targets and would otherwise wait for it (vmcnt(0)) before
// every LDS read; callers track completion with explicit wait_vmcnt.
// lds_addr must be wave-uniform.
T0_DEV void dma_x4(__amdgpu_buffer_rsrc_t r, uint32_t lds_addr, uint32_t voffset) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :: "s"(lds_addr), "v"(voffset), "s"(r) : "memory");
}
T0_DEV void dma_x1(__amdgpu_buffer_rsrc_t r, uint32_t lds_addr, uint32_t voffset) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :: "s"(lds_addr), "v"(voffset), "s"(r) : "memory");
}

T0_DEV u32x4_t buffer_load_x4(__amdgpu_buffer_rsrc_t r, uint32_t voffset) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, 0, 0));
}

T0_DEV u32x2_t buffer_load_x2(__amdgpu_buffer_rsrc_t r, uint32_t voffset) {
    return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, voffset, 0, 0));
}

T0_DEV uint32_t buffer_load_x1(__amdgpu_buffer_rsrc_t r, uint32_t voffset) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voffset, 0, 0);
}

// ------------------------------------------------------------------ bf16 --
T0_DEV float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// f32 -> bf16 round to nearest even (quiet NaN for NaN): v_cvt_pk_bf16_f32.
T0_DEV uint32_t pack2_bf16_rne(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    bf16x2_t v;
    v[0] = (__bf16)lo;
    v[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// --------------------------------------------------------------- epilogue --
T0_DEV float sigmoid_f(float x) { return 1.0f / (1.0f + __expf(-x)); }

T0_DEV float apply_epilogue(float v, uint32_t ops, float bias_v, float scale, float lo, float hi) {
#pragma unroll 1
    for (; ops; ops >>= 4) {
        switch (ops & 0xF) {
        case T0_EPI_BIAS: v = v + bias_v; break;
        case T0_EPI_SCALE: v = v * scale; break;
        case T0_EPI_RELU: v = fmaxf(v, 0.0f); break;
        case T0_EPI_SILU: v = v * sigmoid_f(v); break;
        case T0_EPI_GELU: v = v * sigmoid_f(1.702f * v); break;
        case T0_EPI_ABS: v = fabsf(v); break;
        case T0_EPI_NEG: v = -v; break;
        case T0_EPI_CLAMP: v = fminf(fmaxf(v, lo), hi); break;
        default: break;
        }
    }
    return v;
}

T0_DEV bool epi_has_bias(uint32_t ops) {
    for (; ops; ops >>= 4)
        if ((ops & 0xF) == T0_EPI_BIAS) return true;
    return false;
}

// ------------------------------------------------- cross-workgroup partials --
// Split-K partial sums move between workgroups (possibly on different XCDs,
// each with its own L2) through agent-scope relaxed atomic stores/loads:
// these bypass the non-coherent L2, so no cache-wide writeback/invalidate
// (what a device-scope fence costs) is needed.  Protocol: each workgroup
// stores its partials with st_agent_x4, waits for its stores
// (publish_and_count), then bumps a counter; the workgroup that sees the last
// count reads every partial with ld_agent_x4.
//
// Partials move 16 bytes per lane with the sc1 cache-policy bit (the code
// gfx950 uses for agent-scope relaxed atomics), and a wave covers whole
// 128-byte lines: write-through stores narrower than a line reach HBM as
// masked writes, which the memory controller turns into read-modify-writes
// (a 4-byte-per-lane version of this protocol ran ~20x slower).
constexpr int CPOL_SC1 = 16;   // aux operand of the raw buffer builtins: sc1
T0_DEV void st_agent_x4(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4_t v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, off, 0, CPOL_SC1);
}
T0_DEV f32x4_t ld_agent_x4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CPOL_SC1));
}
// v += sum over q < n of the 16-byte partials at byte offset off + q*stride, in
// q order; loads go out eight at a time before any is consumed.
T0_DEV f32x4_t sum_partials_x4(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t stride, uint32_t n) {
    f32x4_t v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (uint32_t q0 = 0; q0 < n; q0 += 8) {
        f32x4_t t[8];
#pragma unroll
        for (int j = 0; j < 8; j++) t[j] = ld_agent_x4(r, q0 + j < n ? off + (q0 + j) * stride : OOB_OFFSET);
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (q0 + j < n) v += t[j];
    }
    return v;
}
// all of this workgroup's stores are performed, then the counter is bumped by
// one lane; returns true in every thread of the workgroup that arrived last.
T0_DEV bool publish_and_count(uint32_t* counter, uint32_t total, uint32_t* lds_flag) {
    __builtin_amdgcn_s_waitcnt(0);   // vmcnt(0): this thread's stores are done
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *lds_flag = (prev == total - 1) ? 1u : 0u;
    }
    __syncthreads();
    return *lds_flag != 0;
}
T0_DEV void reset_counter(uint32_t* counter) {
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace t0

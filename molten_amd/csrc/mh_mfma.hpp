// mh_mfma.hpp -- building blocks of the matrix-core GEMM kernels on gfx950:
// operand vector types, bf16 packing, explicit vmcnt waits, LDS reads issued
// without a wait, and direct-to-LDS global loads (global_load_lds_dwordx4 /
// _dword), plain and with a scalar base.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mh_device.hpp"

namespace mh {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

typedef __attribute__((address_space(3))) void* lds_ptr;

typedef const __attribute__((address_space(1))) void* glb_ptr;

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// 16-byte LDS read issued without a wait: the caller waits with lds_wait.
// (Written as asm so the compiler does not wait for every outstanding
// direct-to-LDS load before it.)
__device__ __forceinline__ uint4 lds_read16(uint32_t addr) {
    uint4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}

// Direct-to-LDS 16-byte load: lane l's data lands at lds_base + 16 l.
__device__ __forceinline__ void dma16(mh::gbytes src, uint32_t lds_base) {
    __builtin_amdgcn_global_load_lds((glb_ptr)src, (lds_ptr)(uintptr_t)lds_base, 16, 0, 0);
}
// The same 16-byte load in the scalar-base form: base (uniform) + a 32-bit
// per-lane offset, LDS destination lds_base (uniform) + 16 l.  M0 carries
// the LDS address; it is saved and restored around the load, so the
// compiler's own use of M0 is unaffected.  The compiler does not count this
// load for its vmcnt waits (those can then only wait longer, never less);
// the kernel waits for it explicitly.
__device__ __forceinline__ void dma16s(mh::gbytes base, uint32_t voff, uint32_t lds_base) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(base), "s"(lds_base)
        : "memory");
}
// Direct-to-LDS 4-byte load: lane l's dword lands at lds_base + 4 l.
__device__ __forceinline__ void dma4(mh::gbytes src, uint32_t lds_base) {
    __builtin_amdgcn_global_load_lds((glb_ptr)src, (lds_ptr)(uintptr_t)lds_base, 4, 0, 0);
}
__device__ __forceinline__ uint32_t lds_read4(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}
// The same reads with a constant byte offset in the instruction (no address add).
template <int OFF>
__device__ __forceinline__ uint4 lds_read16_at(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
    uint4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
    return v;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_read4_at(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
    return v;
}

// s_waitcnt lgkmcnt(N), tied to the registers it guards so that no use of
// them can be scheduled above it.
template <int N, int M>
__device__ __forceinline__ void lgkm_wait(uint4 (&v)[M]) {
    static_assert(N >= 0 && N <= 15, "lgkmcnt field");
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
#pragma unroll
    for (int i = 0; i < M; ++i) {
        mh::u32x4 t = {v[i].x, v[i].y, v[i].z, v[i].w};
        asm volatile("" : "+v"(t));
        v[i] = make_uint4(t.x, t.y, t.z, t.w);
    }
}
template <int N, int M>
__device__ __forceinline__ void lgkm_wait(uint32_t (&v)[M]) {
    static_assert(N >= 0 && N <= 15, "lgkmcnt field");
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
#pragma unroll
    for (int i = 0; i < M; ++i) {
        auto t = v[i];
        asm volatile("" : "+v"(t));
        v[i] = t;
    }
}

// Ties registers to this point (no use of them is scheduled above it): used
// after an lgkm_wait that already covers the reads that fill them.
template <int M>
__device__ __forceinline__ void tie_regs(uint32_t (&v)[M]) {
#pragma unroll
    for (int i = 0; i < M; ++i) {
        auto t = v[i];
        asm volatile("" : "+v"(t));
        v[i] = t;
    }
}

}  // namespace mh

// ceiling.hip -- measurement kernels that frame the hot path's rooflines on
// this part: what a plain streaming read of HBM reaches, and what the bf16
// matrix cores reach with nothing but independent MFMAs in flight.  They
// have no counterpart in the reference (which publishes its own ceiling as
// a measured streaming read, docs/ARCHITECTURE.md:48); they are not part of
// the operator boundary and live in their own library.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "molten_ceiling.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Streaming read: every thread loads U 16-byte pieces per round (all in
// flight before any is used), rounds stride over the grid.  The xor of the
// data is stored only when it equals a value the data never produces in
// practice, so the loads stay live and almost nothing is written.
template <int U, bool NT>
__global__ __launch_bounds__(256) void k_read(const uint4* __restrict__ p, uint64_t n16, uint32_t* sink) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256u;
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if constexpr (NT) {
                const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p + i + u * stride));
                v[u] = make_uint4(t.x, t.y, t.z, t.w);
            } else {
                v[u] = p[i + u * stride];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) {
        sink[0] = acc;
    }
}

// Copy (read + write of the same byte count), for the counter calibration.
__global__ __launch_bounds__(256) void k_copy(const uint4* __restrict__ src, uint4* __restrict__ dst, uint64_t n16) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * 256u;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x; i < n16; i += stride) {
        dst[i] = src[i];
    }
}

// bf16 matrix-core rate: each wave keeps 8 independent 32x32 accumulators
// and issues v_mfma_f32_32x32x16_bf16 back to back, `iters` rounds of 8.
__global__ __launch_bounds__(256) void k_mfma(float* out, uint32_t iters) {
    const int lane = threadIdx.x & 63;
    bf16x8_t a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = static_cast<__bf16>(0.001f * static_cast<float>(lane + j));
        b[j] = static_cast<__bf16>(0.002f * static_cast<float>(lane - j));
    }
    f32x16_t acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[c][q] = 0.0f;
    for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int q = 0; q < 16; ++q) s += acc[c][q];
    if (s == 1234.5f) {  // keeps the chain live; practically never stored
        out[blockIdx.x * 256 + threadIdx.x] = s;
    }
}

template <int U, bool NT>
void launch_read(const void* p, uint64_t n16, uint32_t grid, uint32_t* sink, hipStream_t s) {
    hipLaunchKernelGGL((k_read<U, NT>), dim3(grid), dim3(256), 0, s, static_cast<const uint4*>(p), n16, sink);
}

int status() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : static_cast<int>(e);
}

// Store-to-visible latency of one 8-byte word between workgroups.
// Workgroups 0..7 (one per XCD under the round-robin dispatch) are
// producers: each waits `delay` ticks of the 100 MHz constant clock after it
// starts, then stores `value` to its own word (a plain store, which stays in
// its XCD's L2, for mode 0; a device-coherent store for mode 1) and records
// the clock.  Every other workgroup polls, with L2-coherent loads, the word
// of producer (its index % 8) -- the same XCD -- and in mode 1 also that of
// producer (its index + 1) % 8 -- another XCD -- until it holds `value`,
// and records the clock when it does (0 if `spins` polls pass first).
// out[4 wg + 0]: the XCD the workgroup ran on; producers: out[4 wg + 3] the
// store's clock; consumers: out[4 wg + 1], out[4 wg + 2] the two times seen.
__device__ __forceinline__ uint64_t clock100() {
    return wall_clock64();
}

__global__ __launch_bounds__(64) void k_exchange(uint64_t* words, uint64_t* out, uint64_t value, int mode,
                                                 uint32_t delay, uint32_t spins) {
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    const uint64_t t0 = clock100();
    const uint32_t b = blockIdx.x;
    const int lane = threadIdx.x;
    if (lane == 0) {
        out[4u * b] = xcc & 0xfu;
    }
    if (b < 8u) {
        while (clock100() < t0 + delay) {
            __builtin_amdgcn_s_sleep(1);
        }
        if (lane == 0) {
            const uint64_t ts = clock100();
            if (mode == 0) {
                __hip_atomic_store(words + 8u * b, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            } else {
                __hip_atomic_store(words + 8u * b, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            out[4u * b + 3u] = ts;
        }
        return;
    }
    // lane 0: this XCD's producer; lane 1 (mode 1): the next XCD's
    if (lane < (mode == 0 ? 1 : 2)) {
        const uint32_t pw = (b + static_cast<uint32_t>(lane)) % 8u;
        uint64_t seen = 0;
        for (uint32_t i = 0; i < spins; ++i) {
            const uint64_t v = __hip_atomic_load(words + 8u * pw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (v == value) {
                seen = clock100();
                break;
            }
        }
        out[4u * b + 1u + static_cast<uint32_t>(lane)] = seen;
    }
}

}  // namespace

// Every word of a workgroup's LDS (the whole 160 KB of a CU: one such
// workgroup fits a CU at a time) set to `pattern`; the stores are volatile,
// so they are not dropped as never read.
constexpr uint32_t kLdsBytes = 160u * 1024u;
__global__ __launch_bounds__(256) void k_lds_fill(uint32_t pattern) {
    extern __shared__ uint32_t lds_words[];
    volatile uint32_t* const w = lds_words;
    for (uint32_t i = threadIdx.x; i < kLdsBytes / 4u; i += blockDim.x) {
        w[i] = pattern;
    }
}

extern "C" {

int mhc_read(const void* src, size_t bytes, uint32_t grid, uint32_t unroll, int nontemporal, uint32_t* sink,
             void* stream) {
    if (src == nullptr || sink == nullptr || bytes % 16 != 0 || grid == 0 ||
        reinterpret_cast<uintptr_t>(src) % 16 != 0) {
        return -1;
    }
    const uint64_t n16 = bytes / 16;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const bool nt = nontemporal != 0;
    switch (unroll) {
        case 1: nt ? launch_read<1, true>(src, n16, grid, sink, s) : launch_read<1, false>(src, n16, grid, sink, s); break;
        case 2: nt ? launch_read<2, true>(src, n16, grid, sink, s) : launch_read<2, false>(src, n16, grid, sink, s); break;
        case 4: nt ? launch_read<4, true>(src, n16, grid, sink, s) : launch_read<4, false>(src, n16, grid, sink, s); break;
        case 8: nt ? launch_read<8, true>(src, n16, grid, sink, s) : launch_read<8, false>(src, n16, grid, sink, s); break;
        default: return -1;
    }
    return status();
}

int mhc_copy(const void* src, void* dst, size_t bytes, uint32_t grid, void* stream) {
    if (src == nullptr || dst == nullptr || bytes % 16 != 0 || grid == 0 ||
        reinterpret_cast<uintptr_t>(src) % 16 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0) {
        return -1;
    }
    hipLaunchKernelGGL(k_copy, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4*>(src), static_cast<uint4*>(dst), static_cast<uint64_t>(bytes / 16));
    return status();
}

int mhc_mfma(float* out, uint32_t workgroups, uint32_t iters, void* stream) {
    if (out == nullptr || workgroups == 0) {
        return -1;
    }
    hipLaunchKernelGGL(k_mfma, dim3(workgroups), dim3(256), 0, static_cast<hipStream_t>(stream), out, iters);
    return status();
}

int mhc_exchange(uint64_t* words, uint64_t* out, uint32_t workgroups, uint64_t value, int mode, uint32_t delay,
                 uint32_t spins, void* stream) {
    if (words == nullptr || out == nullptr || workgroups <= 8u || (mode != 0 && mode != 1) ||
        reinterpret_cast<uintptr_t>(words) % 8 != 0 || spins == 0) {
        return -1;
    }
    hipLaunchKernelGGL(k_exchange, dim3(workgroups), dim3(64), 0, static_cast<hipStream_t>(stream), words, out, value,
                       mode, delay, spins);
    return status();
}

uint64_t mhc_mfma_flops(uint32_t workgroups, uint32_t iters) {
    return static_cast<uint64_t>(workgroups) * 4u * iters * 8u * (32u * 32u * 16u * 2u);
}

int mhc_lds_fill(uint32_t pattern, uint32_t workgroups, void* stream) {
    if (workgroups == 0) {
        return -1;
    }
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_lds_fill),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsBytes));
    if (e != hipSuccess) {
        return static_cast<int>(e);
    }
    hipLaunchKernelGGL(k_lds_fill, dim3(workgroups), dim3(256), kLdsBytes, static_cast<hipStream_t>(stream), pattern);
    return status();
}

}  // extern "C"

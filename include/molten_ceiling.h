/* molten_ceiling.h -- measurement kernels (libmolten_ceiling.so), not part of
 * the operator boundary in molten_hip.h.  They have no counterpart in the
 * reference, whose own ceiling is a measured streaming read
 * (docs/ARCHITECTURE.md:48).  bench.py --ceilings times them to state what
 * HBM streaming and the bf16 matrix cores reach on the part the hot path
 * runs on.  Every function returns 0, -1 for a rejected argument, or a
 * hipError_t (> 0) from the launch. */
#ifndef MOLTEN_CEILING_H
#define MOLTEN_CEILING_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Streaming read of `bytes` (a multiple of 16, 16-byte aligned) with `grid`
 * workgroups of 256 threads, `unroll` (1, 2, 4 or 8) 16-byte loads in flight
 * per thread, non-temporal loads when `nontemporal` != 0.  `sink` is one
 * device word that is written only in the practically impossible case that
 * the data's xor hits a fixed value. */
int mhc_read(const void* src, size_t bytes, uint32_t grid, uint32_t unroll, int nontemporal, uint32_t* sink,
             void* stream);

/* dst = src over `bytes` (a multiple of 16, both 16-byte aligned). */
int mhc_copy(const void* src, void* dst, size_t bytes, uint32_t grid, void* stream);

/* `workgroups` x 4 waves, each issuing iters x 8 independent
 * v_mfma_f32_32x32x16_bf16; `out` is [workgroups x 256] f32, written only
 * in a practically impossible case. */
int mhc_mfma(float* out, uint32_t workgroups, uint32_t iters, void* stream);

/* The bf16 FLOPs of one mhc_mfma launch. */
uint64_t mhc_mfma_flops(uint32_t workgroups, uint32_t iters);

#ifdef __cplusplus
}
#endif

#endif

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

/* Store-to-visible latency between workgroups (the cost of one exchange of
 * the fused decode step's kind): `workgroups` (> 8) workgroups of 64
 * threads; workgroups 0..7 (one per XCD) store `value` into words[8 p]
 * (`words`: 64 u64, 8-byte aligned) `delay` ticks of the 100 MHz clock
 * after they start -- mode 0 with a plain store (it stays in the XCD's L2),
 * mode 1 device-coherent -- and every other workgroup w polls words[8 (w %
 * 8)] (its XCD's producer) and, in mode 1, words[8 ((w + 1) % 8)] (another
 * XCD's) with L2-coherent loads, at most `spins` times each.  out: 4 u64 per
 * workgroup: the XCD it ran on, the clock at which each of the two words
 * was seen (0: not within `spins` polls), and for producers the clock of
 * the store.  Pass a value the words do not hold yet (a launch counter). */
int mhc_exchange(uint64_t* words, uint64_t* out, uint32_t workgroups, uint64_t value, int mode, uint32_t delay,
                 uint32_t spins, void* stream);

/* Every word of the LDS of the CUs `workgroups` workgroups run on set to
 * `pattern` (each workgroup takes a CU's whole 160 KB, so with workgroups
 * >= the CU count every CU's LDS is written): the state a kernel that reads
 * LDS before writing it would see after such a kernel.  A test's
 * precondition, not a measurement. */
int mhc_lds_fill(uint32_t pattern, uint32_t workgroups, void* stream);

/* The bf16 FLOPs of one mhc_mfma launch. */
uint64_t mhc_mfma_flops(uint32_t workgroups, uint32_t iters);

#ifdef __cplusplus
}
#endif

#endif

// mh_host.hpp -- host-side helpers for the extern "C" launchers: the error
// convention, argument validation and device queries.
//
// Error convention (mirrors the reference's `anyhow::ensure!` before any
// dispatch, src/metal.rs:337-353): a launcher validates every argument
// before it touches the HIP runtime.  It returns
//   0                on success,
//   MH_ERR_* (< 0)   when an argument is rejected; nothing was launched and
//                    mh_last_error() holds the message,
//   hipError_t (> 0) when the runtime reports an error at launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "molten_hip.h"

namespace mh {

int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_error(hipError_t e, const char* what);

// Number of compute units of the current device (cached per device).
int cu_count();

// The current device's status word (MH_STATUS_* bits; kernels set bits with
// a device-scope atomic or when a bounded wait expires), or NULL when it
// cannot be resolved.  Cached per device after the first call.
uint32_t* status_word();

inline hipStream_t as_stream(mh_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void* p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

// Shared checks for MLX affine weights (src/kernels/quant.rs:42-66 check_quant):
// bits in {4, 6}; group size a multiple of 32 that divides K (a 32-code chunk
// never crosses a group); codes aligned for the vector loads.
int check_quant(const mh_quant_weights* w, const char* op);
// The same for the dequantizing operators, which also take 8-bit weights
// (src/kernels/quant.rs:42-66 accepts bits 4 and 8; this build adds 6).
int check_quant_dequant(const mh_quant_weights* w, const char* op);

// Launch status after hipLaunchKernelGGL.
// Internal launches of the prefill MoE step (moe_prefill.hip, moe_decode.hip).
// Prefill routing after the router logits: top-k per token with per-block
// expert histograms hb (ceil(m / kPrefillRouteBlock) + 1 rows of e words: the blocks, then
// the totals), their per-expert prefix, then the stable scatter, counts,
// offsets and both block maps (three launches).
constexpr uint32_t kPrefillRouteBlock = 16;  // tokens per routing block (histogram row)
// routed: ids, gw and hb's block rows are already written (route_mma), only
// the prefix and the scatter run.  gu_ord / dn_ord (or null): the two maps
// again in the segment GEMMs' launch order (map_grid entries each; see
// seg_rank_of), for launches that take entry b = workgroup b; the map rows
// (max_gu / (gu_n / gu_bn)) must not exceed kMaxOrderedRows.
int moe_route_sort_maps(const float* logits, const float* bias, int mode, float eps, uint32_t m,
                        uint32_t e, uint32_t topk, uint32_t* ids, uint16_t* gw, uint32_t* hb,
                        uint32_t* counts, uint32_t* offsets, uint32_t* gu_off, uint32_t* dn_off,
                        uint32_t* ids_sorted, uint32_t* slotpos, uint32_t* gu, uint32_t max_gu, uint32_t* dn,
                        uint32_t max_dn, uint32_t bm, uint32_t gu_bn, uint32_t dn_bn, uint32_t gu_n,
                        uint32_t dn_n, mh_stream_t stream, bool routed = false, uint32_t* gu_ord = nullptr,
                        uint32_t* dn_ord = nullptr);

// Launch order of the segment GEMMs (grouped_gemm.hip k_seg) over a block map
// whose rows ("groups": one expert's row segment, nt column-tile entries
// each) are ranked by row count, most first, lower map row first on ties.
// The grid is whole units of 8 x nt workgroups; workgroup b takes rank
// seg_rank_of(b, nt) (units in turn, the 8 XCDs' workgroups b % 8 walking
// the ranks forward on even units and backward on odd ones, so each XCD gets
// a heavy and a light group in turn) and column tile (b / 8) % nt of it.
inline uint32_t map_grid(uint32_t n_blocks, uint32_t nt) {
    const uint32_t unit = 8u * nt;
    return (n_blocks + unit - 1u) / unit * unit;
}
__host__ __device__ inline uint32_t seg_rank_of(uint32_t b, uint32_t nt) {
    const uint32_t x = b % 8u, slot = (b / 8u) / nt;
    return slot * 8u + ((slot & 1u) ? 7u - x : x);
}
// the workgroup that takes column tile t of the group of rank r
__host__ __device__ inline uint32_t seg_workgroup_of(uint32_t r, uint32_t t, uint32_t nt) {
    const uint32_t slot = r / 8u, xr = r % 8u;
    return ((slot * nt + t) * 8u) + ((slot & 1u) ? 7u - xr : xr);
}
constexpr uint32_t kMaxOrderedRows = 1024;  // map rows the scatter ranks in its LDS
// The prefill router and top-k on the matrix cores with exact routing
// (moe_route_mma.hip): logits (chunk-order values for every candidate), ids,
// gw and the routing blocks' expert histograms hb, for a bf16 router.
bool route_mma_fits(const void* w, int w_dtype, const uint16_t* x, uint32_t e, uint32_t k, uint32_t topk);
int route_mma(const uint16_t* x, const uint16_t* w, const float* bias, int mode, float eps, uint32_t m, uint32_t e,
              uint32_t k, uint32_t topk, float* logits, uint32_t* ids, uint16_t* gw, uint32_t* hb,
              hipStream_t stream);
int moe_sort_maps(const uint32_t* ids, uint32_t s, uint32_t e, uint32_t topk, uint32_t* counts,
                  uint32_t* offsets, uint32_t* gu_off, uint32_t* dn_off, uint32_t* ids_sorted,
                  uint32_t* slotpos, uint32_t* gu, uint32_t max_gu, uint32_t* dn, uint32_t max_dn,
                  uint32_t bm, uint32_t gu_bn, uint32_t dn_bn, uint32_t gu_n, uint32_t dn_n,
                  mh_stream_t stream);
int moe_decode_fused(const void* router, int router_dtype, const float* bias, int mode, float eps,
                     const mh_quant_weights* gate, const mh_quant_weights* up,
                     const mh_quant_weights* down, uint32_t n_experts, uint32_t topk,
                     const uint16_t* x, uint16_t* out, float* logits, uint32_t* ids,
                     uint16_t* weights, uint16_t* act, uint32_t* scratch, uint64_t* stamps, hipStream_t stream);
// Workgroups x waves of the fused decode step (the stamp buffer holds
// kGrid * kWaves * MH_MOE_DECODE_STAMPS words).
uint32_t moe_decode_fused_waves();
// The prefill step's grouped GEMMs on the segment kernels (grouped_gemm.hip):
// ordered, the map is in launch order (entry b for workgroup b, map_grid
// entries, from moe_route_sort_maps' gu_ord / dn_ord); stamps (or null), per
// workgroup MH_PREFILL_STAMPS words (measurement).
int gemm_gu_act_seg(const uint16_t* x, const uint32_t* ids_sorted, uint32_t x_rows, const mh_quant_weights* gate,
                    const mh_quant_weights* up, uint16_t* act, const uint32_t* blocks, uint32_t n_blocks,
                    uint32_t s_rows, uint32_t n, uint32_t bm, uint32_t bn, bool ordered, uint64_t* stamps,
                    hipStream_t s);
int gemm_grouped_seg(const uint16_t* a, const mh_quant_weights* w, uint16_t* c, const uint32_t* blocks,
                     uint32_t n_blocks, uint32_t s_rows, uint32_t n, uint32_t bm, uint32_t bn, bool ordered,
                     uint64_t* stamps, hipStream_t s);
// stamps: per-wave phase timestamps (measurement, batch 8 only), or null.
int gemv_mfma(const mh_quant_weights* w, const uint16_t* x, uint16_t* y, uint64_t* slots, uint32_t* ids,
              uint32_t batch, hipStream_t stream, uint64_t* stamps = nullptr);
int router_prefill_logits(const uint16_t* x, const void* w, int w_dtype, float* logits, uint32_t m,
                          uint32_t k, uint32_t e, mh_stream_t stream);

inline int launch_status(const char* what) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? MH_OK : hip_error(e, what);
}

}  // namespace mh

#define MH_ENSURE(cond, code, ...)                      \
    do {                                                \
        if (!(cond)) {                                  \
            return ::mh::set_error((code), __VA_ARGS__); \
        }                                               \
    } while (0)

#define MH_TRY(expr)                 \
    do {                             \
        const int mh_rc_ = (expr);   \
        if (mh_rc_ != MH_OK) {       \
            return mh_rc_;           \
        }                            \
    } while (0)

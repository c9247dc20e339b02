// mh_route.hpp -- top-k expert selection shared by the decode and prefill
// routers (lfm.metal:541-703, :1558-1602).
//
// mode 0 (molten): s = 1/(1+exp(-z)); rank on s + bias; weights
//        bf16(s_r / (eps + s_0 + ... + s_{k-1})).
// mode 1 (softmax): rank on z; weights bf16(e_r / (e_0 + ... + e_{k-1})),
//        e_r = exp(z_r - z_top1) (softmax over all experts restricted to the
//        chosen ones and renormalised).
// Selection is the serial scan of lfm_moe_route_batch: for each slot, the
// greatest unused candidate, an exact tie to the lower expert id, starting
// from (-inf, id 0).  exp is mh::expf_fixed, so CPU and GPU agree bit for bit.
#pragma once

#include "mh_device.hpp"

namespace mh {

constexpr int kMaxExperts = 256;
constexpr int kMaxTopk = 8;

// Per-expert score and candidate (lane-parallel part).
__device__ __forceinline__ void route_score(float z, float bias, int mode, float& s, float& cand) {
    if (mode == 0) {
        s = 1.0f / (1.0f + expf_fixed(-z));
        cand = s + bias;
    } else {
        s = z;
        cand = z;
    }
}

// Serial selection over LDS-resident scores (one thread).  used[] is scratch.
__device__ inline void route_select(const float* s, const float* cand, unsigned char* used,
                                    uint32_t e, uint32_t topk, int mode, float eps,
                                    uint32_t* ids_out, uint16_t* w_out) {
    uint32_t chosen[kMaxTopk];
    for (uint32_t i = 0; i < e; ++i) {
        used[i] = 0;
    }
    for (uint32_t r = 0; r < topk; ++r) {
        float best = -__builtin_inff();
        uint32_t best_e = 0;
        for (uint32_t i = 0; i < e; ++i) {
            if (used[i]) {
                continue;
            }
            const float v = cand[i];
            if (v > best || (v == best && i < best_e)) {
                best = v;
                best_e = i;
            }
        }
        chosen[r] = best_e;
        used[best_e] = 1;
    }
    if (mode == 0) {
        float denom = eps;
        for (uint32_t r = 0; r < topk; ++r) {
            denom = denom + s[chosen[r]];
        }
        for (uint32_t r = 0; r < topk; ++r) {
            ids_out[r] = chosen[r];
            w_out[r] = f32_to_bf16(s[chosen[r]] / denom);
        }
    } else {
        const float top = s[chosen[0]];
        float ev[kMaxTopk];
        float denom = 0.0f;
        for (uint32_t r = 0; r < topk; ++r) {
            ev[r] = expf_fixed(s[chosen[r]] - top);
            denom = denom + ev[r];
        }
        for (uint32_t r = 0; r < topk; ++r) {
            ids_out[r] = chosen[r];
            w_out[r] = f32_to_bf16(ev[r] / denom);
        }
    }
}

}  // namespace mh

// mh_route.hpp -- top-k expert selection shared by the decode and prefill
// routers (lfm.metal:541-703, :1558-1602).
//
// mode 0 (molten): s = 1/(1+exp(-z)); rank on s + bias; weights
//        bf16(s_r / (eps + s_0 + ... + s_{k-1})).
// mode 1 (softmax): rank on z; weights bf16(e_r / (e_0 + ... + e_{k-1})),
//        e_r = exp(z_r - z_top1) (softmax over all experts restricted to the
//        chosen ones and renormalised).
// Selection equals the serial scan of lfm_moe_route_batch: for each slot, the
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

// Selection over LDS-resident scores by one full wave.  For each slot every
// lane takes the best eligible candidate among its experts (lane, lane + 64,
// ...), then the wave reduces with the same rule in two DPP passes: the
// greatest candidate value, then the lowest id among the lanes holding it.
// "value desc, id asc" is a strict total order on eligible candidates (ids
// are distinct), so the winner does not depend on the reduction order and
// equals the serial scan's: that scan starts from (-inf, id 0) and only
// replaces on v > best or (v == best and a lower id), so used experts, NaN
// and -inf never win, and with no eligible candidate it returns expert 0.
// Lane 0 writes ids and weights.
__device__ inline void route_select(const float* s, const float* cand, uint32_t e, uint32_t topk,
                                    int mode, float eps, uint32_t* ids_out, uint16_t* w_out) {
    const uint32_t lane = threadIdx.x & 63u;
    constexpr int kPerLane = kMaxExperts / 64;
    uint32_t used = 0;  // bit j: expert lane + 64 j already chosen
    uint32_t chosen[kMaxTopk];
    for (uint32_t r = 0; r < topk; ++r) {
        float bv = -__builtin_inff();
        uint32_t bi = 0xffffffffu;
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            const uint32_t i = lane + 64u * j;
            if (i < e && !((used >> j) & 1u)) {
                const float v = cand[i];
                if (v > -__builtin_inff() && (v > bv || (v == bv && i < bi))) {
                    bv = v;
                    bi = i;
                }
            }
        }
        // lanes with no eligible candidate hold (-inf, none): they lose to
        // any eligible value and are ignored when the best value is -inf
        const float m = wave_max_f32(bv);
        if (m > -__builtin_inff()) {
            bi = wave_min_u32(bv == m ? bi : 0xffffffffu);
        } else {
            bi = 0xffffffffu;
        }
        const uint32_t pick = bi == 0xffffffffu ? 0u : bi;
        chosen[r] = pick;
        if ((pick & 63u) == lane) {
            used |= 1u << (pick >> 6);
        }
    }
    if (lane != 0) {
        return;
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

// route_select's choice with the scores in registers: lane l holds expert
// l + 64 j in s[j] / cand[j] for j < EB (cand -inf where l + 64 j >= e).
// Same selection rule as route_select; every lane returns the ids and the
// chosen experts' scores sv (wave-uniform), from which route_weights_regs
// computes the weights.  With EB == 1 (e <= 64) a lane holds one candidate
// and the lowest id among the lanes holding the maximum is the lowest set bit
// of a ballot.
template <int TK, int EB>
__device__ inline void route_select_ids(const float (&s)[EB], const float (&cand)[EB], uint32_t (&ids)[TK],
                                        float (&sv)[TK]) {
    static_assert(EB >= 1 && EB <= kMaxExperts / 64, "experts per lane");
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t used = 0;
#pragma unroll
    for (int r = 0; r < TK; ++r) {
        uint32_t pick;
        if (EB == 1) {
            const float v = (used & 1u) ? -__builtin_inff() : cand[0];
            const float m = wave_max_f32(v);
            const unsigned long long hit = __ballot(v == m);
            pick = m > -__builtin_inff() && hit != 0ull ? static_cast<uint32_t>(__builtin_ctzll(hit)) : 0u;
        } else {
            float bv = -__builtin_inff();
            uint32_t bi = 0xffffffffu;
#pragma unroll
            for (int j = 0; j < EB; ++j) {
                // ids rise with j, so a strict > keeps the lowest id on ties;
                // -inf (absent experts) and NaN are never taken
                const float v = cand[j];
                const bool take = !((used >> j) & 1u) && v > bv;
                bv = take ? v : bv;
                bi = take ? lane + 64u * j : bi;
            }
            const float m = wave_max_f32(bv);
            bi = m > -__builtin_inff() ? wave_min_u32(bv == m ? bi : 0xffffffffu) : 0xffffffffu;
            pick = bi == 0xffffffffu ? 0u : bi;
        }
        pick = __builtin_amdgcn_readfirstlane(pick);
        ids[r] = pick;
        // the chosen score: each block's lane value, then a uniform select
        // (the opaque copies keep the compiler from indexing an array in
        // private memory instead)
        float mine = s[0];
#pragma unroll
        for (int j = 1; j < EB; ++j) {
            float sj = s[j];
            asm volatile("" : "+v"(sj));
            mine = (pick >> 6) == static_cast<uint32_t>(j) ? sj : mine;
        }
        sv[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), pick & 63u));
        used |= (pick & 63u) == lane ? 1u << (pick >> 6) : 0u;
    }
}

// route_select's weight arithmetic on the chosen scores sv (wave-uniform):
// one slot per lane, the denominator summed slot by slot in order; returns
// the bf16 weight bits of every slot (wave-uniform).
template <int TK>
__device__ inline void route_weights_regs(const float (&sv)[TK], int mode, float eps, uint32_t (&wbits)[TK]) {
    const uint32_t lane = threadIdx.x & 63u;
    float my = sv[0];
#pragma unroll
    for (int r = 1; r < TK; ++r) {
        my = lane == static_cast<uint32_t>(r) ? sv[r] : my;
    }
    float num, denom;
    if (mode == 0) {
        num = my;
        denom = eps;
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            denom = denom + sv[r];
        }
    } else {
        num = expf_fixed(my - sv[0]);
        denom = 0.0f;
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            denom = denom + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(num), r));
        }
    }
    const int wl = static_cast<int>(f32_to_bf16(num / denom));
#pragma unroll
    for (int r = 0; r < TK; ++r) {
        wbits[r] = static_cast<uint32_t>(__builtin_amdgcn_readlane(wl, r));
    }
}

}  // namespace mh

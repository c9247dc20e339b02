// moe_decode_fused.hip -- the MoE decode step (router -> top-k -> expert
// gate/up + SwiGLU -> down + weighted combine) as one persistent launch.
//
// kGrid workgroups of kWaves waves (one per CU on a 256-CU part, all
// resident at once) run three phases:
//   1. router logits, one row per wave, spread over the workgroups;
//   2. every wave routes the token itself (from the logits, in registers),
//      issues the loads of its down-projection rows, then computes pairs of
//      gate/up rows of the chosen experts and their SwiGLU activations;
//   3. each workgroup stages all activations in LDS and each wave produces
//      one output of the down projection + weighted combine.
// Same arithmetic (chunk order, roundings) as the three-launch path in
// moe_decode.hip, so outputs are bit-identical to it and to the oracle.
//
// Cross-workgroup exchange without grid barriers: a logit, or a pair of
// activations, travels as one 64-bit word {data, epoch} written with a single
// device-coherent store; a consumer polls the words it needs with
// device-coherent loads until each carries the current launch's epoch.  Data
// and tag arrive together, so there is no store-acknowledge wait and no
// arrival counter on the critical path.  Only wave 0 of a workgroup polls
// (with a pause between rounds), so the polls do not crowd out the stores
// they wait for.  The epoch: workgroup b keeps a launch count in scratch
// word b, reads it at its start and writes it back plus one; every launch
// runs all kGrid workgroups once, so the counts advance in lockstep and all
// workgroups of a launch see the same value.  epoch = count + 1 (32-bit,
// never 0, so zeroed words never match, and consecutive launches differ).
//
// Replaces the decode sequence of src/lfm.rs:967-1011 (router_addnorm_route,
// gemv_gather_act, gemv_gather_down_combine4).
#include "mh_device.hpp"
#include "mh_host.hpp"
#include "mh_route.hpp"

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr uint32_t kGrid = 256;
// scratch layout (u32 words)
constexpr uint32_t kEpochWords = 0;       // [kGrid] launch counts
constexpr uint32_t kLogitWords = 512;     // [kMaxExperts] tagged logits (64-bit)
constexpr uint32_t kActWords = 1024;      // [kMaxAct / 2] tagged activation pairs (64-bit)
constexpr int kPairs = 2;          // gate/up row pairs a wave has in flight
constexpr int kMaxTk = 4;
constexpr uint32_t kMaxAct = 8192;  // bf16 activations staged per workgroup (16 KB)
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr uint32_t kSample = 64;          // activation words wave 0 watches before the full read
static_assert(kGrid <= 256 && kLogitWords + 2u * mh::kMaxExperts <= kActWords &&
                  kActWords + kMaxAct <= MH_MOE_DECODE_SCRATCH_WORDS,
              "scratch layout (word 256 is the three-launch path's counter)");

struct FusedArgs {
    const void* rw;        // router [E, K], f32 or bf16
    const float* bias;
    int mode;
    float eps;
    const uint16_t* x;     // [K]
    const uint32_t* gc; const uint16_t* gsc; const uint16_t* gbi;
    const uint32_t* uc; const uint16_t* usc; const uint16_t* ubi;
    const uint32_t* dc; const uint16_t* dsc; const uint16_t* dbi;
    float* logits;         // [E]
    uint32_t* ids;         // [topk]
    uint16_t* weights;     // [topk]
    uint16_t* act;         // [topk, NI]
    uint16_t* out;         // [K]
    uint32_t* scratch;     // launch counts, tagged logits, tagged activation pairs
    uint32_t E, K, NI, gs;
};

__device__ __forceinline__ void put_tagged(uint32_t* scratch, uint32_t word, uint32_t data, uint32_t epoch) {
    __hip_atomic_store(reinterpret_cast<uint64_t*>(scratch) + word,
                       (static_cast<uint64_t>(epoch) << 32) | data, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_tagged(const uint32_t* scratch, uint32_t word) {
    return __hip_atomic_load(reinterpret_cast<const uint64_t*>(scratch) + word, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool fresh(uint64_t w, uint32_t epoch) { return static_cast<uint32_t>(w >> 32) == epoch; }

template <typename WT, int TK>
__global__ __launch_bounds__(kThreads) void k_moe_decode_fused(FusedArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t act_l[kMaxAct];
    __shared__ __attribute__((aligned(16))) float actf_l[kMaxAct];
    __shared__ float xs_l[kMaxAct / 32];
    __shared__ float logit_l[mh::kMaxExperts];
    __shared__ uint32_t epoch_l, bad_l;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t gw = blockIdx.x * kWaves + wave;  // global wave index
    const uint32_t nw = gridDim.x * kWaves;
    const uint32_t C = a.K / 32u;
    const bool live = lane < static_cast<int>(C);
    const uint32_t c = live ? lane : 0u;
    uint32_t* const tl = a.scratch + kLogitWords;  // tagged logits (64-bit words)
    uint32_t* const ta = a.scratch + kActWords;    // tagged activation pairs

    if (threadIdx.x == 0) {
        uint32_t* cnt = a.scratch + kEpochWords + blockIdx.x;
        const uint32_t n = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
        __hip_atomic_store(cnt, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        epoch_l = n;
        bad_l = 0u;
    }
    uint32_t xw[16];
    mh::load_x_words(a.x + 32u * c, xw);

    // ---- phase 1: router logits; row e is computed by wave e / kGrid of
    // workgroup e % kGrid, so the router reads are spread over many CUs
    const uint32_t re = blockIdx.x + static_cast<uint32_t>(wave) * kGrid;
    const bool router = re < a.E;
    float logit = 0.0f;
    if (router) {
        mh::RowWords<WT> rw;
        rw.load(static_cast<const WT*>(a.rw) + static_cast<size_t>(re) * a.K + 32u * c);
        float xr[32], xs, wr[32];
        mh::x_words_to_f32(xw, xr, xs);
        rw.to_f32(wr);
        float p = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            p = __builtin_fmaf(wr[i], xr[i], p);
        }
        float h[4] = {live ? 0.0f + p : 0.0f, 0.0f, 0.0f, 0.0f};
        logit = mh::reduce_rows4(h, lane);
    }
    __syncthreads();  // epoch_l
    const uint32_t epoch = epoch_l;
    if (router && lane == 60) {
        put_tagged(tl, re, __float_as_uint(logit), epoch);
        a.logits[re] = logit;
    }

    // ---- routing: wave 0 polls the tagged logits into LDS, then every wave
    // routes the token itself
    uint32_t ex[TK], wb[TK];
    bool ok = true;
    if (wave == 0) {
        uint32_t pending = 0;
        for (uint32_t i = lane; i < a.E; i += 64u) {
            pending |= 1u << (i / 64u);
        }
        uint32_t spins = 0;
        while (__any(pending != 0u) && spins < kSpinLimit) {
#pragma unroll
            for (int j = 0; j < mh::kMaxExperts / 64; ++j) {
                if ((pending >> j) & 1u) {
                    const uint64_t w = get_tagged(tl, lane + 64u * j);
                    if (fresh(w, epoch)) {
                        logit_l[lane + 64u * j] = __uint_as_float(static_cast<uint32_t>(w));
                        pending &= ~(1u << j);
                    }
                }
            }
            ++spins;
            __builtin_amdgcn_s_sleep(1);
        }
        if (spins >= kSpinLimit && lane == 0) {
            bad_l = 1u;
        }
    }
    __syncthreads();
    ok = bad_l == 0u;
    {
        constexpr int kPerLane = mh::kMaxExperts / 64;
        float sc[kPerLane], cd[kPerLane];
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            const uint32_t i = lane + 64u * j;
            sc[j] = 0.0f;
            cd[j] = -__builtin_inff();
            if (64u * j < a.E && i < a.E) {
                mh::route_score(logit_l[i], a.bias ? a.bias[i] : 0.0f, a.mode, sc[j], cd[j]);
            }
        }
        mh::route_select_regs<TK>(sc, cd, a.E, a.mode, a.eps, ex, wb);
        if (gw == 0 && lane < TK) {
            uint32_t id = ex[0], w = wb[0];
#pragma unroll
            for (int r = 1; r < TK; ++r) {
                id = lane == r ? ex[r] : id;
                w = lane == r ? wb[r] : w;
            }
            a.ids[lane] = id;
            a.weights[lane] = static_cast<uint16_t>(w);
        }
    }

    // ---- this wave's down rows (output gw), loaded now, used in phase 3
    const uint32_t CD = a.NI / 32u;
    const bool dlive = lane < static_cast<int>(CD);
    const uint32_t cd = dlive ? lane : 0u;
    const uint32_t GD = a.NI / a.gs;
    const bool has_out = gw < a.K;
    mh::Chunk<4> dch[TK];
    uint32_t dsr[TK], dbr[TK];
    if (has_out) {
        const uint32_t gcd = (32u * cd) / a.gs;
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            const size_t row = static_cast<size_t>(ex[r]) * a.K + gw;
            dch[r].load_nt(mh::uniform_ptr(reinterpret_cast<const char*>(a.dc) + row * (a.NI / 2u)), cd * 16u);
            dsr[r] = a.dsc[row * GD + gcd];
            dbr[r] = a.dbi[row * GD + gcd];
        }
    }

    // ---- phase 2: gate/up + SwiGLU on pairs of rows (2p, 2p + 1) of one
    // slot, pairs gw, gw + nw, ...; the gate and up dot products of a pair
    // share one 4-row butterfly
    const uint32_t pairs = TK * a.NI / 2u;
    {
        float xr[32], xs;
        mh::x_words_to_f32(xw, xr, xs);
        mh::q4_scale_x(xr);
        const uint32_t row_bytes = a.K / 2u;
        const uint32_t G = a.K / a.gs;
        const uint32_t gc = (32u * c) / a.gs;
        for (uint32_t p0 = gw; p0 < pairs; p0 += nw * kPairs) {
            mh::Chunk<4> ch[kPairs][4];
            uint16_t sv[kPairs][4], bv[kPairs][4];
#pragma unroll
            for (int k = 0; k < kPairs; ++k) {
                const uint32_t p = p0 + k * nw;
                if (p < pairs) {
                    const uint32_t slot = (2u * p) / a.NI;
                    uint32_t e = ex[0];
#pragma unroll
                    for (int r = 1; r < TK; ++r) {
                        e = slot == static_cast<uint32_t>(r) ? ex[r] : e;
                    }
                    const size_t row0 = static_cast<size_t>(e) * a.NI + (2u * p - slot * a.NI);
                    const mh::gbytes gb = mh::uniform_ptr(reinterpret_cast<const char*>(a.gc) + row0 * row_bytes);
                    const mh::gbytes ub = mh::uniform_ptr(reinterpret_cast<const char*>(a.uc) + row0 * row_bytes);
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
                        ch[k][2 * r].load_nt(gb, r * row_bytes + c * 16u);
                        ch[k][2 * r + 1].load_nt(ub, r * row_bytes + c * 16u);
                        const size_t sbi = (row0 + r) * G + gc;
                        sv[k][2 * r] = a.gsc[sbi]; bv[k][2 * r] = a.gbi[sbi];
                        sv[k][2 * r + 1] = a.usc[sbi]; bv[k][2 * r + 1] = a.ubi[sbi];
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < kPairs; ++k) {
                const uint32_t p = p0 + k * nw;
                if (p < pairs) {
                    float h[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float d = ch[k][q].dot(xr);
                        const float hv = __builtin_fmaf(mh::bf16_to_f32(sv[k][q]), d, mh::bf16_to_f32(bv[k][q]) * xs);
                        h[q] = live ? 0.0f + hv : 0.0f;
                    }
                    const int v = __float_as_int(mh::reduce_rows4(h, lane));
                    uint32_t word = 0;
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
                        const float g = mh::round_bf16(__int_as_float(__builtin_amdgcn_readlane(v, 60 + 2 * r)));
                        const float u = mh::round_bf16(__int_as_float(__builtin_amdgcn_readlane(v, 61 + 2 * r)));
                        word |= static_cast<uint32_t>(mh::f32_to_bf16(mh::silu_bf16(g) * u)) << (16 * r);
                    }
                    if (lane == 0) {
                        put_tagged(ta, p, word, epoch);
                        reinterpret_cast<uint32_t*>(a.act)[p] = word;
                    }
                }
            }
        }
    }

    // ---- phase 3: wave 0 watches kSample activation words spread over the
    // buffer; once they are all current every thread reads its share (all of
    // a thread's loads in flight together, stragglers polled again), then one
    // down output per wave with the combine
    {
        if (wave == 0) {
            const uint32_t i = static_cast<uint32_t>(lane) * pairs / kSample;
            bool got = static_cast<uint32_t>(lane) >= kSample;
            uint32_t spins = 0;
            while (!__all(got) && spins < kSpinLimit) {
                if (!got) {
                    got = fresh(get_tagged(ta, i), epoch);
                }
                ++spins;
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
        constexpr int kPer = kMaxAct / 2 / kThreads;  // tagged words per thread
        uint32_t pending = 0, vals[kPer];
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            pending |= threadIdx.x + q * kThreads < pairs ? 1u << q : 0u;
            vals[q] = 0;
        }
        uint32_t spins = 0;
        while (pending != 0u && spins < kSpinLimit) {
            uint64_t w[kPer];
#pragma unroll
            for (int q = 0; q < kPer; ++q) {
                if ((pending >> q) & 1u) {
                    w[q] = get_tagged(ta, threadIdx.x + q * kThreads);
                }
            }
#pragma unroll
            for (int q = 0; q < kPer; ++q) {
                if (((pending >> q) & 1u) && fresh(w[q], epoch)) {
                    vals[q] = static_cast<uint32_t>(w[q]);
                    pending &= ~(1u << q);
                }
            }
            if (pending != 0u) {
                __builtin_amdgcn_s_sleep(1);
            }
            ++spins;
        }
        if (pending != 0u) {
            bad_l = 1u;
        }
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const uint32_t i = threadIdx.x + q * kThreads;
            if (i < pairs) {
                reinterpret_cast<uint32_t*>(act_l)[i] = vals[q];
            }
        }
        __syncthreads();
        // one thread per 32-activation chunk: f32, odd positions scaled for
        // the Q4 dot, float4 k of chunk j stored at slot (k + j) % 8 (the
        // waves' reads below then spread over the LDS banks), and the chunk
        // sum in the order x_words_to_f32 uses
        const uint32_t chunks = TK * a.NI / 32u;
        if (threadIdx.x < chunks) {
            uint32_t w16[16];
            const uint4* src = reinterpret_cast<const uint4*>(&act_l[32u * threadIdx.x]);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint4 v = src[k];
                w16[4 * k] = v.x; w16[4 * k + 1] = v.y; w16[4 * k + 2] = v.z; w16[4 * k + 3] = v.w;
            }
            float xr[32], xs;
            mh::x_words_to_f32(w16, xr, xs);
            mh::q4_scale_x(xr);
            float4* dst = reinterpret_cast<float4*>(&actf_l[32u * threadIdx.x]);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                dst[(k + threadIdx.x) & 7u] = make_float4(xr[4 * k], xr[4 * k + 1], xr[4 * k + 2], xr[4 * k + 3]);
            }
            xs_l[threadIdx.x] = xs;
        }
        __syncthreads();
        ok = ok && bad_l == 0u;
        if (has_out) {
#pragma unroll
            for (int r = 0; r < TK; ++r) {
                dch[r].fence();
                mh::reg_fence(dsr[r]);
                mh::reg_fence(dbr[r]);
            }
            float h[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int r = 0; r < TK; ++r) {
                const uint32_t j = r * CD + cd;  // chunk of slot r read by this lane
                const float4* qv = reinterpret_cast<const float4*>(&actf_l[32u * j]);
                float xr[32];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float4 v = qv[(k + j) & 7u];
                    xr[4 * k] = v.x; xr[4 * k + 1] = v.y; xr[4 * k + 2] = v.z; xr[4 * k + 3] = v.w;
                }
                const float d = dch[r].dot(xr);
                const float hv = __builtin_fmaf(__uint_as_float(dsr[r] << 16), d, __uint_as_float(dbr[r] << 16) * xs_l[j]);
                h[r] = dlive ? 0.0f + hv : 0.0f;
            }
            const int v = __float_as_int(mh::reduce_rows4(h, lane));
            float total = 0.0f;
#pragma unroll
            for (int r = 0; r < TK; ++r) {
                const float vr = mh::round_bf16(__int_as_float(__builtin_amdgcn_readlane(v, 60 + r)));
                total = total + mh::round_bf16(mh::bf16_to_f32(static_cast<uint16_t>(wb[r])) * vr);
            }
            if (lane == 0) {
                a.out[gw] = ok ? mh::f32_to_bf16(total) : static_cast<uint16_t>(0x7fc0);
            }
        }
    }
}

}  // namespace

namespace mh {

// Fused decode step; MH_ERR_UNSUPPORTED when the shapes or the device need
// the three-launch path (the caller then uses it).
int moe_decode_fused(const void* router, int router_dtype, const float* bias, int mode, float eps,
                     const mh_quant_weights* gate, const mh_quant_weights* up,
                     const mh_quant_weights* down, uint32_t n_experts, uint32_t topk,
                     const uint16_t* x, uint16_t* out, float* logits, uint32_t* ids,
                     uint16_t* weights, uint16_t* act, uint32_t* scratch, hipStream_t stream) {
    const uint32_t NI = gate->out_features / n_experts;
    const uint32_t K = gate->in_features;
    // all kGrid workgroups resident (one per CU), one wave per output and
    // per router row, the activations fit the LDS stage
    if (mh::cu_count() < static_cast<int>(kGrid) || K > 2048u || K % 64u != 0 || NI % 64u != 0 ||
        topk < 1 || topk > static_cast<uint32_t>(kMaxTk) || topk * NI > kMaxAct ||
        gate->group_size % 32u != 0 || down->group_size != gate->group_size ||
        up->group_size != gate->group_size || n_experts > static_cast<uint32_t>(kMaxExperts) ||
        K > kGrid * kWaves || !mh::aligned(router, 16) ||
        !mh::aligned(act, 4) || !mh::aligned(logits, 4) || !mh::aligned(scratch, 8)) {
        return MH_ERR_UNSUPPORTED;
    }
    FusedArgs a{};
    a.rw = router; a.bias = bias; a.mode = mode; a.eps = eps; a.x = x;
    a.gc = gate->codes; a.gsc = gate->scales; a.gbi = gate->biases;
    a.uc = up->codes; a.usc = up->scales; a.ubi = up->biases;
    a.dc = down->codes; a.dsc = down->scales; a.dbi = down->biases;
    a.logits = logits; a.ids = ids; a.weights = weights; a.act = act; a.out = out; a.scratch = scratch;
    a.E = n_experts; a.K = K; a.NI = NI; a.gs = gate->group_size;
    const bool f32 = router_dtype == MH_DTYPE_F32;
#define MH_FUSED_LAUNCH(TK)                                                                                  \
    if (f32) hipLaunchKernelGGL((k_moe_decode_fused<float, TK>), dim3(kGrid), dim3(kThreads), 0, stream, a); \
    else hipLaunchKernelGGL((k_moe_decode_fused<uint16_t, TK>), dim3(kGrid), dim3(kThreads), 0, stream, a);
    switch (topk) {
        case 1: MH_FUSED_LAUNCH(1) break;
        case 2: MH_FUSED_LAUNCH(2) break;
        case 3: MH_FUSED_LAUNCH(3) break;
        default: MH_FUSED_LAUNCH(4) break;
    }
#undef MH_FUSED_LAUNCH
    return mh::launch_status("k_moe_decode_fused");
}

}  // namespace mh

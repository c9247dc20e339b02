// moe_route_mma.hip -- the prefill MoE step's router and top-k on the matrix
// cores, the routing exact (src/lfm.rs:860-905: router_prefill, then
// moe_route_batch; lfm.metal:464-537, 1558-1602).
//
// One workgroup routes kTok = 16 consecutive tokens (one routing block: it
// also writes the block's expert histogram).  A bf16 router W [e <= 64, K]
// and bf16 x:
//   1. x's 16 rows are staged in the LDS, W's rows a quarter of K at a time
//      (coalesced loads; a wave reading 16 B of each of 16 rows per
//      instruction took twice as long); each of the 16 waves takes 16
//      experts and a quarter of every round's k and forms, on
//      v_mfma_f32_16x16x32_bf16 (bf16 products are exact in f32), its part of
//      the approximate logit a = sum x w and of c = sum |x| |w|; the four
//      parts are added in order;
//   2. per token, lane x = expert x: the chunk-order logit z (the oracle's
//      and the other routers' value: lane c's fma chain over elements 32 c ..
//      32 c + 31 from 0, then the 64-chunk xor butterfly, then + 0) lies in
//      [a - E, a + E], E = 2^-12 c + 2^-138.  Both a and z sum the same exact
//      products; each term reaches a through at most 32 roundings inside its
//      matrix instruction, one per later instruction of its chain (K / 128
//      - 1) and 3 quarter sums (50 for K = 2048), and z through 32 + 6; with
//      unit roundoff 2^-23 (which also covers truncation) |a - z| <= 88 *
//      2^-23 * sum |x w| < 2^-16 c, so 2^-12 leaves a factor of 16 for the
//      hardware's summation order, and 2^-138 the roundings in the subnormal
//      range.  The matrix cores keep bf16 denormal inputs: a flushed one
//      would fall outside this bound, and tests/test_gpu_prefill.py checks
//      the bound on every logit the kernel does not recompute, with tokens
//      whose logits the denormals dominate;
//   3. the scores' bounds follow: softmax ranks on z itself; sigmoid + bias
//      ranks on 1 / (1 + expf_fixed(-z)) + bias, which over all floats drops
//      at most 2^-24 below its running maximum (tests/test_oracle_math.py),
//      so [s(a - E) - 2^-24, s(a + E) + 2^-24] + bias, widened by a few ulps
//      for the f32 arithmetic, holds the exact score.  An expert can be among
//      the top k only if its upper bound reaches the k-th largest lower
//      bound: those candidates (typically k, a few more on near ties; every
//      expert of a token whose a or E is not finite) get their chunk-order
//      logits computed exactly, the others take part as -inf, and the
//      selection and weights are route_select_ids / route_weights_regs on
//      the exact scores -- the same ids and weight bits as routing every
//      expert's chunk-order logit.
// The logits region receives the chunk-order value of every candidate (every
// chosen expert among them) and a for the other experts.
#include "mh_device.hpp"
#include "mh_host.hpp"
#include "mh_route.hpp"

namespace {

constexpr int kWaves = 16;
constexpr int kThreads = kWaves * 64;
constexpr uint32_t kTok = mh::kPrefillRouteBlock;  // tokens per workgroup (one routing block): one per wave
constexpr uint32_t kMaxK = 2048;
constexpr uint32_t kPitch = kMaxK + 8;        // bf16 per staged x row: rows 16 bytes apart in the banks
constexpr uint32_t kKParts = 4;               // quarters of K, one per wave group
static_assert(kTok == static_cast<uint32_t>(kWaves) && kWaves == 4 * kKParts, "4 expert quarters x 4 K quarters");

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct RmArgs {
    const uint16_t* x;  // [m, k] bf16
    const uint16_t* w;  // [e, k] bf16
    const float* bias;  // [e] or null
    float* logits;      // [m, e]
    uint32_t* ids;      // [m, topk]
    uint16_t* gw;       // [m, topk] bf16
    uint32_t* hb;       // [blocks, e] expert histograms of the routing blocks
    uint32_t m, e, k;
    int mode;
    float eps;
};

__device__ __forceinline__ bf16x8 as_bf16x8(mh::u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ mh::u32x4 abs_bf16x8(mh::u32x4 v) {
    const uint32_t m = 0x7fff7fffu;
    return mh::u32x4{v.x & m, v.y & m, v.z & m, v.w & m};
}

// STEPS: MFMA steps of 32 k per wave (K = 128 STEPS).
template <int TK, int STEPS>
__global__ __launch_bounds__(kThreads) void k_route_mma(RmArgs a) {
    constexpr uint32_t K = 128u * STEPS;
    constexpr uint32_t KQ = K / kKParts;             // k per round
    constexpr uint32_t kWPitch = KQ + 8u;            // bf16 per staged W row: rows 16 bytes apart in the banks
    constexpr uint32_t kXPieces = kTok * (K / 8u) / kThreads;  // 16-byte pieces per thread
    constexpr uint32_t kWPieces = 64u * (KQ / 8u) / kThreads;
    constexpr uint32_t kSub = KQ / 4u;               // k of a round per wave (4 sub-slices)
    static_assert(kXPieces >= 1 && kWPieces >= 1 && kSub % 32u == 0, "tiling");
    static_assert(2u * kKParts * kTok * 64u * 4u <= 64u * (kMaxK / kKParts + 8u) * 2u, "partials fit the W stage");
    __shared__ __attribute__((aligned(16))) uint16_t xt[kTok * kPitch];
    __shared__ __attribute__((aligned(16))) uint16_t ws[64u * (kMaxK / kKParts + 8u)];  // a round's W; then the partials
    __shared__ uint32_t hist[64];
    float (*const za)[kTok][64] = reinterpret_cast<float (*)[kTok][64]>(ws);
    float (*const zc)[kTok][64] = za + kKParts;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t t0 = blockIdx.x * kTok;
    const uint32_t nt = min(kTok, a.m - t0);
    const uint32_t E = a.e;

    // ---- x's rows (a partial last block repeats its last token), then the
    // first round's W: every load coalesced (a wave reads 1 KB of one row)
    mh::u32x4 xv[kXPieces];
#pragma unroll
    for (uint32_t i = 0; i < kXPieces; ++i) {
        const uint32_t p = threadIdx.x + i * kThreads;
        const uint32_t row = p / (K / 8u), col = p % (K / 8u);
        const uint32_t tok = t0 + min(row, nt - 1u);
        xv[i] = *reinterpret_cast<const mh::u32x4*>(a.x + static_cast<size_t>(tok) * K + 8u * col);
    }
    mh::u32x4 wn[kWPieces];
    auto load_round = [&](uint32_t r) {
#pragma unroll
        for (uint32_t i = 0; i < kWPieces; ++i) {
            const uint32_t p = threadIdx.x + i * kThreads;
            const uint32_t row = min(p / (KQ / 8u), E - 1u), col = p % (KQ / 8u);
            wn[i] = *reinterpret_cast<const mh::u32x4*>(a.w + static_cast<size_t>(row) * K + r * KQ + 8u * col);
        }
    };
    load_round(0);
#pragma unroll
    for (uint32_t i = 0; i < kXPieces; ++i) {
        const uint32_t p = threadIdx.x + i * kThreads;
        const uint32_t row = p / (K / 8u), col = p % (K / 8u);
        *reinterpret_cast<mh::u32x4*>(xt + row * kPitch + 8u * col) = xv[i];
    }
    if (threadIdx.x < 64) {
        hist[threadIdx.x] = 0u;
    }

    // ---- 1. approximate logits and the sums of |x| |w|, K in four rounds:
    // the round's W rows staged in the LDS (the next round's loads in flight
    // meanwhile); wave (q, kk) takes experts 16 q + lane % 16 and sub-slice
    // kk of the round's k, k = 8 (lane / 16) .. + 8 of every 32-step
    const uint32_t q = static_cast<uint32_t>(wave) & 3u, kk = static_cast<uint32_t>(wave) >> 2;
    const uint32_t n16 = static_cast<uint32_t>(lane) & 15u, r16 = static_cast<uint32_t>(lane) >> 4;
    const bool busy = 16u * q < E;  // uniform: the wave has experts
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, acb = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t r = 0; r < kKParts; ++r) {
        if (r > 0) {
            __syncthreads();  // every wave is done with the previous round's rows
        }
#pragma unroll
        for (uint32_t i = 0; i < kWPieces; ++i) {
            const uint32_t p = threadIdx.x + i * kThreads;
            const uint32_t row = p / (KQ / 8u), col = p % (KQ / 8u);
            *reinterpret_cast<mh::u32x4*>(ws + row * kWPitch + 8u * col) = wn[i];
        }
        if (r + 1u < kKParts) {
            load_round(r + 1u);
        }
        __syncthreads();
        if (busy) {
            const uint16_t* xr = xt + n16 * kPitch + r * KQ + kk * kSub + 8u * r16;
            const uint16_t* wr = ws + (16u * q + n16) * kWPitch + kk * kSub + 8u * r16;
#pragma unroll
            for (uint32_t s = 0; s < kSub / 32u; ++s) {
                const mh::u32x4 xs = *reinterpret_cast<const mh::u32x4*>(xr + 32u * s);
                const mh::u32x4 wv = *reinterpret_cast<const mh::u32x4*>(wr + 32u * s);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xs), as_bf16x8(wv), acc, 0, 0, 0);
                acb = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(abs_bf16x8(xs)), as_bf16x8(abs_bf16x8(wv)),
                                                              acb, 0, 0, 0);
            }
        }
    }
    __syncthreads();  // the W stage becomes the partials
    if (busy) {
        // lane holds tokens 4 r16 .. + 3 of expert 16 q + n16
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            za[kk][4u * r16 + v][16u * q + n16] = acc[v];
            zc[kk][4u * r16 + v][16u * q + n16] = acb[v];
        }
    }
    __syncthreads();

    // ---- 2. token t = wave (lane = expert): the bounds, the candidates,
    // their chunk-order logits, the exact selection
    const uint32_t t = static_cast<uint32_t>(wave);
    const uint32_t ex = static_cast<uint32_t>(lane);
    const bool valid = ex < E;
    const float bias = a.bias != nullptr && valid ? a.bias[ex] : 0.0f;
    float ap = 0.0f, cp = 0.0f;
    if (valid) {
        ap = ((za[0][t][ex] + za[1][t][ex]) + za[2][t][ex]) + za[3][t][ex];
        cp = ((zc[0][t][ex] + zc[1][t][ex]) + zc[2][t][ex]) + zc[3][t][ex];
    }
    const float bound = __builtin_fmaf(cp, 0x1p-12f, 0x1p-138f);
    const bool fin = __builtin_isfinite(ap) && __builtin_isfinite(bound);
    const bool all = __any(valid && !fin);  // recompute every expert of this token
    float lo, hi;
    if (a.mode == 1) {
        lo = ap - bound;
        hi = ap + bound;
    } else {
        const float sl = 1.0f / (1.0f + mh::expf_fixed(-(ap - bound)));
        const float sh = 1.0f / (1.0f + mh::expf_fixed(-(ap + bound)));
        lo = (sl + bias) - (0x1p-22f + __builtin_fabsf(sl + bias) * 0x1p-20f);
        hi = (sh + bias) + (0x1p-22f + __builtin_fabsf(sh + bias) * 0x1p-20f);
    }
    // the k-th largest lower bound over the valid experts (a NaN bound never
    // counts), then the candidates: upper bound at least that
    float kth = -__builtin_inff();
    {
        float v = valid && lo == lo ? lo : -__builtin_inff();
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            const float mx = mh::wave_max_f32(v);
            kth = mx;
            const unsigned long long at = __ballot(v == mx);
            const uint32_t who = at != 0ull ? static_cast<uint32_t>(__builtin_ctzll(at)) : 64u;
            v = static_cast<uint32_t>(lane) == who ? -__builtin_inff() : v;
        }
    }
    // with fewer than k experts surely eligible (a finite lower bound), the
    // selection's default pick, expert 0, may be taken: its score is then
    // needed exactly too
    const bool sure = __popcll(__ballot(valid && lo > -__builtin_inff())) >= static_cast<uint32_t>(TK);
    const bool pick = valid && (all || hi >= kth || (!sure && ex == 0u));
    unsigned long long cand = __ballot(pick);

    // chunk-order logits of the candidates (lane c = chunk c: its fma chain
    // over elements 32 c .. 32 c + 31 from 0, the 64-chunk butterfly, + 0),
    // up to four at a time with their rows' loads out before the first chain
    constexpr uint32_t C = K / 32u;
    const bool live = static_cast<uint32_t>(lane) < C;
    const uint32_t c = live ? static_cast<uint32_t>(lane) : 0u;
    float xf[32];
    {
        const mh::u32x4* xp = reinterpret_cast<const mh::u32x4*>(xt + t * kPitch + 32u * c);
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
            const mh::u32x4 v = xp[pp];
            const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                xf[8 * pp + 2 * d] = mh::bf16lo(wd[d]);
                xf[8 * pp + 2 * d + 1] = mh::bf16hi(wd[d]);
            }
        }
    }
    float zx = ap;  // this lane's expert: its logit, exact where recomputed
    while (cand != 0ull) {
        uint32_t ce[4];
        uint32_t cnt = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            ce[u] = cand != 0ull ? static_cast<uint32_t>(__builtin_ctzll(cand)) : (u > 0 ? ce[u - 1] : 0u);
            if (cand != 0ull) {
                cand &= cand - 1ull;
                ++cnt;
            }
        }
        mh::u32x4 wv[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const mh::u32x4* wp = reinterpret_cast<const mh::u32x4*>(a.w + static_cast<size_t>(ce[u]) * K + 32u * c);
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
                wv[u][pp] = wp[pp];
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (static_cast<uint32_t>(u) < cnt) {  // uniform
                float acc = 0.0f;
#pragma unroll
                for (int pp = 0; pp < 4; ++pp) {
                    const uint32_t wd[4] = {wv[u][pp].x, wv[u][pp].y, wv[u][pp].z, wv[u][pp].w};
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        acc = __builtin_fmaf(mh::bf16lo(wd[d]), xf[8 * pp + 2 * d], acc);
                        acc = __builtin_fmaf(mh::bf16hi(wd[d]), xf[8 * pp + 2 * d + 1], acc);
                    }
                }
                const float z = mh::lane63(mh::wave_sum_lane63(live ? acc : 0.0f)) + 0.0f;
                zx = ex == ce[u] ? z : zx;
            }
        }
    }
    // exact selection: the candidates with their exact scores, the rest -inf
    float sc[1], cd[1];
    sc[0] = 0.0f;
    cd[0] = -__builtin_inff();
    if (pick) {
        mh::route_score(zx, bias, a.mode, sc[0], cd[0]);
    }
    uint32_t idv[TK];
    float sv[TK];
    mh::route_select_ids<TK, 1>(sc, cd, idv, sv);
    uint32_t wb[TK];
    mh::route_weights_regs<TK>(sv, a.mode, a.eps, wb);
    if (t < nt) {
        const size_t tok = t0 + t;
        if (valid) {
            a.logits[tok * E + ex] = zx;
        }
        if (static_cast<uint32_t>(lane) < static_cast<uint32_t>(TK)) {
            uint32_t id = idv[0], w = wb[0];
#pragma unroll
            for (int r = 1; r < TK; ++r) {
                id = static_cast<uint32_t>(lane) == static_cast<uint32_t>(r) ? idv[r] : id;
                w = static_cast<uint32_t>(lane) == static_cast<uint32_t>(r) ? wb[r] : w;
            }
            a.ids[tok * TK + lane] = id;
            a.gw[tok * TK + lane] = static_cast<uint16_t>(w);
            atomicAdd(&hist[id], 1u);
        }
    }
    __syncthreads();
    if (threadIdx.x < E) {
        a.hb[static_cast<size_t>(blockIdx.x) * E + threadIdx.x] = hist[threadIdx.x];
    }
}

}  // namespace

namespace mh {

// Whether mh_moe_prefill routes with k_route_mma: a bf16 router of at most 64
// experts, K 1024 or 2048 (the model's d_model), 16-byte aligned rows.
bool route_mma_fits(const void* w, int w_dtype, const uint16_t* x, uint32_t e, uint32_t k, uint32_t topk) {
    return w_dtype == MH_DTYPE_BF16 && e >= 1u && e <= 64u && topk >= 1u && topk <= static_cast<uint32_t>(kMaxTopk) &&
           topk <= e && (k == 1024u || k == 2048u) && mh::aligned(w, 16) && mh::aligned(x, 16);
}

int route_mma(const uint16_t* x, const uint16_t* w, const float* bias, int mode, float eps, uint32_t m, uint32_t e,
              uint32_t k, uint32_t topk, float* logits, uint32_t* ids, uint16_t* gw, uint32_t* hb, hipStream_t stream) {
    RmArgs a{};
    a.x = x;
    a.w = w;
    a.bias = bias;
    a.logits = logits;
    a.ids = ids;
    a.gw = gw;
    a.hb = hb;
    a.m = m;
    a.e = e;
    a.k = k;
    a.mode = mode;
    a.eps = eps;
    const dim3 grid((m + kTok - 1u) / kTok);
#define MH_RMMA(TK)                                                                          \
    case TK:                                                                                 \
        if (k == 2048u) {                                                                    \
            hipLaunchKernelGGL((k_route_mma<TK, 16>), grid, dim3(kThreads), 0, stream, a); \
        } else {                                                                             \
            hipLaunchKernelGGL((k_route_mma<TK, 8>), grid, dim3(kThreads), 0, stream, a);  \
        }                                                                                    \
        break;
    switch (topk) {
        MH_RMMA(1) MH_RMMA(2) MH_RMMA(3) MH_RMMA(4) MH_RMMA(5) MH_RMMA(6) MH_RMMA(7) MH_RMMA(8)
        default: return MH_ERR_UNSUPPORTED;
    }
#undef MH_RMMA
    return mh::launch_status("k_route_mma");
}

}  // namespace mh

// moe_decode.hip -- router GEMVs, top-k routing and the decode MoE expert
// GEMVs for gfx950.
//
// Replaces lfm.metal:368-428 (router GEMV), :464-537 (prefill router),
// :541-703 (top-k), :705-855 (fused router + route, minus the add+RMSNorm
// prologue), :1392-1554 (expert gate/up + SwiGLU, dense gate/up, expert down
// + combine) and :1558-1602 (batch routing).
//
// All dot products use the chunk order of mh_device.hpp, so router logits
// (and hence expert ids) and every expert output are bit-identical to the CPU
// oracle.
#include "mh_device.hpp"
#include "mh_host.hpp"
#include "mh_route.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / mh::kWave;
constexpr int kXPitch = 36;

// ------------------------------------------------------------ dense GEMV ---
// y[t, e] = chunk-order dot(W[e, :], x[t, :]) for a tile of TT tokens per
// workgroup (x staged once in LDS) and EPW experts per wave.

template <typename WT>
__device__ __forceinline__ void load_wchunk(const WT* w, float (&wr)[32]);

template <>
__device__ __forceinline__ void load_wchunk<float>(const float* w, float (&wr)[32]) {
    const float4* p = reinterpret_cast<const float4*>(w);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const float4 v = p[q];
        wr[4 * q] = v.x; wr[4 * q + 1] = v.y; wr[4 * q + 2] = v.z; wr[4 * q + 3] = v.w;
    }
}

template <>
__device__ __forceinline__ void load_wchunk<uint16_t>(const uint16_t* w, float (&wr)[32]) {
    const uint4* p = reinterpret_cast<const uint4*>(w);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 v = p[q];
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            wr[8 * q + 2 * j] = mh::bf16lo(u[j]);
            wr[8 * q + 2 * j + 1] = mh::bf16hi(u[j]);
        }
    }
}

struct DenseArgs {
    const void* w;     // [n, k] f32 or bf16
    const uint16_t* x; // bf16 [m, k]
    float* y;          // f32 [m, n]
    uint32_t m, n, k;
    // fused routing (decode): when done != null the last workgroup routes
    const float* bias;
    uint32_t* ids;
    uint16_t* weights;
    uint32_t* done;
    uint32_t topk;
    int mode;
    float eps;
};

// Stage x rows [t0, t0 + nt) into LDS as padded f32 chunks, one 32-element
// chunk per thread per step with 16-byte loads (k % 32 == 0 keeps each
// chunk 64-byte aligned when x is 16-byte aligned).
__device__ inline void stage_x(const uint16_t* x, uint32_t t0, uint32_t nt, uint32_t k,
                               float* xl, int tt) {
    const uint32_t C = k / 32u;
    for (uint32_t i = threadIdx.x; i < static_cast<uint32_t>(tt) * C; i += kThreads) {
        const uint32_t t = i / C, c = i % C;
        float xc[32], s;
        mh::load_x_chunk(x + static_cast<size_t>(t0 + (t < nt ? t : 0)) * k + 32u * c, xc, s);
        float4* d = reinterpret_cast<float4*>(xl + (static_cast<size_t>(t) * C + c) * kXPitch);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            d[q] = make_float4(xc[4 * q], xc[4 * q + 1], xc[4 * q + 2], xc[4 * q + 3]);
        }
    }
}

template <typename WT, int TT, int EPW>
__global__ __launch_bounds__(kThreads) void k_dense_gemv(DenseArgs a) {
    extern __shared__ float xl[];  // [TT][C][kXPitch]
    __shared__ uint32_t last;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t C = a.k / 32u;
    const uint32_t t0 = blockIdx.x * TT;
    const uint32_t nt = min(static_cast<uint32_t>(TT), a.m - t0);
    stage_x(a.x, t0, nt, a.k, xl, TT);
    __syncthreads();
    const WT* w = static_cast<const WT*>(a.w);
#pragma unroll 1
    for (int j = 0; j < EPW; ++j) {
        const uint32_t e = (blockIdx.y * kWaves + wave) * EPW + j;
        if (e >= a.n) {
            break;
        }
        float acc[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            acc[t] = 0.0f;
        }
        for (uint32_t c = lane; c < C; c += 64) {
            float wr[32];
            load_wchunk<WT>(w + static_cast<size_t>(e) * a.k + 32u * c, wr);
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const float4* xs = reinterpret_cast<const float4*>(xl + (static_cast<size_t>(t) * C + c) * kXPitch);
                float p = 0.0f;
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float4 v = xs[q];
                    p = __builtin_fmaf(wr[4 * q], v.x, p);
                    p = __builtin_fmaf(wr[4 * q + 1], v.y, p);
                    p = __builtin_fmaf(wr[4 * q + 2], v.z, p);
                    p = __builtin_fmaf(wr[4 * q + 3], v.w, p);
                }
                acc[t] = acc[t] + p;
            }
        }
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            const float v = mh::lane63(mh::wave_sum_lane63(acc[t]));
            if (lane == 0 && static_cast<uint32_t>(t) < nt) {
                float* dst = a.y + static_cast<size_t>(t0 + t) * a.n + e;
                if (a.done != nullptr) {
                    // published with a returning atomic so the finisher below
                    // reads it from the coherence point without a cache flush
                    const uint32_t old = __hip_atomic_exchange(
                        reinterpret_cast<uint32_t*>(dst), __float_as_uint(v), __ATOMIC_RELAXED,
                        __HIP_MEMORY_SCOPE_AGENT);
                    if (old == 0x7fc00001u) {
                        last = 0;
                    }
                } else {
                    *dst = v;
                }
            }
        }
    }
    if (a.done == nullptr) {
        return;
    }
    // Fused decode routing: the last workgroup to finish routes token 0.
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t total = gridDim.x * gridDim.y;
        const uint32_t prev =
            __hip_atomic_fetch_add(a.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = (prev == total - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (!last) {
        return;
    }
    __shared__ float s[mh::kMaxExperts], cand[mh::kMaxExperts];
    for (uint32_t i = threadIdx.x; i < a.n; i += kThreads) {
        const float z = __uint_as_float(__hip_atomic_fetch_or(reinterpret_cast<uint32_t*>(a.y) + i,
                                                              0u, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT));
        mh::route_score(z, a.bias ? a.bias[i] : 0.0f, a.mode, s[i], cand[i]);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        mh::route_select(s, cand, a.n, a.topk, a.mode, a.eps, a.ids, a.weights);
    }
    if (threadIdx.x == 0) {
        __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Router logits of many tokens, tiled: a workgroup takes kRtTokens tokens
// and kRtExperts experts; the experts' rows are staged once in the LDS as
// f32 (chunk c of row e as 8 pieces of 16 bytes, piece q at q ^ ((c >> 1) &
// 7), so the 16 lanes of a 16-byte read cover all 64 banks once), then each
// wave runs its tokens in groups of four with x in registers (lane c holds
// chunk c; the first group's x is loaded before the rows are staged) against
// one expert row at a time from the LDS (the next row's read in flight; two
// workgroups per CU cover each other's waits).  Per (token, expert) the
// arithmetic is the chunk order of k_dense_gemv: lane c's fma chain over its
// 32 elements from 0, then the xor butterfly over the 64 chunks -- here for
// eight values at once (four tokens x two experts): each lane's eight chain
// values go to the LDS as [value][chunk], lane 8v + j adds chunks 8j .. 8j +
// 7 of value v (levels 1-3) and levels 4-6 are DPP quad_perm and row_shr:4,
// leaving value v in lane 8v + 7; the chunk order's +0 is applied once to
// that sum (an IEEE sum is -0 only when both operands are, so the bits are
// the same).  W comes from the L2 once per workgroup.
constexpr int kRtTokens = 64;
constexpr int kRtExperts = 8;
constexpr int kRtGroup = 4;                                // tokens per group
constexpr int kRtGroups = kRtTokens / (kRtGroup * kWaves);  // groups per wave

template <typename WT>
__global__ __launch_bounds__(kThreads, 2) void k_router_tiles(DenseArgs a) {
    extern __shared__ float wl[];  // [kRtExperts][C][8 pieces][4]
    __shared__ float zl[kRtTokens][kRtExperts];
    __shared__ __attribute__((aligned(16))) float tl[kWaves][8 * 64];  // a wave's chain values, [value][chunk]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t C = a.k / 32u;
    const bool live = lane < static_cast<int>(C);
    const uint32_t c = live ? lane : 0u;
    const uint32_t t_base = blockIdx.x * kRtTokens;
    const uint32_t e0 = blockIdx.y * kRtExperts;
    const uint32_t ne = min(static_cast<uint32_t>(kRtExperts), a.n - e0);
    const uint32_t t_wave = static_cast<uint32_t>(wave * kRtGroup * kRtGroups);
    float* tw = tl[wave];
    auto load_group = [&](int g, uint32_t (&xw)[kRtGroup][16]) {
#pragma unroll
        for (int t = 0; t < kRtGroup; ++t) {
            const uint32_t tok = min(t_base + t_wave + static_cast<uint32_t>(kRtGroup * g + t), a.m - 1u);
            const uint4* xv = reinterpret_cast<const uint4*>(a.x + static_cast<size_t>(tok) * a.k + 32u * c);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 v = xv[q];
                xw[t][4 * q] = v.x; xw[t][4 * q + 1] = v.y; xw[t][4 * q + 2] = v.z; xw[t][4 * q + 3] = v.w;
            }
        }
    };
    uint32_t xw[kRtGroup][16];
    load_group(0, xw);
    // stage rows e0 .. e0 + ne: 8 elements (two pieces) per thread and step
    const WT* w = static_cast<const WT*>(a.w);
    for (uint32_t i = threadIdx.x; i < ne * C * 4u; i += kThreads) {
        const uint32_t e = i / (C * 4u), r = i % (C * 4u), cc = r / 4u, q2 = r % 4u;
        const size_t src = static_cast<size_t>(e0 + e) * a.k + 32u * cc + 8u * q2;
        float v[8];
        if constexpr (sizeof(WT) == 4) {
            const float4 lo = *reinterpret_cast<const float4*>(w + src);
            const float4 hi = *reinterpret_cast<const float4*>(w + src + 4);
            v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
            v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
        } else {
            const uint4 u = *reinterpret_cast<const uint4*>(w + src);
            const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[2 * j] = mh::bf16lo(uw[j]);
                v[2 * j + 1] = mh::bf16hi(uw[j]);
            }
        }
        const uint32_t swz = (cc >> 1) & 7u;
        float* base = wl + static_cast<size_t>(e * C + cc) * 32u;
        *reinterpret_cast<float4*>(base + 4u * ((2u * q2) ^ swz)) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(base + 4u * ((2u * q2 + 1u) ^ swz)) = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();
    const uint32_t swz = (c >> 1) & 7u;
    auto read_row = [&](uint32_t e, float (&wr)[32]) {
        const uint32_t ec = min(e, ne - 1u);  // a missing odd expert reads a staged row; never stored
        const float* base = wl + static_cast<size_t>(ec * C + c) * 32u;
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q) {
            const float4 v = *reinterpret_cast<const float4*>(base + 4u * (q ^ swz));
            wr[4 * q] = v.x; wr[4 * q + 1] = v.y; wr[4 * q + 2] = v.z; wr[4 * q + 3] = v.w;
        }
    };
    // one group of four tokens against the staged experts
    auto group = [&](int g, const uint32_t (&xg)[kRtGroup][16]) {
        float xr[kRtGroup][32];
#pragma unroll
        for (int t = 0; t < kRtGroup; ++t) {
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                xr[t][2 * q] = mh::bf16lo(xg[t][q]);
                xr[t][2 * q + 1] = mh::bf16hi(xg[t][q]);
            }
        }
        // lane c's chain values of the group's four tokens for one expert
        // row into values v0 .. v0 + 3 of the wave's LDS block
        auto chains = [&](const float (&wr)[32], int v0) {
#pragma unroll
            for (int t = 0; t < kRtGroup; ++t) {
                float p = 0.0f;
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    p = __builtin_fmaf(wr[i], xr[t][i], p);
                }
                tw[(v0 + t) * 64 + lane] = live ? p : 0.0f;
            }
        };
        // experts e, e + 1: eight values, then the 64-chunk sums
        float wa[32], wb[32];
        read_row(0, wa);
#pragma unroll 1
        for (uint32_t e = 0; e < ne; e += 2) {
            read_row(e + 1, wb);
            chains(wa, 0);
            if (e + 2 < ne) {
                read_row(e + 2, wa);
            }
            chains(wb, 4);
            __builtin_amdgcn_wave_barrier();
            const float4 q0 = *reinterpret_cast<const float4*>(tw + 8 * lane);
            const float4 q1 = *reinterpret_cast<const float4*>(tw + 8 * lane + 4);
            float v = ((q0.x + q0.y) + (q0.z + q0.w)) + ((q1.x + q1.y) + (q1.z + q1.w));
            v = v + mh::qmove<0xB1>(v);           // chunks xor 8  (quad_perm 1,0,3,2)
            v = v + mh::qmove<0x4E>(v);           // chunks xor 16 (quad_perm 2,3,0,1)
            v = v + mh::dpp_move<0x114, 0xf>(v);  // chunks xor 32 (row_shr:4)
            __builtin_amdgcn_wave_barrier();
            const uint32_t val = static_cast<uint32_t>(lane) >> 3;  // token (val & 3), expert e + (val >> 2)
            const uint32_t ee = e + (val >> 2);
            if ((lane & 7) == 7 && ee < ne) {
                zl[t_wave + kRtGroup * g + (val & 3u)][ee] = v + 0.0f;
            }
        }
    };
    group(0, xw);  // the first group's x was loaded before the staging
#pragma unroll 1
    for (int g = 1; g < kRtGroups; ++g) {
        uint32_t xn[kRtGroup][16];
        load_group(g, xn);
        group(g, xn);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < kRtTokens * ne; i += kThreads) {
        const uint32_t t = i / ne, e = i % ne;
        if (t_base + t < a.m) {
            a.y[static_cast<size_t>(t_base + t) * a.n + e0 + e] = zl[t][e];
        }
    }
}

template <typename WT>
int launch_router_tiles(const DenseArgs& a, hipStream_t stream) {
    const uint32_t C = a.k / 32u;
    const size_t lds = static_cast<size_t>(kRtExperts) * C * 32u * sizeof(float);
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_router_tiles<WT>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) {
        return mh::hip_error(e, "k_router_tiles: LDS attribute");
    }
    const dim3 grid((a.m + kRtTokens - 1) / kRtTokens, (a.n + kRtExperts - 1) / kRtExperts);
    hipLaunchKernelGGL(k_router_tiles<WT>, grid, dim3(kThreads), lds, stream, a);
    return mh::launch_status("k_router_tiles");
}

// Decode router logits only (the routing runs in the expert kernel): one
// wave per 4 experts, x in registers, the four rows reduced together.
template <typename WT>
__global__ __launch_bounds__(64) void k_router_logits(DenseArgs a) {
    const int lane = threadIdx.x;
    const uint32_t C = a.k / 32u;
    const bool live = lane < static_cast<int>(C);
    const uint32_t c = live ? lane : 0u;
    const uint32_t e0 = blockIdx.x * 4u;
    uint32_t xw[16];
    mh::load_x_words(a.x + 32u * c, xw);
    const WT* w = static_cast<const WT*>(a.w) + 32u * c;
    mh::RowWords<WT> rw[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        rw[r].load(w + static_cast<size_t>(min(e0 + r, a.n - 1u)) * a.k);
    }
    mh::x_words_fence(xw);
    float xr[32], xs;
    mh::x_words_to_f32(xw, xr, xs);
    float h[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float wr[32];
        rw[r].to_f32(wr);
        float p = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            p = __builtin_fmaf(wr[i], xr[i], p);
        }
        h[r] = live ? 0.0f + p : 0.0f;
    }
    const float v = mh::reduce_rows4(h, lane);
    if (lane >= 60 && e0 + (lane - 60) < a.n) {
        a.y[e0 + (lane - 60)] = v;
    }
}

template <typename WT, int TT, int EPW>
int launch_dense(const DenseArgs& a, hipStream_t stream) {
    const uint32_t C = a.k / 32u;
    const size_t lds = static_cast<size_t>(TT) * C * kXPitch * sizeof(float);
    const uint32_t per_wg = kWaves * EPW;
    const dim3 grid((a.m + TT - 1) / TT, (a.n + per_wg - 1) / per_wg);
    if (lds > 64u * 1024u) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_dense_gemv<WT, TT, EPW>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 static_cast<int>(lds));
        if (e != hipSuccess) {
            return mh::hip_error(e, "k_dense_gemv: LDS attribute");
        }
    }
    hipLaunchKernelGGL((k_dense_gemv<WT, TT, EPW>), grid, dim3(kThreads), lds, stream, a);
    return mh::launch_status("k_dense_gemv");
}

template <typename WT>
int dispatch_dense(const DenseArgs& a, hipStream_t stream) {
    if (a.m == 1) {
        return launch_dense<WT, 1, 1>(a, stream);
    }
    if (a.k <= 2048u && a.done == nullptr) {
        return launch_router_tiles<WT>(a, stream);
    }
    return launch_dense<WT, 8, 4>(a, stream);
}

int dense_common(const char* op, const void* w, bool w_f32, const uint16_t* x, float* y,
                 uint32_t m, uint32_t n, uint32_t k, DenseArgs& a) {
    MH_ENSURE(w && x && y, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(m > 0 && n > 0 && k > 0, MH_ERR_INVALID, "%s: empty shape m=%u n=%u k=%u", op, m, n, k);
    MH_ENSURE(k % 32 == 0, MH_ERR_UNSUPPORTED, "%s: K=%u is not a multiple of 32", op, k);
    MH_ENSURE(static_cast<size_t>(8) * (k / 32) * kXPitch * 4 <= 160u * 1024u, MH_ERR_UNSUPPORTED,
              "%s: K=%u too large for the LDS tile", op, k);
    MH_ENSURE(mh::aligned(w, 16) && mh::aligned(x, 4) && mh::aligned(y, 4), MH_ERR_ALIGN,
              "%s: W must be 16-byte aligned, x and y 4-byte aligned", op);
    (void)w_f32;
    a = DenseArgs{};
    a.w = w;
    a.x = x;
    a.y = y;
    a.m = m;
    a.n = n;
    a.k = k;
    return MH_OK;
}

// ------------------------------------------------------------ top-k route ---

__global__ __launch_bounds__(64) void k_route(const float* logits, const float* bias,
                                              uint32_t* ids, uint16_t* w, uint32_t e,
                                              uint32_t topk, int mode, float eps) {
    __shared__ float s[mh::kMaxExperts], cand[mh::kMaxExperts];
    const uint32_t t = blockIdx.x;
    for (uint32_t i = threadIdx.x; i < e; i += 64) {
        mh::route_score(logits[static_cast<size_t>(t) * e + i], bias ? bias[i] : 0.0f, mode, s[i],
                        cand[i]);
    }
    __syncthreads();
    mh::route_select(s, cand, e, topk, mode, eps, ids + static_cast<size_t>(t) * topk,
                     w + static_cast<size_t>(t) * topk);
}

int route_checks(const char* op, const float* logits, uint32_t* ids, uint16_t* w, uint32_t m,
                 uint32_t e, uint32_t topk, int mode) {
    MH_ENSURE(logits && ids && w, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(m > 0, MH_ERR_INVALID, "%s: no tokens", op);
    MH_ENSURE(e >= 1 && e <= static_cast<uint32_t>(mh::kMaxExperts), MH_ERR_UNSUPPORTED,
              "%s: %u experts (1..%d supported)", op, e, mh::kMaxExperts);
    MH_ENSURE(topk >= 1 && topk <= e && topk <= static_cast<uint32_t>(mh::kMaxTopk),
              MH_ERR_INVALID, "%s: topk %u not in 1..min(%u, %d)", op, topk, e, mh::kMaxTopk);
    MH_ENSURE(mode == MH_ROUTE_SIGMOID_BIAS || mode == MH_ROUTE_SOFTMAX, MH_ERR_INVALID,
              "%s: unknown routing mode %d", op, mode);
    return MH_OK;
}

// --------------------------------------------------- expert gate/up act ---

struct ActArgs {
    const uint32_t* gc; const uint16_t* gsc; const uint16_t* gbi;
    const uint32_t* uc; const uint16_t* usc; const uint16_t* ubi;
    const uint16_t* x;
    const uint32_t* ids;  // [slots] or null (dense)
    uint16_t* act;        // [slots, n_inter]
    uint32_t slots, n_inter, n_experts, k, gs, row_words, groups;
    // in-kernel routing (decode step): when logits != null every workgroup
    // routes the token itself from the logits, and workgroup 0 stores the
    // ids and weights for the down kernel (ids above is then the output)
    const float* logits;
    const float* bias;
    uint16_t* weights;
    int mode;
    float eps;
};

struct ActLoad {
    mh::Chunk<4> g, u;
    float gs, gb, us, ub;
};

__device__ __forceinline__ void load_act_row(const ActArgs& a, uint32_t v, int lane, bool live,
                                             ActLoad& o) {
    const uint32_t vv = min(v, a.slots * a.n_inter - 1);
    const uint32_t slot = vv / a.n_inter, j = vv % a.n_inter;
    uint32_t e = a.ids ? a.ids[slot] : 0u;
    e = e < a.n_experts ? e : 0u;  // an out-of-range id reads expert 0, never past W
    const size_t row = static_cast<size_t>(e) * a.n_inter + j;
    if (live) {
        o.g.load(a.gc + row * a.row_words + 4u * lane);
        o.u.load(a.uc + row * a.row_words + 4u * lane);
        const uint32_t g = (32u * lane) / a.gs;
        o.gs = mh::bf16_to_f32(a.gsc[row * a.groups + g]);
        o.gb = mh::bf16_to_f32(a.gbi[row * a.groups + g]);
        o.us = mh::bf16_to_f32(a.usc[row * a.groups + g]);
        o.ub = mh::bf16_to_f32(a.ubi[row * a.groups + g]);
    } else {
        o.g.zero();
        o.u.zero();
        o.gs = o.gb = o.us = o.ub = 0.0f;
    }
}

// x (K <= 2048) in registers; each wave takes R virtual rows (slot, j) at a
// time, both matrices, with the next group's loads in flight.
template <int R>
__device__ __forceinline__ void gather_act_rows(const ActArgs& a, const float (&xr)[32], float xs,
                                                int lane, int wave, bool live) {
    const uint32_t rows = a.slots * a.n_inter;
    const uint32_t n_rg = (rows + R - 1) / R;
    const uint32_t stride = gridDim.x * kWaves;
    uint32_t rg = blockIdx.x * kWaves + wave;
    ActLoad cur[R];
    if (rg < n_rg) {
#pragma unroll
        for (int r = 0; r < R; ++r) load_act_row(a, rg * R + r, lane, live, cur[r]);
    }
    while (rg < n_rg) {
        const uint32_t next = rg + stride;
        ActLoad nxt[R];
        if (next < n_rg) {
#pragma unroll
            for (int r = 0; r < R; ++r) load_act_row(a, next * R + r, lane, live, nxt[r]);
        }
        uint16_t mine = 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float pg = cur[r].g.dot(xr);
            const float pu = cur[r].u.dot(xr);
            const float hg = __builtin_fmaf(cur[r].gs, pg, cur[r].gb * xs);
            const float hu = __builtin_fmaf(cur[r].us, pu, cur[r].ub * xs);
            const float gsum = mh::lane63(mh::wave_sum_lane63(live ? 0.0f + hg : 0.0f));
            const float usum = mh::lane63(mh::wave_sum_lane63(live ? 0.0f + hu : 0.0f));
            const float g = mh::round_bf16(gsum);
            const float u = mh::round_bf16(usum);
            const uint16_t v = mh::f32_to_bf16(mh::silu_bf16(g) * u);
            if (lane == r) {
                mine = v;
            }
        }
        const uint32_t my = rg * R + lane;
        if (lane < R && my < rows) {
            a.act[my] = mine;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) cur[r] = nxt[r];
        rg = next;
    }
}

template <int R>
__global__ __launch_bounds__(kThreads) void k_gather_act(ActArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t C = a.k / 32u;
    const bool live = lane < static_cast<int>(C);
    float xr[32];
    float xs;
    mh::load_x_chunk(a.x + 32u * (live ? lane : 0), xr, xs);
    mh::q4_scale_x(xr);
    gather_act_rows<R>(a, xr, xs, lane, wave, live);
}

// Block form of the expert gate/up + SwiGLU (K <= 2048 and n_inter a
// multiple of 4): each wave owns 4 consecutive rows j of one slot, i.e. 4
// consecutive rows of expert ids[slot] in both matrices.  The 8 rows' codes
// are loaded at once (non-temporal), their scales and biases staged in LDS as
// (scale | bias << 16) words, each matrix's 4 row values reduced with the
// 4-row butterfly, and lanes 0..3 apply SwiGLU and store 4 consecutive
// activations.  Chunk order as in k_gather_act.
constexpr int kActBlock = 4;
constexpr int kMaxG = 64;  // groups per row (K / group size) staged in LDS

__device__ __forceinline__ void stage_sb_words(uint32_t* sb, const uint16_t* scales,
                                               const uint16_t* biases, uint32_t elems, int lane) {
    // elems bf16 of scales and of biases, contiguous; even G keeps them dword aligned
    const uint32_t* s2 = reinterpret_cast<const uint32_t*>(scales);
    const uint32_t* b2 = reinterpret_cast<const uint32_t*>(biases);
    for (uint32_t i = lane; i < elems / 2u; i += 64u) {
        const uint32_t sw = s2[i], bw = b2[i];
        *reinterpret_cast<uint2*>(sb + 2u * i) =
            make_uint2(__builtin_amdgcn_perm(bw, sw, 0x05040100u), __builtin_amdgcn_perm(bw, sw, 0x07060302u));
    }
}

__global__ __launch_bounds__(kThreads) void k_act_blocks(ActArgs a) {
    constexpr int R = kActBlock;  // rows per matrix per wave (one 4-row butterfly each)
    __shared__ uint32_t sbl[kWaves][2][R * kMaxG];
    __shared__ float rs[mh::kMaxExperts], rc[mh::kMaxExperts];
    __shared__ uint32_t rids[mh::kMaxTopk];
    __shared__ uint16_t rw[mh::kMaxTopk];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t C = a.k / 32u;
    const bool live = lane < static_cast<int>(C);
    const uint32_t c = live ? lane : 0u;
    const uint32_t G = a.groups;
    uint32_t xw[16];
    mh::load_x_words(a.x + 32u * c, xw);
    if (a.logits != nullptr) {
        if (wave == 0) {
            for (uint32_t i = lane; i < a.n_experts; i += 64) {
                mh::route_score(a.logits[i], a.bias ? a.bias[i] : 0.0f, a.mode, rs[i], rc[i]);
            }
            mh::route_select(rs, rc, a.n_experts, a.slots, a.mode, a.eps, rids, rw);
            if (blockIdx.x == 0 && lane < static_cast<int>(a.slots)) {
                const_cast<uint32_t*>(a.ids)[lane] = rids[lane];
                a.weights[lane] = rw[lane];
            }
        }
        __syncthreads();
    }
    const uint32_t blk = blockIdx.x * kWaves + wave;
    const uint32_t v0 = blk * R;
    if (v0 >= a.slots * a.n_inter) {
        return;
    }
    const uint32_t slot = v0 / a.n_inter, j0 = v0 % a.n_inter;
    uint32_t e = a.logits != nullptr ? rids[slot] : (a.ids ? a.ids[slot] : 0u);
    e = e < a.n_experts ? e : 0u;  // an out-of-range id reads expert 0, never past W
    const uint32_t row0 = e * a.n_inter + j0;
    const uint32_t row_bytes = a.row_words * 4u;
    const mh::gbytes gbase = mh::uniform_ptr(reinterpret_cast<const char*>(a.gc) + static_cast<size_t>(row0) * row_bytes);
    const mh::gbytes ubase = mh::uniform_ptr(reinterpret_cast<const char*>(a.uc) + static_cast<size_t>(row0) * row_bytes);
    const uint32_t code_off = c * 16u;
    mh::Chunk<4> ch[2][R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        ch[0][r].load_nt(gbase, r * row_bytes + code_off);
        ch[1][r].load_nt(ubase, r * row_bytes + code_off);
    }
    stage_sb_words(sbl[wave][0], a.gsc + static_cast<size_t>(row0) * G, a.gbi + static_cast<size_t>(row0) * G,
                   R * G, lane);
    stage_sb_words(sbl[wave][1], a.usc + static_cast<size_t>(row0) * G, a.ubi + static_cast<size_t>(row0) * G,
                   R * G, lane);
    mh::x_words_fence(xw);
    float xr[32], xs;
    mh::x_words_to_f32(xw, xr, xs);
    mh::q4_scale_x(xr);
    const uint32_t gc = (32u * c) / a.gs;
    float yv[2];
#pragma unroll
    for (int mat = 0; mat < 2; ++mat) {
        float h[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t w = sbl[wave][mat][r * G + gc];
            const float p = ch[mat][r].dot(xr);
            const float hv = __builtin_fmaf(__uint_as_float(w << 16), p, __uint_as_float(w & 0xffff0000u) * xs);
            h[r] = live ? 0.0f + hv : 0.0f;
        }
        const float v = mh::reduce_rows4(h, lane);
        yv[mat] = __int_as_float(__builtin_amdgcn_ds_bpermute((60 + (lane & 3)) * 4, __float_as_int(v)));
    }
    if (lane < R) {
        const float g = mh::round_bf16(yv[0]);
        const float u = mh::round_bf16(yv[1]);
        a.act[v0 + lane] = mh::f32_to_bf16(mh::silu_bf16(g) * u);
    }
}

int launch_gather_act(const ActArgs& a, hipStream_t stream) {
    if (a.n_inter % kActBlock == 0 && a.groups % 2 == 0 && a.groups <= static_cast<uint32_t>(kMaxG) &&
        a.gs % 32 == 0) {
        const uint32_t blocks = a.slots * a.n_inter / kActBlock;
        hipLaunchKernelGGL(k_act_blocks, dim3((blocks + kWaves - 1) / kWaves), dim3(kThreads), 0, stream, a);
        return mh::launch_status("k_act_blocks");
    }
    constexpr int R = 2;
    const uint32_t n_rg = (a.slots * a.n_inter + R - 1) / R;
    const uint32_t want = (n_rg + kWaves - 1) / kWaves;
    const uint32_t cap = static_cast<uint32_t>(mh::cu_count()) * 4u;
    hipLaunchKernelGGL(k_gather_act<R>, dim3(want < cap ? want : cap), dim3(kThreads), 0, stream, a);
    return mh::launch_status("k_gather_act");
}

int act_common(const char* op, const mh_quant_weights* gate, const mh_quant_weights* up,
               const uint16_t* x, const uint32_t* ids, uint16_t* act, uint32_t slots,
               uint32_t n_inter, ActArgs& a) {
    MH_TRY(mh::check_quant(gate, op));
    MH_TRY(mh::check_quant(up, op));
    MH_ENSURE(x && act, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(gate->bits == 4 && up->bits == 4, MH_ERR_UNSUPPORTED, "%s: expert GEMVs are 4-bit", op);
    MH_ENSURE(gate->out_features == up->out_features && gate->in_features == up->in_features &&
                  gate->group_size == up->group_size,
              MH_ERR_INVALID, "%s: gate/up shapes differ", op);
    MH_ENSURE(gate->in_features <= 2048, MH_ERR_UNSUPPORTED,
              "%s: in_features %u > 2048 (x is held in registers)", op, gate->in_features);
    MH_ENSURE(n_inter > 0 && gate->out_features % n_inter == 0, MH_ERR_INVALID,
              "%s: %u stacked rows are not a multiple of n_inter %u", op, gate->out_features, n_inter);
    MH_ENSURE(slots >= 1 && slots <= static_cast<uint32_t>(mh::kMaxTopk), MH_ERR_INVALID,
              "%s: %u slots not in 1..%d", op, slots, mh::kMaxTopk);
    MH_ENSURE(mh::aligned(x, 2) && mh::aligned(act, 2), MH_ERR_ALIGN, "%s: x/act alignment", op);
    a = ActArgs{};
    a.gc = gate->codes; a.gsc = gate->scales; a.gbi = gate->biases;
    a.uc = up->codes; a.usc = up->scales; a.ubi = up->biases;
    a.x = x;
    a.ids = ids;
    a.act = act;
    a.slots = slots;
    a.n_inter = n_inter;
    a.n_experts = gate->out_features / n_inter;
    a.k = gate->in_features;
    a.gs = gate->group_size;
    a.row_words = gate->in_features / 8u;
    a.groups = gate->in_features / gate->group_size;
    return MH_OK;
}

// --------------------------------------------------- expert down+combine ---

struct DownArgs {
    const uint32_t* codes; const uint16_t* scales; const uint16_t* biases;
    const uint16_t* act;      // bf16 [topk, k]
    const uint32_t* ids;      // [topk]
    const uint16_t* weights;  // bf16 [topk]
    uint16_t* out;            // bf16 [n_out]
    uint32_t n_out, n_experts, k, gs, row_words, groups;
};

template <int TK>
__device__ __forceinline__ void down_rows(const DownArgs& a, const float (&xr)[TK][32],
                                          const float (&xs)[TK], const uint32_t (&e)[TK],
                                          const float (&wt)[TK], int lane, int wave, bool live) {
    auto load = [&](uint32_t i, mh::Chunk<4>(&ch)[TK], float(&s)[TK], float(&b)[TK]) {
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            const size_t row = static_cast<size_t>(e[r]) * a.n_out + min(i, a.n_out - 1);
            if (live) {
                ch[r].load(a.codes + row * a.row_words + 4u * lane);
                const uint32_t g = (32u * lane) / a.gs;
                s[r] = mh::bf16_to_f32(a.scales[row * a.groups + g]);
                b[r] = mh::bf16_to_f32(a.biases[row * a.groups + g]);
            } else {
                ch[r].zero();
                s[r] = b[r] = 0.0f;
            }
        }
    };
    const uint32_t stride = gridDim.x * kWaves;
    uint32_t i = blockIdx.x * kWaves + wave;
    mh::Chunk<4> cur[TK];
    float cs[TK], cb[TK];
    if (i < a.n_out) load(i, cur, cs, cb);
    while (i < a.n_out) {
        const uint32_t next = i + stride;
        mh::Chunk<4> nxt[TK];
        float ns[TK], nb[TK];
        if (next < a.n_out) load(next, nxt, ns, nb);
        float total = 0.0f;
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            const float p = cur[r].dot(xr[r]);
            const float h = __builtin_fmaf(cs[r], p, cb[r] * xs[r]);
            const float v = mh::round_bf16(mh::lane63(mh::wave_sum_lane63(live ? 0.0f + h : 0.0f)));
            total = total + mh::round_bf16(wt[r] * v);
        }
        if (lane == 0) {
            a.out[i] = mh::f32_to_bf16(total);
        }
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            cur[r] = nxt[r];
            cs[r] = ns[r];
            cb[r] = nb[r];
        }
        i = next;
    }
}

template <int TK>
__global__ __launch_bounds__(kThreads) void k_down_combine(DownArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t C = a.k / 32u;
    const bool live = lane < static_cast<int>(C);
    float xr[TK][32];
    float xs[TK];
    uint32_t e[TK];
    float wt[TK];
#pragma unroll
    for (int r = 0; r < TK; ++r) {
        mh::load_x_chunk(a.act + static_cast<size_t>(r) * a.k + 32u * (live ? lane : 0), xr[r], xs[r]);
        mh::q4_scale_x(xr[r]);
        const uint32_t id = a.ids[r];
        e[r] = id < a.n_experts ? id : 0u;
        wt[r] = mh::bf16_to_f32(a.weights[r]);
    }
    down_rows<TK>(a, xr, xs, e, wt, lane, wave, live);
}

// Block form of the expert down + combine (K <= 2048, topk <= 4, n_out
// even): each wave owns 2 consecutive outputs i; the activation rows of the
// topk slots are in registers (lane c holds chunk c of each), output i's
// topk row values are reduced together in one 4-row butterfly (slot r as row
// r), and the combine bf16(sum_r bf16(w_r * bf16(v_r))) runs on the reduced
// values.  Chunk order as in k_down_combine.
constexpr int kDownOut = 2;

template <int TK>
__global__ __launch_bounds__(kThreads) void k_down_blocks(DownArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t C = a.k / 32u;
    const bool live = lane < static_cast<int>(C);
    const uint32_t c = live ? lane : 0u;
    const uint32_t G = a.groups;
    const uint32_t i0 = (blockIdx.x * kWaves + wave) * kDownOut;
    if (i0 >= a.n_out) {
        return;
    }
    uint32_t e[TK];
    float wt[TK];
#pragma unroll
    for (int r = 0; r < TK; ++r) {
        const uint32_t id = a.ids[r];
        e[r] = id < a.n_experts ? id : 0u;
        wt[r] = mh::bf16_to_f32(a.weights[r]);
    }
    uint32_t xw[TK][16];
#pragma unroll
    for (int r = 0; r < TK; ++r) {
        mh::load_x_words(a.act + static_cast<size_t>(r) * a.k + 32u * c, xw[r]);
    }
    const uint32_t row_bytes = a.row_words * 4u;
    const uint32_t code_off = c * 16u;
    const uint32_t gc = (32u * c) / a.gs;
    mh::Chunk<4> ch[kDownOut][TK];
    uint16_t sr[kDownOut][TK], br[kDownOut][TK];
#pragma unroll
    for (int o = 0; o < kDownOut; ++o) {
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            const size_t row = static_cast<size_t>(e[r]) * a.n_out + i0 + o;
            ch[o][r].load_nt(mh::uniform_ptr(reinterpret_cast<const char*>(a.codes) + row * row_bytes), code_off);
            sr[o][r] = a.scales[row * G + gc];
            br[o][r] = a.biases[row * G + gc];
        }
    }
    float xr[TK][32], xs[TK];
#pragma unroll
    for (int r = 0; r < TK; ++r) {
        mh::x_words_fence(xw[r]);
        mh::x_words_to_f32(xw[r], xr[r], xs[r]);
        mh::q4_scale_x(xr[r]);
    }
    float yv = 0.0f;
#pragma unroll
    for (int o = 0; o < kDownOut; ++o) {
        float h[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            const float p = ch[o][r].dot(xr[r]);
            const float hv = __builtin_fmaf(mh::bf16_to_f32(sr[o][r]), p, mh::bf16_to_f32(br[o][r]) * xs[r]);
            h[r] = live ? 0.0f + hv : 0.0f;
        }
        const float v = mh::reduce_rows4(h, lane);
        float total = 0.0f;
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            const float vr = mh::round_bf16(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 60 + r)));
            total = total + mh::round_bf16(wt[r] * vr);
        }
        if (lane == o) {
            yv = total;
        }
    }
    if (lane < kDownOut && i0 + lane < a.n_out) {
        a.out[i0 + lane] = mh::f32_to_bf16(yv);
    }
}

int launch_down(const DownArgs& a, uint32_t topk, hipStream_t stream) {
    if (a.n_out % kDownOut == 0 && a.gs % 32 == 0) {
        const dim3 grid((a.n_out / kDownOut + kWaves - 1) / kWaves);
        switch (topk) {
            case 1: hipLaunchKernelGGL(k_down_blocks<1>, grid, dim3(kThreads), 0, stream, a); break;
            case 2: hipLaunchKernelGGL(k_down_blocks<2>, grid, dim3(kThreads), 0, stream, a); break;
            case 3: hipLaunchKernelGGL(k_down_blocks<3>, grid, dim3(kThreads), 0, stream, a); break;
            case 4: hipLaunchKernelGGL(k_down_blocks<4>, grid, dim3(kThreads), 0, stream, a); break;
            default: return mh::set_error(MH_ERR_UNSUPPORTED, "down combine: topk %u not in 1..4", topk);
        }
        return mh::launch_status("k_down_blocks");
    }
    const uint32_t want = (a.n_out + kWaves - 1) / kWaves;
    const uint32_t cap = static_cast<uint32_t>(mh::cu_count()) * 4u;
    const dim3 grid(want < cap ? want : cap);
    switch (topk) {
        case 1: hipLaunchKernelGGL(k_down_combine<1>, grid, dim3(kThreads), 0, stream, a); break;
        case 2: hipLaunchKernelGGL(k_down_combine<2>, grid, dim3(kThreads), 0, stream, a); break;
        case 3: hipLaunchKernelGGL(k_down_combine<3>, grid, dim3(kThreads), 0, stream, a); break;
        case 4: hipLaunchKernelGGL(k_down_combine<4>, grid, dim3(kThreads), 0, stream, a); break;
        default: return mh::set_error(MH_ERR_UNSUPPORTED, "down combine: topk %u not in 1..4", topk);
    }
    return mh::launch_status("k_down_combine");
}

int down_common(const char* op, const mh_quant_weights* down, const uint16_t* act,
                const uint32_t* ids, const uint16_t* weights, uint16_t* out, uint32_t topk,
                uint32_t n_out, DownArgs& a) {
    MH_TRY(mh::check_quant(down, op));
    MH_ENSURE(act && ids && weights && out, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(down->bits == 4, MH_ERR_UNSUPPORTED, "%s: expert GEMVs are 4-bit", op);
    MH_ENSURE(topk >= 1 && topk <= 4, MH_ERR_UNSUPPORTED, "%s: topk %u not in 1..4", op, topk);
    MH_ENSURE(down->in_features <= 2048, MH_ERR_UNSUPPORTED,
              "%s: in_features %u > 2048 (act is held in registers)", op, down->in_features);
    MH_ENSURE(n_out > 0 && down->out_features % n_out == 0, MH_ERR_INVALID,
              "%s: %u stacked rows are not a multiple of n_out %u", op, down->out_features, n_out);
    MH_ENSURE(mh::aligned(act, 2) && mh::aligned(out, 2), MH_ERR_ALIGN, "%s: alignment", op);
    a = DownArgs{};
    a.codes = down->codes; a.scales = down->scales; a.biases = down->biases;
    a.act = act;
    a.ids = ids;
    a.weights = weights;
    a.out = out;
    a.n_out = n_out;
    a.n_experts = down->out_features / n_out;
    a.k = down->in_features;
    a.gs = down->group_size;
    a.row_words = down->in_features / 8u;
    a.groups = down->in_features / down->group_size;
    return MH_OK;
}

}  // namespace

extern "C" {

int mh_gemv_f32(const float* w, const uint16_t* x, float* y, uint32_t n, uint32_t k,
                mh_stream_t stream) {
    DenseArgs a;
    MH_TRY(dense_common("mh_gemv_f32", w, true, x, y, 1, n, k, a));
    return dispatch_dense<float>(a, mh::as_stream(stream));
}

int mh_gemv_bf16(const uint16_t* w, const uint16_t* x, float* y, uint32_t n, uint32_t k,
                 mh_stream_t stream) {
    DenseArgs a;
    MH_TRY(dense_common("mh_gemv_bf16", w, false, x, y, 1, n, k, a));
    return dispatch_dense<uint16_t>(a, mh::as_stream(stream));
}

int mh_router_prefill(const uint16_t* x, const void* w, int w_dtype, float* out, uint32_t m,
                      uint32_t k, uint32_t e, mh_stream_t stream) {
    MH_ENSURE(w_dtype == MH_DTYPE_F32 || w_dtype == MH_DTYPE_BF16, MH_ERR_INVALID,
              "mh_router_prefill: router dtype %d", w_dtype);
    DenseArgs a;
    MH_TRY(dense_common("mh_router_prefill", w, w_dtype == MH_DTYPE_F32, x, out, m, e, k, a));
    return w_dtype == MH_DTYPE_F32 ? dispatch_dense<float>(a, mh::as_stream(stream))
                                   : dispatch_dense<uint16_t>(a, mh::as_stream(stream));
}

int mh_route_token(const float* logits, const float* bias, uint32_t* ids, uint16_t* weights,
                   uint32_t e, uint32_t topk, int mode, float eps, mh_stream_t stream) {
    MH_TRY(route_checks("mh_route_token", logits, ids, weights, 1, e, topk, mode));
    hipLaunchKernelGGL(k_route, dim3(1), dim3(64), 0, mh::as_stream(stream), logits, bias, ids,
                       weights, e, topk, mode, eps);
    return mh::launch_status("mh_route_token");
}

}  // extern "C"

namespace mh {

// Prefill router logits (mh_moe_prefill's first step; the routing follows).
int router_prefill_logits(const uint16_t* x, const void* w, int w_dtype, float* logits, uint32_t m,
                          uint32_t k, uint32_t e, mh_stream_t stream) {
    const char* op = "mh_moe_prefill (router)";
    MH_ENSURE(w_dtype == MH_DTYPE_F32 || w_dtype == MH_DTYPE_BF16, MH_ERR_INVALID,
              "%s: router dtype %d", op, w_dtype);
    DenseArgs a;
    MH_TRY(dense_common(op, w, w_dtype == MH_DTYPE_F32, x, logits, m, e, k, a));
    return w_dtype == MH_DTYPE_F32 ? dispatch_dense<float>(a, mh::as_stream(stream))
                                   : dispatch_dense<uint16_t>(a, mh::as_stream(stream));
}

}  // namespace mh

extern "C" {

int mh_moe_route_batch(const float* logits, const float* bias, uint32_t* ids, uint16_t* gw,
                       uint32_t m, uint32_t e, uint32_t topk, int mode, float eps,
                       mh_stream_t stream) {
    MH_TRY(route_checks("mh_moe_route_batch", logits, ids, gw, m, e, topk, mode));
    hipLaunchKernelGGL(k_route, dim3(m), dim3(64), 0, mh::as_stream(stream), logits, bias, ids, gw,
                       e, topk, mode, eps);
    return mh::launch_status("mh_moe_route_batch");
}

int mh_router_route(const void* w, int w_dtype, const uint16_t* x, float* logits,
                    const float* bias, uint32_t* ids, uint16_t* weights, uint32_t* counter,
                    uint32_t e, uint32_t k, uint32_t topk, int mode, float eps,
                    mh_stream_t stream) {
    MH_ENSURE(w_dtype == MH_DTYPE_F32 || w_dtype == MH_DTYPE_BF16, MH_ERR_INVALID,
              "mh_router_route: router dtype %d", w_dtype);
    MH_ENSURE(counter != nullptr, MH_ERR_INVALID, "mh_router_route: counter is NULL");
    MH_TRY(route_checks("mh_router_route", logits, ids, weights, 1, e, topk, mode));
    DenseArgs a;
    MH_TRY(dense_common("mh_router_route", w, w_dtype == MH_DTYPE_F32, x, logits, 1, e, k, a));
    a.bias = bias;
    a.ids = ids;
    a.weights = weights;
    a.done = counter;
    a.topk = topk;
    a.mode = mode;
    a.eps = eps;
    return w_dtype == MH_DTYPE_F32 ? launch_dense<float, 1, 1>(a, mh::as_stream(stream))
                                   : launch_dense<uint16_t, 1, 1>(a, mh::as_stream(stream));
}

int mh_gemv_gather_act(const mh_quant_weights* gate, const mh_quant_weights* up,
                       const uint16_t* x, const uint32_t* ids, uint16_t* act, uint32_t topk,
                       uint32_t n_inter, mh_stream_t stream) {
    MH_ENSURE(ids != nullptr, MH_ERR_INVALID, "mh_gemv_gather_act: ids is NULL");
    ActArgs a;
    MH_TRY(act_common("mh_gemv_gather_act", gate, up, x, ids, act, topk, n_inter, a));
    return launch_gather_act(a, mh::as_stream(stream));
}

int mh_gemv_gu_act(const mh_quant_weights* gate, const mh_quant_weights* up, const uint16_t* x,
                   uint16_t* act, mh_stream_t stream) {
    MH_ENSURE(gate != nullptr, MH_ERR_INVALID, "mh_gemv_gu_act: gate is NULL");
    ActArgs a;
    MH_TRY(act_common("mh_gemv_gu_act", gate, up, x, nullptr, act, 1, gate->out_features, a));
    return launch_gather_act(a, mh::as_stream(stream));
}

int mh_gemv_gather_down_combine(const mh_quant_weights* down, const uint16_t* act,
                                const uint32_t* ids, const uint16_t* weights, uint16_t* out,
                                uint32_t topk, uint32_t n_out, mh_stream_t stream) {
    DownArgs a;
    MH_TRY(down_common("mh_gemv_gather_down_combine", down, act, ids, weights, out, topk, n_out, a));
    return launch_down(a, topk, mh::as_stream(stream));
}

int mh_moe_decode(const void* router, int router_dtype, const float* bias, int mode, float eps,
                  const mh_quant_weights* gate, const mh_quant_weights* up,
                  const mh_quant_weights* down, uint32_t n_experts, uint32_t topk,
                  const uint16_t* x, uint16_t* out, float* logits, uint32_t* ids,
                  uint16_t* weights, uint16_t* act, uint32_t* scratch, mh_stream_t stream) {
    const char* op = "mh_moe_decode";
    MH_ENSURE(gate && up && down, MH_ERR_INVALID, "%s: NULL weights", op);
    MH_ENSURE(n_experts > 0 && gate->out_features % n_experts == 0 &&
                  down->out_features % n_experts == 0,
              MH_ERR_INVALID, "%s: stacked rows not divisible by %u experts", op, n_experts);
    const uint32_t n_inter = gate->out_features / n_experts;
    const uint32_t d_model = down->out_features / n_experts;
    MH_ENSURE(gate->in_features == d_model && down->in_features == n_inter, MH_ERR_INVALID,
              "%s: gate [%u x %u] / down [%u x %u] do not chain", op, n_inter, gate->in_features,
              d_model, down->in_features);
    // validate all three stages before launching any of them
    DenseArgs ra;
    MH_ENSURE(router_dtype == MH_DTYPE_F32 || router_dtype == MH_DTYPE_BF16, MH_ERR_INVALID,
              "%s: router dtype %d", op, router_dtype);
    MH_ENSURE(scratch != nullptr, MH_ERR_INVALID, "%s: scratch is NULL", op);
    MH_TRY(route_checks(op, logits, ids, weights, 1, n_experts, topk, mode));
    MH_TRY(dense_common(op, router, router_dtype == MH_DTYPE_F32, x, logits, 1, n_experts, d_model, ra));
    ActArgs aa;
    MH_TRY(act_common(op, gate, up, x, ids, act, topk, n_inter, aa));
    DownArgs da;
    MH_TRY(down_common(op, down, act, ids, weights, out, topk, d_model, da));
    const hipStream_t s = mh::as_stream(stream);
    const int fused = mh::moe_decode_fused(router, router_dtype, bias, mode, eps, gate, up, down, n_experts,
                                           topk, x, out, logits, ids, weights, act, scratch, nullptr, s);
    if (fused != MH_ERR_UNSUPPORTED) {
        return fused;
    }
    if (d_model <= 2048u && n_inter % kActBlock == 0 && aa.groups % 2 == 0 &&
        aa.groups <= static_cast<uint32_t>(kMaxG) && d_model % kDownOut == 0) {
        // logits -> (routing inside every expert workgroup) -> down + combine
        const dim3 rg((n_experts + 3) / 4);
        if (router_dtype == MH_DTYPE_F32) {
            hipLaunchKernelGGL(k_router_logits<float>, rg, dim3(64), 0, s, ra);
        } else {
            hipLaunchKernelGGL(k_router_logits<uint16_t>, rg, dim3(64), 0, s, ra);
        }
        MH_TRY(mh::launch_status("k_router_logits"));
        aa.logits = logits;
        aa.bias = bias;
        aa.weights = weights;
        aa.mode = mode;
        aa.eps = eps;
        MH_TRY(launch_gather_act(aa, s));
        return launch_down(da, topk, s);
    }
    ra.bias = bias;
    ra.ids = ids;
    ra.weights = weights;
    ra.done = scratch + 256;  // a word the single-launch kernel never uses
    ra.topk = topk;
    ra.mode = mode;
    ra.eps = eps;
    const int rc = router_dtype == MH_DTYPE_F32 ? launch_dense<float, 1, 1>(ra, s)
                                                : launch_dense<uint16_t, 1, 1>(ra, s);
    MH_TRY(rc);
    MH_TRY(launch_gather_act(aa, s));
    return launch_down(da, topk, s);
}

int mh_moe_decode_stamped(const void* router, int router_dtype, const float* bias, int mode, float eps,
                          const mh_quant_weights* gate, const mh_quant_weights* up, const mh_quant_weights* down,
                          uint32_t n_experts, uint32_t topk, const uint16_t* x, uint16_t* out, float* logits,
                          uint32_t* ids, uint16_t* weights, uint16_t* act, uint32_t* scratch, uint64_t* stamps,
                          mh_stream_t stream) {
    const char* op = "mh_moe_decode_stamped";
    MH_ENSURE(stamps != nullptr && mh::aligned(stamps, 8), MH_ERR_INVALID, "%s: stamps NULL or not 8-byte aligned",
              op);
    MH_ENSURE(gate && up && down && scratch, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(n_experts > 0 && gate->out_features % n_experts == 0 && down->out_features % n_experts == 0,
              MH_ERR_INVALID, "%s: stacked rows not divisible by %u experts", op, n_experts);
    const uint32_t n_inter = gate->out_features / n_experts;
    const uint32_t d_model = down->out_features / n_experts;
    MH_ENSURE(gate->in_features == d_model && down->in_features == n_inter, MH_ERR_INVALID,
              "%s: gate / down do not chain", op);
    DenseArgs ra;
    MH_TRY(route_checks(op, logits, ids, weights, 1, n_experts, topk, mode));
    MH_TRY(dense_common(op, router, router_dtype == MH_DTYPE_F32, x, logits, 1, n_experts, d_model, ra));
    ActArgs aa;
    MH_TRY(act_common(op, gate, up, x, ids, act, topk, n_inter, aa));
    DownArgs da;
    MH_TRY(down_common(op, down, act, ids, weights, out, topk, d_model, da));
    const int rc = mh::moe_decode_fused(router, router_dtype, bias, mode, eps, gate, up, down, n_experts, topk, x,
                                        out, logits, ids, weights, act, scratch, stamps, mh::as_stream(stream));
    MH_ENSURE(rc != MH_ERR_UNSUPPORTED, MH_ERR_UNSUPPORTED, "%s: the shape runs as three launches (no timeline)", op);
    return rc;
}

}  // extern "C"

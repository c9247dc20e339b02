// sample.hip -- the temperature-only Gumbel draw over stored bf16 logits
// (lfm_sample.metal:157-190 lfm_sample_gumbel;
// src/lfm/sample.rs:264-285 encode_draw with neither top-k nor top-p): the
// sampled token is the argmax of w_i + G_i, w_i = pen(v_i) / T (the seen set's
// repetition penalty, -0 folded to +0), G_i a Gumbel(0, 1) variate from
// Philox4x32-10 with key = seed and counter = (i / 4, pos, "SAMP", 0), word
// i % 4.  The result is folded into the greedy head's 64-bit key word, which
// mh_token_tail reads and clears.  logf is this library's own (mh_device.hpp),
// so the draw is reproducible bit for bit by the CPU restatement.
#include "mh_device.hpp"
#include "mh_host.hpp"

namespace {

constexpr int kThreads = 256;  // 4 tokens per thread, 1024 per workgroup
constexpr uint32_t kDomain = 0x53414D50u;  // "SAMP", Philox counter word 2

__device__ __forceinline__ float processed(float v, bool seen, const mh_sample_params& p) {
    if (seen) {
        v = v > 0.0f ? v * p.inv_penalty : v * p.penalty;
    }
    uint32_t u = __float_as_uint(v * p.inv_temp);
    if ((u << 1) == 0u) {
        u = 0u;
    }
    return __uint_as_float(u);
}

__global__ __launch_bounds__(kThreads) void k_sample_gumbel(const uint16_t* logits, uint32_t n, const uint32_t* seen,
                                                            mh_sample_params p, unsigned long long* best) {
    __shared__ unsigned long long part[kThreads / 64];
    const uint32_t q = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t i0 = 4u * q;
    unsigned long long k = 0ull;
    if (i0 < n) {
        const uint2 raw = *reinterpret_cast<const uint2*>(logits + i0);
        const float v[4] = {mh::bf16lo(raw.x), mh::bf16hi(raw.x), mh::bf16lo(raw.y), mh::bf16hi(raw.y)};
        const uint32_t bits = p.use_penalty != 0u ? (seen[i0 >> 5] >> (i0 & 31u)) : 0u;
        const mh::u32x4 r = mh::philox4x32_10(mh::u32x4{q, p.pos, kDomain, 0u}, p.seed_lo, p.seed_hi);
        const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float w = processed(v[j], ((bits >> j) & 1u) != 0u, p) + mh::gumbel_of(rw[j]);
            const unsigned long long kj = mh::argmax_key(w, i0 + j);
            k = kj > k ? kj : k;
        }
    }
    k = mh::wave_max_u64(k);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        part[wave] = k;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < kThreads / 64; ++w) {
            k = part[w] > k ? part[w] : k;
        }
        // read first: most workgroups hold no key above the word's
        if (k > __hip_atomic_load(best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            __hip_atomic_fetch_max(best, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ----------------------------------------------------------------------------
// The kept-set draw (top-k and / or top-p; lfm_sample.metal:16-27 semantics,
// src/lfm/sample.rs:286-330): kept = {w >= tau}, tau the k-th largest w (ties
// kept), then, among the kept, the largest value t with mass(w >= t) >=
// top_p x mass(kept) (tie groups whole), each token's mass exp(w - M) in 2^-40
// fixed point (truncated) so that every mass sum is an exact integer and the
// decision does not depend on the order of any sum.  tau is found exactly by
// a radix select over the orderable 32-bit keys of w: three rounds of 11, 11
// and 10 bits, each round one launch in which every workgroup histograms its
// tokens' digits (counts and masses) in LDS and adds them to a global
// histogram, and the last workgroup to arrive picks the digit that holds the
// threshold and writes the next round's prefix (a count phase for top-k, then
// a mass phase for top-p restricted to the top-k set).  The draw then folds
// the Gumbel-max over {w >= tau} into the key word, as the temperature draw.
//
// Workspace (caller-owned, zeroed once, left zero by every call): w f32[n],
// the histogram, and the plan words.
constexpr uint32_t kBlock = 4u * kThreads;  // tokens per workgroup
constexpr int kDigits = 2048;               // 11-bit digits

struct SmpPlan {
    uint32_t max_key;     // orderable key of M (atomic max by the prep kernel)
    uint32_t arrive;      // workgroups done with the current launch
    uint32_t prefix;      // digits chosen so far in this phase
    uint32_t restrict_key;  // the mass phase's floor (tau_k, or 0)
    uint32_t tau_key;     // the final threshold's key (0: every token)
    uint32_t pad0;
    unsigned long long base;    // count / mass above the current band
    unsigned long long target;  // the phase's target (k, or the mass target)
};

struct SmpWs {
    float* w;
    uint32_t* hcnt;
    unsigned long long* hmass;
    SmpPlan* plan;
};

size_t smp_align(size_t b) { return (b + 255u) & ~static_cast<size_t>(255u); }

SmpWs smp_layout(void* ws, uint32_t n) {
    char* p = static_cast<char*>(ws);
    SmpWs l;
    l.w = reinterpret_cast<float*>(p);
    p += smp_align(static_cast<size_t>(n) * 4u);
    l.hcnt = reinterpret_cast<uint32_t*>(p);
    p += smp_align(kDigits * 4u);
    l.hmass = reinterpret_cast<unsigned long long*>(p);
    p += smp_align(kDigits * 8u);
    l.plan = reinterpret_cast<SmpPlan*>(p);
    return l;
}

size_t smp_bytes(uint32_t n) { return smp_align(static_cast<size_t>(n) * 4u) + smp_align(kDigits * 4u) +
                                      smp_align(kDigits * 8u) + smp_align(sizeof(SmpPlan)); }

__device__ __forceinline__ uint32_t smp_fkey(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u << 1) == 0u) {
        u = 0u;
    }
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float smp_kfloat(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// exp(w - m) in 2^-40 fixed point, truncated (w <= m: at most 2^40).
__device__ __forceinline__ unsigned long long smp_mass(float w, float m) {
    return static_cast<unsigned long long>(mh::expf_fixed(w - m) * 1099511627776.0f);
}

// The least integer >= top_p * z (top_p in (0, 1), exact).
__device__ unsigned long long smp_mass_target(unsigned long long z, float top_p) {
    const uint32_t u = __float_as_uint(top_p);
    const uint32_t ex = (u >> 23) & 0xffu;
    const unsigned long long mant = ex ? ((u & 0x7fffffu) | 0x800000u) : (u & 0x7fffffu);
    const int s = 150 - static_cast<int>(ex ? ex : 1u);
    const unsigned __int128 prod = static_cast<unsigned __int128>(mant) * z;
    if (s >= 128) {
        return prod != 0 ? 1ull : 0ull;
    }
    unsigned long long t = static_cast<unsigned long long>(prod >> s);
    if ((prod & ((static_cast<unsigned __int128>(1) << s) - 1)) != 0) {
        t += 1ull;
    }
    return t;
}

__device__ __forceinline__ uint32_t coherent_load(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long coherent_load(const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// w of every token and the vocabulary's max key.
__global__ __launch_bounds__(kThreads) void k_smp_prep(const uint16_t* logits, uint32_t n, const uint32_t* seen,
                                                       mh_sample_params p, SmpWs ws) {
    __shared__ uint32_t part[kThreads / 64];
    const uint32_t i0 = 4u * (blockIdx.x * kThreads + threadIdx.x);
    uint32_t kmax = 0u;
    if (i0 < n) {
        const uint2 raw = *reinterpret_cast<const uint2*>(logits + i0);
        const float v[4] = {mh::bf16lo(raw.x), mh::bf16hi(raw.x), mh::bf16lo(raw.y), mh::bf16hi(raw.y)};
        const uint32_t bits = p.use_penalty != 0u ? (seen[i0 >> 5] >> (i0 & 31u)) : 0u;
        float w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            w[j] = processed(v[j], ((bits >> j) & 1u) != 0u, p);
            kmax = max(kmax, smp_fkey(w[j]));
        }
        *reinterpret_cast<float4*>(ws.w + i0) = make_float4(w[0], w[1], w[2], w[3]);
    }
    kmax = mh::wave_max_u32(kmax);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        part[wave] = kmax;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < kThreads / 64; ++w) {
            kmax = max(kmax, part[w]);
        }
        __hip_atomic_fetch_max(&ws.plan->max_key, kmax, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// One radix round.  phase 0 counts (top-k), phase 1 masses (top-p); round r
// takes digit bits [shift, shift + width) of the keys in the current band
// (keys whose bits above shift + width equal the prefix, and >= the phase's
// floor).  final_round: the last round of the last phase.
__global__ __launch_bounds__(kThreads) void k_smp_round(uint32_t n, mh_sample_params p, SmpWs ws, int phase,
                                                        int round, int final_round) {
    __shared__ uint32_t lcnt[kDigits];
    __shared__ unsigned long long lmass[kDigits];
    __shared__ uint32_t last_l;
    __shared__ unsigned long long sum_l[kThreads];
    __shared__ uint32_t pick_l;
    const int shift = round == 0 ? 21 : round == 1 ? 10 : 0;
    const int width = round == 2 ? 10 : 11;
    const uint32_t hi_mask = round == 0 ? 0u : ~((1u << (shift + width)) - 1u);
    const uint32_t prefix = coherent_load(&ws.plan->prefix);
    const uint32_t floor_key = phase == 1 ? coherent_load(&ws.plan->restrict_key) : 0u;
    const float m = smp_kfloat(coherent_load(&ws.plan->max_key));
    for (int d = threadIdx.x; d < kDigits; d += kThreads) {
        lcnt[d] = 0u;
        lmass[d] = 0ull;
    }
    __syncthreads();
    const uint32_t i0 = 4u * (blockIdx.x * kThreads + threadIdx.x);
    if (i0 < n) {
        const float4 w4 = *reinterpret_cast<const float4*>(ws.w + i0);
        const float w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t key = smp_fkey(w[j]);
            if ((key & hi_mask) == prefix && key >= floor_key) {
                const uint32_t d = (key >> shift) & ((1u << width) - 1u);
                if (phase == 0) {
                    atomicAdd(&lcnt[d], 1u);
                } else {
                    atomicAdd(&lmass[d], smp_mass(w[j], m));
                }
            }
        }
    }
    __syncthreads();
    for (int d = threadIdx.x; d < kDigits; d += kThreads) {
        if (phase == 0 && lcnt[d] != 0u) {
            __hip_atomic_fetch_add(ws.hcnt + d, lcnt[d], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (phase == 1 && lmass[d] != 0ull) {
            __hip_atomic_fetch_add(ws.hmass + d, lmass[d], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // the last workgroup to arrive sees every workgroup's additions
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t done = __hip_atomic_fetch_add(&ws.plan->arrive, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last_l = done == gridDim.x - 1u ? 1u : 0u;
    }
    __syncthreads();
    if (last_l == 0u) {
        return;
    }
    __threadfence();
    // digits 8t .. 8t + 7 per thread: values, their sum, and a suffix scan
    // over the threads (high digits first) of the sums
    constexpr int kPer = kDigits / kThreads;
    unsigned long long val[kPer];
    unsigned long long tsum = 0ull;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int d = threadIdx.x * kPer + j;
        val[j] = phase == 0 ? static_cast<unsigned long long>(coherent_load(ws.hcnt + d)) : coherent_load(ws.hmass + d);
        tsum += val[j];
        if (phase == 0) {
            __hip_atomic_store(ws.hcnt + d, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            __hip_atomic_store(ws.hmass + d, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    sum_l[threadIdx.x] = tsum;
    if (threadIdx.x == 0) {
        pick_l = 0u;  // 1 + the chosen digit (0: none yet)
    }
    __syncthreads();
    unsigned long long base = round == 0 ? 0ull : coherent_load(&ws.plan->base);
    unsigned long long target;
    if (round == 0) {
        if (phase == 0) {
            target = p.top_k;
        } else {
            unsigned long long z = 0ull;
            for (int t = 0; t < kThreads; ++t) {
                z += sum_l[t];
            }
            target = smp_mass_target(z, p.top_p);
        }
    } else {
        target = coherent_load(&ws.plan->target);
    }
    // the mass / count above this thread's digits (threads above it, in order)
    unsigned long long above = base;
    for (int t = kThreads - 1; t > static_cast<int>(threadIdx.x); --t) {
        above += sum_l[t];
    }
    // the highest digit d with above(d) + val(d) >= target
    uint32_t mine = 0xffffffffu;
    unsigned long long mine_above = 0ull;
#pragma unroll
    for (int j = kPer - 1; j >= 0; --j) {
        if (mine == 0xffffffffu && above + val[j] >= target) {
            mine = static_cast<uint32_t>(threadIdx.x * kPer + j);
            mine_above = above;
        }
        above += val[j];
    }
    if (mine != 0xffffffffu) {
        atomicMax(&pick_l, mine + 1u);  // LDS: the highest qualifying digit
    }
    __syncthreads();
    const uint32_t d = pick_l - 1u;
    if (pick_l != 0u && mine == d) {
        // (exactly one thread: the digit's owner)
        const uint32_t key = prefix | (d << shift);
        SmpPlan* pl = ws.plan;
        if (round < 2) {
            __hip_atomic_store(&pl->prefix, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&pl->base, mine_above, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&pl->target, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            // the phase's threshold: the next phase starts from a clean band
            __hip_atomic_store(&pl->prefix, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&pl->base, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&pl->target, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (phase == 0) {
                __hip_atomic_store(&pl->restrict_key, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __hip_atomic_store(&pl->tau_key, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (final_round) {
                __hip_atomic_store(&pl->max_key, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&pl->restrict_key, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if (threadIdx.x == 0) {
        __hip_atomic_store(&ws.plan->arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The Gumbel-max over {w >= tau}, folded into the key word; the last
// workgroup clears the threshold word (the workspace is left zero).
__global__ __launch_bounds__(kThreads) void k_smp_draw(uint32_t n, mh_sample_params p, SmpWs ws,
                                                       unsigned long long* best) {
    __shared__ unsigned long long part[kThreads / 64];
    __shared__ uint32_t last_l;
    const uint32_t tau = coherent_load(&ws.plan->tau_key);
    const uint32_t q = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t i0 = 4u * q;
    unsigned long long k = 0ull;
    if (i0 < n) {
        const float4 w4 = *reinterpret_cast<const float4*>(ws.w + i0);
        const float w[4] = {w4.x, w4.y, w4.z, w4.w};
        const mh::u32x4 r = mh::philox4x32_10(mh::u32x4{q, p.pos, kDomain, 0u}, p.seed_lo, p.seed_hi);
        const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (smp_fkey(w[j]) >= tau) {
                const unsigned long long kj = mh::argmax_key(w[j] + mh::gumbel_of(rw[j]), i0 + j);
                k = kj > k ? kj : k;
            }
        }
    }
    k = mh::wave_max_u64(k);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        part[wave] = k;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < kThreads / 64; ++w) {
            k = part[w] > k ? part[w] : k;
        }
        if (k != 0ull && k > __hip_atomic_load(best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            __hip_atomic_fetch_max(best, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const uint32_t done = __hip_atomic_fetch_add(&ws.plan->arrive, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last_l = done == gridDim.x - 1u ? 1u : 0u;
    }
    __syncthreads();
    if (last_l != 0u && threadIdx.x == 0) {
        __hip_atomic_store(&ws.plan->tau_key, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&ws.plan->arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

__global__ void k_smp_mark(const uint32_t* tok, uint32_t* seen, uint32_t n) {
    if (threadIdx.x == 0) {
        const uint32_t t = tok[0];
        if (t < n) {
            seen[t >> 5] |= 1u << (t & 31u);
        }
    }
}

}  // namespace

extern "C" size_t mh_sample_workspace_bytes(uint32_t n) { return smp_bytes(n); }

extern "C" int mh_sample_draw(const uint16_t* logits, uint32_t n, const uint32_t* seen,
                              const mh_sample_params* params, uint64_t* best, void* workspace,
                              size_t workspace_bytes, mh_stream_t stream) {
    const char* op = "mh_sample_draw";
    MH_ENSURE(logits && params && best, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(n > 0 && n % 4u == 0u, MH_ERR_INVALID, "%s: vocabulary %u not a positive multiple of 4", op, n);
    MH_ENSURE(params->use_penalty == 0u || seen != nullptr, MH_ERR_INVALID, "%s: the penalty needs the seen set", op);
    MH_ENSURE(params->top_p > 0.0f, MH_ERR_INVALID, "%s: top_p must be in (0, 1]", op);
    MH_ENSURE(mh::aligned(logits, 8) && mh::aligned(best, 8) && mh::aligned(seen, 4), MH_ERR_ALIGN,
              "%s: logits / key alignment", op);
    const bool use_k = params->top_k != 0u && params->top_k < n;
    const bool use_p = params->top_p < 1.0f;
    if (!use_k && !use_p) {
        mh_sample_params full = *params;
        full.top_k = 0u;
        return mh_sample_gumbel(logits, n, seen, &full, best, stream);
    }
    MH_ENSURE(workspace != nullptr && workspace_bytes >= smp_bytes(n), MH_ERR_INVALID,
              "%s: workspace holds %zu bytes, needs %zu", op, workspace_bytes, smp_bytes(n));
    MH_ENSURE(mh::aligned(workspace, 256), MH_ERR_ALIGN, "%s: workspace not 256-byte aligned", op);
    const SmpWs ws = smp_layout(workspace, n);
    const hipStream_t s = mh::as_stream(stream);
    const uint32_t grid = (n + kBlock - 1u) / kBlock;
    hipLaunchKernelGGL(k_smp_prep, dim3(grid), dim3(kThreads), 0, s, logits, n, seen, *params, ws);
    MH_TRY(mh::launch_status("k_smp_prep"));
    for (int phase = 0; phase < 2; ++phase) {
        if ((phase == 0 && !use_k) || (phase == 1 && !use_p)) {
            continue;
        }
        for (int round = 0; round < 3; ++round) {
            const int final_round = round == 2 && (phase == 1 || !use_p) ? 1 : 0;
            hipLaunchKernelGGL(k_smp_round, dim3(grid), dim3(kThreads), 0, s, n, *params, ws, phase, round,
                               final_round);
            MH_TRY(mh::launch_status("k_smp_round"));
        }
    }
    hipLaunchKernelGGL(k_smp_draw, dim3(grid), dim3(kThreads), 0, s, n, *params, ws,
                       reinterpret_cast<unsigned long long*>(best));
    return mh::launch_status("k_smp_draw");
}

extern "C" int mh_sample_mark(const uint32_t* tok, uint32_t* seen, uint32_t n, mh_stream_t stream) {
    MH_ENSURE(tok && seen, MH_ERR_INVALID, "mh_sample_mark: NULL argument");
    hipLaunchKernelGGL(k_smp_mark, dim3(1), dim3(64), 0, mh::as_stream(stream), tok, seen, n);
    return mh::launch_status("k_smp_mark");
}

extern "C" int mh_sample_gumbel(const uint16_t* logits, uint32_t n, const uint32_t* seen,
                                const mh_sample_params* params, uint64_t* best, mh_stream_t stream) {
    const char* op = "mh_sample_gumbel";
    MH_ENSURE(logits && params && best, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(n > 0 && n % 4u == 0u, MH_ERR_INVALID, "%s: vocabulary %u not a positive multiple of 4", op, n);
    MH_ENSURE(params->top_k == 0u && !(params->top_p < 1.0f), MH_ERR_UNSUPPORTED,
              "%s: top-k / top-p need the kept-set draw (mh_sample_draw)", op);
    MH_ENSURE(params->use_penalty == 0u || seen != nullptr, MH_ERR_INVALID, "%s: the penalty needs the seen set", op);
    MH_ENSURE(mh::aligned(logits, 8) && mh::aligned(best, 8) && mh::aligned(seen, 4), MH_ERR_ALIGN,
              "%s: logits / key alignment", op);
    const uint32_t grid = (n / 4u + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(k_sample_gumbel, dim3(grid), dim3(kThreads), 0, mh::as_stream(stream), logits, n, seen,
                       *params, reinterpret_cast<unsigned long long*>(best));
    return mh::launch_status("k_sample_gumbel");
}

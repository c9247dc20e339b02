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
// and 10 bits per phase (a count phase for top-k, then a mass phase for top-p
// restricted to the top-k set).  Each round is one launch in which every
// workgroup histograms its tokens' digits in LDS and adds the nonzero bins to
// that round's global histogram.  The digit a round picks is decided at the
// start of the next launch, by every workgroup alike, from the round's
// histogram and the state the round ran with (a suffix scan over the bins):
// no arrival counter, no fence and no serial tail between rounds.  The first
// count round runs inside the launch that computes w.  The draw launch
// decides the last round and folds the Gumbel-max over {w >= tau} into the
// key word, as the temperature draw.  With both top-k and top-p on, the mass
// phase has no launches of its own: the draw launch appends the top-k set to
// a list and its last workgroup decides top-p over the list
// (k_smp_draw_kept).
//
// Workspace (caller-owned; its head -- the kept list's counters and the
// first round's histogram -- zeroed before the first call and left zero by
// every call; the rest is rewritten by every call): w f32[n], the
// per-workgroup max keys, one histogram per round, the state each round ran
// with, and the kept list.
constexpr int kGroups = 4;                          // groups of 4 tokens per thread
constexpr uint32_t kBlock = 4u * kGroups * kThreads;  // tokens per workgroup
constexpr int kDigits = 2048;                       // 11-bit digits
constexpr int kRounds = 6;                          // 3 count + 3 mass rounds at most
constexpr int kPer = kDigits / kThreads;            // bins per thread in the scan

// The band a round histograms (keys whose bits above the round's digit equal
// prefix, and >= restrict_key) and the target the next decision meets.
struct SmpState {
    uint32_t prefix;        // digits chosen so far in this phase
    uint32_t restrict_key;  // the mass phase's floor (the top-k threshold, or 0)
    uint32_t tau_key;       // the latest phase threshold (0: every token)
    uint32_t pad0;
    unsigned long long base;    // count / mass of the keys above the band
    unsigned long long target;  // k, or the mass target (0: set by the first mass round)
};

// The zeroed head of the workspace (with the first round's histogram after
// it): the kept-set draw's append counter and finished-workgroup count.
struct SmpCtl {
    uint32_t kept;
    uint32_t done;
};
constexpr uint32_t kKeptCap = 256;  // kept tokens the finishing workgroup takes from the list
constexpr size_t kCtlBytes = 256;
constexpr size_t kZeroBytes = kCtlBytes + static_cast<size_t>(kDigits) * 8u;  // ctl + round 0's bins
static_assert(kZeroBytes == MH_SAMPLE_ZERO_BYTES, "the header's zero-region size");

struct SmpWs {
    float* w;
    uint32_t* wmax;             // per-workgroup max key
    unsigned long long* hist;   // kRounds x kDigits
    SmpState* plan;             // the state each round ran with
    SmpCtl* ctl;
    unsigned long long* kept;   // kKeptCap x {key << 32 | 2^31 | index, mass, draw key}
};

size_t smp_align(size_t b) { return (b + 255u) & ~static_cast<size_t>(255u); }

uint32_t smp_grid(uint32_t n) { return (n + kBlock - 1u) / kBlock; }

SmpWs smp_layout(void* ws, uint32_t n) {
    char* p = static_cast<char*>(ws);
    SmpWs l;
    l.ctl = reinterpret_cast<SmpCtl*>(p);
    p += kCtlBytes;
    l.hist = reinterpret_cast<unsigned long long*>(p);
    p += smp_align(static_cast<size_t>(kRounds) * kDigits * 8u);
    l.plan = reinterpret_cast<SmpState*>(p);
    p += smp_align(kRounds * sizeof(SmpState));
    l.wmax = reinterpret_cast<uint32_t*>(p);
    p += smp_align(static_cast<size_t>(smp_grid(n)) * 4u);
    l.kept = reinterpret_cast<unsigned long long*>(p);
    p += smp_align(static_cast<size_t>(kKeptCap) * 3u * 8u);
    l.w = reinterpret_cast<float*>(p);
    return l;
}

size_t smp_bytes(uint32_t n) {
    return kCtlBytes + smp_align(static_cast<size_t>(kRounds) * kDigits * 8u) +
           smp_align(kRounds * sizeof(SmpState)) + smp_align(static_cast<size_t>(smp_grid(n)) * 4u) +
           smp_align(static_cast<size_t>(kKeptCap) * 3u * 8u) + smp_align(static_cast<size_t>(n) * 4u);
}

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

// exp(w - m) in 2^-40 fixed point, truncated (w <= m: at most 2^40).  w - m
// is NaN when both are the same infinity (every logit -inf, or the maximum
// +inf): the token then has the maximum's mass exp(0); a NaN w or m has none.
__device__ __forceinline__ unsigned long long smp_mass(float w, float m) {
    float d = w - m;
    if (d != d) {
        d = w == m ? 0.0f : -__builtin_inff();
    }
    return static_cast<unsigned long long>(mh::expf_fixed(d) * 1099511627776.0f);
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

__device__ __forceinline__ int smp_shift(int round) { return round == 0 ? 21 : round == 1 ? 10 : 0; }
__device__ __forceinline__ int smp_width(int round) { return round == 2 ? 10 : 11; }

// tokens i0 .. i0 + 3 of group g of this thread (coalesced within a group)
__device__ __forceinline__ uint32_t smp_token0(int g) {
    return blockIdx.x * kBlock + static_cast<uint32_t>(g) * (4u * kThreads) + 4u * threadIdx.x;
}

struct SmpDecideLds {
    unsigned long long wsum[kThreads / 64];
    uint32_t pick;  // 1 + the chosen digit (0: none yet)
    SmpState out;
};

// A round's histogram bins of this thread and the state the round ran with.
struct SmpPrev {
    SmpState in;
    unsigned long long val[kPer];
};

// (issued before the launch's other loads are waited for)
__device__ __forceinline__ SmpPrev smp_prev_load(const SmpWs& ws, int prev) {
    SmpPrev r;
    r.in = ws.plan[prev];
    const unsigned long long* h = ws.hist + static_cast<size_t>(prev) * kDigits + threadIdx.x * kPer;
#pragma unroll
    for (int j = 0; j < kPer; j += 2) {
        const ulonglong2 v2 = *reinterpret_cast<const ulonglong2*>(h + j);
        r.val[j] = v2.x;
        r.val[j + 1] = v2.y;
    }
    return r;
}

// The state of the round after `prev` (phase pp, round pr): the highest digit
// d of prev's histogram whose cumulative count / mass from the top reaches
// the target.  Every workgroup computes the same state from the same words.
__device__ SmpState smp_decide(const SmpPrev& pv, int pp, int pr, const mh_sample_params& p, SmpDecideLds& l) {
    const SmpState& in = pv.in;
    const unsigned long long* val = pv.val;
    unsigned long long tsum = 0ull;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        tsum += val[j];
    }
    // inclusive suffix sum over the lanes (lane l: lanes l .. 63), then the
    // waves' totals
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    unsigned long long suf = tsum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const unsigned long long o = __shfl_down(suf, off);
        if (lane + off < 64) {
            suf += o;
        }
    }
    if (lane == 0) {
        l.wsum[wave] = suf;
    }
    if (threadIdx.x == 0) {
        l.pick = 0u;
    }
    __syncthreads();
    unsigned long long later = 0ull, total = 0ull;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
        total += l.wsum[w];
        later += w > wave ? l.wsum[w] : 0ull;
    }
    const unsigned long long target = (pp == 1 && pr == 0) ? smp_mass_target(total, p.top_p) : in.target;
    // the count / mass above this thread's bins, then the highest bin d with
    // above(d) + val(d) >= target
    unsigned long long above = in.base + later + (suf - tsum);
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
        atomicMax(&l.pick, mine + 1u);  // LDS: the highest qualifying digit
    }
    __syncthreads();
    const uint32_t pick = l.pick;
    if (pick == 0u ? threadIdx.x == 0 : mine == pick - 1u) {
        // (exactly one thread; no digit reaches the target only if the
        // histogram is empty, and the band is then kept whole)
        const uint32_t d = pick == 0u ? 0u : pick - 1u;
        const uint32_t key = in.prefix | (d << smp_shift(pr));
        SmpState o = in;
        if (pr < 2) {
            o.prefix = key;
            o.base = pick == 0u ? in.base : mine_above;
            o.target = target;
        } else {
            o.prefix = 0u;
            o.base = 0ull;
            o.target = 0ull;
            o.restrict_key = pp == 0 ? key : in.restrict_key;
            o.tau_key = key;
        }
        l.out = o;
    }
    __syncthreads();
    return l.out;
}

// w of every token, the workgroups' max keys, and (COUNT0) the first count
// round's histogram; zeroes the other rounds' histograms.
template <bool COUNT0>
__global__ __launch_bounds__(kThreads) void k_smp_prep(const uint16_t* logits, uint32_t n, const uint32_t* seen,
                                                       mh_sample_params p, SmpWs ws) {
    __shared__ uint32_t lcnt[COUNT0 ? kDigits : 1];
    __shared__ uint32_t part[kThreads / 64];
    if (COUNT0) {
        for (int d = threadIdx.x; d < kDigits; d += kThreads) {
            lcnt[d] = 0u;
        }
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            SmpState s0 = {};
            s0.target = p.top_k;
            ws.plan[0] = s0;
        }
    }
    for (uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < (kRounds - 1) * kDigits; i += gridDim.x * kThreads) {
        ws.hist[kDigits + i] = 0ull;
    }
    if (COUNT0) {
        __syncthreads();
    }
    uint32_t kmax = 0u;
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        const uint32_t i0 = smp_token0(g);
        if (i0 < n) {
            const uint2 raw = *reinterpret_cast<const uint2*>(logits + i0);
            const float v[4] = {mh::bf16lo(raw.x), mh::bf16hi(raw.x), mh::bf16lo(raw.y), mh::bf16hi(raw.y)};
            const uint32_t bits = p.use_penalty != 0u ? (seen[i0 >> 5] >> (i0 & 31u)) : 0u;
            float w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                w[j] = processed(v[j], ((bits >> j) & 1u) != 0u, p);
                const uint32_t key = smp_fkey(w[j]);
                kmax = max(kmax, key);
                if (COUNT0) {
                    atomicAdd(&lcnt[key >> 21], 1u);
                }
            }
            *reinterpret_cast<float4*>(ws.w + i0) = make_float4(w[0], w[1], w[2], w[3]);
        }
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
        ws.wmax[blockIdx.x] = kmax;
    }
    if (COUNT0) {
        for (int d = threadIdx.x; d < kDigits; d += kThreads) {
            if (lcnt[d] != 0u) {
                __hip_atomic_fetch_add(ws.hist + d, static_cast<unsigned long long>(lcnt[d]), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// The vocabulary's max key, from the workgroups' max keys.
__device__ uint32_t smp_max_key(const SmpWs& ws, uint32_t* part) {
    uint32_t k = 0u;
    for (uint32_t i = threadIdx.x; i < gridDim.x; i += kThreads) {
        k = max(k, ws.wmax[i]);
    }
    k = mh::wave_max_u32(k);
    if ((threadIdx.x & 63) == 0) {
        part[threadIdx.x >> 6] = k;
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
        k = max(k, part[w]);
    }
    return k;
}

// Round `step` of this call (phase PHASE, digit round `round`): decides the
// previous round (phase pp, round pr) unless step is 0, records the state,
// and histograms the band's digits (counts, or masses exp(w - M)).
template <int PHASE>
__global__ __launch_bounds__(kThreads) void k_smp_round(uint32_t n, mh_sample_params p, SmpWs ws, int step,
                                                        int round, int pp, int pr) {
    __shared__ uint32_t lcnt[PHASE == 0 ? kDigits : 1];
    __shared__ unsigned long long lmass[PHASE == 1 ? kDigits : 1];
    __shared__ SmpDecideLds dl;
    __shared__ uint32_t part[kThreads / 64];
    // every load of the launch is issued before any is waited for: the
    // tokens, the previous round's bins and state, the max keys
    float4 w4[kGroups];
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        const uint32_t i0 = smp_token0(g);
        w4[g] = i0 < n ? *reinterpret_cast<const float4*>(ws.w + i0) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const SmpPrev pv = smp_prev_load(ws, step > 0 ? step - 1 : 0);
    for (int d = threadIdx.x; d < kDigits; d += kThreads) {
        if (PHASE == 0) {
            lcnt[d] = 0u;
        } else {
            lmass[d] = 0ull;
        }
    }
    float m = 0.0f;
    if (PHASE == 1) {
        m = smp_kfloat(smp_max_key(ws, part));
    }
    SmpState st = {};
    if (step == 0) {
        st.target = PHASE == 0 ? p.top_k : 0ull;
    } else {
        st = smp_decide(pv, pp, pr, p, dl);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        ws.plan[step] = st;
    }
    __syncthreads();
    const int shift = smp_shift(round), width = smp_width(round);
    const uint32_t hi_mask = round == 0 ? 0u : ~((1u << (shift + width)) - 1u);
    const uint32_t floor_key = PHASE == 1 ? st.restrict_key : 0u;
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        const uint32_t i0 = smp_token0(g);
        if (i0 < n) {
            const float w[4] = {w4[g].x, w4[g].y, w4[g].z, w4[g].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t key = smp_fkey(w[j]);
                if ((key & hi_mask) == st.prefix && key >= floor_key) {
                    const uint32_t d = (key >> shift) & ((1u << width) - 1u);
                    if (PHASE == 0) {
                        atomicAdd(&lcnt[d], 1u);
                    } else {
                        atomicAdd(&lmass[d], smp_mass(w[j], m));
                    }
                }
            }
        }
    }
    __syncthreads();
    unsigned long long* h = ws.hist + static_cast<size_t>(step) * kDigits;
    for (int d = threadIdx.x; d < kDigits; d += kThreads) {
        const unsigned long long v = PHASE == 0 ? static_cast<unsigned long long>(lcnt[d]) : lmass[d];
        if (v != 0ull) {
            __hip_atomic_fetch_add(h + d, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Decides the last round (step `last`: phase pp, round 2), then folds the
// Gumbel-max over {w >= tau} into the key word; zeroes the first round's
// histogram for the next call.
__global__ __launch_bounds__(kThreads) void k_smp_draw(uint32_t n, mh_sample_params p, SmpWs ws, int last, int pp,
                                                       unsigned long long* best) {
    __shared__ unsigned long long part[kThreads / 64];
    __shared__ SmpDecideLds dl;
    float4 w4[kGroups];
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        const uint32_t i0 = smp_token0(g);
        w4[g] = i0 < n ? *reinterpret_cast<const float4*>(ws.w + i0) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const SmpPrev pv = smp_prev_load(ws, last);
    // the perturbed values (w + G) while the loads are in flight
    float y[kGroups][4];
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        const uint32_t i0 = smp_token0(g);
        const mh::u32x4 r = mh::philox4x32_10(mh::u32x4{i0 / 4u, p.pos, kDomain, 0u}, p.seed_lo, p.seed_hi);
        y[g][0] = mh::gumbel_of(r.x);
        y[g][1] = mh::gumbel_of(r.y);
        y[g][2] = mh::gumbel_of(r.z);
        y[g][3] = mh::gumbel_of(r.w);
    }
    const uint32_t tau = smp_decide(pv, pp, 2, p, dl).tau_key;
    for (uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < kDigits; i += gridDim.x * kThreads) {
        ws.hist[i] = 0ull;
    }
    unsigned long long k = 0ull;
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        const uint32_t i0 = smp_token0(g);
        if (i0 < n) {
            const float w[4] = {w4[g].x, w4[g].y, w4[g].z, w4[g].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (smp_fkey(w[j]) >= tau) {
                    const unsigned long long kj = mh::argmax_key(w[j] + y[g][j], i0 + j);
                    k = kj > k ? kj : k;
                }
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
    }
}

// Exclusive prefix of v over the workgroup's threads (and the total).
__device__ uint32_t smp_block_excl(uint32_t v, uint32_t* part, uint32_t& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(inc, off);
        if (lane >= off) {
            inc += o;
        }
    }
    if (lane == 63) {
        part[wave] = inc;
    }
    __syncthreads();
    uint32_t before = 0u;
    total = 0u;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
        before += w < wave ? part[w] : 0u;
        total += part[w];
    }
    __syncthreads();
    return before + inc - v;
}

// The kept-set draw when both top-k and top-p are on, in one launch after
// the count rounds: every workgroup decides the last count round (tau_k),
// appends its tokens with key >= tau_k to the kept list (key and index, mass,
// draw key) and counts itself finished; the last workgroup to finish takes
// top-p over the list -- tau_p is the greatest kept key whose cumulative
// mass (every kept token with a key >= it) reaches the target, which is the
// radix select's tie-group walk -- and folds the draw over {key >= tau_p}
// into the key word.  A list longer than kKeptCap (ties at the threshold, or
// a large k) is decided by that workgroup alone with the mass phase's three
// radix rounds over all tokens.  The finishing workgroup leaves the counters
// zero for the next call.
__global__ __launch_bounds__(kThreads) void k_smp_draw_kept(uint32_t n, mh_sample_params p, SmpWs ws, int last,
                                                            unsigned long long* best) {
    __shared__ unsigned long long partk[kThreads / 64];
    __shared__ uint32_t partu[kThreads / 64];
    __shared__ SmpDecideLds dl;
    __shared__ uint32_t wg_base, is_last;
    __shared__ unsigned long long lk[kKeptCap], lm[kKeptCap], lg[kKeptCap];
    __shared__ unsigned long long lmass[kDigits];
    __shared__ uint32_t tau_l;
    float4 w4[kGroups];
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        const uint32_t i0 = smp_token0(g);
        w4[g] = i0 < n ? *reinterpret_cast<const float4*>(ws.w + i0) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const SmpPrev pv = smp_prev_load(ws, last);
    float y[kGroups][4];
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        const uint32_t i0 = smp_token0(g);
        const mh::u32x4 r = mh::philox4x32_10(mh::u32x4{i0 / 4u, p.pos, kDomain, 0u}, p.seed_lo, p.seed_hi);
        y[g][0] = mh::gumbel_of(r.x);
        y[g][1] = mh::gumbel_of(r.y);
        y[g][2] = mh::gumbel_of(r.z);
        y[g][3] = mh::gumbel_of(r.w);
    }
    const float m = smp_kfloat(smp_max_key(ws, partu));
    const uint32_t tau_k = smp_decide(pv, 0, 2, p, dl).tau_key;
    for (uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < kDigits; i += gridDim.x * kThreads) {
        __hip_atomic_store(ws.hist + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // this workgroup's kept tokens into the list
    uint32_t cnt = 0u;
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        const uint32_t i0 = smp_token0(g);
        const float w[4] = {w4[g].x, w4[g].y, w4[g].z, w4[g].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            cnt += i0 < n && smp_fkey(w[j]) >= tau_k ? 1u : 0u;
        }
    }
    uint32_t total = 0u;
    const uint32_t excl = smp_block_excl(cnt, partu, total);
    if (threadIdx.x == 0) {
        wg_base = total != 0u ? __hip_atomic_fetch_add(&ws.ctl->kept, total, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT)
                              : 0u;
    }
    __syncthreads();
    // entries as device-coherent stores (no dirty L2 lines for the release
    // below to write back), then the finished count with release / acquire
    uint32_t pos = wg_base + excl;
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
        const uint32_t i0 = smp_token0(g);
        const float w[4] = {w4[g].x, w4[g].y, w4[g].z, w4[g].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t key = smp_fkey(w[j]);
            if (i0 < n && key >= tau_k) {
                if (pos < kKeptCap) {
                    __hip_atomic_store(ws.kept + 3u * pos, (static_cast<unsigned long long>(key) << 32) | 0x80000000u | (i0 + j), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(ws.kept + 3u * pos + 1u, smp_mass(w[j], m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(ws.kept + 3u * pos + 2u, mh::argmax_key(w[j] + y[g][j], i0 + j), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                ++pos;
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");  // every wave's entries
    __syncthreads();
    if (threadIdx.x == 0) {
        is_last = __hip_atomic_fetch_add(&ws.ctl->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                          gridDim.x - 1u
                      ? 1u
                      : 0u;
    }
    __syncthreads();
    if (is_last == 0u) {
        return;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // the other workgroups' entries
    const uint32_t K = __hip_atomic_load(&ws.ctl->kept, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned long long kb = 0ull;  // this thread's best draw key
    if (K <= kKeptCap) {
        const uint32_t t = threadIdx.x;
        if (t < K) {
            lk[t] = __hip_atomic_load(ws.kept + 3u * t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            lm[t] = __hip_atomic_load(ws.kept + 3u * t + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            lg[t] = __hip_atomic_load(ws.kept + 3u * t + 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (t == 0) {
            tau_l = tau_k;
        }
        __syncthreads();
        // z: the kept mass; entry t's cumulative mass (keys >= its key)
        unsigned long long z = 0ull, cum = 0ull;
        const uint32_t kt = t < K ? static_cast<uint32_t>(lk[t] >> 32) : 0u;
        if (t < K) {
            for (uint32_t j = 0; j < K; ++j) {
                const unsigned long long mj = lm[j];
                z += mj;
                cum += static_cast<uint32_t>(lk[j] >> 32) >= kt ? mj : 0ull;
            }
            const unsigned long long target = smp_mass_target(z, p.top_p);
            if (cum >= target) {
                atomicMax(&tau_l, kt);  // LDS: the greatest qualifying key
            }
        }
        __syncthreads();
        const uint32_t tau = tau_l;
        if (t < K && kt >= tau) {
            kb = lg[t];
        }
    } else {
        // the mass phase's radix rounds over every token, by this workgroup
        SmpState st = {};
        st.restrict_key = tau_k;
        for (int round = 0; round < 3; ++round) {
            for (int d = threadIdx.x; d < kDigits; d += kThreads) {
                lmass[d] = 0ull;
            }
            __syncthreads();
            const int shift = smp_shift(round), width = smp_width(round);
            const uint32_t hi_mask = round == 0 ? 0u : ~((1u << (shift + width)) - 1u);
            for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
                const float w = ws.w[i];
                const uint32_t key = smp_fkey(w);
                if ((key & hi_mask) == st.prefix && key >= st.restrict_key) {
                    atomicAdd(&lmass[(key >> shift) & ((1u << width) - 1u)], smp_mass(w, m));
                }
            }
            __syncthreads();
            SmpPrev hv;
            hv.in = st;
#pragma unroll
            for (int j = 0; j < kPer; ++j) {
                hv.val[j] = lmass[threadIdx.x * kPer + j];
            }
            st = smp_decide(hv, 1, round, p, dl);
        }
        const uint32_t tau = st.tau_key;
        for (uint32_t i0 = 4u * threadIdx.x; i0 < n; i0 += 4u * kThreads) {
            const float4 v = *reinterpret_cast<const float4*>(ws.w + i0);
            const float w[4] = {v.x, v.y, v.z, v.w};
            const mh::u32x4 r = mh::philox4x32_10(mh::u32x4{i0 / 4u, p.pos, kDomain, 0u}, p.seed_lo, p.seed_hi);
            const float g[4] = {mh::gumbel_of(r.x), mh::gumbel_of(r.y), mh::gumbel_of(r.z), mh::gumbel_of(r.w)};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (smp_fkey(w[j]) >= tau) {
                    const unsigned long long kj = mh::argmax_key(w[j] + g[j], i0 + j);
                    kb = kj > kb ? kj : kb;
                }
            }
        }
    }
    kb = mh::wave_max_u64(kb);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        partk[wave] = kb;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < kThreads / 64; ++w) {
            kb = partk[w] > kb ? partk[w] : kb;
        }
        __hip_atomic_store(&ws.ctl->kept, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&ws.ctl->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (kb != 0ull && kb > __hip_atomic_load(best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            __hip_atomic_fetch_max(best, kb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
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
    MH_ENSURE(n > 0 && n % 4u == 0u && n <= 0x80000000u, MH_ERR_INVALID,
              "%s: vocabulary %u not a positive multiple of 4 (at most 2^31)", op, n);
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
    const uint32_t grid = smp_grid(n);
    if (use_k) {
        hipLaunchKernelGGL(k_smp_prep<true>, dim3(grid), dim3(kThreads), 0, s, logits, n, seen, *params, ws);
    } else {
        hipLaunchKernelGGL(k_smp_prep<false>, dim3(grid), dim3(kThreads), 0, s, logits, n, seen, *params, ws);
    }
    MH_TRY(mh::launch_status("k_smp_prep"));
    // the rounds of this call: (phase, round); a count round 0 ran in prep.
    // With both on, the mass phase is decided over the top-k list by the
    // kept-set draw's last workgroup (k_smp_draw_kept).
    const bool kept_draw = use_k && use_p;
    int step = 0, pp = 0, pr = 0;
    for (int phase = 0; phase < 2; ++phase) {
        if ((phase == 0 && !use_k) || (phase == 1 && (!use_p || kept_draw))) {
            continue;
        }
        for (int round = 0; round < 3; ++round) {
            if (!(phase == 0 && round == 0)) {
                if (phase == 0) {
                    hipLaunchKernelGGL(k_smp_round<0>, dim3(grid), dim3(kThreads), 0, s, n, *params, ws, step, round,
                                       pp, pr);
                } else {
                    hipLaunchKernelGGL(k_smp_round<1>, dim3(grid), dim3(kThreads), 0, s, n, *params, ws, step, round,
                                       pp, pr);
                }
                MH_TRY(mh::launch_status("k_smp_round"));
            }
            pp = phase;
            pr = round;
            ++step;
        }
    }
    if (kept_draw) {
        hipLaunchKernelGGL(k_smp_draw_kept, dim3(grid), dim3(kThreads), 0, s, n, *params, ws, step - 1,
                           reinterpret_cast<unsigned long long*>(best));
        return mh::launch_status("k_smp_draw_kept");
    }
    hipLaunchKernelGGL(k_smp_draw, dim3(grid), dim3(kThreads), 0, s, n, *params, ws, step - 1, pp,
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

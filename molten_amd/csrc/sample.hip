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

}  // namespace

extern "C" int mh_sample_gumbel(const uint16_t* logits, uint32_t n, const uint32_t* seen,
                                const mh_sample_params* params, uint64_t* best, mh_stream_t stream) {
    const char* op = "mh_sample_gumbel";
    MH_ENSURE(logits && params && best, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(n > 0 && n % 4u == 0u, MH_ERR_INVALID, "%s: vocabulary %u not a positive multiple of 4", op, n);
    MH_ENSURE(params->top_k == 0u && !(params->top_p < 1.0f), MH_ERR_UNSUPPORTED,
              "%s: top-k / top-p sampling is not built (temperature-only draw)", op);
    MH_ENSURE(params->use_penalty == 0u || seen != nullptr, MH_ERR_INVALID, "%s: the penalty needs the seen set", op);
    MH_ENSURE(mh::aligned(logits, 8) && mh::aligned(best, 8) && mh::aligned(seen, 4), MH_ERR_ALIGN,
              "%s: logits / key alignment", op);
    const uint32_t grid = (n / 4u + kThreads - 1) / kThreads;
    hipLaunchKernelGGL(k_sample_gumbel, dim3(grid), dim3(kThreads), 0, mh::as_stream(stream), logits, n, seen,
                       *params, reinterpret_cast<unsigned long long*>(best));
    return mh::launch_status("k_sample_gumbel");
}

// moe_decode_fused.hip -- the MoE decode step (router -> top-k -> expert
// gate/up + SwiGLU -> down + weighted combine) as one persistent launch.
//
// kGrid workgroups of kWaves waves (one per CU on a 256-CU part, all
// resident at once) run three phases:
//   1. router logits: wave 0 of workgroup e computes row e;
//   2. every wave routes the token itself (from the logits, in registers),
//      computes three SwiGLU activations (three gate rows and three up rows
//      of the chosen experts), then issues the loads of its down-projection
//      rows;
//   3. each workgroup stages all activations in LDS and each wave produces
//      one output of the down projection + weighted combine.
// Same arithmetic (chunk order, roundings) as the three-launch path in
// moe_decode.hip, so outputs are bit-identical to it and to the oracle.
//
// Cross-workgroup exchange without grid barriers: a logit, or three
// activations, travel as one 64-bit word {data, tag} written with a single
// device-coherent store; a consumer polls the words it needs with
// device-coherent loads until each carries the current launch's tag.  Data
// and tag arrive together, so there is no store-acknowledge wait and no
// arrival counter on the critical path.  The logits are stored kReplicas
// times (one copy per XCD: workgroup b reads copy b % kReplicas), so the
// pollers of a copy are the 32 workgroups of one XCD.  The epoch: workgroup
// b keeps a launch count in scratch word b, reads it at its start and writes
// it back plus one; every launch runs all kGrid workgroups once, so the
// counts advance in lockstep and all workgroups of a launch see the same
// value.  epoch = count + 1 (32-bit, never 0, so zeroed words never match,
// and consecutive launches differ); activation words carry the 16-bit tag
// epoch % 65535 + 1 (never 0; every launch rewrites every word it reads, so
// a word's previous tag is the previous launch's).
//
// Replaces the decode sequence of src/lfm.rs:967-1011 (router_addnorm_route,
// gemv_gather_act, gemv_gather_down_combine4).
#include <atomic>

#include "mh_device.hpp"
#include "mh_host.hpp"
#include "mh_route.hpp"

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr uint32_t kGrid = 256;
constexpr uint32_t kReplicas = 8;   // logit copies, one per XCD
constexpr int kPollWave = 1;        // polls the logits (wave 0 has the router row's stores in flight)
// scratch layout (u32 words)
constexpr uint32_t kEpochWords = 0;       // [kGrid] launch counts (word 256: the three-launch path's counter)
constexpr uint32_t kLogitWords = 512;     // kReplicas x [kMaxExperts] tagged logits (64-bit)
constexpr uint32_t kLogitStride = 2u * mh::kMaxExperts;
constexpr uint32_t kActWords = kLogitWords + kReplicas * kLogitStride;  // tagged activation triples (64-bit)
constexpr int kMaxTk = 4;
constexpr uint32_t kMaxAct = 8192;  // bf16 activations staged per workgroup (16 KB)
constexpr uint32_t kMaxTriples = ((kMaxAct + 2u) / 3u + 1u) / 2u * 2u;  // ceil(kMaxAct / 3), rounded up to even
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr int kReadsPerThread = (kMaxTriples / 2 + kThreads - 1) / kThreads;  // 16-byte reads
static_assert(kGrid * kWaves <= MH_MOE_DECODE_STAMP_WAVES, "stamp buffer");
static_assert(kMaxTriples % 2 == 0 && 3u * kMaxTriples >= kMaxAct && mh::kMaxExperts <= kGrid &&
                  kActWords + 2u * kMaxTriples <= MH_MOE_DECODE_SCRATCH_WORDS,
              "scratch layout");

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
    uint32_t* scratch;     // launch counts, tagged logits, tagged activation triples
    uint32_t* status;      // device status word (MH_STATUS_*), or null
    uint64_t* stamps;      // per wave kStamps words of phase timestamps (STAMPS kernels only)
    uint32_t E, K, NI, gs;
};

// Phase timestamps (the 100 MHz constant clock) of one launch, written by
// lane 0 of every wave in the STAMPS instantiation only (the product
// instantiation carries no stamp code: even disabled, it measurably changed
// the kernel's schedule): the timeline of the step, summarized by bench.py
// --timeline.
constexpr int kStamps = 10;
enum Stamp {
    ST_START = 0,      // the wave began
    ST_LOGIT = 1,      // router row stored (router waves), the epoch known (others)
    ST_ROUTED = 2,     // the experts chosen
    ST_GU_ISSUED = 3,  // the first triple's gate/up loads issued
    ST_ACT = 4,        // the first triple's activations published
    ST_ACT_LAST = 5,   // the wave's last triple published (waves with two)
    ST_DOWN_ISSUED = 6,
    ST_EXCHANGED = 7,  // the workgroup holds every activation
    ST_OUT = 8,        // the wave's output stored
    ST_XCC = 9         // (a value, not a time) the XCD this workgroup ran on
};

template <bool STAMPS>
__device__ __forceinline__ void stamp(const FusedArgs& a, uint32_t gw, int lane, int which) {
    if constexpr (STAMPS) {
        if (lane == 0) {
            a.stamps[static_cast<size_t>(gw) * kStamps + which] = wall_clock64();
        }
    }
}

__device__ __forceinline__ void put_tagged(uint32_t* scratch, uint32_t word, uint64_t v) {
    __hip_atomic_store(reinterpret_cast<uint64_t*>(scratch) + word, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_tagged(const uint32_t* scratch, uint32_t word) {
    return __hip_atomic_load(reinterpret_cast<const uint64_t*>(scratch) + word, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}

// Three device-coherent 16-byte loads (the same cache policy as the 64-bit
// atomic loads above: sc1) and the wait for them.  Each 64-bit half is
// checked for its tag by the caller, so a half read before its store simply
// fails the check.
__device__ __forceinline__ void load3_coherent(const uint32_t* p0, const uint32_t* p1, const uint32_t* p2,
                                               mh::u32x4& a, mh::u32x4& b, mh::u32x4& c) {
    asm volatile(
        "global_load_dwordx4 %0, %3, off sc1\n\t"
        "global_load_dwordx4 %1, %4, off sc1\n\t"
        "global_load_dwordx4 %2, %5, off sc1\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(a), "=&v"(b), "=&v"(c)
        : "v"(p0), "v"(p1), "v"(p2)
        : "memory");
}

template <typename WT, int TK, int EB, bool STAMPS>
__global__ __launch_bounds__(kThreads) void k_moe_decode_fused(FusedArgs a) {
    static_assert(kReadsPerThread == 3, "load3_coherent covers a thread's share");
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
    uint32_t* const ta = a.scratch + kActWords;    // tagged activation triples

    // ---- phase 1: router logits; row e is computed by wave 0 of workgroup e
    // (e < kMaxExperts <= kGrid).  Wave 0 issues the read of the launch
    // count first and waits for it with the router's loads (loads complete
    // in order), so the two round trips overlap.
    const uint32_t re = blockIdx.x;
    stamp<STAMPS>(a, gw, lane, ST_START);
    if constexpr (STAMPS) {
        if (lane == 0) {
            uint32_t xcc;
            asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
            a.stamps[static_cast<size_t>(gw) * kStamps + ST_XCC] = xcc & 0xfu;
        }
    }
    uint32_t xw[16];
    mh::load_x_words(a.x + 32u * c, xw);
    float bias_r[EB];
#pragma unroll
    for (int j = 0; j < EB; ++j) {
        const uint32_t i = lane + 64u * j;
        bias_r[j] = a.bias != nullptr && i < a.E ? a.bias[i] : 0.0f;
    }
    float logit = 0.0f;
    uint32_t epoch = 0;
    if (wave == 0) {
        uint32_t count;
        asm volatile("global_load_dword %0, %1, off sc1"
                     : "=v"(count)
                     : "v"(a.scratch + kEpochWords + blockIdx.x)
                     : "memory");
        if (re < a.E) {
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
        asm volatile("s_waitcnt vmcnt(0)" : "+v"(count) : : "memory");
        epoch = count + 1u;
    }
    // x and the bias are in registers from here on, before any store: no
    // later use waits again (behind this wave's stores)
    mh::x_words_fence(xw);
#pragma unroll
    for (int j = 0; j < EB; ++j) {
        asm volatile("" : "+v"(bias_r[j]));
    }
    if (threadIdx.x == 0) {
        __hip_atomic_store(a.scratch + kEpochWords + blockIdx.x, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        epoch_l = epoch;
        bad_l = 0u;
    }
    __syncthreads();  // epoch_l
    epoch = epoch_l;
    if (wave == 0 && re < a.E && lane == 60) {
        const uint64_t word = (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(logit);
#pragma unroll
        for (uint32_t rp = 0; rp < kReplicas; ++rp) {
            put_tagged(tl + rp * kLogitStride, re, word);
        }
        a.logits[re] = logit;
    }
    stamp<STAMPS>(a, gw, lane, ST_LOGIT);

    // ---- routing: one wave polls this XCD's copy of the tagged logits into
    // LDS, then every wave chooses the experts itself
    uint32_t ex[TK];
    float exs[TK];     // the chosen experts' scores
    uint32_t exv = 0;  // lane r < TK: ex[r] (read back with a lane-select, not an indexed array)
    if (wave == kPollWave) {
        const uint32_t* rep = tl + (blockIdx.x % kReplicas) * kLogitStride;
        uint32_t pending = 0;
#pragma unroll
        for (int j = 0; j < EB; ++j) {
            pending |= lane + 64u * j < a.E ? 1u << j : 0u;
        }
        uint32_t spins = 0;
        while (__any(pending != 0u) && spins < kSpinLimit) {
#pragma unroll
            for (int j = 0; j < EB; ++j) {
                if ((pending >> j) & 1u) {
                    const uint64_t w = get_tagged(rep, lane + 64u * j);
                    if (static_cast<uint32_t>(w >> 32) == epoch) {
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
    bool ok = bad_l == 0u;
    {
        float sc[EB], cd[EB];
#pragma unroll
        for (int j = 0; j < EB; ++j) {
            const uint32_t i = lane + 64u * j;
            sc[j] = 0.0f;
            cd[j] = -__builtin_inff();
            if (i < a.E) {
                mh::route_score(logit_l[i], bias_r[j], a.mode, sc[j], cd[j]);
            }
        }
        mh::route_select_ids<TK, EB>(sc, cd, ex, exs);
        exv = ex[0];
#pragma unroll
        for (int r = 1; r < TK; ++r) {
            exv = lane == r ? ex[r] : exv;
        }
    }
    stamp<STAMPS>(a, gw, lane, ST_ROUTED);

    // ---- phase 2: gate/up + SwiGLU on triples of activations: triple t is
    // activations 3t .. 3t+2 of the flattened [TK, NI] block (its six rows'
    // dot products share two 4-row butterflies); triples gw, gw + nw, ...
    // A triple's loads go out row by row (codes, scale, bias) and its dots
    // are taken in the same order, so each waits only for its own row.
    const uint32_t acts = TK * a.NI;
    const uint32_t triples = (acts + 2u) / 3u;
    const uint32_t row_bytes = a.K / 2u;
    const uint32_t G = a.K / a.gs;
    const uint32_t gc = (32u * c) / a.gs;
    mh::Chunk<4> ch[6];
    uint16_t sv[6], bv[6];
    auto load_triple = [&](uint32_t t) {
        // activations past the end (last triple) load a valid row and are
        // never stored
        const uint32_t slot0 = (3u * t) / a.NI;
        const uint32_t i0 = 3u * t - slot0 * a.NI;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const bool wrap = i0 + j >= a.NI;
            const bool past = 3u * t + j >= acts;
            const uint32_t slot = past ? slot0 : slot0 + (wrap ? 1u : 0u);
            const uint32_t i = past ? i0 : i0 + j - (wrap ? a.NI : 0u);
            const uint32_t e = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(exv), slot));
            const size_t row = static_cast<size_t>(e) * a.NI + i;
            const size_t sbi = row * G + gc;
            ch[2 * j].load_nt(mh::uniform_ptr(reinterpret_cast<const char*>(a.gc) + row * row_bytes), c * 16u);
            sv[2 * j] = a.gsc[sbi];
            bv[2 * j] = a.gbi[sbi];
            ch[2 * j + 1].load_nt(mh::uniform_ptr(reinterpret_cast<const char*>(a.uc) + row * row_bytes), c * 16u);
            sv[2 * j + 1] = a.usc[sbi];
            bv[2 * j + 1] = a.ubi[sbi];
        }
    };
    uint32_t t = gw;
    if (t < triples) {
        load_triple(t);
    }
    stamp<STAMPS>(a, gw, lane, ST_GU_ISSUED);

    // routing weights, off the gate/up loads' path
    uint32_t wb[TK];
    mh::route_weights_regs<TK>(exs, a.mode, a.eps, wb);
    if (gw == 0 && lane < TK) {
        uint32_t w = wb[0];
#pragma unroll
        for (int r = 1; r < TK; ++r) {
            w = lane == r ? wb[r] : w;
        }
        a.ids[lane] = exv;
        a.weights[lane] = static_cast<uint16_t>(w);
    }

    const uint32_t tag = epoch % 65535u + 1u;
    {
        float xr[32], xs;
        mh::x_words_to_f32(xw, xr, xs);
        mh::q4_scale_x(xr);
        while (t < triples) {
            float h[8];
#pragma unroll
            for (int q = 0; q < 6; ++q) {
                const float d = ch[q].dot(xr);
                const float hv = __builtin_fmaf(mh::bf16_to_f32(sv[q]), d, mh::bf16_to_f32(bv[q]) * xs);
                h[q] = live ? 0.0f + hv : 0.0f;
            }
            h[6] = h[7] = 0.0f;
            const float h0[4] = {h[0], h[1], h[2], h[3]}, h1[4] = {h[4], h[5], h[6], h[7]};
            const int v0 = __float_as_int(mh::reduce_rows4(h0, lane));
            const int v1 = __float_as_int(mh::reduce_rows4(h1, lane));
            // the three SwiGLUs side by side: lane j < 3 takes activation j
            const int g0 = __builtin_amdgcn_readlane(v0, 60), u0 = __builtin_amdgcn_readlane(v0, 61);
            const int g1 = __builtin_amdgcn_readlane(v0, 62), u1 = __builtin_amdgcn_readlane(v0, 63);
            const int g2 = __builtin_amdgcn_readlane(v1, 60), u2 = __builtin_amdgcn_readlane(v1, 61);
            const float g = __int_as_float(lane == 0 ? g0 : lane == 1 ? g1 : g2);
            const float u = __int_as_float(lane == 0 ? u0 : lane == 1 ? u1 : u2);
            const int av = static_cast<int>(mh::f32_to_bf16(mh::silu_bf16(mh::round_bf16(g)) * mh::round_bf16(u)));
            const uint32_t a0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(av, 0));
            const uint32_t a1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(av, 1));
            const uint32_t a2 = static_cast<uint32_t>(__builtin_amdgcn_readlane(av, 2));
            if (lane == 0) {
                put_tagged(ta, t, (static_cast<uint64_t>(a2 | (tag << 16)) << 32) | a0 | (a1 << 16));
                a.act[3u * t] = static_cast<uint16_t>(a0);
                if (3u * t + 1u < acts) {
                    a.act[3u * t + 1u] = static_cast<uint16_t>(a1);
                }
                if (3u * t + 2u < acts) {
                    a.act[3u * t + 2u] = static_cast<uint16_t>(a2);
                }
            }
            stamp<STAMPS>(a, gw, lane, t == gw ? ST_ACT : ST_ACT_LAST);
            t += nw;
            if (t < triples) {
                load_triple(t);
            }
        }
    }

    // ---- this wave's down rows (output gw), loaded once its gate/up rows
    // are in (they are not needed before the activations arrive), used in
    // phase 3
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
    stamp<STAMPS>(a, gw, lane, ST_DOWN_ISSUED);

    // ---- phase 3: once the workgroup's own activations are out, every
    // thread polls its share of the activation words (16 bytes at a time)
    // into LDS, then one down output per wave with the combine.  (The down
    // rows arrive while the words are polled.)  Waves that finish early do
    // not start polling alone: their rounds would only load the memory
    // system the workgroup's remaining gate/up rows are streaming through.
    {
        __syncthreads();
        // thread's 16-byte reads q = threadIdx.x + k * kThreads hold triples
        // 2q and 2q + 1; bit 2k + h of pending: triple 2q + h not yet current
        const uint32_t pairs = (triples + 1u) / 2u;
        uint32_t pending = 0;
        const uint32_t* src[kReadsPerThread];
#pragma unroll
        for (int k = 0; k < kReadsPerThread; ++k) {
            const uint32_t q = threadIdx.x + k * kThreads;
            src[k] = ta + 4u * (q < pairs ? q : 0u);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                pending |= q < pairs && 2u * q + h < triples ? 1u << (2 * k + h) : 0u;
            }
        }
        auto take = [&](const mh::u32x4 (&v)[kReadsPerThread]) {
#pragma unroll
            for (int k = 0; k < kReadsPerThread; ++k) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t lo = h ? v[k].z : v[k].x, hi = h ? v[k].w : v[k].y;
                    if (((pending >> (2 * k + h)) & 1u) && (hi >> 16) == tag) {
                        const uint32_t tr = 2u * (threadIdx.x + k * kThreads) + h;
                        act_l[3u * tr] = static_cast<uint16_t>(lo);
                        if (3u * tr + 1u < acts) {
                            act_l[3u * tr + 1u] = static_cast<uint16_t>(lo >> 16);
                        }
                        if (3u * tr + 2u < acts) {
                            act_l[3u * tr + 2u] = static_cast<uint16_t>(hi);
                        }
                        pending &= ~(1u << (2 * k + h));
                    }
                }
            }
        };
        uint32_t spins = 0;
        while (pending != 0u && spins < kSpinLimit) {
            if (spins != 0u) {
                __builtin_amdgcn_s_sleep(8);  // ~0.25 us: fewer rounds in flight
            }
            mh::u32x4 v[kReadsPerThread];
            load3_coherent(src[0], src[1], src[2], v[0], v[1], v[2]);
            take(v);
            ++spins;
        }
        if (pending != 0u) {
            bad_l = 1u;
        }
        __syncthreads();
        // one thread per 32-activation chunk: f32, odd positions scaled for
        // the Q4 dot, and the chunk sum in the order x_words_to_f32 uses.
        // LDS has 64 banks (256 bytes a cycle, 16 lanes of a 16-byte access):
        // float4 k of chunk j (128 bytes of f32) is stored at slot
        // (k + j / 2) % 8, so the 16 consecutive chunks read by 16 lanes in
        // the waves' down dots below touch 16 distinct bank groups
        const uint32_t chunks = TK * a.NI / 32u;
        if (threadIdx.x < chunks) {
            const uint32_t j = threadIdx.x;
            uint32_t w16[16];
            const uint4* src = reinterpret_cast<const uint4*>(&act_l[32u * j]);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint4 v = src[k];
                w16[4 * k] = v.x; w16[4 * k + 1] = v.y; w16[4 * k + 2] = v.z; w16[4 * k + 3] = v.w;
            }
            float xr[32], xs;
            mh::x_words_to_f32(w16, xr, xs);
            mh::q4_scale_x(xr);
            float4* dst = reinterpret_cast<float4*>(&actf_l[32u * j]);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                dst[(k + (j >> 1)) & 7u] = make_float4(xr[4 * k], xr[4 * k + 1], xr[4 * k + 2], xr[4 * k + 3]);
            }
            xs_l[j] = xs;
        }
        __syncthreads();
        stamp<STAMPS>(a, gw, lane, ST_EXCHANGED);
        ok = ok && bad_l == 0u;
        // an expired wait (logits or activations): NaN outputs, and the
        // status bit the host reads (one store per workgroup)
        if (!ok && threadIdx.x == 0 && a.status != nullptr) {
            __hip_atomic_fetch_or(a.status, MH_STATUS_DECODE_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (has_out) {
            float h[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int r = 0; r < TK; ++r) {
                const uint32_t j = r * CD + cd;  // chunk of slot r read by this lane
                const float4* qv = reinterpret_cast<const float4*>(&actf_l[32u * j]);
                float xr[32];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float4 v = qv[(k + (j >> 1)) & 7u];
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
        stamp<STAMPS>(a, gw, lane, ST_OUT);
    }
}

// Whether one workgroup of this instantiation fits a CU on the current
// device (its registers and LDS), asked once per device: with fewer than one
// resident workgroup per CU the kGrid workgroups would not all run at once
// and the exchange waits could only expire.
constexpr int kOccDevices = 64;
template <typename WT, int TK, int EB, bool ST>
bool fits_one_per_cu() {
    static std::atomic<int> fits[kOccDevices];  // 0 unknown, 1 yes, 2 no
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kOccDevices) {
        return false;
    }
    int f = fits[dev].load(std::memory_order_relaxed);
    if (f == 0) {
        int blocks = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &blocks, reinterpret_cast<const void*>(k_moe_decode_fused<WT, TK, EB, ST>), kThreads, 0);
        f = e == hipSuccess && blocks >= 1 ? 1 : 2;
        fits[dev].store(f, std::memory_order_relaxed);
    }
    return f == 1;
}

template <typename WT, int TK, int EB, bool ST>
int launch_fused(const FusedArgs& a, hipStream_t stream) {
    if (!fits_one_per_cu<WT, TK, EB, ST>()) {
        return MH_ERR_UNSUPPORTED;
    }
    hipLaunchKernelGGL((k_moe_decode_fused<WT, TK, EB, ST>), dim3(kGrid), dim3(kThreads), 0, stream, a);
    return mh::launch_status("k_moe_decode_fused");
}

}  // namespace

namespace mh {

uint32_t moe_decode_fused_waves() { return kGrid * kWaves; }

// Fused decode step; MH_ERR_UNSUPPORTED when the shapes or the device need
// the three-launch path (the caller then uses it).
int moe_decode_fused(const void* router, int router_dtype, const float* bias, int mode, float eps,
                     const mh_quant_weights* gate, const mh_quant_weights* up,
                     const mh_quant_weights* down, uint32_t n_experts, uint32_t topk,
                     const uint16_t* x, uint16_t* out, float* logits, uint32_t* ids,
                     uint16_t* weights, uint16_t* act, uint32_t* scratch, uint64_t* stamps, hipStream_t stream) {
    const uint32_t NI = gate->out_features / n_experts;
    const uint32_t K = gate->in_features;
    // all kGrid workgroups resident (one per CU), one wave per output and
    // per router row, the activations fit the LDS stage
    if (mh::cu_count() < static_cast<int>(kGrid) || K > 2048u || K % 64u != 0 || NI % 64u != 0 ||
        NI > 64u * 32u ||  // a slot's down chunks are one butterfly's lanes (lane = chunk)
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
    a.status = mh::status_word();
    a.stamps = stamps;
    a.E = n_experts; a.K = K; a.NI = NI; a.gs = gate->group_size;
    const bool f32 = router_dtype == MH_DTYPE_F32;
    const bool eb1 = n_experts <= 64u;  // one expert per lane in the routing
#define MH_FUSED_LAUNCH_ST(TK, EB, ST)                                    \
    if (f32) return launch_fused<float, TK, EB, ST>(a, stream);             \
    else return launch_fused<uint16_t, TK, EB, ST>(a, stream);
#define MH_FUSED_LAUNCH_EB(TK, EB)          \
    if (stamps) { MH_FUSED_LAUNCH_ST(TK, EB, true) } \
    else { MH_FUSED_LAUNCH_ST(TK, EB, false) }
#define MH_FUSED_LAUNCH(TK)            \
    if (eb1) { MH_FUSED_LAUNCH_EB(TK, 1) } \
    else { MH_FUSED_LAUNCH_EB(TK, 4) }
    switch (topk) {
        case 1: MH_FUSED_LAUNCH(1)
        case 2: MH_FUSED_LAUNCH(2)
        case 3: MH_FUSED_LAUNCH(3)
        default: MH_FUSED_LAUNCH(4)
    }
#undef MH_FUSED_LAUNCH_ST
#undef MH_FUSED_LAUNCH_EB
#undef MH_FUSED_LAUNCH
}

}  // namespace mh

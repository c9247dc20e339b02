// gemv.hip -- decode GEMVs over MLX affine Q4/Q6 weights for gfx950.
//
// Layout of the work: one wave64 owns R consecutive rows at a time and one
// 32-code chunk per lane (a K=2048 Q4 row is 64 lanes x 16 B, one coalesced
// dwordx4 per lane; a Q6 row is 64 lanes x 24 B).  Codes are dequantized in
// registers, products accumulate in f32 with fma in the chunk order (see
// mh_device.hpp), and the row value is the wave's xor-butterfly.  No MFMA:
// the path is HBM-bound at batch 1.  Waves loop over row groups with the next
// group's loads issued before the current group's arithmetic.
//
// Replaces lfm.metal:100-297 (GEMV_Q4_BODY, lfm_gemv_q4_bf16[_k*],
// lfm_gemv_q6_bf16[_x4]) and :1113-1386 (argmax, head argmax, token tail).
#include <mutex>

#include "mh_device.hpp"
#include "mh_host.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / mh::kWave;
constexpr int kXPitch = 36;  // LDS floats per staged x chunk (32 + 4: no bank conflicts)
constexpr uint32_t kArgSlots = MH_ARGMAX_SLOTS;
constexpr uint32_t kSpinLimit = 1u << 24;  // bound of the collector's wait for one slot
#ifndef MH_ROWS_GRID_CAP
#define MH_ROWS_GRID_CAP MH_ARGMAX_SLOTS
#endif
constexpr uint32_t kRowsGridCap = MH_ROWS_GRID_CAP;  // batch-1 GEMV workgroups (<= the finisher's slots)
static_assert(kRowsGridCap <= kArgSlots, "one finisher slot per workgroup");

struct GemvArgs {
    const uint32_t* codes;
    const uint16_t* scales;
    const uint16_t* biases;
    const uint16_t* x;          // bf16 [batch, k]
    uint16_t* y;                // bf16 [batch, n] or null
    unsigned long long* best;   // [batch] keys (reference head argmax), or null
    unsigned long long* slots;  // [batch][kArgSlots] finisher scratch, or null
    uint32_t* ids;              // [batch] tokens written by the finisher
    unsigned long long* launches;  // the finisher's launch count (after the slots), or null
    uint32_t* status;           // device status word (MH_STATUS_*), or null
    uint64_t* stamps;           // per wave MH_GEMV_STAMPS phase words (stamped kernels only)
    uint32_t n, k, gs, row_words, groups;
};

// Phase timestamps of the batch-1 head (the 100 MHz constant clock), lane 0
// of every wave, stamped instantiation only.
enum GemvStamp {
    GS_START = 0,      // the wave began
    GS_ISSUED = 1,     // its block's loads (and wave 0's count read) issued
    GS_X = 2,          // x converted and shared (after the workgroup barrier)
    GS_ROWS = 3,       // the block's row values computed and stored
    GS_KEYS = 4,       // the workgroup's wave keys in the LDS (after its barrier)
    GS_PUBLISHED = 5,  // wave 0: the workgroup's key published (not the collector)
    GS_COLLECTED = 6,  // collector workgroup: every slot read, the ids written
    GS_XCC = 7         // the XCD the workgroup ran on
};
static_assert(GS_XCC + 1 == MH_GEMV_STAMPS, "stamp words");

template <bool ST>
__device__ __forceinline__ void gemv_stamp(const GemvArgs& a, uint32_t gw, int lane, int which) {
    if constexpr (ST) {
        if (lane == 0) {
            a.stamps[static_cast<size_t>(gw) * MH_GEMV_STAMPS + which] = wall_clock64();
        }
    }
}

__device__ __forceinline__ unsigned long long amax(unsigned long long* p, unsigned long long v) {
    return __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Atomic max that first reads the word and skips the atomic when it already
// holds a key >= v (it only grows, so the result is the same).  Device-scope
// atomics on one word serialize (~12 ns each); most workgroups finish after
// a greater key is in and issue none.
__device__ __forceinline__ void amax_if_greater(unsigned long long* p, unsigned long long v) {
    if (v > __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
        amax(p, v);
    }
}

// Argmax epilogue with the finisher.  Keys are published by "units" (waves
// of the batch-1 kernel, workgroups of the staged kernel) into their own
// slots, so no two units contend on one address.  The last workgroup of the
// grid is dispatched after all others have started, so its wait for their
// slots ends; it reduces the slots with its own units' keys, writes the token
// ids, re-zeroes the slots and counts the launch.
//
// A slot holds the unit's key for this launch as a 48-bit key (the bf16
// logit's 16-bit orderable value above ~index: the argmax runs over bf16
// values, whose orderable f32 word has a constant low half) under a 16-bit
// tag derived from the launch count (the scratch word after the slots, read
// at kernel start and bumped by the collector at its end).  The collector
// accepts only slots that carry this launch's tag, so a key that a unit of an
// earlier launch wrote before that launch's collector gave up is never taken
// for a later launch's, and a zero slot (tag 0) is never a key.
//
// A unit that reads the count only after the collector gave up and bumped it
// (it started that late) publishes under the next launch's tag, which no tag
// can tell apart.  So a collector whose wait expired also sets kPoison in the
// count word: the next launch's collector then treats its own result as lost
// too (ids 0xffffffff, MH_STATUS_ARGMAX_WAIT), re-zeroes every slot and
// clears the bit.  Stream order ends every unit of a launch before the next
// launch starts, so a launch after that one is clean again.
constexpr unsigned long long kPoison = 1ull << 63;

__device__ __forceinline__ unsigned long long launch_tag(unsigned long long launches) {
    return ((launches & ~kPoison) % 0xffffull + 1ull) << 48;
}

__device__ __forceinline__ unsigned long long key48(unsigned long long key64) {
    return ((key64 >> 48) << 32) | (key64 & 0xffffffffull);
}

constexpr unsigned long long kTagMask = 0xffff000000000000ull;

__device__ __forceinline__ void publish_key(const GemvArgs& a, uint32_t b, uint32_t unit, unsigned long long tag,
                                            unsigned long long key) {
    __hip_atomic_store(a.slots + static_cast<size_t>(b) * kArgSlots + unit, tag | key48(key), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// The launch count, read by every workgroup of a finisher launch before it
// publishes (the collector only bumps it after every unit has published).
__device__ __forceinline__ unsigned long long read_launches(const GemvArgs& a) {
    return a.launches != nullptr ? __hip_atomic_load(a.launches, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
}

// The same where a.launches is never null (the batch-1 kernel's argmax
// launches): no branch, so the load's wait falls where the value is used
// instead of at a merge right after it.
// The address goes through an opaque register so the value stays a vector
// register: a uniform load is moved to scalar registers right after it, which
// waits for every load issued before it.
__device__ __forceinline__ unsigned long long read_launches_nn(const GemvArgs& a) {
    return __hip_atomic_load(a.launches + mh::opaque(0u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Run by the whole collector workgroup.  own[b]: the collector's own key.
// Each thread reads its slots together; the ones without this launch's tag
// (their unit has not published yet) are read again together until they
// carry it.
template <int B>
__device__ void collect_keys(const GemvArgs& a, uint32_t n_units, const unsigned long long* own,
                             unsigned long long launches) {
    __shared__ unsigned long long sk[kWaves];
    constexpr int kPer = kArgSlots / kThreads;  // slots per collector thread
    static_assert(kPer <= 32, "pending mask is 32 bits");
    const int lane = threadIdx.x & (mh::kWave - 1), wave = threadIdx.x / mh::kWave;
    const unsigned long long tag = launch_tag(launches);
    const bool poisoned = (launches & kPoison) != 0ull;
    bool expired = false;  // uniform: some row's wait expired in this launch
    for (int b = 0; b < B; ++b) {
        unsigned long long* sl = a.slots + static_cast<size_t>(b) * kArgSlots + threadIdx.x;
        unsigned long long v[kPer];
        uint32_t pend = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const bool mine = threadIdx.x + j * kThreads < n_units;
            v[j] = mine ? __hip_atomic_load(sl + j * kThreads, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : tag;
            pend |= ((v[j] & kTagMask) != tag ? 1u : 0u) << j;
        }
        uint32_t spins = 0;
        while (pend != 0u && ++spins < kSpinLimit) {
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int j = 0; j < kPer; ++j) {
                if ((pend >> j) & 1u) {
                    v[j] = __hip_atomic_load(sl + j * kThreads, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
#pragma unroll
            for (int j = 0; j < kPer; ++j) {
                if ((v[j] & kTagMask) == tag) {
                    pend &= ~(1u << j);
                }
            }
        }
        const bool lost = pend != 0u;
        unsigned long long m = 0;
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            if (threadIdx.x + j * kThreads < n_units) {
                const unsigned long long k = (v[j] & kTagMask) == tag ? v[j] & ~kTagMask : 0ull;
                m = k > m ? k : m;
                __hip_atomic_store(sl + j * kThreads, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        m = mh::wave_max_u64(m);
        const bool row_expired = __syncthreads_or(lost) != 0;
        expired = expired || row_expired;
        const bool any_lost = row_expired || poisoned;
        if (any_lost && threadIdx.x == 0 && a.status != nullptr) {
            __hip_atomic_fetch_or(a.status, MH_STATUS_ARGMAX_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (lane == 0) {
            sk[wave] = m;
        }
        __syncthreads();
        // wave 0: the waves' maxima and the collector's own key
        if (wave == 0) {
            const unsigned long long t = mh::wave_max_u64(
                lane < kWaves ? sk[lane < kWaves ? lane : 0] : (lane == kWaves ? key48(own[b]) : 0ull));
            if (lane == 0) {
                a.ids[b] = any_lost ? 0xffffffffu : ~static_cast<uint32_t>(t & 0xffffffffull);
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0 && a.launches != nullptr) {
        __hip_atomic_store(a.launches, ((launches & ~kPoison) + 1ull) | (expired ? kPoison : 0ull), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Workgroup argmax of the staged kernel: waves' (bv, bi) per batch row merged
// in LDS; then one atomic max per workgroup into best[b] (the reference's
// gemv_head_argmax) or the finisher's slots.
template <int B>
__device__ void finish_argmax(const GemvArgs& a, const float (&bv)[B], const uint32_t (&bi)[B],
                              int lane, int wave, unsigned long long launches) {
    __shared__ float sv[kWaves][B];
    __shared__ uint32_t si[kWaves][B];
    __shared__ unsigned long long own[B];
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            sv[wave][b] = bv[b];
            si[wave][b] = bi[b];
        }
    }
    __syncthreads();
    unsigned long long key = 0;
    if (threadIdx.x < B) {
        const int b = threadIdx.x;
        float v = sv[0][b];
        uint32_t i = si[0][b];
        for (int w = 1; w < kWaves; ++w) {
            mh::argmax_merge(v, i, sv[w][b], si[w][b]);
        }
        key = mh::argmax_key(v, i);
    }
    if (a.slots == nullptr) {
        if (threadIdx.x < B) {
            amax_if_greater(a.best + threadIdx.x, key);
        }
        return;
    }
    const uint32_t last = gridDim.x - 1;
    if (blockIdx.x != last) {
        if (threadIdx.x < B) {
            publish_key(a, threadIdx.x, blockIdx.x, launch_tag(launches), key);
        }
        return;
    }
    if (threadIdx.x < B) {
        own[threadIdx.x] = key;
    }
    __syncthreads();
    collect_keys<B>(a, last, own, launches);
}

// Key of the wave's argmax over per-lane bests (bv, bi) kept by argmax_merge:
// the greatest value (NaN never wins, -0 == +0), ties to the lowest index;
// with no non-NaN candidate the serial scan's (-inf, 0).
__device__ __forceinline__ unsigned long long wave_argmax_key(float bv, uint32_t bi) {
    const float m = mh::wave_max_f32(bv);
    if (m != m) {
        return mh::argmax_key(-__builtin_inff(), 0u);
    }
    const uint32_t i = mh::wave_min_u32(bv == m ? bi : 0xffffffffu);
    return mh::argmax_key(m, i);
}

// Rows of the batch-1 kernel: each wave owns blocks of kBlockRows consecutive
// rows; lane c owns chunk c of every row (K <= 2048).
constexpr int kBlockRows = 8;
constexpr int kGroupRows = 4;
constexpr int kMaxGroups = 64;  // K / group size <= 2048 / 32

// Batch 1, K <= 2048, even K / group size.  Each wave owns blocks of
// kBlockRows consecutive rows (one block per wave up to kArgSlots
// workgroups).  Per block: the scales and biases are read with a few wide
// loads and staged in LDS as f32 (scale, bias) pairs; the codes of the
// block's two row groups are loaded non-temporally (each byte is read once)
// and computed one group after the other.  x is converted once per
// workgroup: wave 0 turns its chunk words into the f32 values the chunk dots
// take (odd positions times 1/16 for Q4) and the ascending chunk sums, and
// the other waves read them from LDS after one barrier.  Each lane's eight
// row values go to LDS as [row][chunk]; lane 8r + j then reads chunks
// 8j .. 8j + 7 of row r and adds them as the chunk order's butterfly does
// (pairs, quads, octets: levels 1-3), and levels 4-6 (chunks xor 8, 16,
// 32) are the lane pairs j ^ 1, j ^ 2 (quad_perm) and j ^ 4 (row_shr:4),
// leaving row r's sum in lane 8r + 7.  Adding +0 to that sum instead of to
// every lane's value gives the same bits: an IEEE sum is -0 only when both
// operands are -0, so zero signs change nothing else in the tree.
// FAST: K == 2048, group size 64 and N a multiple of kBlockRows (every lane
// owns a chunk, 32 groups per row, no partial block).  ARGMAX: per-lane
// bests, a DPP wave argmax, then the finisher (or the reference's atomic
// max).  WV: waves per workgroup (2 only without the argmax, whose
// publication and collector take 4).  ST: phase timestamps (measurement).
// The Q4 head (FAST, ARGMAX, two groups) is held to five workgroups per CU:
// 94 VGPRs instead of 99 (no spills), so five waves share a SIMD instead of
// four and 1280 of its 2048 workgroups start at once (26 KB of LDS each).
// The Q6 head spills at that bound and keeps four.
template <int BITS, bool FAST, bool ARGMAX, int NG, int WV = kWaves, bool ST = false>
__global__ __launch_bounds__(kThreads, (BITS == 4 && FAST && ARGMAX && NG == 2) ? 5 : 1) void k_gemv_rows(GemvArgs a) {
    static_assert(NG == 1 || NG == 2, "one or two 4-row groups per block");
    static_assert(WV == kWaves || (WV == 2 && !ARGMAX), "two-wave workgroups only without the argmax");
    constexpr int R = kGroupRows, BR = NG * R;
    constexpr int GM = FAST ? 32 : kMaxGroups;     // staged groups per row
    constexpr int NSB = BR * GM / 128;              // scale / bias word loads per lane
    __shared__ uint4 sbl[kWaves][BR * GM / 2];      // (s, b) f32 pairs of groups 2i, 2i + 1
    __shared__ float tl[kWaves][kBlockRows * 64];   // the block's lane values, [row][chunk]
    __shared__ float xl[64 * kXPitch];              // x as the chunk dots take it
    __shared__ float xsl[64];                       // ascending sums of the x chunks
    const int lane = threadIdx.x & (mh::kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / mh::kWave);
    const uint32_t C = a.k / 32u;
    const uint32_t N = a.n;
    const uint32_t G = FAST ? 32u : a.groups;
    const bool live = FAST || lane < static_cast<int>(C);
    const uint32_t c = live ? lane : 0u;
    const uint32_t code_off = c * BITS * 4u;
    const uint32_t gc = FAST ? static_cast<uint32_t>(lane) / 2u : (32u * c) / a.gs;
    const uint32_t row_bytes = FAST ? 2048u * BITS / 8u : a.row_words * 4u;
    const uint32_t n_blocks = (N + BR - 1) / BR;
    const uint32_t stride = gridDim.x * WV;
    const uint32_t gw = blockIdx.x * WV + wave;
    gemv_stamp<ST>(a, gw, lane, GS_START);
    if constexpr (ST) {
        if (lane == 0) {
            uint32_t xcc;
            asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
            a.stamps[static_cast<size_t>(gw) * MH_GEMV_STAMPS + GS_XCC] = xcc & 0xfu;
        }
    }

    uint32_t xw[16];
    if (wave == 0) {
        mh::load_x_words(a.x + 32u * c, xw);
    }
    uint32_t sw[NSB], bw[NSB];
    mh::Chunk<BITS> A[R], Bc[R];  // Bc: NG == 2 only
    // a block's scale / bias words (clamped indices: every lane loads) and
    // its groups of codes
    auto issue = [&](uint32_t blk) {
        const uint32_t row0 = blk * BR;
        const uint32_t nrows = FAST ? static_cast<uint32_t>(BR) : min(static_cast<uint32_t>(BR), N - row0);
        const uint32_t nd = nrows * G / 2u;
        const uint32_t* s2 = reinterpret_cast<const uint32_t*>(a.scales + static_cast<size_t>(row0) * G);
        const uint32_t* b2 = reinterpret_cast<const uint32_t*>(a.biases + static_cast<size_t>(row0) * G);
#pragma unroll
        for (int j = 0; j < NSB; ++j) {
            const uint32_t i = lane + mh::kWave * j;
            const uint32_t ic = FAST || i < nd ? i : nd - 1u;
            sw[j] = s2[ic];
            bw[j] = b2[ic];
        }
        const char* codes = reinterpret_cast<const char*>(a.codes) + static_cast<size_t>(row0) * row_bytes;
#pragma unroll
        for (int r = 0; r < NG * R; ++r) {
            const uint32_t rr = FAST ? r : min(static_cast<uint32_t>(r), nrows - 1u);
            (r < R ? A[r] : Bc[r - R]).load_nt(mh::uniform_ptr(codes + rr * row_bytes), code_off);
        }
    };
    // the first block's loads go out unconditionally (a wave past the last
    // block re-reads it; only the last workgroup can have one), so that no
    // path without them meets the x conversion's wait
    const uint32_t blk0 = blockIdx.x * WV + wave;
    issue(min(blk0, n_blocks - 1u));
    // the launch count behind the block's loads, needed only at the end and
    // only by wave 0 (the publisher; it hands the count to the collector's
    // other waves through the LDS): one device-coherent read of the word per
    // workgroup, not per wave
    asm volatile("" ::: "memory");
    unsigned long long launches = ARGMAX && wave == 0 ? read_launches_nn(a) : 0ull;
    gemv_stamp<ST>(a, gw, lane, GS_ISSUED);

    // x: wave 0 converts, every wave reads after the barrier
    float xr[32];
    float xs = 0.0f;
    if (wave == 0) {
        mh::x_words_fence(xw);
        mh::x_words_to_f32(xw, xr, xs);
        if (BITS == 4) {
            mh::q4_scale_x(xr);
        } else {
            mh::q6_scale_x(xr);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            *reinterpret_cast<float4*>(xl + lane * kXPitch + 4 * q) =
                make_float4(xr[4 * q], xr[4 * q + 1], xr[4 * q + 2], xr[4 * q + 3]);
        }
        xsl[lane] = xs;
    }
    // LDS writes done, then the barrier; the asm's memory clobber keeps the
    // reads below it (the code loads above stay in flight)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (wave != 0) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 v = *reinterpret_cast<const float4*>(xl + lane * kXPitch + 4 * q);
            xr[4 * q] = v.x; xr[4 * q + 1] = v.y; xr[4 * q + 2] = v.z; xr[4 * q + 3] = v.w;
        }
        xs = xsl[lane];
    }
    gemv_stamp<ST>(a, gw, lane, GS_X);

    uint4* sb = sbl[wave];
    float* tw = tl[wave];
    float lbv = -__builtin_inff();  // per-lane best of the rows this lane stored
    uint32_t lbi = 0u;
    // one block from the loaded words: stage (s, b), both groups, the row sums
    auto process = [&](uint32_t blk) {
        const uint32_t row0 = blk * BR;
        const uint32_t nrows = FAST ? static_cast<uint32_t>(BR) : min(static_cast<uint32_t>(BR), N - row0);
        // (s, b) as f32 bits: word i holds groups 2i (low halves) and 2i + 1
#pragma unroll
        for (int j = 0; j < NSB; ++j) {
            const uint32_t i = lane + mh::kWave * j;
            sb[i] = make_uint4(sw[j] << 16, bw[j] << 16, sw[j] & 0xffff0000u, bw[j] & 0xffff0000u);
        }
        const uint2* sbp = reinterpret_cast<const uint2*>(sb);
        auto compute = [&](int grp, const mh::Chunk<BITS>(&ch)[R]) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t rr = FAST ? grp * R + r : min(static_cast<uint32_t>(grp * R + r), nrows - 1u);
                const uint2 w = sbp[rr * G + gc];
                float p;
                if constexpr (BITS == 6) {
                    p = ch[r].dot_s(xr);  // x scaled by q6_scale_x above
                } else {
                    p = ch[r].dot(xr);
                }
                const float hv = __builtin_fmaf(__uint_as_float(w.x), p, __uint_as_float(w.y) * xs);
                tw[(grp * R + r) * 64 + lane] = live ? hv : 0.0f;
            }
        };
        compute(0, A);
        if constexpr (NG == 2) {
            compute(1, Bc);
        }
        __builtin_amdgcn_wave_barrier();
        // lane 8r + j: chunks 8j .. 8j + 7 of row r (rows past the block's
        // NG * 4 hold stale values and are never emitted)
        const float4 t0 = *reinterpret_cast<const float4*>(tw + 8 * lane);
        const float4 t1 = *reinterpret_cast<const float4*>(tw + 8 * lane + 4);
        float v = ((t0.x + t0.y) + (t0.z + t0.w)) + ((t1.x + t1.y) + (t1.z + t1.w));
        v = v + mh::qmove<0xB1>(v);             // chunks xor 8  (quad_perm 1,0,3,2)
        v = v + mh::qmove<0x4E>(v);             // chunks xor 16 (quad_perm 2,3,0,1)
        v = v + mh::dpp_move<0x114, 0xf>(v);    // chunks xor 32 (row_shr:4; lanes 8r+4..7)
        __builtin_amdgcn_wave_barrier();
        const uint32_t r = static_cast<uint32_t>(lane) >> 3;
        if ((lane & 7) == 7 && r < nrows) {
            const uint16_t yb = mh::f32_to_bf16(v + 0.0f);
            if (a.y != nullptr) {
                a.y[row0 + r] = yb;
            }
            if (ARGMAX) {
                mh::argmax_merge(lbv, lbi, mh::bf16_to_f32(yb), row0 + r);
            }
        }
    };
    if (blk0 < n_blocks) {
        process(blk0);
    }
    // later rounds (more blocks than the grid has waves)
    for (uint32_t blk = blk0 + stride; blk < n_blocks; blk += stride) {
        issue(blk);
        process(blk);
    }
    gemv_stamp<ST>(a, gw, lane, GS_ROWS);
    if (!ARGMAX) {
        return;
    }
    // workgroup key: the waves' keys, maxed by wave 0 (one publication or
    // atomic per workgroup)
    const unsigned long long key = wave_argmax_key(lbv, lbi);
    __shared__ unsigned long long wk[kWaves];
    __shared__ unsigned long long own[2];  // the collector's own key, the launch count
    if (lane == 0) {
        wk[wave] = key;
    }
    __syncthreads();
    gemv_stamp<ST>(a, gw, lane, GS_KEYS);
    const uint32_t last = gridDim.x - 1;
    if (wave == 0) {
        const unsigned long long t = mh::wave_max_u64(lane < kWaves ? wk[lane < kWaves ? lane : 0] : 0ull);
        if (lane == 0) {
            if (a.slots == nullptr) {
                amax_if_greater(a.best, t);
            } else if (blockIdx.x != last) {
                publish_key(a, 0, blockIdx.x, launch_tag(launches), t);
            } else {
                own[0] = t;
                own[1] = launches;
            }
        }
        if (blockIdx.x != last) {
            gemv_stamp<ST>(a, gw, lane, GS_PUBLISHED);
        }
    }
    if (a.slots == nullptr || blockIdx.x != last) {
        return;
    }
    __syncthreads();
    launches = own[1];
    collect_keys<1>(a, last, own, launches);
    gemv_stamp<ST>(a, gw, lane, GS_COLLECTED);
}

// Row values (wave-uniform) of one row group of the staged kernel: store and
// argmax.
template <int B, int R>
__device__ __forceinline__ void emit_rows(const GemvArgs& a, uint32_t rg, const float (&v)[R][B],
                                          float (&bv)[B], uint32_t (&bi)[B], int lane) {
    const uint32_t N = a.n;
#pragma unroll
    for (int b = 0; b < B; ++b) {
        uint16_t mine = 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint16_t vb = mh::f32_to_bf16(v[r][b]);
            const uint32_t row = rg * R + r;
            if (lane == r) {
                mine = vb;
            }
            if (row < N) {
                mh::argmax_merge(bv[b], bi[b], mh::bf16_to_f32(vb), row);
            }
        }
        const uint32_t my_row = rg * R + lane;
        if (a.y != nullptr && lane < R && my_row < N) {
            a.y[static_cast<size_t>(b) * N + my_row] = mine;
        }
    }
}

template <int BITS>
__device__ __forceinline__ void load_row_chunk(const GemvArgs& a, uint32_t row, uint32_t c,
                                               mh::Chunk<BITS>& ch, float& s, float& b) {
    ch.load(a.codes + static_cast<size_t>(row) * a.row_words + static_cast<size_t>(c) * BITS);
    const uint32_t g = (32u * c) / a.gs;
    s = mh::bf16_to_f32(a.scales[static_cast<size_t>(row) * a.groups + g]);
    b = mh::bf16_to_f32(a.biases[static_cast<size_t>(row) * a.groups + g]);
}

// General form: any K, batch 1..8.  x is staged in LDS, one padded 32-float
// slot per (batch, chunk); lanes walk chunks c = lane, lane + 64, ...
template <int BITS, int B, int R>
__global__ __launch_bounds__(kThreads) void k_gemv_staged(GemvArgs a) {
    extern __shared__ float lds[];
    const int lane = threadIdx.x & (mh::kWave - 1);
    const int wave = threadIdx.x / mh::kWave;
    const uint32_t C = a.k / 32u;
    const uint32_t N = a.n;
    float* xl = lds;                                          // [B*C][kXPitch]
    float* xsl = lds + static_cast<size_t>(B) * C * kXPitch;  // [B*C]
    const unsigned long long launches = read_launches(a);

    for (uint32_t t = threadIdx.x; t < B * C; t += kThreads) {
        const uint32_t b = t / C, c = t % C;
        float xc[32], s;
        mh::load_x_chunk(a.x + static_cast<size_t>(b) * a.k + 32u * c, xc, s);
        if (BITS == 4) {
            mh::q4_scale_x(xc);
        }
        float4* dst = reinterpret_cast<float4*>(xl + static_cast<size_t>(t) * kXPitch);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            dst[q] = make_float4(xc[4 * q], xc[4 * q + 1], xc[4 * q + 2], xc[4 * q + 3]);
        }
        xsl[t] = s;
    }
    __syncthreads();

    float bv[B];
    uint32_t bi[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        bv[b] = -__builtin_inff();
        bi[b] = 0u;
    }
    const uint32_t n_rg = (N + R - 1) / R;
    const uint32_t stride = gridDim.x * kWaves;
    for (uint32_t rg = blockIdx.x * kWaves + wave; rg < n_rg; rg += stride) {
        float acc[R][B];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                acc[r][b] = 0.0f;
            }
        }
        for (uint32_t c = lane; c < C; c += mh::kWave) {
            mh::Chunk<BITS> ch[R];
            float s[R], bb[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t row = min(rg * R + r, N - 1);
                load_row_chunk<BITS>(a, row, c, ch[r], s[r], bb[r]);
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                float xc[32];
                const float4* src =
                    reinterpret_cast<const float4*>(xl + (static_cast<size_t>(b) * C + c) * kXPitch);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float4 v = src[q];
                    xc[4 * q] = v.x;
                    xc[4 * q + 1] = v.y;
                    xc[4 * q + 2] = v.z;
                    xc[4 * q + 3] = v.w;
                }
                const float xs = xsl[static_cast<size_t>(b) * C + c];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float p = ch[r].dot(xc);
                    acc[r][b] = acc[r][b] + __builtin_fmaf(s[r], p, bb[r] * xs);
                }
            }
        }
        float v[R][B];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int b = 0; b < B; ++b) {
                v[r][b] = mh::lane63(mh::wave_sum_lane63(acc[r][b]));
            }
        }
        emit_rows<B, R>(a, rg, v, bv, bi, lane);
    }
    if (a.best != nullptr || a.slots != nullptr) {
        finish_argmax<B>(a, bv, bi, lane, wave, launches);
    }
}

constexpr int kWgPerCu = 4;

template <typename K>
int launch(K kernel, const GemvArgs& a, uint32_t grid, size_t lds, hipStream_t stream,
           const char* name, uint32_t threads = kThreads) {
    if (lds > 64u * 1024u) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 static_cast<int>(lds));
        if (e != hipSuccess) {
            return mh::hip_error(e, name);
        }
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(threads), lds, stream, a);
    return mh::launch_status(name);
}

// Workgroups for `units` wave-sized work items, capped by `cap`.
uint32_t grid_for(uint32_t units, uint32_t cap) {
    const uint32_t want = (units + kWaves - 1) / kWaves;
    return want < cap ? want : cap;
}

// Batch 1 with K > 2048 (the dense FFN down, K = 11776), no argmax: R rows
// per workgroup, the row's chunks split across the workgroup's waves in
// slabs of 64 (slab s: chunks 64 s + lane), so every wave holds little and
// the whole matrix is in flight at once.  Each chunk value h_c goes to LDS;
// then wave r sums row r's lane l values h_l, h_{l+64}, ... in ascending slab
// order from +0 and takes the xor butterfly: the chunk order exactly.
constexpr int kSplitRows = 4;
constexpr int kSplitSlabs = 16;  // K <= 16 * 64 * 32 = 32768

constexpr int kSplitWaves = 8;

template <int BITS>
__global__ __launch_bounds__(kSplitWaves * 64) void k_gemv_splitk(GemvArgs a) {
    constexpr int R = kSplitRows;
    __shared__ float hs[R][kSplitSlabs][mh::kWave];
    const int lane = threadIdx.x & (mh::kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / mh::kWave);
    const uint32_t N = a.n, C = a.k / 32u;
    const uint32_t S = (C + mh::kWave - 1) / mh::kWave;
    const uint32_t row0 = blockIdx.x * R;
    for (uint32_t sl = wave; sl < S; sl += kSplitWaves) {
        const uint32_t c = sl * mh::kWave + lane;
        const bool live = c < C;
        const uint32_t cc = live ? c : 0u;
        mh::Chunk<BITS> ch[R];
        float sc[R], bi[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = min(row0 + r, N - 1u);
            load_row_chunk<BITS>(a, row, cc, ch[r], sc[r], bi[r]);
        }
        float xr[32], xs;
        mh::load_x_chunk(a.x + 32u * cc, xr, xs);
        if (BITS == 4) {
            mh::q4_scale_x(xr);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float p = ch[r].dot(xr);
            hs[r][sl][lane] = live ? __builtin_fmaf(sc[r], p, bi[r] * xs) : 0.0f;
        }
    }
    __syncthreads();
    if (wave < R && row0 + wave < N) {
        float v = 0.0f;
        for (uint32_t sl = 0; sl < S; ++sl) {
            v = v + hs[wave][sl][lane];
        }
        v = mh::lane63(mh::wave_sum_lane63(v));
        if (lane == 0) {
            a.y[row0 + wave] = mh::f32_to_bf16(v);
        }
    }
}

template <int BITS>
int launch_splitk(const GemvArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(k_gemv_splitk<BITS>, dim3((a.n + kSplitRows - 1) / kSplitRows), dim3(kSplitWaves * 64), 0,
                       stream, a);
    return mh::launch_status("k_gemv_splitk");
}

template <int BITS, int B, int R>
int launch_staged(const GemvArgs& a, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(B) * (a.k / 32u) * (kXPitch + 1) * sizeof(float);
    uint32_t cap = static_cast<uint32_t>(mh::cu_count()) * kWgPerCu;
    cap = cap < kArgSlots ? cap : kArgSlots;
    return launch(k_gemv_staged<BITS, B, R>, a, grid_for((a.n + R - 1) / R, cap), lds, stream,
                  "k_gemv_staged");
}

template <int BITS, bool ARGMAX>
int launch_rows(const GemvArgs& a, hipStream_t stream) {
    // one block per wave while the finisher has a slot for every workgroup
    // (the hardware keeps as many workgroups resident as registers allow);
    // beyond that the waves loop over blocks.  Matrices with fewer 8-row
    // blocks than the chip has SIMDs x 4 take 4-row blocks: twice the waves,
    // half the serial arithmetic per wave (latency-bound sizes).
    const uint32_t blocks8 = (a.n + kBlockRows - 1) / kBlockRows;
    const bool small = blocks8 < static_cast<uint32_t>(mh::cu_count()) * 4u * kWaves;
    const bool fast = a.k == 2048u && a.gs == 64u && a.n % (small ? kGroupRows : kBlockRows) == 0u;
    if (small) {
        // between one and four 4-row blocks per CU (no argmax): two-wave
        // workgroups, so the blocks spread over twice the CUs (2048 x 2048:
        // 3.17 -> 3.08 us; fewer or more blocks measured slower that way)
        const uint32_t units = (a.n + kGroupRows - 1) / kGroupRows;
        const uint32_t cus = static_cast<uint32_t>(mh::cu_count());
        if constexpr (!ARGMAX) {
            if (units >= cus && units <= 4u * cus) {
                const uint32_t want = (units + 1u) / 2u;
                const uint32_t grid = want < kRowsGridCap ? want : kRowsGridCap;
                return fast ? launch(k_gemv_rows<BITS, true, false, 1, 2>, a, grid, 0, stream, "k_gemv_rows", 128u)
                            : launch(k_gemv_rows<BITS, false, false, 1, 2>, a, grid, 0, stream, "k_gemv_rows", 128u);
            }
        }
        const uint32_t grid = grid_for(units, kRowsGridCap);
        return fast ? launch(k_gemv_rows<BITS, true, ARGMAX, 1>, a, grid, 0, stream, "k_gemv_rows")
                    : launch(k_gemv_rows<BITS, false, ARGMAX, 1>, a, grid, 0, stream, "k_gemv_rows");
    }
    const uint32_t grid = grid_for(blocks8, kRowsGridCap);
    return fast ? launch(k_gemv_rows<BITS, true, ARGMAX, 2>, a, grid, 0, stream, "k_gemv_rows")
                : launch(k_gemv_rows<BITS, false, ARGMAX, 2>, a, grid, 0, stream, "k_gemv_rows");
}

// The stamped head: batch 1 with the finisher, only where launch_rows takes
// k_gemv_rows<BITS, true, true, 2> (K 2048, group 64, N a multiple of 8 and
// at least the chip's SIMDs x 32 rows, at most one block per wave).
template <int BITS>
int launch_rows_stamped(const GemvArgs& a, hipStream_t stream) {
    const uint32_t blocks8 = (a.n + kBlockRows - 1) / kBlockRows;
    const bool small = blocks8 < static_cast<uint32_t>(mh::cu_count()) * 4u * kWaves;
    const bool fast = a.k == 2048u && a.gs == 64u && a.n % kBlockRows == 0u;
    if (small || !fast || blocks8 > kRowsGridCap * kWaves) {
        return MH_ERR_UNSUPPORTED;
    }
    return launch(k_gemv_rows<BITS, true, true, 2, kWaves, true>, a, grid_for(blocks8, kRowsGridCap), 0, stream,
                  "k_gemv_rows");
}

template <int BITS>
int dispatch_gemv(const GemvArgs& a, uint32_t batch, hipStream_t stream) {
    switch (batch) {
        case 1:
            if (a.k <= 2048u && a.groups <= static_cast<uint32_t>(kMaxGroups) && (a.groups & 1u) == 0u) {
                return (a.best != nullptr || a.slots != nullptr) ? launch_rows<BITS, true>(a, stream)
                                                                 : launch_rows<BITS, false>(a, stream);
            }
            if (a.best == nullptr && a.slots == nullptr && a.y != nullptr &&
                a.k <= 32u * mh::kWave * kSplitSlabs) {
                return launch_splitk<BITS>(a, stream);
            }
            return launch_staged<BITS, 1, 4>(a, stream);
        case 2: return launch_staged<BITS, 2, 2>(a, stream);
        case 3: return launch_staged<BITS, 3, 2>(a, stream);
        case 4: return launch_staged<BITS, 4, 2>(a, stream);
        case 5: return launch_staged<BITS, 5, 2>(a, stream);
        case 6: return launch_staged<BITS, 6, 2>(a, stream);
        case 7: return launch_staged<BITS, 7, 2>(a, stream);
        case 8: return launch_staged<BITS, 8, 2>(a, stream);
        default: return mh::set_error(MH_ERR_UNSUPPORTED, "gemv: batch %u not in 1..8", batch);
    }
}

// Largest LDS request of the staged path: B * C * (kXPitch + 1) floats.
constexpr size_t kMaxLds = 160u * 1024u;

int gemv_common(const char* op, const mh_quant_weights* w, const uint16_t* x, uint16_t* y,
                uint64_t* best, bool finisher, uint32_t* ids, uint32_t batch,
                mh_stream_t stream, uint64_t* stamps = nullptr) {
    MH_TRY(mh::check_quant(w, op));
    MH_ENSURE(x != nullptr, MH_ERR_INVALID, "%s: x is NULL", op);
    MH_ENSURE(batch >= 1 && batch <= 8, MH_ERR_UNSUPPORTED, "%s: batch %u not in 1..8", op, batch);
    MH_ENSURE(mh::aligned(x, 2) && (y == nullptr || mh::aligned(y, 2)), MH_ERR_ALIGN,
              "%s: x/y not 2-byte aligned", op);
    MH_ENSURE(best == nullptr || mh::aligned(best, 8), MH_ERR_ALIGN,
              "%s: argmax key not 8-byte aligned", op);
    MH_ENSURE(!finisher || (best != nullptr && ids != nullptr), MH_ERR_INVALID,
              "%s: the argmax finisher needs the scratch and ids", op);
    MH_ENSURE(ids == nullptr || mh::aligned(ids, 4), MH_ERR_ALIGN, "%s: ids not 4-byte aligned", op);
    const uint32_t C = w->in_features / 32u;
    const bool xreg = batch == 1 && w->in_features <= 2048u;
    MH_ENSURE(xreg || static_cast<size_t>(batch) * C * (kXPitch + 1) * 4 <= kMaxLds,
              MH_ERR_UNSUPPORTED, "%s: batch %u x in_features %u exceeds the LDS staging", op,
              batch, w->in_features);
    GemvArgs a{};
    a.codes = w->codes;
    a.scales = w->scales;
    a.biases = w->biases;
    a.x = x;
    a.y = y;
    a.best = finisher ? nullptr : reinterpret_cast<unsigned long long*>(best);
    a.slots = finisher ? reinterpret_cast<unsigned long long*>(best) : nullptr;
    a.ids = ids;
    a.n = w->out_features;
    a.k = w->in_features;
    a.gs = w->group_size;
    a.row_words = w->in_features * w->bits / 32u;
    a.groups = w->in_features / w->group_size;
    // the count word of a finisher launch; in the atomic-max mode (whose
    // kernels read it but never use it) a readable word: the keys
    a.launches = finisher ? reinterpret_cast<unsigned long long*>(best) + static_cast<size_t>(batch) * kArgSlots
                          : reinterpret_cast<unsigned long long*>(best);
    a.status = mh::status_word();
    const hipStream_t s = mh::as_stream(stream);
    if (stamps != nullptr) {
        a.stamps = stamps;
        int rc = MH_ERR_UNSUPPORTED;
        if (batch == 1u) {
            rc = w->bits == 4 ? launch_rows_stamped<4>(a, s) : w->bits == 6 ? launch_rows_stamped<6>(a, s)
                                                                             : MH_ERR_UNSUPPORTED;
        } else if (batch == 8u) {
            rc = mh::gemv_mfma(w, x, y, best, ids, batch, s, stamps);
        }
        MH_ENSURE(rc != MH_ERR_UNSUPPORTED, MH_ERR_UNSUPPORTED,
                  "%s: batch %u, %u x %u Q%u is not a measured head shape", op, batch, w->out_features,
                  w->in_features, w->bits);
        return rc;
    }
    // batch > 1 without the reference's atomic-max key: the matrix-core
    // kernel where its shape limits allow
    if (batch > 1 && (finisher || best == nullptr)) {
        const int rc = mh::gemv_mfma(w, x, y, finisher ? best : nullptr, ids, batch, s);
        if (rc != MH_ERR_UNSUPPORTED) {
            return rc;
        }
    }
    return w->bits == 4 ? dispatch_gemv<4>(a, batch, s) : dispatch_gemv<6>(a, batch, s);
}

// ------------------------------------------------------------- dequant ---

template <int BITS>
// Thread t dequantizes chunk t of the [n, C] chunks, whose 32 values are
// out[32 t .. 32 t + 31]: a wave's 64 chunks are 4 KB contiguous, which a
// full wave passes through the LDS so that each store instruction writes
// 1 KB contiguous (16 bytes per lane at a 64-byte stride otherwise).
__global__ __launch_bounds__(256) void k_dequant(const uint32_t* codes, const uint16_t* scales,
                                                 const uint16_t* biases, uint16_t* out,
                                                 uint32_t n, uint32_t k, uint32_t gs) {
    __shared__ uint4 tr[4][4 * 64];  // per wave: its 16-byte pieces in output order
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t C = k / 32u;
    const size_t total = static_cast<size_t>(n) * C;
    const uint32_t row_words = k * BITS / 32u;
    const uint32_t groups = k / gs;
    for (size_t t = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const uint32_t row = static_cast<uint32_t>(t / C);
        const uint32_t c = static_cast<uint32_t>(t % C);
        mh::Chunk<BITS> ch;
        ch.load(codes + static_cast<size_t>(row) * row_words + static_cast<size_t>(c) * BITS);
        const uint32_t g = 32u * c / gs;
        const float s = mh::bf16_to_f32(scales[static_cast<size_t>(row) * groups + g]);
        const float b = mh::bf16_to_f32(biases[static_cast<size_t>(row) * groups + g]);
        uint32_t packed[16];
        mh::dequant_chunk<BITS>(ch.w, s, b, packed);
        const size_t t0 = t - lane;
        if (t0 + 64u <= total) {  // uniform: a full wave
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                tr[wave][4u * lane + q] = make_uint4(packed[4 * q], packed[4 * q + 1], packed[4 * q + 2], packed[4 * q + 3]);
            }
            __builtin_amdgcn_wave_barrier();
            uint4* base = reinterpret_cast<uint4*>(out + 32u * t0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                base[64u * j + lane] = tr[wave][64u * j + lane];
            }
            __builtin_amdgcn_wave_barrier();  // the next round's writes after these reads
            continue;
        }
        uint4* dst = reinterpret_cast<uint4*>(out + static_cast<size_t>(row) * k + 32u * c);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            dst[q] = make_uint4(packed[4 * q], packed[4 * q + 1], packed[4 * q + 2], packed[4 * q + 3]);
        }
    }
}

int dequant_common(const char* op, const mh_quant_weights* w, uint16_t* out, mh_stream_t stream) {
    MH_TRY(mh::check_quant_dequant(w, op));
    MH_ENSURE(out != nullptr, MH_ERR_INVALID, "%s: out is NULL", op);
    MH_ENSURE(mh::aligned(out, 16), MH_ERR_ALIGN, "%s: out not 16-byte aligned", op);
    const size_t total = static_cast<size_t>(w->out_features) * (w->in_features / 32u);
    const size_t want = (total + 255) / 256;
    const size_t cap = static_cast<size_t>(mh::cu_count()) * 16;
    const unsigned grid = static_cast<unsigned>(want < cap ? want : cap);
    const hipStream_t s = mh::as_stream(stream);
    if (w->bits == 4) {
        hipLaunchKernelGGL(k_dequant<4>, dim3(grid), dim3(256), 0, s, w->codes, w->scales,
                           w->biases, out, w->out_features, w->in_features, w->group_size);
    } else if (w->bits == 8) {
        hipLaunchKernelGGL(k_dequant<8>, dim3(grid), dim3(256), 0, s, w->codes, w->scales,
                           w->biases, out, w->out_features, w->in_features, w->group_size);
    } else {
        hipLaunchKernelGGL(k_dequant<6>, dim3(grid), dim3(256), 0, s, w->codes, w->scales,
                           w->biases, out, w->out_features, w->in_features, w->group_size);
    }
    return mh::launch_status(op);
}

// ----------------------------------------------------------- token tail ---

__global__ void k_token_tail(unsigned long long* best, uint32_t* out_tok, uint32_t batch) {
    const uint32_t b = threadIdx.x;
    if (b < batch) {
        const unsigned long long key = best[b];
        best[b] = 0ull;
        out_tok[b] = ~static_cast<uint32_t>(key & 0xffffffffull);
    }
}

// --------------------------------------------------- two-stage argmax ---

constexpr int kArgmaxGroups = 64;

struct ArgPair {
    float v;
    uint32_t i;
};

__device__ void block_argmax(float& bv, uint32_t& bi) {
    __shared__ float sv[256 / mh::kWave];
    __shared__ uint32_t si[256 / mh::kWave];
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t oi = __shfl_xor(bi, off);
        mh::argmax_merge(bv, bi, ov, oi);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < static_cast<int>(blockDim.x / mh::kWave); ++w) {
            mh::argmax_merge(bv, bi, sv[w], si[w]);
        }
    }
}

__global__ __launch_bounds__(256) void k_argmax_partial(const uint16_t* x, ArgPair* partials,
                                                        uint32_t n, uint32_t chunk) {
    float bv = -__builtin_inff();
    uint32_t bi = 0;
    const uint32_t begin = blockIdx.x * chunk;
    const uint32_t end = min(begin + chunk, n);
    for (uint32_t i = begin + threadIdx.x; i < end; i += blockDim.x) {
        mh::argmax_merge(bv, bi, mh::bf16_to_f32(x[i]), i);
    }
    block_argmax(bv, bi);
    if (threadIdx.x == 0) {
        partials[blockIdx.x].v = bv;
        partials[blockIdx.x].i = bi;
    }
}

__global__ __launch_bounds__(256) void k_argmax_final(const ArgPair* partials, uint32_t* out,
                                                      uint32_t groups) {
    float bv = -__builtin_inff();
    uint32_t bi = 0;
    for (uint32_t g = threadIdx.x; g < groups; g += blockDim.x) {
        mh::argmax_merge(bv, bi, partials[g].v, partials[g].i);
    }
    block_argmax(bv, bi);
    if (threadIdx.x == 0) {
        out[0] = bi;
    }
}

// ------------------------------------------------------ no-alloc head ---
// The finisher scratch of mh_gemv_quant_argmax_noalloc: one array per device
// (each device holds its own copy until the process ends).  Host code never
// uses this name as an address: it uses the pointer hipGetSymbolAddress
// returns for the current device (the name is a host-side stand-in).
constexpr uint32_t kNoAllocMaxBatch = 8;
static __device__ __align__(256) unsigned long long scratch[MH_ARGMAX_SCRATCH_WORDS(kNoAllocMaxBatch)];

constexpr int kNoAllocDevices = 64;
std::mutex g_noalloc_mu;
unsigned long long* g_noalloc_ptr[kNoAllocDevices];  // per device, under g_noalloc_mu

// The current device's scratch address; on the first call on a device it is
// resolved and zeroed (a fill kernel on `stream`, ordered before the call's
// own launch).  Nothing is allocated.
int noalloc_scratch(unsigned long long** out, mh_stream_t stream) {
    int dev = 0;
    const hipError_t ge = hipGetDevice(&dev);
    if (ge != hipSuccess) {
        return mh::hip_error(ge, "hipGetDevice");
    }
    MH_ENSURE(dev >= 0 && dev < kNoAllocDevices, MH_ERR_UNSUPPORTED,
              "mh_gemv_quant_argmax_noalloc: device %d beyond the %d this library tracks", dev, kNoAllocDevices);
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (g_noalloc_ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) {
            return mh::hip_error(e, "hipGetSymbolAddress(scratch)");
        }
        MH_ENSURE(p != nullptr, MH_ERR_RUNTIME, "hipGetSymbolAddress(scratch) returned NULL");
        MH_TRY(mh_zero(p, sizeof(scratch), stream));
        g_noalloc_ptr[dev] = static_cast<unsigned long long*>(p);
    }
    *out = g_noalloc_ptr[dev];
    return MH_OK;
}

}  // namespace

extern "C" {

int mh_gemv_quant_argmax_noalloc(const mh_quant_weights* w, const uint16_t* x, uint16_t* y, uint32_t* ids,
                                 uint32_t batch, mh_stream_t stream) {
    MH_ENSURE(ids != nullptr, MH_ERR_INVALID, "mh_gemv_quant_argmax_noalloc: ids is NULL");
    MH_ENSURE(batch >= 1 && batch <= kNoAllocMaxBatch, MH_ERR_INVALID,
              "mh_gemv_quant_argmax_noalloc: batch %u exceeds the library's scratch (batch 1..%u)", batch,
              kNoAllocMaxBatch);
    MH_TRY(mh::check_quant(w, "mh_gemv_quant_argmax_noalloc"));
    MH_ENSURE(x != nullptr, MH_ERR_INVALID, "mh_gemv_quant_argmax_noalloc: x is NULL");
    unsigned long long* ws = nullptr;
    MH_TRY(noalloc_scratch(&ws, stream));
    return gemv_common("mh_gemv_quant_argmax_noalloc", w, x, y, reinterpret_cast<uint64_t*>(ws), true, ids, batch,
                       stream);
}

int mh_gemv_quant(const mh_quant_weights* w, const uint16_t* x, uint16_t* y, uint32_t batch,
                  mh_stream_t stream) {
    MH_ENSURE(y != nullptr, MH_ERR_INVALID, "mh_gemv_quant: y is NULL");
    return gemv_common("mh_gemv_quant", w, x, y, nullptr, false, nullptr, batch, stream);
}

int mh_gemv_head_argmax(const mh_quant_weights* w, const uint16_t* x, uint64_t* best,
                        uint32_t batch, mh_stream_t stream) {
    MH_ENSURE(best != nullptr, MH_ERR_INVALID, "mh_gemv_head_argmax: best is NULL");
    return gemv_common("mh_gemv_head_argmax", w, x, nullptr, best, false, nullptr, batch,
                       stream);
}

int mh_gemv_quant_argmax(const mh_quant_weights* w, const uint16_t* x, uint16_t* y,
                         uint64_t* scratch, uint32_t* ids, uint32_t batch, mh_stream_t stream) {
    MH_ENSURE(scratch != nullptr && ids != nullptr, MH_ERR_INVALID,
              "mh_gemv_quant_argmax: scratch/ids is NULL");
    return gemv_common("mh_gemv_quant_argmax", w, x, y, scratch, true, ids, batch, stream);
}

int mh_gemv_quant_argmax_stamped(const mh_quant_weights* w, const uint16_t* x, uint16_t* y, uint64_t* scratch,
                                 uint32_t* ids, uint32_t batch, uint64_t* stamps, mh_stream_t stream) {
    const char* op = "mh_gemv_quant_argmax_stamped";
    MH_ENSURE(scratch != nullptr && ids != nullptr, MH_ERR_INVALID, "%s: scratch/ids is NULL", op);
    MH_ENSURE(stamps != nullptr && mh::aligned(stamps, 8), MH_ERR_INVALID, "%s: stamps NULL or not 8-byte aligned",
              op);
    MH_ENSURE(batch == 1u || batch == 8u, MH_ERR_UNSUPPORTED, "%s: batch %u (1 or 8)", op, batch);
    return gemv_common(op, w, x, y, scratch, true, ids, batch, stream, stamps);
}

int mh_token_tail(uint64_t* best, uint32_t* out_tok, uint32_t batch, mh_stream_t stream) {
    MH_ENSURE(best != nullptr && out_tok != nullptr, MH_ERR_INVALID,
              "mh_token_tail: best/out_tok is NULL");
    MH_ENSURE(mh::aligned(best, 8), MH_ERR_ALIGN, "mh_token_tail: key not 8-byte aligned");
    MH_ENSURE(batch >= 1 && batch <= 64, MH_ERR_INVALID, "mh_token_tail: batch %u not in 1..64",
              batch);
    hipLaunchKernelGGL(k_token_tail, dim3(1), dim3(64), 0, mh::as_stream(stream),
                       reinterpret_cast<unsigned long long*>(best), out_tok, batch);
    return mh::launch_status("mh_token_tail");
}

int mh_argmax_bf16(const uint16_t* x, uint32_t n, void* partials, uint32_t* out,
                   mh_stream_t stream) {
    MH_ENSURE(x && partials && out, MH_ERR_INVALID, "mh_argmax_bf16: NULL argument");
    MH_ENSURE(n > 0, MH_ERR_INVALID, "mh_argmax_bf16: empty input");
    MH_ENSURE(mh::aligned(partials, 8), MH_ERR_ALIGN, "mh_argmax_bf16: partials not 8-byte aligned");
    const uint32_t chunk = (n + kArgmaxGroups - 1) / kArgmaxGroups;
    const hipStream_t s = mh::as_stream(stream);
    hipLaunchKernelGGL(k_argmax_partial, dim3(kArgmaxGroups), dim3(256), 0, s, x,
                       static_cast<ArgPair*>(partials), n, chunk);
    MH_TRY(mh::launch_status("k_argmax_partial"));
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s,
                       static_cast<const ArgPair*>(partials), out,
                       static_cast<uint32_t>(kArgmaxGroups));
    return mh::launch_status("k_argmax_final");
}

int mh_dequant_to_bf16(const mh_quant_weights* w, uint16_t* out, mh_stream_t stream) {
    return dequant_common("mh_dequant_to_bf16", w, out, stream);
}

int mh_dequant_q4_bf16_bulk(const mh_quant_weights* w, uint16_t* out, mh_stream_t stream) {
    MH_ENSURE(w != nullptr && w->bits == 4 && w->in_features % 128 == 0, MH_ERR_INVALID,
              "mh_dequant_q4_bf16_bulk: bulk dequant needs 4-bit weights with K %% 128 == 0");
    return dequant_common("mh_dequant_q4_bf16_bulk", w, out, stream);
}

}  // extern "C"

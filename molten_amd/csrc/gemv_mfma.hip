// gemv_mfma.hip -- the quantized head GEMV for 2..8 rows of x on the matrix
// cores (src/kernels/quant.rs gemv / gemv_head_argmax at batch > 1).
//
// A row's codes are widened to bf16 as q + 128 (exact: the bf16 with bits
// 0x4300 | q), x stays bf16, and v_mfma_f32_16x16x32_bf16 forms the exact
// products and sums each 64-code group in f32; then, per group,
//     y += s * P_g + (b - 128 s) * X_g,   P_g = sum (q + 128) x,  X_g = sum x.
// The logits agree with the chunk-order oracle to f32 rounding, not bit for
// bit.  The argmax stays exact: every row value v carries a bound E with
// |v - v_chunk| <= E (v_chunk: the chunk-order value), the rows whose upper
// bound can reach the greatest lower bound (in bf16, the argmax's domain)
// are kept as candidates, and the last workgroup recomputes them in chunk
// order and takes the reference's key (value desc, index asc).
//
// Tiles of 16 rows x all of K per wave.  MFMA operand layout (16x16x32):
// lane l holds A row l % 16 and B column l % 16, k = 8 (l / 16) .. + 8; the
// result rows 4 (l / 16) .. + 4 of column l % 16.  The k order inside a
// group is permuted so that lane quarter q owns the 16 consecutive codes
// 16q .. 16q + 15 of the group (step t of the group uses codes 16q + 8t ..
// + 8): its codes are one contiguous 12-byte (Q6) or 8-byte (Q4) piece, and
// x is staged in LDS in the same order.  The B columns are the batch rows
// (columns >= batch are zero).
#include "mh_device.hpp"
#include "mh_host.hpp"

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr uint32_t kGrid = 256;
constexpr int kTileRows = 16;
constexpr int kStageGroups = 8;  // groups of 64 codes per pipeline stage
constexpr int kDepth = 2;        // stages in the pipeline (even: LDS regions alternate); one ahead
                                 // measured fastest: more loads in flight only queue behind each other
constexpr uint32_t kMaxK = 2048;
constexpr uint32_t kMaxG = kMaxK / 64;
constexpr int kMaxB = 8;
constexpr int kSlotWords = 6;  // per (batch row, workgroup): lower bound, dropped bound, 4 candidates
constexpr int kPerKind = kGrid / 64;  // a finisher lane's words of one kind (word kind * kGrid + workgroup)
constexpr int kCand = 4;
constexpr int kRecompute = 4;  // rows whose chunk-order values the finisher forms per round of loads
constexpr uint32_t kArgSlots = MH_ARGMAX_SLOTS;
constexpr uint32_t kMaxCand = kTileRows * 68;  // finisher's candidate list (a wave's stage buffer)
constexpr uint32_t kSpinLimit = 1u << 24;
static_assert(kGrid * kSlotWords <= kArgSlots && kGrid % 64 == 0, "finisher slots");
static_assert(kGrid * kCand <= kMaxCand, "candidate list");
// a stage's scales / biases are read by all 64 lanes: row l / 4, groups
// 2 (l % 4) and 2 (l % 4) + 1 -- exactly 16 rows x 8 groups
static_assert(kStageGroups == 8 && kTileRows == 16, "scale / bias staging covers 16 rows x 8 groups");

struct MfmaArgs {
    const char* codes;
    const uint16_t* scales;
    const uint16_t* biases;
    const uint16_t* x;          // [batch, K] bf16, 16-byte aligned
    uint16_t* y;                // [batch, N] bf16, or null
    unsigned long long* slots;  // [batch][kArgSlots] finisher scratch, or null (no argmax)
    uint32_t* ids;              // [batch]
    uint32_t* status;           // device status word (MH_STATUS_*), or null
    uint64_t* stamps;           // per wave MH_GEMV_STAMPS phase words (stamped kernels only)
    uint32_t n, k, groups, row_bytes;
};

// Phase timestamps (the 100 MHz constant clock), lane 0 of every wave,
// stamped instantiation only.
enum MfmaStamp {
    MS_START = 0,      // the wave began
    MS_X = 1,          // x, its group sums and sum |x| in the LDS (the barrier after them)
    MS_LOOP = 2,       // the wave's main loop (its tiles) done
    MS_SUMMARY = 3,    // waves b < B: batch row b's summary published (or kept, the finisher)
    MS_WORDS = 4,      // finisher wave b: every workgroup's words read
    MS_ID = 5,         // finisher wave b: batch row b's id written
    MS_CAND = 6,       // finisher wave b: the rows recomputed in chunk order (a count)
    MS_XCC = 7         // the XCD the workgroup ran on
};
static_assert(MS_XCC + 1 == MH_GEMV_STAMPS, "stamp words");

template <bool ST>
__device__ __forceinline__ void mfma_stamp(const MfmaArgs& a, uint32_t gw, int lane, int which) {
    if constexpr (ST) {
        if (lane == 0) {
            a.stamps[static_cast<size_t>(gw) * MH_GEMV_STAMPS + which] = wall_clock64();
        }
    }
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// A bf16(q + 128) pair from a field t holding the low code at bit 0 and the
// high code at bit S: (((t << (16 - S)) | t) & M) | 0x43004300, M = the two
// code masks.  Written as two instructions (v_lshl_or_b32, v_and_or_b32) so
// that the compiler cannot split them into more; the exponent word lives in
// a VGPR (a VOP3 reads at most one SGPR on this target).
template <int SH>
__device__ __forceinline__ uint32_t bf16_pair(uint32_t t, uint32_t m, uint32_t e) {
    uint32_t u, o;
    asm("v_lshl_or_b32 %0, %1, %2, %1" : "=v"(u) : "v"(t), "n"(SH));
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(o) : "v"(u), "s"(m), "v"(e));
    return o;
}

// Codes of one lane for one group (16 codes) and their bf16(q + 128) pairs.
template <int BITS>
struct Piece;
template <>
struct Piece<6> {
    uint32_t w[3];
    __device__ __forceinline__ void read(const uint32_t* l) {  // LDS, 4-byte aligned
        w[0] = l[0];
        w[1] = l[1];
        w[2] = l[2];
    }
    // pair j: the 12-bit field 12 j .. 12 j + 11 (codes 2j, 2j + 1); a field's
    // bits 16..21 must be clear (they would reach the high code), the rest
    // above bit 11 is masked off
    __device__ __forceinline__ void widen(uint32_t (&o)[8], uint32_t e) const {
        uint32_t t[8];
        t[0] = w[0] & 0xfffu;
        t[1] = __builtin_amdgcn_ubfe(w[0], 12, 12);
        t[2] = __builtin_amdgcn_perm(w[1], w[0], 0x0c0c0403u);  // bytes w0.3, w1.0, 0, 0
        t[3] = __builtin_amdgcn_ubfe(w[1], 4, 12);
        t[4] = __builtin_amdgcn_ubfe(w[1], 16, 12);
        t[5] = __builtin_amdgcn_alignbit(w[2], w[1], 28) & 0xfffu;
        t[6] = __builtin_amdgcn_ubfe(w[2], 8, 12);
        t[7] = w[2] >> 20;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            o[j] = bf16_pair<10>(t[j], 0x003f003fu, e);
        }
    }
};
template <>
struct Piece<4> {
    uint32_t w[2];
    __device__ __forceinline__ void read(const uint32_t* l) {  // LDS, 8-byte aligned
        w[0] = l[0];
        w[1] = l[1];
    }
    // pair j: byte j (codes 2j, 2j + 1 are its low and high nibble)
    __device__ __forceinline__ void widen(uint32_t (&o)[8], uint32_t e) const {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            o[j] = bf16_pair<12>(__builtin_amdgcn_ubfe(w[j >> 2], 8 * (j & 3), 8), 0x000f000fu, e);
        }
    }
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const mh::u32x4 v = {a, b, c, d};
    return __builtin_bit_cast(bf16x8, v);
}

// Value of an argmax_key (its high word), the inverse of the orderable map
// (a select, no branch).
__device__ __forceinline__ float key_value(unsigned long long key) {
    const uint32_t o = static_cast<uint32_t>(key >> 32);
    const uint32_t neg = static_cast<uint32_t>(static_cast<int32_t>(o) >> 31);  // all ones if the value is >= +0
    return __uint_as_float((o & 0x7fffffffu & neg) | (~o & ~neg));
}

// A word a workgroup publishes for the finisher: an argmax_key's high word
// (the orderable value), then the launch's 8-bit tag and 24 low bits (~row
// of a candidate, rows < 2^24; 0 for none; all ones for a bound).  The
// finisher takes only words with its launch's tag, so neither a word an
// earlier launch's workgroup wrote late (after that finisher's wait expired)
// nor leftover scratch contents are read as this launch's (consecutive
// launches differ in tag).
constexpr uint32_t kRowMask = 0xffffffu;
__device__ __forceinline__ unsigned long long pack_word(unsigned long long key, uint32_t tag, uint32_t low24) {
    return (key & 0xffffffff00000000ull) | (tag << 24) | low24;
}
__device__ __forceinline__ uint32_t word_tag(unsigned long long w) { return static_cast<uint32_t>(w) >> 24; }

// Chunk-order values of U rows for one batch row (the staged kernel's
// formula: lane c owns chunk c, K <= 2048): the exact values the argmax is
// taken on.  Every row's loads go out before the first dot.
template <int BITS, int U>
__device__ void chunk_values(const MfmaArgs& a, const uint32_t (&rows)[U], const float (&xr)[32], float xs,
                             bool live, uint32_t c, float (&out)[U], uint32_t cnt = U) {
    mh::Chunk<BITS> ch[U];
    float s[U], b[U];
    const uint32_t g = (32u * c) / 64u;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        ch[u].load(reinterpret_cast<const uint32_t*>(a.codes + static_cast<size_t>(rows[u]) * a.row_bytes) + c * BITS);
        s[u] = mh::bf16_to_f32(a.scales[static_cast<size_t>(rows[u]) * a.groups + g]);
        b[u] = mh::bf16_to_f32(a.biases[static_cast<size_t>(rows[u]) * a.groups + g]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        out[u] = 0.0f;
        if (static_cast<uint32_t>(u) < cnt) {  // uniform: rows past cnt repeat the last one
            const float p = ch[u].dot(xr);
            const float acc = live ? 0.0f + __builtin_fmaf(s[u], p, b[u] * xs) : 0.0f;
            out[u] = mh::lane63(mh::wave_sum_lane63(acc));
        }
    }
}

// A stage of a tile: 16 rows x kStageGroups groups of codes, loaded with
// contiguous 16-byte pieces (lane and load i take piece 64 i + lane, row =
// piece / RP), staged in the wave's LDS rows (stride: conflict-free reads of
// the lanes' pieces), read back as (row l % 16, piece 16 codes of quarter
// l / 16).
template <int BITS>
struct StageShape {
    static constexpr int kRowBytes = kStageGroups * 64 * BITS / 8;      // 384 (Q6), 256 (Q4)
    static constexpr int kRowPieces = kRowBytes / 16;
    static constexpr int kLoads = kTileRows * kRowPieces / 64;          // 6, 4
    static constexpr int kStrideWords = BITS == 6 ? 100 : 68;           // LDS row stride
};

template <int BITS, int B, bool ST = false>
__global__ __launch_bounds__(kThreads) void k_gemv_mfma(MfmaArgs a) {
    constexpr int PW = BITS == 6 ? 12 : 8;  // bytes of a lane's piece of a group
    using SS = StageShape<BITS>;
    __shared__ __attribute__((aligned(16))) uint32_t stg[kWaves][kTileRows * SS::kStrideWords];
    __shared__ __attribute__((aligned(16))) mh::u32x4 xl[kMaxG * 2 * 4 * 16];  // x in B-operand order, 16 columns
    __shared__ float xg[kMaxG * 16];                                         // group sums of x, 16 columns
    __shared__ float xga[kMaxG * 16];                                       // group sums of |x|
    __shared__ float xa[B];                                                 // sum |x| per batch row
    __shared__ __attribute__((aligned(16))) float sbl[kWaves][2][2][kStageGroups][kTileRows];  // s, b - 128 s
    __shared__ float mrow[kWaves][2][kTileRows];                            // max |s|, max |b| per row
    __shared__ float m_lb[B][kWaves * 4], m_u1[B][kWaves * 4], m_du[B][kWaves * 4];
    __shared__ uint32_t m_r1[B][kWaves * 4];
    __shared__ unsigned long long own[B][kSlotWords];
    __shared__ uint32_t fin_expired, fin_arrived;  // the finisher waves' expired waits, arrivals

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t gw = blockIdx.x * kWaves + static_cast<uint32_t>(wave);
    mfma_stamp<ST>(a, gw, lane, MS_START);
    if constexpr (ST) {
        if (lane == 0) {
            uint32_t xcc;
            asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
            a.stamps[static_cast<size_t>(gw) * MH_GEMV_STAMPS + MS_XCC] = xcc & 0xfu;
        }
    }
    const uint32_t q = static_cast<uint32_t>(lane) >> 4;  // lane quarter
    const uint32_t n = static_cast<uint32_t>(lane) & 15u;  // B column (batch row)
    const bool col = n < static_cast<uint32_t>(B);
    const uint32_t G = a.groups;
    const uint32_t K = a.k;

    // ---- tiles: stages of kStageGroups groups; the next stage's codes and
    // scales / biases are in flight while a stage is computed (buffers A, B
    // and LDS regions 0, 1 alternate)
    const uint32_t n_st = (G + kStageGroups - 1) / kStageGroups;  // stages per tile
    const uint32_t n_tiles = a.n / kTileRows;
    const uint32_t stride = gridDim.x * kWaves;
    mh::u32x4 pbuf[kDepth][SS::kLoads];         // codes of the stages in flight
    uint32_t svbuf[kDepth], bvbuf[kDepth];        // scales / biases: row l / 4, groups 2 (l % 4) .. + 1
    const uint32_t srow = static_cast<uint32_t>(lane) >> 2, sg = 2u * (static_cast<uint32_t>(lane) & 3u);

    auto issue = [&](uint32_t tile, uint32_t st, mh::u32x4(&p)[SS::kLoads], uint32_t& sv, uint32_t& bv) {
        const uint32_t g0 = st * kStageGroups;
        const mh::gbytes base = mh::uniform_ptr(a.codes + static_cast<size_t>(tile) * kTileRows * a.row_bytes +
                                                st * SS::kRowBytes);
#pragma unroll
        for (int i = 0; i < SS::kLoads; ++i) {
            const uint32_t pc = i * 64u + static_cast<uint32_t>(lane);
            const uint32_t off = (pc / SS::kRowPieces) * a.row_bytes + (pc % SS::kRowPieces) * 16u;
            p[i] = __builtin_nontemporal_load(reinterpret_cast<const __attribute__((address_space(1))) mh::u32x4*>(base + off));
        }
        const size_t sbi = (static_cast<size_t>(tile) * kTileRows + srow) * G + g0 + sg;
        sv = *reinterpret_cast<const uint32_t*>(a.scales + sbi);
        bv = *reinterpret_cast<const uint32_t*>(a.biases + sbi);
    };
    // a stage's scales / biases into LDS as f32 (s, b - 128 s), and the
    // rows' running max |s|, |b| (restarted at a tile's first stage)
    // a stage's scales / biases into LDS as f32 (s, b - 128 s), and the
    // rows' running max |s|, |b| in registers (bits of non-negative floats
    // order as integers; every lane of a row's quad holds its row's maxima),
    // restarted at a tile's first stage
    uint32_t rms = 0u, rmb = 0u;
    auto stage_sb = [&](int region, uint32_t st, uint32_t sv, uint32_t bv) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float s = e ? mh::bf16hi(sv) : mh::bf16lo(sv);
            const float b = e ? mh::bf16hi(bv) : mh::bf16lo(bv);
            sbl[wave][region][0][sg + e][srow] = s;
            sbl[wave][region][1][sg + e][srow] = __builtin_fmaf(-128.0f, s, b);
        }
        uint32_t ms = max((sv << 16) & 0x7fffffffu, sv & 0x7fff0000u);
        uint32_t mb = max((bv << 16) & 0x7fffffffu, bv & 0x7fff0000u);
        // max over the row's four lanes (lanes 4 srow .. + 3): quad_perm 1,0,3,2 and 2,3,0,1
        ms = max(ms, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(ms), 0xB1, 0xf, 0xf, false)));
        mb = max(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0xB1, 0xf, 0xf, false)));
        ms = max(ms, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(ms), 0x4E, 0xf, 0xf, false)));
        mb = max(mb, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(mb), 0x4E, 0xf, 0xf, false)));
        rms = st == 0u ? ms : max(rms, ms);
        rmb = st == 0u ? mb : max(rmb, mb);
    };
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](int region, uint32_t st, const mh::u32x4(&p)[SS::kLoads]) {
        const uint32_t g0 = st * kStageGroups;
        const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
        uint32_t* const sw = stg[wave];
#pragma unroll
        for (int i = 0; i < SS::kLoads; ++i) {
            const uint32_t pc = i * 64u + static_cast<uint32_t>(lane);
            *reinterpret_cast<mh::u32x4*>(sw + (pc / SS::kRowPieces) * SS::kStrideWords + (pc % SS::kRowPieces) * 4u) = p[i];
        }
        const uint32_t* const mine = sw + static_cast<uint32_t>(lane & 15) * SS::kStrideWords + q * (PW / 4);
        const uint32_t kExp = mh::opaque(0x43004300u);  // the exponent word of bf16 128, in a VGPR
        // the stage's group products first (independent: their LDS reads and
        // matrix-core chains overlap), then the per-group scaling in order
        f32x4 pgs[kStageGroups];
#pragma unroll
        for (int g = 0; g < kStageGroups; ++g) {
            const uint32_t ga = g0 + g;
            Piece<BITS> codes;
            codes.read(mine + g * PW);
            uint32_t o[8];
            codes.widen(o, kExp);
            const mh::u32x4 b0 = xl[(ga * 8u + q) * 16u + n];
            const mh::u32x4 b1 = xl[(ga * 8u + 4u + q) * 16u + n];
            f32x4 pg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(o[0], o[1], o[2], o[3]),
                                                               __builtin_bit_cast(bf16x8, b0), zero, 0, 0, 0);
            pgs[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(o[4], o[5], o[6], o[7]),
                                                             __builtin_bit_cast(bf16x8, b1), pg, 0, 0, 0);
        }
#pragma unroll
        for (int g = 0; g < kStageGroups; ++g) {
            const float xgv = xg[(g0 + g) * 16u + n];
            const float4 s4 = *reinterpret_cast<const float4*>(&sbl[wave][region][0][g][4u * q]);
            const float4 b4 = *reinterpret_cast<const float4*>(&sbl[wave][region][1][g][4u * q]);
            acc[0] = __builtin_fmaf(s4.x, pgs[g][0], acc[0]);
            acc[1] = __builtin_fmaf(s4.y, pgs[g][1], acc[1]);
            acc[2] = __builtin_fmaf(s4.z, pgs[g][2], acc[2]);
            acc[3] = __builtin_fmaf(s4.w, pgs[g][3], acc[3]);
            acc[0] = __builtin_fmaf(b4.x, xgv, acc[0]);
            acc[1] = __builtin_fmaf(b4.y, xgv, acc[1]);
            acc[2] = __builtin_fmaf(b4.z, xgv, acc[2]);
            acc[3] = __builtin_fmaf(b4.w, xgv, acc[3]);
        }
    };

    // argmax state of this lane's batch row (lanes with col)
    float lbv = -__builtin_inff();         // greatest bf16 lower bound seen
    float u1 = -__builtin_inff();          // greatest upper bound, its row
    uint32_t r1 = 0xffffffffu;
    float du = -__builtin_inff();          // greatest upper bound of the other rows
    float an = 0.0f;  // sum |x| of batch row n: set once xa is staged (below), before any tile

    // a tile's rows 4q .. 4q + 3 of batch row n: store, bounds, candidates
    auto finish_tile = [&](uint32_t tile) {
        // rows 4q .. 4q + 3 of batch row n
        const uint32_t row0 = tile * kTileRows + 4u * q;
        if (col) {
            uint16_t yb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                yb[i] = mh::f32_to_bf16(acc[i]);
            }
            if (a.y != nullptr) {
                *reinterpret_cast<uint2*>(a.y + static_cast<size_t>(n) * a.n + row0) =
                    make_uint2(yb[0] | (static_cast<uint32_t>(yb[1]) << 16), yb[2] | (static_cast<uint32_t>(yb[3]) << 16));
            }
            if (a.slots != nullptr) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // |acc - chunk value| <= 2^-16 (336 max|s| + 3 max|b|) sum|x|: f32
                    // rounding of both orders (at most 130 and 40 roundings deep,
                    // K <= 2048); 2^-85 covers bf16 / f32 denormals the matrix core
                    // may flush.  e doubles the bound and adds 2^-21 |v| and the
                    // least normal, so fl(v - e) and fl(v + e) bracket the chunk value.
                    const float ms = mrow[wave][0][4u * q + i], mb = mrow[wave][1][4u * q + i];
                    const float v = acc[i];
                    const float e = __builtin_fmaf(__builtin_fmaf(0x1p-15f, an, 0x1p-85f),
                                                   __builtin_fmaf(336.0f, ms, 3.0f * mb),
                                                   __builtin_fmaf(0x1p-21f, fabsf(v), 0x1p-126f));
                    const float lo = v - e, hi = v + e;
                    const uint32_t row = row0 + i;
                    if (!(fabsf(lo) <= 3.0e38f && fabsf(hi) <= 3.0e38f)) {
                        du = __builtin_inff();  // no usable bound: the finisher recomputes every row
                        continue;
                    }
                    lbv = fmaxf(lbv, mh::round_bf16(lo));
                    if (hi > u1 || (hi == u1 && row < r1)) {
                        du = fmaxf(du, u1);
                        u1 = hi;
                        r1 = row;
                    } else {
                        du = fmaxf(du, hi);
                    }
                }
            }
        }
    };

    // the wave's stages in order: stage s is stage s % n_st of its tile
    // s / n_st (tiles first, first + stride, ...); kDepth - 1 stages ahead
    // are in flight
    const uint32_t first = blockIdx.x * kWaves + wave;
    const uint32_t my_tiles = first < n_tiles ? (n_tiles - first + stride - 1) / stride : 0u;
    const uint32_t n_stages = my_tiles * n_st;
    auto tile_of = [&](uint32_t st) { return first + (st / n_st) * stride; };
    // stages past the end reload the wave's last stage (valid addresses, an
    // L2 hit), so every step issues the same loads and the compiler's load
    // counting stays exact across the loop
    const uint32_t last_st = n_stages > 0u ? n_stages - 1u : 0u;
    const uint32_t first_c = first < n_tiles ? first : 0u;
    auto tile_c = [&](uint32_t st) { return n_stages > 0u ? tile_of(st < n_stages ? st : last_st) : first_c; };
    auto stage_c = [&](uint32_t st) { return (st < n_stages ? st : last_st) % n_st; };
    // the launch count (the scratch word after the slots; the finisher bumps
    // it once every workgroup has published), read before x so that the wait
    // for x covers it
    const unsigned long long launches_v =
        a.slots != nullptr
            ? __hip_atomic_load(a.slots + static_cast<size_t>(B) * kArgSlots, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
            : 0ull;
    // ---- x to LDS in operand order (columns >= B zero), clamped addresses.
    // Waves 0..3 stage x (each thread B of its 256 x B live entries, then
    // 16 - B zero entries; groups >= G hold group 0's x and are never read)
    // and issue their first stages' code loads once x has arrived: issued
    // after a wave's code loads, its x would wait behind tens of MB of HBM
    // reads in flight across the chip.  Waves 4..7 issue their first stages
    // at once and take no part in staging x.
    static_assert(kWaves == 8 && kMaxG * 8 * 16 == (kThreads / 2) * 16, "x staged by four waves, 16 entries each");
    const bool xwave = wave < kWaves / 2;
    if (!xwave) {
#pragma unroll
        for (int u = 0; u < kDepth - 1; ++u) {
            issue(tile_c(u), stage_c(u), pbuf[u], svbuf[u], bvbuf[u]);
        }
    } else {
        const uint32_t tx = threadIdx.x;  // 0 .. 255
        mh::u32x4 xv[B];
#pragma unroll
        for (int j = 0; j < B; ++j) {
            const uint32_t L = tx + j * (kThreads / 2u);
            const uint32_t nb = L % static_cast<uint32_t>(B), rest = L / static_cast<uint32_t>(B);
            const uint32_t qq = rest % 4u, t = (rest / 4u) % 2u, g = rest / 8u;
            const uint32_t gcl = g < G ? g : 0u;
            const uint4 v = *reinterpret_cast<const uint4*>(a.x + static_cast<size_t>(nb) * K + 64u * gcl + 16u * qq + 8u * t);
            xv[j] = mh::u32x4{v.x, v.y, v.z, v.w};
        }
#pragma unroll
        for (int j = 0; j < B; ++j) {
            const uint32_t L = tx + j * (kThreads / 2u);
            xl[(L / static_cast<uint32_t>(B)) * 16u + L % static_cast<uint32_t>(B)] = xv[j];
        }
        constexpr uint32_t kDead = 16u - static_cast<uint32_t>(B);
#pragma unroll
        for (uint32_t j = 0; j < kDead; ++j) {
            const uint32_t D = tx + j * (kThreads / 2u);
            xl[(D / kDead) * 16u + static_cast<uint32_t>(B) + D % kDead] = mh::u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kDepth - 1; ++u) {
            issue(tile_c(u), stage_c(u), pbuf[u], svbuf[u], bvbuf[u]);
        }
    }
    // (uniform; its load went out before every other, so no later wait)
    const unsigned long long launches =
        (static_cast<unsigned long long>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(launches_v >> 32))) << 32) |
        __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(launches_v));
    // bit 63 of the count word: the previous launch's wait expired (see the
    // finisher)
    const bool poisoned = (launches >> 63) != 0ull;
    const uint32_t tag = static_cast<uint32_t>((launches & ~(1ull << 63)) % 255ull) + 1u;
    __syncthreads();
    static_assert(kMaxG * 16 == kThreads, "one group sum per thread");
    {
        const uint32_t u = threadIdx.x;
        const uint32_t nb = u % 16u, g = u / 16u;
        float s = 0.0f, sa = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {  // the group's 64 values in order: pieces (q, t) = (j / 2, j % 2)
            const mh::u32x4 v = xl[(g * 8u + (j & 1) * 4u + (j >> 1)) * 16u + nb];
            const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s = s + mh::bf16lo(w4[e]);
                s = s + mh::bf16hi(w4[e]);
                sa = sa + fabsf(mh::bf16lo(w4[e]));
                sa = sa + fabsf(mh::bf16hi(w4[e]));
            }
        }
        xg[u] = s;
        xga[u] = sa;
    }
    __syncthreads();
    // sum |x| per batch row: wave 0, lane l sums groups l / 16 + 4 i of
    // column l % 16, then the four partial sums are added
    if (wave == 0) {
        const uint32_t nb = static_cast<uint32_t>(lane) % 16u, p = static_cast<uint32_t>(lane) / 16u;
        float s = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < kMaxG / 4; ++i) {
            const uint32_t g = p + 4u * i;
            s = s + (g < G ? xga[g * 16u + nb] : 0.0f);
        }
        s = s + __shfl_xor(s, 16);
        s = s + __shfl_xor(s, 32);
        if (lane < B) {
            xa[lane] = s;
        }
    }
    __syncthreads();
    an = col ? xa[n] : 0.0f;
    mfma_stamp<ST>(a, gw, lane, MS_X);

    for (uint32_t s0 = 0; s0 < n_stages; s0 += kDepth) {
#pragma unroll
        for (int u = 0; u < kDepth; ++u) {
            const uint32_t st = s0 + u;
            const uint32_t sn = st + kDepth - 1;
            const int un = (u + kDepth - 1) % kDepth;  // a constant once unrolled
            issue(tile_c(sn), stage_c(sn), pbuf[un], svbuf[un], bvbuf[un]);
            if (st < n_stages) {
                stage_sb(u & 1, st % n_st, svbuf[u], bvbuf[u]);
                compute(u & 1, st % n_st, pbuf[u]);
                if (st % n_st == n_st - 1u) {
                    if ((lane & 3) == 0) {
                        mrow[wave][0][srow] = __uint_as_float(rms);
                        mrow[wave][1][srow] = __uint_as_float(rmb);
                    }
                    finish_tile(tile_of(st));
                    acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                }
            }
        }
    }
    mfma_stamp<ST>(a, gw, lane, MS_LOOP);
    if (a.slots == nullptr) {
        return;
    }

    // ---- workgroup summary per batch row: greatest lower bound, up to four
    // candidates (upper bound and row), the greatest upper bound of the rest
    if (col) {
        m_lb[n][wave * 4 + q] = lbv;
        m_u1[n][wave * 4 + q] = u1;
        m_r1[n][wave * 4 + q] = r1;
        m_du[n][wave * 4 + q] = du;
    }
    __syncthreads();
    // wave b < B summarises batch row b: lane e < 32 holds entry e (wave e / 4,
    // quarter e % 4).  The candidates are the entries whose bf16 upper bound
    // reaches the workgroup's lower bound when there are at most four of them,
    // else the four greatest keys (upper bound desc, row asc); either way every
    // row that can still reach the global lower bound is a candidate or raises
    // the dropped bound, so the finisher decides the same
    const uint32_t last = gridDim.x - 1;
    if (wave < B) {
        const uint32_t b = static_cast<uint32_t>(wave);
        const bool ent = lane < kWaves * 4;
        const int e = ent ? lane : 0;
        float lb = ent ? m_lb[b][e] : -__builtin_inff();
        float dmax = ent ? m_du[b][e] : -__builtin_inff();
        unsigned long long key = ent && m_r1[b][e] != 0xffffffffu ? mh::argmax_key(m_u1[b][e], m_r1[b][e]) : 0ull;
        lb = mh::wave_max_f32(lb);
        unsigned long long out[kSlotWords];
        out[0] = mh::argmax_key(lb, 0u);
        // the entries whose bf16 upper bound reaches this workgroup's lower
        // bound (the others can never reach the global one); at most kCand of
        // them (the usual case) are the candidates as they are, in lane order
        const bool take = key != 0ull && static_cast<uint32_t>(key >> 32) >= mh::bf16_ge_threshold(lb);
        unsigned long long tm = __ballot(take);
        if (__popcll(tm) <= kCand) {
#pragma unroll
            for (int c = 0; c < kCand; ++c) {
                unsigned long long m = mh::argmax_key(-__builtin_inff(), 0xffffffffu);
                if (tm != 0ull) {
                    const int pos = __builtin_ctzll(tm);
                    m = (static_cast<unsigned long long>(static_cast<uint32_t>(
                             __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(key >> 32)), pos)))
                         << 32) |
                        static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(key)), pos));
                    tm &= tm - 1ull;
                }
                out[2 + c] = m;
            }
            key = take ? 0ull : key;
        } else {
            // the four greatest keys, one per round by a wave max
#pragma unroll
            for (int c = 0; c < kCand; ++c) {
                const unsigned long long m = mh::wave_max_u64(key);
                out[2 + c] = m != 0ull ? m : mh::argmax_key(-__builtin_inff(), 0xffffffffu);
                key = key == m ? 0ull : key;  // keys are distinct (distinct rows)
            }
        }
        // the rest of the entries' upper bounds join the dropped bound
        dmax = fmaxf(dmax, key != 0ull ? key_value(key) : -__builtin_inff());
        dmax = mh::wave_max_f32(dmax);
        out[1] = mh::argmax_key(dmax, 0u);
        // as tagged words
#pragma unroll
        for (int j = 0; j < kSlotWords; ++j) {
            out[j] = pack_word(out[j], tag, static_cast<uint32_t>(out[j]) & kRowMask);
        }
        // word j of this workgroup at slot j * kGrid + workgroup
        if (blockIdx.x != last) {
            if (lane < kSlotWords) {
                unsigned long long w = out[0];
#pragma unroll
                for (int j = 1; j < kSlotWords; ++j) {
                    w = lane == j ? out[j] : w;
                }
                __hip_atomic_store(a.slots + static_cast<size_t>(b) * kArgSlots + lane * kGrid + blockIdx.x, w,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        } else if (lane == 0) {
#pragma unroll
            for (int j = 0; j < kSlotWords; ++j) {
                own[b][j] = out[j];
            }
        }
        mfma_stamp<ST>(a, gw, lane, MS_SUMMARY);
    }
    if (blockIdx.x != last) {
        return;
    }

    // ---- finisher (the last workgroup: every other one has started).  Wave
    // b takes batch row b: it reads the other workgroups' words (polling the
    // ones without this launch's tag), clears them, and forms the greatest lower bound,
    // the greatest dropped upper bound and the candidates.  The argmax row is
    // always a candidate unless a dropped bound reaches the lower bound, so a
    // single candidate is the answer; several are recomputed in chunk order;
    // otherwise every row is.
    if (threadIdx.x == 0) {
        fin_expired = 0u;
        fin_arrived = 0u;
    }
    __syncthreads();
    if (wave >= B) {
        return;
    }
    const uint32_t b = static_cast<uint32_t>(wave);
    // this lane's chunk of x for a recompute, loaded while the words arrive
    const uint32_t C = K / 32u;
    const bool live = static_cast<uint32_t>(lane) < C;
    const uint32_t c = live ? static_cast<uint32_t>(lane) : 0u;
    float xr[32], xs;
    mh::load_x_chunk(a.x + static_cast<size_t>(b) * K + 32u * c, xr, xs);
    if (BITS == 4) {
        mh::q4_scale_x(xr);
    }
    // word j: kind j / kPerKind, workgroup lane + 64 (j % kPerKind)
    constexpr int kWords = kSlotWords * kPerKind;
    static_assert(kWords <= 32, "pending mask");
    unsigned long long* const sl = a.slots + static_cast<size_t>(b) * kArgSlots;
    auto word_at = [&](int j) {
        return static_cast<uint32_t>(j / kPerKind) * kGrid + static_cast<uint32_t>(lane) + 64u * (j % kPerKind);
    };
    auto word_valid = [&](int j) { return static_cast<uint32_t>(lane) + 64u * (j % kPerKind) < last; };
    unsigned long long v[kWords];
    uint32_t pend = 0;
#pragma unroll
    for (int j = 0; j < kWords; ++j) {
        // missing workgroups read as the least value with no candidate
        v[j] = word_valid(j) ? __hip_atomic_load(sl + word_at(j), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                             : pack_word(0ull, tag, 0u);
        pend |= (word_tag(v[j]) != tag ? 1u : 0u) << j;
    }
    uint32_t spins = 0;
    while (__any(pend != 0u) && ++spins < kSpinLimit) {
        __builtin_amdgcn_s_sleep(1);
        // all of a round's loads in flight together, then the checks
#pragma unroll
        for (int j = 0; j < kWords; ++j) {
            if ((pend >> j) & 1u) {
                v[j] = __hip_atomic_load(sl + word_at(j), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
#pragma unroll
        for (int j = 0; j < kWords; ++j) {
            if (word_tag(v[j]) == tag) {
                pend &= ~(1u << j);
            }
        }
    }
    mfma_stamp<ST>(a, gw, lane, MS_WORDS);
    // an expired wait, or one in the previous launch: a workgroup that read
    // the count only after that finisher bumped it published under this
    // launch's tag, so this launch's words cannot be trusted either
    const bool expired = __any(pend != 0u);
    const bool lost = expired || poisoned;
    // lower bounds (kind 0) and dropped bounds (kind 1): maxima of the keys'
    // orderable high words
    uint32_t olb = lane == 0 ? static_cast<uint32_t>(own[b][0] >> 32) : 0u;
    uint32_t odu = lane == 0 ? static_cast<uint32_t>(own[b][1] >> 32) : 0u;
#pragma unroll
    for (int j = 0; j < kPerKind; ++j) {
        olb = max(olb, static_cast<uint32_t>(v[j] >> 32));
        odu = max(odu, static_cast<uint32_t>(v[kPerKind + j] >> 32));
    }
    // every workgroup has read the count by now, unless a wait expired: then
    // the count carries the poison bit for the next launch.  The finisher
    // waves report to wave 0 through the LDS (they are resident together, so
    // its wait ends); wave 0 alone writes the word.
    if (lane == 0) {
        if (expired) {
            __hip_atomic_fetch_or(&fin_expired, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        __hip_atomic_fetch_add(&fin_arrived, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (b == 0u) {
            while (__hip_atomic_load(&fin_arrived, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
                   static_cast<uint32_t>(B)) {
                __builtin_amdgcn_s_sleep(1);
            }
            const bool any = __hip_atomic_load(&fin_expired, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u;
            __hip_atomic_store(a.slots + static_cast<size_t>(B) * kArgSlots,
                               ((launches & ~(1ull << 63)) + 1ull) | (any ? 1ull << 63 : 0ull), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    const float lb = key_value(static_cast<unsigned long long>(mh::wave_max_u32(olb)) << 32);
    const float dmax = key_value(static_cast<unsigned long long>(mh::wave_max_u32(odu)) << 32);
    // a candidate's bf16 upper bound reaches lb: one compare of the high word
    const uint32_t thr = mh::bf16_ge_threshold(lb);
    // candidates (row ids) into this wave's stage buffer (free now)
    uint32_t* const cand = stg[wave];
    uint32_t nc = 0;
    auto collect = [&](unsigned long long key, bool valid) {
        const bool take = valid && (static_cast<uint32_t>(key) & kRowMask) != 0u &&
                          static_cast<uint32_t>(key >> 32) >= thr;
        const unsigned long long m = __ballot(take);
        if (m != 0ull) {  // uniform: most words hold no candidate
            if (take) {
                cand[nc + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u))] =
                    ~static_cast<uint32_t>(key) & kRowMask;
            }
            nc += static_cast<uint32_t>(__popcll(m));
        }
    };
#pragma unroll
    for (int j = 2 * kPerKind; j < kWords; ++j) {
        collect(v[j], word_valid(j));
    }
    collect(lane < kCand ? own[b][2 + (lane < kCand ? lane : 0)] : 0ull, lane < kCand);
    const bool all_rows = !(mh::round_bf16(dmax) < lb);
    uint32_t id;
    if (!all_rows && nc == 1u) {
        id = cand[0];
    } else {
        // chunk-order values of the candidates (or of every row), four rows'
        // loads at a time; the staged kernel's merge: NaN never wins, with no
        // other value (-inf, 0)
        const uint32_t count = all_rows ? a.n : nc;
        unsigned long long best = mh::argmax_key(-__builtin_inff(), 0u);
        for (uint32_t i0 = 0; i0 < count; i0 += kRecompute) {
            uint32_t rows[kRecompute];
#pragma unroll
            for (int u = 0; u < kRecompute; ++u) {
                const uint32_t i = i0 + u < count ? i0 + u : count - 1u;
                rows[u] = all_rows ? i : cand[i];
            }
            float vals[kRecompute];
            chunk_values<BITS, kRecompute>(a, rows, xr, xs, live, c, vals, count - i0);
#pragma unroll
            for (int u = 0; u < kRecompute; ++u) {
                const float val = mh::round_bf16(vals[u]);
                if (val == val && i0 + u < count) {
                    const unsigned long long key = mh::argmax_key(val, rows[u]);
                    best = key > best ? key : best;
                }
            }
        }
        id = ~static_cast<uint32_t>(best & 0xffffffffull);
    }
    if (lane == 0) {
        a.ids[b] = lost ? 0xffffffffu : id;
        if (lost && a.status != nullptr) {
            __hip_atomic_fetch_or(a.status, MH_STATUS_ARGMAX_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    mfma_stamp<ST>(a, gw, lane, MS_ID);
    if constexpr (ST) {
        if (lane == 0) {
            a.stamps[static_cast<size_t>(gw) * MH_GEMV_STAMPS + MS_CAND] =
                (!all_rows && nc == 1u) ? 0u : (all_rows ? a.n : nc);
        }
    }
    // clear the words for the next launch (last: no later load waits on them)
#pragma unroll
    for (int j = 0; j < kWords; ++j) {
        if (word_valid(j)) {
            __hip_atomic_store(sl + word_at(j), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int BITS, int B>
int launch(const MfmaArgs& a, hipStream_t stream) {
    if (a.stamps != nullptr) {
        hipLaunchKernelGGL((k_gemv_mfma<BITS, B, true>), dim3(kGrid), dim3(kThreads), 0, stream, a);
    } else {
        hipLaunchKernelGGL((k_gemv_mfma<BITS, B>), dim3(kGrid), dim3(kThreads), 0, stream, a);
    }
    return mh::launch_status("k_gemv_mfma");
}

template <int BITS>
int dispatch(const MfmaArgs& a, uint32_t batch, hipStream_t stream) {
    if (a.stamps != nullptr) {  // the measured shape only: the stamped instantiations are batch 8
        return batch == 8u ? launch<BITS, 8>(a, stream) : MH_ERR_UNSUPPORTED;
    }
    switch (batch) {
        case 2: return launch<BITS, 2>(a, stream);
        case 3: return launch<BITS, 3>(a, stream);
        case 4: return launch<BITS, 4>(a, stream);
        case 5: return launch<BITS, 5>(a, stream);
        case 6: return launch<BITS, 6>(a, stream);
        case 7: return launch<BITS, 7>(a, stream);
        default: return launch<BITS, 8>(a, stream);
    }
}

}  // namespace

namespace mh {

// Batched head GEMV on the matrix cores; MH_ERR_UNSUPPORTED when the shape
// needs the staged chunk-order kernel (the caller then uses it).
int gemv_mfma(const mh_quant_weights* w, const uint16_t* x, uint16_t* y, uint64_t* slots, uint32_t* ids,
              uint32_t batch, hipStream_t stream, uint64_t* stamps) {
    const uint32_t K = w->in_features;
    if (batch < 2 || batch > static_cast<uint32_t>(kMaxB) || w->group_size != 64u || K % (64u * kStageGroups) != 0 ||
        K > kMaxK || w->out_features % kTileRows != 0 || w->out_features > kRowMask || !mh::aligned(x, 16) || !mh::aligned(w->codes, 8) ||
        !mh::aligned(w->scales, 8) || !mh::aligned(w->biases, 8) ||
        (y != nullptr && !mh::aligned(y, 8)) || (slots != nullptr && ids == nullptr)) {
        return MH_ERR_UNSUPPORTED;
    }
    MfmaArgs a{};
    a.codes = reinterpret_cast<const char*>(w->codes);
    a.scales = w->scales;
    a.biases = w->biases;
    a.x = x;
    a.y = y;
    a.slots = reinterpret_cast<unsigned long long*>(slots);
    a.ids = ids;
    a.n = w->out_features;
    a.k = K;
    a.groups = K / 64u;
    a.row_bytes = K * w->bits / 8u;
    a.status = mh::status_word();
    a.stamps = stamps;
    return w->bits == 4 ? dispatch<4>(a, batch, stream) : dispatch<6>(a, batch, stream);
}

}  // namespace mh

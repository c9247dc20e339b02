// grouped_gemm.hip -- block-mapped grouped Q4 GEMM on gfx950 bf16 MFMA.
//
// Replaces quant_nax.metal:4091-4701 (MLX qmm_t bodies over molten's block
// map) behind src/kernels/quant.rs:151-266.  Each block-map entry
// (m0, e*N + n0, n0, m_end) is one workgroup computing
//   C[m, n0 + j] = sum_k A[m, k] * bf16(fma(s, q, b))[e*N + n0 + j, k]
// for m in [m0, m_end) with f32 accumulation on v_mfma_f32_32x32x16_bf16.
//
// Work split (MI355X-first, not MLX's simdgroup tiling):
//   * a workgroup is WAVES wave64s; each wave owns NBW distinct 32-column
//     blocks of the tile and all BM rows, so it dequantizes its own B
//     fragments straight into registers (one Q4 word = the 8 consecutive k
//     of one column that a lane feeds to the MFMA) and reuses every fragment
//     for BM/32 row blocks;
//   * the A tile (with the ids_sorted row gather fused into the load) is
//     staged once per workgroup in a 3-stage LDS ring filled by
//     direct-to-LDS loads, 64 k at a time, XOR-swizzled rows (conflict-free
//     16-byte reads);
//   * k is permuted identically for A and B inside each 64-k block: lane
//     half h and MFMA step j use k = 32h + 8j + t, so a lane's codes for a
//     block are one 16-byte load.
// Epilogues: store C; store gate and up separately; or SwiGLU
// act = bf16(bf16(silu(bf16 g)) * bf16 u) with two accumulators per tile.
#include <type_traits>

#include "mh_device.hpp"
#include "mh_host.hpp"
#include "mh_mfma.hpp"

namespace {

using mh::bf16x2_t;
using mh::bf16x8_t;
using mh::dma16;
using mh::dma16s;
using mh::dma4;
using mh::f32x16_t;
using mh::f32x2_t;
using mh::glb_ptr;
using mh::lgkm_wait;
using mh::tie_regs;
using mh::lds_ptr;
using mh::lds_read16;
using mh::lds_read16_at;
using mh::lds_read4;
using mh::lds_read4_at;
using mh::pack_bf16;
using mh::wait_vmcnt;

constexpr int kBK = 64;

enum Epi { EPI_STORE = 0, EPI_GATE_UP = 1, EPI_SWIGLU = 2 };

struct GemmArgs {
    const uint16_t* a;       // [a_rows, k] bf16
    const uint32_t* gather;  // row i of the tile reads a[gather[i]]; null: a[i]
    const uint32_t* c0; const uint16_t* s0; const uint16_t* b0;  // gate / the matrix
    const uint32_t* c1; const uint16_t* s1; const uint16_t* b1;  // up
    uint16_t* out0;          // [s_rows, n]: C, gate, or act
    uint16_t* out1;          // [s_rows, n]: up (EPI_GATE_UP)
    const uint4* blocks;     // block map; null: a dense product (entries computed)
    uint32_t k, n, s_rows, a_rows, w_rows;
    uint32_t dense_bm;       // rows per entry of a dense product (k_seg)
    uint32_t ordered;        // k_seg: the map is in launch order (entry b for workgroup b)
    uint64_t* stamps;        // per workgroup MH_PREFILL_STAMPS words (stamped k_seg only), or null
};

// One Q4 word (8 codes, low nibble first) -> bf16(fma(s, q, b)) x 8.  High
// nibbles are converted as 16q and scaled by s/16: the product is exactly
// q*s, so every value is the one-rounding fma of the reference dequant.
__device__ __forceinline__ bf16x8_t deq_word(uint32_t w, float s, float s16, float b) {
    const uint32_t lo = mh::opaque(w & 0x0f0f0f0fu);
    const uint32_t hi = mh::opaque(w & 0xf0f0f0f0u);
    uint32_t p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float v0 = __builtin_fmaf(mh::ubyte_f32(lo, j), s, b);
        const float v1 = __builtin_fmaf(mh::ubyte_f32(hi, j), s16, b);
        p[j] = pack_bf16(v0, v1);
    }
    const uint4 u = make_uint4(p[0], p[1], p[2], p[3]);
    return __builtin_bit_cast(bf16x8_t, u);
}

// Workgroup -> block-map entry.  Entries come in groups of nt = n / bn (the
// column tiles of one expert row tile, which read the same A rows); groups
// are dealt round-robin to the 8 XCDs (workgroup i runs on XCD i % 8), so
// every XCD gets an equal share of the real entries (the map's tail is
// padding) and a group's tiles share one XCD's L2.  The grid is a multiple
// of 8 * nt (grid_for_map); indices past the map are padding.
__device__ __forceinline__ uint32_t entry_of_block(uint32_t nt) {
    const uint32_t x = blockIdx.x % 8u, j = blockIdx.x / 8u;
    return ((j / nt) * 8u + x) * nt + j % nt;
}

inline uint32_t grid_for_map(uint32_t n_blocks, uint32_t nt) { return mh::map_grid(n_blocks, nt); }
constexpr int kStages = 3;  // LDS ring depth: two K-blocks in flight while one is consumed

// Tile of BM rows x (NW * NBW * 32) columns per matrix; NW waves, wave w owns
// column blocks [w * NBW, (w + 1) * NBW) of every matrix and all BM rows.
// K advances 64 at a time through a kStages-deep LDS ring:
//   A (the BM x 64 activation block, rows gathered) arrives by direct-to-LDS
//     loads shared by the workgroup, 16-byte chunks XOR-swizzled by row so the
//     MFMA operand reads are bank-conflict free;
//   B codes (16 bytes per lane: a column's 32 codes of one k-half) arrive by
//     direct-to-LDS loads into the owning wave's region;
//   scales and biases are register loads.
// Each wave waits for its own loads of a stage (vmcnt), one barrier then
// publishes the A block and frees the slot the next stage overwrites.
// Row blocks of 32 past the expert's segment are skipped.  Block-map entries
// are dealt to XCDs in column-tile groups (entry_of_block).
template <int BM, int NBW, int NW, bool GATHER, int EPI>
__global__ __launch_bounds__(NW * 64, NW == 4 ? 2 : 1) void k_grouped(GemmArgs a, uint32_t n_entries) {
    constexpr int kThr = NW * 64;
    constexpr int RB = BM / 32;
    constexpr int NMAT = (EPI == EPI_STORE) ? 1 : 2;
    constexpr int QA = BM / (8 * NW);             // A loads (8 rows each) per wave per stage
    constexpr int NB = NMAT * NBW;                // B column blocks per wave
    constexpr int A_BYTES = BM * 128;
    constexpr int B_BYTES = NW * NB * 1024;
    constexpr int SB_BYTES = NW * NB * 256;
    constexpr int STAGE = A_BYTES + B_BYTES + SB_BYTES;
    constexpr int STAGE_OPS = QA + 2 * NB;        // vector memory ops per wave per stage
    static_assert(BM % (8 * NW) == 0, "A rows per wave");
    extern __shared__ __attribute__((aligned(16))) char lds[];
    (void)kThr;

    const uint32_t ent = entry_of_block(a.n / (NW * NBW * 32u));
    if (ent >= n_entries) {
        return;
    }
    uint4 blk;
    if (a.blocks == nullptr) {  // dense: one matrix, entry = (row tile, column tile)
        const uint32_t nt = a.n / (NW * NBW * 32u);
        const uint32_t mr = (ent / nt) * BM, nc = (ent % nt) * (NW * NBW * 32u);
        blk = make_uint4(mr, nc, nc, min(mr + BM, a.s_rows));
    } else {
        blk = a.blocks[ent];
    }
    const uint32_t m0 = blk.x, brow = blk.y, n0 = blk.z, m_end = blk.w;
    if (m0 >= m_end) {
        return;
    }
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i32 = lane & 31, h = lane >> 5;
    const uint32_t K = a.k, nkb = K / kBK;
    const uint32_t groups = K / 64u;
    const uint32_t live_rb = min(static_cast<uint32_t>(RB), (m_end - m0 + 31u) / 32u);
    const uint32_t lds0 = static_cast<uint32_t>((uintptr_t)((lds_ptr)lds));

    // 32-bit byte offsets from wave-uniform bases (launch_t rejects operands
    // past 4 GiB), so each load is scalar base + vector offset.
    const mh::gbytes abase = mh::uniform_ptr(a.a);
    mh::gbytes cbase[NMAT], sbase[NMAT], bbase[NMAT];
    cbase[0] = mh::uniform_ptr(a.c0);
    sbase[0] = mh::uniform_ptr(a.s0);
    bbase[0] = mh::uniform_ptr(a.b0);
    if (NMAT == 2) {
        cbase[NMAT - 1] = mh::uniform_ptr(a.c1);
        sbase[NMAT - 1] = mh::uniform_ptr(a.s1);
        bbase[NMAT - 1] = mh::uniform_ptr(a.b1);
    }
    // A: this lane's source row for each of its QA loads (clamped into the segment)
    uint32_t aoffs[QA];
#pragma unroll
    for (int q = 0; q < QA; ++q) {
        const uint32_t r = 8u * (wave * QA + q) + static_cast<uint32_t>(lane >> 3);
        const uint32_t m = min(m0 + r, m_end - 1u);
        uint32_t src = GATHER ? a.gather[m] : m;
        src = min(src, a.a_rows - 1u);
        const uint32_t chunk = static_cast<uint32_t>(lane & 7) ^ (r & 7u);
        aoffs[q] = src * K * 2u + chunk * 16u;
    }
    // B: this lane's weight row (column) per column block and matrix.  The
    // scale/bias load is one dword per lane: lanes 0-31 the column's scale
    // pair (groups kb & ~1, kb | 1), lanes 32-63 its bias pair.
    uint32_t boffs[NB], sboffs[NB];
#pragma unroll
    for (int cb = 0; cb < NBW; ++cb) {
        const uint32_t col = static_cast<uint32_t>((wave * NBW + cb) * 32 + i32);
        const uint32_t r = min(brow + col, a.w_rows - 1u);
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat) {
            boffs[mat * NBW + cb] = r * (K / 2u) + 16u * h;
            sboffs[mat * NBW + cb] = r * groups * 2u;
        }
    }

    auto issue = [&](uint32_t kb, int slot) {
        const uint32_t base = lds0 + slot * STAGE;
#pragma unroll
        for (int q = 0; q < QA; ++q) {
            dma16(abase + aoffs[q] + kb * 128u, base + (wave * QA + q) * 1024u);
        }
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            dma16(cbase[t / NBW] + boffs[t] + kb * 32u, base + A_BYTES + (wave * NB + t) * 1024u);
        }
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            const mh::gbytes sb = h ? bbase[t / NBW] : sbase[t / NBW];
            dma4(sb + sboffs[t] + (kb & ~1u) * 2u, base + A_BYTES + B_BYTES + (wave * NB + t) * 256u);
        }
    };

    f32x16_t acc[NMAT][RB][NBW];
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int cb = 0; cb < NBW; ++cb)
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[mat][rb][cb][q] = 0.0f;

    // A operand addresses: row rb*32 + i32, logical chunk 4h + j, swizzled
    uint32_t aoff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        aoff[j] = static_cast<uint32_t>(i32) * 128u + ((static_cast<uint32_t>(4 * h + j) ^ static_cast<uint32_t>(i32 & 7)) * 16u);
    }

#pragma unroll
    for (int d = 0; d < kStages - 1; ++d) {
        if (static_cast<uint32_t>(d) < nkb) {
            issue(d, d);
        }
    }
    for (uint32_t kb0 = 0; kb0 < nkb; kb0 += kStages) {
#pragma unroll
        for (int u = 0; u < kStages; ++u) {
            const uint32_t kb = kb0 + u;
            if (kb >= nkb) {
                break;
            }
            // own loads of stage kb done (later stages may stay in flight)
            if (kb + 1 < nkb) {
                wait_vmcnt<STAGE_OPS>();
            } else {
                wait_vmcnt<0>();
            }
            __builtin_amdgcn_s_barrier();  // no fence: later stages stay in flight
            if (kb + kStages - 1 < nkb) {
                issue(kb + kStages - 1, (u + kStages - 1) % kStages);
            }
            const uint32_t base = lds0 + u * STAGE;
            uint4 bcode[NB];
            uint32_t sw[NB], bw[NB];
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                bcode[t] = lds_read16(base + A_BYTES + (wave * NB + t) * 1024u + lane * 16u);
                const uint32_t sbl = base + A_BYTES + B_BYTES + (wave * NB + t) * 256u + i32 * 4u;
                sw[t] = lds_read4(sbl);
                bw[t] = lds_read4(sbl + 128u);
            }
            lgkm_wait<0>(bcode);
            tie_regs(sw);
            tie_regs(bw);
            const uint32_t half = (kb & 1u) ? 0u : 16u;  // bf16 of group kb in the high half
            float sf[NB], s16[NB], bf[NB];
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                sf[t] = __uint_as_float((sw[t] << half) & 0xffff0000u);
                s16[t] = sf[t] * 0.0625f;
                bf[t] = __uint_as_float((bw[t] << half) & 0xffff0000u);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                bf16x8_t bfr[NB];
#pragma unroll
                for (int t = 0; t < NB; ++t) {
                    const uint32_t wv = j == 0 ? bcode[t].x : j == 1 ? bcode[t].y : j == 2 ? bcode[t].z : bcode[t].w;
                    bfr[t] = deq_word(wv, sf[t], s16[t], bf[t]);
                }
                uint4 av[RB];
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    if (static_cast<uint32_t>(rb) < live_rb) {
                        av[rb] = lds_read16(base + rb * 4096u + aoff[j]);
                    }
                }
                lgkm_wait<0>(av);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    if (static_cast<uint32_t>(rb) < live_rb) {
                        const bf16x8_t af = __builtin_bit_cast(bf16x8_t, av[rb]);
#pragma unroll
                        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                            for (int cb = 0; cb < NBW; ++cb)
                                acc[mat][rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                    af, bfr[mat * NBW + cb], acc[mat][rb][cb], 0, 0, 0);
                    }
                }
            }
        }
    }

    // ---- epilogue: D lane layout row = 8*(q/4) + 4*h + q%4, col = i32
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < NBW; ++cb)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const uint32_t row = m0 + rb * 32 + 8 * (q / 4) + 4 * h + (q % 4);
                if (row >= m_end) continue;
                const size_t o = static_cast<size_t>(row) * a.n + n0 + (wave * NBW + cb) * 32 + i32;
                if constexpr (EPI == EPI_STORE) {
                    a.out0[o] = mh::f32_to_bf16(acc[0][rb][cb][q]);
                } else if constexpr (EPI == EPI_GATE_UP) {
                    a.out0[o] = mh::f32_to_bf16(acc[0][rb][cb][q]);
                    a.out1[o] = mh::f32_to_bf16(acc[1][rb][cb][q]);
                } else {
                    const float g = mh::round_bf16(acc[0][rb][cb][q]);
                    const float u = mh::round_bf16(acc[1][rb][cb][q]);
                    a.out0[o] = mh::f32_to_bf16(mh::silu_bf16(g) * u);
                }
            }
}

// ------------------------------------------------------------------------
// Segment kernel: one workgroup per block-map entry of any row count (maps
// built with bm = 256 or 512), 4 waves, one workgroup per CU.  The entry's
// rows are covered in passes of RB <= 9 row blocks of 32 (passes balanced:
// a 300-row segment runs as 5 + 5 blocks, not 9 + 1); RB is a template
// argument of the pass, so the K loop has no per-row-block branches.  The
// accumulators (RB x NMAT x NBW tiles of 32x32 f32) of the first 8 row
// blocks fill the 256 AGPRs; a ninth row block's 32 live in arch VGPRs
// (mfma_vacc), so an expert of up to 288 rows -- nearly every expert of a
// 4096-token, 64-expert, top-4 routing -- runs in one pass and its B codes
// are loaded and dequantized once.  Per K-step of 16 the wave issues the
// next step's A fragment reads before this step's MFMAs and dequantizes the
// next step's B words between them, so LDS latency and the dequant VALU
// work run under the matrix pipe.

constexpr int kSegWaves = 4;
#ifndef MH_SEG_RBMAX
#define MH_SEG_RBMAX 9
#endif
constexpr int kSegRBMax = MH_SEG_RBMAX;  // row blocks of 32 per pass (max)
constexpr int kSegAgprBlocks = 8;        // row blocks whose accumulators fit the AGPRs (NMAT * NBW == 2)

// v_mfma_f32_32x32x16_bf16 with its accumulator in arch VGPRs.  The
// compiler keeps every accumulator of the builtin in AGPRs and, once they
// exceed the 256 AGPRs, shuffles them through VGPRs on every iteration
// (v_accvgpr moves); the "+v" operand pins these 16 to VGPRs instead.  As
// inline asm the MFMA is outside the compiler's hazard tracking: its
// operands are written long before it (a step earlier) and the accumulator
// is read by VALU only after mfma_vacc_drain().
__device__ __forceinline__ f32x16_t mfma_vacc(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
    return c;
}
// Wait states between the last mfma_vacc and a VALU read of its result (an
// 8-pass XDL op needs fewer than these 24), and between the VALU writes that
// zero the accumulators and the first mfma_vacc reading them.  The
// accumulators pass through the asm, so every use of them on the far side
// is ordered after the wait states.
__device__ __forceinline__ void mfma_vacc_drain(f32x16_t& c0, f32x16_t& c1) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(c0), "+v"(c1) : : "memory");
}
__device__ __forceinline__ void mfma_vacc_ready(f32x16_t& c0, f32x16_t& c1) {
    asm volatile("s_nop 4" : "+v"(c0), "+v"(c1));
}
#ifndef MH_SEG_STAGES
#define MH_SEG_STAGES 3
#endif
constexpr int kSegStages = MH_SEG_STAGES;  // LDS ring depth

// Compile-time loop: f(std::integral_constant<int, i>) for i in [0, N).
template <int I, int N, typename F>
__device__ __forceinline__ void static_for_impl(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for_impl<I + 1, N>(f);
    }
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl<0, N>(f);
}

// Fast SiLU for the GEMM epilogue (the gate/up values it sees already
// carry MFMA accumulation error): g * 1 / (1 + 2^(-g log2 e)) with the
// hardware exp2 and reciprocal (1 ulp each).
__device__ __forceinline__ float silu_hw(float g) {
    const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
    return g * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float bf16_round_hw(float v) {
    const f32x2_t p = {v, 0.0f};
    const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(p, bf16x2_t));
    return __uint_as_float(u << 16);
}

// Wait until at most c (<= C) later stages of OPS vector memory ops each are
// still in flight.
template <int OPS, int C>
__device__ __forceinline__ void wait_stages(uint32_t c) {
    if constexpr (C == 0) {
        wait_vmcnt<0>();
    } else {
        static_assert(C * OPS <= 63, "vmcnt field");
        if (c >= static_cast<uint32_t>(C)) {
            wait_vmcnt<C * OPS>();
        } else {
            wait_stages<OPS, C - 1>(c);
        }
    }
}

template <int RBMAX, int NBW, int NMAT, int NS = kStages>
struct SegLayout {
    static constexpr int NB = NMAT * NBW;                    // B fragments per wave
    static constexpr int A_STAGE = RBMAX * 32 * 128;         // RBMAX*32 rows x 64 k bf16
    static constexpr int B_HALF = kSegWaves * NB * 2048;     // codes of 2 stages (k 128)
    static constexpr int SB_BLK = kSegWaves * NB * 1024;     // scales + biases of 8 groups
    static constexpr int B_OFF = NS * A_STAGE;               // A ring, then two B slots,
    static constexpr int SB_OFF = B_OFF + 2 * B_HALF;        // then two scale/bias slots
    static constexpr int LDS = SB_OFF + 2 * SB_BLK;
};

// One pass: rows [mp0, mp0 + 32 RB) of the segment (clamped to m_end),
// columns of this wave, the whole K.
//
// Loads are direct-to-LDS and shaped for few L2 requests per 64-k stage:
//   * A: RB*32 rows x 128 bytes (one line per row) into a 3-slot ring shared
//     by the workgroup; chunk c of row r sits at position c ^ ((r >> 1) & 7),
//     so a 16-byte read by 16 lanes (16 rows, one chunk each) covers all 64
//     banks once;
//   * B codes: every other stage, the next two stages' codes of each column
//     (64 bytes, half a line; 4 lanes per column) into a per-wave region of
//     one of two slots, chunks swizzled by ((column >> 2) & 3) so the MFMA
//     operand reads (lane i32, half h, stage s: chunk 2s + h; 16 lanes per
//     64-bank cycle) are bank-conflict free;
//   * scales and biases: every 8 stages, 16 bytes (8 groups) of the column's
//     scale row (lanes 0-31) and bias row (lanes 32-63), two slots.
// Stage g's loads ("group g": its A, plus the B half-block that starts at g,
// plus the scale/bias block that starts at g) are spread over the MFMA steps
// 0..2 of stage g - 2, one load after each row block's MFMAs, so the wave's
// vector-memory issue never holds up a run of MFMAs.  One barrier per stage,
// before its step 3 (the wave's own loads of group g + 1 waited for, its
// reads of the stage's A slot done), publishes every wave's group g + 1 and
// frees the slot that group g + 3 refills; the next stage's first A
// fragments and B words are then read under step 3's MFMAs.
template <int RB, int RBMAX, int NS, int NBW, int NMAT, bool GATHER, int EPI>
__device__ __forceinline__ void seg_pass(const GemmArgs& a, uint32_t brow, uint32_t n0,
                                         uint32_t mp0, uint32_t m_end, uint32_t lds0, int lane_in,
                                         int wave) {
    using L = SegLayout<RBMAX, NBW, NMAT, NS>;
    static_assert(NS == 3, "loads run two stages ahead through a 3-slot A ring");
    constexpr int NB = L::NB;
    constexpr int QA = RB;  // A loads (8 rows each) per wave per stage
    // the lane-derived offsets are recomputed in every pass (a few VALU ops):
    // hoisted out of the pass loop they outlive the registers and are spilled
    const int lane = static_cast<int>(mh::opaque(static_cast<uint32_t>(lane_in)));
    const int i32 = lane & 31, h = lane >> 5;
    const uint32_t K = a.k, nkb = K / kBK, groups = K / 64u;

    const mh::gbytes abase = mh::uniform_ptr(a.a);
    mh::gbytes cbase[NMAT], sbase[NMAT], bbase[NMAT];
    cbase[0] = mh::uniform_ptr(a.c0);
    sbase[0] = mh::uniform_ptr(a.s0);
    bbase[0] = mh::uniform_ptr(a.b0);
    if (NMAT == 2) {
        cbase[NMAT - 1] = mh::uniform_ptr(a.c1);
        sbase[NMAT - 1] = mh::uniform_ptr(a.s1);
        bbase[NMAT - 1] = mh::uniform_ptr(a.b1);
    }
    uint32_t aoffs[QA];
#pragma unroll
    for (int q = 0; q < QA; ++q) {
        const uint32_t r = 8u * (wave * QA + q) + static_cast<uint32_t>(lane >> 3);
        const uint32_t m = min(mp0 + r, m_end - 1u);
        uint32_t src = GATHER ? a.gather[m] : m;
        src = min(src, a.a_rows - 1u);
        const uint32_t chunk = static_cast<uint32_t>(lane & 7) ^ ((r >> 1) & 7u);
        aoffs[q] = src * K * 2u + chunk * 16u;
    }
    // B half-block load p of fragment t: columns 16p .. 16p + 15, lane l =
    // 4c' + q stores LDS chunk q of column c = 16p + c', holding global chunk
    // q ^ ((c >> 2) & 3).  Scale/bias block: lane (i32, h) loads 16 bytes of
    // column i32's scale (h = 0) or bias (h = 1) row.
    uint32_t bcoffs[NB][2], sboff[NB];
#pragma unroll
    for (int cb = 0; cb < NBW; ++cb) {
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat) {
            const int t = mat * NBW + cb;
            const uint32_t col0 = brow + static_cast<uint32_t>((wave * NBW + cb) * 32);
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const uint32_t c = 16u * p + static_cast<uint32_t>(lane >> 2);
                const uint32_t r = min(col0 + c, a.w_rows - 1u);
                const uint32_t g = static_cast<uint32_t>(lane & 3) ^ ((c >> 2) & 3u);
                bcoffs[t][p] = r * (K / 2u) + g * 16u;
            }
            sboff[t] = min(col0 + static_cast<uint32_t>(i32), a.w_rows - 1u) * groups * 2u;
        }
    }
    // the loads of group g: A load q, then the B codes (one load per
    // fragment half, even groups) and the scale/bias words (every 8th group);
    // load i of the group is issued when sel(i) is true
    auto issue_sel = [&](uint32_t g, auto&& sel) {
        const uint32_t abuf = __builtin_amdgcn_readfirstlane(lds0 + (g % 3u) * L::A_STAGE + wave * QA * 1024u);
        const mh::gbytes ag = mh::uniform_ptr(abase + g * 128u);
#pragma unroll
        for (int q = 0; q < QA; ++q) {
            if (sel(q)) {
                dma16s(ag, aoffs[q], abuf + q * 1024u);
            }
        }
        if ((g & 1u) == 0) {
            const uint32_t hb = g >> 1;
            const uint32_t bbuf = __builtin_amdgcn_readfirstlane(lds0 + L::B_OFF + (hb & 1u) * L::B_HALF + wave * NB * 2048u);
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                const mh::gbytes cg = mh::uniform_ptr(cbase[t / NBW] + hb * 64u);
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    if (sel(QA + 2 * t + p)) {
                        dma16s(cg, bcoffs[t][p], bbuf + t * 2048u + p * 1024u);
                    }
                }
            }
        }
        if ((g & 7u) == 0) {
            const uint32_t sbk = g >> 3;
            const uint32_t sbuf = lds0 + L::SB_OFF + (sbk & 1u) * L::SB_BLK + wave * NB * 1024u;
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                if (sel(QA + 2 * NB + t)) {
                    const mh::gbytes src = h ? bbase[t / NBW] : sbase[t / NBW];
                    dma16(src + sboff[t] + sbk * 16u, sbuf + t * 1024u);
                }
            }
        }
    };
    auto issue_group = [&](uint32_t g) {
        const uint32_t abuf = __builtin_amdgcn_readfirstlane(lds0 + (g % 3u) * L::A_STAGE + wave * QA * 1024u);
        const mh::gbytes ag = mh::uniform_ptr(abase + g * 128u);
#pragma unroll
        for (int q = 0; q < QA; ++q) {
            dma16s(ag, aoffs[q], abuf + q * 1024u);
        }
        if ((g & 1u) == 0) {
            const uint32_t hb = g >> 1;
            const uint32_t bbuf = __builtin_amdgcn_readfirstlane(lds0 + L::B_OFF + (hb & 1u) * L::B_HALF + wave * NB * 2048u);
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                const mh::gbytes cg = mh::uniform_ptr(cbase[t / NBW] + hb * 64u);
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    dma16s(cg, bcoffs[t][p], bbuf + t * 2048u + p * 1024u);
                }
            }
        }
        if ((g & 7u) == 0) {
            const uint32_t sbk = g >> 3;
            const uint32_t sbuf = lds0 + L::SB_OFF + (sbk & 1u) * L::SB_BLK + wave * NB * 1024u;
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                const mh::gbytes src = h ? bbase[t / NBW] : sbase[t / NBW];
                dma16(src + sboff[t] + sbk * 16u, sbuf + t * 1024u);
            }
        }
    };

    // accumulators of row blocks past kSegAgprBlocks stay in arch VGPRs
    static_assert(NMAT * NBW * 16 * kSegAgprBlocks == 256, "the first kSegAgprBlocks row blocks fill the AGPRs");
    auto seg_mma = [](int rb, bf16x8_t bw, bf16x8_t af, f32x16_t c) {
        return rb >= kSegAgprBlocks ? mfma_vacc(bw, af, c) : __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw, af, c, 0, 0, 0);
    };
    f32x16_t acc[NMAT][RB][NBW];
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int cb = 0; cb < NBW; ++cb)
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[mat][rb][cb][q] = 0.0f;
    if constexpr (RB > kSegAgprBlocks) {
        mfma_vacc_ready(acc[0][kSegAgprBlocks][0], acc[NMAT - 1][kSegAgprBlocks][NBW - 1]);
    }

    uint32_t aoff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        aoff[j] = static_cast<uint32_t>(i32) * 128u +
                  ((static_cast<uint32_t>(4 * h + j) ^ ((static_cast<uint32_t>(i32) >> 1) & 7u)) * 16u);
    }

    // Own loads of group g are complete once only the group after it may
    // still be in flight.  B codes and scale/bias words sit in per-wave
    // regions that only the wave's own loads fill, so they are readable then;
    // A (loaded by all four waves) also needs a barrier.
    auto wait_own = [&](uint32_t g) {
        const uint32_t g1 = g + 1;
        if (g1 >= nkb) {
            wait_vmcnt<0>();
        } else if ((g1 & 7u) == 0) {
            wait_vmcnt<QA + 3 * NB>();
        } else if ((g1 & 1u) == 0) {
            wait_vmcnt<QA + 2 * NB>();
        } else {
            wait_vmcnt<QA>();
        }
    };
    // LDS reads (no wait) of stage kb's B codes (chunk 2 (kb % 2) + h of the
    // lane's column) and scale/bias words (group kb: word (kb % 8) / 2)
    auto read_bsb = [&](uint32_t kb, uint4 (&bc)[NB], uint32_t (&sbw)[2 * NB]) {
        const uint32_t pos = ((2u * (kb & 1u) + static_cast<uint32_t>(h)) ^ ((static_cast<uint32_t>(i32) >> 2) & 3u)) * 16u;
        const uint32_t bl = lds0 + L::B_OFF + ((kb >> 1) & 1u) * L::B_HALF + wave * NB * 2048u + i32 * 64u + pos;
        static_for<NB>([&](auto t) { bc[t] = lds_read16_at<t * 2048>(bl); });
        const uint32_t sl = lds0 + L::SB_OFF + ((kb >> 3) & 1u) * L::SB_BLK + wave * NB * 1024u + i32 * 16u + ((kb & 7u) >> 1) * 4u;
        static_for<NB>([&](auto t) {
            sbw[2 * t] = lds_read4_at<t * 1024>(sl);
            sbw[2 * t + 1] = lds_read4_at<t * 1024 + 512>(sl);
        });
    };
    auto read_a = [&](uint32_t kb, int j, uint4 (&av)[RB]) {
        const uint32_t ab = lds0 + (kb % 3u) * L::A_STAGE + aoff[j];
        static_for<RB>([&](auto rb) { av[rb] = lds_read16_at<rb * 4096>(ab); });
    };
    float sf[NB], s16[NB], bf[NB];
    auto scale_bias = [&](uint32_t kb, const uint32_t (&sbw)[2 * NB]) {
        const uint32_t half = (kb & 1u) ? 0u : 16u;  // group kb's bf16 is the high half when kb is odd
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            sf[t] = __uint_as_float((sbw[2 * t] << half) & 0xffff0000u);
            s16[t] = sf[t] * 0.0625f;
            bf[t] = __uint_as_float((sbw[2 * t + 1] << half) & 0xffff0000u);
        }
    };

    // Group g is issued after the barrier that ends stage g - 3 (the barrier
    // frees that stage's A slot, which g reuses), groups 0..2 up front.
    issue_group(0);
    if (nkb > 1) {
        issue_group(1);
    }
    uint4 bc[NB];
    uint32_t sbw[2 * NB];
    uint4 av[2][RB];
    bf16x8_t bfr[2][NB];
    wait_own(0);
    read_bsb(0, bc, sbw);
    lgkm_wait<0>(bc);
    lgkm_wait<0>(sbw);
    scale_bias(0, sbw);
#pragma unroll
    for (int t = 0; t < NB; ++t) {
        bfr[0][t] = deq_word(bc[t].x, sf[t], s16[t], bf[t]);
    }
    __builtin_amdgcn_s_barrier();
    read_a(0, 0, av[0]);
    // stage kb; LOADS: group kb + 2 exists (its loads are spread over steps
    // 0..2), NEXT: stage kb + 1 exists
    auto stage = [&](uint32_t kb, auto loads_c, auto next_c) {
        constexpr bool LOADS = decltype(loads_c)::value, NEXT = decltype(next_c)::value;
        // steps 0..2: the next step's A reads in flight and its B words
        // dequantized while this step's MFMAs run
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int cur = j & 1, nxt = cur ^ 1;
            read_a(kb, j + 1, av[nxt]);
            lgkm_wait<RB>(av[cur]);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const bf16x8_t af = __builtin_bit_cast(bf16x8_t, av[cur][rb]);
#pragma unroll
                for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                    for (int cb = 0; cb < NBW; ++cb)
                        acc[mat][rb][cb] = seg_mma(rb, bfr[cur][mat * NBW + cb], af, acc[mat][rb][cb]);
                if (rb == 0) {
#pragma unroll
                    for (int t = 0; t < NB; ++t) {
                        const uint32_t wv = j == 0 ? bc[t].y : j == 1 ? bc[t].z : bc[t].w;
                        bfr[nxt][t] = deq_word(wv, sf[t], s16[t], bf[t]);
                    }
                }
                // group kb + 2's loads, one after each row block's MFMAs:
                // load i in step i % 3 after row block (i / 3) % RB
                if constexpr (LOADS) {
                    issue_sel(kb + 2, [&](int i) { return i % 3 == j && (i / 3) % RB == rb; });
                }
            }
        }
        // step 3.  Before it: this wave's loads of group kb + 1 have landed
        // and its reads of stage kb's A slot are done; one barrier then
        // publishes every wave's group kb + 1 and frees the slot.  The next
        // stage's B codes, scale/bias words and first A fragments are read
        // under step 3's MFMAs, and that stage's step-0 B words dequantized.
        lgkm_wait<0>(av[1]);
        if constexpr (NEXT) {
            wait_own(kb + 1);
            __builtin_amdgcn_s_barrier();
            read_bsb(kb + 1, bc, sbw);
            read_a(kb + 1, 0, av[0]);
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const bf16x8_t af = __builtin_bit_cast(bf16x8_t, av[1][rb]);
#pragma unroll
            for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                for (int cb = 0; cb < NBW; ++cb)
                    acc[mat][rb][cb] = seg_mma(rb, bfr[1][mat * NBW + cb], af, acc[mat][rb][cb]);
            if constexpr (NEXT) {
                if (rb == (RB - 1) / 2) {
                    // (the RB A reads issued after them may still be in flight)
                    lgkm_wait<RB>(bc);
                    lgkm_wait<RB>(sbw);
                    scale_bias(kb + 1, sbw);
#pragma unroll
                    for (int t = 0; t < NB; ++t) {
                        bfr[0][t] = deq_word(bc[t].x, sf[t], s16[t], bf[t]);
                    }
                }
            }
        }
    };
    using yes = std::true_type;
    using no = std::false_type;
    uint32_t kb = 0;
    for (; kb + 2 < nkb; ++kb) {
        stage(kb, yes{}, yes{});
    }
    stage(kb, no{}, yes{});
    stage(kb + 1, no{}, no{});
    if constexpr (RB > kSegAgprBlocks) {
        static_assert(RB == kSegAgprBlocks + 1 && NMAT * NBW == 2, "one VGPR row block of two tiles");
        mfma_vacc_drain(acc[0][kSegAgprBlocks][0], acc[NMAT - 1][kSegAgprBlocks][NBW - 1]);
    }
    // every wave is done with the ring before another pass refills it
    __builtin_amdgcn_s_barrier();

    // ---- epilogue.  The MFMAs computed C^T (W fragment as the first
    // operand): lane (i32, h) holds row mp0 + 32 rb + i32 and, at q = 4p + r,
    // column 8p + 4h + r of its 32-column block.  Values become bf16 pairs;
    // permlane32_swap of the (p even, p odd) pairs gives lane h = 0 columns
    // 8p..8p+7 of p = 0, 2 and lane h = 1 those of p = 1, 3, stored 16 bytes
    // at a time.
    const mh::gbytes ob0 = mh::uniform_ptr(reinterpret_cast<const char*>(a.out0));
    const mh::gbytes ob1 = mh::uniform_ptr(reinterpret_cast<const char*>(a.out1 ? a.out1 : a.out0));
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const uint32_t row = mp0 + rb * 32u + static_cast<uint32_t>(i32);
#pragma unroll
        for (int cb = 0; cb < NBW; ++cb) {
            constexpr int NOUT = (EPI == EPI_GATE_UP) ? 2 : 1;
            uint32_t w[NOUT][4][2];  // [output][p][pair]
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                float v[NOUT][4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int q = 4 * p + r;
                    if constexpr (EPI == EPI_SWIGLU) {
                        const float g = bf16_round_hw(acc[0][rb][cb][q]);
                        const float u = bf16_round_hw(acc[1][rb][cb][q]);
                        v[0][r] = bf16_round_hw(silu_hw(g)) * u;
                    } else {
#pragma unroll
                        for (int o = 0; o < NOUT; ++o) {
                            v[o][r] = acc[o][rb][cb][q];
                        }
                    }
                }
#pragma unroll
                for (int o = 0; o < NOUT; ++o) {
                    w[o][p][0] = pack_bf16(v[o][0], v[o][1]);
                    w[o][p][1] = pack_bf16(v[o][2], v[o][3]);
                }
            }
            const uint32_t col = n0 + static_cast<uint32_t>((wave * NBW + cb) * 32 + 8 * h);
            const uint32_t off = (row * a.n + col) * 2u;
#pragma unroll
            for (int o = 0; o < NOUT; ++o) {
#pragma unroll
                for (int pp = 0; pp < 2; ++pp) {
#pragma unroll
                    for (int d = 0; d < 2; ++d) {
                        const auto r = __builtin_amdgcn_permlane32_swap(w[o][2 * pp][d], w[o][2 * pp + 1][d], false, false);
                        w[o][2 * pp][d] = r[0];
                        w[o][2 * pp + 1][d] = r[1];
                    }
                }
                if (row < m_end) {
                    const mh::gbytes ob = o == 0 ? ob0 : ob1;
                    typedef __attribute__((address_space(1))) mh::u32x4* g4;
                    // columns 8h .. 8h+7 (pp = 0) and 16 + 8h .. (pp = 1)
                    *reinterpret_cast<g4>(const_cast<char __attribute__((address_space(1)))*>(ob) + off) =
                        mh::u32x4{w[o][0][0], w[o][0][1], w[o][1][0], w[o][1][1]};
                    *reinterpret_cast<g4>(const_cast<char __attribute__((address_space(1)))*>(ob) + off + 32u) =
                        mh::u32x4{w[o][2][0], w[o][2][1], w[o][3][0], w[o][3][1]};
                }
            }
        }
    }
}


// Balanced workgroup -> entry mapping of the segment kernels.  A "group" is
// nt consecutive map entries (one expert row tile across its column tiles,
// which read the same A rows), weighted by its row count (0 for padding).
// Groups are ranked by weight (descending, ties by index) and dealt to the
// 8 XCDs in snake order (rank k -> XCD k % 8 on even rounds, 7 - k % 8 on
// odd ones; slot k / 8), so XCD totals come out nearly equal and each XCD
// runs its largest groups first; workgroup i (XCD i % 8, j = i / 8) takes
// column tile j % nt of the group in slot j / nt of its XCD (mh::seg_rank_of).
// Every workgroup ranks the groups itself (a few hundred instructions; the
// weights and its tile's entries go through the LDS, which is free before
// the pass starts).  Returns n_entries for padding workgroups; blk: the
// entry (with a block map).
__device__ uint32_t balanced_entry(const GemmArgs& a, uint32_t n_entries, uint32_t nt, char* lds, uint4& blk) {
    const uint4* blocks = a.blocks;
    __shared__ uint32_t s_group;
    __shared__ uint4 s_blk;
    const uint32_t C = (n_entries + nt - 1u) / nt;
    const uint32_t t = (blockIdx.x / 8u) % nt;
    const uint32_t k_target = mh::seg_rank_of(blockIdx.x, nt);
    // each group's entry of this workgroup's column tile t and its rows (for
    // a well-formed map every entry of a group has the group's rows; ranked
    // per tile, the (group, tile) pairs are dealt out once each either way),
    // so the chosen entry needs no second read of the map
    // weights padded with zeros to a multiple of 4 (read 16 bytes at a time;
    // a zero at d >= C never ranks ahead of any group)
    const uint32_t C4 = (C + 3u) & ~3u;
    uint4* ents = reinterpret_cast<uint4*>(lds);                 // [C]
    uint32_t* wts = reinterpret_cast<uint32_t*>(lds + 16u * C);  // [C4] group weights
    for (uint32_t c = threadIdx.x; c < C4; c += blockDim.x) {
        if (c >= C) {
            wts[c] = 0u;
        } else if (blocks == nullptr) {  // dense: row segments of dense_bm, the last partial
            wts[c] = min(a.dense_bm, a.s_rows - c * a.dense_bm);
        } else {
            const uint32_t i = c * nt + t;
            const uint4 e = i < n_entries ? blocks[i] : make_uint4(0u, 0u, 0u, 0u);
            ents[c] = e;
            wts[c] = e.x < e.w ? e.w - e.x : 0u;
        }
    }
    if (threadIdx.x == 0) {
        s_group = 0xffffffffu;
    }
    __syncthreads();
    if (k_target < C) {
        const uint4* w4 = reinterpret_cast<const uint4*>(wts);
        for (uint32_t c = threadIdx.x; c < C; c += blockDim.x) {
            const uint32_t w = wts[c];
            uint32_t rank = 0;
#pragma unroll 4
            for (uint32_t d = 0; d < C4; d += 4u) {
                const uint4 v = w4[d / 4u];
                rank += (v.x > w || (v.x == w && d < c)) ? 1u : 0u;
                rank += (v.y > w || (v.y == w && d + 1u < c)) ? 1u : 0u;
                rank += (v.z > w || (v.z == w && d + 2u < c)) ? 1u : 0u;
                rank += (v.w > w || (v.w == w && d + 3u < c)) ? 1u : 0u;
            }
            if (rank == k_target) {
                s_group = c;
                if (blocks != nullptr) {
                    s_blk = ents[c];
                }
            }
        }
    }
    __syncthreads();
    const uint32_t g = s_group;
    if (blocks != nullptr) {
        blk = s_blk;  // (a static variable: the staging reuses the dynamic LDS)
    }
    return g == 0xffffffffu ? n_entries : g * nt + t;
}

// Workgroup stamps of the stamped k_seg (thread 0): the 100 MHz constant
// clock at the start (word 0), at the end after every wave's last store was
// issued (word 1), and once the workgroup's entry is read (word 3; not for
// padding or empty entries), and the workgroup's entry (0xffffffff: padding)
// | row count << 32 (word 2).
template <bool ST>
__device__ __forceinline__ void seg_stamp(const GemmArgs& a, int which, uint64_t v) {
    if constexpr (ST) {
        if (threadIdx.x == 0) {
            a.stamps[static_cast<size_t>(blockIdx.x) * MH_PREFILL_STAMPS + which] = v;
        }
    }
}

template <int RBMAX, int NS, int NBW, int NMAT, bool GATHER, int EPI, bool ST = false>
__global__ __launch_bounds__(kSegWaves * 64, (SegLayout<RBMAX, NBW, NMAT, NS>::LDS <= 80 * 1024 ? 2 : 1))
void k_seg(GemmArgs a, uint32_t n_entries) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lds0 = static_cast<uint32_t>((uintptr_t)((lds_ptr)lds));
    seg_stamp<ST>(a, 0, wall_clock64());
    const uint32_t nt = a.n / (kSegWaves * NBW * 32u);
    // a launch-ordered map names this workgroup's entry directly; otherwise
    // the groups are ranked here (mh::seg_rank_of)
    uint4 blk;
    const uint32_t ent = a.ordered ? static_cast<uint32_t>(blockIdx.x) : balanced_entry(a, n_entries, nt, lds, blk);
    if (ent >= n_entries) {
        seg_stamp<ST>(a, 2, 0xffffffffull);
        seg_stamp<ST>(a, 1, wall_clock64());
        return;
    }
    if (a.blocks == nullptr) {  // dense: entry = (row segment, column tile)
        const uint32_t mr = (ent / nt) * a.dense_bm, nc = (ent % nt) * (kSegWaves * NBW * 32u);
        blk = make_uint4(mr, nc, nc, min(mr + a.dense_bm, a.s_rows));
    } else if (a.ordered) {
        blk = a.blocks[ent];
    }
    const uint32_t m0 = blk.x, brow = blk.y, n0 = blk.z, m_end = blk.w;
    seg_stamp<ST>(a, 2, ent | (static_cast<uint64_t>(m_end > m0 ? m_end - m0 : 0u) << 32));
    if (m0 >= m_end) {
        seg_stamp<ST>(a, 1, wall_clock64());
        return;
    }
    seg_stamp<ST>(a, 3, wall_clock64());
    const uint32_t nrb = (m_end - m0 + 31u) / 32u;
    const uint32_t passes = (nrb + RBMAX - 1u) / RBMAX;
    uint32_t mp0 = m0;
    for (uint32_t p = 0; p < passes; ++p) {
        // balanced passes: this one takes ceil(remaining blocks / remaining passes)
        const uint32_t left = (m_end - mp0 + 31u) / 32u;
        const uint32_t rb = (left + (passes - p) - 1u) / (passes - p);
#define MH_SEG_CASE(R)                                                                      \
    case R:                                                                                 \
        if constexpr (R <= RBMAX) {                                                         \
            seg_pass<R, RBMAX, NS, NBW, NMAT, GATHER, EPI>(a, brow, n0, mp0, m_end, lds0, lane, wave); \
        }                                                                                   \
        break;
        switch (rb) {
            MH_SEG_CASE(1) MH_SEG_CASE(2) MH_SEG_CASE(3) MH_SEG_CASE(4)
            MH_SEG_CASE(5) MH_SEG_CASE(6) MH_SEG_CASE(7) MH_SEG_CASE(8)
            MH_SEG_CASE(9)
            default: break;
        }
#undef MH_SEG_CASE
        mp0 += rb * 32u;
    }
    if constexpr (ST) {
        __syncthreads();
        seg_stamp<ST>(a, 1, wall_clock64());
    }
}

template <int RBMAX, int NS, int NBW, int NMAT, bool GATHER, int EPI>
int launch_seg(const GemmArgs& a, uint32_t n_blocks, hipStream_t s) {
    constexpr size_t lds = SegLayout<RBMAX, NBW, NMAT, NS>::LDS;
    static_assert(lds <= 160 * 1024, "LDS per workgroup");
    // the ranking's entries and weights (balanced_entry) fit the LDS
    const size_t groups = n_blocks / (a.n / (kSegWaves * NBW * 32u)) + 4u;
    MH_ENSURE(a.ordered || groups * 20u <= lds, MH_ERR_UNSUPPORTED, "k_seg: %zu map rows exceed the LDS ranking",
              groups);
    if (a.stamps != nullptr) {
        const uint32_t grid = grid_for_map(n_blocks, a.n / (kSegWaves * NBW * 32u));
        MH_ENSURE(grid <= MH_PREFILL_STAMP_WGS, MH_ERR_UNSUPPORTED, "k_seg: %u workgroups exceed the stamp buffer",
                  grid);
        auto kst = k_seg<RBMAX, NS, NBW, NMAT, GATHER, EPI, true>;
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kst),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) {
            return mh::hip_error(e, "k_seg");
        }
        hipLaunchKernelGGL(kst, dim3(grid), dim3(kSegWaves * 64), lds, s, a, n_blocks);
        return mh::launch_status("k_seg");
    }
    auto kern = k_seg<RBMAX, NS, NBW, NMAT, GATHER, EPI>;
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(lds));
    if (e != hipSuccess) {
        return mh::hip_error(e, "k_seg");
    }
    const uint32_t grid = grid_for_map(n_blocks, a.n / (kSegWaves * NBW * 32u));
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kSegWaves * 64), lds, s, a, n_blocks);
    return mh::launch_status("k_seg");
}

template <int BM, int NBW, int NW, bool GATHER, int EPI>
int launch_t(const GemmArgs& a, uint32_t n_blocks, hipStream_t s) {
    // k_grouped forms A and weight offsets in 32 bits from uniform bases
    MH_ENSURE(static_cast<uint64_t>(a.a_rows) * a.k * 2u < (1ull << 32) &&
                  static_cast<uint64_t>(a.w_rows) * a.k / 2u < (1ull << 32),
              MH_ERR_UNSUPPORTED, "grouped GEMM: A (%u rows x %u) or the weights (%u rows) exceed 4 GiB",
              a.a_rows, a.k, a.w_rows);
    constexpr int NMAT = (EPI == EPI_STORE) ? 1 : 2;
    constexpr size_t lds = static_cast<size_t>(kStages) * (BM * 128 + NW * NMAT * NBW * (1024 + 256));
    auto kern = k_grouped<BM, NBW, NW, GATHER, EPI>;
    if (lds > 64u * 1024u) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 static_cast<int>(lds));
        if (e != hipSuccess) {
            return mh::hip_error(e, "k_grouped");
        }
    }
    const uint32_t grid = grid_for_map(n_blocks, a.n / (NW * NBW * 32u));
    hipLaunchKernelGGL(kern, dim3(grid), dim3(NW * 64), lds, s, a, n_blocks);
    return mh::launch_status("k_grouped");
}

// Tiles: plain (bm x bn) with NBW = 2 column blocks per wave; gate/up tiles
// with one column block per wave and matrix.
template <bool GATHER, int EPI>
int dispatch(const GemmArgs& a, uint32_t n_blocks, uint32_t bm, uint32_t bn, hipStream_t s) {
    MH_ENSURE(bn > 0 && a.n % bn == 0, MH_ERR_INVALID, "grouped GEMM: N %u not a multiple of the tile width %u",
              a.n, bn);
    // segment kernels: 32-bit byte offsets from uniform bases for every
    // operand, 16-byte output stores
    const bool seg = (bm == 256 || bm == 512) && a.k % 512u == 0u &&
                     static_cast<uint64_t>(a.a_rows) * a.k * 2u < (1ull << 32) &&
                     static_cast<uint64_t>(a.w_rows) * a.k / 2u < (1ull << 32) &&
                     static_cast<uint64_t>(a.s_rows) * a.n * 2u < (1ull << 32) &&
                     mh::aligned(a.out0, 16) && (a.out1 == nullptr || mh::aligned(a.out1, 16));
    if (a.stamps != nullptr || a.ordered) {  // launch-ordered maps, measurement: the segment kernels only
        if constexpr (EPI == EPI_STORE) {
            if (seg && bn == 256) return launch_seg<kSegRBMax, kSegStages, 2, 1, GATHER, EPI>(a, n_blocks, s);
        } else {
            if (seg && bn == 128) return launch_seg<kSegRBMax, kSegStages, 1, 2, GATHER, EPI>(a, n_blocks, s);
        }
        return mh::set_error(MH_ERR_UNSUPPORTED, "grouped GEMM: launch-ordered maps and stamps need the segment "
                                                 "kernel's tiles");
    }
    if constexpr (EPI == EPI_STORE) {
        if (bm == 32 && bn == 64) return launch_t<32, 2, 1, GATHER, EPI>(a, n_blocks, s);
        if (bm == 128 && bn == 64) return launch_t<128, 2, 1, GATHER, EPI>(a, n_blocks, s);
        if (bm == 128 && bn == 256) return launch_t<128, 2, 4, GATHER, EPI>(a, n_blocks, s);
        if (seg && bn == 256) return launch_seg<kSegRBMax, kSegStages, 2, 1, GATHER, EPI>(a, n_blocks, s);
    } else {
        if (bm == 32 && bn == 64) return launch_t<32, 1, 2, GATHER, EPI>(a, n_blocks, s);
        if (bm == 128 && bn == 64) return launch_t<128, 1, 2, GATHER, EPI>(a, n_blocks, s);
        if (bm == 128 && bn == 128) return launch_t<128, 1, 4, GATHER, EPI>(a, n_blocks, s);
        if (seg && bn == 128) return launch_seg<kSegRBMax, kSegStages, 1, 2, GATHER, EPI>(a, n_blocks, s);
    }
    return mh::set_error(MH_ERR_UNSUPPORTED, "grouped GEMM: no %ux%u tile for this form", bm, bn);
}

int gemm_checks(const char* op, const uint16_t* a, const mh_quant_weights* w, const void* out,
                const uint32_t* blocks, uint32_t n_blocks, uint32_t s_rows, uint32_t n) {
    MH_TRY(mh::check_quant(w, op));
    MH_ENSURE(a && out && blocks, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(w->bits == 4 && w->group_size == 64 && w->in_features % 64 == 0, MH_ERR_UNSUPPORTED,
              "%s: grouped GEMM needs 4-bit group-64 weights and K %% 64 == 0", op);
    MH_ENSURE(n > 0 && n % 64 == 0, MH_ERR_INVALID, "%s: N %u not a multiple of 64", op, n);
    MH_ENSURE(w->out_features % n == 0, MH_ERR_INVALID,
              "%s: %u stacked weight rows are not a multiple of N %u", op, w->out_features, n);
    MH_ENSURE(n_blocks > 0 && s_rows > 0, MH_ERR_INVALID, "%s: empty block map or output", op);
    MH_ENSURE(mh::aligned(a, 16) && mh::aligned(blocks, 16), MH_ERR_ALIGN,
              "%s: A rows and the block map must be 16-byte aligned", op);
    MH_ENSURE(mh::aligned(out, 2), MH_ERR_ALIGN, "%s: output alignment", op);
    return MH_OK;
}

GemmArgs make_args(const uint16_t* a, const uint32_t* gather, uint32_t a_rows,
                   const mh_quant_weights* w0, const mh_quant_weights* w1, uint16_t* out0,
                   uint16_t* out1, const uint32_t* blocks, uint32_t s_rows, uint32_t n) {
    GemmArgs g{};
    g.a = a;
    g.gather = gather;
    g.c0 = w0->codes; g.s0 = w0->scales; g.b0 = w0->biases;
    if (w1) {
        g.c1 = w1->codes; g.s1 = w1->scales; g.b1 = w1->biases;
    }
    g.out0 = out0;
    g.out1 = out1;
    g.blocks = reinterpret_cast<const uint4*>(blocks);
    g.k = w0->in_features;
    g.n = n;
    g.s_rows = s_rows;
    g.a_rows = a_rows;
    g.w_rows = w0->out_features;
    return g;
}

}  // namespace

namespace mh {

// The prefill step's two grouped GEMMs (as mh_gemm_q4_grouped_gu_act and
// mh_gemm_q4_grouped, the segment kernels only): on a launch-ordered map
// (n_blocks: its map_grid entries) and / or with workgroup stamps.
int gemm_gu_act_seg(const uint16_t* x, const uint32_t* ids_sorted, uint32_t x_rows, const mh_quant_weights* gate,
                    const mh_quant_weights* up, uint16_t* act, const uint32_t* blocks, uint32_t n_blocks,
                    uint32_t s_rows, uint32_t n, uint32_t bm, uint32_t bn, bool ordered, uint64_t* stamps,
                    hipStream_t s) {
    GemmArgs g = make_args(x, ids_sorted, x_rows, gate, up, act, nullptr, blocks, s_rows, n);
    g.ordered = ordered ? 1u : 0u;
    g.stamps = stamps;
    return dispatch<true, EPI_SWIGLU>(g, n_blocks, bm, bn, s);
}

int gemm_grouped_seg(const uint16_t* a, const mh_quant_weights* w, uint16_t* c, const uint32_t* blocks,
                     uint32_t n_blocks, uint32_t s_rows, uint32_t n, uint32_t bm, uint32_t bn, bool ordered,
                     uint64_t* stamps, hipStream_t s) {
    GemmArgs g = make_args(a, nullptr, s_rows, w, nullptr, c, nullptr, blocks, s_rows, n);
    g.ordered = ordered ? 1u : 0u;
    g.stamps = stamps;
    return dispatch<false, EPI_STORE>(g, n_blocks, bm, bn, s);
}

}  // namespace mh

extern "C" {

int mh_gemm_q4_grouped(const uint16_t* a, const mh_quant_weights* w, uint16_t* c,
                       const uint32_t* blocks, uint32_t n_blocks, uint32_t s_rows, uint32_t n,
                       uint32_t bm, uint32_t bn, mh_stream_t stream) {
    MH_TRY(gemm_checks("mh_gemm_q4_grouped", a, w, c, blocks, n_blocks, s_rows, n));
    const GemmArgs g = make_args(a, nullptr, s_rows, w, nullptr, c, nullptr, blocks, s_rows, n);
    return dispatch<false, EPI_STORE>(g, n_blocks, bm, bn, mh::as_stream(stream));
}

int mh_gemm_q4_dense(const uint16_t* a, uint32_t m, const mh_quant_weights* w, uint16_t* c,
                     mh_stream_t stream) {
    const char* op = "mh_gemm_q4_dense";
    MH_TRY(mh::check_quant(w, op));
    MH_ENSURE(a && c, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(w->bits == 4 && w->group_size == 64 && w->in_features % 64 == 0, MH_ERR_UNSUPPORTED,
              "%s: needs 4-bit group-64 weights and K %% 64 == 0", op);
    MH_ENSURE(m > 0, MH_ERR_INVALID, "%s: no rows", op);
    MH_ENSURE(w->out_features % 64 == 0, MH_ERR_UNSUPPORTED, "%s: N %u not a multiple of 64", op,
              w->out_features);
    MH_ENSURE(mh::aligned(a, 16) && mh::aligned(c, 4), MH_ERR_ALIGN, "%s: A 16-byte, C 4-byte alignment", op);
    const uint32_t n = w->out_features;
    GemmArgs g = make_args(a, nullptr, m, w, nullptr, c, nullptr, nullptr, m, n);
    const hipStream_t s = mh::as_stream(stream);
    // segment entries of 256 x 256 when they fill the chip (>= one per CU),
    // else of 128 x 256 when those do (one 4-row-block pass each), provided
    // the segment kernel's 32-bit offsets hold; else 128 x 256 tiles
    const uint32_t segs = (m + 255u) / 256u * (n / 256u);
    const uint32_t segs128 = (m + 127u) / 128u * (n / 256u);
    if (n % 256 == 0 && segs128 >= 256u && w->in_features % 512u == 0 &&
        static_cast<uint64_t>(m) * w->in_features * 2u < (1ull << 32) &&
        static_cast<uint64_t>(n) * w->in_features / 2u < (1ull << 32) &&
        static_cast<uint64_t>(m) * n * 2u < (1ull << 32) && mh::aligned(c, 16)) {
        g.dense_bm = segs >= 256u ? 256u : 128u;
        return launch_seg<kSegRBMax, kSegStages, 2, 1, false, EPI_STORE>(g, segs >= 256u ? segs : segs128, s);
    }
    const uint32_t mt = (m + 127u) / 128u;
    if (n % 256 == 0) {
        return launch_t<128, 2, 4, false, EPI_STORE>(g, mt * (n / 256u), s);
    }
    return launch_t<128, 2, 1, false, EPI_STORE>(g, mt * (n / 64u), s);
}

int mh_gemm_q4_grouped_gu(const uint16_t* a, const mh_quant_weights* gate,
                          const mh_quant_weights* up, uint16_t* gate_out, uint16_t* up_out,
                          const uint32_t* blocks, uint32_t n_blocks, uint32_t s_rows, uint32_t n,
                          uint32_t bm, uint32_t bn, mh_stream_t stream) {
    const char* op = "mh_gemm_q4_grouped_gu";
    MH_TRY(gemm_checks(op, a, gate, gate_out, blocks, n_blocks, s_rows, n));
    MH_TRY(mh::check_quant(up, op));
    MH_ENSURE(up_out != nullptr, MH_ERR_INVALID, "%s: up_out is NULL", op);
    MH_ENSURE(up->out_features == gate->out_features && up->in_features == gate->in_features &&
                  up->bits == 4 && up->group_size == 64,
              MH_ERR_INVALID, "%s: gate/up shapes differ", op);
    const GemmArgs g = make_args(a, nullptr, s_rows, gate, up, gate_out, up_out, blocks, s_rows, n);
    return dispatch<false, EPI_GATE_UP>(g, n_blocks, bm, bn, mh::as_stream(stream));
}

int mh_gemm_q4_grouped_gu_act(const uint16_t* x, const uint32_t* ids_sorted, uint32_t x_rows,
                              const mh_quant_weights* gate, const mh_quant_weights* up,
                              uint16_t* act, const uint32_t* blocks, uint32_t n_blocks,
                              uint32_t s_rows, uint32_t n, uint32_t bm, uint32_t bn,
                              mh_stream_t stream) {
    const char* op = "mh_gemm_q4_grouped_gu_act";
    MH_TRY(gemm_checks(op, x, gate, act, blocks, n_blocks, s_rows, n));
    MH_TRY(mh::check_quant(up, op));
    MH_ENSURE(x_rows > 0, MH_ERR_INVALID, "%s: x has no rows", op);
    MH_ENSURE(up->out_features == gate->out_features && up->in_features == gate->in_features &&
                  up->bits == 4 && up->group_size == 64,
              MH_ERR_INVALID, "%s: gate/up shapes differ", op);
    const GemmArgs g = make_args(x, ids_sorted, ids_sorted ? x_rows : s_rows, gate, up, act, nullptr,
                                 blocks, s_rows, n);
    const hipStream_t s = mh::as_stream(stream);
    return ids_sorted ? dispatch<true, EPI_SWIGLU>(g, n_blocks, bm, bn, s)
                      : dispatch<false, EPI_SWIGLU>(g, n_blocks, bm, bn, s);
}

// The launch-ordered forms: entry b of the map is workgroup b's (a whole
// number of 8 x (n / bn) units), segment tiles only.
static int ordered_checks(const char* op, uint32_t n_entries, uint32_t n, uint32_t bn) {
    MH_ENSURE(n_entries % (8u * (n / bn)) == 0u, MH_ERR_INVALID,
              "%s: a launch-ordered map holds whole units of 8 x %u entries, not %u", op, n / bn, n_entries);
    return MH_OK;
}

int mh_gemm_q4_grouped_ordered(const uint16_t* a, const mh_quant_weights* w, uint16_t* c, const uint32_t* ord,
                               uint32_t n_entries, uint32_t s_rows, uint32_t n, uint32_t bm, uint32_t bn,
                               mh_stream_t stream) {
    const char* op = "mh_gemm_q4_grouped_ordered";
    MH_TRY(gemm_checks(op, a, w, c, ord, n_entries, s_rows, n));
    MH_ENSURE(bn == 256u && n % bn == 0u, MH_ERR_UNSUPPORTED, "%s: tile width %u (256 only)", op, bn);
    MH_TRY(ordered_checks(op, n_entries, n, bn));
    return mh::gemm_grouped_seg(a, w, c, ord, n_entries, s_rows, n, bm, bn, true, nullptr, mh::as_stream(stream));
}

int mh_gemm_q4_grouped_gu_act_ordered(const uint16_t* x, const uint32_t* ids_sorted, uint32_t x_rows,
                                      const mh_quant_weights* gate, const mh_quant_weights* up, uint16_t* act,
                                      const uint32_t* ord, uint32_t n_entries, uint32_t s_rows, uint32_t n,
                                      uint32_t bm, uint32_t bn, mh_stream_t stream) {
    const char* op = "mh_gemm_q4_grouped_gu_act_ordered";
    MH_TRY(gemm_checks(op, x, gate, act, ord, n_entries, s_rows, n));
    MH_TRY(mh::check_quant(up, op));
    MH_ENSURE(ids_sorted != nullptr && x_rows > 0, MH_ERR_INVALID, "%s: needs ids_sorted and x rows", op);
    MH_ENSURE(up->out_features == gate->out_features && up->in_features == gate->in_features &&
                  up->bits == 4 && up->group_size == 64,
              MH_ERR_INVALID, "%s: gate/up shapes differ", op);
    MH_ENSURE(bn == 128u && n % bn == 0u, MH_ERR_UNSUPPORTED, "%s: tile width %u (128 only)", op, bn);
    MH_TRY(ordered_checks(op, n_entries, n, bn));
    return mh::gemm_gu_act_seg(x, ids_sorted, x_rows, gate, up, act, ord, n_entries, s_rows, n, bm, bn, true,
                               nullptr, mh::as_stream(stream));
}

}  // extern "C"

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
//     staged once per workgroup in double-buffered LDS, 64 k at a time, row
//     pitch 72 bf16 (conflict-free 16-byte reads);
//   * k is permuted identically for A and B inside each 64-k block: lane
//     half h and MFMA step j use k = 32h + 8j + t, so a lane's codes for a
//     block are one 16-byte load.
// Epilogues: store C; store gate and up separately; or SwiGLU
// act = bf16(bf16(silu(bf16 g)) * bf16 u) with two accumulators per tile.
#include "mh_device.hpp"
#include "mh_host.hpp"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kBK = 64;

enum Epi { EPI_STORE = 0, EPI_GATE_UP = 1, EPI_SWIGLU = 2 };

struct GemmArgs {
    const uint16_t* a;       // [a_rows, k] bf16
    const uint32_t* gather;  // row i of the tile reads a[gather[i]]; null: a[i]
    const uint32_t* c0; const uint16_t* s0; const uint16_t* b0;  // gate / the matrix
    const uint32_t* c1; const uint16_t* s1; const uint16_t* b1;  // up
    uint16_t* out0;          // [s_rows, n]: C, gate, or act
    uint16_t* out1;          // [s_rows, n]: up (EPI_GATE_UP)
    const uint4* blocks;
    uint32_t k, n, s_rows, a_rows, w_rows;
};

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

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

typedef __attribute__((address_space(3))) void* lds_ptr;
typedef const __attribute__((address_space(1))) void* glb_ptr;

constexpr int kStages = 3;  // LDS ring depth: two K-blocks in flight while one is consumed

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// 16-byte LDS read issued without a wait: the caller waits with lds_wait.
// (Written as asm so the compiler does not wait for every outstanding
// direct-to-LDS load before it.)
__device__ __forceinline__ uint4 lds_read16(uint32_t addr) {
    uint4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}

// Direct-to-LDS 16-byte load: lane l's data lands at lds_base + 16 l.
__device__ __forceinline__ void dma16(mh::gbytes src, uint32_t lds_base) {
    __builtin_amdgcn_global_load_lds((glb_ptr)src, (lds_ptr)(uintptr_t)lds_base, 16, 0, 0);
}
// Direct-to-LDS 4-byte load: lane l's dword lands at lds_base + 4 l.
__device__ __forceinline__ void dma4(mh::gbytes src, uint32_t lds_base) {
    __builtin_amdgcn_global_load_lds((glb_ptr)src, (lds_ptr)(uintptr_t)lds_base, 4, 0, 0);
}
__device__ __forceinline__ uint32_t lds_read4(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}

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
// are taken XCD by XCD: workgroup i runs entry (i % 8) * L + i / 8, so the
// entries that share A rows (one expert's row tile across its column tiles)
// run on one XCD and hit its L2.
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

    const uint32_t per_xcd = (n_entries + 7u) / 8u;
    const uint32_t ent = (blockIdx.x % 8u) * per_xcd + blockIdx.x / 8u;
    if (ent >= n_entries) {
        return;
    }
    const uint4 blk = a.blocks[ent];
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

    // 32-bit byte offsets from wave-uniform bases (the host checks that the
    // operands fit in 4 GiB), so each load is scalar base + vector offset.
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
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
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
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
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

template <int BM, int NBW, int NW, bool GATHER, int EPI>
int launch_t(const GemmArgs& a, uint32_t n_blocks, hipStream_t s) {
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
    const uint32_t grid = (n_blocks + 7u) / 8u * 8u;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(NW * 64), lds, s, a, n_blocks);
    return mh::launch_status("k_grouped");
}

// Tiles: plain (bm x bn) with NBW = 2 column blocks per wave; gate/up tiles
// with one column block per wave and matrix.
template <bool GATHER, int EPI>
int dispatch(const GemmArgs& a, uint32_t n_blocks, uint32_t bm, uint32_t bn, hipStream_t s) {
    if constexpr (EPI == EPI_STORE) {
        if (bm == 32 && bn == 64) return launch_t<32, 2, 1, GATHER, EPI>(a, n_blocks, s);
        if (bm == 128 && bn == 64) return launch_t<128, 2, 1, GATHER, EPI>(a, n_blocks, s);
        if (bm == 128 && bn == 256) return launch_t<128, 2, 4, GATHER, EPI>(a, n_blocks, s);
    } else {
        if (bm == 32 && bn == 64) return launch_t<32, 1, 2, GATHER, EPI>(a, n_blocks, s);
        if (bm == 128 && bn == 64) return launch_t<128, 1, 2, GATHER, EPI>(a, n_blocks, s);
        if (bm == 128 && bn == 128) return launch_t<128, 1, 4, GATHER, EPI>(a, n_blocks, s);
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

extern "C" {

int mh_gemm_q4_grouped(const uint16_t* a, const mh_quant_weights* w, uint16_t* c,
                       const uint32_t* blocks, uint32_t n_blocks, uint32_t s_rows, uint32_t n,
                       uint32_t bm, uint32_t bn, mh_stream_t stream) {
    MH_TRY(gemm_checks("mh_gemm_q4_grouped", a, w, c, blocks, n_blocks, s_rows, n));
    const GemmArgs g = make_args(a, nullptr, s_rows, w, nullptr, c, nullptr, blocks, s_rows, n);
    return dispatch<false, EPI_STORE>(g, n_blocks, bm, bn, mh::as_stream(stream));
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

}  // extern "C"

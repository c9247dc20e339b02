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
constexpr int kAPitch = kBK + 8;  // bf16 elements per LDS row

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

template <int BM, int NBW, int WAVES, bool GATHER, int EPI>
__global__ __launch_bounds__(WAVES * 64) void k_grouped(GemmArgs a) {
    constexpr int kThr = WAVES * 64;
    constexpr int RB = BM / 32;
    constexpr int NMAT = (EPI == EPI_STORE) ? 1 : 2;
    constexpr int SEGS = (BM * 8 + kThr - 1) / kThr;  // 16-byte A segments per thread per block
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kAPitch];

    const uint4 blk = a.blocks[blockIdx.x];
    const uint32_t m0 = blk.x, brow = blk.y, n0 = blk.z, m_end = blk.w;
    if (m0 >= m_end) {
        return;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i32 = lane & 31, h = lane >> 5;
    const uint32_t K = a.k, nkb = K / kBK;
    const uint32_t words = K / 8u, groups = K / 64u;

    // ---- A staging
    uint4 ra[SEGS];
    size_t arow[SEGS];
    int lrow[SEGS], lseg[SEGS];
    bool lval[SEGS];
#pragma unroll
    for (int i = 0; i < SEGS; ++i) {
        const int idx = threadIdx.x + i * kThr;
        lval[i] = idx < BM * 8;
        lrow[i] = idx / 8;
        lseg[i] = idx % 8;
        const uint32_t m = min(m0 + static_cast<uint32_t>(lrow[i]), m_end - 1);
        uint32_t src = m;
        if (GATHER) {
            src = a.gather[m];
        }
        src = min(src, a.a_rows - 1);
        arow[i] = static_cast<size_t>(src) * K;
    }
    auto load_a = [&](uint32_t kb) {
#pragma unroll
        for (int i = 0; i < SEGS; ++i) {
            if (lval[i]) {
                ra[i] = *reinterpret_cast<const uint4*>(a.a + arow[i] + kb * kBK + 8 * lseg[i]);
            }
        }
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int i = 0; i < SEGS; ++i) {
            if (lval[i]) {
                *reinterpret_cast<uint4*>(&As[buf][lrow[i] * kAPitch + 8 * lseg[i]]) = ra[i];
            }
        }
    };

    // ---- B: this lane's weight rows (one per column block and matrix)
    size_t wrow[NMAT][NBW];
#pragma unroll
    for (int cb = 0; cb < NBW; ++cb) {
        const uint32_t r = min(brow + static_cast<uint32_t>(wave * 32 * NBW + cb * 32 + i32), a.w_rows - 1);
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat) {
            wrow[mat][cb] = r;
        }
    }
    uint4 bc[NMAT][NBW];
    float bs[NMAT][NBW], bb[NMAT][NBW];
    auto load_b = [&](uint32_t kb, uint4(&c)[NMAT][NBW], float(&s)[NMAT][NBW], float(&b)[NMAT][NBW]) {
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat) {
            const uint32_t* cp = mat == 0 ? a.c0 : a.c1;
            const uint16_t* sp = mat == 0 ? a.s0 : a.s1;
            const uint16_t* bp = mat == 0 ? a.b0 : a.b1;
#pragma unroll
            for (int cb = 0; cb < NBW; ++cb) {
                const size_t r = wrow[mat][cb];
                c[mat][cb] = *reinterpret_cast<const uint4*>(cp + r * words + 8u * kb + 4u * h);
                s[mat][cb] = mh::bf16_to_f32(sp[r * groups + kb]);
                b[mat][cb] = mh::bf16_to_f32(bp[r * groups + kb]);
            }
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

    load_a(0);
    load_b(0, bc, bs, bb);
    store_a(0);
    __syncthreads();

    for (uint32_t kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        const bool more = kb + 1 < nkb;
        uint4 nc[NMAT][NBW];
        float ns[NMAT][NBW], nb[NMAT][NBW];
        if (more) {
            load_a(kb + 1);
            load_b(kb + 1, nc, ns, nb);
        }
        bf16x8_t bf[NMAT][NBW][4];
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
            for (int cb = 0; cb < NBW; ++cb) {
                const float s = bs[mat][cb], s16 = s * 0.0625f, b = bb[mat][cb];
                const uint32_t wv[4] = {bc[mat][cb].x, bc[mat][cb].y, bc[mat][cb].z, bc[mat][cb].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) bf[mat][cb][j] = deq_word(wv[j], s, s16, b);
            }
        const uint16_t* at = As[buf];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const uint4 av = *reinterpret_cast<const uint4*>(at + (rb * 32 + i32) * kAPitch + 32 * h + 8 * j);
                const bf16x8_t af = __builtin_bit_cast(bf16x8_t, av);
#pragma unroll
                for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                    for (int cb = 0; cb < NBW; ++cb)
                        acc[mat][rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            af, bf[mat][cb][j], acc[mat][rb][cb], 0, 0, 0);
            }
        }
        if (more) {
            store_a(buf ^ 1);
#pragma unroll
            for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
                for (int cb = 0; cb < NBW; ++cb) {
                    bc[mat][cb] = nc[mat][cb];
                    bs[mat][cb] = ns[mat][cb];
                    bb[mat][cb] = nb[mat][cb];
                }
        }
        __syncthreads();
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
                const size_t o = static_cast<size_t>(row) * a.n + n0 + wave * 32 * NBW + cb * 32 + i32;
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

template <int BM, int NBW, int WAVES, bool GATHER, int EPI>
int launch_t(const GemmArgs& a, uint32_t n_blocks, hipStream_t s) {
    hipLaunchKernelGGL((k_grouped<BM, NBW, WAVES, GATHER, EPI>), dim3(n_blocks), dim3(WAVES * 64), 0,
                       s, a);
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

// gemm_bf16.hip -- dense bf16 GEMM C[M, N] = A[M, K] . B[N, K]^T with f32
// accumulation on the gfx950 matrix cores, and the generic quantized GEMM
// built on it (dequantize W into a caller scratch, then the GEMM).
//
// Replaces src/kernels/gemm.rs:33-60 gemm_bf16_nt (gemm.metal's NAX tile
// GEMMs) and src/kernels/quant.rs:126-146 gemm_quant_bf16_nt, so that
// src/lfm.rs:649-675 `project` keeps all three of its branches.
//
// Work split: 256 x 128 output tiles (128 x 128 when the larger ones give
// fewer tiles than CUs), one workgroup of 4 waves each (a 2 x 2 grid of
// 128 x 64 or 64 x 64 wave tiles, v_mfma_f32_32x32x16_bf16 accumulators).  K advances 64 at a time through a 3-slot LDS ring filled by
// direct-to-LDS 16-byte loads (global_load_lds_dwordx4): the A and B tiles
// are both rows of K, so both are staged the same way, 16-byte chunks
// XOR-swizzled by row so that the fragment reads are bank-conflict free.
// Within each 64-k block, MFMA step j of lane half h uses k = 32 h + 8 j +
// (0..7) for A and B alike (a permutation of k inside the block: the dot
// products are unchanged), so a lane's fragment is one 16-byte read.  Tiles
// are dealt to the 8 XCDs in contiguous runs (tile t on XCD t / per_xcd), so
// the tiles of one row of C run on one XCD and share its L2 copy of A.
// Rows of A or B past M or N are clamped (loaded, never stored).
//
// Shapes the tile kernel does not take (K % 64 != 0, operands not 16-byte
// aligned, or 4 GiB and larger) run a plain per-element kernel, f32 fma in
// ascending k.
#include "mh_device.hpp"
#include "mh_host.hpp"
#include "mh_mfma.hpp"

namespace {

constexpr int kTileN = 128;  // output columns per tile
constexpr int kBK = 64;
constexpr int kThreads = 256;
constexpr int kStages = 3;

// Tiles of TM (128 or 256) rows x 128 columns: the 4 waves form a 2 x 2 grid
// of (TM / 2) x 64 wave tiles, RB = TM / 64 row blocks of 32 by two column
// blocks of 32 each.  The larger tile reads 0.75 KB of LDS fragments per
// MFMA instead of 1 KB.
template <int TM>
struct NtShape {
    static constexpr int RB = TM / 64;                          // 32-row blocks per wave
    static constexpr uint32_t A_BYTES = TM * kBK * 2;           // A's TM x 64 bf16 block
    static constexpr uint32_t B_BYTES = kTileN * kBK * 2;       // B's 128 x 64 bf16 block
    static constexpr uint32_t STAGE = A_BYTES + B_BYTES;
    static constexpr uint32_t LDS = kStages * STAGE;            // 96 KB (TM 128), 144 KB (TM 256)
    static constexpr int QA = TM / 32, QB = kTileN / 32;        // 1 KB loads per wave per stage
    static constexpr int OPS = QA + QB;
    static constexpr int HALF_READS = 2 * (RB + 2);             // fragment reads of steps 0-1
    static_assert(HALF_READS <= 15, "lgkmcnt field");
};

struct NtArgs {
    const uint16_t* a;  // [m, k]
    const uint16_t* b;  // [n, k]
    uint16_t* c;        // [m, n]
    uint32_t m, n, k;
    uint32_t tiles_n, tiles, per_xcd;
};

template <int TM>
__global__ __launch_bounds__(kThreads, 1) void k_gemm_nt(NtArgs p) {
    using S = NtShape<TM>;
    constexpr int RB = S::RB;
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const uint32_t t = (blockIdx.x % 8u) * p.per_xcd + blockIdx.x / 8u;
    if (t >= p.tiles) {
        return;
    }
    const uint32_t m0 = (t / p.tiles_n) * TM, n0 = (t % p.tiles_n) * kTileN;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i32 = lane & 31, h = lane >> 5;
    const uint32_t K = p.k, nkb = K / kBK;
    const uint32_t lds0 = static_cast<uint32_t>((uintptr_t)((mh::lds_ptr)lds));
    const mh::gbytes abase = mh::uniform_ptr(p.a);
    const mh::gbytes bbase = mh::uniform_ptr(p.b);

    // this lane's A and B loads per stage: row r of the block, 16-byte chunk
    // (lane & 7) of its LDS row, holding global chunk (lane & 7) ^ (r & 7)
    uint32_t aoff[S::QA], boff[S::QB];
#pragma unroll
    for (int q = 0; q < S::QA; ++q) {
        const uint32_t r = 8u * static_cast<uint32_t>(wave * S::QA + q) + static_cast<uint32_t>(lane >> 3);
        const uint32_t chunk = static_cast<uint32_t>(lane & 7) ^ (r & 7u);
        aoff[q] = min(m0 + r, p.m - 1u) * K * 2u + chunk * 16u;
    }
#pragma unroll
    for (int q = 0; q < S::QB; ++q) {
        const uint32_t r = 8u * static_cast<uint32_t>(wave * S::QB + q) + static_cast<uint32_t>(lane >> 3);
        const uint32_t chunk = static_cast<uint32_t>(lane & 7) ^ (r & 7u);
        boff[q] = min(n0 + r, p.n - 1u) * K * 2u + chunk * 16u;
    }
    auto issue = [&](uint32_t kb, int slot) {
        const uint32_t base = lds0 + static_cast<uint32_t>(slot) * S::STAGE;
#pragma unroll
        for (int q = 0; q < S::QA; ++q) {
            mh::dma16(abase + aoff[q] + kb * 128u, base + static_cast<uint32_t>(wave * S::QA + q) * 1024u);
        }
#pragma unroll
        for (int q = 0; q < S::QB; ++q) {
            mh::dma16(bbase + boff[q] + kb * 128u, base + S::A_BYTES + static_cast<uint32_t>(wave * S::QB + q) * 1024u);
        }
    };

    // fragment addresses inside a stage: row (col) of the wave's block, chunk 4h + j
    const uint32_t wr = static_cast<uint32_t>(wave >> 1) * (TM / 2u), wc = static_cast<uint32_t>(wave & 1) * 64u;
    uint32_t afr[RB][4], bfr[2][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t c = static_cast<uint32_t>(4 * h + j);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const uint32_t ra = wr + rb * 32u + static_cast<uint32_t>(i32);
            afr[rb][j] = ra * 128u + ((c ^ (ra & 7u)) * 16u);
        }
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const uint32_t rbn = wc + cb * 32u + static_cast<uint32_t>(i32);
            bfr[cb][j] = S::A_BYTES + rbn * 128u + ((c ^ (rbn & 7u)) * 16u);
        }
    }

    mh::f32x16_t acc[RB][2];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[rb][cb][q] = 0.0f;

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
            // this wave's loads of stage kb are in (the next stage's may be
            // in flight); the barrier publishes every wave's and frees the
            // slot the next issue overwrites
            if (kb + 1 < nkb) {
                mh::wait_vmcnt<S::OPS>();
            } else {
                mh::wait_vmcnt<0>();
            }
            __builtin_amdgcn_s_barrier();
            if (kb + kStages - 1 < nkb) {
                issue(kb + kStages - 1, (u + kStages - 1) % kStages);
            }
            const uint32_t base = lds0 + static_cast<uint32_t>(u) * S::STAGE;
            // two halves of the stage (steps 0-1, 2-3): the second half's
            // fragment reads are in flight under the first half's MFMAs
            uint4 av[2][2][RB], bv[2][2][2];  // [half][step][rb / cb]
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) {
                        av[hf][jj][rb] = mh::lds_read16(base + afr[rb][2 * hf + jj]);
                    }
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb) {
                        bv[hf][jj][cb] = mh::lds_read16(base + bfr[cb][2 * hf + jj]);
                    }
                }
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                // the waits are tied to the fragment registers, so that no
                // MFMA reading them is scheduled above them (hf 0: the
                // second half's reads may still be in flight)
                if (hf == 0) {
                    mh::lgkm_wait<S::HALF_READS>(reinterpret_cast<uint4(&)[2 * RB]>(av[0]));
                    mh::lgkm_wait<S::HALF_READS>(reinterpret_cast<uint4(&)[4]>(bv[0]));
                } else {
                    mh::lgkm_wait<0>(reinterpret_cast<uint4(&)[2 * RB]>(av[1]));
                    mh::lgkm_wait<0>(reinterpret_cast<uint4(&)[4]>(bv[1]));
                }
#pragma unroll
                for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                        for (int cb = 0; cb < 2; ++cb)
                            acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                __builtin_bit_cast(mh::bf16x8_t, av[hf][jj][rb]),
                                __builtin_bit_cast(mh::bf16x8_t, bv[hf][jj][cb]), acc[rb][cb], 0, 0, 0);
            }
        }
    }

    // D lane layout: row 8 (q / 4) + 4 h + q % 4, column i32
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const uint32_t row = m0 + wr + rb * 32u + 8u * (q / 4) + 4u * h + (q % 4);
                const uint32_t col = n0 + wc + cb * 32u + static_cast<uint32_t>(i32);
                if (row < p.m && col < p.n) {
                    p.c[static_cast<size_t>(row) * p.n + col] = mh::f32_to_bf16(acc[rb][cb][q]);
                }
            }
}

__global__ __launch_bounds__(256) void k_gemm_nt_plain(const uint16_t* a, const uint16_t* b, uint16_t* c, uint32_t m,
                                                       uint32_t n, uint32_t k) {
    const size_t total = static_cast<size_t>(m) * n;
    for (size_t e = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
         e += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const size_t row = e / n, col = e % n;
        const uint16_t* ar = a + row * k;
        const uint16_t* br = b + col * k;
        float s = 0.0f;
        for (uint32_t i = 0; i < k; ++i) {
            s = __builtin_fmaf(mh::bf16_to_f32(ar[i]), mh::bf16_to_f32(br[i]), s);
        }
        c[e] = mh::f32_to_bf16(s);
    }
}

int gemm_nt(const char* op, const uint16_t* a, const uint16_t* b, uint16_t* c, uint32_t m, uint32_t n, uint32_t k,
            hipStream_t s) {
    const bool tiled = k % kBK == 0 && mh::aligned(a, 16) && mh::aligned(b, 16) &&
                       static_cast<uint64_t>(m) * k * 2u < (1ull << 32) &&
                       static_cast<uint64_t>(n) * k * 2u < (1ull << 32);
    if (!tiled) {
        const size_t total = static_cast<size_t>(m) * n;
        const size_t want = (total + 255) / 256;
        const size_t cap = static_cast<size_t>(mh::cu_count()) * 8;
        hipLaunchKernelGGL(k_gemm_nt_plain, dim3(static_cast<unsigned>(want < cap ? want : cap)), dim3(256), 0, s, a,
                           b, c, m, n, k);
        return mh::launch_status(op);
    }
    NtArgs p{};
    p.a = a;
    p.b = b;
    p.c = c;
    p.m = m;
    p.n = n;
    p.k = k;
    p.tiles_n = (n + kTileN - 1) / kTileN;
    // 256-row tiles when they still give every CU one
    const uint32_t tiles256 = ((m + 255u) / 256u) * p.tiles_n;
    const bool big = tiles256 >= static_cast<uint32_t>(mh::cu_count());
    const uint32_t tm = big ? 256u : 128u;
    p.tiles = ((m + tm - 1) / tm) * p.tiles_n;
    p.per_xcd = (p.tiles + 7u) / 8u;
    // the attribute is set on every tiled launch (a cheap host call): no
    // shared flag for concurrent callers to race on, and right on every device
    const void* kern = big ? reinterpret_cast<const void*>(k_gemm_nt<256>) : reinterpret_cast<const void*>(k_gemm_nt<128>);
    const uint32_t lds = big ? NtShape<256>::LDS : NtShape<128>::LDS;
    const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) {
        return mh::hip_error(e, op);
    }
    if (big) {
        hipLaunchKernelGGL(k_gemm_nt<256>, dim3(8u * p.per_xcd), dim3(kThreads), lds, s, p);
    } else {
        hipLaunchKernelGGL(k_gemm_nt<128>, dim3(8u * p.per_xcd), dim3(kThreads), lds, s, p);
    }
    return mh::launch_status(op);
}

}  // namespace

extern "C" {

int mh_gemm_bf16_nt(const uint16_t* a, const uint16_t* b, uint16_t* c, uint32_t m, uint32_t n, uint32_t k,
                    mh_stream_t stream) {
    MH_ENSURE(a != nullptr && b != nullptr && c != nullptr, MH_ERR_INVALID, "mh_gemm_bf16_nt: NULL operand");
    MH_ENSURE(mh::aligned(a, 2) && mh::aligned(b, 2) && mh::aligned(c, 2), MH_ERR_ALIGN,
              "mh_gemm_bf16_nt: operands not 2-byte aligned");
    MH_ENSURE(k > 0 || m == 0 || n == 0, MH_ERR_INVALID, "mh_gemm_bf16_nt: K is 0");
    if (m == 0 || n == 0) {
        return MH_OK;
    }
    return gemm_nt("mh_gemm_bf16_nt", a, b, c, m, n, k, mh::as_stream(stream));
}

int mh_gemm_quant_bf16_nt(const uint16_t* a, uint32_t m, const mh_quant_weights* w, uint16_t* c, uint16_t* scratch,
                          size_t scratch_elems, mh_stream_t stream) {
    MH_TRY(mh::check_quant_dequant(w, "mh_gemm_quant_bf16_nt"));
    MH_ENSURE(a != nullptr && c != nullptr && scratch != nullptr, MH_ERR_INVALID,
              "mh_gemm_quant_bf16_nt: NULL operand");
    const size_t need = static_cast<size_t>(w->out_features) * w->in_features;
    MH_ENSURE(scratch_elems >= need, MH_ERR_INVALID,
              "dequant scratch holds %zu bf16 elements, needs %zu", scratch_elems, need);
    MH_ENSURE(mh::aligned(scratch, 16), MH_ERR_ALIGN, "mh_gemm_quant_bf16_nt: scratch not 16-byte aligned");
    MH_ENSURE(mh::aligned(a, 2) && mh::aligned(c, 2), MH_ERR_ALIGN, "mh_gemm_quant_bf16_nt: a/c not 2-byte aligned");
    if (m == 0) {
        return MH_OK;
    }
    MH_TRY(mh_dequant_to_bf16(w, scratch, stream));
    return gemm_nt("mh_gemm_quant_bf16_nt", a, scratch, c, m, w->out_features, w->in_features,
                   mh::as_stream(stream));
}

}  // extern "C"

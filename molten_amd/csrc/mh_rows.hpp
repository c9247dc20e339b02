// mh_rows.hpp -- the batch-1 row-block walk of the decode GEMV epilogue
// variants (src/kernels/lfm.rs proj3_gemv_scatter, conv3_gemv): a wave
// computes kBlockRows consecutive rows of one quantized matrix at a time,
// lane c owning the 32-code chunk c of every row (K <= 2048) with x in
// registers -- the arithmetic of k_gemv_rows (gemv.hip), which keeps its own
// copy of the loop so that its x loads stay in flight across its first
// block's loads.
#pragma once
#include "mh_device.hpp"

namespace mh {

constexpr int kBlockRows = 8;
constexpr int kGroupRows = 4;
constexpr int kMaxGroups = 64;  // K / group size <= 2048 / 32

// One quantized matrix as the walk reads it.
struct RowMatrix {
    const char* codes;       // row r at codes + r * row_bytes
    const uint16_t* scales;  // [rows, G]
    const uint16_t* biases;
};

// The lane's fixed part of the walk.  FAST: K == 2048 and group size 64
// (every lane owns a chunk, 32 groups per row, blocks always full).
template <int BITS, bool FAST>
struct RowWalk {
    uint32_t G;          // groups per row
    uint32_t row_bytes;  // code bytes per row
    uint32_t code_off;   // byte offset of the lane's chunk in a row
    uint32_t gc;         // the lane's group
    bool live;           // the lane owns a chunk
    int lane;
    uint32_t* sb;        // the wave's LDS: kBlockRows * G (scale | bias << 16) words

    __device__ __forceinline__ void init(uint32_t k, uint32_t gs, uint32_t groups, uint32_t row_words, uint32_t* lds,
                                         int lane_) {
        lane = lane_;
        const uint32_t C = k / 32u;
        live = FAST || static_cast<uint32_t>(lane) < C;
        const uint32_t c = live ? static_cast<uint32_t>(lane) : 0u;
        G = FAST ? 32u : groups;
        row_bytes = FAST ? 2048u * BITS / 8u : row_words * 4u;
        code_off = c * BITS * 4u;
        gc = FAST ? static_cast<uint32_t>(lane) / 2u : (32u * c) / gs;
        sb = lds;
    }
    __device__ __forceinline__ uint32_t chunk() const { return live ? static_cast<uint32_t>(lane) : 0u; }

    // Rows row0 .. row0 + nrows - 1 (nrows <= 4 NG; FAST: == 4 NG) of m: the
    // block's scales and biases are read with a few word loads and staged in
    // LDS as (scale | bias << 16) words; the codes of the block's NG row
    // groups are loaded non-temporally (each byte is read once), group 1
    // while group 0 is computed; each group's four row values are reduced
    // together.  Lane j < nrows receives row row0 + j's f32 sum in the chunk
    // order.  prep() runs once the first group's loads are out (the caller
    // may finish preparing xr / xs there).
    template <int NG = 2, typename Prep>
    __device__ __forceinline__ float block(const RowMatrix& m, uint32_t row0, uint32_t nrows, float (&xr)[32],
                                           float& xs, Prep&& prep) const {
        static_assert(NG == 1 || NG == 2, "one or two 4-row groups");
        constexpr int R = kGroupRows, BR = NG * R;
        const uint32_t nd = nrows * G / 2u;
        const uint32_t* s2 = reinterpret_cast<const uint32_t*>(m.scales + static_cast<size_t>(row0) * G);
        const uint32_t* b2 = reinterpret_cast<const uint32_t*>(m.biases + static_cast<size_t>(row0) * G);
        const char* codes = m.codes + static_cast<size_t>(row0) * row_bytes;
        auto load = [&](int grp, Chunk<BITS>(&ch)[R]) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t rr = FAST ? grp * R + r : min(static_cast<uint32_t>(grp * R + r), nrows - 1u);
                ch[r].load_nt(uniform_ptr(codes + rr * row_bytes), code_off);
            }
        };
        // scale / bias words (clamped indices: every lane loads, no branch),
        // then the first group's codes, then the words into LDS (a wait for
        // the words only); entries past the block are never read
        constexpr int NSB = BR * (FAST ? 32 : kMaxGroups) / 128;
        uint32_t sw[NSB], bw[NSB];
#pragma unroll
        for (int j = 0; j < NSB; ++j) {
            const uint32_t i = lane + kWave * j;
            const uint32_t ic = FAST || i < nd ? i : nd - 1u;
            sw[j] = s2[ic];
            bw[j] = b2[ic];
        }
        Chunk<BITS> A[R], Bc[R];
        load(0, A);
#pragma unroll
        for (int j = 0; j < NSB; ++j) {
            const uint32_t i = lane + kWave * j;
            *reinterpret_cast<uint2*>(sb + 2u * i) =
                make_uint2(__builtin_amdgcn_perm(bw[j], sw[j], 0x05040100u),   // s.lo | b.lo << 16
                           __builtin_amdgcn_perm(bw[j], sw[j], 0x07060302u));  // s.hi | b.hi << 16
        }
        float yv = 0.0f;
        auto compute = [&](int grp, const Chunk<BITS>(&ch)[R]) {
            float h[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t rr = FAST ? grp * R + r : min(static_cast<uint32_t>(grp * R + r), nrows - 1u);
                const uint32_t w = sb[rr * G + gc];
                const float p = ch[r].dot(xr);
                const float hv = __builtin_fmaf(__uint_as_float(w << 16), p, __uint_as_float(w & 0xffff0000u) * xs);
                h[r] = live ? 0.0f + hv : 0.0f;
            }
            const float v = reduce_rows4(h, lane);
            const float mv = __int_as_float(__builtin_amdgcn_ds_bpermute((60 + (lane & 3)) * 4, __float_as_int(v)));
            if ((lane >> 2) == grp) {
                yv = mv;
            }
        };
        // keeps the scheduler from lifting prep (which may wait for x) above
        // the loads issued so far
        __builtin_amdgcn_sched_barrier(0);
        prep();
        if constexpr (NG == 2) {
            load(1, Bc);
        }
        compute(0, A);
        if constexpr (NG == 2) {
            compute(1, Bc);
        }
        return yv;
    }
};

// x (bf16, the lane's chunk c) to registers: xr, xs as the chunk dots expect.
template <int BITS>
__device__ __forceinline__ void x_chunk_regs(const uint16_t* x, uint32_t c, float (&xr)[32], float& xs) {
    uint32_t xw[16];
    load_x_words(x + 32u * c, xw);
    x_words_fence(xw);
    x_words_to_f32(xw, xr, xs);
    if (BITS == 4) {
        q4_scale_x(xr);
    }
}

}  // namespace mh

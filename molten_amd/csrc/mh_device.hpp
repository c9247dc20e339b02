// mh_device.hpp -- device-side building blocks shared by the gfx950 kernels.
//
// Every floating-point step that feeds an integer decision (argmax ids, top-k
// ids) is written as explicit IEEE operations in a fixed order, the "chunk
// order":
//   a K-long dot product is cut into C = K/32 chunks of 32 elements;
//   p_c  = fma chain over the chunk's 32 elements in ascending k from +0;
//   xs_c = ascending sum of the chunk's x from +0;
//   h_c  = fma(s_g, p_c, b_g * xs_c)  (quantized; dense rows use h_c = p_c);
//   virtual lane l (0..63) sums h_l, h_{l+64}, ... in ascending order from +0;
//   the row value is the xor-butterfly (masks 1, 2, 4, 8, 16, 32) of the 64
//   lane sums.
// Files are built with -ffp-contract=off, so a*b+c is a multiply and an add
// unless written as __builtin_fmaf, and f32 denormals are kept.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mh {

constexpr int kWave = 64;

// Global-memory (address space 1) byte pointer.
typedef const __attribute__((address_space(1))) char* gbytes;

// A wave-uniform pointer pinned to scalar registers as a global pointer, so
// that adding a 32-bit per-lane offset selects the scalar-base +
// vector-offset global load form (no per-lane 64-bit address arithmetic).
__device__ __forceinline__ gbytes uniform_ptr(const void* p) {
    const uint64_t u = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
    return reinterpret_cast<gbytes>((static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ gbytes uniform_ptr(gbytes p) {
    const uint64_t u = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
    return reinterpret_cast<gbytes>((static_cast<uint64_t>(hi) << 32) | lo);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Load from a scalar base plus a 32-bit per-lane byte offset.
template <typename T>
__device__ __forceinline__ T gload(gbytes base, uint32_t off) {
    return *reinterpret_cast<const __attribute__((address_space(1))) T*>(base + off);
}

// Makes the wave wait for v: used on a returning atomic's old value, so the
// atomic has been performed at the coherence point before any later
// instruction (a barrier, another workgroup's signal) of this wave.
__device__ __forceinline__ void consume(unsigned long long v) { asm volatile("" ::"v"(v)); }
__device__ __forceinline__ void consume(uint32_t v) { asm volatile("" ::"v"(v)); }

// ------------------------------------------------------------------ bf16 ---

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Low / high bf16 of a packed pair.
__device__ __forceinline__ float bf16lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// Round to nearest even; NaN becomes a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return static_cast<uint16_t>((u >> 16) | 0x0040u);
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// ------------------------------------------------------------------ exp ----
// exp(x) in f32: Cody-Waite reduction x = n*ln2 + r with ln2 split into a
// 16-bit head and a tail, degree-7 Taylor polynomial (coefficients 1/k!
// rounded to f32) in Horner form with fma, and scaling by 2^n as two exact
// power-of-two multiplies so an underflowing result rounds once.  Written out
// so the CPU restatement reproduces it bit for bit.

__device__ __forceinline__ float pow2i(int k) {  // 2^k, k in [-126, 127]
    return __uint_as_float(static_cast<uint32_t>(k + 127) << 23);
}

__device__ __forceinline__ float expf_fixed(float x) {
    if (x != x) {
        return x + x;
    }
    if (x > 0x1.62e430p+6f) {
        return __uint_as_float(0x7f800000u);
    }
    if (x < -0x1.9fe36ap+6f) {
        return 0.0f;
    }
    const float n = __builtin_rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(-n, 0x1.62e400p-1f, x);
    r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0x1.000000p-1f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ni = static_cast<int>(n);
    const int n1 = ni / 2;
    const int n2 = ni - n1;
    return (p * pow2i(n1)) * pow2i(n2);
}

// log(x) in f32 for finite x > 0 (the sampler's Gumbel transform): x =
// m 2^k with m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(s), s = (m - 1) /
// (m + 1), as the odd series 2 s (1 + s^2/3 + s^4/5 + ... + s^10/11) in
// Horner form with fma, plus k ln2 with ln2 split into a 16-bit head and a
// tail.  Written out so the CPU restatement reproduces it bit for bit.
__device__ __forceinline__ float logf_fixed(float x) {
    uint32_t u = __float_as_uint(x);
    int k = static_cast<int>(u >> 23) - 127;
    if ((u >> 23) == 0u) {  // denormal: scale into the normal range
        u = __float_as_uint(x * 0x1p25f);
        k = static_cast<int>(u >> 23) - 127 - 25;
    }
    float m = __uint_as_float((u & 0x007fffffu) | 0x3f800000u);  // [1, 2)
    if (m > 1.41421356f) {
        m = m * 0.5f;
        k += 1;
    }
    const float s = (m - 1.0f) / (m + 1.0f);
    const float s2 = s * s;
    float p = 0x1.745d18p-4f;                  // 1/11
    p = __builtin_fmaf(p, s2, 0x1.c71c72p-4f);  // 1/9
    p = __builtin_fmaf(p, s2, 0x1.24924ap-3f);  // 1/7
    p = __builtin_fmaf(p, s2, 0x1.99999ap-3f);  // 1/5
    p = __builtin_fmaf(p, s2, 0x1.555556p-2f);  // 1/3
    p = __builtin_fmaf(p, s2, 1.0f);
    const float lm = (2.0f * s) * p;
    const float kf = static_cast<float>(k);
    return __builtin_fmaf(kf, 0x1.62e400p-1f, __builtin_fmaf(kf, 0x1.7f7d1cp-20f, lm));
}

// Philox4x32-10 (Salmon et al., SC 2011): ten rounds of the two 32x32->64
// multiplies, the key bumped by the Weyl constants after each round.
__device__ __forceinline__ u32x4 philox4x32_10(u32x4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c.x;
        const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c.z;
        c = u32x4{static_cast<uint32_t>(p1 >> 32) ^ c.y ^ k0, static_cast<uint32_t>(p1),
                  static_cast<uint32_t>(p0 >> 32) ^ c.w ^ k1, static_cast<uint32_t>(p0)};
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c;
}

// Gumbel(0, 1) from a 32-bit uniform word (lfm_sample.metal:141-155): V =
// (x + 0.5) 2^-32, E = -log(1 - V) (its series below V = 1/64), G = -log E.
__device__ __forceinline__ float gumbel_of(uint32_t x) {
    const float v = (static_cast<float>(x) + 0.5f) * 2.3283064365386963e-10f;
    float e;
    if (v < 0.015625f) {
        e = v * (1.0f + v * (0.5f + v * (0.33333334f + v * 0.25f)));
    } else {
        e = -logf_fixed(fmaxf(1.0f - v, 2.9802322387695312e-08f));
    }
    return -logf_fixed(e);
}

// bf16(silu(g)) with silu(g) = g / (1 + exp(-g)), IEEE division.
__device__ __forceinline__ float silu_bf16(float g) {
    return round_bf16(g / (1.0f + expf_fixed(-g)));
}

// ------------------------------------------------------- wave reductions ---

// xor-butterfly sum over the 64 lanes; every lane ends with the same value
// (float addition is commutative, so a_l + a_{l^m} == a_{l^m} + a_l).
__device__ __forceinline__ float wave_butterfly(float v) {
    v = v + __shfl_xor(v, 1);
    v = v + __shfl_xor(v, 2);
    v = v + __shfl_xor(v, 4);
    v = v + __shfl_xor(v, 8);
    v = v + __shfl_xor(v, 16);
    v = v + __shfl_xor(v, 32);
    return v;
}

// The same tree with DPP lane moves (no LDS traffic), result valid in lane 63.
// row_shr:1/2/4/8 pair lane l with l-1, l-2, l-4, l-8 inside each 16-lane
// row; the lanes read below always have bits 0..(level-1) set, so each partner
// is exactly l ^ m and the pairing is the xor butterfly's.  row_bcast:15 adds
// row r-1's total into rows 1 and 3, row_bcast:31 adds rows 0-1 into rows
// 2-3, so lane 63 = ((S0 + S1) + (S2 + S3)) with S_r the row tree sums.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

__device__ __forceinline__ float wave_sum_lane63(float v) {
    v = v + dpp_move<0x111, 0xf>(v);  // row_shr:1
    v = v + dpp_move<0x112, 0xf>(v);  // row_shr:2
    v = v + dpp_move<0x114, 0xf>(v);  // row_shr:4
    v = v + dpp_move<0x118, 0xf>(v);  // row_shr:8
    v = v + dpp_move<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
    v = v + dpp_move<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
    return v;
}

// Four row values h[0..3] per lane reduced with the chunk order's xor
// butterfly, four rows in one register: levels 1 and 2 (xor 1, xor 2) pair
// lanes holding the same row, after which lane l carries row (l & 3); levels
// 3..6 use row_shr:4 (correct where bit 2 of the lane is set), row_ror:8
// (xor 8) and the permlane16/32 swaps (xor 16, xor 32).  Every addition is
// a_l + a_{l^m} of the single-row butterfly (addition is commutative), so
// lane 60 + j ends with row j's butterfly value.
template <int CTRL>
__device__ __forceinline__ float qmove(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float reduce_rows4(const float (&h)[4], int lane) {
    const bool b0 = lane & 1, b1 = (lane >> 1) & 1;
    const float s01 = (b0 ? h[1] : h[0]) + qmove<0xB1>(b0 ? h[0] : h[1]);  // quad_perm 1,0,3,2
    const float s23 = (b0 ? h[3] : h[2]) + qmove<0xB1>(b0 ? h[2] : h[3]);
    float v = (b1 ? s23 : s01) + qmove<0x4E>(b1 ? s01 : s23);              // quad_perm 2,3,0,1
    v = v + dpp_move<0x114, 0xf>(v);  // row_shr:4
    v = v + dpp_move<0x128, 0xf>(v);  // row_ror:8
    {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    return v;
}

// Lane 63's value as a wave-uniform scalar.
__device__ __forceinline__ float lane63(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Wave max / min with the DPP tree of wave_sum_lane63 (valid in lane 63).
__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, dpp_move<0x111, 0xf>(v));
    v = fmaxf(v, dpp_move<0x112, 0xf>(v));
    v = fmaxf(v, dpp_move<0x114, 0xf>(v));
    v = fmaxf(v, dpp_move<0x118, 0xf>(v));
    v = fmaxf(v, dpp_move<0x142, 0xa>(v));
    v = fmaxf(v, dpp_move<0x143, 0xc>(v));
    return lane63(v);
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(-1, static_cast<int>(v), CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, dpp_u32<0x111, 0xf>(v));
    v = min(v, dpp_u32<0x112, 0xf>(v));
    v = min(v, dpp_u32<0x114, 0xf>(v));
    v = min(v, dpp_u32<0x118, 0xf>(v));
    v = min(v, dpp_u32<0x142, 0xa>(v));
    v = min(v, dpp_u32<0x143, 0xc>(v));
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// ------------------------------------------------------------ argmax key ---
// "value desc, index asc" as one orderable u64 (lfm.metal:1119-1124):
// -0 ties +0, NaN candidates are never produced by the merge below.
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t i) {
    uint32_t u = __float_as_uint(v);
    if ((u << 1) == 0u) {
        u = 0u;
    }
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (static_cast<unsigned long long>(o) << 32) | static_cast<unsigned long long>(~i);
}

// The orderable high word of argmax_key for the least f32 h whose bf16
// rounding (nearest even) is >= lb, lb a bf16 value or -inf: for h not NaN,
// round_bf16(h) >= lb exactly when (argmax_key(h, .) >> 32) >= the result.
// For lb > 0 that h is the midpoint below lb (lb's mantissa even: the tie
// rounds up to lb) or the next f32 above it; for lb <= -0 the midpoint below
// |lb| in magnitude, bounded the other way; for +-0, -(0x8000 in bits), the
// last negative value that still rounds to -0.  (Checked exhaustively over
// every bf16 lb and the f32 values around its neighbours.)
__device__ __forceinline__ uint32_t bf16_ge_threshold(float lb) {
    const uint32_t L = __float_as_uint(lb);
    uint32_t t;
    if (L == 0xff800000u) {
        t = L;
    } else if ((L << 1) == 0u) {
        t = 0x80008000u;
    } else if (!(L & 0x80000000u)) {
        t = (L - 0x8000u) + ((L >> 16) & 1u);
    } else {
        const uint32_t m = (L & 0x7fffffffu) + 0x8000u;
        t = 0x80000000u | (m - ((L >> 16) & 1u));
    }
    return static_cast<uint32_t>(argmax_key(__uint_as_float(t), 0u) >> 32);
}

// Wave max of a u32 / u64 (0 is the identity), as a uniform value: the DPP
// tree of wave_max_f32, both halves of a u64 moved together.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xf, 0xf, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xf, 0xf, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xf, 0xf, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xf, 0xf, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xa, 0xf, false)));
    v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xc, 0xf, false)));
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ unsigned long long dpp_max_u64(unsigned long long v) {
    const uint32_t lo = static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v)), CTRL, ROW_MASK, 0xf, false));
    const uint32_t hi = static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v >> 32)), CTRL, ROW_MASK, 0xf, false));
    const unsigned long long o = (static_cast<unsigned long long>(hi) << 32) | lo;
    return o > v ? o : v;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
    v = dpp_max_u64<0x111, 0xf>(v);
    v = dpp_max_u64<0x112, 0xf>(v);
    v = dpp_max_u64<0x114, 0xf>(v);
    v = dpp_max_u64<0x118, 0xf>(v);
    v = dpp_max_u64<0x142, 0xa>(v);
    v = dpp_max_u64<0x143, 0xc>(v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), 63));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), 63));
    return (static_cast<unsigned long long>(hi) << 32) | lo;
}

__device__ __forceinline__ void argmax_merge(float& bv, uint32_t& bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// ----------------------------------------------------------- chunk dots ---
// Byte j of v as f32 (compiles to v_cvt_f32_ubyte{j}).
__device__ __forceinline__ float ubyte_f32(uint32_t v, int j) {
    return static_cast<float>((v >> (8 * j)) & 0xffu);
}

// Opaque copy: hides a value's known bits from the optimizer so that a whole
// word masked once is converted byte by byte with v_cvt_f32_ubyte{0..3},
// instead of being re-extracted per byte.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Q4 chunk: 32 nibble codes in four words, low nibble first (code 8d+n at
// bits 4n of word d).  xr holds the chunk's x with odd positions
// pre-multiplied by 1/16 (q4_scale_x): the high nibble of a byte is converted
// as 16 q (v_cvt_f32_ubyte on the word masked once) and multiplied by x/16.
// Both are exact (a bf16 times 2^-4 is an f32, denormals kept), so every fma
// sees the exact product q*x and the chain equals fma(q_k, x_k, p) in
// ascending k.  (Measured on gfx950: the f16-denormal v_fma_mix_f32 form and
// the fp8-conversion form of the same dot are both exact but not faster:
// v_fma_mix_f32 and v_cvt_pk_f32_fp8 issue at a fraction of v_fmac_f32's rate.)
__device__ __forceinline__ float q4_chunk_dot(const uint32_t (&w)[4], const float* xr) {
    float p = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t lo = opaque(w[d] & 0x0f0f0f0fu);
        const uint32_t hi = opaque(w[d] & 0xf0f0f0f0u);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            p = __builtin_fmaf(ubyte_f32(lo, j), xr[8 * d + 2 * j], p);
            p = __builtin_fmaf(ubyte_f32(hi, j), xr[8 * d + 2 * j + 1], p);
        }
    }
    return p;
}

// Q6 chunk: 32 six-bit codes in six words (code i at bit 6i).  xr is plain x.
__device__ __forceinline__ float q6_chunk_dot(const uint32_t (&w)[6], const float* xr) {
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int bit = 6 * i;
        const int d = bit >> 5;
        const int o = bit & 31;
        uint32_t v;
        if (o + 6 <= 32) {
            v = (w[d] >> o) & 63u;
        } else {
            v = __builtin_amdgcn_alignbit(w[d + 1], w[d], o) & 63u;
        }
        p = __builtin_fmaf(static_cast<float>(v), xr[i], p);
    }
    return p;
}

// The same with x pre-scaled by q6_scale_x (odd positions times 1/4,
// exact).  Of every 3 bytes (4 codes) of the chunk, code 4j sits in bits 0-5
// of the first byte and code 4j + 3 in bits 2-7 of the third: both are
// converted straight from their byte of the word masked once (v_cvt_f32_ubyte:
// q and 4q).  The two codes between them straddle bytes; in the chunk's bit
// stream shifted right by 4 (v_alignbit of two words) code 4j + 1 sits in
// bits 2-7 of byte 3j and code 4j + 2 in bits 0-5 of byte 3j + 1, so they too
// are converted from the shifted word masked once (4q and q).  q x and
// (4q)(x / 4) are the same reals, so the chain equals fma(q_k, x_k, p) in
// ascending k with every code one conversion.
__host__ __device__ constexpr uint32_t q6_byte_mask(int d) {
    uint32_t m = 0;
    for (int k = 0; k < 4; ++k) {
        const int b = 4 * d + k;
        m |= (b % 3 == 0 ? 0x3fu : (b % 3 == 2 ? 0xfcu : 0u)) << (8 * k);
    }
    return m;
}
// Mask of word d of the stream shifted right by 4: bytes 3j (code 4j + 1 as
// 4q) and 3j + 1 (code 4j + 2).
__host__ __device__ constexpr uint32_t q6_shift_mask(int d) {
    uint32_t m = 0;
    for (int k = 0; k < 4; ++k) {
        const int b = 4 * d + k;
        m |= (b % 3 == 0 ? 0xfcu : (b % 3 == 1 ? 0x3fu : 0u)) << (8 * k);
    }
    return m;
}
__device__ __forceinline__ float q6_chunk_dot_s(const uint32_t (&w)[6], const float* xr) {
    uint32_t m[6], ms[6];
#pragma unroll
    for (int d = 0; d < 6; ++d) {
        m[d] = opaque(w[d] & q6_byte_mask(d));
        // word d of the stream >> 4 (the last word's top bits lie past the
        // chunk and are never used)
        const uint32_t sh = d < 5 ? __builtin_amdgcn_alignbit(w[d + 1], w[d], 4) : (w[5] >> 4);
        ms[d] = opaque(sh & q6_shift_mask(d));
    }
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int j = i >> 2, r = i & 3;
        float v;
        if (r == 0) {
            v = ubyte_f32(m[(3 * j) >> 2], (3 * j) & 3);
        } else if (r == 3) {
            v = ubyte_f32(m[(3 * j + 2) >> 2], (3 * j + 2) & 3);
        } else if (r == 1) {
            v = ubyte_f32(ms[(3 * j) >> 2], (3 * j) & 3);
        } else {
            v = ubyte_f32(ms[(3 * j + 1) >> 2], (3 * j + 1) & 3);
        }
        p = __builtin_fmaf(v, xr[i], p);
    }
    return p;
}

// A lane's 32-element bf16 chunk of x: the raw words (16-byte loads when the
// chunk is aligned), then as f32 plus the ascending sum.  Split so a kernel
// can issue its weight loads before it waits for x.
// The alignment is lane 0's: every caller offsets lanes by multiples of 64
// bytes, so the test is uniform and compiles to a scalar branch (a per-lane
// test made both paths masked blocks whose merge waited for the loads).
__device__ __forceinline__ void load_x_words(const uint16_t* xp, uint32_t (&xw)[16]) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(xp)));
    if ((lo & 15u) == 0) {
        const uint4* xv = reinterpret_cast<const uint4*>(xp);
        const uint4 v0 = xv[0], v1 = xv[1], v2 = xv[2], v3 = xv[3];
        const uint4 v[4] = {v0, v1, v2, v3};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            xw[4 * q] = v[q].x; xw[4 * q + 1] = v[q].y; xw[4 * q + 2] = v[q].z; xw[4 * q + 3] = v[q].w;
        }
    } else {
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            xw[q] = static_cast<uint32_t>(xp[2 * q]) | (static_cast<uint32_t>(xp[2 * q + 1]) << 16);
        }
    }
}

// The same for a chunk known to be 16-byte aligned (the host checks x): no
// branch, so no merge of two load paths' registers (whose copies wait for the
// data) between the loads and their first use.
__device__ __forceinline__ void load_x_words_a16(const uint16_t* xp, uint32_t (&xw)[16]) {
    const uint4* xv = reinterpret_cast<const uint4*>(xp);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 v = xv[q];
        xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
    }
}

__device__ __forceinline__ void x_words_to_f32(const uint32_t (&xw)[16], float (&xr)[32], float& xs) {
    xs = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const float lo = bf16lo(xw[q]), hi = bf16hi(xw[q]);
        xs = xs + lo;
        xs = xs + hi;
        xr[2 * q] = lo;
        xr[2 * q + 1] = hi;
    }
}

// Pins x's words after the memory operations issued so far: the compiler can
// neither hoist their conversion above those loads nor sink the loads below it.
__device__ __forceinline__ void x_words_fence(uint32_t (&xw)[16]) {
    asm volatile(""
                 : "+v"(xw[0]), "+v"(xw[1]), "+v"(xw[2]), "+v"(xw[3]), "+v"(xw[4]), "+v"(xw[5]),
                   "+v"(xw[6]), "+v"(xw[7]), "+v"(xw[8]), "+v"(xw[9]), "+v"(xw[10]), "+v"(xw[11]),
                   "+v"(xw[12]), "+v"(xw[13]), "+v"(xw[14]), "+v"(xw[15])
                 :
                 : "memory");
}

// Ties a register to this point: a load feeding it is waited for here, and
// nothing computed from it is moved above (keeps early-issued loads in flight).
__device__ __forceinline__ void reg_fence(uint32_t& v) { asm volatile("" : "+v"(v)); }

__device__ __forceinline__ void load_x_chunk(const uint16_t* xp, float (&xr)[32], float& xs) {
    uint32_t xw[16];
    load_x_words(xp, xw);
    x_words_to_f32(xw, xr, xs);
}

// Scale a raw x chunk for q6_chunk_dot_s: odd positions (codes 4j + 1 and
// 4j + 3, converted as 4q) times 1/4 (exact).
__device__ __forceinline__ void q6_scale_x(float (&xr)[32]) {
#pragma unroll
    for (int i = 1; i < 32; i += 2) {
        xr[i] = xr[i] * 0.25f;
    }
}

// Scale a raw x chunk for q4_chunk_dot: odd positions times 1/16 (exact).
__device__ __forceinline__ void q4_scale_x(float (&xr)[32]) {
#pragma unroll
    for (int i = 1; i < 32; i += 2) {
        xr[i] = xr[i] * 0.0625f;
    }
}

// ---------------------------------------------------------- chunk loads ---
template <int BITS>
struct Chunk;

template <>
struct Chunk<4> {
    uint32_t w[4];
    __device__ __forceinline__ void load(const uint32_t* p) {  // 16-byte aligned
        const uint4 v = *reinterpret_cast<const uint4*>(p);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
    __device__ __forceinline__ void load(gbytes base, uint32_t off) {  // 16-byte aligned
        const u32x4 v = gload<u32x4>(base, off);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
    __device__ __forceinline__ void zero() { w[0] = w[1] = w[2] = w[3] = 0u; }
    __device__ __forceinline__ void load_nt(gbytes base, uint32_t off) {  // streamed once
        const u32x4 v = __builtin_nontemporal_load(
            reinterpret_cast<const __attribute__((address_space(1))) u32x4*>(base + off));
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
    __device__ __forceinline__ float dot(const float* xr) const { return q4_chunk_dot(w, xr); }
    __device__ __forceinline__ void fence() {
        reg_fence(w[0]); reg_fence(w[1]); reg_fence(w[2]); reg_fence(w[3]);
    }
};

template <>
struct Chunk<6> {
    uint32_t w[6];
    __device__ __forceinline__ void load(const uint32_t* p) {  // 8-byte aligned
        const uint2* q = reinterpret_cast<const uint2*>(p);
        const uint2 a = q[0], b = q[1], c = q[2];
        w[0] = a.x; w[1] = a.y; w[2] = b.x; w[3] = b.y; w[4] = c.x; w[5] = c.y;
    }
    __device__ __forceinline__ void load(gbytes base, uint32_t off) {  // 8-byte aligned
        const u32x2 a = gload<u32x2>(base, off), b = gload<u32x2>(base, off + 8),
                    c = gload<u32x2>(base, off + 16);
        w[0] = a.x; w[1] = a.y; w[2] = b.x; w[3] = b.y; w[4] = c.x; w[5] = c.y;
    }
    __device__ __forceinline__ void zero() { w[0] = w[1] = w[2] = w[3] = w[4] = w[5] = 0u; }
    __device__ __forceinline__ void load_nt(gbytes base, uint32_t off) {  // streamed once
        typedef const __attribute__((address_space(1))) u32x2* p2;
        const u32x2 a = __builtin_nontemporal_load(reinterpret_cast<p2>(base + off));
        const u32x2 b = __builtin_nontemporal_load(reinterpret_cast<p2>(base + off + 8));
        const u32x2 c = __builtin_nontemporal_load(reinterpret_cast<p2>(base + off + 16));
        w[0] = a.x; w[1] = a.y; w[2] = b.x; w[3] = b.y; w[4] = c.x; w[5] = c.y;
    }
    __device__ __forceinline__ float dot(const float* xr) const { return q6_chunk_dot(w, xr); }
    __device__ __forceinline__ float dot_s(const float* xr) const { return q6_chunk_dot_s(w, xr); }
};

template <>
struct Chunk<8> {  // 32 byte codes in eight words (dequantization only)
    uint32_t w[8];
    __device__ __forceinline__ void load(const uint32_t* p) {  // 16-byte aligned
        const uint4* q = reinterpret_cast<const uint4*>(p);
        const uint4 a = q[0], b = q[1];
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    }
};

// A chunk's 32 codes dequantized to bf16 as bf16(fma(s, q, b)) (MLX
// dequantize, quant_nax.metal:2908-2993), packed two per word in code order.
template <int BITS>
__device__ __forceinline__ void dequant_chunk(const uint32_t* w, float s, float b, uint32_t (&packed)[16]) {
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
        uint32_t q0, q1;
        if constexpr (BITS == 4) {
            q0 = (w[i >> 3] >> (4 * (i & 7))) & 15u;
            q1 = (w[(i + 1) >> 3] >> (4 * ((i + 1) & 7))) & 15u;
        } else if constexpr (BITS == 8) {
            q0 = (w[i >> 2] >> (8 * (i & 3))) & 255u;
            q1 = (w[(i + 1) >> 2] >> (8 * ((i + 1) & 3))) & 255u;
        } else {
            const int b0 = 6 * i, b1 = 6 * (i + 1);
            q0 = ((b0 & 31) + 6 <= 32) ? (w[b0 >> 5] >> (b0 & 31)) & 63u
                                       : __builtin_amdgcn_alignbit(w[(b0 >> 5) + 1], w[b0 >> 5], b0 & 31) & 63u;
            q1 = ((b1 & 31) + 6 <= 32) ? (w[b1 >> 5] >> (b1 & 31)) & 63u
                                       : __builtin_amdgcn_alignbit(w[(b1 >> 5) + 1], w[b1 >> 5], b1 & 31) & 63u;
        }
        const uint16_t lo = f32_to_bf16(__builtin_fmaf(s, static_cast<float>(q0), b));
        const uint16_t hi = f32_to_bf16(__builtin_fmaf(s, static_cast<float>(q1), b));
        packed[i >> 1] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
    }
}

// One lane's 32-element chunk of a router row (bf16 or f32 weights), held
// as raw words until converted.
template <typename WT>
struct RowWords;
template <>
struct RowWords<uint16_t> {  // 32 bf16 = 16 words
    uint4 v[4];
    __device__ __forceinline__ void load(const uint16_t* p) {
        const uint4* q = reinterpret_cast<const uint4*>(p);
        v[0] = q[0]; v[1] = q[1]; v[2] = q[2]; v[3] = q[3];
    }
    __device__ __forceinline__ void to_f32(float (&w)[32]) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t u[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                w[8 * i + 2 * j] = mh::bf16lo(u[j]);
                w[8 * i + 2 * j + 1] = mh::bf16hi(u[j]);
            }
        }
    }
};
template <>
struct RowWords<float> {  // 32 f32
    float4 v[8];
    __device__ __forceinline__ void load(const float* p) {
        const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = q[i];
    }
    __device__ __forceinline__ void to_f32(float (&w)[32]) const {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            w[4 * i] = v[i].x; w[4 * i + 1] = v[i].y; w[4 * i + 2] = v[i].z; w[4 * i + 3] = v[i].w;
        }
    }
};

}  // namespace mh

// embed.hip -- the Q6 embedding table on the decode path: the dequantizing
// row gather (lfm.metal:430-462 lfm_gather_rows_q6_bf16; src/kernels/lfm.rs
// :337-363 gather_rows_q6) and the token tail that turns the head's argmax
// key into the token and the next step's input row plus its RMSNorm
// (lfm.metal:1284-1386 lfm_token_tail; src/kernels/lfm.rs:850-888 token_tail
// with `next`).  Dequantized values are bf16(fma(s, q, b)), bit-equal to
// mh_dequant_to_bf16's.
#include "mh_device.hpp"
#include "mh_host.hpp"

namespace {

// Row ids[t] of the table into out[t, :].  Workgroup (x, t): one wave, lane
// l dequantizes chunk 64 x + l (32 codes) of token t's row.  A wave whose 64
// chunks are all in the row passes its 4 KB through the LDS, so that each
// store instruction writes 1 KB contiguous instead of 16 bytes per lane at a
// 64-byte stride.
__global__ __launch_bounds__(64) void k_gather_rows_q6(const uint32_t* codes, const uint16_t* scales,
                                                       const uint16_t* biases, const uint32_t* ids, uint16_t* out,
                                                       uint32_t k, uint32_t n_rows) {
    __shared__ uint4 tr[4 * 64];  // the wave's 16-byte pieces in row order
    const uint32_t c = blockIdx.x * 64u + threadIdx.x;
    const uint32_t t = blockIdx.y;
    const uint32_t C = k / 32u;
    const bool full = blockIdx.x * 64u + 64u <= C;  // uniform
    if (c >= C) {
        return;
    }
    const uint32_t row = ids[t];
    if (row >= n_rows) {  // out-of-range id: the row is left unwritten
        return;
    }
    const uint32_t groups = k / 64u;
    mh::Chunk<6> ch;
    ch.load(codes + static_cast<size_t>(row) * (k * 6u / 32u) + static_cast<size_t>(c) * 6u);
    const float s = mh::bf16_to_f32(scales[static_cast<size_t>(row) * groups + c / 2u]);
    const float b = mh::bf16_to_f32(biases[static_cast<size_t>(row) * groups + c / 2u]);
    uint32_t packed[16];
    mh::dequant_chunk<6>(ch.w, s, b, packed);
    if (full) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            tr[4u * threadIdx.x + q] = make_uint4(packed[4 * q], packed[4 * q + 1], packed[4 * q + 2], packed[4 * q + 3]);
        }
        __builtin_amdgcn_wave_barrier();
        uint4* row = reinterpret_cast<uint4*>(out + static_cast<size_t>(t) * k + 2048u * blockIdx.x);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            row[64u * j + threadIdx.x] = tr[64u * j + threadIdx.x];
        }
        return;
    }
    uint4* dst = reinterpret_cast<uint4*>(out + static_cast<size_t>(t) * k + 32u * c);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        dst[q] = make_uint4(packed[4 * q], packed[4 * q + 1], packed[4 * q + 2], packed[4 * q + 3]);
    }
}

// One wave: the key -> token (key cleared), then the token's embedding row
// (lane c: chunk c, K <= 2048) into x and bf16((v * inv_rms) * w) into
// normed, inv_rms = 1 / sqrt(sum v^2 / K + eps) over the bf16 row values.
__global__ __launch_bounds__(64) void k_token_tail_embed(unsigned long long* best, uint32_t* out_tok,
                                                         const uint32_t* codes, const uint16_t* scales,
                                                         const uint16_t* biases, const uint16_t* w, uint16_t* x,
                                                         uint16_t* normed, uint32_t k, uint32_t n_rows, float eps) {
    const uint32_t lane = threadIdx.x;
    const unsigned long long key = best[0];
    const uint32_t tok = ~static_cast<uint32_t>(key & 0xffffffffull);
    if (lane == 0) {
        best[0] = 0ull;
        out_tok[0] = tok;
    }
    if (tok >= n_rows) {  // no token (an empty key) or out of the table: no row
        return;
    }
    const uint32_t C = k / 32u;
    const bool live = lane < C;
    const uint32_t c = live ? lane : 0u;
    mh::Chunk<6> ch;
    ch.load(codes + static_cast<size_t>(tok) * (k * 6u / 32u) + static_cast<size_t>(c) * 6u);
    const float s = mh::bf16_to_f32(scales[static_cast<size_t>(tok) * (k / 64u) + c / 2u]);
    const float b = mh::bf16_to_f32(biases[static_cast<size_t>(tok) * (k / 64u) + c / 2u]);
    uint32_t packed[16];
    mh::dequant_chunk<6>(ch.w, s, b, packed);
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float lo = mh::bf16lo(packed[i]), hi = mh::bf16hi(packed[i]);
        ss = __builtin_fmaf(lo, lo, ss);
        ss = __builtin_fmaf(hi, hi, ss);
    }
    const float total = mh::lane63(mh::wave_sum_lane63(live ? ss : 0.0f));
    const float inv = 1.0f / __builtin_sqrtf(total / static_cast<float>(k) + eps);
    if (!live) {
        return;
    }
    uint4* xo = reinterpret_cast<uint4*>(x + 32u * c);
    const uint4* wv = reinterpret_cast<const uint4*>(w + 32u * c);
    uint4* no = reinterpret_cast<uint4*>(normed + 32u * c);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        xo[q] = make_uint4(packed[4 * q], packed[4 * q + 1], packed[4 * q + 2], packed[4 * q + 3]);
        const uint4 g4 = wv[q];
        const uint32_t gw[4] = {g4.x, g4.y, g4.z, g4.w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t v = packed[4 * q + e];
            const uint16_t lo = mh::f32_to_bf16((mh::bf16lo(v) * inv) * mh::bf16lo(gw[e]));
            const uint16_t hi = mh::f32_to_bf16((mh::bf16hi(v) * inv) * mh::bf16hi(gw[e]));
            o[e] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
        }
        no[q] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

int check_table(const mh_quant_weights* e, const char* op) {
    MH_TRY(mh::check_quant(e, op));
    MH_ENSURE(e->bits == 6 && e->group_size == 64, MH_ERR_UNSUPPORTED, "%s: the embedding table is 6-bit/64", op);
    MH_ENSURE(e->in_features % 64u == 0, MH_ERR_UNSUPPORTED, "%s: width %u not a multiple of 64", op,
              e->in_features);
    return MH_OK;
}

}  // namespace

extern "C" {

int mh_gather_rows_q6(const mh_quant_weights* w, const uint32_t* ids, uint32_t m, uint16_t* out,
                      mh_stream_t stream) {
    const char* op = "mh_gather_rows_q6";
    MH_TRY(check_table(w, op));
    MH_ENSURE(ids && out, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(m >= 1 && m <= 65535u, MH_ERR_INVALID, "%s: %u rows (1..65535)", op, m);
    MH_ENSURE(mh::aligned(ids, 4) && mh::aligned(out, 16), MH_ERR_ALIGN, "%s: ids 4-byte, out 16-byte alignment",
              op);
    const uint32_t C = w->in_features / 32u;
    hipLaunchKernelGGL(k_gather_rows_q6, dim3((C + 63u) / 64u, m), dim3(64), 0, mh::as_stream(stream), w->codes,
                       w->scales, w->biases, ids, out, w->in_features, w->out_features);
    return mh::launch_status("k_gather_rows_q6");
}

int mh_token_tail_embed(uint64_t* best, uint32_t* out_tok, const mh_quant_weights* e, const uint16_t* w,
                        uint16_t* x, uint16_t* normed, float eps, mh_stream_t stream) {
    const char* op = "mh_token_tail_embed";
    MH_TRY(check_table(e, op));
    MH_ENSURE(best && out_tok && w && x && normed, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(e->in_features <= 2048u, MH_ERR_UNSUPPORTED, "%s: width %u > 2048 (one row per wave)", op,
              e->in_features);
    MH_ENSURE(mh::aligned(best, 8) && mh::aligned(out_tok, 4), MH_ERR_ALIGN, "%s: key / token alignment", op);
    MH_ENSURE(mh::aligned(w, 16) && mh::aligned(x, 16) && mh::aligned(normed, 16), MH_ERR_ALIGN,
              "%s: rows must be 16-byte aligned", op);
    hipLaunchKernelGGL(k_token_tail_embed, dim3(1), dim3(64), 0, mh::as_stream(stream),
                       reinterpret_cast<unsigned long long*>(best), out_tok, e->codes, e->scales, e->biases, w, x,
                       normed, e->in_features, e->out_features, eps);
    return mh::launch_status("k_token_tail_embed");
}

}  // extern "C"

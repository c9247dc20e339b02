// gemv_epi.hip -- decode GEMV epilogue variants on the batch-1 row-block walk
// (mh_rows.hpp): the Q/K/V projection with the V rows written into the KV
// cache (lfm.metal:1023-1067 lfm_proj3_gemv_scatter_bf16; src/kernels/lfm.rs
// :155-218 proj3_gemv_scatter) and the short-conv input projection fused with
// the conv (lfm.metal:1074-1109 lfm_conv3_gemv_split_bf16; src/kernels/lfm.rs
// :220-256 conv3_gemv).  The row values are the chunk-order sums of
// mh_gemv_quant, so the outputs equal the oracle's bit for bit.
#include "mh_host.hpp"
#include "mh_rows.hpp"

namespace {

// 4-row blocks: these projections are latency-bound (a few MB), so twice the
// waves with half the serial arithmetic each finish sooner than 8-row blocks
constexpr int kNG = 1;
constexpr int BR = kNG * mh::kGroupRows;

// ------------------------------------------------------------- proj3 ---

struct Proj3Args {
    mh::RowMatrix m[3];  // q, k, v
    uint32_t rows[3];    // NQ, NK, NV
    uint32_t blocks[3];  // row blocks of each
    const uint16_t* x;
    uint16_t* q_out;
    uint16_t* k_out;
    uint16_t* v_cache;  // [NV / 64, max_seq, 64]
    uint32_t max_seq, pos;
    uint32_t k, gs, groups, row_words;
};

// One row block per workgroup of one wave (a few hundred blocks at decode
// shapes: spread over every CU): blocks of q first, then k, then v (each
// matrix's blocks start at its row 0; a partial last block has fewer rows).
template <bool FAST>
__global__ __launch_bounds__(64) void k_proj3(Proj3Args a) {
    __shared__ uint32_t sbl[BR * mh::kMaxGroups];
    const int lane = threadIdx.x;
    uint32_t blk = blockIdx.x;
    int seg = 0;
    if (blk >= a.blocks[0]) {
        blk -= a.blocks[0];
        seg = 1;
        if (blk >= a.blocks[1]) {
            blk -= a.blocks[1];
            seg = 2;
            if (blk >= a.blocks[2]) {
                return;
            }
        }
    }
    mh::RowWalk<4, FAST> walk;
    walk.init(a.k, a.gs, a.groups, a.row_words, sbl, lane);
    float xr[32], xs;
    mh::x_chunk_regs<4>(a.x, walk.chunk(), xr, xs);
    // (selects, not an indexed argument array: that would go through scratch)
    const mh::RowMatrix m = seg == 0 ? a.m[0] : (seg == 1 ? a.m[1] : a.m[2]);
    const uint32_t rows = seg == 0 ? a.rows[0] : (seg == 1 ? a.rows[1] : a.rows[2]);
    const uint32_t row0 = blk * BR;
    const uint32_t nrows = FAST ? static_cast<uint32_t>(BR) : min(static_cast<uint32_t>(BR), rows - row0);
    const float yv = walk.template block<kNG>(m, row0, nrows, xr, xs, [] {});
    if (lane < static_cast<int>(nrows)) {
        const uint32_t j = row0 + lane;
        const uint16_t yb = mh::f32_to_bf16(yv);
        if (seg == 0) {
            a.q_out[j] = yb;
        } else if (seg == 1) {
            a.k_out[j] = yb;
        } else {
            a.v_cache[(static_cast<size_t>(j / 64u) * a.max_seq + a.pos) * 64u + j % 64u] = yb;
        }
    }
}

// ------------------------------------------------------------- conv3 ---

struct Conv3Args {
    mh::RowMatrix m;        // [3H, K]: B rows, C rows, X rows
    const uint16_t* x;
    const uint16_t* taps;   // [H, 3]
    const uint16_t* state;  // [2, H]
    uint16_t* out;          // [H]
    uint16_t* new_state;    // [2, H]
    uint32_t h;
    uint32_t k, gs, groups, row_words;
};

// One block of 8 channels per workgroup of three waves: wave w computes the
// channels' row block w (B, C, X: rows c0.., H + c0.., 2H + c0..), the values
// meet in LDS, and lanes j < 8 of wave 0 run channel c0 + j's conv.
template <bool FAST>
__global__ __launch_bounds__(192) void k_conv3(Conv3Args a) {
    __shared__ uint32_t sbl[3][BR * mh::kMaxGroups];
    __shared__ float vals[3][BR];
    const int lane = threadIdx.x & (mh::kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / mh::kWave);
    const uint32_t c0 = blockIdx.x * BR;
    const uint32_t H = a.h;
    mh::RowWalk<4, FAST> walk;
    walk.init(a.k, a.gs, a.groups, a.row_words, sbl[wave], lane);
    float xr[32], xs;
    mh::x_chunk_regs<4>(a.x, walk.chunk(), xr, xs);
    const uint32_t nrows = FAST ? static_cast<uint32_t>(BR) : min(static_cast<uint32_t>(BR), H - c0);
    const float y = walk.template block<kNG>(a.m, static_cast<uint32_t>(wave) * H + c0, nrows, xr, xs, [] {});
    if (lane < BR) {
        vals[wave][lane] = y;
    }
    __syncthreads();
    if (wave == 0 && lane < static_cast<int>(nrows)) {
        const uint32_t c = c0 + lane;
        const float b = mh::round_bf16(vals[0][lane]);
        const float cv = mh::round_bf16(vals[1][lane]);
        const float xv = mh::round_bf16(vals[2][lane]);
        const uint16_t s1 = a.state[H + c];
        const float v0 = mh::bf16_to_f32(a.state[c]);
        const float v1 = mh::bf16_to_f32(s1);
        const float v2 = mh::round_bf16(b * xv);
        const float z = mh::bf16_to_f32(a.taps[3u * c]) * v0 + mh::bf16_to_f32(a.taps[3u * c + 1u]) * v1 +
                        mh::bf16_to_f32(a.taps[3u * c + 2u]) * v2;
        a.out[c] = mh::f32_to_bf16(cv * mh::round_bf16(z));
        a.new_state[H + c] = mh::f32_to_bf16(v2);
        a.new_state[c] = s1;
    }
}

// The walk's shape limits (the batch-1 GEMV's): K <= 2048, an even number of
// groups per row, scales / biases readable as 32-bit words.
int check_walk(const mh_quant_weights* w, const char* op) {
    MH_TRY(mh::check_quant(w, op));
    MH_ENSURE(w->bits == 4 && w->group_size == 64, MH_ERR_UNSUPPORTED, "%s: %u-bit group %u (4-bit/64 only)", op,
              w->bits, w->group_size);
    MH_ENSURE(w->in_features <= 2048u && w->in_features % 128u == 0, MH_ERR_UNSUPPORTED,
              "%s: in_features %u (a multiple of 128, at most 2048)", op, w->in_features);
    MH_ENSURE(mh::aligned(w->scales, 4) && mh::aligned(w->biases, 4), MH_ERR_ALIGN,
              "%s: scales/biases not 4-byte aligned", op);
    return MH_OK;
}

uint32_t blocks_of(uint32_t rows) { return (rows + BR - 1) / BR; }

}  // namespace

extern "C" {

int mh_proj3_gemv_scatter(const mh_quant_weights* q, const mh_quant_weights* k, const mh_quant_weights* v,
                          const uint16_t* x, uint16_t* q_out, uint16_t* k_out, uint16_t* v_cache,
                          uint32_t max_seq, uint32_t pos, mh_stream_t stream) {
    const char* op = "mh_proj3_gemv_scatter";
    MH_TRY(check_walk(q, op));
    MH_TRY(check_walk(k, op));
    MH_TRY(check_walk(v, op));
    MH_ENSURE(x && q_out && k_out && v_cache, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(q->in_features == k->in_features && q->in_features == v->in_features, MH_ERR_INVALID,
              "%s: input widths differ (%u, %u, %u)", op, q->in_features, k->in_features, v->in_features);
    MH_ENSURE(v->out_features % 64u == 0, MH_ERR_INVALID, "%s: NV %u not a multiple of 64", op, v->out_features);
    MH_ENSURE(pos < max_seq, MH_ERR_INVALID, "%s: pos %u >= max_seq %u", op, pos, max_seq);
    MH_ENSURE(mh::aligned(x, 2) && mh::aligned(q_out, 2) && mh::aligned(k_out, 2) && mh::aligned(v_cache, 2),
              MH_ERR_ALIGN, "%s: x / outputs alignment", op);
    Proj3Args a{};
    const mh_quant_weights* w[3] = {q, k, v};
    uint32_t total = 0;
    bool fast = q->in_features == 2048u;
    for (int i = 0; i < 3; ++i) {
        a.m[i] = mh::RowMatrix{reinterpret_cast<const char*>(w[i]->codes), w[i]->scales, w[i]->biases};
        a.rows[i] = w[i]->out_features;
        a.blocks[i] = blocks_of(w[i]->out_features);
        total += a.blocks[i];
        fast = fast && w[i]->out_features % BR == 0;
    }
    a.x = x;
    a.q_out = q_out;
    a.k_out = k_out;
    a.v_cache = v_cache;
    a.max_seq = max_seq;
    a.pos = pos;
    a.k = q->in_features;
    a.gs = q->group_size;
    a.groups = q->in_features / q->group_size;
    a.row_words = q->in_features / 8u;
    if (fast) {
        hipLaunchKernelGGL(k_proj3<true>, dim3(total), dim3(64), 0, mh::as_stream(stream), a);
    } else {
        hipLaunchKernelGGL(k_proj3<false>, dim3(total), dim3(64), 0, mh::as_stream(stream), a);
    }
    return mh::launch_status("k_proj3");
}

int mh_conv3_gemv(const mh_quant_weights* wproj, const uint16_t* x, const uint16_t* taps, const uint16_t* state,
                  uint16_t* out, uint16_t* new_state, mh_stream_t stream) {
    const char* op = "mh_conv3_gemv";
    MH_TRY(check_walk(wproj, op));
    MH_ENSURE(x && taps && state && out && new_state, MH_ERR_INVALID, "%s: NULL argument", op);
    MH_ENSURE(wproj->out_features % 3u == 0, MH_ERR_INVALID, "%s: %u rows are not 3 H", op, wproj->out_features);
    MH_ENSURE(mh::aligned(x, 2) && mh::aligned(taps, 2) && mh::aligned(state, 2) && mh::aligned(out, 2) &&
                  mh::aligned(new_state, 2),
              MH_ERR_ALIGN, "%s: alignment", op);
    Conv3Args a{};
    a.m = mh::RowMatrix{reinterpret_cast<const char*>(wproj->codes), wproj->scales, wproj->biases};
    a.x = x;
    a.taps = taps;
    a.state = state;
    a.out = out;
    a.new_state = new_state;
    a.h = wproj->out_features / 3u;
    a.k = wproj->in_features;
    a.gs = wproj->group_size;
    a.groups = wproj->in_features / wproj->group_size;
    a.row_words = wproj->in_features / 8u;
    const dim3 grid(blocks_of(a.h));
    if (a.k == 2048u && a.h % BR == 0) {
        hipLaunchKernelGGL(k_conv3<true>, grid, dim3(192), 0, mh::as_stream(stream), a);
    } else {
        hipLaunchKernelGGL(k_conv3<false>, grid, dim3(192), 0, mh::as_stream(stream), a);
    }
    return mh::launch_status("k_conv3");
}

}  // extern "C"

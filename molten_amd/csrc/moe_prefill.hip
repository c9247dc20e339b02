// moe_prefill.hip -- the integer half of the prefill MoE (counting sort and
// block maps) plus the row gather, SwiGLU and the weighted combine.
//
// Replaces lfm.metal:1604-1770 (moe_zero_counts, moe_count, moe_offsets,
// moe_sorted_parallel, moe_zero_blocks, moe_block_offsets, moe_blocks),
// lfm.metal:859-940 (combine) and elementwise.metal:7-52 (SwiGLU, gather).
// Every integer output is a deterministic function of the ids: the sort is
// stable in slot order (token-major, rank-major), like the reference's.
#include "mh_device.hpp"
#include "mh_host.hpp"
#include "mh_route.hpp"

namespace {

__global__ void k_fill_u32(uint32_t* p, size_t n, uint32_t v) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        p[i] = v;
    }
}

// Histogram: per-workgroup LDS counts, one atomic per (workgroup, expert).
__global__ __launch_bounds__(256) void k_count(const uint32_t* ids, uint32_t* counts, uint32_t s,
                                               uint32_t e) {
    __shared__ uint32_t h[256];
    for (uint32_t i = threadIdx.x; i < e; i += 256) h[i] = 0;
    __syncthreads();
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < s; i += gridDim.x * 256) {
        const uint32_t x = ids[i];
        if (x < e) atomicAdd(&h[x], 1u);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < e; i += 256) {
        if (h[i]) atomicAdd(&counts[i], h[i]);
    }
}

// Exclusive scan of counts (e <= 1024) by one workgroup.
__global__ __launch_bounds__(1024) void k_offsets(const uint32_t* counts, uint32_t* offsets,
                                                  uint32_t e) {
    __shared__ uint32_t sh[1024];
    const uint32_t t = threadIdx.x;
    sh[t] = t < e ? counts[t] : 0u;
    __syncthreads();
    for (uint32_t d = 1; d < 1024; d <<= 1) {
        const uint32_t v = t >= d ? sh[t - d] : 0u;
        __syncthreads();
        sh[t] += v;
        __syncthreads();
    }
    if (t < e) offsets[t] = sh[t] - counts[t];
}

// Exclusive prefix sum over the workgroup (1024 threads, thread order) of
// one value per thread; returns this thread's exclusive prefix, *total the
// workgroup total.  Uses LDS wave totals; ends with a barrier.
__device__ __forceinline__ uint32_t block_excl_scan_1024(uint32_t v, uint32_t* total) {
    __shared__ uint32_t wtot[16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_up(inc, d);
        if (lane >= d) inc += o;
    }
    if (lane == 63) wtot[wave] = inc;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
        const uint32_t t = wtot[w];
        before += w < wave ? t : 0u;
        all += t;
    }
    __syncthreads();
    *total = all;
    return before + inc - v;
}

// Stable scatter of expert e's slots by one 1024-thread workgroup: four
// consecutive slots per thread per pass (slot order = thread order, then the
// thread's four), positions from a workgroup prefix count.
__device__ __forceinline__ void scatter_expert(const uint32_t* ids, uint32_t e, uint32_t base,
                                               uint32_t* ids_sorted, uint32_t* slotpos, uint32_t s,
                                               uint32_t topk) {
    for (uint32_t t0 = 0; t0 < s; t0 += 4096u) {
        const uint32_t i0 = t0 + 4u * threadIdx.x;
        uint32_t id[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) id[j] = i0 + j < s ? ids[i0 + j] : 0xffffffffu;
        uint32_t hit[4], cnt = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            hit[j] = id[j] == e ? 1u : 0u;
            cnt += hit[j];
        }
        uint32_t total;
        uint32_t pos = base + block_excl_scan_1024(cnt, &total);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (hit[j]) {
                ids_sorted[pos] = (i0 + j) / topk;
                slotpos[i0 + j] = pos;
                ++pos;
            }
        }
        base += total;
    }
}

__global__ __launch_bounds__(1024) void k_sorted(const uint32_t* ids, const uint32_t* offsets,
                                                 uint32_t* ids_sorted, uint32_t* slotpos,
                                                 uint32_t s, uint32_t topk) {
    scatter_expert(ids, blockIdx.x, offsets[blockIdx.x], ids_sorted, slotpos, s, topk);
}

__global__ __launch_bounds__(1024) void k_block_offsets(const uint32_t* counts, uint32_t* gu_off,
                                                        uint32_t* dn_off, uint32_t e, uint32_t bm,
                                                        uint32_t gu_tiles, uint32_t dn_tiles) {
    const uint32_t i = threadIdx.x;
    const uint32_t rows = i < e ? (counts[i] + bm - 1) / bm : 0u;
    uint32_t total;
    const uint32_t before = block_excl_scan_1024(rows, &total);
    if (i < e) {
        gu_off[i] = before * gu_tiles;
        dn_off[i] = before * dn_tiles;
    }
}

__device__ inline void write_map(uint4* map, uint32_t max_entries, uint32_t base, uint32_t n,
                                 uint32_t off, uint32_t ex, uint32_t bm, uint32_t bn,
                                 uint32_t n_cols) {
    const uint32_t rows = (n + bm - 1) / bm;
    const uint32_t tiles = n_cols / bn;
    for (uint32_t i = threadIdx.x; i < rows * tiles; i += blockDim.x) {
        if (base + i >= max_entries) break;
        const uint32_t mt = i / tiles, nt = i % tiles;
        const uint32_t m0 = off + mt * bm;
        const uint32_t m_end = min(m0 + bm, off + n);
        const uint32_t n0 = nt * bn;
        map[base + i] = make_uint4(m0, ex * n_cols + n0, n0, m_end);
    }
}

__global__ __launch_bounds__(128) void k_blocks(const uint32_t* counts, const uint32_t* offsets,
                                                const uint32_t* gu_off, const uint32_t* dn_off,
                                                uint4* gu, uint32_t max_gu, uint4* dn,
                                                uint32_t max_dn, uint32_t bm, uint32_t gu_bn,
                                                uint32_t dn_bn, uint32_t gu_n, uint32_t dn_n) {
    const uint32_t ex = blockIdx.x;
    const uint32_t n = counts[ex];
    if (n == 0) return;
    write_map(gu, max_gu, gu_off[ex], n, offsets[ex], ex, bm, gu_bn, gu_n);
    write_map(dn, max_dn, dn_off[ex], n, offsets[ex], ex, bm, dn_bn, dn_n);
}

// out[i, :] = table[ids[i], :]; 16-byte vectors when h % 8 == 0.
__global__ __launch_bounds__(256) void k_gather_rows(const uint16_t* table, const uint32_t* ids,
                                                     uint16_t* out, uint32_t m, uint32_t h,
                                                     uint32_t n_table) {
    const uint32_t h8 = h / 8;
    const size_t total = static_cast<size_t>(m) * h8;
    for (size_t t = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const uint32_t i = static_cast<uint32_t>(t / h8), c = static_cast<uint32_t>(t % h8);
        const uint32_t r = min(ids[i], n_table - 1);
        reinterpret_cast<uint4*>(out + static_cast<size_t>(i) * h)[c] =
            reinterpret_cast<const uint4*>(table + static_cast<size_t>(r) * h)[c];
    }
}

__global__ __launch_bounds__(256) void k_silu_mul(const uint16_t* gate, const uint16_t* up,
                                                  uint16_t* out, size_t n) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const float g = mh::bf16_to_f32(gate[i]);
        out[i] = mh::f32_to_bf16(mh::silu_bf16(g) * mh::bf16_to_f32(up[i]));
    }
}

// out[t, c] = bf16( sum_r f32(bf16(w[t,r] * sorted[slotpos[t,r], c])) ), r
// ascending from +0; eight columns per thread.
// TK = topk: a token's slot positions and weights are read together, then
// its TK rows' pieces together (two round trips, not 2 TK), and summed in
// slot order.
template <int TK>
__global__ __launch_bounds__(256) void k_combine(const uint16_t* sorted, const uint32_t* slotpos,
                                                 const uint16_t* w, uint16_t* out, uint32_t m,
                                                 uint32_t h, uint32_t n_sorted) {
    const uint32_t h8 = h / 8;
    const size_t total = static_cast<size_t>(m) * h8;
    for (size_t t = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const uint32_t tok = static_cast<uint32_t>(t / h8), c = static_cast<uint32_t>(t % h8);
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
        uint32_t p[TK];
        float wr[TK];
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            p[r] = min(slotpos[static_cast<size_t>(tok) * TK + r], n_sorted - 1);
            wr[r] = mh::bf16_to_f32(w[static_cast<size_t>(tok) * TK + r]);
        }
        uint4 v[TK];
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            v[r] = reinterpret_cast<const uint4*>(sorted + static_cast<size_t>(p[r]) * h)[c];
        }
#pragma unroll
        for (int r = 0; r < TK; ++r) {
            const uint32_t u[4] = {v[r].x, v[r].y, v[r].z, v[r].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[2 * j] = acc[2 * j] + mh::round_bf16(wr[r] * mh::bf16lo(u[j]));
                acc[2 * j + 1] = acc[2 * j + 1] + mh::round_bf16(wr[r] * mh::bf16hi(u[j]));
            }
        }
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            o[j] = static_cast<uint32_t>(mh::f32_to_bf16(acc[2 * j])) |
                   (static_cast<uint32_t>(mh::f32_to_bf16(acc[2 * j + 1])) << 16);
        }
        reinterpret_cast<uint4*>(out + static_cast<size_t>(tok) * h)[c] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// Prefill step, routing half 1: counts (LDS histogram of the slots),
// offsets and both block-map offsets in one 1024-thread workgroup (e <= 1024).
__global__ __launch_bounds__(1024) void k_count_scan(const uint32_t* ids, uint32_t s, uint32_t e,
                                                     uint32_t* counts, uint32_t* offsets,
                                                     uint32_t* gu_off, uint32_t* dn_off,
                                                     uint32_t bm, uint32_t gu_tiles,
                                                     uint32_t dn_tiles) {
    __shared__ uint32_t hist[1024];
    const uint32_t t = threadIdx.x;
    hist[t] = 0u;
    __syncthreads();
    for (uint32_t i = t; i < s; i += 1024u) {
        const uint32_t x = ids[i];
        if (x < e) atomicAdd(&hist[x], 1u);
    }
    __syncthreads();
    const uint32_t c = t < e ? hist[t] : 0u;
    const uint32_t rows = (c + bm - 1u) / bm;
    uint32_t total;
    const uint32_t before = block_excl_scan_1024(c, &total);
    const uint32_t rbefore = block_excl_scan_1024(rows, &total);
    if (t < e) {
        counts[t] = c;
        offsets[t] = before;
        gu_off[t] = rbefore * gu_tiles;
        dn_off[t] = rbefore * dn_tiles;
    }
}

// Prefill step, routing half 2: workgroup ex < e scatters expert ex's slots
// and writes its block-map entries; workgroup e zeroes both maps' unused
// tails (entries past the last expert's), which the GEMMs skip.
__global__ __launch_bounds__(1024) void k_sorted_blocks(const uint32_t* ids, const uint32_t* counts,
                                                        const uint32_t* offsets, const uint32_t* gu_off,
                                                        const uint32_t* dn_off, uint32_t* ids_sorted,
                                                        uint32_t* slotpos, uint32_t s, uint32_t topk,
                                                        uint32_t e, uint4* gu, uint32_t max_gu,
                                                        uint4* dn, uint32_t max_dn, uint32_t bm,
                                                        uint32_t gu_bn, uint32_t dn_bn, uint32_t gu_n,
                                                        uint32_t dn_n) {
    const uint32_t ex = blockIdx.x;
    if (ex == e) {
        const uint32_t rows = (counts[e - 1] + bm - 1) / bm;
        const uint32_t gu_end = gu_off[e - 1] + rows * (gu_n / gu_bn);
        const uint32_t dn_end = dn_off[e - 1] + rows * (dn_n / dn_bn);
        for (uint32_t i = gu_end + threadIdx.x; i < max_gu; i += blockDim.x) gu[i] = make_uint4(0, 0, 0, 0);
        for (uint32_t i = dn_end + threadIdx.x; i < max_dn; i += blockDim.x) dn[i] = make_uint4(0, 0, 0, 0);
        return;
    }
    const uint32_t n = counts[ex];
    if (n == 0) {
        return;
    }
    write_map(gu, max_gu, gu_off[ex], n, offsets[ex], ex, bm, gu_bn, gu_n);
    write_map(dn, max_dn, dn_off[ex], n, offsets[ex], ex, bm, dn_bn, dn_n);
    scatter_expert(ids, ex, offsets[ex], ids_sorted, slotpos, s, topk);
}

// Prefill routing in three launches after the router logits (kRouteBlock
// tokens per block; one block's slots fit one 256-thread workgroup).
//
// k_route_hist: workgroup j routes tokens [16 j, 16 j + 16), one per wave,
// with the scores in registers (lane l holds experts l + 64 i) and the
// selection and weights of route_select_ids / route_weights_regs; it writes
// the ids and weights and the block's expert histogram hb[j][0 .. e).
constexpr uint32_t kRouteBlock = mh::kPrefillRouteBlock;

template <int TK, int EB>
__global__ __launch_bounds__(1024) void k_route_hist(const float* logits, const float* bias, uint32_t m,
                                                     uint32_t e, int mode, float eps, uint32_t* ids, uint16_t* gw,
                                                     uint32_t* hb) {
    __shared__ uint32_t hist[mh::kMaxExperts];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t t0 = blockIdx.x * kRouteBlock;
    const uint32_t nt = min(kRouteBlock, m - t0);
    for (uint32_t i = threadIdx.x; i < e; i += blockDim.x) {
        hist[i] = 0u;
    }
    const uint32_t t = t0 + min(wave, nt - 1u);
    float sc[EB], cd[EB];
#pragma unroll
    for (int q = 0; q < EB; ++q) {
        const uint32_t i = lane + 64u * q;
        sc[q] = 0.0f;
        cd[q] = -__builtin_inff();
        if (i < e) {
            mh::route_score(logits[static_cast<size_t>(t) * e + i], bias ? bias[i] : 0.0f, mode, sc[q], cd[q]);
        }
    }
    uint32_t idv[TK];
    float sv[TK];
    mh::route_select_ids<TK, EB>(sc, cd, idv, sv);
    uint32_t wb[TK];
    mh::route_weights_regs<TK>(sv, mode, eps, wb);
    __syncthreads();
    if (wave < nt && lane < static_cast<uint32_t>(TK)) {
        uint32_t x = idv[0], w = wb[0];
#pragma unroll
        for (int r = 1; r < TK; ++r) {
            x = lane == static_cast<uint32_t>(r) ? idv[r] : x;
            w = lane == static_cast<uint32_t>(r) ? wb[r] : w;
        }
        ids[static_cast<size_t>(t) * TK + lane] = x;
        gw[static_cast<size_t>(t) * TK + lane] = static_cast<uint16_t>(w);
        atomicAdd(&hist[x], 1u);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < e; i += blockDim.x) {
        hb[static_cast<size_t>(blockIdx.x) * e + i] = hist[i];
    }
}

// Exclusive prefix over a 256-thread workgroup (one value per thread);
// *total the sum.  Ends with a barrier.
__device__ __forceinline__ uint32_t block_excl_scan_256(uint32_t v, uint32_t* total) {
    __shared__ uint32_t wtot[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_up(inc, d);
        if (lane >= d) inc += o;
    }
    if (lane == 63) wtot[wave] = inc;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t t = wtot[w];
        before += w < wave ? t : 0u;
        all += t;
    }
    __syncthreads();
    *total = all;
    return before + inc - v;
}

// k_hist_prefix: workgroup x scans expert x's column of the block
// histograms in block order: hb[b][x] becomes the count of expert x's slots
// in blocks before b (in place), tot[x] the expert's total.
__global__ __launch_bounds__(256) void k_hist_prefix(uint32_t* hb, uint32_t* tot, uint32_t nblk, uint32_t e) {
    const uint32_t x = blockIdx.x;
    uint32_t carry = 0u;
    for (uint32_t b0 = 0; b0 < nblk; b0 += 256u) {
        const uint32_t b = b0 + threadIdx.x;
        const uint32_t v = b < nblk ? hb[static_cast<size_t>(b) * e + x] : 0u;
        uint32_t all;
        const uint32_t before = block_excl_scan_256(v, &all);
        if (b < nblk) {
            hb[static_cast<size_t>(b) * e + x] = carry + before;
        }
        carry += all;
    }
    if (threadIdx.x == 0) {
        tot[x] = carry;
    }
}

// The map rows of expert ex in launch order (gu_ord / dn_ord, see
// mh::seg_rank_of): its row r's rank among all rows by row count (rows_l:
// every map row's count), then its nt entries at their workgroups.
__device__ void write_ordered(uint4* ord, uint32_t rank, uint32_t m0, uint32_t m_end, uint32_t ex, uint32_t bn,
                              uint32_t n_cols) {
    const uint32_t nt = n_cols / bn;
    for (uint32_t t = threadIdx.x; t < nt; t += blockDim.x) {
        ord[mh::seg_workgroup_of(rank, t, nt)] = make_uint4(m0, ex * n_cols + t * bn, t * bn, m_end);
    }
}

// k_scatter_maps: workgroup j takes the expert totals (counts, offsets and
// both block-map offsets by two workgroup scans) and its block's prefix row,
// scatters block j's slots stably (slot order; ranks within each 64-slot
// chunk from ballots), writes the block-map entries of experts j, j + G, ...
// and zeroes its share of both maps' unused tails.  Workgroup 0 writes
// counts, offsets and the block-map offsets.  With gu_ord / dn_ord, the same
// entries again in launch order (unused workgroups' entries zero).
__global__ __launch_bounds__(256) void k_scatter_maps(const uint32_t* ids, const uint32_t* pre, const uint32_t* tot,
                                                      uint32_t m, uint32_t e, uint32_t topk, uint32_t* counts,
                                                      uint32_t* offsets, uint32_t* gu_off, uint32_t* dn_off,
                                                      uint32_t* ids_sorted, uint32_t* slotpos, uint4* gu,
                                                      uint32_t max_gu, uint4* dn, uint32_t max_dn, uint32_t bm,
                                                      uint32_t gu_bn, uint32_t dn_bn, uint32_t gu_n, uint32_t dn_n,
                                                      uint4* gu_ord, uint4* dn_ord, uint32_t gu_grid,
                                                      uint32_t dn_grid) {
    __shared__ uint32_t tot_l[mh::kMaxExperts], off_l[mh::kMaxExperts], base_l[mh::kMaxExperts],
        rb_l[mh::kMaxExperts];
    __shared__ uint32_t chist[4][mh::kMaxExperts];
    __shared__ uint32_t rows_l[mh::kMaxOrderedRows];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t j = blockIdx.x;
    const uint32_t total = tid < e ? tot[tid] : 0u;
    const uint32_t before = tid < e ? pre[static_cast<size_t>(j) * e + tid] : 0u;
    // this block's slots (at most 256, one per thread)
    const uint32_t s0 = j * kRouteBlock * topk;
    const uint32_t ns = min(kRouteBlock, m - j * kRouteBlock) * topk;
    const bool act = tid < ns;
    const uint32_t v = act ? ids[s0 + tid] : 0xffffffffu;
    uint32_t all;
    const uint32_t off = block_excl_scan_256(total, &all);
    const uint32_t rows = tid < e ? (total + bm - 1u) / bm : 0u;
    uint32_t rows_all;
    const uint32_t rbefore = block_excl_scan_256(rows, &rows_all);
    const uint32_t gu_tiles = gu_n / gu_bn, dn_tiles = dn_n / dn_bn;
    if (tid < e) {
        tot_l[tid] = total;
        off_l[tid] = off;
        base_l[tid] = off + before;
        rb_l[tid] = rbefore;
        if (j == 0) {
            counts[tid] = total;
            offsets[tid] = off;
            gu_off[tid] = rbefore * gu_tiles;
            dn_off[tid] = rbefore * dn_tiles;
        }
    }
    for (uint32_t i = tid; i < 4u * mh::kMaxExperts; i += 256u) {
        (&chist[0][0])[i] = 0u;
    }
    __syncthreads();
    // block-map entries of experts j, j + G, ...
    for (uint32_t ex = j; ex < e; ex += gridDim.x) {
        if (tot_l[ex] != 0u) {
            write_map(gu, max_gu, rb_l[ex] * gu_tiles, tot_l[ex], off_l[ex], ex, bm, gu_bn, gu_n);
            write_map(dn, max_dn, rb_l[ex] * dn_tiles, tot_l[ex], off_l[ex], ex, bm, dn_bn, dn_n);
        }
    }
    // the maps' unused tails
    for (uint32_t i = rows_all * gu_tiles + j * 256u + tid; i < max_gu; i += gridDim.x * 256u) {
        gu[i] = make_uint4(0, 0, 0, 0);
    }
    for (uint32_t i = rows_all * dn_tiles + j * 256u + tid; i < max_dn; i += gridDim.x * 256u) {
        dn[i] = make_uint4(0, 0, 0, 0);
    }
    if (gu_ord != nullptr) {
        // every map row's count (rows_all <= kMaxOrderedRows, checked on the host)
        for (uint32_t ex = tid; ex < e; ex += 256u) {
            for (uint32_t r = 0; r * bm < tot_l[ex]; ++r) {
                rows_l[rb_l[ex] + r] = min(bm, tot_l[ex] - r * bm);
            }
        }
        __syncthreads();
        for (uint32_t ex = j; ex < e; ex += gridDim.x) {
            for (uint32_t r = 0; r * bm < tot_l[ex]; ++r) {
                const uint32_t c = rb_l[ex] + r, w = rows_l[c];
                uint32_t ahead = 0u;
                for (uint32_t d = tid; d < rows_all; d += 256u) {
                    const uint32_t v = rows_l[d];
                    ahead += (v > w || (v == w && d < c)) ? 1u : 0u;
                }
                uint32_t rank;
                (void)block_excl_scan_256(ahead, &rank);
                const uint32_t m0 = off_l[ex] + r * bm, m_end = min(m0 + bm, off_l[ex] + tot_l[ex]);
                write_ordered(gu_ord, rank, m0, m_end, ex, gu_bn, gu_n);
                write_ordered(dn_ord, rank, m0, m_end, ex, dn_bn, dn_n);
            }
        }
        // workgroups past the used rows' ranks take no entry
        for (uint32_t b = j * 256u + tid; b < gu_grid; b += gridDim.x * 256u) {
            if (mh::seg_rank_of(b, gu_tiles) >= rows_all) {
                gu_ord[b] = make_uint4(0, 0, 0, 0);
            }
        }
        for (uint32_t b = j * 256u + tid; b < dn_grid; b += gridDim.x * 256u) {
            if (mh::seg_rank_of(b, dn_tiles) >= rows_all) {
                dn_ord[b] = make_uint4(0, 0, 0, 0);
            }
        }
    }
    // rank within the wave's 64-slot chunk by ballots over the distinct experts
    const unsigned long long below = (1ull << lane) - 1ull;
    unsigned long long todo = __ballot(act);
    uint32_t rank = 0u;
    while (todo != 0ull) {
        const int leader = __ffsll(static_cast<long long>(todo)) - 1;
        const uint32_t lv = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), leader));
        const unsigned long long same = __ballot(v == lv);
        if (v == lv) {
            rank = static_cast<uint32_t>(__popcll(same & below));
        }
        if (lane == static_cast<uint32_t>(leader)) {
            chist[wave][lv] = static_cast<uint32_t>(__popcll(same));
        }
        todo &= ~same;
    }
    __syncthreads();
    if (act) {
        uint32_t pos = base_l[v] + rank;
        for (uint32_t c = 0; c < wave; ++c) {
            pos += chist[c][v];
        }
        ids_sorted[pos] = (s0 + tid) / topk;
        slotpos[s0 + tid] = pos;
    }
}

unsigned grid_for(size_t n, unsigned per = 256) {
    const size_t want = (n + per - 1) / per;
    const size_t cap = static_cast<size_t>(mh::cu_count()) * 16;
    return static_cast<unsigned>(want == 0 ? 1 : (want < cap ? want : cap));
}

}  // namespace

extern "C" {

int mh_moe_zero_counts(uint32_t* counts, uint32_t e, mh_stream_t stream) {
    MH_ENSURE(counts && e > 0, MH_ERR_INVALID, "mh_moe_zero_counts: bad arguments");
    hipLaunchKernelGGL(k_fill_u32, dim3(1), dim3(256), 0, mh::as_stream(stream), counts,
                       static_cast<size_t>(e), 0u);
    return mh::launch_status("mh_moe_zero_counts");
}

int mh_moe_count_slots(const uint32_t* ids, uint32_t* counts, uint32_t s, uint32_t e,
                       mh_stream_t stream) {
    MH_ENSURE(ids && counts, MH_ERR_INVALID, "mh_moe_count_slots: NULL argument");
    MH_ENSURE(e >= 1 && e <= 256, MH_ERR_UNSUPPORTED, "mh_moe_count_slots: %u experts", e);
    if (s == 0) return MH_OK;
    hipLaunchKernelGGL(k_count, dim3(grid_for(s, 4096)), dim3(256), 0, mh::as_stream(stream), ids,
                       counts, s, e);
    return mh::launch_status("mh_moe_count_slots");
}

int mh_moe_offsets(const uint32_t* counts, uint32_t* offsets, uint32_t e, mh_stream_t stream) {
    MH_ENSURE(counts && offsets, MH_ERR_INVALID, "mh_moe_offsets: NULL argument");
    MH_ENSURE(e >= 1 && e <= 1024, MH_ERR_UNSUPPORTED, "mh_moe_offsets: %u experts", e);
    hipLaunchKernelGGL(k_offsets, dim3(1), dim3(1024), 0, mh::as_stream(stream), counts, offsets, e);
    return mh::launch_status("mh_moe_offsets");
}

int mh_moe_sorted(const uint32_t* ids, const uint32_t* offsets, uint32_t* ids_sorted,
                  uint32_t* slotpos, uint32_t m, uint32_t e, uint32_t topk, mh_stream_t stream) {
    MH_ENSURE(ids && offsets && ids_sorted && slotpos, MH_ERR_INVALID, "mh_moe_sorted: NULL argument");
    MH_ENSURE(e >= 1 && topk >= 1, MH_ERR_INVALID, "mh_moe_sorted: e=%u topk=%u", e, topk);
    if (m == 0) return MH_OK;
    hipLaunchKernelGGL(k_sorted, dim3(e), dim3(1024), 0, mh::as_stream(stream), ids, offsets,
                       ids_sorted, slotpos, m * topk, topk);
    return mh::launch_status("mh_moe_sorted");
}

int mh_moe_zero_blocks(uint32_t* gu, uint32_t* dn, uint32_t n_gu, uint32_t n_dn,
                       mh_stream_t stream) {
    MH_ENSURE(gu && dn, MH_ERR_INVALID, "mh_moe_zero_blocks: NULL argument");
    const hipStream_t s = mh::as_stream(stream);
    hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(4ull * n_gu)), dim3(256), 0, s, gu,
                       4ull * n_gu, 0u);
    hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(4ull * n_dn)), dim3(256), 0, s, dn,
                       4ull * n_dn, 0u);
    return mh::launch_status("mh_moe_zero_blocks");
}

int mh_moe_block_offsets(const uint32_t* counts, uint32_t* gu_off, uint32_t* dn_off, uint32_t e,
                         uint32_t bm, uint32_t gu_bn, uint32_t dn_bn, uint32_t gu_n,
                         uint32_t dn_n, mh_stream_t stream) {
    MH_ENSURE(counts && gu_off && dn_off, MH_ERR_INVALID, "mh_moe_block_offsets: NULL argument");
    MH_ENSURE(bm > 0 && gu_bn > 0 && dn_bn > 0 && gu_n % gu_bn == 0 && dn_n % dn_bn == 0,
              MH_ERR_INVALID, "mh_moe_block_offsets: tiles bm=%u bn=%u/%u do not divide %u/%u",
              bm, gu_bn, dn_bn, gu_n, dn_n);
    MH_ENSURE(e >= 1 && e <= 1024, MH_ERR_UNSUPPORTED, "mh_moe_block_offsets: %u experts", e);
    hipLaunchKernelGGL(k_block_offsets, dim3(1), dim3(1024), 0, mh::as_stream(stream), counts, gu_off,
                       dn_off, e, bm, gu_n / gu_bn, dn_n / dn_bn);
    return mh::launch_status("mh_moe_block_offsets");
}

int mh_moe_blocks(const uint32_t* counts, const uint32_t* offsets, const uint32_t* gu_off,
                  const uint32_t* dn_off, uint32_t* gu, uint32_t max_gu, uint32_t* dn,
                  uint32_t max_dn, uint32_t e, uint32_t bm, uint32_t gu_bn, uint32_t dn_bn,
                  uint32_t gu_n, uint32_t dn_n, mh_stream_t stream) {
    MH_ENSURE(counts && offsets && gu_off && dn_off && gu && dn, MH_ERR_INVALID,
              "mh_moe_blocks: NULL argument");
    MH_ENSURE(mh::aligned(gu, 16) && mh::aligned(dn, 16), MH_ERR_ALIGN,
              "mh_moe_blocks: maps must be 16-byte aligned");
    MH_ENSURE(bm > 0 && gu_bn > 0 && dn_bn > 0 && gu_n % gu_bn == 0 && dn_n % dn_bn == 0,
              MH_ERR_INVALID, "mh_moe_blocks: tiles bm=%u bn=%u/%u do not divide %u/%u", bm,
              gu_bn, dn_bn, gu_n, dn_n);
    hipLaunchKernelGGL(k_blocks, dim3(e), dim3(128), 0, mh::as_stream(stream), counts, offsets,
                       gu_off, dn_off, reinterpret_cast<uint4*>(gu), max_gu,
                       reinterpret_cast<uint4*>(dn), max_dn, bm, gu_bn, dn_bn, gu_n, dn_n);
    return mh::launch_status("mh_moe_blocks");
}

}  // extern "C"

namespace mh {

// Internal to mh_moe_prefill (declared in mh_host.hpp, not in the public
// header): the two fused routing launches above.
int moe_route_sort_maps(const float* logits, const float* bias, int mode, float eps, uint32_t m,
                        uint32_t e, uint32_t topk, uint32_t* ids, uint16_t* gw, uint32_t* hb,
                        uint32_t* counts, uint32_t* offsets, uint32_t* gu_off, uint32_t* dn_off,
                        uint32_t* ids_sorted, uint32_t* slotpos, uint32_t* gu, uint32_t max_gu, uint32_t* dn,
                        uint32_t max_dn, uint32_t bm, uint32_t gu_bn, uint32_t dn_bn, uint32_t gu_n,
                        uint32_t dn_n, mh_stream_t stream, bool routed, uint32_t* gu_ord, uint32_t* dn_ord) {
    static_assert(kRouteBlock * mh::kMaxTopk <= 256, "a block's slots, one per thread");
    MH_ENSURE(e >= 1 && e <= static_cast<uint32_t>(mh::kMaxExperts) && topk >= 1 &&
                  topk <= static_cast<uint32_t>(mh::kMaxTopk) && topk <= e,
              MH_ERR_INVALID, "prefill routing: %u experts, top-%u", e, topk);
    const hipStream_t st = mh::as_stream(stream);
    const uint32_t nblk = (m + kRouteBlock - 1u) / kRouteBlock;
    const bool eb1 = e <= 64u;
#define MH_ROUTE_HIST(TK)                                                                                   \
    case TK:                                                                                                \
        if (eb1) {                                                                                          \
            hipLaunchKernelGGL((k_route_hist<TK, 1>), dim3(nblk), dim3(1024), 0, st, logits, bias, m, e, mode, \
                               eps, ids, gw, hb);                                                           \
        } else {                                                                                            \
            hipLaunchKernelGGL((k_route_hist<TK, 4>), dim3(nblk), dim3(1024), 0, st, logits, bias, m, e, mode, \
                               eps, ids, gw, hb);                                                           \
        }                                                                                                   \
        break;
    if (!routed) {
        switch (topk) {
            MH_ROUTE_HIST(1) MH_ROUTE_HIST(2) MH_ROUTE_HIST(3) MH_ROUTE_HIST(4)
            MH_ROUTE_HIST(5) MH_ROUTE_HIST(6) MH_ROUTE_HIST(7) MH_ROUTE_HIST(8)
            default: break;
        }
        MH_TRY(mh::launch_status("k_route_hist"));
    }
#undef MH_ROUTE_HIST
    uint32_t* tot = hb + static_cast<size_t>(nblk) * e;
    hipLaunchKernelGGL(k_hist_prefix, dim3(e), dim3(256), 0, st, hb, tot, nblk, e);
    MH_TRY(mh::launch_status("k_hist_prefix"));
    const uint32_t gu_tiles = gu_n / gu_bn, dn_tiles = dn_n / dn_bn;
    if (gu_ord != nullptr || dn_ord != nullptr) {
        MH_ENSURE(gu_ord != nullptr && dn_ord != nullptr && max_gu / gu_tiles == max_dn / dn_tiles &&
                      max_gu / gu_tiles <= mh::kMaxOrderedRows,
                  MH_ERR_UNSUPPORTED, "prefill routing: launch-ordered maps of %u rows", max_gu / gu_tiles);
    }
    hipLaunchKernelGGL(k_scatter_maps, dim3(nblk), dim3(256), 0, st, ids, hb, tot, m, e, topk, counts, offsets,
                       gu_off, dn_off, ids_sorted, slotpos, reinterpret_cast<uint4*>(gu), max_gu,
                       reinterpret_cast<uint4*>(dn), max_dn, bm, gu_bn, dn_bn, gu_n, dn_n,
                       reinterpret_cast<uint4*>(gu_ord), reinterpret_cast<uint4*>(dn_ord),
                       mh::map_grid(max_gu, gu_tiles), mh::map_grid(max_dn, dn_tiles));
    return mh::launch_status("k_scatter_maps");
}

int moe_sort_maps(const uint32_t* ids, uint32_t s, uint32_t e, uint32_t topk,
                              uint32_t* counts, uint32_t* offsets, uint32_t* gu_off,
                              uint32_t* dn_off, uint32_t* ids_sorted, uint32_t* slotpos,
                              uint32_t* gu, uint32_t max_gu, uint32_t* dn, uint32_t max_dn,
                              uint32_t bm, uint32_t gu_bn, uint32_t dn_bn, uint32_t gu_n,
                              uint32_t dn_n, mh_stream_t stream) {
    const hipStream_t st = mh::as_stream(stream);
    hipLaunchKernelGGL(k_count_scan, dim3(1), dim3(1024), 0, st, ids, s, e, counts, offsets, gu_off,
                       dn_off, bm, gu_n / gu_bn, dn_n / dn_bn);
    MH_TRY(mh::launch_status("k_count_scan"));
    hipLaunchKernelGGL(k_sorted_blocks, dim3(e + 1), dim3(1024), 0, st, ids, counts, offsets, gu_off,
                       dn_off, ids_sorted, slotpos, s, topk, e, reinterpret_cast<uint4*>(gu), max_gu,
                       reinterpret_cast<uint4*>(dn), max_dn, bm, gu_bn, dn_bn, gu_n, dn_n);
    return mh::launch_status("k_sorted_blocks");
}

}  // namespace mh

extern "C" {

int mh_gather_rows_bf16(const uint16_t* table, const uint32_t* ids, uint16_t* out, uint32_t m,
                        uint32_t h, uint32_t n_table, mh_stream_t stream) {
    MH_ENSURE(table && ids && out, MH_ERR_INVALID, "mh_gather_rows_bf16: NULL argument");
    MH_ENSURE(h % 8 == 0 && n_table > 0, MH_ERR_UNSUPPORTED,
              "mh_gather_rows_bf16: row width %u not a multiple of 8", h);
    MH_ENSURE(mh::aligned(table, 16) && mh::aligned(out, 16), MH_ERR_ALIGN,
              "mh_gather_rows_bf16: rows must be 16-byte aligned");
    if (m == 0) return MH_OK;
    hipLaunchKernelGGL(k_gather_rows, dim3(grid_for(static_cast<size_t>(m) * h / 8)), dim3(256), 0,
                       mh::as_stream(stream), table, ids, out, m, h, n_table);
    return mh::launch_status("mh_gather_rows_bf16");
}

int mh_silu_mul_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n,
                     mh_stream_t stream) {
    MH_ENSURE(gate && up && out, MH_ERR_INVALID, "mh_silu_mul_bf16: NULL argument");
    if (n == 0) return MH_OK;
    hipLaunchKernelGGL(k_silu_mul, dim3(grid_for(n)), dim3(256), 0, mh::as_stream(stream), gate, up,
                       out, n);
    return mh::launch_status("mh_silu_mul_bf16");
}

int mh_moe_combine_rows(const uint16_t* sorted, const uint32_t* slotpos, const uint16_t* weights,
                        uint16_t* out, uint32_t m, uint32_t h, uint32_t topk, mh_stream_t stream) {
    MH_ENSURE(sorted && slotpos && weights && out, MH_ERR_INVALID,
              "mh_moe_combine_rows: NULL argument");
    MH_ENSURE(h % 8 == 0, MH_ERR_UNSUPPORTED, "mh_moe_combine_rows: width %u not a multiple of 8", h);
    MH_ENSURE(topk >= 1 && topk <= 8, MH_ERR_INVALID, "mh_moe_combine_rows: topk %u", topk);
    MH_ENSURE(mh::aligned(sorted, 16) && mh::aligned(out, 16), MH_ERR_ALIGN,
              "mh_moe_combine_rows: rows must be 16-byte aligned");
    if (m == 0) return MH_OK;
    const dim3 grid(grid_for(static_cast<size_t>(m) * h / 8));
    const hipStream_t st = mh::as_stream(stream);
#define MH_COMBINE(TK)                                                                                   \
    case TK:                                                                                             \
        hipLaunchKernelGGL(k_combine<TK>, grid, dim3(256), 0, st, sorted, slotpos, weights, out, m, h, m * TK); \
        break;
    switch (topk) {
        MH_COMBINE(1) MH_COMBINE(2) MH_COMBINE(3) MH_COMBINE(4)
        MH_COMBINE(5) MH_COMBINE(6) MH_COMBINE(7) MH_COMBINE(8)
        default: break;
    }
#undef MH_COMBINE
    return mh::launch_status("mh_moe_combine_rows");
}

}  // extern "C"

/*
 * oracle_prefill.c -- prefill MoE: counting sort, block maps, row gather,
 * SwiGLU, combine and the grouped Q4 GEMM.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ORC_THREADS (orc_get_threads())

static inline float bfr(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

/* ------------------------------------------------------ counting sort --- */

void orc_moe_count(const uint32_t* ids, uint32_t s, uint32_t e, uint32_t* counts) {
    memset(counts, 0, e * sizeof(uint32_t));
    for (uint32_t i = 0; i < s; ++i) {
        counts[ids[i]] += 1;
    }
}

void orc_moe_offsets(const uint32_t* counts, uint32_t e, uint32_t* offsets) {
    uint32_t acc = 0;
    for (uint32_t i = 0; i < e; ++i) {
        offsets[i] = acc;
        acc += counts[i];
    }
}

void orc_moe_sorted(const uint32_t* ids, const uint32_t* offsets, uint32_t m, uint32_t e,
                    uint32_t topk, uint32_t* ids_sorted, uint32_t* slotpos) {
    uint32_t* next = (uint32_t*)malloc(e * sizeof(uint32_t));
    memcpy(next, offsets, e * sizeof(uint32_t));
    for (uint32_t t = 0; t < m; ++t) {
        for (uint32_t r = 0; r < topk; ++r) {
            const uint32_t ex = ids[(size_t)t * topk + r];
            const uint32_t pos = next[ex]++;
            ids_sorted[pos] = t;
            slotpos[(size_t)t * topk + r] = pos;
        }
    }
    free(next);
}

/* ---------------------------------------------------------- block map --- */

void orc_moe_block_offsets(const uint32_t* counts, uint32_t e, uint32_t bm, uint32_t gu_bn,
                           uint32_t dn_bn, uint32_t gu_n, uint32_t dn_n, uint32_t* gu_off,
                           uint32_t* dn_off) {
    uint32_t ag = 0, ad = 0;
    for (uint32_t i = 0; i < e; ++i) {
        gu_off[i] = ag;
        dn_off[i] = ad;
        const uint32_t rows = (counts[i] + bm - 1) / bm;
        ag += rows * (gu_n / gu_bn);
        ad += rows * (dn_n / dn_bn);
    }
}

static void fill_map(uint32_t count, uint32_t off, uint32_t base, uint32_t ex, uint32_t bm,
                     uint32_t bn, uint32_t n_cols, uint32_t* map, uint32_t max_entries) {
    const uint32_t rows = (count + bm - 1) / bm;
    const uint32_t tiles = n_cols / bn;
    for (uint32_t i = 0; i < rows * tiles; ++i) {
        if (base + i >= max_entries) {
            return;
        }
        const uint32_t mt = i / tiles, nt = i % tiles;
        const uint32_t m0 = off + mt * bm;
        const uint32_t m_end = (m0 + bm < off + count) ? m0 + bm : off + count;
        const uint32_t n0 = nt * bn;
        uint32_t* d = map + 4 * (size_t)(base + i);
        d[0] = m0;
        d[1] = ex * n_cols + n0;
        d[2] = n0;
        d[3] = m_end;
    }
}

void orc_moe_blocks(const uint32_t* counts, const uint32_t* offsets, const uint32_t* gu_off,
                    const uint32_t* dn_off, uint32_t e, uint32_t bm, uint32_t gu_bn,
                    uint32_t dn_bn, uint32_t gu_n, uint32_t dn_n, uint32_t* gu, uint32_t max_gu,
                    uint32_t* dn, uint32_t max_dn) {
    memset(gu, 0, (size_t)max_gu * 16);
    memset(dn, 0, (size_t)max_dn * 16);
    for (uint32_t i = 0; i < e; ++i) {
        if (counts[i] == 0) {
            continue;
        }
        fill_map(counts[i], offsets[i], gu_off[i], i, bm, gu_bn, gu_n, gu, max_gu);
        fill_map(counts[i], offsets[i], dn_off[i], i, bm, dn_bn, dn_n, dn, max_dn);
    }
}

/* --------------------------------------------------------- elementwise --- */

void orc_gather_rows_bf16(const uint16_t* table, const uint32_t* ids, uint32_t m, uint32_t h,
                          uint16_t* out) {
    for (uint32_t i = 0; i < m; ++i) {
        memcpy(out + (size_t)i * h, table + (size_t)ids[i] * h, (size_t)h * 2);
    }
}

void orc_silu_mul_bf16(const uint16_t* gate, const uint16_t* up, size_t n, uint16_t* out) {
    for (size_t i = 0; i < n; ++i) {
        const float g = orc_bf16_to_f32(gate[i]);
        const float s = bfr(g / (1.0f + orc_expf(-g)));
        out[i] = orc_f32_to_bf16(s * orc_bf16_to_f32(up[i]));
    }
}

void orc_moe_combine_rows(const uint16_t* sorted, const uint32_t* slotpos, const uint16_t* w,
                          uint32_t m, uint32_t h, uint32_t topk, uint16_t* out) {
#pragma omp parallel for schedule(static) num_threads(ORC_THREADS)
    for (long t = 0; t < (long)m; ++t) {
        for (uint32_t c = 0; c < h; ++c) {
            float sum = 0.0f;
            for (uint32_t r = 0; r < topk; ++r) {
                const uint32_t p = slotpos[(size_t)t * topk + r];
                const float wr = orc_bf16_to_f32(w[(size_t)t * topk + r]);
                sum = sum + bfr(wr * orc_bf16_to_f32(sorted[(size_t)p * h + c]));
            }
            out[(size_t)t * h + c] = orc_f32_to_bf16(sum);
        }
    }
}

/* -------------------------------------------------------- grouped GEMM --- */

/* Dequantize rows [r0, r0 + nr) of a Q4 matrix to f32, transposed: wt[k][j]. */
static void dequant_rows_t(const orc_qw* w, uint32_t r0, uint32_t nr, float* wt) {
    const uint32_t K = w->k, G = K / w->gs;
    const size_t words = (size_t)K * w->bits / 32;
    for (uint32_t j = 0; j < nr; ++j) {
        const uint32_t r = r0 + j;
        const uint32_t* row = w->codes + (size_t)r * words;
        for (uint32_t kk = 0; kk < K; ++kk) {
            const uint32_t bit = w->bits * kk;
            uint32_t v = row[bit >> 5] >> (bit & 31u);
            if ((bit & 31u) + w->bits > 32u) {
                v |= row[(bit >> 5) + 1] << (32u - (bit & 31u));
            }
            const float q = (float)(v & ((1u << w->bits) - 1u));
            const float s = orc_bf16_to_f32(w->scales[(size_t)r * G + kk / w->gs]);
            const float b = orc_bf16_to_f32(w->biases[(size_t)r * G + kk / w->gs]);
            wt[(size_t)kk * nr + j] = bfr(fmaf(s, q, b));
        }
    }
}

/* acc[i][j] = sum_k a[i][k] * wt[k][j], ascending k, fmaf chain per element. */
static void rows_times_wt(const float* a, uint32_t nrows, uint32_t K, const float* wt,
                          uint32_t nc, float* acc) {
    for (uint32_t i = 0; i < nrows; ++i) {
        float* ai = acc + (size_t)i * nc;
        for (uint32_t j = 0; j < nc; ++j) {
            ai[j] = 0.0f;
        }
        const float* xr = a + (size_t)i * K;
        for (uint32_t kk = 0; kk < K; ++kk) {
            const float xv = xr[kk];
            const float* wr = wt + (size_t)kk * nc;
            for (uint32_t j = 0; j < nc; ++j) {
                ai[j] = fmaf(xv, wr[j], ai[j]);
            }
        }
    }
}

void orc_gemm_q4_grouped(const uint16_t* a, const orc_qw* w, uint16_t* c,
                         const uint32_t* blocks, uint32_t n_blocks, uint32_t n, uint32_t bn) {
    const uint32_t K = w->k;
#pragma omp parallel for schedule(dynamic) num_threads(ORC_THREADS)
    for (long bi = 0; bi < (long)n_blocks; ++bi) {
        const uint32_t* blk = blocks + 4 * (size_t)bi;
        const uint32_t m0 = blk[0], brow = blk[1], n0 = blk[2], m_end = blk[3];
        if (m0 >= m_end) {
            continue;
        }
        const uint32_t nr = m_end - m0;
        float* wt = (float*)malloc((size_t)K * bn * sizeof(float));
        float* af = (float*)malloc((size_t)nr * K * sizeof(float));
        float* acc = (float*)malloc((size_t)nr * bn * sizeof(float));
        dequant_rows_t(w, brow, bn, wt);
        for (size_t i = 0; i < (size_t)nr * K; ++i) {
            af[i] = orc_bf16_to_f32(a[(size_t)m0 * K + i]);
        }
        rows_times_wt(af, nr, K, wt, bn, acc);
        for (uint32_t i = 0; i < nr; ++i) {
            for (uint32_t j = 0; j < bn; ++j) {
                c[(size_t)(m0 + i) * n + n0 + j] = orc_f32_to_bf16(acc[(size_t)i * bn + j]);
            }
        }
        free(acc);
        free(af);
        free(wt);
    }
}

/* --------------------------------------------------------- MoE prefill --- */

void orc_moe_prefill_masked(const void* router, int router_is_f32, const float* bias, int mode,
                            float eps, const orc_qw* gate, const orc_qw* up, const orc_qw* down,
                            uint32_t n_experts, uint32_t topk, uint32_t d_model, uint32_t n_inter,
                            uint32_t m, const uint16_t* x, const uint8_t* token_mask,
                            uint16_t* out, uint32_t* ids_o, uint16_t* gw_o, uint32_t* counts_o,
                            uint32_t* offsets_o, uint32_t* ids_sorted_o, uint32_t* slotpos_o,
                            uint16_t* act_o, uint16_t* ed_o) {
    const uint32_t s = m * topk, E = n_experts, H = d_model, I = n_inter;
    float* logits = (float*)malloc((size_t)m * E * sizeof(float));
    uint32_t* ids = (uint32_t*)malloc((size_t)s * 4);
    uint16_t* gw = (uint16_t*)malloc((size_t)s * 2);
    uint32_t* counts = (uint32_t*)malloc(E * 4);
    uint32_t* offsets = (uint32_t*)malloc(E * 4);
    uint32_t* ids_sorted = (uint32_t*)malloc((size_t)s * 4);
    uint32_t* slotpos = (uint32_t*)malloc((size_t)s * 4);
    uint16_t* act = (uint16_t*)malloc((size_t)s * I * 2);
    uint16_t* ed = (uint16_t*)malloc((size_t)s * H * 2);

    orc_gemv_dense(router, router_is_f32, x, m, E, H, logits);
    orc_route(logits, bias, m, E, topk, mode, eps, ids, gw);
    orc_moe_count(ids, s, E, counts);
    orc_moe_offsets(counts, E, offsets);
    orc_moe_sorted(ids, offsets, m, E, topk, ids_sorted, slotpos);

    enum { RB = 8 };
    /* rows of each expert segment to compute (all, or those of masked-in tokens) */
    uint32_t* live = (uint32_t*)malloc((size_t)s * 4);
    uint32_t* n_live = (uint32_t*)calloc(E, 4);
    for (uint32_t ex = 0; ex < E; ++ex) {
        for (uint32_t i = 0; i < counts[ex]; ++i) {
            const uint32_t row = offsets[ex] + i;
            if (!token_mask || token_mask[ids_sorted[row]]) {
                live[offsets[ex] + n_live[ex]++] = row;
            }
        }
    }
    memset(act, 0, (size_t)s * I * 2);
    memset(ed, 0, (size_t)s * H * 2);
#pragma omp parallel for schedule(dynamic) num_threads(ORC_THREADS)
    for (long ex = 0; ex < (long)E; ++ex) {
        const uint32_t cnt = n_live[ex], off = offsets[ex];
        if (cnt == 0) {
            continue;
        }
        float* wg = (float*)malloc((size_t)H * I * sizeof(float));
        float* wu = (float*)malloc((size_t)H * I * sizeof(float));
        float* wd = (float*)malloc((size_t)I * H * sizeof(float));
        float* xa = (float*)malloc((size_t)RB * H * sizeof(float));
        float* ga = (float*)malloc((size_t)RB * I * sizeof(float));
        float* ua = (float*)malloc((size_t)RB * I * sizeof(float));
        float* aa = (float*)malloc((size_t)RB * I * sizeof(float));
        float* da = (float*)malloc((size_t)RB * H * sizeof(float));
        dequant_rows_t(gate, (uint32_t)ex * I, I, wg);
        dequant_rows_t(up, (uint32_t)ex * I, I, wu);
        dequant_rows_t(down, (uint32_t)ex * H, H, wd);
        for (uint32_t i0 = 0; i0 < cnt; i0 += RB) {
            const uint32_t nr = (cnt - i0 < RB) ? cnt - i0 : RB;
            for (uint32_t i = 0; i < nr; ++i) {
                const uint32_t t = ids_sorted[live[off + i0 + i]];
                for (uint32_t kk = 0; kk < H; ++kk) {
                    xa[(size_t)i * H + kk] = orc_bf16_to_f32(x[(size_t)t * H + kk]);
                }
            }
            rows_times_wt(xa, nr, H, wg, I, ga);
            rows_times_wt(xa, nr, H, wu, I, ua);
            for (uint32_t i = 0; i < nr; ++i) {
                for (uint32_t j = 0; j < I; ++j) {
                    const float g = bfr(ga[(size_t)i * I + j]);
                    const float u = bfr(ua[(size_t)i * I + j]);
                    const float sg = bfr(g / (1.0f + orc_expf(-g)));
                    const uint16_t av = orc_f32_to_bf16(sg * u);
                    act[(size_t)live[off + i0 + i] * I + j] = av;
                    aa[(size_t)i * I + j] = orc_bf16_to_f32(av);
                }
            }
            rows_times_wt(aa, nr, I, wd, H, da);
            for (uint32_t i = 0; i < nr; ++i) {
                for (uint32_t h = 0; h < H; ++h) {
                    ed[(size_t)live[off + i0 + i] * H + h] = orc_f32_to_bf16(da[(size_t)i * H + h]);
                }
            }
        }
        free(da);
        free(aa);
        free(ua);
        free(ga);
        free(xa);
        free(wd);
        free(wu);
        free(wg);
    }
    free(n_live);
    free(live);
    orc_moe_combine_rows(ed, slotpos, gw, m, H, topk, out);

    if (ids_o) memcpy(ids_o, ids, (size_t)s * 4);
    if (gw_o) memcpy(gw_o, gw, (size_t)s * 2);
    if (counts_o) memcpy(counts_o, counts, E * 4);
    if (offsets_o) memcpy(offsets_o, offsets, E * 4);
    if (ids_sorted_o) memcpy(ids_sorted_o, ids_sorted, (size_t)s * 4);
    if (slotpos_o) memcpy(slotpos_o, slotpos, (size_t)s * 4);
    if (act_o) memcpy(act_o, act, (size_t)s * I * 2);
    if (ed_o) memcpy(ed_o, ed, (size_t)s * H * 2);
    free(ed);
    free(act);
    free(slotpos);
    free(ids_sorted);
    free(offsets);
    free(counts);
    free(gw);
    free(ids);
    free(logits);
}

void orc_moe_prefill(const void* router, int router_is_f32, const float* bias, int mode,
                     float eps, const orc_qw* gate, const orc_qw* up, const orc_qw* down,
                     uint32_t n_experts, uint32_t topk, uint32_t d_model, uint32_t n_inter,
                     uint32_t m, const uint16_t* x, uint16_t* out, uint32_t* ids_o,
                     uint16_t* gw_o, uint32_t* counts_o, uint32_t* offsets_o,
                     uint32_t* ids_sorted_o, uint32_t* slotpos_o, uint16_t* act_o,
                     uint16_t* ed_o) {
    orc_moe_prefill_masked(router, router_is_f32, bias, mode, eps, gate, up, down, n_experts,
                           topk, d_model, n_inter, m, x, NULL, out, ids_o, gw_o, counts_o,
                           offsets_o, ids_sorted_o, slotpos_o, act_o, ed_o);
}

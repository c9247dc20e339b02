/*
 * oracle_core.c -- scalar helpers, unpack/pack, dequant, the chunk-order
 * GEMV family, argmax, routing and the decode MoE step.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 0;

void orc_set_threads(int n) { g_threads = n; }

int orc_get_threads(void) {
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}

#define ORC_THREADS (orc_get_threads())

/* ------------------------------------------------------------ scalars --- */

float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return (uint16_t)((u >> 16) | 0x0040u);
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline float bfr(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

static inline float pow2f(int k) { /* 2^k for k in [-126, 127] */
    uint32_t u = (uint32_t)(k + 127) << 23;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float orc_expf(float x) {
    if (x != x) {
        return x + x;
    }
    if (x > 0x1.62e430p+6f) {
        return INFINITY;
    }
    if (x < -0x1.9fe36ap+6f) {
        return 0.0f;
    }
    const float n = rintf(x * 0x1.715476p+0f);
    float r = fmaf(-n, 0x1.62e400p-1f, x);
    r = fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0x1.000000p-1f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ni = (int)n;
    const int n1 = ni / 2;
    const int n2 = ni - n1;
    return (p * pow2f(n1)) * pow2f(n2);
}

/* -------------------------------------------------------- unpack/pack --- */

static inline uint32_t code_at(const uint32_t* row, uint32_t bits, uint32_t j) {
    const uint32_t bit = bits * j;
    const uint32_t w = bit >> 5;
    const uint32_t o = bit & 31u;
    uint32_t v = row[w] >> o;
    if (o + bits > 32u) {
        v |= row[w + 1] << (32u - o);
    }
    return v & ((1u << bits) - 1u);
}

void orc_unpack(const uint32_t* codes, uint32_t bits, size_t n_codes, uint8_t* q) {
    for (size_t j = 0; j < n_codes; ++j) {
        const size_t bit = (size_t)bits * j;
        const size_t w = bit >> 5;
        const uint32_t o = (uint32_t)(bit & 31u);
        uint32_t v = codes[w] >> o;
        if (o + bits > 32u) {
            v |= codes[w + 1] << (32u - o);
        }
        q[j] = (uint8_t)(v & ((1u << bits) - 1u));
    }
}

void orc_pack(const uint8_t* q, uint32_t bits, size_t n_codes, uint32_t* codes) {
    const size_t n_words = (n_codes * bits + 31) / 32;
    memset(codes, 0, n_words * 4);
    for (size_t j = 0; j < n_codes; ++j) {
        const size_t bit = (size_t)bits * j;
        const size_t w = bit >> 5;
        const uint32_t o = (uint32_t)(bit & 31u);
        const uint32_t v = (uint32_t)q[j] & ((1u << bits) - 1u);
        codes[w] |= v << o;
        if (o + bits > 32u) {
            codes[w + 1] |= v >> (32u - o);
        }
    }
}

/* ------------------------------------------------------------ dequant --- */

static inline size_t row_words(const orc_qw* w) { return (size_t)w->k * w->bits / 32; }

void orc_dequant_bf16(const orc_qw* w, uint16_t* out) {
    const uint32_t groups = w->k / w->gs;
#pragma omp parallel for schedule(static) num_threads(ORC_THREADS)
    for (long r = 0; r < (long)w->n; ++r) {
        const uint32_t* row = w->codes + (size_t)r * row_words(w);
        for (uint32_t j = 0; j < w->k; ++j) {
            const uint32_t g = j / w->gs;
            const float s = orc_bf16_to_f32(w->scales[(size_t)r * groups + g]);
            const float b = orc_bf16_to_f32(w->biases[(size_t)r * groups + g]);
            const float q = (float)code_at(row, w->bits, j);
            out[(size_t)r * w->k + j] = orc_f32_to_bf16(fmaf(s, q, b));
        }
    }
}

/* ----------------------------------------------------- chunk-order dot --- */

static inline float butterfly64(float* a) {
    float t[64];
    for (uint32_t m = 1; m < 64; m <<= 1) {
        for (uint32_t l = 0; l < 64; ++l) {
            t[l] = a[l] + a[l ^ m];
        }
        memcpy(a, t, sizeof(t));
    }
    return a[0];
}

/* x-sums of every 32-element chunk of xf[0..k). */
static void chunk_xsums(const float* xf, uint32_t k, float* xs) {
    for (uint32_t c = 0; c < k / 32; ++c) {
        float s = 0.0f;
        for (uint32_t i = 0; i < 32; ++i) {
            s = s + xf[32 * c + i];
        }
        xs[c] = s;
    }
}

/* Chunk-order value of quantized row r against f32 x (xs = chunk x-sums). */
static float qrow_value(const orc_qw* w, uint32_t r, const float* xf, const float* xs) {
    const uint32_t C = w->k / 32;
    const uint32_t groups = w->k / w->gs;
    const uint32_t* row = w->codes + (size_t)r * row_words(w);
    float a[64];
    for (uint32_t l = 0; l < 64; ++l) {
        a[l] = 0.0f;
    }
    for (uint32_t c = 0; c < C; ++c) {
        float p = 0.0f;
        for (uint32_t i = 0; i < 32; ++i) {
            const uint32_t kk = 32 * c + i;
            p = fmaf((float)code_at(row, w->bits, kk), xf[kk], p);
        }
        const uint32_t g = (32 * c) / w->gs;
        const float s = orc_bf16_to_f32(w->scales[(size_t)r * groups + g]);
        const float b = orc_bf16_to_f32(w->biases[(size_t)r * groups + g]);
        const float h = fmaf(s, p, b * xs[c]);
        a[c & 63u] = a[c & 63u] + h;
    }
    return butterfly64(a);
}

static float* to_f32(const uint16_t* x, size_t n) {
    float* f = (float*)malloc(n * sizeof(float));
    for (size_t i = 0; i < n; ++i) {
        f[i] = orc_bf16_to_f32(x[i]);
    }
    return f;
}

void orc_gemv_quant(const orc_qw* w, const uint16_t* x, uint32_t batch, uint16_t* y,
                    float* yf) {
    const uint32_t K = w->k, C = K / 32;
    float* xf = to_f32(x, (size_t)batch * K);
    float* xs = (float*)malloc((size_t)batch * C * sizeof(float));
    for (uint32_t b = 0; b < batch; ++b) {
        chunk_xsums(xf + (size_t)b * K, K, xs + (size_t)b * C);
    }
#pragma omp parallel for schedule(static) num_threads(ORC_THREADS)
    for (long r = 0; r < (long)w->n; ++r) {
        for (uint32_t b = 0; b < batch; ++b) {
            const float v = qrow_value(w, (uint32_t)r, xf + (size_t)b * K, xs + (size_t)b * C);
            if (y) {
                y[(size_t)b * w->n + r] = orc_f32_to_bf16(v);
            }
            if (yf) {
                yf[(size_t)b * w->n + r] = v;
            }
        }
    }
    free(xs);
    free(xf);
}

void orc_gemv_quant_rows(const orc_qw* w, const uint16_t* x, uint32_t batch,
                         const uint32_t* rows, uint32_t n_rows, uint16_t* y) {
    const uint32_t K = w->k, C = K / 32;
    float* xf = to_f32(x, (size_t)batch * K);
    float* xs = (float*)malloc((size_t)batch * C * sizeof(float));
    for (uint32_t b = 0; b < batch; ++b) {
        chunk_xsums(xf + (size_t)b * K, K, xs + (size_t)b * C);
    }
#pragma omp parallel for schedule(static) num_threads(ORC_THREADS)
    for (long i = 0; i < (long)n_rows; ++i) {
        for (uint32_t b = 0; b < batch; ++b) {
            const float v = qrow_value(w, rows[i], xf + (size_t)b * K, xs + (size_t)b * C);
            y[(size_t)b * n_rows + i] = orc_f32_to_bf16(v);
        }
    }
    free(xs);
    free(xf);
}

/* ----------------------------------------- decode GEMV epilogue variants --- */

/* lfm.metal:1023-1067 lfm_proj3_gemv_scatter_bf16: rows of q, k and v
 * against one x; q and k stored, v row j stored into the cache at
 * ((j / 64) * max_seq + pos) * 64 + j % 64. */
void orc_proj3(const orc_qw* q, const orc_qw* k, const orc_qw* v, const uint16_t* x,
               uint16_t* q_out, uint16_t* k_out, uint16_t* v_cache, uint32_t max_seq, uint32_t pos) {
    const uint32_t K = q->k, C = K / 32;
    float* xf = to_f32(x, K);
    float* xs = (float*)malloc((size_t)C * sizeof(float));
    chunk_xsums(xf, K, xs);
    const long total = (long)q->n + k->n + v->n;
#pragma omp parallel for schedule(static) num_threads(ORC_THREADS)
    for (long row = 0; row < total; ++row) {
        if (row < (long)q->n) {
            q_out[row] = orc_f32_to_bf16(qrow_value(q, (uint32_t)row, xf, xs));
        } else if (row < (long)(q->n + k->n)) {
            const uint32_t j = (uint32_t)(row - q->n);
            k_out[j] = orc_f32_to_bf16(qrow_value(k, j, xf, xs));
        } else {
            const uint32_t j = (uint32_t)(row - q->n - k->n);
            const size_t at = ((size_t)(j / 64u) * max_seq + pos) * 64u + j % 64u;
            v_cache[at] = orc_f32_to_bf16(qrow_value(v, j, xf, xs));
        }
    }
    free(xs);
    free(xf);
}

/* lfm.metal:1074-1109 lfm_conv3_gemv_split_bf16: for channel c < H the rows
 * c (B), H + c (C) and 2H + c (X) of w, each rounded to bf16; then
 * v2 = bf16(B X), z = w0 s0 + w1 s1 + w2 v2 (in that order, f32),
 * out = bf16(C bf16(z)), new_state = [s1, v2] with s0 = state[c],
 * s1 = state[H + c], taps w_j = taps[3c + j]. */
void orc_conv3(const orc_qw* w, const uint16_t* x, const uint16_t* taps, const uint16_t* state,
               uint16_t* out, uint16_t* new_state) {
    const uint32_t K = w->k, C = K / 32, H = w->n / 3;
    float* xf = to_f32(x, K);
    float* xs = (float*)malloc((size_t)C * sizeof(float));
    chunk_xsums(xf, K, xs);
#pragma omp parallel for schedule(static) num_threads(ORC_THREADS)
    for (long cl = 0; cl < (long)H; ++cl) {
        const uint32_t c = (uint32_t)cl;
        const float b = bfr(qrow_value(w, c, xf, xs));
        const float cc = bfr(qrow_value(w, H + c, xf, xs));
        const float xv = bfr(qrow_value(w, 2u * H + c, xf, xs));
        const uint16_t s1 = state[H + c];
        const float v0 = orc_bf16_to_f32(state[c]);
        const float v1 = orc_bf16_to_f32(s1);
        const float v2 = bfr(b * xv);
        const float z = orc_bf16_to_f32(taps[3u * c]) * v0 + orc_bf16_to_f32(taps[3u * c + 1u]) * v1 +
                        orc_bf16_to_f32(taps[3u * c + 2u]) * v2;
        out[c] = orc_f32_to_bf16(cc * bfr(z));
        new_state[H + c] = orc_f32_to_bf16(v2);
        new_state[c] = s1;
    }
    free(xs);
    free(xf);
}

/* lfm.metal:1284-1386 lfm_token_tail with `embed`: the key's token (the key
 * cleared), the token's row of the Q6 table dequantized as bf16(fma(s, q,
 * b)) into x, and its RMSNorm into normed: thread t of 256 sums v^2 (fma) of
 * elements t + 256 j in order, the threads' sums are added in thread order
 * (the reference's simd_sum then the 8 partials), inv = 1 / sqrt(total / K +
 * eps), normed = bf16((v * inv) * w).  K a multiple of 256; tok < rows. */
void orc_token_tail_embed(uint64_t* best, uint32_t* out_tok, const orc_qw* e, const uint16_t* w,
                          uint16_t* x, uint16_t* normed, float eps) {
    const uint32_t tok = ~(uint32_t)(*best & 0xffffffffull);
    *best = 0;
    *out_tok = tok;
    const uint32_t K = e->k, groups = K / e->gs;
    uint8_t* q = (uint8_t*)malloc(K);
    orc_unpack(e->codes + (size_t)tok * (K * e->bits / 32), e->bits, K, q);
    for (uint32_t j = 0; j < K; ++j) {
        const float sc = orc_bf16_to_f32(e->scales[(size_t)tok * groups + j / e->gs]);
        const float bi = orc_bf16_to_f32(e->biases[(size_t)tok * groups + j / e->gs]);
        x[j] = orc_f32_to_bf16(fmaf(sc, (float)q[j], bi));
    }
    float total = 0.0f;
    for (uint32_t t = 0; t < 256; ++t) {
        float acc = 0.0f;
        for (uint32_t j = 0; j < K / 256; ++j) {
            const float v = orc_bf16_to_f32(x[t + 256 * j]);
            acc = fmaf(v, v, acc);
        }
        total += acc;
    }
    const float inv = 1.0f / sqrtf(total / (float)K + eps);
    for (uint32_t j = 0; j < K; ++j) {
        normed[j] = orc_f32_to_bf16((orc_bf16_to_f32(x[j]) * inv) * orc_bf16_to_f32(w[j]));
    }
    free(q);
}

/* ------------------------------------------------------------ sampling --- */

/* log(x), x finite > 0: the device's logf_fixed step for step (m 2^k, m in
 * [sqrt(1/2), sqrt(2)), 2 atanh((m-1)/(m+1)) as an odd series to s^11, k ln2
 * split). */
float orc_logf(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    int k = (int)(u >> 23) - 127;
    if ((u >> 23) == 0u) {
        const float xs = x * 0x1p25f;
        memcpy(&u, &xs, 4);
        k = (int)(u >> 23) - 127 - 25;
    }
    const uint32_t mu = (u & 0x007fffffu) | 0x3f800000u;
    float m;
    memcpy(&m, &mu, 4);
    if (m > 1.41421356f) {
        m = m * 0.5f;
        k += 1;
    }
    const float s = (m - 1.0f) / (m + 1.0f);
    const float s2 = s * s;
    float p = 0x1.745d18p-4f;
    p = fmaf(p, s2, 0x1.c71c72p-4f);
    p = fmaf(p, s2, 0x1.24924ap-3f);
    p = fmaf(p, s2, 0x1.99999ap-3f);
    p = fmaf(p, s2, 0x1.555556p-2f);
    p = fmaf(p, s2, 1.0f);
    const float lm = (2.0f * s) * p;
    const float kf = (float)k;
    return fmaf(kf, 0x1.62e400p-1f, fmaf(kf, 0x1.7f7d1cp-20f, lm));
}

/* Philox4x32-10 (Salmon et al., SC 2011), as lfm_sample.metal:124-135. */
void orc_philox(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1, n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* lfm_sample.metal:141-155 smp_gumbel. */
float orc_gumbel(uint32_t x) {
    const float v = ((float)x + 0.5f) * 2.3283064365386963e-10f;
    float e;
    if (v < 0.015625f) {
        e = v * (1.0f + v * (0.5f + v * (0.33333334f + v * 0.25f)));
    } else {
        const float a = 1.0f - v;
        e = -orc_logf(a > 2.9802322387695312e-08f ? a : 2.9802322387695312e-08f);
    }
    return -orc_logf(e);
}

/* lfm_sample.metal:157-190 lfm_sample_gumbel over the whole row: the key of
 * argmax_i (w_i + G_i), folded with *best. */
uint64_t orc_sample_gumbel(const uint16_t* logits, uint32_t n, const uint32_t* seen, float inv_temp, float penalty,
                           float inv_penalty, int use_penalty, uint32_t seed_lo, uint32_t seed_hi, uint32_t pos,
                           uint64_t best) {
    const uint32_t key[2] = {seed_lo, seed_hi};
    for (uint32_t q = 0; q < n / 4; ++q) {
        const uint32_t ctr[4] = {q, pos, 0x53414D50u, 0u};
        uint32_t r[4];
        orc_philox(ctr, key, r);
        for (uint32_t j = 0; j < 4; ++j) {
            const uint32_t i = 4 * q + j;
            float v = orc_bf16_to_f32(logits[i]);
            if (use_penalty && ((seen[i >> 5] >> (i & 31u)) & 1u)) {
                v = v > 0.0f ? v * inv_penalty : v * penalty;
            }
            float w = v * inv_temp;
            uint32_t u;
            memcpy(&u, &w, 4);
            if ((u << 1) == 0u) {
                w = 0.0f;
            }
            const uint64_t k = orc_argmax_key(w + orc_gumbel(r[j]), i);
            best = k > best ? k : best;
        }
    }
    return best;
}

/* The kept-set draw (lfm_sample.metal:16-27 semantics; src/lfm/sample.rs:286-330).
 * Kept set {w >= tau}: top-k keeps every token whose w is at least the k-th
 * largest (ties kept); top-p keeps, among those, the smallest set {w >= t}
 * whose mass is at least top_p times the set's mass (tie groups whole).  A
 * token's mass is exp(w - M) (M the vocabulary's max w, exp the library's own)
 * in 2^-40 fixed point, truncated, so every mass sum is an exact integer and
 * the decision does not depend on any summation order.  The draw is the
 * Gumbel-max over the kept tokens, keyed as the temperature-only draw. */
static inline uint32_t smp_fkey(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    if ((u << 1) == 0u) {
        u = 0u;
    }
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static inline float smp_kfloat(uint32_t k) {
    const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    float v;
    memcpy(&v, &u, 4);
    return v;
}

/* w - m is NaN when both are the same infinity (every logit -inf, or the
 * maximum +inf): the token then has the maximum's mass exp(0); a NaN w or m
 * has none.  So the masses stay in [0, 2^40] for every input. */
uint64_t orc_mass_fixed(float w, float m) {
    float d = w - m;
    if (d != d) {
        d = w == m ? 0.0f : -INFINITY;
    }
    return (uint64_t)(orc_expf(d) * 1099511627776.0f);  /* 2^40, truncated */
}

/* The least integer T >= top_p * z (top_p in (0, 1), exact). */
uint64_t orc_mass_target(uint64_t z, float top_p) {
    uint32_t u;
    memcpy(&u, &top_p, 4);
    const uint32_t ex = (u >> 23) & 0xffu;
    const uint64_t mant = ex ? (uint64_t)((u & 0x7fffffu) | 0x800000u) : (uint64_t)(u & 0x7fffffu);
    const int s = 150 - (int)(ex ? ex : 1u);  /* top_p = mant * 2^-s */
    const unsigned __int128 prod = (unsigned __int128)mant * z;
    if (s >= 128) {
        return prod != 0 ? 1u : 0u;
    }
    uint64_t t = (uint64_t)(prod >> s);
    if ((prod & ((((unsigned __int128)1) << s) - 1)) != 0) {
        t += 1u;
    }
    return t;
}

static int cmp_desc_u32(const void* a, const void* b) {
    const uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
    return x < y ? 1 : x > y ? -1 : 0;
}

uint64_t orc_sample_draw(const uint16_t* logits, uint32_t n, const uint32_t* seen, float inv_temp, float penalty,
                         float inv_penalty, int use_penalty, uint32_t top_k, float top_p, uint32_t seed_lo,
                         uint32_t seed_hi, uint32_t pos, uint64_t best, uint32_t* tau_key_out) {
    float* w = (float*)malloc((size_t)n * sizeof(float));
    uint32_t* keys = (uint32_t*)malloc((size_t)n * sizeof(uint32_t));
    uint32_t mkey = 0u;
    for (uint32_t i = 0; i < n; ++i) {
        float v = orc_bf16_to_f32(logits[i]);
        if (use_penalty && ((seen[i >> 5] >> (i & 31u)) & 1u)) {
            v = v > 0.0f ? v * inv_penalty : v * penalty;
        }
        float x = v * inv_temp;
        uint32_t u;
        memcpy(&u, &x, 4);
        if ((u << 1) == 0u) {
            x = 0.0f;
        }
        w[i] = x;
        keys[i] = smp_fkey(x);
        mkey = keys[i] > mkey ? keys[i] : mkey;
    }
    uint32_t tau = 0u;
    const int use_k = top_k != 0u && top_k < n;
    const int use_p = top_p < 1.0f;
    if (use_k || use_p) {
        uint32_t* sorted = (uint32_t*)malloc((size_t)n * sizeof(uint32_t));
        memcpy(sorted, keys, (size_t)n * sizeof(uint32_t));
        qsort(sorted, n, sizeof(uint32_t), cmp_desc_u32);
        if (use_k) {
            tau = sorted[top_k - 1u];
        }
        if (use_p) {
            const float m = smp_kfloat(mkey);
            uint64_t z = 0u;
            for (uint32_t i = 0; i < n; ++i) {
                if (keys[i] >= tau) {
                    z += orc_mass_fixed(w[i], m);
                }
            }
            const uint64_t target = orc_mass_target(z, top_p);
            /* walk the distinct values downward; the first whose cumulative
             * mass reaches the target is tau_p */
            uint64_t cum = 0u;
            uint32_t i = 0;
            uint32_t tau_p = tau;
            while (i < n && sorted[i] >= tau) {
                const uint32_t k = sorted[i];
                while (i < n && sorted[i] == k) {
                    cum += orc_mass_fixed(smp_kfloat(k), m);
                    ++i;
                }
                if (cum >= target) {
                    tau_p = k;
                    break;
                }
            }
            tau = tau_p > tau ? tau_p : tau;
        }
        free(sorted);
    }
    const uint32_t key[2] = {seed_lo, seed_hi};
    for (uint32_t q = 0; q < n / 4; ++q) {
        const uint32_t ctr[4] = {q, pos, 0x53414D50u, 0u};
        uint32_t r[4];
        orc_philox(ctr, key, r);
        for (uint32_t j = 0; j < 4; ++j) {
            const uint32_t i = 4 * q + j;
            if (keys[i] >= tau) {
                const uint64_t k = orc_argmax_key(w[i] + orc_gumbel(r[j]), i);
                best = k > best ? k : best;
            }
        }
    }
    if (tau_key_out) {
        *tau_key_out = tau;
    }
    free(keys);
    free(w);
    return best;
}

/* ------------------------------------------------------------- argmax --- */

uint32_t orc_argmax_bf16(const uint16_t* x, size_t n) {
    float bv = -INFINITY;
    uint32_t bi = 0;
    for (size_t i = 0; i < n; ++i) {
        const float v = orc_bf16_to_f32(x[i]);
        if (v > bv || (v == bv && (uint32_t)i < bi)) {
            bv = v;
            bi = (uint32_t)i;
        }
    }
    return bi;
}

uint64_t orc_argmax_key(float v, uint32_t i) {
    uint32_t u;
    memcpy(&u, &v, 4);
    if ((u << 1) == 0u) {
        u = 0u;
    }
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (uint64_t)(~i);
}

/* --------------------------------------------------------- dense GEMV --- */

void orc_gemv_dense(const void* w, int w_is_f32, const uint16_t* x, uint32_t m,
                    uint32_t n, uint32_t k, float* y) {
    const uint32_t C = k / 32;
    float* xf = to_f32(x, (size_t)m * k);
#pragma omp parallel for collapse(2) schedule(static) num_threads(ORC_THREADS)
    for (long t = 0; t < (long)m; ++t) {
        for (long e = 0; e < (long)n; ++e) {
            const float* xr = xf + (size_t)t * k;
            float a[64];
            for (uint32_t l = 0; l < 64; ++l) {
                a[l] = 0.0f;
            }
            for (uint32_t c = 0; c < C; ++c) {
                float p = 0.0f;
                for (uint32_t i = 0; i < 32; ++i) {
                    const size_t kk = 32 * c + i;
                    const float wv = w_is_f32
                        ? ((const float*)w)[(size_t)e * k + kk]
                        : orc_bf16_to_f32(((const uint16_t*)w)[(size_t)e * k + kk]);
                    p = fmaf(wv, xr[kk], p);
                }
                a[c & 63u] = a[c & 63u] + p;
            }
            y[(size_t)t * n + e] = butterfly64(a);
        }
    }
    free(xf);
}

/* ------------------------------------------------------------ routing --- */

/* Largest drop of the sigmoid score s(z) = 1 / (1 + orc_expf(-z)) (route_one's
 * mode 0) below its running maximum, over every float z from -inf to +inf in
 * increasing order: the monotonicity defect a bound on s must allow for
 * (0 would mean non-decreasing).  Chunks in parallel, each keeping its max,
 * min and internal drop; a chunk's drop under an earlier running maximum M is
 * max(internal, M - min). */
double orc_sigmoid_max_drop(void) {
    const int64_t half = (int64_t)0x7f800001;  /* -inf .. -0, then +0 .. +inf */
    const int64_t total = 2 * half;
    enum { CH = 8192 };
    float cmax[CH], cmin[CH];
    double cdrop[CH];
#pragma omp parallel for schedule(dynamic, 16)
    for (int ch = 0; ch < CH; ++ch) {
        const int64_t lo = total * ch / CH, hi = total * (ch + 1) / CH;
        float run = -1.0f, mn = 2.0f;
        double drop = 0.0;
        for (int64_t i = lo; i < hi; ++i) {
            const uint32_t u = i < half ? (uint32_t)(0xff800000u - (uint32_t)i) : (uint32_t)(i - half);
            float z;
            memcpy(&z, &u, 4);
            const float sv = 1.0f / (1.0f + orc_expf(-z));
            if (sv < run && (double)run - sv > drop) drop = (double)run - sv;
            if (sv > run) run = sv;
            if (sv < mn) mn = sv;
        }
        cmax[ch] = run;
        cmin[ch] = mn;
        cdrop[ch] = drop;
    }
    double d = 0.0;
    float m = -1.0f;
    for (int ch = 0; ch < CH; ++ch) {
        if (cdrop[ch] > d) d = cdrop[ch];
        if ((double)m - cmin[ch] > d) d = (double)m - cmin[ch];
        if (cmax[ch] > m) m = cmax[ch];
    }
    return d;
}

static void route_one(const float* z, const float* bias, uint32_t e, uint32_t topk,
                      int mode, float eps, uint32_t* ids, uint16_t* w) {
    float s[256];
    float cand[256];
    unsigned char used[256];
    for (uint32_t i = 0; i < e; ++i) {
        if (mode == 0) {
            s[i] = 1.0f / (1.0f + orc_expf(-z[i]));
            cand[i] = s[i] + (bias ? bias[i] : 0.0f);
        } else {
            s[i] = z[i];
            cand[i] = z[i];
        }
        used[i] = 0;
    }
    uint32_t chosen[16];
    for (uint32_t r = 0; r < topk; ++r) {
        float best = -INFINITY;
        uint32_t best_e = 0;
        for (uint32_t i = 0; i < e; ++i) {
            if (used[i]) {
                continue;
            }
            const float v = cand[i];
            if (v > best || (v == best && i < best_e)) {
                best = v;
                best_e = i;
            }
        }
        chosen[r] = best_e;
        used[best_e] = 1;
    }
    if (mode == 0) {
        float denom = eps;
        for (uint32_t r = 0; r < topk; ++r) {
            denom += s[chosen[r]];
        }
        for (uint32_t r = 0; r < topk; ++r) {
            ids[r] = chosen[r];
            w[r] = orc_f32_to_bf16(s[chosen[r]] / denom);
        }
    } else {
        const float top = z[chosen[0]];
        float ev[16];
        float denom = 0.0f;
        for (uint32_t r = 0; r < topk; ++r) {
            ev[r] = orc_expf(z[chosen[r]] - top);
            denom = denom + ev[r];
        }
        for (uint32_t r = 0; r < topk; ++r) {
            ids[r] = chosen[r];
            w[r] = orc_f32_to_bf16(ev[r] / denom);
        }
    }
}

void orc_route(const float* logits, const float* bias, uint32_t m, uint32_t e,
               uint32_t topk, int mode, float eps, uint32_t* ids, uint16_t* w) {
#pragma omp parallel for schedule(static) num_threads(ORC_THREADS)
    for (long t = 0; t < (long)m; ++t) {
        route_one(logits + (size_t)t * e, bias, e, topk, mode, eps, ids + (size_t)t * topk,
                  w + (size_t)t * topk);
    }
}

/* ------------------------------------------------- decode expert GEMVs --- */

static inline float silu_bf16(float g) {
    return bfr(g / (1.0f + orc_expf(-g)));
}

void orc_gather_act(const orc_qw* gate, const orc_qw* up, uint32_t n_inter,
                    const uint16_t* x, const uint32_t* ids, uint32_t topk, uint16_t* act) {
    const uint32_t K = gate->k, C = K / 32;
    const uint32_t slots = ids ? topk : 1;
    float* xf = to_f32(x, K);
    float* xs = (float*)malloc(C * sizeof(float));
    chunk_xsums(xf, K, xs);
#pragma omp parallel for collapse(2) schedule(static) num_threads(ORC_THREADS)
    for (long r = 0; r < (long)slots; ++r) {
        for (long j = 0; j < (long)n_inter; ++j) {
            const uint32_t row = (ids ? ids[r] * n_inter : 0u) + (uint32_t)j;
            const float gv = bfr(qrow_value(gate, row, xf, xs));
            const float uv = bfr(qrow_value(up, row, xf, xs));
            act[(size_t)r * n_inter + j] = orc_f32_to_bf16(silu_bf16(gv) * uv);
        }
    }
    free(xs);
    free(xf);
}

void orc_down_combine(const orc_qw* down, uint32_t n_out, const uint16_t* act,
                      const uint32_t* ids, const uint16_t* w, uint32_t topk, uint16_t* out) {
    const uint32_t K = down->k, C = K / 32;
    float* af = to_f32(act, (size_t)topk * K);
    float* xs = (float*)malloc((size_t)topk * C * sizeof(float));
    for (uint32_t r = 0; r < topk; ++r) {
        chunk_xsums(af + (size_t)r * K, K, xs + (size_t)r * C);
    }
#pragma omp parallel for schedule(static) num_threads(ORC_THREADS)
    for (long i = 0; i < (long)n_out; ++i) {
        float total = 0.0f;
        for (uint32_t r = 0; r < topk; ++r) {
            const float p = bfr(qrow_value(down, ids[r] * n_out + (uint32_t)i,
                                           af + (size_t)r * K, xs + (size_t)r * C));
            total = total + bfr(orc_bf16_to_f32(w[r]) * p);
        }
        out[i] = orc_f32_to_bf16(total);
    }
    free(xs);
    free(af);
}

void orc_moe_decode(const void* router, int router_is_f32, const float* bias, int mode,
                    float eps, const orc_qw* gate, const orc_qw* up, const orc_qw* down,
                    uint32_t n_experts, uint32_t topk, uint32_t d_model, uint32_t n_inter,
                    const uint16_t* x, uint16_t* out, float* logits, uint32_t* ids,
                    uint16_t* w, uint16_t* act) {
    float* lg = (float*)malloc(n_experts * sizeof(float));
    uint32_t id[16];
    uint16_t wt[16];
    uint16_t* a = (uint16_t*)malloc((size_t)topk * n_inter * sizeof(uint16_t));
    orc_gemv_dense(router, router_is_f32, x, 1, n_experts, d_model, lg);
    orc_route(lg, bias, 1, n_experts, topk, mode, eps, id, wt);
    orc_gather_act(gate, up, n_inter, x, id, topk, a);
    orc_down_combine(down, d_model, a, id, wt, topk, out);
    if (logits) {
        memcpy(logits, lg, n_experts * sizeof(float));
    }
    if (ids) {
        memcpy(ids, id, topk * sizeof(uint32_t));
    }
    if (w) {
        memcpy(w, wt, topk * sizeof(uint16_t));
    }
    if (act) {
        memcpy(act, a, (size_t)topk * n_inter * sizeof(uint16_t));
    }
    free(a);
    free(lg);
}

/*
 * oracle.h -- CPU restatement of molten's quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (molten_amd/, include/)
 * includes, links or calls this code.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load it, and only as the checker / the
 * timed CPU baseline.  It is plain C99 + OpenMP, built by oracle/Makefile
 * with -ffp-contract=off so that every floating-point operation below is the
 * one written (explicit fmaf() where a fused multiply-add is meant).
 *
 * Semantics follow the reference (zhangshuibai/molten) file:line cited at
 * each function.  Where the reference leaves an order unspecified (Metal
 * simd_sum trees, fast-math contraction) this oracle fixes one canonical
 * order, the "chunk order" below, and the HIP kernels follow the same order,
 * so that outputs that feed integer decisions (argmax ids, top-k ids) are
 * bit-identical between CPU and GPU.
 *
 * Chunk order (every GEMV-family dot product of length K, K % 32 == 0):
 *   C = K / 32 chunks of 32 consecutive elements.
 *   p_c  = +0.0f; for k = 32c .. 32c+31 ascending: p_c = fmaf(q_k, x_k, p_c)
 *          (dense weights: fmaf(w_k, x_k, p_c))
 *   xs_c = +0.0f; for k ascending: xs_c = xs_c + x_k
 *   h_c  = fmaf(s_g, p_c, b_g * xs_c), g = 32c / group_size   (dense: h_c = p_c)
 *   a_l  = +0.0f; for c = l, l+64, l+128, ... < C: a_l = a_l + h_c   (l = 0..63)
 *   v    = butterfly over the 64 lane sums: for m = 1,2,4,8,16,32:
 *          a_l = a_l + a_{l^m}  (all l simultaneously); v = a_0.
 *
 * Parity status of each function is stated at its declaration; the checks
 * that pin it live in tests/test_oracle_*.py.
 */
#ifndef MOLTEN_ORACLE_H
#define MOLTEN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* MLX affine quantized matrix, molten's QuantWeights (src/weights.rs:11-30):
 * codes U32 [n, k*bits/32] (code j of a row at bit bits*j of the row's
 * little-endian byte stream), scales/biases bf16 [n, k/gs]. */
typedef struct orc_qw {
    const uint32_t* codes;
    const uint16_t* scales;
    const uint16_t* biases;
    uint32_t n, k, gs, bits;
} orc_qw;

/* ---- scalar helpers ---------------------------------------------------- */

/* bf16 -> f32 is exact; f32 -> bf16 rounds to nearest even (NaN -> quiet NaN).
 * Pinned: exhaustive over all 65536 bf16 values against numpy, and RNE ties. */
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);

/* exp(x) in f32: Cody-Waite reduction x = n*ln2 + r (ln2 split hi/lo),
 * degree-7 Taylor polynomial in Horner form with fmaf, scaling by 2^n as
 * exact power-of-two multiplies.  Used by sigmoid, SiLU and softmax so the
 * GPU can reproduce it bit for bit.  Pinned: max error vs float64 exp over a
 * dense sweep (tests/test_oracle_math.py). */
float orc_expf(float x);
/* max over floats z of (max_{t <= z} s(t)) - s(z), s(z) = 1 / (1 + orc_expf(-z)) */
double orc_sigmoid_max_drop(void);

/* ---- a2 / a3: unpack and pack (lfm.metal:102-109, :186-199;
 *      quant_nax.metal:2947-2953, :2975-2986) --------------------------------
 * q[j] = (stream >> bits*j) & (2^bits - 1).  bits in {4, 6, 8}.
 * Pinned: known-answer words (0x76543210 -> 0..7; Q6 [1,2,3,4] -> 81 30 10)
 * and pack/unpack round trips. */
void orc_unpack(const uint32_t* codes, uint32_t bits, size_t n_codes, uint8_t* q);
void orc_pack(const uint8_t* q, uint32_t bits, size_t n_codes, uint32_t* codes);

/* ---- dequant_to_bf16 / dequant_q4_bf16_bulk (src/kernels/quant.rs:69, :95;
 *      quant.metal:45-114; MLX dequantize quant_nax.metal:2908-2993) --------
 * out[r, j] = bf16(fmaf(s, q, b)).  Pinned: closed form vs numpy float64
 * (one rounding of s*q+b) and the all-zero / s=0 special cases. */
void orc_dequant_bf16(const orc_qw* w, uint16_t* out);

/* ---- a4 / a5: affine quantized GEMV (lfm.metal:100-297, GEMV_Q4_BODY,
 *      lfm_gemv_q6_bf16_x4; src/kernels/lfm.rs:112-149) ---------------------
 * y[b, r] = bf16(v) with v the chunk-order value of row r against x[b, :].
 * batch rows are independent.  yf (nullable) receives v before rounding.
 * Pinned: numpy float64 of the dequantized matrix (tolerance), closed forms
 * (all codes 0, s = 0, one-hot x, x = 1), and a pure-Python replay of the
 * chunk order on tiny shapes (bit-exact). */
void orc_gemv_quant(const orc_qw* w, const uint16_t* x, uint32_t batch,
                    uint16_t* y, float* yf);
/* Only the listed rows (for sampled checks at full size): y[b * n_rows + i]. */
void orc_gemv_quant_rows(const orc_qw* w, const uint16_t* x, uint32_t batch,
                         const uint32_t* rows, uint32_t n_rows, uint16_t* y);

/* ---- next rows: decode GEMV epilogue variants on the same row values ---
 * proj3 (lfm.metal:1023-1067; src/kernels/lfm.rs:155-218): q_out, k_out =
 * bf16 rows of q, k; v row j into v_cache[((j / 64) * max_seq + pos) * 64 +
 * j % 64].  Pinned: equal to orc_gemv_quant of each matrix with the cache
 * index computed independently in the test.
 * conv3 (lfm.metal:1074-1109; src/kernels/lfm.rs:220-256): w has 3H rows;
 * per channel c: B, C, X = bf16 rows c, H + c, 2H + c; v2 = bf16(B X);
 * z = w0 state[c] + w1 state[H + c] + w2 v2; out[c] = bf16(C bf16(z));
 * new_state = [state[H + c], v2].  Pinned: one-hot tap cases that reduce to
 * the inputs (w = e0: out = bf16(C s0); w = e2: out = bf16(C v2)), the state
 * shift, and B X against the GEMV rows. */
void orc_proj3(const orc_qw* q, const orc_qw* k, const orc_qw* v, const uint16_t* x,
               uint16_t* q_out, uint16_t* k_out, uint16_t* v_cache, uint32_t max_seq, uint32_t pos);
void orc_conv3(const orc_qw* w, const uint16_t* x, const uint16_t* taps, const uint16_t* state,
               uint16_t* out, uint16_t* new_state);

/* ---- next row: token tail + Q6 embedding (lfm.metal:430-462, :1284-1386;
 * src/kernels/lfm.rs:337-363, :850-888) --------------------------------------
 * token = ~low32(key), key cleared; x = the token's table row dequantized
 * (bf16(fma(s, q, b)), = orc_dequant_bf16's row); normed = bf16((x * inv) *
 * w), inv = 1 / sqrt(sum x^2 / K + eps) summed in the reference's thread
 * order.  The embedding gather is orc_dequant_bf16's rows.  Pinned: the row
 * against orc_dequant_bf16, normed against float64 RMSNorm (tolerance) and a
 * constant row's closed form. */
void orc_token_tail_embed(uint64_t* best, uint32_t* out_tok, const orc_qw* e, const uint16_t* w,
                          uint16_t* x, uint16_t* normed, float eps);

/* ---- next row: the temperature-only Gumbel draw (lfm_sample.metal:124-190;
 * src/lfm/sample.rs:264-285) ---------------------------------------------------
 * orc_philox: Philox4x32-10.  Pinned: Random123's published known-answer
 * vectors.  orc_logf: the device's own log.  Pinned: <= 2 ulp vs float64 over
 * a dense sweep, exact powers of two.  orc_gumbel: -log(-log(1 - V)).  Pinned:
 * vs float64 within tolerance on both branches.  orc_sample_gumbel: the draw's
 * key.  Pinned: the empirical token frequencies over many positions match
 * softmax(w) (chi-square), the penalty and temperature closed forms.  Parity
 * with the reference's own bits is unpinned where Metal's log decides them. */
float orc_logf(float x);
void orc_philox(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
float orc_gumbel(uint32_t x);
uint64_t orc_sample_gumbel(const uint16_t* logits, uint32_t n, const uint32_t* seen, float inv_temp, float penalty,
                           float inv_penalty, int use_penalty, uint32_t seed_lo, uint32_t seed_hi, uint32_t pos,
                           uint64_t best);

/* ---- next row: the kept-set draw (top-k / top-p; lfm_sample.metal:16-27,
 * 196-931; src/lfm/sample.rs:286-353) -------------------------------------
 * orc_mass_fixed: exp(w - m) in 2^-40 fixed point, truncated.  orc_mass_target:
 * the least integer >= top_p * z, exact (128-bit).  Pinned: closed forms and
 * float64 over random and edge values.  orc_sample_draw: w as the temperature
 * draw; tau = the k-th largest w (top-k, ties kept), then the largest value t
 * among the kept with mass(w >= t) >= target(mass of the kept, top_p) (top-p,
 * tie groups whole); the Gumbel-max over {w >= tau}; *tau_key_out = tau's
 * orderable key (0: every token).  Pinned: the kept set equals numpy's
 * (partition for top-k, float64 cumulative softmax for top-p on logits with
 * clear gaps), k = 1 and a tiny top_p reduce to greedy, top_k >= n and
 * top_p = 1 to the temperature draw, and the draws' frequencies over many
 * positions match softmax renormalized over the kept set (chi-square). */
uint64_t orc_mass_fixed(float w, float m);
uint64_t orc_mass_target(uint64_t z, float top_p);
uint64_t orc_sample_draw(const uint16_t* logits, uint32_t n, const uint32_t* seen, float inv_temp, float penalty,
                         float inv_penalty, int use_penalty, uint32_t top_k, float top_p, uint32_t seed_lo,
                         uint32_t seed_hi, uint32_t pos, uint64_t best, uint32_t* tau_key_out);

/* ---- a6: argmax over bf16 logits (lfm.metal:1113-1282) ------------------
 * value desc, index asc; -0 == +0; NaN never taken; none -> 0.  Pinned by
 * known-answer ties and numpy argmax on tie-free rows. */
uint32_t orc_argmax_bf16(const uint16_t* x, size_t n);
/* Orderable 64-bit key (lfm.metal:1119-1124): larger key = larger value, or
 * equal value at a lower index. */
uint64_t orc_argmax_key(float v, uint32_t i);

/* ---- a7 / a12: dense router GEMV (src/kernels/lfm.rs:314-335, :366-388;
 *      lfm.metal:368-428, :470-537) ----------------------------------------
 * y[t, e] = chunk-order dot of W[e, :] and x[t, :] (h_c = p_c), f32 out.
 * w_is_f32: 1 -> W is f32 [n, k] (the reference's router), 0 -> bf16 [n, k]
 * (BASELINE's router).  Pinned: numpy float64 (tolerance) and Python replay
 * (bit-exact) on tiny shapes. */
void orc_gemv_dense(const void* w, int w_is_f32, const uint16_t* x,
                    uint32_t m, uint32_t n, uint32_t k, float* y);

/* ---- a8 / a12: top-k routing (lfm.metal:541-703, :1558-1602) ------------
 * mode 0 (reference): s = 1/(1+exp(-z)); rank on s + bias[e]; weights
 *        bf16(s_r / (eps + sum_r s_r)), sum in rank order from eps.
 * mode 1 (BASELINE): rank on the logits z; weights
 *        bf16(e_r / (e_0 + ... + e_{k-1})), e_r = exp(z_r - z_top1).
 * Ties go to the lower expert id.  bias may be NULL (treated as 0).
 * Pinned: constructed ties, numpy ranking, softmax/sigmoid closed forms. */
void orc_route(const float* logits, const float* bias, uint32_t m, uint32_t e,
               uint32_t topk, int mode, float eps, uint32_t* ids, uint16_t* w);

/* ---- a9 / a11: gate/up GEMV + SwiGLU (lfm.metal:1392-1498) ---------------
 * act[r, j] = bf16( bf16(silu(g)) * u ), g = f32(bf16(gate row)),
 * u = f32(bf16(up row)), silu(g) = g / (1 + exp(-g)).
 * Rows of expert ids[r] are ids[r]*n_inter + j of the stacked matrices.
 * ids == NULL: dense (one slot, rows j).  Pinned: composition of pinned
 * parts (GEMV, expf, bf16) plus a float64 end-to-end check. */
void orc_gather_act(const orc_qw* gate, const orc_qw* up, uint32_t n_inter,
                    const uint16_t* x, const uint32_t* ids, uint32_t topk,
                    uint16_t* act);

/* ---- a10: down GEMV + weighted combine (lfm.metal:1503-1554) --------------
 * p_r = bf16(down row ids[r]*n_out + i against act[r]);
 * out[i] = bf16( sum_r f32(bf16(w_r * p_r)) ), r ascending from +0.0f. */
void orc_down_combine(const orc_qw* down, uint32_t n_out, const uint16_t* act,
                      const uint32_t* ids, const uint16_t* w, uint32_t topk,
                      uint16_t* out);

/* ---- a19 decode: whole MoE decode step (src/lfm.rs:967-1011) ------------
 * router -> route -> gather_act -> down_combine.  logits/ids/w/act are
 * outputs too (any may be NULL). */
void orc_moe_decode(const void* router, int router_is_f32, const float* bias,
                    int mode, float eps, const orc_qw* gate, const orc_qw* up,
                    const orc_qw* down, uint32_t n_experts, uint32_t topk,
                    uint32_t d_model, uint32_t n_inter, const uint16_t* x,
                    uint16_t* out, float* logits, uint32_t* ids, uint16_t* w,
                    uint16_t* act);

/* ---- a13: counting sort (lfm.metal:1604-1685) ----------------------------
 * counts[e] = #slots routed to e; offsets = exclusive scan; stable scatter in
 * token-major, rank-major order: ids_sorted[pos] = t, slotpos[t*topk+r] = pos.
 * Pinned: numpy bincount / cumsum / argsort(kind="stable"). */
void orc_moe_count(const uint32_t* ids, uint32_t s, uint32_t e, uint32_t* counts);
void orc_moe_offsets(const uint32_t* counts, uint32_t e, uint32_t* offsets);
void orc_moe_sorted(const uint32_t* ids, const uint32_t* offsets, uint32_t m,
                    uint32_t e, uint32_t topk, uint32_t* ids_sorted,
                    uint32_t* slotpos);

/* ---- a14: block maps (lfm.metal:1687-1770; src/lfm.rs:896-933) ------------
 * Entry i of expert e: uint4(m0, e*N + n0, n0, m_end), row tiles of bm,
 * column tiles of gu_bn / dn_bn (the reference uses one bn for both), expert
 * order; the tail up to max_* is zero.
 * Pinned: brute-force enumeration from the definition in Python. */
void orc_moe_block_offsets(const uint32_t* counts, uint32_t e, uint32_t bm,
                           uint32_t gu_bn, uint32_t dn_bn, uint32_t gu_n, uint32_t dn_n,
                           uint32_t* gu_off, uint32_t* dn_off);
void orc_moe_blocks(const uint32_t* counts, const uint32_t* offsets,
                    const uint32_t* gu_off, const uint32_t* dn_off, uint32_t e,
                    uint32_t bm, uint32_t gu_bn, uint32_t dn_bn, uint32_t gu_n, uint32_t dn_n,
                    uint32_t* gu, uint32_t max_gu, uint32_t* dn, uint32_t max_dn);

/* ---- a15 / a17 / a18: gather, SwiGLU, combine (elementwise.metal:7-52;
 *      lfm.metal:859-940) ---------------------------------------------------- */
void orc_gather_rows_bf16(const uint16_t* table, const uint32_t* ids, uint32_t m,
                          uint32_t h, uint16_t* out);
void orc_silu_mul_bf16(const uint16_t* gate, const uint16_t* up, size_t n,
                       uint16_t* out);
void orc_moe_combine_rows(const uint16_t* sorted, const uint32_t* slotpos,
                          const uint16_t* w, uint32_t m, uint32_t h,
                          uint32_t topk, uint16_t* out);

/* ---- a16: block-mapped grouped Q4 GEMM (src/kernels/quant.rs:151-266;
 *      quant_nax.metal:4091-4234, :4392-4699) ------------------------------
 * For every entry (m0, e*N + n0, n0, m_end) of blocks[0..n_blocks):
 *   C[m, n0 + j] = bf16( sum_k f32(A[m, k]) * f32(bf16(fmaf(s, q, b))) ),
 *   m in [m0, m_end), j in [0, bn), f32 accumulation in ascending k.
 * Pinned: reduction to per-expert dense GEMMs checked with numpy float64. */
void orc_gemm_q4_grouped(const uint16_t* a, const orc_qw* w, uint16_t* c,
                         const uint32_t* blocks, uint32_t n_blocks, uint32_t n,
                         uint32_t bn);

/* Whole prefill MoE for m tokens (src/lfm.rs:847-965): router_prefill ->
 * route -> counting sort -> gather -> grouped gate/up -> SwiGLU -> grouped
 * down -> combine.  The grouped GEMMs are computed per sorted row directly
 * (the block map only partitions the same sums).  Intermediates are outputs
 * when non-NULL. */
void orc_moe_prefill(const void* router, int router_is_f32, const float* bias,
                     int mode, float eps, const orc_qw* gate, const orc_qw* up,
                     const orc_qw* down, uint32_t n_experts, uint32_t topk,
                     uint32_t d_model, uint32_t n_inter, uint32_t m,
                     const uint16_t* x, uint16_t* out, uint32_t* ids,
                     uint16_t* gw, uint32_t* counts, uint32_t* offsets,
                     uint32_t* ids_sorted, uint32_t* slotpos, uint16_t* act,
                     uint16_t* ed);

/* The same with the expert GEMMs computed only for tokens whose mask byte is
 * non-zero (routing and sort still cover all m tokens); rows of masked-out
 * tokens in act / ed / out are zero.  Used to check full-size prefill runs on
 * a token sample. */
void orc_moe_prefill_masked(const void* router, int router_is_f32, const float* bias, int mode,
                            float eps, const orc_qw* gate, const orc_qw* up, const orc_qw* down,
                            uint32_t n_experts, uint32_t topk, uint32_t d_model, uint32_t n_inter,
                            uint32_t m, const uint16_t* x, const uint8_t* token_mask,
                            uint16_t* out, uint32_t* ids_o, uint16_t* gw_o, uint32_t* counts_o,
                            uint32_t* offsets_o, uint32_t* ids_sorted_o, uint32_t* slotpos_o,
                            uint16_t* act_o, uint16_t* ed_o);

/* OpenMP thread count used by the heavy loops (0 = library default). */
void orc_set_threads(int n);
int orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif

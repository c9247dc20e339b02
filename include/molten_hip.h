/*
 * molten_hip.h -- C ABI of the MI355X (gfx950) quantized-matmul hot path of
 * molten (zhangshuibai/molten).
 *
 * This header is the drop-in boundary.  Each launcher replaces one operator
 * wrapper of the reference's Rust/Metal operator layer; the replaced wrapper
 * is cited as file:line under /root/reference.  The Rust side binds these
 * with a thin `src/hip.rs` of extern "C" declarations and keeps the operator
 * signatures of the src/kernels/ modules.
 *
 * Conventions
 *   - All tensors are device pointers (hipMalloc'd or views into one).
 *     bf16 tensors are uint16_t bit patterns; ids/counts are uint32_t.
 *   - Operators borrow their arguments and never allocate device memory.
 *     Scratch words (argmax keys, counters) are caller-owned, must be zero on
 *     entry and are left zero on exit where stated (the reference contract,
 *     src/kernels/lfm.rs:259-263, :822-825).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the default stream)
 *     in call order.  Launchers do not synchronize.
 *   - Return value: 0 = OK; < 0 = argument rejected before anything was
 *     launched (message in mh_last_error()); > 0 = hipError_t at launch.
 *
 * Quantized weights use molten's MLX affine layout (src/weights.rs:11-30):
 * codes U32 [out, in*bits/32], code j of a row at bit bits*j of the row's
 * little-endian byte stream (Q4: 8 codes per word, low nibble first; Q6: 4
 * codes per 3 bytes); scales and biases bf16 [out, in/group_size];
 * w = scale*q + bias.  Stacked experts are one matrix of E*rows rows.
 */
#ifndef MOLTEN_HIP_H
#define MOLTEN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ status --- */

enum {
    MH_OK = 0,
    MH_ERR_INVALID = -1,     /* bad shape, null pointer or out-of-range value */
    MH_ERR_ALIGN = -2,       /* pointer or stride misaligned for the kernel   */
    MH_ERR_UNSUPPORTED = -3, /* valid request this build has no kernel for   */
    MH_ERR_RUNTIME = -4      /* runtime query failed before launch           */
};

/* Message of the last failure on the calling thread ("" if none). */
const char* mh_last_error(void);

/* Library version, e.g. "molten-hip 0.1.0 gfx950". */
const char* mh_version(void);

/* Routing rule of the top-k (lfm.metal:541-703): MH_ROUTE_SIGMOID_BIAS is
 * molten's (rank on sigmoid(z) + bias, weights s_r / (eps + sum s));
 * MH_ROUTE_SOFTMAX ranks on the logits and renormalises the softmax over the
 * chosen experts.  Ties go to the lower expert id in both. */
enum { MH_ROUTE_SIGMOID_BIAS = 0, MH_ROUTE_SOFTMAX = 1 };

/* Element type of a dense router matrix. */
enum { MH_DTYPE_F32 = 0, MH_DTYPE_BF16 = 1, MH_DTYPE_U32 = 2, MH_DTYPE_OTHER = 3 };

typedef void* mh_stream_t; /* hipStream_t */
typedef void* mh_event_t;  /* hipEvent_t  */

/* MLX affine quantized matrix: molten's QuantWeights (src/weights.rs:11-30). */
typedef struct mh_quant_weights {
    const uint32_t* codes;  /* U32  [out_features, in_features*bits/32] */
    const uint16_t* scales; /* bf16 [out_features, in_features/group_size] */
    const uint16_t* biases; /* bf16 [out_features, in_features/group_size] */
    uint32_t out_features;
    uint32_t in_features;
    uint32_t group_size;
    uint32_t bits;
} mh_quant_weights;

/* ------------------------------------------------- device runtime ---
 * Replaces MetalContext / ComputePass / Tensor host access
 * (src/metal.rs:92-416, src/tensor.rs:100-192).  A "pass" is a stream:
 * dispatches run serially in call order; commit = mh_event_record,
 * PendingPass::wait = mh_event_synchronize. */
int mh_device_count(int* count);
int mh_set_device(int device);
int mh_stream_create(mh_stream_t* stream);
int mh_stream_destroy(mh_stream_t stream);
int mh_stream_synchronize(mh_stream_t stream);
int mh_event_create(mh_event_t* event);
int mh_event_destroy(mh_event_t event);
int mh_event_record(mh_event_t event, mh_stream_t stream);
int mh_event_synchronize(mh_event_t event);
int mh_malloc(void** ptr, size_t bytes);
int mh_free(void* ptr);
/* kind: 1 host->device, 2 device->host, 3 device->device.  Ordered on
 * `stream`; returns after the copy completed. */
int mh_memcpy(void* dst, const void* src, size_t bytes, int kind, mh_stream_t stream);
/* Stream-ordered zero fill with a kernel (no hipMemsetAsync, so it is safe
 * inside graph capture). */
int mh_zero(void* dst, size_t bytes, mh_stream_t stream);

/* Device status word: kernels that wait on other workgroups bound every
 * wait, and when one expires they finish with a defined result (token id
 * 0xffffffff, NaN outputs) and set a bit here.  mh_status waits for `stream`,
 * reads the current device's word into *status and, when `clear` != 0,
 * resets it; the counterpart of the reference surfacing a failed command
 * buffer at commit_wait (src/metal.rs:385-399).  Not for graph capture. */
#define MH_STATUS_ARGMAX_WAIT 1u /* a head GEMV's argmax collector gave up  */
#define MH_STATUS_DECODE_WAIT 2u /* the fused MoE decode step's exchange wait expired */
int mh_status(uint32_t* status, int clear, mh_stream_t stream);

/* ------------------------------------------------------ checkpoint ---
 * src/safetensors.rs:85-196 Checkpoint and src/lfm.rs:261-316 load_tensor /
 * load_quant: the MLX safetensors checkpoint, unchanged.  open() reads the
 * shard headers (model.safetensors.index.json's shards, else
 * model.safetensors); tensors are listed by name (sorted); read() streams a
 * tensor into device memory through two pinned staging buffers (file reads
 * overlap the copies) and returns once it is there; load_quant() checks and
 * reads base.weight (U32 codes), base.scales and base.biases (BF16), infers
 * bits = 32 * cols / K (must equal `bits`) and fills `out` with the device
 * pointers.  Errors: MH_ERR_INVALID with the reference's messages.  Names
 * stay valid until close(); reads on one checkpoint share its staging buffers,
 * so concurrent calls on one checkpoint from several threads race. */
#define MH_MAX_DIMS 8
typedef struct mh_checkpoint mh_checkpoint;
typedef struct {
    int dtype; /* MH_DTYPE_F32 / BF16 / U32, or MH_DTYPE_OTHER */
    uint32_t ndim;
    uint64_t shape[MH_MAX_DIMS];
    uint64_t bytes;
} mh_tensor_meta;
int mh_checkpoint_open(const char* dir, mh_checkpoint** out);
void mh_checkpoint_close(mh_checkpoint* ck);
uint32_t mh_checkpoint_count(const mh_checkpoint* ck);
const char* mh_checkpoint_name(const mh_checkpoint* ck, uint32_t i);
int mh_checkpoint_meta(const mh_checkpoint* ck, const char* name, mh_tensor_meta* meta);
int mh_checkpoint_read(mh_checkpoint* ck, const char* name, void* dst, size_t bytes, mh_stream_t stream);
int mh_load_quant(mh_checkpoint* ck, const char* base, uint32_t rows, uint32_t k, uint32_t bits,
                  uint32_t* codes, uint16_t* scales, uint16_t* biases, mh_quant_weights* out,
                  mh_stream_t stream);

/* ------------------------------------------------------ dequantize ---
 * src/kernels/quant.rs:69 dequant_to_bf16 and :95 dequant_q4_bf16_bulk:
 * out[r, j] = bf16(fma(scale, q, bias)), out bf16 [out, in] (16-byte
 * aligned).  dequant_to_bf16 takes 4-, 6- and 8-bit weights (the reference's
 * check_quant, quant.rs:42-66, takes 4 and 8: dequant_q4_bf16 /
 * dequant_q8_bf16, quant.metal:10-67); the bulk form 4-bit with K % 128 == 0. */
int mh_dequant_to_bf16(const mh_quant_weights* w, uint16_t* out, mh_stream_t stream);
int mh_dequant_q4_bf16_bulk(const mh_quant_weights* w, uint16_t* out, mh_stream_t stream);

/* --------------------------------------------------- decode GEMVs ---
 * src/kernels/lfm.rs:112 gemv_quant: y[b, :] = bf16(W x[b, :]), f32
 * accumulation in the chunk order, bits 4 or 6.  `batch` rows of x
 * (1..8; the reference has batch 1).  x bf16 [batch, in], y bf16
 * [batch, out].  Batch 2..8 with group size 64, in <= 2048 (a multiple of
 * 512), out a multiple of 16 and x 16-byte aligned runs on the matrix cores:
 * f32 sums in the MFMA's order, logits within one bf16 ulp (plus f32
 * rounding) of the chunk order instead of bit-equal. */
int mh_gemv_quant(const mh_quant_weights* w, const uint16_t* x, uint16_t* y, uint32_t batch,
                  mh_stream_t stream);

/* src/kernels/lfm.rs:826 gemv_head_argmax: the head GEMV with an argmax
 * epilogue; logits are not stored.  best[b] (u64, zero on entry) receives
 * the orderable key of row b's argmax (value desc, index asc over the
 * bf16-rounded logits); mh_token_tail reads and clears it. */
int mh_gemv_head_argmax(const mh_quant_weights* w, const uint16_t* x, uint64_t* best,
                        uint32_t batch, mh_stream_t stream);

/* Head GEMV that stores the bf16 logits (y, may be NULL) and writes
 * ids[b] = argmax token of row b in the same launch; the ids are the
 * chunk-order argmax on every path (on the matrix-core path, candidates
 * within a rigorous error bound are recomputed in chunk order).  Every
 * workgroup but the last publishes its key(s) for each batch row into its
 * own scratch slots;
 * the last-dispatched workgroup (every other one has started by then) collects
 * the slots, writes the token ids and re-zeroes the slots, so no two
 * workgroups contend on one atomic.  scratch: MH_ARGMAX_SCRATCH_WORDS(batch)
 * u64 words, zeroed before the first call; the slots are left zero and the
 * last word counts the finisher's launches in bits 0..62 (every published
 * key carries a tag of the count, so a key an earlier launch's workgroup
 * wrote before that launch's collector gave up is never taken for a later
 * launch's); calls that overlap on one scratch buffer race.  When the
 * collector's bounded wait expires the ids are 0xffffffff and
 * MH_STATUS_ARGMAX_WAIT is set; the collector then also sets bit 63 of the
 * count word, because a workgroup that started only after it gave up
 * publishes under the next launch's tag: the next launch reports the same
 * way (ids 0xffffffff, the status bit), re-zeroes the slots and clears the
 * bit, and the launch after it is exact again.  No reference counterpart
 * (BASELINE configs 2 and 5 store the logits; molten's head stores none). */
#define MH_ARGMAX_SLOTS 2048u
#define MH_ARGMAX_SCRATCH_WORDS(batch) (MH_ARGMAX_SLOTS * (batch) + 1u)
int mh_gemv_quant_argmax(const mh_quant_weights* w, const uint16_t* x, uint16_t* y,
                         uint64_t* scratch, uint32_t* ids, uint32_t batch, mh_stream_t stream);

/* Measurement only (no reference counterpart): mh_gemv_quant_argmax with
 * phase timestamps for the measured head shapes; otherwise
 * MH_ERR_UNSUPPORTED.  `stamps` holds MH_GEMV_STAMP_WAVES x MH_GEMV_STAMPS u64
 * words; lane 0 of each of the launch's waves w writes its words at w *
 * MH_GEMV_STAMPS, word 7 the XCD its workgroup ran on, the others the 100
 * MHz constant clock:
 *   batch 1 (the chunk-order kernel; K 2048, group 64, N a multiple of 8 from
 *   16 x 8 rows per CU up to 65536 rows: 32768..65536 on a 256-CU part; 4
 *   waves per workgroup, one 8-row block per wave): wave start, block loads
 *   issued, x shared, row values stored, workgroup keys merged, workgroup key
 *   published (wave 0 of every workgroup but the collector), slots collected
 *   and ids written (the collector's waves);
 *   batch 8 (the matrix-core kernel: 256 workgroups of 8 waves): wave start,
 *   x staged, main loop done, batch row b's summary published (waves b < 8),
 *   then in the finisher (the last workgroup) wave b: every workgroup's words
 *   read, row b's id written, and in word 6 not a time but the number of
 *   rows whose chunk-order values it formed for row b (0: one candidate).
 * Outputs are mh_gemv_quant_argmax's. */
#define MH_GEMV_STAMP_WAVES 8192u
#define MH_GEMV_STAMPS 8u
int mh_gemv_quant_argmax_stamped(const mh_quant_weights* w, const uint16_t* x, uint16_t* y, uint64_t* scratch,
                                 uint32_t* ids, uint32_t batch, uint64_t* stamps, mh_stream_t stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): mh_gemv_quant_argmax with its finisher scratch held by
 * the library in a file-scope device array of MH_ARGMAX_SCRATCH_WORDS(8) u64
 * words (128 KiB + 8 B on each device it runs on, held until the process
 * ends), resolved and zeroed on the first call on each device.  batch must
 * be 1..8 (the array's size; larger is MH_ERR_INVALID).  The caller passes
 * the weights, x, y (may be NULL) and ids as for mh_gemv_quant_argmax;
 * nothing is allocated.  Every call on a device shares that device's array
 * and keeps it in the state the kernels leave (slots zero, a launch count):
 * calls that overlap on one device race, so issue them on one stream. */
int mh_gemv_quant_argmax_noalloc(const mh_quant_weights* w, const uint16_t* x, uint16_t* y, uint32_t* ids,
                                 uint32_t batch, mh_stream_t stream);

/* src/kernels/lfm.rs:155-218 proj3_gemv_scatter (lfm.metal:1023-1067): the
 * Q, K and V projections of one x in one launch; q_out[NQ], k_out[NK] bf16,
 * V row j written to v_cache[((j / 64) * max_seq + pos) * 64 + j % 64]
 * (v_cache bf16 [NV / 64, max_seq, 64]).  Rows are mh_gemv_quant's values.
 * Q4, group 64, in_features a multiple of 128 up to 2048 (the reference:
 * exactly its hidden size 2048), NV a multiple of 64, pos < max_seq. */
int mh_proj3_gemv_scatter(const mh_quant_weights* q, const mh_quant_weights* k,
                          const mh_quant_weights* v, const uint16_t* x, uint16_t* q_out,
                          uint16_t* k_out, uint16_t* v_cache, uint32_t max_seq, uint32_t pos,
                          mh_stream_t stream);

/* src/kernels/lfm.rs:220-256 conv3_gemv (lfm.metal:1074-1109): the decode
 * short-conv input projection and the conv.  wproj has 3H rows (B, C, X
 * blocks of H); taps bf16 [H, 3]; state, new_state bf16 [2, H]; out bf16 [H].
 * Per channel c: B, C, X = bf16 rows c, H + c, 2H + c; v2 = bf16(B X);
 * z = t0 state[c] + t1 state[H + c] + t2 v2; out[c] = bf16(C bf16(z));
 * new_state[c] = state[H + c], new_state[H + c] = v2.  Same shape limits as
 * mh_proj3_gemv_scatter. */
int mh_conv3_gemv(const mh_quant_weights* wproj, const uint16_t* x, const uint16_t* taps,
                  const uint16_t* state, uint16_t* out, uint16_t* new_state, mh_stream_t stream);

/* src/kernels/lfm.rs:850 token_tail without `next`: out_tok[b] = token of
 * key best[b]; best[b] is cleared. */
int mh_token_tail(uint64_t* best, uint32_t* out_tok, uint32_t batch, mh_stream_t stream);

/* src/kernels/lfm.rs:850-888 token_tail with `next` (lfm.metal:1284-1386):
 * out_tok[0] = token of key best[0] (cleared); then the token's row of the Q6
 * embedding table e (6-bit, group 64, width K <= 2048, a multiple of 64) is
 * dequantized into x [K] (bf16(fma(s, q, b))) and RMSNorm'd into normed [K]:
 * bf16((x * inv) * w), inv = 1 / sqrt(sum x^2 / K + eps).  w, x, normed
 * 16-byte aligned.  A token outside the table (an empty key) writes no rows. */
int mh_token_tail_embed(uint64_t* best, uint32_t* out_tok, const mh_quant_weights* e,
                        const uint16_t* w, uint16_t* x, uint16_t* normed, float eps,
                        mh_stream_t stream);

/* src/kernels/lfm.rs:337-363 gather_rows_q6 (lfm.metal:430-462): out[t, :] =
 * dequantized row ids[t] of the Q6 table w (6-bit, group 64), t < m.  out
 * 16-byte aligned; an id outside the table leaves its row unwritten. */
int mh_gather_rows_q6(const mh_quant_weights* w, const uint32_t* ids, uint32_t m, uint16_t* out,
                      mh_stream_t stream);

/* src/lfm/sample.rs:264-285 encode_draw without top-k / top-p
 * (lfm_sample.metal:157-190 lfm_sample_gumbel): the temperature draw from the
 * bf16 logits row [n] folded into the greedy key word *best (zero or an
 * earlier key; mh_token_tail reads and clears it): token = argmax_i w_i + G_i,
 * w_i = v_i / p (v_i > 0) or v_i p (v_i <= 0) for seen tokens (bit i of seen
 * [n / 32] words; only read when use_penalty), then times inv_temp, -0 folded
 * to +0; G_i = -log(-log(1 - V)), V = (x_i + 0.5) 2^-32, x_i word i % 4 of
 * Philox4x32-10(counter (i / 4, pos, 0x53414D50, 0), key (seed_lo, seed_hi));
 * ties to the lower id.  The layout is the reference's SmpParams head.
 * top_k != 0 or top_p < 1 (the kept-set path) -> MH_ERR_UNSUPPORTED. */
typedef struct {
    float inv_temp;
    float penalty;
    float inv_penalty;
    uint32_t use_penalty;
    uint32_t top_k;
    float top_p;
    uint32_t seed_lo, seed_hi;
    uint32_t pos;
    uint32_t pad0;
} mh_sample_params;
int mh_sample_gumbel(const uint16_t* logits, uint32_t n, const uint32_t* seen,
                     const mh_sample_params* params, uint64_t* best, mh_stream_t stream);

/* src/lfm/sample.rs:264-330 encode_draw, every case (lfm_sample.metal
 * lfm_sample_prep / _levels / _gather / _finish): the draw over the kept set
 * {w >= tau}: top_k (0 = off; k >= n keeps every token) keeps the tokens
 * whose w is at least the k-th largest (ties kept); top_p (< 1) then keeps,
 * among those, the smallest set {w >= t} whose mass is at least top_p times
 * the kept mass (tie groups whole); mass = exp(w - max w) in 2^-40 fixed
 * point, so the decision is exact and independent of any summation order.
 * The Gumbel-max over the kept tokens is folded into `best` as by
 * mh_sample_gumbel (which this calls when neither is on).  workspace:
 * mh_sample_workspace_bytes(n) bytes, 256-byte aligned, zeroed before the
 * first call; every call leaves the part that must start at zero (its first
 * MH_SAMPLE_ZERO_BYTES bytes) zero again and rewrites the rest.  Calls
 * sharing one workspace must not overlap.  top_p must be in (0, 1]; n at
 * most 2^31. */
#define MH_SAMPLE_ZERO_BYTES 16640u
size_t mh_sample_workspace_bytes(uint32_t n);
int mh_sample_draw(const uint16_t* logits, uint32_t n, const uint32_t* seen, const mh_sample_params* params,
                   uint64_t* best, void* workspace, size_t workspace_bytes, mh_stream_t stream);

/* src/lfm/sample.rs:332-353 encode_mark (lfm_sample.metal lfm_sample_mark):
 * adds the drawn token *tok (ignored when >= n) to the seen-token bitmap. */
int mh_sample_mark(const uint32_t* tok, uint32_t* seen, uint32_t n, mh_stream_t stream);

/* src/kernels/lfm.rs:794 argmax_bf16: two-stage argmax of a bf16 row,
 * ties to the lowest index.  partials: scratch of >= 64*8 bytes. */
int mh_argmax_bf16(const uint16_t* x, uint32_t n, void* partials, uint32_t* out,
                   mh_stream_t stream);

/* ------------------------------------------------- router / routing ---
 * src/kernels/lfm.rs:314 gemv_f32: y[e] = W[e, :] . x, W f32 [n, k], x bf16
 * [k], y f32 [n], chunk order (so expert ids are reproducible bit for bit). */
int mh_gemv_f32(const float* w, const uint16_t* x, float* y, uint32_t n, uint32_t k,
                mh_stream_t stream);
/* The same with a bf16 router matrix (BASELINE config 3's router). */
int mh_gemv_bf16(const uint16_t* w, const uint16_t* x, float* y, uint32_t n, uint32_t k,
                 mh_stream_t stream);

/* src/kernels/lfm.rs:391 route_token: top-k of one token's logits [e] ->
 * ids u32 [topk], weights bf16 [topk].  bias f32 [e] (may be NULL = 0) is
 * used by MH_ROUTE_SIGMOID_BIAS only.  e <= 256, topk <= 8. */
int mh_route_token(const float* logits, const float* bias, uint32_t* ids, uint16_t* weights,
                   uint32_t e, uint32_t topk, int mode, float eps, mh_stream_t stream);

/* src/kernels/lfm.rs:266 router_addnorm_route without the residual add +
 * RMSNorm prologue: router GEMV (x already normalised) and top-k in one
 * launch; the last workgroup to finish routes.  logits f32 [e] are written
 * too.  counter: one u32, zero on entry, left zero. */
int mh_router_route(const void* w, int w_dtype, const uint16_t* x, float* logits,
                    const float* bias, uint32_t* ids, uint16_t* weights, uint32_t* counter,
                    uint32_t e, uint32_t k, uint32_t topk, int mode, float eps,
                    mh_stream_t stream);

/* ------------------------------------------------- decode experts ---
 * src/kernels/lfm.rs:421 gemv_gather_act: for slot r < topk and row
 * j < n_inter, act[r, j] = bf16(bf16(silu(g)) * u) with g, u the bf16 gate
 * and up rows ids[r]*n_inter + j of the stacked matrices against x.
 * in_features <= 2048, 4-bit weights. */
int mh_gemv_gather_act(const mh_quant_weights* gate, const mh_quant_weights* up,
                       const uint16_t* x, const uint32_t* ids, uint16_t* act, uint32_t topk,
                       uint32_t n_inter, mh_stream_t stream);

/* src/kernels/lfm.rs:464 gemv_gu_act: the dense (unrouted) form, act[j]. */
int mh_gemv_gu_act(const mh_quant_weights* gate, const mh_quant_weights* up, const uint16_t* x,
                   uint16_t* act, mh_stream_t stream);

/* src/kernels/lfm.rs:499 gemv_gather_down_combine4: p_r = bf16(down row
 * ids[r]*n_out + i . act[r]); out[i] = bf16(sum_r bf16(w_r * p_r)), r
 * ascending.  topk 1..4, in_features <= 2048, 4-bit weights. */
int mh_gemv_gather_down_combine(const mh_quant_weights* down, const uint16_t* act,
                                const uint32_t* ids, const uint16_t* weights, uint16_t* out,
                                uint32_t topk, uint32_t n_out, mh_stream_t stream);

/* One MoE decode step (src/lfm.rs:967-1011 moe_decode with the routing of
 * :266): router GEMV + top-k -> gate/up + SwiGLU -> down + combine.
 * Stacked experts: gate/up [E*n_inter, d_model], down [E*d_model, n_inter].
 * logits f32 [E], ids [topk], weights bf16 [topk], act bf16 [topk, n_inter]
 * are written as intermediates.  scratch: MH_MOE_DECODE_SCRATCH_WORDS u32,
 * 8-byte aligned, zeroed once before the first call and then owned by this
 * function (it keeps the words consistent from call to call; no other use,
 * and calls sharing one scratch must not overlap).  Runs as one launch
 * (workgroups exchange logits and activations through the scratch, every
 * workgroup resident) when d_model <= 2048, n_inter % 64 == 0, topk <= 4,
 * topk * n_inter <= 8192, the router is 16-byte and act 4-byte aligned and
 * the device has >= 256 CUs; otherwise as three launches. */
#define MH_MOE_DECODE_SCRATCH_WORDS 10240u
int mh_moe_decode(const void* router, int router_dtype, const float* bias, int mode, float eps,
                  const mh_quant_weights* gate, const mh_quant_weights* up,
                  const mh_quant_weights* down, uint32_t n_experts, uint32_t topk,
                  const uint16_t* x, uint16_t* out, float* logits, uint32_t* ids,
                  uint16_t* weights, uint16_t* act, uint32_t* scratch, mh_stream_t stream);


/* Measurement only (no reference counterpart): mh_moe_decode on the
 * single-launch path with phase timestamps.  `stamps` holds
 * MH_MOE_DECODE_STAMP_WAVES x MH_MOE_DECODE_STAMPS u64 words; lane 0 of each
 * of the launch's waves w writes its words at w * MH_MOE_DECODE_STAMPS: the
 * 100 MHz constant clock at wave start, router row stored, experts chosen,
 * first gate/up loads issued, first and last activation triple published,
 * down loads issued, activations all in, output stored; word 9 the XCD the
 * workgroup ran on.  Outputs are mh_moe_decode's.  MH_ERR_UNSUPPORTED where
 * the step runs as three launches. */
#define MH_MOE_DECODE_STAMP_WAVES 2048u
#define MH_MOE_DECODE_STAMPS 10u
int mh_moe_decode_stamped(const void* router, int router_dtype, const float* bias, int mode, float eps,
                          const mh_quant_weights* gate, const mh_quant_weights* up, const mh_quant_weights* down,
                          uint32_t n_experts, uint32_t topk, const uint16_t* x, uint16_t* out, float* logits,
                          uint32_t* ids, uint16_t* weights, uint16_t* act, uint32_t* scratch, uint64_t* stamps,
                          mh_stream_t stream);

/* ------------------------------------------------- prefill routing ---
 * src/kernels/lfm.rs:366 router_prefill: logits f32 [m, e] = x [m, k] W^T,
 * W f32 or bf16 [e, k], chunk order. */
int mh_router_prefill(const uint16_t* x, const void* w, int w_dtype, float* out, uint32_t m,
                      uint32_t k, uint32_t e, mh_stream_t stream);

/* src/kernels/lfm.rs:536 moe_route_batch: route_token for m tokens; ids u32
 * [m, topk], gw bf16 [m, topk]. */
int mh_moe_route_batch(const float* logits, const float* bias, uint32_t* ids, uint16_t* gw,
                       uint32_t m, uint32_t e, uint32_t topk, int mode, float eps,
                       mh_stream_t stream);

/* ---------------------------------------------- prefill counting sort ---
 * src/kernels/lfm.rs:557-624.  counts u32 [e] (zeroed by
 * mh_moe_zero_counts, then accumulated); offsets = exclusive scan; the
 * stable scatter in slot order (token-major, rank-major): ids_sorted[pos] =
 * token, slotpos[t*topk + r] = pos.  e <= 256. */
int mh_moe_zero_counts(uint32_t* counts, uint32_t e, mh_stream_t stream);
int mh_moe_count_slots(const uint32_t* ids, uint32_t* counts, uint32_t s, uint32_t e,
                       mh_stream_t stream);
int mh_moe_offsets(const uint32_t* counts, uint32_t* offsets, uint32_t e, mh_stream_t stream);
int mh_moe_sorted(const uint32_t* ids, const uint32_t* offsets, uint32_t* ids_sorted,
                  uint32_t* slotpos, uint32_t m, uint32_t e, uint32_t topk, mh_stream_t stream);

/* ------------------------------------------------ prefill block maps ---
 * src/kernels/lfm.rs:626-697 with the column tile given per map (the
 * reference uses one bn for both; its tiles have gu_bn == dn_bn == 64).
 * Entry i of expert e is uint4(m0, e*N + n0, n0, m_end), in expert order;
 * mh_moe_zero_blocks clears the maps first (unused tail entries stay zero
 * and are skipped by the GEMMs). */
int mh_moe_zero_blocks(uint32_t* gu, uint32_t* dn, uint32_t n_gu, uint32_t n_dn,
                       mh_stream_t stream);
int mh_moe_block_offsets(const uint32_t* counts, uint32_t* gu_off, uint32_t* dn_off, uint32_t e,
                         uint32_t bm, uint32_t gu_bn, uint32_t dn_bn, uint32_t gu_n,
                         uint32_t dn_n, mh_stream_t stream);
int mh_moe_blocks(const uint32_t* counts, const uint32_t* offsets, const uint32_t* gu_off,
                  const uint32_t* dn_off, uint32_t* gu, uint32_t max_gu, uint32_t* dn,
                  uint32_t max_dn, uint32_t e, uint32_t bm, uint32_t gu_bn, uint32_t dn_bn,
                  uint32_t gu_n, uint32_t dn_n, mh_stream_t stream);

/* ----------------------------------------------------- elementwise ---
 * src/kernels/elementwise.rs:59 gather_rows_bf16: out[i, :] = table[ids[i], :]
 * (h % 8 == 0; ids clamped to n_table - 1).  :48 silu_mul_bf16:
 * out = bf16(bf16(silu(g)) * u).  src/kernels/lfm.rs:701 moe_combine_rows:
 * out[t, c] = bf16(sum_r bf16(w[t, r] * sorted[slotpos[t, r], c])). */
int mh_gather_rows_bf16(const uint16_t* table, const uint32_t* ids, uint16_t* out, uint32_t m,
                        uint32_t h, uint32_t n_table, mh_stream_t stream);
int mh_silu_mul_bf16(const uint16_t* gate, const uint16_t* up, uint16_t* out, size_t n,
                     mh_stream_t stream);
int mh_moe_combine_rows(const uint16_t* sorted, const uint32_t* slotpos, const uint16_t* weights,
                        uint16_t* out, uint32_t m, uint32_t h, uint32_t topk, mh_stream_t stream);

/* ------------------------------------------------- grouped Q4 GEMM ---
 * src/kernels/quant.rs:223 gemm_q4_grouped_mlx: for every block-map entry
 * (m0, e*N + n0, n0, m_end): C[m, n0 + j] = A[m, :] . dequant(W[e*N + n0 + j, :])
 * (bf16 dequant, f32 MFMA accumulation, bf16 store), m in [m0, m_end).
 * A bf16 [s_rows, K], C bf16 [s_rows, n], W 4-bit group 64 [E*n, K].
 * Tiles (bm x bn): 32x64 and 128x64 (the reference's MoeTile shapes) and
 * 128x256.  The map's column tile must equal bn. */
int mh_gemm_q4_grouped(const uint16_t* a, const mh_quant_weights* w, uint16_t* c,
                       const uint32_t* blocks, uint32_t n_blocks, uint32_t s_rows, uint32_t n,
                       uint32_t bm, uint32_t bn, mh_stream_t stream);

/* src/kernels/gemm.rs:33-60 gemm_bf16_nt (gemm.metal's gemm_bf16_nt_nax /
 * _wide): C[M, N] = A[M, K] . B[N, K]^T, bf16 operands, f32 accumulation on
 * the matrix cores (128 x 128 tiles), bf16 store (round to nearest even).
 * Any M, N, K: K a multiple of 64 with 16-byte aligned A and B (each under
 * 4 GiB) runs the tile kernel, other shapes a per-element kernel (f32 fma in
 * ascending k).  M or N of 0 is a no-op. */
int mh_gemm_bf16_nt(const uint16_t* a, const uint16_t* b, uint16_t* c, uint32_t m, uint32_t n, uint32_t k,
                    mh_stream_t stream);

/* src/kernels/quant.rs:126-146 gemm_quant_bf16_nt: W (4, 6 or 8 bits, [N,
 * K]) dequantized into `scratch` (bf16, at least N * K elements, 16-byte
 * aligned; the reference's error text when it is too small), then
 * mh_gemm_bf16_nt(A [M, K], scratch, C [M, N]). */
int mh_gemm_quant_bf16_nt(const uint16_t* a, uint32_t m, const mh_quant_weights* w, uint16_t* c, uint16_t* scratch,
                          size_t scratch_elems, mh_stream_t stream);

/* src/lfm.rs:661-671 project (prefill): dequant_q4_bf16_bulk + gemm_bf16_nt
 * fused: C[m, :] = A[m, :] . dequant(W)^T for every row m < M, A bf16 [M, K]
 * (16-byte aligned), W 4-bit group 64 [N, K], C bf16 [M, N]; the grouped
 * GEMM's kernel (bf16 dequant, f32 MFMA accumulation) over a dense tiling
 * (128 x 256 tiles, 128 x 64 when N % 256 != 0).  N a multiple of 64. */
int mh_gemm_q4_dense(const uint16_t* a, uint32_t m, const mh_quant_weights* w, uint16_t* c,
                     mh_stream_t stream);

/* src/kernels/quant.rs:151 gemm_q4_grouped_mlx_gu: gate and up over the
 * same map and A, stored separately.  Tiles 32x64, 128x64, 128x128. */
int mh_gemm_q4_grouped_gu(const uint16_t* a, const mh_quant_weights* gate,
                          const mh_quant_weights* up, uint16_t* gate_out, uint16_t* up_out,
                          const uint32_t* blocks, uint32_t n_blocks, uint32_t s_rows, uint32_t n,
                          uint32_t bm, uint32_t bn, mh_stream_t stream);

/* gate/up + SwiGLU fused (gemm_q4_grouped_mlx_gu followed by silu_mul_bf16,
 * src/lfm.rs:953-961), with the row gather of gather_rows_bf16 folded into
 * the A load: tile row m reads x[ids_sorted[m]] (ids_sorted may be NULL: A =
 * x [s_rows, K]).  act bf16 [s_rows, n]. */
int mh_gemm_q4_grouped_gu_act(const uint16_t* x, const uint32_t* ids_sorted, uint32_t x_rows,
                              const mh_quant_weights* gate, const mh_quant_weights* up,
                              uint16_t* act, const uint32_t* blocks, uint32_t n_blocks,
                              uint32_t s_rows, uint32_t n, uint32_t bm, uint32_t bn,
                              mh_stream_t stream);

/* No reference counterpart: the two grouped GEMMs above on a block map in
 * launch order, for callers that hold one (mh_moe_prefill's workspace regions
 * MH_PREFILL_WS_GU_ORD / DN_ORD): entry b is workgroup b's, the map holds a
 * whole number of 8 x (n / bn) entries, all-zero entries for workgroups
 * without one.  Each workgroup reads its entry with one load instead of
 * ranking the map's rows.  Segment tiles only: bm 256 or 512 (rows per
 * entry), bn 256 (down) or 128 (gate/up + SwiGLU, with ids_sorted); K a
 * multiple of 512.  Same outputs as the reference-order calls over the same
 * entries. */
int mh_gemm_q4_grouped_ordered(const uint16_t* a, const mh_quant_weights* w, uint16_t* c, const uint32_t* ord,
                               uint32_t n_entries, uint32_t s_rows, uint32_t n, uint32_t bm, uint32_t bn,
                               mh_stream_t stream);
int mh_gemm_q4_grouped_gu_act_ordered(const uint16_t* x, const uint32_t* ids_sorted, uint32_t x_rows,
                                      const mh_quant_weights* gate, const mh_quant_weights* up, uint16_t* act,
                                      const uint32_t* ord, uint32_t n_entries, uint32_t s_rows, uint32_t n,
                                      uint32_t bm, uint32_t bn, mh_stream_t stream);

/* ------------------------------------------------- prefill MoE step ---
 * src/lfm.rs:847-965 moe_prefill for m tokens on a caller workspace
 * (no allocation): router -> route -> sort -> maps -> gate/up+SwiGLU ->
 * down -> combine.  out bf16 [m, d_model].  The workspace holds the
 * intermediates below; mh_moe_prefill_workspace returns its size and (if
 * offsets != NULL) each region's byte offset.  With a bf16 router of at most
 * 64 experts and d_model 1024 or 2048 the router runs on the matrix cores:
 * the logits region then holds the chunk-order logit of every expert that
 * could reach a token's top-k (every chosen one among them) and, for the
 * others, an approximation within 2^-12 sum |x w| + 2^-138 of it; ids and
 * weights are the chunk-order routing's either way.  GU_ORD / DN_ORD hold
 * the two block maps' entries again in the grouped GEMMs' launch order
 * (entry b for workgroup b, all-zero entries for workgroups without one;
 * map rows ranked by row count, most first), when the map has at most 1024
 * rows (else they are unused and the GEMMs rank the rows themselves). */
enum {
    MH_PREFILL_WS_LOGITS = 0, MH_PREFILL_WS_IDS, MH_PREFILL_WS_GW, MH_PREFILL_WS_COUNTS,
    MH_PREFILL_WS_OFFSETS, MH_PREFILL_WS_IDS_SORTED, MH_PREFILL_WS_SLOTPOS,
    MH_PREFILL_WS_GU_OFF, MH_PREFILL_WS_DN_OFF, MH_PREFILL_WS_GU_MAP, MH_PREFILL_WS_DN_MAP,
    MH_PREFILL_WS_ACT, MH_PREFILL_WS_ED, MH_PREFILL_WS_GU_ORD, MH_PREFILL_WS_DN_ORD, MH_PREFILL_WS_REGIONS
};
size_t mh_moe_prefill_workspace(uint32_t m, uint32_t n_experts, uint32_t topk, uint32_t d_model,
                                uint32_t n_inter, size_t* offsets);
int mh_moe_prefill(const void* router, int router_dtype, const float* bias, int mode, float eps,
                   const mh_quant_weights* gate, const mh_quant_weights* up,
                   const mh_quant_weights* down, uint32_t n_experts, uint32_t topk,
                   const uint16_t* x, uint32_t m, uint16_t* out, void* workspace,
                   size_t workspace_bytes, mh_stream_t stream);

/* Measurement only (no reference counterpart): mh_moe_prefill with the two
 * grouped GEMMs stamped per workgroup.  `stamps` holds 2 x
 * MH_PREFILL_STAMP_WGS x MH_PREFILL_STAMPS u64 words (gate/up + SwiGLU, then
 * down); workgroup g of a GEMM writes at g * MH_PREFILL_STAMPS: the 100 MHz
 * constant clock at its start (word 0) and at its end (after its last stores
 * were issued, word 1), its block-map entry (0xffffffff for a padding
 * workgroup; with launch-ordered maps the index into GU_ORD / DN_ORD) | the
 * entry's row count << 32 (word 2), and the clock once its entry was read
 * (word 3; 0 for padding and empty entries).  Outputs are mh_moe_prefill's.
 * MH_ERR_UNSUPPORTED where the GEMMs do not take the segment kernels or
 * need more workgroups than the buffer holds. */
#define MH_PREFILL_STAMP_WGS 4096u
#define MH_PREFILL_STAMPS 4u
int mh_moe_prefill_stamped(const void* router, int router_dtype, const float* bias, int mode, float eps,
                           const mh_quant_weights* gate, const mh_quant_weights* up,
                           const mh_quant_weights* down, uint32_t n_experts, uint32_t topk,
                           const uint16_t* x, uint32_t m, uint16_t* out, void* workspace,
                           size_t workspace_bytes, uint64_t* stamps, mh_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MOLTEN_HIP_H */

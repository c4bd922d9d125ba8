/*
 * pbsample.h -- C ABI of the MI355X (gfx950) decode-step token sampler.
 *
 * Drop-in for promptboot's sampler path.  Reference interfaces replaced (paths
 * relative to the promptboot repository root):
 *
 *   SamplingState, new/state/draws/next_24 crates/promptboot-core/src/inference.rs:772-810
 *   sample_token_with_repetition          crates/promptboot-core/src/inference.rs:919-965
 *   sample_token                          crates/promptboot-core/src/inference.rs:914-917
 *   greedy_token                          crates/promptboot-core/src/inference.rs:861-881
 *   top_logits_8                          crates/promptboot-core/src/inference.rs:814-859
 *   InferenceError / status / domain /    crates/promptboot-core/src/inference.rs:155-264
 *   field-kind codes
 *   policy constants                      crates/promptboot-core/src/inference.rs:16-23
 *
 * Conventions kept from the reference: floats never cross the ABI (logits are
 * binary32 bit patterns in uint32_t words, fp32_sse2.rs:1-6); every call
 * returns an InferenceStatus value and fills a 48-byte error record; errors
 * are transactional (logits, the `seen` scratch and the sampling state are
 * left untouched and no draw is consumed).  The host keeps the xorshift64*
 * generator; devices only ever see 24-bit uniforms.
 *
 * Entry points:
 *   - host single-row drop-ins (pointers to host memory, one GPU call each):
 *     pb_sample_token_with_repetition, pb_sample_token, pb_greedy_token,
 *     pb_top_logits_8;
 *   - batched device entry points (pointers to device memory, asynchronous on
 *     the given HIP stream): pb_sample_batch, pb_sample_batch_inplace;
 *   - the fused Q4_0 LM head + sampler: pb_lmhead_pack_q4_0,
 *     pb_lmhead_sample_batch; the Q8_0 head: pb_lmhead_pack_q8_0,
 *     pb_lmhead_q8_sample_batch, pb_lmhead_q8_decode_step;
 *   - one step of the REPL's decode loop for many sequences
 *     (src/model_repl.rs:928-1150): pb_decode_step, pb_lmhead_decode_step,
 *     with the host helpers pb_decode_draw and pb_decode_settle;
 *   - host PRNG helpers: pb_sampling_state_new, pb_next_24, pb_fill_random_24.
 */
#ifndef PBSAMPLE_H
#define PBSAMPLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PB_VOCAB 151936u                   /* LOGIT_WORDS, inference.rs:16 */
#define PB_TOP_K 20u                       /* SAMPLING_TOP_K, inference.rs:20 */
#define PB_SEEN_BYTES ((PB_VOCAB + 7u) / 8u) /* 18,992 */
#define PB_SAMPLING_TEMPERATURE_MILLI 700u /* inference.rs:19 */
#define PB_SAMPLING_TOP_P_MILLI 800u       /* inference.rs:21 */
#define PB_SAMPLING_REPETITION_PENALTY_MILLI 1100u /* inference.rs:22 */
#define PB_SAMPLING_POLICY "temperature_0p7_top_k_20_top_p_0p8_repetition_penalty_1p1"
#define PB_NO_LAYER 0xffffffffu
#define PB_NO_TENSOR 0xffffffffu
#define PB_NO_TOKEN 0xffffffffu

/* InferenceStatus (inference.rs:155-169). */
enum pb_status {
  PB_OK = 0, PB_STATE = 1, PB_CONTEXT = 2, PB_TOKEN_ID = 3, PB_CAPACITY = 4,
  PB_ALIGNMENT = 5, PB_NONFINITE_INPUT = 6, PB_NONFINITE_OUTPUT = 7, PB_MODEL = 8,
  PB_ARITHMETIC = 9, PB_FAULTED = 10,
  /* Not in the reference: the HIP runtime failed (no device, launch error). */
  PB_DEVICE = 0x100
};
/* InferenceDomain values used by the sampler (inference.rs:171-194). */
enum pb_domain { PB_DOMAIN_NONE = 0, PB_DOMAIN_LOGITS = 18, PB_DOMAIN_ARGMAX = 19 };
/* InferenceFieldKind values used by the sampler (inference.rs:196-212). */
enum pb_field_kind {
  PB_FIELD_NONE = 0, PB_FIELD_TOKEN = 2, PB_FIELD_BYTES = 4, PB_FIELD_ALIGNMENT = 5,
  PB_FIELD_FINITE = 7, PB_FIELD_LOGITS = 12
};

/* SamplingState (inference.rs:772-776): 16 bytes, repr(C). */
typedef struct pb_sampling_state {
  uint64_t state;
  uint64_t draws;
} pb_sampling_state;

/* InferenceError (inference.rs:226-237): 48 bytes, detail = kind << 32 | sub. */
typedef struct pb_inference_error {
  uint32_t status, domain, layer, position, tensor_id, reserved;
  uint64_t needed, available, detail;
} pb_inference_error;

/* TopLogit (inference.rs:767-770). */
typedef struct pb_top_logit {
  uint32_t token;
  uint32_t logit_bits;
} pb_top_logit;

/* Layout checks at compile time, as the reference makes them for its repr(C)
 * types (InferenceError: inference.rs:287-288; SamplingState: :812).  A C11
 * or C++11 consumer whose struct layout differs does not compile. */
#ifdef __cplusplus
#define PB_STATIC_ASSERT(cond, msg) static_assert(cond, msg)
#define PB_ALIGNOF(type) alignof(type)
#else
#define PB_STATIC_ASSERT(cond, msg) _Static_assert(cond, msg)
#define PB_ALIGNOF(type) _Alignof(type)
#endif
PB_STATIC_ASSERT(sizeof(pb_sampling_state) == 16, "SamplingState is 16 bytes");
PB_STATIC_ASSERT(PB_ALIGNOF(pb_sampling_state) == 8, "SamplingState is 8-byte aligned");
PB_STATIC_ASSERT(sizeof(pb_inference_error) == 48, "InferenceError is 48 bytes");
PB_STATIC_ASSERT(PB_ALIGNOF(pb_inference_error) == 8, "InferenceError is 8-byte aligned");
PB_STATIC_ASSERT(offsetof(pb_inference_error, tensor_id) == 16, "InferenceError.tensor_id at 16");
PB_STATIC_ASSERT(offsetof(pb_inference_error, needed) == 24, "InferenceError.needed at 24");
PB_STATIC_ASSERT(offsetof(pb_inference_error, available) == 32, "InferenceError.available at 32");
PB_STATIC_ASSERT(offsetof(pb_inference_error, detail) == 40, "InferenceError.detail at 40");
PB_STATIC_ASSERT(sizeof(pb_top_logit) == 8, "TopLogit is 8 bytes");

/* Per-row evidence beside each draw.  Not in the reference (it returns only the
 * token): the top-20 in rank order, their penalised logits and softmax
 * weights, the kept-survivor probabilities w[i]/kept_total (0 past `kept`),
 * the top-p survivor count, the drawn rank and boundary flags
 * (PB_FLAG_*).  On a row error every byte is 0xff. */
typedef struct pb_sample_detail {
  uint32_t ids[PB_TOP_K];
  uint32_t value_bits[PB_TOP_K];
  uint32_t weight_bits[PB_TOP_K];
  float probs[PB_TOP_K];
  uint32_t kept;
  uint32_t rank;
  uint32_t flags;
  uint32_t token;
} pb_sample_detail;
PB_STATIC_ASSERT(sizeof(pb_sample_detail) == 336, "pb_sample_detail is 84 words");

#define PB_FLAG_DRAW_BOUNDARY 1u   /* target within 1e-6 * kept_total of a CDF step */
#define PB_FLAG_CUTOFF_BOUNDARY 2u /* top-p cutoff within 1e-6 * total of a prefix */

/* ---- host PRNG (inference.rs:779-810) ---- */

/* SamplingState::new: seed 0 is replaced by 0x9e3779b97f4a7c15. */
void pb_sampling_state_new(pb_sampling_state *state, uint64_t seed);
/* SamplingState::next_24 (crate-private in the reference): one xorshift64*
 * step, draws += 1, returns the top 24 bits of the scrambled state. */
uint32_t pb_next_24(pb_sampling_state *state);
/* One next_24 per row: out[i] = pb_next_24(&states[i]). */
void pb_fill_random_24(pb_sampling_state *states, uint32_t rows, uint32_t *out);

/* ---- single-row drop-ins (host memory, synchronous) ----
 * They run on the library's default context (the current HIP device).  The
 * logits row, history and (for the drop-in with repetition) the penalised
 * write-back are staged through pinned buffers; all selection arithmetic runs
 * on the GPU.  Returns the InferenceStatus; *err is always written. */

/* sample_token_with_repetition (inference.rs:919-965).  On success `logits`
 * holds the penalised row (once per unique history id, in place), `seen` is
 * returned with the history bits cleared, the state advanced by one draw. */
uint32_t pb_sample_token_with_repetition(uint32_t *logits, size_t logits_len,
                                         const uint32_t *tokens, size_t tokens_len,
                                         uint8_t *seen, size_t seen_len,
                                         pb_sampling_state *state, uint32_t *out_token,
                                         pb_inference_error *err);

/* sample_token (inference.rs:914-917): no penalty; logits are not modified. */
uint32_t pb_sample_token(const uint32_t *logits, size_t logits_len, pb_sampling_state *state,
                         uint32_t *out_token, pb_inference_error *err);

/* greedy_token (inference.rs:861-881): argmax, lowest id on ties. */
uint32_t pb_greedy_token(const uint32_t *logits, size_t logits_len, uint32_t *out_token,
                         pb_inference_error *err);

/* top_logits_8 (inference.rs:814-859): output untouched on error. */
uint32_t pb_top_logits_8(const uint32_t *logits, size_t logits_len, pb_top_logit output[8],
                         pb_inference_error *err);

/* ---- batched device sampler ---- */

typedef struct pb_context pb_context;

/* Creates a context on `device` (-1 = current device).  The context owns the
 * inter-kernel workspace of the batched calls and the staging buffers of the
 * drop-ins; every allocation happens here or in pb_context_reserve.  At
 * creation it holds the sampler's workspace for any batch under the
 * automatic slice plan and the drop-ins' staging for histories of up to
 * PB_CONTEXT_IDS ids; the LM head needs pb_context_reserve first. */
#define PB_CONTEXT_IDS 32768u /* CONTEXT_LIMIT, inference.rs:13 */
uint32_t pb_context_create(int device, pb_context **out);
void pb_context_destroy(pb_context *ctx);

/* Sizes the context's workspace for batched calls of up to `rows` rows: the
 * sampler's slice workspace under the context's current slice plan
 * (pb_context_set_segments), and, when cols > 0, the fused LM head's
 * workspace for hidden states of up to `cols` columns (either head format,
 * rows <= PB_LMHEAD_MAX_ROWS; logits only for the steps of up to 64 rows that
 * keep them there, since a wider step without a logits buffer runs in one
 * pass and keeps none: 40.2 MB at 256 rows of 896 columns).  Allocates only
 * when the workspace grows; never shrinks it.  A workspace it outgrows stays
 * allocated until pb_context_destroy, so launches already enqueued and HIP
 * graphs captured before the growth keep valid memory (they keep using the
 * old workspace).  Call it at set-up: the batched entry points below never
 * allocate, never wait, and return PB_CAPACITY (needed/available = workspace
 * bytes) when a call needs more than was reserved, so a reserved context's
 * calls can be captured in a HIP graph. */
uint32_t pb_context_reserve(pb_context *ctx, uint32_t rows, size_t cols, pb_inference_error *err);

/* Threading and streams: one context's batched calls share its workspace.
 * Calls on one context must be ordered -- issued on one stream, or the
 * caller orders the streams -- and calls that overlap on the device race on
 * the workspace.  The host side takes the context's lock, so concurrent
 * host threads are safe; different contexts are independent. */

/*
 * Samples `rows` independent rows.  All pointers are device pointers; the
 * call only enqueues work on `stream` (a hipStream_t, NULL = default stream).
 *
 *   d_logits     rows x ld binary32 words; vocab must be PB_VOCAB; ld >= vocab,
 *                ld % 4 == 0, 16-byte aligned.  Not modified.
 *   d_hist       rows x hist_ld token ids (may be NULL when every length is 0),
 *   d_hist_len   valid ids per row (NULL = 0); lengths above hist_ld are clamped.
 *   d_random_24  one next_24 value per row (the host advanced one
 *                SamplingState per row; only the low 24 bits are used).
 *   d_token      out: selected id, PB_NO_TOKEN on a row error.
 *   d_detail     out (optional): pb_sample_detail per row.
 *   d_err        out (optional): pb_inference_error per row (all-zero on success).
 *
 * Row semantics are sample_token_with_repetition's: non-finite logit ->
 * NONFINITE_OUTPUT (first index), else history id >= vocab -> TOKEN_ID (first
 * position), else penalty + top-k/top-p draw.  A failing row consumes no
 * draw: the caller restores that row's SamplingState.
 * Returns PB_OK when the work was enqueued, else a status with *err filled
 * (err may be NULL) and nothing enqueued.
 */
uint32_t pb_sample_batch(pb_context *ctx, const uint32_t *d_logits, size_t vocab, size_t ld,
                         uint32_t rows, const uint32_t *d_hist, size_t hist_ld,
                         const uint32_t *d_hist_len, const uint32_t *d_random_24,
                         uint32_t *d_token, pb_sample_detail *d_detail,
                         pb_inference_error *d_err, void *stream, pb_inference_error *err);

/* pb_sample_batch without any allocation, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Its workspace is a static
 * device array of 3,646,464 bytes per device, held until the process ends,
 * instead of the context's workspace: the tile words of PB_TILE_SELECT_ROWS
 * rows, which also hold the slice records of every batch of the automatic
 * slice plan, so every batch takes the path pb_sample_batch takes.  A slice
 * plan forced on the context (pb_context_set_segments) that needs more than
 * the array (over 21,705 row x slice records) is refused with PB_CAPACITY
 * (needed/available = bytes) before anything is enqueued.  Every context on
 * one device shares that device's array: calls that overlap on the device,
 * from any context or stream, race on it.  The context supplies the device
 * and the slice plan; its own workspace is not used. */
uint32_t pb_sample_batch_noalloc(pb_context *ctx, const uint32_t *d_logits, size_t vocab,
                                 size_t ld, uint32_t rows, const uint32_t *d_hist,
                                 size_t hist_ld, const uint32_t *d_hist_len,
                                 const uint32_t *d_random_24, uint32_t *d_token,
                                 pb_sample_detail *d_detail, pb_inference_error *d_err,
                                 void *stream, pb_inference_error *err);

/* As pb_sample_batch, then applies the repetition penalty in place to every
 * successful row (once per unique history id), as the reference mutates the
 * caller's logits (fp32_sse2.rs:1848-1876).  d_seen (optional, rows x
 * PB_SEEN_BYTES) is the per-row `seen` scratch: ids whose bit is already set
 * are not penalised (the reference's dedupe), and the history bits are
 * cleared on success rows. */
uint32_t pb_sample_batch_inplace(pb_context *ctx, uint32_t *d_logits, size_t vocab, size_t ld,
                                 uint32_t rows, const uint32_t *d_hist, size_t hist_ld,
                                 const uint32_t *d_hist_len, const uint32_t *d_random_24,
                                 uint8_t *d_seen, uint32_t *d_token,
                                 pb_sample_detail *d_detail, pb_inference_error *d_err,
                                 void *stream, pb_inference_error *err);

/* ---- fused Q4_0 LM head + sampler ----
 * Replaces, for a batch of hidden states, the reference's
 * inference_prepare_q8 + inference_q4_matvec_rows_prepared
 * (crates/promptboot-core/src/fp32_sse2.rs:956-983, 1217-1248) followed by
 * sample_token_with_repetition (inference.rs:919-965) on each logits row.
 * The logits are bit-identical to the reference's Q4 head (int8 MFMA for the
 * exact block dots, the reference's per-block binary32 epilogue in order). */

/* Largest batch of one LM-head call (either format) and of an LM-head
 * reservation: the kernels address the quantised activations (at most
 * 64 blocks x 32 bytes per row) with 32-bit offsets.  More rows are refused
 * with PB_CAPACITY (needed = this limit, available = rows). */
#define PB_LMHEAD_MAX_ROWS 262144u

/* Bytes of the device layout of a Q4_0 head: the source size (rows * cols /
 * 32 blocks of 18 bytes) plus one flag word per 64-id tile. */
size_t pb_lmhead_packed_bytes(size_t vocab, size_t cols);

/* Repacks a Q4_0 matrix in promptboot's layout (vocab rows of cols/32 blocks
 * of 18 bytes: fp16 scale, 16 nibble bytes with element i in the low and
 * 16 + i in the high nibble; the token_embd layout of model.rs:810-812) into
 * the device layout (tiles of 64 ids: vocab must be a multiple of 64, as
 * PB_VOCAB is).  Device pointers; d_packed 16-byte aligned and
 * pb_lmhead_packed_bytes long.  Done once per model, outside the decode step. */
uint32_t pb_lmhead_pack_q4_0(const uint8_t *d_q4, size_t vocab, size_t cols, uint8_t *d_packed,
                             void *stream, pb_inference_error *err);

/* One decode step for `rows` sequences: hidden states (rows x cols binary32
 * words, 16-byte aligned) through the packed head, then the sampler exactly as pb_sample_batch
 * on the resulting logits (repetition penalty, top-k 20, temperature 0.7,
 * top-p 0.8, draw).  vocab must be PB_VOCAB, cols a multiple of 32 up to 2048
 * (896 for Qwen2.5-0.5B).  packed_bytes is the size of d_packed and must be
 * pb_lmhead_packed_bytes(vocab, cols): a head packed for another width or
 * format is refused (PB_CAPACITY) before anything is enqueued.  d_logits
 * (optional, rows x vocab words) receives the raw logits.  Without it, a step
 * of more than 64 rows runs in one pass: the head writes no logits at all,
 * only two words per (row, 64-id tile), and the selection recomputes the few
 * tiles it has to read from the packed head (same results, bit for bit); up
 * to 64 rows the logits go through the context's workspace.  Per-row outputs
 * and error records as pb_sample_batch (non-finite logit, bad history id).
 * Needs a context reserved (pb_context_reserve) for at least `rows` rows and
 * `cols` columns, and rows <= PB_LMHEAD_MAX_ROWS. */
uint32_t pb_lmhead_sample_batch(pb_context *ctx, const uint8_t *d_packed, size_t packed_bytes,
                                size_t vocab, size_t cols, const uint32_t *d_hidden, uint32_t rows,
                                const uint32_t *d_hist, size_t hist_ld,
                                const uint32_t *d_hist_len, const uint32_t *d_random_24,
                                uint32_t *d_token, pb_sample_detail *d_detail,
                                pb_inference_error *d_err, uint32_t *d_logits, void *stream,
                                pb_inference_error *err);

/* ---- fused Q8_0 LM head + sampler ----
 * The model's own output head is Q8_0 (tensor 290, model.rs:817-818;
 * inference.rs:1739-1749 runs it through coordinator.q8).  These replace
 * inference_prepare_q8 + inference_q8_matvec_rows_prepared
 * (fp32_sse2.rs:956-983, 1251-1280) followed by the sampler, with the Q8_0
 * head's own epilogue: total = add(total, mul(f32(dot), mul(w_scale,
 * a_scale))) over the blocks in order.  Same arguments, limits and outputs
 * as the Q4_0 functions above. */

/* Bytes of the device layout of a Q8_0 head (equal to the source size:
 * rows * cols / 32 blocks of 34 bytes). */
size_t pb_lmhead_q8_packed_bytes(size_t vocab, size_t cols);

/* Repacks a Q8_0 matrix in promptboot's layout (vocab rows of cols/32 blocks
 * of 34 bytes: fp16 scale, 32 signed weights) into the device layout (tiles of
 * 64 ids: vocab must be a multiple of 64).  Device pointers; d_packed 16-byte
 * aligned and pb_lmhead_q8_packed_bytes long.  Once per model. */
uint32_t pb_lmhead_pack_q8_0(const uint8_t *d_q8, size_t vocab, size_t cols, uint8_t *d_packed,
                             void *stream, pb_inference_error *err);

/* pb_lmhead_sample_batch for a head packed by pb_lmhead_pack_q8_0
 * (packed_bytes = pb_lmhead_q8_packed_bytes(vocab, cols)). */
uint32_t pb_lmhead_q8_sample_batch(pb_context *ctx, const uint8_t *d_packed,
                                   size_t packed_bytes, size_t vocab, size_t cols, const uint32_t *d_hidden, uint32_t rows,
                                   const uint32_t *d_hist, size_t hist_ld,
                                   const uint32_t *d_hist_len, const uint32_t *d_random_24,
                                   uint32_t *d_token, pb_sample_detail *d_detail,
                                   pb_inference_error *d_err, uint32_t *d_logits, void *stream,
                                   pb_inference_error *err);

/* ---- decode loop (src/model_repl.rs:928-1150) ----
 * One generation step for `rows` sequences at once, with the REPL's caller
 * contract kept on the device:
 *   - the history handed to the sampler is the row's whole working context
 *     (prompt + generated so far: working[..prompt_count + generated],
 *     model_repl.rs:961-968);
 *   - a sampled token is appended to that context; an end-of-sequence piece
 *     (<|im_end|> 151645 or <|endoftext|> 151643, tokenizer.rs:38-39, 1047)
 *     is stored as <|im_end|> and ends the row (model_repl.rs:1099-1103,
 *     1119-1150);
 *   - a row whose context reaches its length limit ends (the REPL's
 *     MAX_NEW_TOKENS / CONTEXT_LIMIT stop);
 *   - a row error ends the row with no append and no draw;
 *   - a row whose context is already at its limit when the step starts is
 *     not sampled (the REPL stops before sampling when there is no room):
 *     it ends with PB_ROW_LIMIT and token PB_NO_TOKEN, and its draw is
 *     returned by pb_decode_settle.
 * Row states (d_row_state, one word per row, updated in place): */
enum pb_row_state {
  PB_ROW_ACTIVE = 0, /* sampled this step */
  PB_ROW_EOS = 1,    /* ended on an end-of-sequence piece */
  PB_ROW_LIMIT = 2,  /* context reached its length limit */
  PB_ROW_ERROR = 3   /* the sampler returned an error (record in d_err) */
};
#define PB_IM_END 151645u      /* IM_END, src/repl_contract.rs:26 */
#define PB_END_OF_TEXT 151643u /* END_OF_TEXT, tokenizer.rs:39 */

/* Samples every row whose state is PB_ROW_ACTIVE, exactly as pb_sample_batch,
 * then appends the token to d_hist[row] at d_hist_len[row] and increments
 * d_hist_len[row].  d_max_len (optional) caps each row's context length
 * (default hist_ld): the append that reaches it ends the row with
 * PB_ROW_LIMIT.  Rows in any other state are skipped: their token is
 * PB_NO_TOKEN, their detail and error records are not written, and they
 * consume no uniform.  d_hist and d_hist_len are required. */
uint32_t pb_decode_step(pb_context *ctx, const uint32_t *d_logits, size_t vocab, size_t ld,
                        uint32_t rows, uint32_t *d_hist, size_t hist_ld, uint32_t *d_hist_len,
                        const uint32_t *d_max_len, uint32_t *d_row_state,
                        const uint32_t *d_random_24, uint32_t *d_token,
                        pb_sample_detail *d_detail, pb_inference_error *d_err, void *stream,
                        pb_inference_error *err);

/* The same step with the fused Q4_0 LM head in front (pb_lmhead_sample_batch
 * for the active rows, then the decode-loop bookkeeping above). */
uint32_t pb_lmhead_decode_step(pb_context *ctx, const uint8_t *d_packed, size_t packed_bytes,
                               size_t vocab, size_t cols, const uint32_t *d_hidden, uint32_t rows,
                               uint32_t *d_hist, size_t hist_ld, uint32_t *d_hist_len,
                               const uint32_t *d_max_len, uint32_t *d_row_state,
                               const uint32_t *d_random_24, uint32_t *d_token,
                               pb_sample_detail *d_detail, pb_inference_error *d_err,
                               uint32_t *d_logits, void *stream, pb_inference_error *err);

/* The same step with the fused Q8_0 head (pb_lmhead_q8_sample_batch): the
 * REPL's own configuration, whose logits come from the Q8_0 output tensor. */
uint32_t pb_lmhead_q8_decode_step(pb_context *ctx, const uint8_t *d_packed,
                                  size_t packed_bytes, size_t vocab, size_t cols, const uint32_t *d_hidden, uint32_t rows,
                                  uint32_t *d_hist, size_t hist_ld, uint32_t *d_hist_len,
                                  const uint32_t *d_max_len, uint32_t *d_row_state,
                                  const uint32_t *d_random_24, uint32_t *d_token,
                                  pb_sample_detail *d_detail, pb_inference_error *d_err,
                                  uint32_t *d_logits, void *stream, pb_inference_error *err);

/* Host side of a step: saves every states[i] into saved[i]; for each row with
 * row_state[i] == PB_ROW_ACTIVE writes out[i] = pb_next_24(&states[i]); other
 * rows keep their state and get out[i] = 0.  The REPL draws once per sampled
 * token and never for a failed sample (inference.rs:954-963). */
void pb_decode_draw(pb_sampling_state *states, const uint32_t *row_state, uint32_t rows,
                    uint32_t *out, pb_sampling_state *saved);
/* After the step: rows that were PB_ROW_ACTIVE before it and got no token
 * (tokens[i] == PB_NO_TOKEN: a row error, or a row already at its limit) get
 * their saved state back, since no sample consumed their draw.  Returns the
 * number of rows restored. */
uint32_t pb_decode_settle(pb_sampling_state *states, const pb_sampling_state *saved,
                          const uint32_t *state_before, const uint32_t *tokens, uint32_t rows);

/* Batches of up to PB_TILE_SELECT_ROWS rows under the automatic plan (and
 * without a `seen` exclusion) are sampled through per-tile summaries of the
 * logits and the fused LM head's selection kernel; larger batches, and every
 * batch under a forced slice plan, stream each row in slices. */
#define PB_TILE_SELECT_ROWS 192u

/* Slices per row of the slice plan for `rows` (diagnostic; see
 * PB_TILE_SELECT_ROWS for the batches that do not use it). */
uint32_t pb_segments_for_rows(uint32_t rows);

/* Forces the number of row slices of this context's batched calls (0 = auto,
 * otherwise clamped to 1..32).  For tuning and for testing the
 * single-workgroup and the multi-slice paths on the same rows (a forced plan
 * also turns off the small batches' tile selection). */
void pb_context_set_segments(pb_context *ctx, uint32_t segments);

/* ---- device arithmetic probes (verification hooks, no reference
 * counterpart): evaluate, on the GPU, the exact binary32 routines the sampler
 * uses, n words each, enqueued on `stream`:
 *   expf:     the restated libm expf (fp32_sse2.rs:404-469)
 *   penalize: the repetition penalty of one logit (fp32_sse2.rs:1860-1866) */
uint32_t pb_device_expf_bits(const uint32_t *d_in, uint32_t *d_out, size_t n, void *stream);
uint32_t pb_device_penalize_bits(const uint32_t *d_in, uint32_t *d_out, size_t n, void *stream);
/* One-wave self-test of the lane exchanges (DPP, permlane swaps) and wave
 * reductions the selection uses; writes 11 x 64 words to d_out. */
uint32_t pb_device_wave_selftest(uint32_t *d_out, void *stream);
/* One-wave self-test of the int8 MFMA fragment layout the LM head uses:
 * writes the 32 x 32 int32 product of A[i][k] = (7i + 3k) % 17 - 8 and
 * B[k][j] = (5k + 11j) % 15 - 7 (k < 32) to d_out[32 i + j]. */
uint32_t pb_device_mfma_selftest(int32_t *d_out, void *stream);

/* Read-only stream probe (diagnostic, no reference counterpart): `blocks`
 * workgroups read the n_words words at d_in (16-byte aligned) with the
 * sampler's load pattern, workgroup g a contiguous run of ceil(n_words / 4 /
 * blocks) 16-byte groups, and d_out[g] receives the XOR of the words it
 * read.  Timing it gives the read bandwidth the sampler's stream can reach. */
uint32_t pb_device_read_probe(const uint32_t *d_in, size_t n_words, uint32_t *d_out,
                              uint32_t blocks, void *stream);
/* The same read in grid-stride order (diagnostic, no reference counterpart):
 * the buffer is cut into 32 KiB chunks and workgroup g reads chunks g,
 * g + blocks, ... (d_out[g] receives the XOR of their words), so the
 * workgroups resident at once read one compact window that moves through the
 * buffer (the fastest plain read pattern measured on MI355X). */
uint32_t pb_device_read_probe_grid_stride(const uint32_t *d_in, size_t n_words, uint32_t *d_out,
                                          uint32_t blocks, void *stream);

/* Library version string: "pbsample <version> src:<hash of the sources it was
 * built from> gfx950". */
const char *pb_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PBSAMPLE_H */

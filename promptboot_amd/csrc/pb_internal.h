// pb_internal.h -- launch parameters shared by the kernels and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "pbsample.h"

namespace pb {

// float4 per lane per streaming chunk (register-resident, double-buffered).
constexpr int kChunkF4 = 8;

struct RowParams {
  const uint32_t* logits;  // rows x ld binary32 words
  size_t ld;
  uint32_t rows;
  const uint32_t* hist;    // rows x hist_ld ids, or null
  size_t hist_ld;
  const uint32_t* hist_len;
  const uint8_t* excl;     // rows x PB_SEEN_BYTES ids not to penalise, or null
  const uint32_t* random_24;
  uint32_t* token;
  pb_sample_detail* detail;
  pb_inference_error* err;
  uint64_t* part_keys;     // rows x segs x 20 (segs > 1)
  uint32_t* part_meta;     // rows x segs x {first non-finite index, first bad history position}
  uint32_t segs;           // slices per row
  uint32_t seg_f4;         // float4 per slice, multiple of 8
  uint32_t hist_vec4;      // history rows are 16-byte aligned: load 4 ids at a time
  // One slice per row only (0: rows in batch order).  Workgroups from
  // order_from on take the remaining rows longest history first, ranked in
  // groups of kOrderGroup rows by min(length, hist_ld) >> order_shift.
  uint32_t order_from;
  uint32_t order_shift;
  // Decode-loop mode (null row_state: plain sampling).  Rows not in
  // PB_ROW_ACTIVE are skipped; a sampled token is appended to the row's
  // context (hist_out / hist_len_out alias hist / hist_len) and the row
  // state updated.
  uint32_t* row_state;
  uint32_t* hist_out;
  uint32_t* hist_len_out;
  const uint32_t* max_len; // per-row context cap, or null (hist_ld)
  // Select kernel only (null otherwise; no `excl`): rows x hist_ld, the
  // penalised logit at each history id, for q < the row's history length.
  uint32_t* gather;
};

struct WritebackParams {
  uint32_t* logits;
  size_t ld;
  uint32_t rows;
  const uint32_t* hist;
  size_t hist_ld;
  const uint32_t* hist_len;
  uint8_t* seen;           // rows x PB_SEEN_BYTES, or null
  const uint32_t* token;   // PB_NO_TOKEN marks a failed row
  uint32_t* gather;        // rows x hist_ld final values at the history ids, or null
};

// Fused Q4_0 / Q8_0 LM head + sampler (pb_lmhead.hip).
struct LmParams {
  const uint8_t* weights;   // packed head: [blocks][vocab][16] nibbles (Q4_0) or [32] int8
                            // (Q8_0), then [blocks][vocab] fp16 scales
  bool q8;                  // the head is Q8_0 (else Q4_0)
  bool fused_quant;         // the GEMM quantises the activations itself (few rows)
  const uint32_t* hidden;   // rows x cols binary32 words
  uint32_t rows;
  uint32_t rows_pad;        // rows rounded up to 64
  uint32_t cols;            // hidden width, multiple of 32
  int8_t* act_q;            // [blocks][rows_pad][32] Q8_0 quants
  float* act_s;             // [blocks][rows_pad] activation scales (a_scale / 16 for Q4_0, a_scale for Q8_0)
  uint32_t* logits;         // rows x logits_ld raw logits (binary32 words); null for
                            // the wide GEMM's one pass (tilesec then set)
  size_t logits_ld;
  uint32_t* tilemax;        // rows x 2,374 order word of the largest raw logit per 64-id
                            // tile, 0xffffffff when the tile holds a non-finite logit
  uint32_t* tilesec;        // rows x 2,374 second words (narrow GEMM and one pass, else null):
                            // a bound above every other logit's order word of the tile
                            // (a multiple of 64) plus the maximum's index in the tile
  // tile_words_kernel only (null / 0 otherwise): the logits it reads are also
  // stored at logits_copy (same ld), and stage_v4 16-byte groups are copied
  // from stage_src to stage_dst on the way, so that logits and small inputs
  // read from pinned host memory reach the device in the same launch.
  uint32_t* logits_copy;
  const uint32_t* stage_src;
  uint32_t* stage_dst;
  uint32_t stage_v4;
};

// Batches up to this size take the narrow GEMM.
constexpr uint32_t kNarrowRows = 64;
// Rows up to which the narrow GEMM quantises the activations itself.
constexpr uint32_t kFusedQuantRows = 4;

hipError_t launch_lm_pack(const uint8_t* in, uint8_t* out, uint32_t vocab, uint32_t blocks,
                          hipStream_t stream);
hipError_t launch_lm_pack_q8(const uint8_t* in, uint8_t* out, uint32_t vocab, uint32_t blocks,
                             hipStream_t stream);
hipError_t launch_lm_sample(const LmParams& p, const RowParams& rp, hipStream_t stream);
// The batched sampler through the LM head's selection: tile words of the
// logits (p.logits, p.logits_ld, p.tilemax, p.tilesec, p.rows), then the
// select kernel.
hipError_t launch_tile_select(const LmParams& p, const RowParams& rp, hipStream_t stream);
// Batches up to this size take launch_tile_select (without a `seen`
// exclusion or a forced slice plan): rows x 2,374 x 8 bytes of workspace.
// Measured per step (us, tile selection / slice plan), full-context
// histories: B = 128 34.3 / 36.1, 192 40.6 / 42.2, 255 47.5 / 45.7, 512
// 87.7 / 63.2; histories of at most 4,096 ids, B = 128: 23.9 / 28.7.
constexpr uint32_t kTileSelectRows = PB_TILE_SELECT_ROWS;
constexpr size_t kTileSelectBytesPerRow = (size_t)(PB_VOCAB / 64) * 8;
hipError_t launch_mfma_selftest(int32_t* out, hipStream_t stream);

uint32_t segments_for_rows(uint32_t rows);
// forced_segments == 0 picks segments_for_rows(rows).
void plan_segments(uint32_t rows, uint32_t forced_segments, uint32_t* segs, uint32_t* seg_f4);
// Rows ranked together by history length (one slice per row).
constexpr uint32_t kOrderGroup = 4096;
// Workgroups of segment_kernel<.., true> that `device` holds at once, looked
// up once per device (the first call on a device queries the runtime).
hipError_t resident_rows(int device, uint32_t* out);
// Sets p->order_from and p->order_shift for a one-slice plan on `device`:
// rows past the first residency round run longest history first.
void plan_row_order(int device, RowParams* p);
hipError_t launch_sample(const RowParams& p, hipStream_t stream);
hipError_t launch_writeback(const WritebackParams& p, hipStream_t stream);
hipError_t launch_probe(int which, const uint32_t* in, uint32_t* out, size_t n,
                        hipStream_t stream);
hipError_t launch_wave_selftest(uint32_t* out, hipStream_t stream);
hipError_t launch_read_probe(const uint32_t* in, size_t n_words, uint32_t* out, uint32_t blocks,
                             bool grid_stride, hipStream_t stream);

// The context's device (pb_api.cpp).
int context_device(const pb_context* ctx);
// pb_sample_batch with `work` (work_bytes) as the slice workspace in place of
// the context's own; PB_CAPACITY when the slice plan needs more (pb_api.cpp).
uint32_t enqueue_sample_with_workspace(pb_context* ctx, void* work, size_t work_bytes,
                                       const uint32_t* d_logits, size_t vocab, size_t ld,
                                       uint32_t rows, const uint32_t* d_hist, size_t hist_ld,
                                       const uint32_t* d_hist_len, const uint32_t* d_random_24,
                                       uint32_t* d_token, pb_sample_detail* d_detail,
                                       pb_inference_error* d_err, hipStream_t stream,
                                       pb_inference_error* err);
// Device address of pb_sample_batch_noalloc's static scratch on `device`,
// looked up once per device (pb_static.hip).
hipError_t static_scratch_address(int device, void** out);

}  // namespace pb

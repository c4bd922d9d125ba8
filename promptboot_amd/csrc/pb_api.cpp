// pb_api.cpp -- C ABI of the gfx950 decode-step sampler (include/pbsample.h).
//
// Host side of the drop-in.  Mirrors promptboot's sampler API
// (crates/promptboot-core/src/inference.rs:737-965): argument meaning, error
// tuples, error precedence (length, non-finite, scratch length, history ids)
// and transactional failure (no mutation, no draw).  The selection itself
// always runs on the GPU; there is no host fallback.
#include <hip/hip_runtime.h>
#include <string.h>

#include <map>
#include <mutex>
#include <vector>

#include "pb_internal.h"
#include "pbsample.h"

namespace {

constexpr size_t kRowBytes = (size_t)PB_VOCAB * 4;

void set_error(pb_inference_error* e, uint32_t status, uint32_t domain, uint64_t needed,
               uint64_t available, uint32_t kind, uint32_t sub) {
  if (!e) return;
  e->status = status;
  e->domain = domain;
  e->layer = PB_NO_LAYER;
  e->position = 0;
  e->tensor_id = PB_NO_TENSOR;
  e->reserved = 0;
  e->needed = needed;
  e->available = available;
  e->detail = ((uint64_t)kind << 32) | sub;
}

void clear_error(pb_inference_error* e) {
  if (e) memset(e, 0, sizeof *e);
}

uint32_t device_error(pb_inference_error* e, hipError_t code) {
  set_error(e, PB_DEVICE, PB_DOMAIN_NONE, 0, (uint64_t)code, PB_FIELD_NONE, 0);
  return PB_DEVICE;
}

// Restores the caller's current device on scope exit.
struct DeviceGuard {
  int saved = -1;
  explicit DeviceGuard(int device) {
    if (hipGetDevice(&saved) != hipSuccess) saved = -1;
    if (device >= 0 && device != saved) (void)hipSetDevice(device);
  }
  ~DeviceGuard() {
    int now = -1;
    if (saved >= 0 && hipGetDevice(&now) == hipSuccess && now != saved) (void)hipSetDevice(saved);
  }
};

}  // namespace

struct pb_context {
  int device = 0;
  hipStream_t stream = nullptr;  // used by the single-row drop-ins
  std::mutex mu;                 // held by every call on this context

  uint32_t forced_segments = 0;  // 0 = automatic slices per row
  void* d_work = nullptr;  // multi-slice workspace: slice top-20 lists and slice records
  size_t list_bytes = 0;

  void* d_lm = nullptr;  // fused LM head workspace
  size_t lm_bytes = 0;
  // Workspaces that pb_context_reserve outgrew.  A HIP graph captured before
  // the growth still launches kernels on them, so they stay allocated until
  // pb_context_destroy.
  std::vector<void*> retired;

  // Single-row staging: one input region, pinned on the host and mirrored on
  // the device ([row][history length, uniform, -, -][history ids]), and one
  // output region ([token, -, -, -][error record][detail][penalised history
  // values]).  The pinned regions are coherent and mapped (z_in, z_out are
  // their device addresses): a call reads the input region from the host in
  // its first launch, which leaves a copy in d_in, and its kernels write the
  // outputs straight into h_out.  Calls with a non-zero `seen` copy the
  // regions instead, one copy each way.  The pointers below point into them;
  // `seen` has its own pair, copied only when non-zero.
  size_t hist_cap = 0;
  uint8_t* d_in = nullptr;
  uint8_t* h_in = nullptr;
  uint8_t* d_out = nullptr;
  uint8_t* h_out = nullptr;
  uint8_t* z_in = nullptr;
  uint8_t* z_out = nullptr;
  uint32_t* d_small = nullptr;  // [0] history length, [1] uniform
  uint32_t* d_row = nullptr;
  uint32_t* d_hist = nullptr;
  uint32_t* h_small = nullptr;
  uint32_t* h_row = nullptr;
  uint32_t* h_hist = nullptr;
  uint32_t* h_token = nullptr;
  pb_inference_error* h_err = nullptr;
  pb_sample_detail* h_detail = nullptr;
  uint32_t* h_gather = nullptr;
  uint8_t* d_seen = nullptr;
  uint8_t* h_seen = nullptr;
};

// Offsets inside the staging regions.  The row comes first, 16-byte aligned
// for the float4 loads; the scalars and the history ids follow it, so that
// they are one 16-byte aligned range.
constexpr size_t kInRow = 0;
constexpr size_t kInSmall = kRowBytes;
constexpr size_t kInHist = kInSmall + 16;
constexpr size_t kOutErr = 16;
constexpr size_t kOutDetail = 64;
constexpr size_t kOutGather = (kOutDetail + sizeof(pb_sample_detail) + 15) / 16 * 16;
static_assert(kOutErr + sizeof(pb_inference_error) <= kOutDetail, "error record overlaps");
static_assert(kInSmall % 16 == 0 && kInHist % 16 == 0, "history ids must stay 16-byte aligned");

// Grows a device workspace to `bytes` (never shrinks it).  Only set-up calls
// (pb_context_create, pb_context_reserve) use it.  The outgrown buffer is not
// freed but kept on `retired` until the context is destroyed: launches
// already enqueued, and HIP graphs captured earlier, keep its address.
static hipError_t grow_device(void** buf, size_t* have, size_t bytes,
                              std::vector<void*>* retired) {
  if (bytes <= *have) return hipSuccess;
  void* fresh = nullptr;
  hipError_t e = hipMalloc(&fresh, bytes);
  if (e != hipSuccess) return e;
  if (*buf) retired->push_back(*buf);
  *buf = fresh;
  *have = bytes;
  return hipSuccess;
}

// Slice workspace of `slots` (row, slice) pairs: 20 keys and 2 words each.
static size_t slice_workspace_bytes(size_t slots) { return slots * (PB_TOP_K * 8 + 8); }

// Largest rows x slices a batch of up to `rows` rows uses under the slice
// plan (forced slices, or the automatic plan, which uses one slice per row
// from 256 rows on and needs no workspace there).
static size_t max_slots(uint32_t rows, uint32_t forced_segments) {
  size_t best = 0;
  const uint32_t top = forced_segments ? rows : (rows < 256u ? rows : 255u);
  const uint32_t from = forced_segments ? rows : 1u;
  for (uint32_t r = from; r <= top && r > 0; ++r) {
    uint32_t segs = 0, seg_f4 = 0;
    pb::plan_segments(r, forced_segments, &segs, &seg_f4);
    if (segs > 1 && (size_t)r * segs > best) best = (size_t)r * segs;
  }
  return best;
}

// Batched sampler workspace for batches of up to `rows` rows: the slice
// plan's lists, or the tile words of the small batches that take the LM
// head's selection (the same region).
static size_t sample_workspace_bytes(uint32_t rows, uint32_t forced_segments) {
  const size_t slices = slice_workspace_bytes(max_slots(rows, forced_segments));
  const size_t tiles =
      forced_segments ? 0 : (size_t)(rows < pb::kTileSelectRows ? rows : pb::kTileSelectRows) *
                                pb::kTileSelectBytesPerRow;
  return slices > tiles ? slices : tiles;
}

// Fused LM head workspace for `rows` rows of `cols` columns (either format):
// the Q8_0 activations and their scales, the tile maxima and second words and, unless the
// caller keeps them, the logits.
struct LmLayout {
  size_t act_q, act_s, tilemax, tilesec, logits, total;
};
static LmLayout lm_layout(uint32_t rows, size_t cols, bool with_logits) {
  auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
  const size_t rows_pad = ((size_t)rows + 63u) & ~(size_t)63u;
  const size_t blocks = cols / 32;
  LmLayout l;
  l.act_q = 0;
  l.act_s = l.act_q + align(blocks * rows_pad * 32);
  l.tilemax = l.act_s + align(blocks * rows_pad * 4);
  l.tilesec = l.tilemax + align((size_t)rows * (PB_VOCAB / 64) * 4);
  l.logits = l.tilesec + align((size_t)rows * (PB_VOCAB / 64) * 4);
  l.total = l.logits + (with_logits ? align((size_t)rows * PB_VOCAB * 4) : 0);
  return l;
}
static size_t lm_workspace_bytes(uint32_t rows, size_t cols, bool with_logits) {
  return lm_layout(rows, cols, with_logits).total;
}
// Workspace that every step of up to `rows` rows fits in: the logits only
// for the narrow steps (up to kNarrowRows rows without a logits buffer from
// the caller), which keep them there; a wider step keeps none (one pass) and
// any step given a logits buffer writes the caller's.  At 256 rows of width
// 896 that is 40.2 MB instead of 160.7 MB.
static size_t lm_reserve_bytes(uint32_t rows, size_t cols) {
  const size_t wide = lm_workspace_bytes(rows, cols, false);
  const size_t narrow =
      lm_workspace_bytes(rows < pb::kNarrowRows ? rows : pb::kNarrowRows, cols, true);
  return wide > narrow ? wide : narrow;
}

static void free_staging(pb_context* ctx) {
  if (ctx->d_in) (void)hipFree(ctx->d_in);
  if (ctx->d_out) (void)hipFree(ctx->d_out);
  if (ctx->h_in) (void)hipHostFree(ctx->h_in);
  if (ctx->h_out) (void)hipHostFree(ctx->h_out);
  ctx->d_in = ctx->d_out = ctx->h_in = ctx->h_out = ctx->z_in = ctx->z_out = nullptr;
  ctx->hist_cap = 0;
}

// Pinned staging that kernels read and write in place: coherent, so that no
// GPU cache holds a previous call's bytes and the host sees a kernel's
// stores once the stream has synchronised.
constexpr unsigned kMappedFlags = hipHostMallocMapped | hipHostMallocCoherent;

// Staging regions for histories of up to `ids` ids.  The drop-ins hold the
// context's lock and synchronise before they return, so no copy or launch
// still uses the old regions when they are freed.
static hipError_t ensure_staging(pb_context* ctx, size_t ids) {
  if (ctx->d_in && ids <= ctx->hist_cap) return hipSuccess;
  size_t cap = ctx->hist_cap ? ctx->hist_cap : 1024;
  while (cap < ids) cap *= 2;
  free_staging(ctx);
  const size_t in_bytes = kInHist + cap * 4, out_bytes = kOutGather + cap * 4;
  hipError_t e;
  if ((e = hipMalloc(&ctx->d_in, in_bytes)) != hipSuccess ||
      (e = hipMalloc(&ctx->d_out, out_bytes)) != hipSuccess ||
      (e = hipHostMalloc(&ctx->h_in, in_bytes, kMappedFlags)) != hipSuccess ||
      (e = hipHostMalloc(&ctx->h_out, out_bytes, kMappedFlags)) != hipSuccess ||
      (e = hipHostGetDevicePointer(reinterpret_cast<void**>(&ctx->z_in), ctx->h_in, 0)) !=
          hipSuccess ||
      (e = hipHostGetDevicePointer(reinterpret_cast<void**>(&ctx->z_out), ctx->h_out, 0)) !=
          hipSuccess) {
    free_staging(ctx);
    return e;
  }
  ctx->hist_cap = cap;
  ctx->d_small = reinterpret_cast<uint32_t*>(ctx->d_in + kInSmall);
  ctx->d_row = reinterpret_cast<uint32_t*>(ctx->d_in + kInRow);
  ctx->d_hist = reinterpret_cast<uint32_t*>(ctx->d_in + kInHist);
  ctx->h_small = reinterpret_cast<uint32_t*>(ctx->h_in + kInSmall);
  ctx->h_row = reinterpret_cast<uint32_t*>(ctx->h_in + kInRow);
  ctx->h_hist = reinterpret_cast<uint32_t*>(ctx->h_in + kInHist);
  ctx->h_token = reinterpret_cast<uint32_t*>(ctx->h_out);
  ctx->h_err = reinterpret_cast<pb_inference_error*>(ctx->h_out + kOutErr);
  ctx->h_detail = reinterpret_cast<pb_sample_detail*>(ctx->h_out + kOutDetail);
  ctx->h_gather = reinterpret_cast<uint32_t*>(ctx->h_out + kOutGather);
  return hipSuccess;
}

static void release(pb_context* ctx) {
  if (!ctx) return;
  DeviceGuard guard(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  free_staging(ctx);
  void* dev[] = {ctx->d_work, ctx->d_lm, ctx->d_seen};
  for (void* p : dev)
    if (p) (void)hipFree(p);
  for (void* p : ctx->retired) (void)hipFree(p);
  if (ctx->h_seen) (void)hipHostFree(ctx->h_seen);
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

extern "C" {

// ---- PRNG: xorshift64* with draw counter (inference.rs:779-810) ----

void pb_sampling_state_new(pb_sampling_state* state, uint64_t seed) {
  state->state = seed == 0 ? 0x9e3779b97f4a7c15ull : seed;
  state->draws = 0;
}

uint32_t pb_next_24(pb_sampling_state* state) {
  uint64_t v = state->state;
  v ^= v >> 12;
  v ^= v << 25;
  v ^= v >> 27;
  state->state = v;
  state->draws += 1;
  return (uint32_t)((v * 0x2545f4914f6cdd1dull) >> 40);
}

void pb_fill_random_24(pb_sampling_state* states, uint32_t rows, uint32_t* out) {
  for (uint32_t r = 0; r < rows; ++r) out[r] = pb_next_24(&states[r]);
}

// PB_SOURCE_HASH (set by the Makefile) identifies the sources the library was
// built from, so a measurement recorded against one build can be told apart
// from another build's.
#ifndef PB_SOURCE_HASH
#define PB_SOURCE_HASH "unknown"
#endif
const char* pb_version(void) { return "pbsample 0.2 src:" PB_SOURCE_HASH " gfx950"; }

uint32_t pb_segments_for_rows(uint32_t rows) {
  uint32_t segs = 0, seg_f4 = 0;
  pb::plan_segments(rows, 0, &segs, &seg_f4);
  return segs;
}

void pb_context_set_segments(pb_context* ctx, uint32_t segments) {
  ctx->forced_segments = segments > 32 ? 32 : segments;
}

uint32_t pb_device_expf_bits(const uint32_t* d_in, uint32_t* d_out, size_t n, void* stream) {
  return pb::launch_probe(0, d_in, d_out, n, static_cast<hipStream_t>(stream)) == hipSuccess
             ? PB_OK
             : PB_DEVICE;
}

uint32_t pb_device_penalize_bits(const uint32_t* d_in, uint32_t* d_out, size_t n, void* stream) {
  return pb::launch_probe(1, d_in, d_out, n, static_cast<hipStream_t>(stream)) == hipSuccess
             ? PB_OK
             : PB_DEVICE;
}

uint32_t pb_device_wave_selftest(uint32_t* d_out, void* stream) {
  return pb::launch_wave_selftest(d_out, static_cast<hipStream_t>(stream)) == hipSuccess
             ? PB_OK
             : PB_DEVICE;
}

uint32_t pb_device_read_probe(const uint32_t* d_in, size_t n_words, uint32_t* d_out,
                              uint32_t blocks, void* stream) {
  if (((uintptr_t)d_in & 15u) != 0) return PB_ALIGNMENT;
  return pb::launch_read_probe(d_in, n_words, d_out, blocks, false,
                               static_cast<hipStream_t>(stream)) == hipSuccess
             ? PB_OK
             : PB_DEVICE;
}

uint32_t pb_device_read_probe_grid_stride(const uint32_t* d_in, size_t n_words, uint32_t* d_out,
                                          uint32_t blocks, void* stream) {
  if (((uintptr_t)d_in & 15u) != 0) return PB_ALIGNMENT;
  return pb::launch_read_probe(d_in, n_words, d_out, blocks, true,
                               static_cast<hipStream_t>(stream)) == hipSuccess
             ? PB_OK
             : PB_DEVICE;
}

uint32_t pb_context_create(int device, pb_context** out) {
  *out = nullptr;
  if (device < 0 && hipGetDevice(&device) != hipSuccess) return PB_DEVICE;
  DeviceGuard guard(device);
  pb_context* ctx = new pb_context();
  ctx->device = device;
  hipError_t e = hipSuccess;
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipMalloc(&ctx->d_seen, PB_SEEN_BYTES);
  if (e == hipSuccess) e = hipHostMalloc(&ctx->h_seen, PB_SEEN_BYTES, hipHostMallocDefault);
  // the drop-ins' staging for a whole context, and the slice workspace of
  // the automatic plan for any batch
  if (e == hipSuccess) e = ensure_staging(ctx, PB_CONTEXT_IDS);
  if (e == hipSuccess)
    e = grow_device(&ctx->d_work, &ctx->list_bytes, sample_workspace_bytes(255, 0),
                    &ctx->retired);
  // the device address of pb_sample_batch_noalloc's static scratch, once per device
  void* scratch = nullptr;
  if (e == hipSuccess) e = pb::static_scratch_address(device, &scratch);
  // the batch size from which rows run longest history first, once per device
  uint32_t resident = 0;
  if (e == hipSuccess) e = pb::resident_rows(device, &resident);
  if (e != hipSuccess) {
    release(ctx);
    return PB_DEVICE;
  }
  *out = ctx;
  return PB_OK;
}

void pb_context_destroy(pb_context* ctx) { release(ctx); }

uint32_t pb_context_reserve(pb_context* ctx, uint32_t rows, size_t cols, pb_inference_error* err) {
  clear_error(err);
  if (cols != 0 && (cols % 32 != 0 || cols > 2048)) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_NONE, 32, cols, PB_FIELD_BYTES, 4);
    return PB_CAPACITY;
  }
  if (cols != 0 && rows > PB_LMHEAD_MAX_ROWS) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_NONE, PB_LMHEAD_MAX_ROWS, rows, PB_FIELD_BYTES, 8);
    return PB_CAPACITY;
  }
  std::lock_guard<std::mutex> lock(ctx->mu);
  DeviceGuard guard(ctx->device);
  hipError_t e = grow_device(&ctx->d_work, &ctx->list_bytes,
                             sample_workspace_bytes(rows, ctx->forced_segments), &ctx->retired);
  if (e == hipSuccess && cols != 0 && rows != 0)
    e = grow_device(&ctx->d_lm, &ctx->lm_bytes, lm_reserve_bytes(rows, cols), &ctx->retired);
  return e == hipSuccess ? PB_OK : device_error(err, e);
}

}  // extern "C"

// Decode-loop arguments of pb_decode_step / pb_lmhead_decode_step.
struct DecodeArgs {
  uint32_t* hist;
  uint32_t* hist_len;
  const uint32_t* max_len;
  uint32_t* row_state;
};

static void set_decode(pb::RowParams& p, const DecodeArgs* dec) {
  p.row_state = dec ? dec->row_state : nullptr;
  p.hist_out = dec ? dec->hist : nullptr;
  p.hist_len_out = dec ? dec->hist_len : nullptr;
  p.max_len = dec ? dec->max_len : nullptr;
}

static bool decode_args_ok(const DecodeArgs& dec, pb_inference_error* err) {
  if (dec.hist == nullptr || dec.hist_len == nullptr || dec.row_state == nullptr) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_ARGMAX, 1, 0, PB_FIELD_BYTES, 5);
    return false;
  }
  return true;
}

// Validates and enqueues one batched sample (every variant) with the slice
// workspace `work` of `work_bytes` bytes.  Never allocates: a plan that
// needs more workspace than that is refused with PB_CAPACITY.
// A single-row drop-in's inputs still in mapped pinned memory: the tile-words
// launch reads the row at `row` and stores it at d_logits, and copies v4
// 16-byte groups from src to dst (the scalars and the history ids); the
// select kernel writes the history's penalised logits to `gather`.
struct StagedInput {
  const uint32_t* row;
  const uint32_t* src;
  uint32_t* dst;
  uint32_t v4;
  uint32_t* gather;  // the penalised logits at the history ids (the write-back), or null
};

static uint32_t enqueue_sample_in(int device, uint32_t forced_segments, void* work,
                                  size_t work_bytes, const uint32_t* d_logits, size_t vocab,
                                  size_t ld, uint32_t rows, const uint32_t* d_hist,
                                  size_t hist_ld, const uint32_t* d_hist_len,
                                  const uint32_t* d_random_24, const uint8_t* d_excl,
                                  uint32_t* d_token, pb_sample_detail* d_detail,
                                  pb_inference_error* d_err, hipStream_t stream,
                                  pb_inference_error* err, const DecodeArgs* dec = nullptr,
                                  const StagedInput* staged = nullptr) {
  clear_error(err);
  if (vocab != PB_VOCAB) {
    // logits_error (inference.rs:737-754)
    set_error(err, PB_CAPACITY, PB_DOMAIN_LOGITS, PB_VOCAB, vocab, PB_FIELD_LOGITS, 0);
    return PB_CAPACITY;
  }
  if (ld < vocab) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_LOGITS, vocab, ld, PB_FIELD_LOGITS, 1);
    return PB_CAPACITY;
  }
  if ((ld & 3u) != 0 || ((uintptr_t)d_logits & 15u) != 0) {
    set_error(err, PB_ALIGNMENT, PB_DOMAIN_LOGITS, 16, ((uintptr_t)d_logits & 15u) | (ld & 3u),
              PB_FIELD_ALIGNMENT, 0);
    return PB_ALIGNMENT;
  }
  if (rows == 0) return PB_OK;
  if (d_logits == nullptr || d_random_24 == nullptr || d_token == nullptr ||
      (d_hist_len != nullptr && d_hist == nullptr)) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_ARGMAX, 1, 0, PB_FIELD_BYTES, 3);
    return PB_CAPACITY;
  }
  pb::RowParams p{};
  p.logits = d_logits;
  p.ld = ld;
  p.rows = rows;
  p.hist = d_hist_len ? d_hist : nullptr;
  p.hist_ld = hist_ld;
  p.hist_len = d_hist_len;
  p.excl = d_excl;
  p.random_24 = d_random_24;
  p.token = d_token;
  p.detail = d_detail;
  p.err = d_err;
  p.hist_vec4 = (p.hist != nullptr && hist_ld >= 4u && (hist_ld & 3u) == 0 &&
                 ((uintptr_t)d_hist & 15u) == 0);
  set_decode(p, dec);
  // Small batches (no `seen` exclusion, the automatic plan): the tile words
  // of the logits, then the LM head's selection, when the workspace holds
  // the words.
  if (forced_segments == 0 && d_excl == nullptr && rows <= pb::kTileSelectRows &&
      work != nullptr && work_bytes >= rows * pb::kTileSelectBytesPerRow) {
    pb::LmParams lp{};
    lp.logits = const_cast<uint32_t*>(d_logits);  // read only
    lp.logits_ld = ld;
    lp.rows = rows;
    lp.tilemax = static_cast<uint32_t*>(work);
    lp.tilesec = lp.tilemax + (size_t)rows * (PB_VOCAB / 64);
    if (staged) {
      lp.logits = const_cast<uint32_t*>(staged->row);  // read only
      lp.logits_copy = const_cast<uint32_t*>(d_logits);
      lp.stage_src = staged->src;
      lp.stage_dst = staged->dst;
      lp.stage_v4 = staged->v4;
      p.gather = staged->gather;
    }
    p.segs = 1;
    DeviceGuard guard(device);
    hipError_t e = pb::launch_tile_select(lp, p, stream);
    return e == hipSuccess ? PB_OK : device_error(err, e);
  }
  if (staged) {  // only the tile selection copies staged inputs
    set_error(err, PB_STATE, PB_DOMAIN_NONE, 2, 0, PB_FIELD_NONE, 0);
    return PB_STATE;
  }
  pb::plan_segments(rows, forced_segments, &p.segs, &p.seg_f4);
  p.part_keys = nullptr;
  p.part_meta = nullptr;
  if (p.segs > 1) {
    const size_t slots = (size_t)rows * p.segs;
    const size_t need = slice_workspace_bytes(slots);
    if (need > work_bytes || work == nullptr) {
      set_error(err, PB_CAPACITY, PB_DOMAIN_NONE, need, work_bytes, PB_FIELD_BYTES, 6);
      return PB_CAPACITY;
    }
    char* base = static_cast<char*>(work);
    p.part_keys = reinterpret_cast<uint64_t*>(base);
    p.part_meta = reinterpret_cast<uint32_t*>(base + slots * PB_TOP_K * 8);
  }
  DeviceGuard guard(device);
  pb::plan_row_order(device, &p);
  hipError_t e = pb::launch_sample(p, stream);
  if (e != hipSuccess) return device_error(err, e);
  return PB_OK;
}

// enqueue_sample_in on the context's own workspace.  The arguments are
// checked before the context is touched; then the context's lock is taken
// unless the caller (a drop-in) already holds it.
struct Workspace {
  void* base;
  size_t bytes;
};

static uint32_t enqueue_sample(pb_context* ctx, const uint32_t* d_logits, size_t vocab, size_t ld,
                               uint32_t rows, const uint32_t* d_hist, size_t hist_ld,
                               const uint32_t* d_hist_len, const uint32_t* d_random_24,
                               const uint8_t* d_excl, uint32_t* d_token,
                               pb_sample_detail* d_detail, pb_inference_error* d_err,
                               hipStream_t stream, pb_inference_error* err,
                               const DecodeArgs* dec = nullptr, bool locked = false,
                               const Workspace* ws = nullptr,
                               const StagedInput* staged = nullptr) {
  uint32_t st = enqueue_sample_in(-1, 0, nullptr, 0, d_logits, vocab, ld, 0, d_hist, hist_ld,
                                  d_hist_len, d_random_24, d_excl, d_token, d_detail, d_err,
                                  stream, err, dec);
  if (st != PB_OK || rows == 0) return st;
  if (d_logits == nullptr || d_random_24 == nullptr || d_token == nullptr ||
      (d_hist_len != nullptr && d_hist == nullptr)) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_ARGMAX, 1, 0, PB_FIELD_BYTES, 3);
    return PB_CAPACITY;
  }
  if (ctx == nullptr) {
    set_error(err, PB_STATE, PB_DOMAIN_NONE, 1, 0, PB_FIELD_NONE, 0);
    return PB_STATE;
  }
  std::unique_lock<std::mutex> lock(ctx->mu, std::defer_lock);
  if (!locked) lock.lock();
  void* work = ws ? ws->base : ctx->d_work;
  const size_t work_bytes = ws ? ws->bytes : ctx->list_bytes;
  return enqueue_sample_in(ctx->device, ctx->forced_segments, work, work_bytes, d_logits, vocab,
                           ld, rows, d_hist, hist_ld, d_hist_len, d_random_24, d_excl, d_token,
                           d_detail, d_err, stream, err, dec, staged);
}

namespace pb {

int context_device(const pb_context* ctx) { return ctx->device; }

uint32_t enqueue_sample_with_workspace(pb_context* ctx, void* work, size_t work_bytes,
                                       const uint32_t* d_logits, size_t vocab, size_t ld,
                                       uint32_t rows, const uint32_t* d_hist, size_t hist_ld,
                                       const uint32_t* d_hist_len, const uint32_t* d_random_24,
                                       uint32_t* d_token, pb_sample_detail* d_detail,
                                       pb_inference_error* d_err, hipStream_t stream,
                                       pb_inference_error* err) {
  const Workspace ws{work, work_bytes};
  return enqueue_sample(ctx, d_logits, vocab, ld, rows, d_hist, hist_ld, d_hist_len, d_random_24,
                        nullptr, d_token, d_detail, d_err, stream, err, nullptr, false, &ws);
}

}  // namespace pb

extern "C" {

uint32_t pb_sample_batch(pb_context* ctx, const uint32_t* d_logits, size_t vocab, size_t ld,
                         uint32_t rows, const uint32_t* d_hist, size_t hist_ld,
                         const uint32_t* d_hist_len, const uint32_t* d_random_24,
                         uint32_t* d_token, pb_sample_detail* d_detail,
                         pb_inference_error* d_err, void* stream, pb_inference_error* err) {
  return enqueue_sample(ctx, d_logits, vocab, ld, rows, d_hist, hist_ld, d_hist_len, d_random_24,
                        nullptr, d_token, d_detail, d_err, static_cast<hipStream_t>(stream), err);
}

uint32_t pb_sample_batch_inplace(pb_context* ctx, uint32_t* d_logits, size_t vocab, size_t ld,
                                 uint32_t rows, const uint32_t* d_hist, size_t hist_ld,
                                 const uint32_t* d_hist_len, const uint32_t* d_random_24,
                                 uint8_t* d_seen, uint32_t* d_token,
                                 pb_sample_detail* d_detail, pb_inference_error* d_err,
                                 void* stream, pb_inference_error* err) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (ctx == nullptr)  // the arguments are checked first, then the context is refused
    return enqueue_sample(nullptr, d_logits, vocab, ld, rows, d_hist, hist_ld, d_hist_len,
                          d_random_24, d_seen, d_token, d_detail, d_err, s, err);
  // Both launches go out under one hold of the context's lock: no other
  // call on this context lands between them.
  std::lock_guard<std::mutex> lock(ctx->mu);
  uint32_t st = enqueue_sample(ctx, d_logits, vocab, ld, rows, d_hist, hist_ld, d_hist_len,
                               d_random_24, d_seen, d_token, d_detail, d_err, s, err, nullptr,
                               true);
  if (st != PB_OK || rows == 0 || d_hist_len == nullptr) return st;
  pb::WritebackParams w;
  w.logits = d_logits;
  w.ld = ld;
  w.rows = rows;
  w.hist = d_hist;
  w.hist_ld = hist_ld;
  w.hist_len = d_hist_len;
  w.seen = d_seen;
  w.token = d_token;
  w.gather = nullptr;
  DeviceGuard guard(ctx->device);
  hipError_t e = pb::launch_writeback(w, s);
  if (e != hipSuccess) return device_error(err, e);
  return PB_OK;
}

// ---- fused Q4_0 LM head + sampler ----

// The Q4_0 layout ends with one flag word per 64-id tile (a tile with an
// infinite or NaN weight scale).
size_t pb_lmhead_packed_bytes(size_t vocab, size_t cols) {
  return vocab * (cols / 32) * 18 + vocab / 64 * 4;
}

size_t pb_lmhead_q8_packed_bytes(size_t vocab, size_t cols) { return vocab * (cols / 32) * 34; }

}  // extern "C"

// Argument checks shared by the Q4_0 and Q8_0 repacks.
static uint32_t check_pack_args(size_t vocab, size_t cols, const uint8_t* d_packed,
                                pb_inference_error* err) {
  clear_error(err);
  if (cols == 0 || cols % 32 != 0) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_NONE, 32, cols, PB_FIELD_BYTES, 4);
    return PB_CAPACITY;
  }
  // the device layout groups the vocabulary in tiles of 64 ids
  if (vocab == 0 || vocab % 64 != 0 || vocab > 0xffffffffu) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_LOGITS, 64, vocab, PB_FIELD_LOGITS, 1);
    return PB_CAPACITY;
  }
  if (((uintptr_t)d_packed & 15u) != 0) {
    set_error(err, PB_ALIGNMENT, PB_DOMAIN_NONE, 16, (uintptr_t)d_packed & 15u,
              PB_FIELD_ALIGNMENT, 1);
    return PB_ALIGNMENT;
  }
  return PB_OK;
}

extern "C" {

uint32_t pb_lmhead_pack_q4_0(const uint8_t* d_q4, size_t vocab, size_t cols, uint8_t* d_packed,
                             void* stream, pb_inference_error* err) {
  const uint32_t st = check_pack_args(vocab, cols, d_packed, err);
  if (st != PB_OK) return st;
  hipError_t e = pb::launch_lm_pack(d_q4, d_packed, (uint32_t)vocab, (uint32_t)(cols / 32),
                                    static_cast<hipStream_t>(stream));
  return e == hipSuccess ? PB_OK : device_error(err, e);
}

uint32_t pb_lmhead_pack_q8_0(const uint8_t* d_q8, size_t vocab, size_t cols, uint8_t* d_packed,
                             void* stream, pb_inference_error* err) {
  const uint32_t st = check_pack_args(vocab, cols, d_packed, err);
  if (st != PB_OK) return st;
  hipError_t e = pb::launch_lm_pack_q8(d_q8, d_packed, (uint32_t)vocab, (uint32_t)(cols / 32),
                                       static_cast<hipStream_t>(stream));
  return e == hipSuccess ? PB_OK : device_error(err, e);
}

}  // extern "C"

static uint32_t enqueue_lmhead(pb_context* ctx, const uint8_t* d_packed, size_t packed_bytes,
                               size_t vocab, size_t cols, const uint32_t* d_hidden, uint32_t rows,
                               const uint32_t* d_hist, size_t hist_ld,
                               const uint32_t* d_hist_len, const uint32_t* d_random_24,
                               uint32_t* d_token, pb_sample_detail* d_detail,
                               pb_inference_error* d_err, uint32_t* d_logits, void* stream,
                               pb_inference_error* err, const DecodeArgs* dec, bool q8) {
  clear_error(err);
  if (vocab != PB_VOCAB) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_LOGITS, PB_VOCAB, vocab, PB_FIELD_LOGITS, 0);
    return PB_CAPACITY;
  }
  // The wide head keeps every block's scales (a tile's weight scales and a
  // 128-row group's activation scales) in 64 KB of LDS at 2,048 columns, and
  // the selection stages a row's activations for up to 64 blocks: up to
  // 2,048 columns (Qwen2.5-0.5B has 896).
  if (cols == 0 || cols % 32 != 0 || cols > 2048) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_NONE, 32, cols, PB_FIELD_BYTES, 4);
    return PB_CAPACITY;
  }
  // the head must have been packed for this width and format
  const size_t want = q8 ? pb_lmhead_q8_packed_bytes(vocab, cols) : pb_lmhead_packed_bytes(vocab, cols);
  if (packed_bytes != want) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_NONE, want, packed_bytes, PB_FIELD_BYTES, 7);
    return PB_CAPACITY;
  }
  if (((uintptr_t)d_packed & 15u) != 0 || ((uintptr_t)d_logits & 15u) != 0 ||
      ((uintptr_t)d_hidden & 15u) != 0) {
    set_error(err, PB_ALIGNMENT, PB_DOMAIN_NONE, 16, 0, PB_FIELD_ALIGNMENT, 2);
    return PB_ALIGNMENT;
  }
  if (rows == 0) return PB_OK;
  // the kernels' 32-bit offsets into the quantised activations
  if (rows > PB_LMHEAD_MAX_ROWS) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_NONE, PB_LMHEAD_MAX_ROWS, rows, PB_FIELD_BYTES, 8);
    return PB_CAPACITY;
  }
  if (d_packed == nullptr || d_hidden == nullptr || d_random_24 == nullptr ||
      d_token == nullptr || (d_hist_len != nullptr && d_hist == nullptr)) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_ARGMAX, 1, 0, PB_FIELD_BYTES, 3);
    return PB_CAPACITY;
  }
  const uint32_t rows_pad = (rows + 63u) & ~63u;
  std::lock_guard<std::mutex> lock(ctx->mu);
  // Above kNarrowRows rows without a logits buffer the step is one pass: the
  // wide GEMM writes only the tile and second words, and the selection
  // recomputes the few tiles it reads from the packed head.  Narrow batches
  // keep their logits in the workspace (0.6 MB per row against the head's
  // 76.6 MB) and the selection reads them.
  const bool one_pass = d_logits == nullptr && rows > pb::kNarrowRows;
  const LmLayout lay = lm_layout(rows, cols, d_logits == nullptr && !one_pass);
  const size_t need = lay.total;
  if (need > ctx->lm_bytes) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_NONE, need, ctx->lm_bytes, PB_FIELD_BYTES, 6);
    return PB_CAPACITY;
  }
  DeviceGuard guard(ctx->device);
  char* base = static_cast<char*>(ctx->d_lm);
  pb::LmParams p{};
  p.weights = d_packed;
  p.q8 = q8;
  p.hidden = d_hidden;
  p.rows = rows;
  p.rows_pad = rows_pad;
  p.cols = (uint32_t)cols;
  p.fused_quant = rows <= pb::kFusedQuantRows;
  p.act_q = reinterpret_cast<int8_t*>(base + lay.act_q);
  p.act_s = reinterpret_cast<float*>(base + lay.act_s);
  p.tilemax = reinterpret_cast<uint32_t*>(base + lay.tilemax);
  p.tilesec = rows <= pb::kNarrowRows || one_pass ? reinterpret_cast<uint32_t*>(base + lay.tilesec)
                                                 : nullptr;
  p.logits = d_logits ? d_logits : one_pass ? nullptr : reinterpret_cast<uint32_t*>(base + lay.logits);
  p.logits_ld = PB_VOCAB;

  pb::RowParams rp;
  memset(&rp, 0, sizeof rp);
  rp.logits = p.logits;
  rp.ld = PB_VOCAB;
  rp.rows = rows;
  rp.hist = d_hist_len ? d_hist : nullptr;
  rp.hist_ld = hist_ld;
  rp.hist_len = d_hist_len;
  rp.hist_vec4 = (rp.hist != nullptr && hist_ld >= 4u && (hist_ld & 3u) == 0 &&
                  ((uintptr_t)d_hist & 15u) == 0);
  rp.random_24 = d_random_24;
  rp.token = d_token;
  rp.detail = d_detail;
  rp.err = d_err;
  rp.segs = 1;
  set_decode(rp, dec);
  hipError_t e = pb::launch_lm_sample(p, rp, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? PB_OK : device_error(err, e);
}

extern "C" {

uint32_t pb_lmhead_sample_batch(pb_context* ctx, const uint8_t* d_packed, size_t packed_bytes,
                                size_t vocab, size_t cols, const uint32_t* d_hidden, uint32_t rows,
                                const uint32_t* d_hist, size_t hist_ld,
                                const uint32_t* d_hist_len, const uint32_t* d_random_24,
                                uint32_t* d_token, pb_sample_detail* d_detail,
                                pb_inference_error* d_err, uint32_t* d_logits, void* stream,
                                pb_inference_error* err) {
  return enqueue_lmhead(ctx, d_packed, packed_bytes, vocab, cols, d_hidden, rows, d_hist, hist_ld, d_hist_len,
                        d_random_24, d_token, d_detail, d_err, d_logits, stream, err, nullptr,
                        false);
}

uint32_t pb_lmhead_q8_sample_batch(pb_context* ctx, const uint8_t* d_packed,
                                   size_t packed_bytes, size_t vocab, size_t cols, const uint32_t* d_hidden, uint32_t rows,
                                   const uint32_t* d_hist, size_t hist_ld,
                                   const uint32_t* d_hist_len, const uint32_t* d_random_24,
                                   uint32_t* d_token, pb_sample_detail* d_detail,
                                   pb_inference_error* d_err, uint32_t* d_logits, void* stream,
                                   pb_inference_error* err) {
  return enqueue_lmhead(ctx, d_packed, packed_bytes, vocab, cols, d_hidden, rows, d_hist, hist_ld, d_hist_len,
                        d_random_24, d_token, d_detail, d_err, d_logits, stream, err, nullptr,
                        true);
}

// ---- decode loop (src/model_repl.rs:928-1150) ----

uint32_t pb_decode_step(pb_context* ctx, const uint32_t* d_logits, size_t vocab, size_t ld,
                        uint32_t rows, uint32_t* d_hist, size_t hist_ld, uint32_t* d_hist_len,
                        const uint32_t* d_max_len, uint32_t* d_row_state,
                        const uint32_t* d_random_24, uint32_t* d_token,
                        pb_sample_detail* d_detail, pb_inference_error* d_err, void* stream,
                        pb_inference_error* err) {
  clear_error(err);
  const DecodeArgs dec{d_hist, d_hist_len, d_max_len, d_row_state};
  if (rows != 0 && !decode_args_ok(dec, err)) return PB_CAPACITY;
  return enqueue_sample(ctx, d_logits, vocab, ld, rows, d_hist, hist_ld, d_hist_len, d_random_24,
                        nullptr, d_token, d_detail, d_err, static_cast<hipStream_t>(stream), err,
                        &dec);
}

uint32_t pb_lmhead_decode_step(pb_context* ctx, const uint8_t* d_packed, size_t packed_bytes,
                               size_t vocab, size_t cols, const uint32_t* d_hidden, uint32_t rows,
                               uint32_t* d_hist, size_t hist_ld, uint32_t* d_hist_len,
                               const uint32_t* d_max_len, uint32_t* d_row_state,
                               const uint32_t* d_random_24, uint32_t* d_token,
                               pb_sample_detail* d_detail, pb_inference_error* d_err,
                               uint32_t* d_logits, void* stream, pb_inference_error* err) {
  clear_error(err);
  const DecodeArgs dec{d_hist, d_hist_len, d_max_len, d_row_state};
  if (rows != 0 && !decode_args_ok(dec, err)) return PB_CAPACITY;
  return enqueue_lmhead(ctx, d_packed, packed_bytes, vocab, cols, d_hidden, rows, d_hist, hist_ld, d_hist_len,
                        d_random_24, d_token, d_detail, d_err, d_logits, stream, err, &dec, false);
}

uint32_t pb_lmhead_q8_decode_step(pb_context* ctx, const uint8_t* d_packed,
                                  size_t packed_bytes, size_t vocab, size_t cols, const uint32_t* d_hidden, uint32_t rows,
                                  uint32_t* d_hist, size_t hist_ld, uint32_t* d_hist_len,
                                  const uint32_t* d_max_len, uint32_t* d_row_state,
                                  const uint32_t* d_random_24, uint32_t* d_token,
                                  pb_sample_detail* d_detail, pb_inference_error* d_err,
                                  uint32_t* d_logits, void* stream, pb_inference_error* err) {
  clear_error(err);
  const DecodeArgs dec{d_hist, d_hist_len, d_max_len, d_row_state};
  if (rows != 0 && !decode_args_ok(dec, err)) return PB_CAPACITY;
  return enqueue_lmhead(ctx, d_packed, packed_bytes, vocab, cols, d_hidden, rows, d_hist, hist_ld, d_hist_len,
                        d_random_24, d_token, d_detail, d_err, d_logits, stream, err, &dec, true);
}

void pb_decode_draw(pb_sampling_state* states, const uint32_t* row_state, uint32_t rows,
                    uint32_t* out, pb_sampling_state* saved) {
  for (uint32_t r = 0; r < rows; ++r) {
    saved[r] = states[r];
    out[r] = row_state[r] == PB_ROW_ACTIVE ? pb_next_24(&states[r]) : 0u;
  }
}

uint32_t pb_decode_settle(pb_sampling_state* states, const pb_sampling_state* saved,
                          const uint32_t* state_before, const uint32_t* tokens, uint32_t rows) {
  uint32_t restored = 0;
  for (uint32_t r = 0; r < rows; ++r) {
    if (state_before[r] == PB_ROW_ACTIVE && tokens[r] == PB_NO_TOKEN) {
      states[r] = saved[r];
      ++restored;
    }
  }
  return restored;
}

uint32_t pb_device_mfma_selftest(int32_t* d_out, void* stream) {
  return pb::launch_mfma_selftest(d_out, static_cast<hipStream_t>(stream)) == hipSuccess
             ? PB_OK
             : PB_DEVICE;
}

}  // extern "C"

// ---- single-row drop-ins on the default context ----

static std::mutex g_contexts_mu;
static std::map<int, pb_context*> g_contexts;

static pb_context* default_context(pb_inference_error* err) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) {
    device_error(err, e);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_contexts_mu);
  auto it = g_contexts.find(device);
  if (it != g_contexts.end()) return it->second;
  pb_context* ctx = nullptr;
  if (pb_context_create(device, &ctx) != PB_OK) {
    set_error(err, PB_DEVICE, PB_DOMAIN_NONE, 0, 0, PB_FIELD_NONE, 1);
    return nullptr;
  }
  g_contexts[device] = ctx;
  return ctx;
}

enum RowMode { kSample = 0, kSampleWithHistory = 1 };

// Runs one row through the batched kernels on the context's own stream.
// Fills *ctx->h_token, ctx->h_detail and ctx->h_err; when `history` is
// non-null also the penalised write-back values in h_gather and, with
// `seen_dirty`, the updated scratch in h_seen.  Each copy on the stream costs
// several microseconds of latency, more than its bytes: without a dirty
// `seen` (and with the automatic plan) the call makes none and launches
// twice.  The tile-words launch reads the staged row, scalars and history
// from the mapped pinned region and leaves them in d_in; the select launch
// writes the token, records and the penalised history values into the mapped
// output region.  Otherwise the scalars, the row and the history go up in one
// copy, a write-back launch follows the selection and the results come back
// in one copy.
static uint32_t run_single_row(pb_context* ctx, const uint32_t* logits, const uint32_t* history,
                               size_t history_len, const uint8_t* seen, bool seen_dirty,
                               uint32_t random_24, pb_inference_error* err) {
  DeviceGuard guard(ctx->device);
  hipStream_t s = ctx->stream;
  hipError_t e;
  const bool with_hist = history != nullptr && history_len > 0;
  if (with_hist && (e = ensure_staging(ctx, history_len)) != hipSuccess)
    return device_error(err, e);
  const bool mapped = !(with_hist && seen_dirty) && ctx->forced_segments == 0;
  ctx->h_small[0] = (uint32_t)history_len;
  ctx->h_small[1] = random_24;
  memcpy(ctx->h_row, logits, kRowBytes);
  if (with_hist) memcpy(ctx->h_hist, history, history_len * 4);
  StagedInput staged{};
  if (mapped) {
    staged.row = reinterpret_cast<const uint32_t*>(ctx->z_in + kInRow);
    staged.src = reinterpret_cast<const uint32_t*>(ctx->z_in + kInSmall);
    staged.dst = ctx->d_small;
    staged.v4 = (uint32_t)((kInHist - kInSmall + (with_hist ? history_len * 4 : 0) + 15) / 16);
    staged.gather = with_hist ? reinterpret_cast<uint32_t*>(ctx->z_out + kOutGather) : nullptr;
  } else {
    const size_t in_bytes = kInHist + (with_hist ? history_len * 4 : 0);
    if ((e = hipMemcpyAsync(ctx->d_in, ctx->h_in, in_bytes, hipMemcpyHostToDevice, s)) !=
        hipSuccess)
      return device_error(err, e);
  }
  // Without history ids the scratch is returned as it came, so it stays on the host.
  if (with_hist && seen_dirty) {
    memcpy(ctx->h_seen, seen, PB_SEEN_BYTES);
    if ((e = hipMemcpyAsync(ctx->d_seen, ctx->h_seen, PB_SEEN_BYTES, hipMemcpyHostToDevice, s)) !=
        hipSuccess)
      return device_error(err, e);
  }

  uint8_t* out = mapped ? ctx->z_out : ctx->d_out;
  uint32_t* token = reinterpret_cast<uint32_t*>(out);
  uint8_t* seen_dev = with_hist && seen_dirty ? ctx->d_seen : nullptr;
  pb_inference_error enqueue_err;
  uint32_t st = enqueue_sample(
      ctx, ctx->d_row, PB_VOCAB, PB_VOCAB, 1, with_hist ? ctx->d_hist : nullptr, ctx->hist_cap,
      with_hist ? ctx->d_small : nullptr, ctx->d_small + 1, seen_dev, token,
      reinterpret_cast<pb_sample_detail*>(out + kOutDetail),
      reinterpret_cast<pb_inference_error*>(out + kOutErr), s, &enqueue_err, nullptr, true,
      nullptr, mapped ? &staged : nullptr);
  if (st != PB_OK) {
    if (err) *err = enqueue_err;
    return st;
  }
  if (with_hist && !mapped) {
    pb::WritebackParams w;
    w.logits = ctx->d_row;
    w.ld = PB_VOCAB;
    w.rows = 1;
    w.hist = ctx->d_hist;
    w.hist_ld = ctx->hist_cap;
    w.hist_len = ctx->d_small;
    w.seen = seen_dev;
    w.token = token;
    w.gather = reinterpret_cast<uint32_t*>(out + kOutGather);
    if ((e = pb::launch_writeback(w, s)) != hipSuccess) return device_error(err, e);
    if (seen_dirty &&
        (e = hipMemcpyAsync(ctx->h_seen, ctx->d_seen, PB_SEEN_BYTES, hipMemcpyDeviceToHost, s)) !=
            hipSuccess)
      return device_error(err, e);
  }
  if (!mapped) {
    const size_t out_bytes = kOutGather + (with_hist ? history_len * 4 : 0);
    if ((e = hipMemcpyAsync(ctx->h_out, ctx->d_out, out_bytes, hipMemcpyDeviceToHost, s)) !=
        hipSuccess)
      return device_error(err, e);
  }
  if ((e = hipStreamSynchronize(s)) != hipSuccess) return device_error(err, e);
  return PB_OK;
}

// OR of 8-byte words, which the compiler vectorises (a byte loop with an
// early exit does not vectorise: 11.5 us against 0.9 us for the 18,992-byte
// scratch on one host core).
static bool any_nonzero(const uint8_t* p, size_t n) {
  uint64_t acc = 0;
  size_t i = 0;
  for (; i + 8 <= n; i += 8) {
    uint64_t w;
    memcpy(&w, p + i, 8);
    acc |= w;
  }
  for (; i < n; ++i) acc |= p[i];
  return acc != 0;
}

extern "C" {

uint32_t pb_sample_token_with_repetition(uint32_t* logits, size_t logits_len,
                                         const uint32_t* tokens, size_t tokens_len,
                                         uint8_t* seen, size_t seen_len,
                                         pb_sampling_state* state, uint32_t* out_token,
                                         pb_inference_error* err) {
  clear_error(err);
  if (logits_len != PB_VOCAB) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_LOGITS, PB_VOCAB, logits_len, PB_FIELD_LOGITS, 0);
    return PB_CAPACITY;
  }
  pb_context* ctx = default_context(err);
  if (!ctx) return PB_DEVICE;
  std::lock_guard<std::mutex> lock(ctx->mu);
  const bool seen_ok = seen_len >= PB_SEEN_BYTES;
  const bool seen_dirty = seen_ok && any_nonzero(seen, PB_SEEN_BYTES);
  pb_sampling_state next = *state;
  const uint32_t r24 = pb_next_24(&next);
  // The history goes to the GPU even when `seen` is short: a non-finite logit
  // takes precedence over the scratch-length error (inference.rs:925-938).
  uint32_t st = run_single_row(ctx, logits, tokens, tokens_len, seen, seen_dirty, r24, err);
  if (st != PB_OK) return st;
  const pb_inference_error& row_err = *ctx->h_err;
  if (row_err.status == PB_NONFINITE_OUTPUT) {
    if (err) *err = row_err;
    return row_err.status;
  }
  if (!seen_ok) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_ARGMAX, PB_SEEN_BYTES, seen_len, PB_FIELD_BYTES, 2);
    return PB_CAPACITY;
  }
  if (row_err.status != PB_OK) {
    if (err) *err = row_err;
    return row_err.status;
  }
  // success: publish the in-place penalty, the cleared scratch and the draw
  // (a NULL history is an empty one, as in run_single_row)
  if (tokens != nullptr)
    for (size_t q = 0; q < tokens_len; ++q) logits[tokens[q]] = ctx->h_gather[q];
  if (seen_dirty && tokens != nullptr && tokens_len > 0) memcpy(seen, ctx->h_seen, PB_SEEN_BYTES);
  *state = next;
  *out_token = *ctx->h_token;
  return PB_OK;
}

uint32_t pb_sample_token(const uint32_t* logits, size_t logits_len, pb_sampling_state* state,
                         uint32_t* out_token, pb_inference_error* err) {
  clear_error(err);
  if (logits_len != PB_VOCAB) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_LOGITS, PB_VOCAB, logits_len, PB_FIELD_LOGITS, 0);
    return PB_CAPACITY;
  }
  pb_context* ctx = default_context(err);
  if (!ctx) return PB_DEVICE;
  std::lock_guard<std::mutex> lock(ctx->mu);
  pb_sampling_state next = *state;
  const uint32_t r24 = pb_next_24(&next);
  uint32_t st = run_single_row(ctx, logits, nullptr, 0, nullptr, false, r24, err);
  if (st != PB_OK) return st;
  if (ctx->h_err->status != PB_OK) {
    if (err) *err = *ctx->h_err;
    return ctx->h_err->status;
  }
  *state = next;
  *out_token = *ctx->h_token;
  return PB_OK;
}

uint32_t pb_greedy_token(const uint32_t* logits, size_t logits_len, uint32_t* out_token,
                         pb_inference_error* err) {
  clear_error(err);
  if (logits_len != PB_VOCAB) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_LOGITS, PB_VOCAB, logits_len, PB_FIELD_LOGITS, 0);
    return PB_CAPACITY;
  }
  pb_context* ctx = default_context(err);
  if (!ctx) return PB_DEVICE;
  std::lock_guard<std::mutex> lock(ctx->mu);
  uint32_t st = run_single_row(ctx, logits, nullptr, 0, nullptr, false, 0, err);
  if (st != PB_OK) return st;
  if (ctx->h_err->status != PB_OK) {
    if (err) *err = *ctx->h_err;
    return ctx->h_err->status;
  }
  *out_token = ctx->h_detail->ids[0];
  return PB_OK;
}

uint32_t pb_top_logits_8(const uint32_t* logits, size_t logits_len, pb_top_logit output[8],
                         pb_inference_error* err) {
  clear_error(err);
  if (logits_len != PB_VOCAB) {
    set_error(err, PB_CAPACITY, PB_DOMAIN_LOGITS, PB_VOCAB, logits_len, PB_FIELD_LOGITS, 0);
    return PB_CAPACITY;
  }
  pb_context* ctx = default_context(err);
  if (!ctx) return PB_DEVICE;
  std::lock_guard<std::mutex> lock(ctx->mu);
  uint32_t st = run_single_row(ctx, logits, nullptr, 0, nullptr, false, 0, err);
  if (st != PB_OK) return st;
  if (ctx->h_err->status != PB_OK) {
    if (err) *err = *ctx->h_err;
    return ctx->h_err->status;
  }
  for (int i = 0; i < 8; ++i) {
    output[i].token = ctx->h_detail->ids[i];
    output[i].logit_bits = ctx->h_detail->value_bits[i];
  }
  return PB_OK;
}

}  // extern "C"

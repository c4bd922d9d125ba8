// pb_static.hip -- pb_sample_batch_noalloc: the batched sampler with its
// workspace in a file-scope device array instead of memory the library
// allocates.
//
// The batched sampler passes intermediate results from its first launch to
// its second through a workspace: for batches of up to PB_TILE_SELECT_ROWS
// rows the tile words of every (row, 64-id tile) (tile_words_kernel, then
// lm_select_kernel), for the slice plan rows x slices records of each
// slice's top-20 keys and first-bad positions (segment_kernel, then
// finish_kernel).  This file keeps one such workspace per device in
// `scratch`, sized for the tile words of PB_TILE_SELECT_ROWS rows, which also
// holds the records of every batch of the automatic slice plan, so a caller
// that cannot allocate (code under HIP graph capture, a tight serving loop)
// takes the same paths as pb_sample_batch.  Nothing in it has to start at
// zero: the first launch writes every word the second reads.  Every call on
// one device, from any context, shares that device's array, so calls that
// overlap on the device race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "pb_internal.h"
#include "pbsample.h"

namespace {

// The tile words of PB_TILE_SELECT_ROWS rows: 192 x 2,374 x 8 = 3,646,464
// bytes.  The automatic slice plan cuts a batch of up to 255 rows into at
// most 1,024 (row, slice) records of 20 keys + 2 words (172,032 bytes) and
// from 256 rows on uses one slice per row and no workspace, so the array
// also holds every batch of the automatic plan; a forced plan may hold up to
// 21,705 records.
constexpr size_t kScratchBytes = (size_t)pb::kTileSelectRows * pb::kTileSelectBytesPerRow;
static_assert(kScratchBytes >= 1024 * (PB_TOP_K * 8 + 8), "the automatic slice plan fits");
constexpr int kMaxDevices = 64;

std::mutex g_mu;
void* g_scratch[kMaxDevices];  // device address of each device's copy of `scratch`

}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace pb {

// The device address of `scratch` on `device`, looked up once per device with
// that device current (each device holds its own copy of the array).  In host
// code `scratch` names a host-side stand-in, never the device memory: only the
// address returned here is passed to kernels.
hipError_t static_scratch_address(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[device] == nullptr) {
    int current = -1;
    hipError_t e = hipGetDevice(&current);
    if (e != hipSuccess) return e;
    if (current != device && (e = hipSetDevice(device)) != hipSuccess) return e;
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (current != device) (void)hipSetDevice(current);
    if (e != hipSuccess) return e;
    g_scratch[device] = ptr;
  }
  *out = g_scratch[device];
  return hipSuccess;
}

}  // namespace pb

extern "C" uint32_t pb_sample_batch_noalloc(pb_context* ctx, const uint32_t* d_logits,
                                            size_t vocab, size_t ld, uint32_t rows,
                                            const uint32_t* d_hist, size_t hist_ld,
                                            const uint32_t* d_hist_len,
                                            const uint32_t* d_random_24, uint32_t* d_token,
                                            pb_sample_detail* d_detail, pb_inference_error* d_err,
                                            void* stream, pb_inference_error* err) {
  void* ptr = nullptr;
  if (ctx != nullptr) {
    // pb_context_create looked the address up already; this only reads the table
    const hipError_t e = pb::static_scratch_address(pb::context_device(ctx), &ptr);
    if (e != hipSuccess) {
      if (err) {
        *err = pb_inference_error{PB_DEVICE, PB_DOMAIN_NONE, PB_NO_LAYER, 0, PB_NO_TENSOR, 0,
                                  0, (uint64_t)e, 0};
      }
      return PB_DEVICE;
    }
  }
  return pb::enqueue_sample_with_workspace(ctx, ptr, kScratchBytes, d_logits, vocab, ld, rows,
                                           d_hist, hist_ld, d_hist_len, d_random_24, d_token,
                                           d_detail, d_err, static_cast<hipStream_t>(stream), err);
}

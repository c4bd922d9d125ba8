// pb_static.hip -- pb_sample_batch_noalloc: the batched sampler with its
// slice workspace in a file-scope device array instead of memory the
// library allocates.
//
// The multi-slice sampler (segment_kernel + finish_kernel) passes each
// slice's top-20 keys and first-bad positions from the first launch to the
// second through a workspace of rows x slices records.  This file keeps one
// such workspace per device in `scratch`, sized for every batch of the
// automatic slice plan, so a caller that cannot allocate (code under HIP
// graph capture, a tight serving loop) can still sample.  No record has to
// start at zero: segment_kernel writes every record a launch uses before
// finish_kernel reads it.  Every call on one device shares that device's
// array, so calls that overlap on the device race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "pb_internal.h"
#include "pbsample.h"

namespace {

// (row, slice) records the array holds: the automatic plan cuts a batch of
// up to 64 rows into at most 1,024 / rows slices, one of up to 255 rows into
// at most 512 / rows, and from 256 rows on uses one slice per row and no
// workspace, so 1,024 records cover every batch.  20 keys + 2 words each.
constexpr size_t kScratchSlots = 1024;
constexpr size_t kScratchBytes = kScratchSlots * (PB_TOP_K * 8 + 8);  // 172,032 bytes
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

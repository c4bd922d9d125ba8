// pb_sampler.hip -- gfx950 kernels of the decode-step token sampler.
//
// Reference path (promptboot, crates/promptboot-core/src/):
//   validate_sample_logits        inference.rs:883-903   (finite scan)
//   token-range check             inference.rs:939-953
//   apply_repetition_penalty      fp32_sse2.rs:1848-1876
//   sample_top_k_top_p            fp32_sse2.rs:1786-1846
//
// Work decomposition (one launch covers every row of the batch):
//
//   segment_kernel   grid = rows x S workgroups of 256 threads.  A workgroup
//                    owns one contiguous slice (segment) of one row.  It
//                    builds the row's history bitmap for its slice in LDS,
//                    streams the slice once from HBM in register chunks of
//                    256 x F float4, and keeps the exact top-20 of the
//                    penalised values with 64-bit keys (value, -id).  The
//                    penalty is evaluated only for elements that pass the
//                    running threshold: the penalty never raises a value, so
//                    the unpenalised value is a valid upper bound.  With S == 1
//                    the same workgroup finishes the row (softmax, top-p,
//                    draw); otherwise it writes its 20 keys to the workspace.
//   finalize_kernel  (S > 1) one wave per row merges the S x 20 keys and
//                    finishes the row.
//   writeback_kernel (in-place variant only) applies the penalty to the
//                    caller's logits once per unique history id.
//
// Threshold logic per wave: the first chunk seeds a threshold from the 20th
// best lane maximum (20 distinct real elements are at least that good, so
// nothing below it can be in the top-20); later candidates must reach the
// wave's current 20th-best key (or the workgroup-wide best of those), and are
// merged 44 at a time with a 64-lane bitonic sort.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pb_device.h"
#include "pb_internal.h"

#pragma clang fp contract(off)

namespace pb {

constexpr uint32_t kBlock = 256;
constexpr uint32_t kWaves = kBlock / 64;
constexpr uint32_t kRowF4 = kVocab / 4;             // 37,984 float4 per row
constexpr uint32_t kRowWords = kVocab / 32;         // 4,748 bitmap words per row
constexpr uint32_t kBufCap = 128;                   // candidate slots per wave
constexpr uint64_t kErrDetailFinite = (uint64_t)7 << 32;
constexpr uint64_t kErrDetailToken = (uint64_t)2 << 32;

// Block index -> work item.  Consecutive work items (the segments of one row,
// and neighbouring rows) land on the same XCD, which the hardware picks
// round-robin from the block index; the history of a row is then read from
// HBM once and served from that XCD's L2 to every segment.
__device__ __forceinline__ uint32_t xcd_work_item(uint32_t block, uint32_t n) {
  if ((n & 7u) != 0) return block;
  return (block & 7u) * (n >> 3) + (block >> 3);
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const uint32_t o = (uint32_t)__shfl_xor((int)v, m, 64);
    v = o < v ? o : v;
  }
  return v;
}

// Finishes one row on one wave: lanes 0..19 hold the row's top-20 keys in
// rank order.  Softmax weights, top-p cutoff and the categorical draw follow
// fp32_sse2.rs:1818-1845 operation for operation; the binary64 sums run as a
// lane-serial chain in rank order, so every partial sum is the reference's.
__device__ void finalize_row(const RowParams& p, uint32_t row, uint64_t key, uint32_t bad_logit,
                             uint32_t bad_hist, uint32_t lane) {
  if (bad_logit != kNone || bad_hist != kNone) {
    pb_inference_error e;
    e.layer = PB_NO_LAYER;
    e.position = 0;
    e.tensor_id = PB_NO_TENSOR;
    e.reserved = 0;
    e.domain = PB_DOMAIN_ARGMAX;
    if (bad_logit != kNone) {
      e.status = PB_NONFINITE_OUTPUT;
      e.needed = 0;
      e.available = p.logits[(size_t)row * p.ld + bad_logit];
      e.detail = kErrDetailFinite | bad_logit;
    } else {
      e.status = PB_TOKEN_ID;
      e.needed = kVocab;
      e.available = p.hist[(size_t)row * p.hist_ld + bad_hist];
      e.detail = kErrDetailToken;
    }
    if (lane == 0) {
      p.token[row] = kNone;
      if (p.err) p.err[row] = e;
    }
    if (p.detail) {
      uint32_t* d = reinterpret_cast<uint32_t*>(p.detail + row);
      for (uint32_t i = lane; i < sizeof(pb_sample_detail) / 4; i += 64) d[i] = 0xffffffffu;
    }
    return;
  }

  const uint32_t id = key_id(key);
  const uint32_t vbits = key_value_bits(key);
  const float maximum = f_of((uint32_t)__shfl((int)vbits, 0, 64));
  float w = 0.0f;
  if (lane < (uint32_t)kTopK) {
    const float shifted = f_of(vbits) - maximum;
    w = expf_ref(shifted / f_of(kTemperatureBits));
  }
  double running = 0.0, mine = 0.0;
#pragma unroll
  for (int i = 0; i < kTopK; ++i) {
    const float wi = __shfl(w, i, 64);
    running = running + (double)wi;
    if (lane == (uint32_t)i) mine = running;
  }
  const double total = running;
  const float cutoff = (float)total * f_of(kTopPBits);
  const uint64_t stop = __ballot(lane < (uint32_t)kTopK && !(cutoff > (float)mine));
  const uint32_t kept = stop ? (uint32_t)__ffsll((unsigned long long)stop) : (uint32_t)kTopK;
  const double kept_total = __shfl(mine, (int)kept - 1, 64);
  const uint32_t r24 = p.random_24[row];
  const float unit = (float)(r24 & 0x00ffffffu) / f_of(kTwoPow24Bits);
  const float target = (float)kept_total * unit;
  const uint64_t hit = __ballot(lane < kept && (float)mine > target);
  const uint32_t rank = hit ? (uint32_t)__ffsll((unsigned long long)hit) - 1 : kept - 1;
  const uint32_t token = (uint32_t)__shfl((int)id, (int)rank, 64);

  if (lane == 0) p.token[row] = token;
  if (p.err && lane < sizeof(pb_inference_error) / 4) {
    reinterpret_cast<uint32_t*>(p.err + row)[lane] = 0u;
  }
  if (p.detail) {
    const double draw_tol = 1e-6 * (double)(float)kept_total;
    const double cut_tol = 1e-6 * (double)(float)total;
    const double pm = (double)(float)mine;
    const bool near_draw = lane < kept && __builtin_fabs(pm - (double)target) <= draw_tol;
    const bool near_cut = lane < (uint32_t)kTopK && __builtin_fabs(pm - (double)cutoff) <= cut_tol;
    const uint32_t flags = (__ballot(near_draw) ? kFlagDrawBoundary : 0u) |
                           (__ballot(near_cut) ? kFlagCutoffBoundary : 0u);
    pb_sample_detail* d = p.detail + row;
    if (lane < (uint32_t)kTopK) {
      d->ids[lane] = id;
      d->value_bits[lane] = vbits;
      d->weight_bits[lane] = b_of(w);
      d->probs[lane] = lane < kept ? (float)((double)w / kept_total) : 0.0f;
    }
    if (lane == 0) {
      d->kept = kept;
      d->rank = rank;
      d->flags = flags;
      d->token = token;
    }
  }
}

typedef float v4f __attribute__((ext_vector_type(4)));

template <int F>
__device__ __forceinline__ void load_chunk(v4f (&dst)[F], const v4f* __restrict__ rowp,
                                           uint32_t base, uint32_t f_hi, uint32_t tid) {
#pragma unroll
  for (int j = 0; j < F; ++j) {
    const uint32_t f = base + (uint32_t)j * kBlock + tid;
    dst[j] = f < f_hi ? rowp[f] : v4f{0.f, 0.f, 0.f, 0.f};
  }
}

template <int F, bool kFinalize>
__global__ __launch_bounds__(kBlock) void segment_kernel(RowParams p) {
  __shared__ uint32_t bm[kRowWords];
  __shared__ uint64_t top[kWaves][kTopK];
  __shared__ uint64_t buf[kWaves][kBufCap];
  __shared__ unsigned long long wg_thr;
  __shared__ uint32_t bad_logit, bad_hist, nonfinite_seen;

  const uint32_t n = p.rows * p.segs;
  const uint32_t item = xcd_work_item(blockIdx.x, n);
  const uint32_t row = item / p.segs;
  const uint32_t seg = item - row * p.segs;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;

  const uint32_t f_lo = seg * p.seg_f4;
  const uint32_t f_hi = min(f_lo + p.seg_f4, kRowF4);
  const uint32_t e_lo = f_lo * 4u;  // multiple of 32: seg_f4 % 8 == 0
  const uint32_t e_span = (f_hi - f_lo) * 4u;
  const uint32_t nwords = e_span / 32u;

  // ---- phase 0: clear LDS state ----
  for (uint32_t i = tid; i < nwords; i += kBlock) bm[i] = 0u;
  if (tid < kWaves * kTopK) (&top[0][0])[tid] = 0u;
  if (tid == 0) {
    wg_thr = 0u;
    bad_logit = kNone;
    bad_hist = kNone;
    nonfinite_seen = 0u;
  }
  __syncthreads();

  // ---- phase 1: history ids -> bitmap of this slice, first bad position ----
  uint32_t hist_len = 0;
  const uint32_t* __restrict__ hrow = nullptr;
  if (p.hist != nullptr && p.hist_len != nullptr) {
    hist_len = p.hist_len[row];
    if ((size_t)hist_len > p.hist_ld) hist_len = (uint32_t)p.hist_ld;
    hrow = p.hist + (size_t)row * p.hist_ld;
  }
  uint32_t my_bad = kNone;
  if (p.hist_vec4) {
    const uint4* h4 = reinterpret_cast<const uint4*>(hrow);
    const uint32_t n4 = (hist_len + 3u) / 4u;
    for (uint32_t q4 = tid; q4 < n4; q4 += kBlock) {
      const uint4 v = h4[q4];
      const uint32_t ids[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t q = q4 * 4u + (uint32_t)c;
        const uint32_t id = ids[c];
        if (q < hist_len) {
          if (id >= kVocab) {
            my_bad = min(my_bad, q);
          } else if (id - e_lo < e_span) {
            atomicOr(&bm[(id - e_lo) >> 5], 1u << (id & 31u));
          }
        }
      }
    }
  } else {
    for (uint32_t q = tid; q < hist_len; q += kBlock) {
      const uint32_t id = hrow[q];
      if (id >= kVocab) {
        my_bad = min(my_bad, q);
      } else if (id - e_lo < e_span) {
        atomicOr(&bm[(id - e_lo) >> 5], 1u << (id & 31u));
      }
    }
  }
  my_bad = wave_min_u32(my_bad);
  if (lane == 0 && my_bad != kNone) atomicMin(&bad_hist, my_bad);
  __syncthreads();
  if (p.excl != nullptr) {
    // ids already set in the caller's `seen` scratch are not penalised
    const uint32_t* ex = reinterpret_cast<const uint32_t*>(p.excl + (size_t)row * PB_SEEN_BYTES);
    for (uint32_t i = tid; i < nwords; i += kBlock) bm[i] &= ~ex[e_lo / 32u + i];
    __syncthreads();
  }

  // ---- phase 2: one streaming pass over the slice ----
  const v4f* __restrict__ rowp = reinterpret_cast<const v4f*>(p.logits + (size_t)row * p.ld);
  const uint32_t chunk_f4 = kBlock * (uint32_t)F;
  const uint32_t nchunks = (f_hi - f_lo + chunk_f4 - 1u) / chunk_f4;
  uint64_t* my_top = top[wave];
  uint64_t* my_buf = buf[wave];
  uint64_t thr = 0;      // this wave's current 20th-best key (a lower bound)
  uint32_t cnt = 0;      // pending candidates in my_buf
  float nan_probe = 0.0f;

  v4f cur[F];
  load_chunk<F>(cur, rowp, f_lo, f_hi, tid);
  for (uint32_t c = 0; c < nchunks; ++c) {
    const uint32_t base = f_lo + c * chunk_f4;
    v4f nxt[F];
    if (c + 1 < nchunks) load_chunk<F>(nxt, rowp, base + chunk_f4, f_hi, tid);

    if (c == 0) {
      // Seed: the best element of each lane (largest value, lowest id), its
      // penalised key, and the 20th best of those 64 keys.
      float bx = 0.0f;
      uint32_t be = kNone;
#pragma unroll
      for (int j = 0; j < F; ++j) {
        const uint32_t f = base + (uint32_t)j * kBlock + tid;
        const float xs[4] = {cur[j].x, cur[j].y, cur[j].z, cur[j].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (f < f_hi && (be == kNone || xs[k] > bx)) {
            bx = xs[k];
            be = f * 4u + (uint32_t)k;
          }
        }
      }
      uint64_t lane_key = 0;
      if (be != kNone) {
        const uint32_t e = be - e_lo;
        const uint32_t xb = b_of(bx);
        const uint32_t yb = ((bm[e >> 5] >> (e & 31u)) & 1u) ? penalize_bits(xb) : xb;
        lane_key = make_key(yb, be);
      }
      lane_key = wave_sort_desc(lane_key, lane);
      thr = shfl64(lane_key, kTopK - 1);
      if (lane == 0 && thr != 0) atomicMax(&wg_thr, thr);
    }

    uint64_t shared_thr = __hip_atomic_load(&wg_thr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    uint64_t thr_eff = thr > shared_thr ? thr : shared_thr;
    float thr_f = key_floor_value(thr_eff);

#pragma unroll
    for (int j = 0; j < F; ++j) {
      const uint32_t f = base + (uint32_t)j * kBlock + tid;
      const v4f x = cur[j];
      nan_probe = __builtin_fmaf(x.x, 0.0f, nan_probe);
      nan_probe = __builtin_fmaf(x.y, 0.0f, nan_probe);
      nan_probe = __builtin_fmaf(x.z, 0.0f, nan_probe);
      nan_probe = __builtin_fmaf(x.w, 0.0f, nan_probe);
      const float m = fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w));
      const bool pass = f < f_hi && m >= thr_f;
      if (__ballot(pass)) {
        // Slow path (rare once the threshold has settled): exact keys.
        uint32_t nib = 0;
        if (pass) {
          const uint32_t e = f * 4u - e_lo;
          nib = bm[e >> 5] >> (e & 31u);
        }
        const float xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          uint64_t key = 0;
          if (pass && xs[k] >= thr_f) {
            const uint32_t xb = b_of(xs[k]);
            const uint32_t yb = ((nib >> k) & 1u) ? penalize_bits(xb) : xb;
            key = make_key(yb, f * 4u + (uint32_t)k);
            if (key < thr_eff) key = 0;
          }
          const uint64_t mask = __ballot(key != 0);
          if (key != 0) my_buf[cnt + lanes_below(mask)] = key;
          cnt += (uint32_t)__popcll((unsigned long long)mask);
          if (cnt >= kMergeTake) {
            __builtin_amdgcn_wave_barrier();
            while (cnt >= kMergeTake) {
              const uint64_t t = merge_round(my_top, my_buf + (cnt - kMergeTake), kMergeTake, lane);
              cnt -= kMergeTake;
              if (t > thr) thr = t;
            }
            if (lane == 0 && thr != 0) atomicMax(&wg_thr, thr);
            shared_thr = __hip_atomic_load(&wg_thr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            thr_eff = thr > shared_thr ? thr : shared_thr;
            thr_f = key_floor_value(thr_eff);
          }
        }
      }
    }
    if (c + 1 < nchunks) {
#pragma unroll
      for (int j = 0; j < F; ++j) cur[j] = nxt[j];
    }
  }
  // drain pending candidates
  __builtin_amdgcn_wave_barrier();
  while (cnt > 0) {
    const uint32_t take = cnt < kMergeTake ? cnt : kMergeTake;
    merge_round(my_top, my_buf + (cnt - take), take, lane);
    cnt -= take;
  }
  if (__ballot(nan_probe != nan_probe) && lane == 0) nonfinite_seen = 1u;
  __syncthreads();

  // ---- non-finite rows only: find the first non-finite index of the slice ----
  if (nonfinite_seen) {
    uint32_t first = kNone;
    const uint32_t* words = p.logits + (size_t)row * p.ld;
    for (uint32_t e = e_lo + tid; e < e_lo + e_span; e += kBlock) {
      if ((words[e] & 0x7f800000u) == 0x7f800000u) {
        first = e;
        break;
      }
    }
    first = wave_min_u32(first);
    if (lane == 0 && first != kNone) atomicMin(&bad_logit, first);
    __syncthreads();
  }

  // ---- phase 3: workgroup top-20, then finish the row or publish the slice ----
  if (wave == 0) {
    merge_all(my_top, &top[1][0], (kWaves - 1) * (uint32_t)kTopK, lane);
    const uint64_t key = lane < (uint32_t)kTopK ? my_top[lane] : 0;
    if (kFinalize) {
      finalize_row(p, row, key, bad_logit, bad_hist, lane);
    } else {
      const size_t slot = (size_t)row * p.segs + seg;
      if (lane < (uint32_t)kTopK) p.part_keys[slot * kTopK + lane] = key;
      if (lane == 0) {
        p.part_meta[slot * 2 + 0] = bad_logit;
        p.part_meta[slot * 2 + 1] = bad_hist;
      }
    }
  }
}

// One wave per row: merge the S published top-20 lists, then finish the row.
__global__ __launch_bounds__(kBlock) void finalize_kernel(RowParams p) {
  __shared__ uint64_t top[kWaves][kTopK];
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t row = blockIdx.x * kWaves + wave;
  if (row >= p.rows) return;
  const uint64_t* keys = p.part_keys + (size_t)row * p.segs * kTopK;
  uint64_t* my_top = top[wave];
  if (lane < (uint32_t)kTopK) my_top[lane] = keys[lane];
  __builtin_amdgcn_wave_barrier();
  merge_all(my_top, keys + kTopK, (p.segs - 1) * (uint32_t)kTopK, lane);
  uint32_t bad_logit = kNone;
  for (uint32_t s = lane; s < p.segs; s += 64) {
    const uint32_t b = p.part_meta[((size_t)row * p.segs + s) * 2];
    bad_logit = b < bad_logit ? b : bad_logit;
  }
  bad_logit = wave_min_u32(bad_logit);
  const uint32_t bad_hist = p.part_meta[(size_t)row * p.segs * 2 + 1];
  const uint64_t key = lane < (uint32_t)kTopK ? my_top[lane] : 0;
  finalize_row(p, row, key, bad_logit, bad_hist, lane);
}

// In-place penalty for successful rows (fp32_sse2.rs:1848-1876): the first
// occurrence of each id not already set in `seen` penalises that logit once.
// With `seen` given, the history bits are cleared there afterwards.  When
// `gather` is given, gather[row * hist_ld + q] receives the final value of
// logits[hist[q]] (used by the host drop-in to write its own buffer).
__global__ __launch_bounds__(kBlock) void writeback_kernel(WritebackParams p) {
  __shared__ uint32_t taken[kRowWords];
  __shared__ uint32_t hbits[kRowWords];
  const uint32_t row = blockIdx.x;
  const uint32_t tid = threadIdx.x;
  if (p.token[row] == kNone) return;  // failed rows stay untouched
  uint32_t* seen_words =
      p.seen ? reinterpret_cast<uint32_t*>(p.seen + (size_t)row * PB_SEEN_BYTES) : nullptr;
  for (uint32_t i = tid; i < kRowWords; i += kBlock) {
    taken[i] = seen_words ? seen_words[i] : 0u;
    hbits[i] = 0u;
  }
  __syncthreads();
  uint32_t hist_len = p.hist_len[row];
  if ((size_t)hist_len > p.hist_ld) hist_len = (uint32_t)p.hist_ld;
  const uint32_t* hrow = p.hist + (size_t)row * p.hist_ld;
  uint32_t* lrow = p.logits + (size_t)row * p.ld;
  for (uint32_t q = tid; q < hist_len; q += kBlock) {
    const uint32_t id = hrow[q];
    const uint32_t bit = 1u << (id & 31u);
    atomicOr(&hbits[id >> 5], bit);
    const uint32_t old = atomicOr(&taken[id >> 5], bit);
    if ((old & bit) == 0u) lrow[id] = penalize_bits(lrow[id]);
  }
  __syncthreads();
  if (seen_words) {
    for (uint32_t i = tid; i < kRowWords; i += kBlock) seen_words[i] &= ~hbits[i];
  }
  if (p.gather) {
    __threadfence_block();
    for (uint32_t q = tid; q < hist_len; q += kBlock) {
      p.gather[(size_t)row * p.hist_ld + q] = lrow[hrow[q]];
    }
  }
}

// ---- host-side launchers ----

uint32_t segments_for_rows(uint32_t rows) {
  // Enough workgroups to cover the 256 CUs several times over, but never more
  // than 64 slices per row (the finalize merge grows with S).
  if (rows == 0) return 1;
  uint32_t s = 2048u / rows;
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  return s;
}

void plan_segments(uint32_t rows, uint32_t forced_segments, uint32_t* segs, uint32_t* seg_f4) {
  uint32_t s = forced_segments ? forced_segments : segments_for_rows(rows);
  if (s > 64) s = 64;
  uint32_t len = (kRowF4 + s - 1) / s;
  len = (len + 7u) & ~7u;  // slices start on a 32-element bitmap word
  *seg_f4 = len;
  *segs = (kRowF4 + len - 1) / len;
}

hipError_t launch_sample(const RowParams& p, hipStream_t stream) {
  const uint32_t blocks = p.rows * p.segs;
  if (p.segs == 1) {
    hipLaunchKernelGGL((segment_kernel<kChunkF4, true>), dim3(blocks), dim3(kBlock), 0, stream, p);
  } else {
    hipLaunchKernelGGL((segment_kernel<kChunkF4, false>), dim3(blocks), dim3(kBlock), 0, stream, p);
    hipLaunchKernelGGL(finalize_kernel, dim3((p.rows + kWaves - 1) / kWaves), dim3(kBlock), 0,
                       stream, p);
  }
  return hipGetLastError();
}

__global__ __launch_bounds__(kBlock) void probe_kernel(int which, const uint32_t* in,
                                                      uint32_t* out, size_t n) {
  const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  out[i] = which == 0 ? b_of(expf_ref(f_of(in[i]))) : penalize_bits(in[i]);
}

hipError_t launch_probe(int which, const uint32_t* in, uint32_t* out, size_t n,
                        hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const size_t blocks = (n + kBlock - 1) / kBlock;
  hipLaunchKernelGGL(probe_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0, stream, which, in,
                     out, n);
  return hipGetLastError();
}

hipError_t launch_writeback(const WritebackParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(writeback_kernel, dim3(p.rows), dim3(kBlock), 0, stream, p);
  return hipGetLastError();
}

}  // namespace pb

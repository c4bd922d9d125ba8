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
//                    streams the slice once from HBM (two register chunks of
//                    256 x F float4 in flight per thread, each float4
//                    reloaded as soon as it has been examined), and keeps the
//                    exact top-20 of the penalised values with 64-bit keys
//                    (value, -id).  Candidates are keyed by their raw value
//                    and penalised when merged: the penalty never raises a
//                    value, so a raw key below the threshold is below it
//                    penalised as well.  With S == 1 the same workgroup
//                    finishes the row (softmax, top-p, draw); otherwise it
//                    publishes its 20 keys.
//   finish_kernel    (S > 1 only) one wave per row merges the S published
//                    lists and finishes the row.
//   writeback_kernel (in-place variant only) applies the penalty to the
//                    caller's logits once per unique history id.
//
// Threshold logic: a key below the threshold is dropped, so the threshold
// must never exceed the slice's final 20th-best key; it is a lower bound
// backed by at least 20 distinct elements.  The first chunk seeds it from the
// lane maxima (the 20th best of a wave's 64, and the smallest of the waves'
// 5th best: 4 x 5 distinct elements).  Later the same two bounds come from the
// waves' top lists, which absorb pending candidates 24 at a time with a
// 64-lane bitonic sort.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "pb_device.h"
#include "pb_internal.h"
#include "pb_rows.h"

#pragma clang fp contract(off)

namespace pb {

constexpr uint32_t kBlock = 256;
constexpr uint32_t kWaves = kBlock / 64;
// Keys each wave contributes to the workgroup threshold: kWaves * kQuota >= 20.
constexpr uint32_t kQuota = (kTopK + kWaves - 1) / kWaves;
constexpr uint32_t kRowF4 = kVocab / 4;             // 37,984 float4 per row
constexpr uint32_t kRowWords = kVocab / 32;         // 4,748 bitmap words per row
constexpr uint32_t kBufCap = 128;                   // candidate slots per wave
// Pending keys that trigger a merge: an earlier merge raises the wave's
// threshold sooner, and fewer later elements reach the slow path.
constexpr uint32_t kMergeAt = 24;
static_assert(kMergeAt >= 1 && kMergeAt - 1 + 64 <= kBufCap, "one ballot of keys must fit");
// Staged float4 per wave: a float4 whose maximum reaches the threshold is
// parked in LDS with its index, and the staged float4 are keyed and merged
// together by one copy of the keying and merging code instead of one per
// float4 of the unrolled loop.  The stage is flushed at the end of a chunk
// once it holds kFlushAt float4 (a flush costs a wave a few hundred cycles
// without loads; once the threshold has settled a chunk stages one or two),
// at once when it is half full, and before the final drain.  Measured on
// MI355X at B=4096: a flush at every chunk end with anything staged gave
// 0.4114-0.4138 ms per launch, kFlushAt = 16 or 32 gives 0.406 ms.
constexpr uint32_t kStageCap = 128;
constexpr uint32_t kFlushAt = 16;
static_assert(kStageCap >= 2 * 64, "a flush at half capacity leaves room for one ballot");
constexpr uint32_t kMaxSegments = 32;               // slices per row, at most

// Block index -> work item when rows are cut into slices.  Consecutive work
// items (the segments of one row, and neighbouring rows) land on the same
// XCD, which the hardware picks round-robin from the block index; the history
// of a row is then read from HBM once and served from that XCD's L2 to every
// segment.  With one segment per row the block index is the row: the rows
// then spread round-robin over the XCDs, which measured 0.6-1.4 % faster at
// B = 1024 (flat 0.1003 -> 0.0997 ms, history over half the vocabulary
// 0.1460 -> 0.1441 ms) and even at B = 4096.
__device__ __forceinline__ uint32_t xcd_work_item(uint32_t block, uint32_t n) {
  if ((n & 7u) != 0) return block;
  return (block & 7u) * (n >> 3) + (block >> 3);
}

// ---- row order: longest history first after the first residency round ----
// With one slice per row, workgroups below p.order_from (the workgroups the
// GPU holds at once) take rows in batch order and start streaming at once.
// Each later workgroup ranks the rows of its group (kOrderGroup rows from
// order_from on, the last group shorter) by bucketed history length, longest
// first and in batch order within a bucket, and takes the row at its own
// rank: every workgroup of a group computes the same ranking, so each row is
// taken once.  Those workgroups start while others stream, which hides the
// ranking, and the launch ends on short rows instead of on whichever rows
// came last.  Measured on MI355X with the rows permuted on the host the same
// way (B = 4096, histories U[16, 32768], HIP events): 0.4063 -> 0.4005 ms,
// the same as ranking every row.
struct RowOrderScratch {
  uint32_t count[64];  // rows per slot; slot 0 holds the longest bucket
  uint32_t hits[64];   // per (k, wave): rows of the chosen slot
  uint64_t mask[64];   // per (k, wave): their lanes
  uint32_t pick[2];
};
constexpr uint32_t kOrderPerThread = kOrderGroup / kBlock;
static_assert(kOrderPerThread * kWaves == 64, "one wave scans the (k, wave) entries");

__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v, uint32_t lane) {
#pragma unroll
  for (uint32_t d = 1; d < 64u; d <<= 1) {
    const uint32_t t = __shfl_up(v, d, 64);
    if (lane >= d) v += t;
  }
  return v;
}

// Position of set bit number n (from 0, lowest first) of m; n < popcount(m).
__device__ __forceinline__ uint32_t nth_set_bit(uint64_t m, uint32_t n) {
  uint32_t pos = 0;
#pragma unroll
  for (uint32_t w = 32; w >= 1u; w >>= 1) {
    const uint32_t lo = (uint32_t)__popcll(m & ((1ull << w) - 1ull));
    if (n >= lo) {
      n -= lo;
      m >>= w;
      pos += w;
    }
  }
  return pos;
}

// The row of work item `item` >= p.order_from (one slice per row).
__device__ __forceinline__ uint32_t ordered_row(const RowParams& p, uint32_t item,
                                                RowOrderScratch& s) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  const uint32_t rel = item - p.order_from;
  const uint32_t base = p.order_from + rel / kOrderGroup * kOrderGroup;
  const uint32_t m = min(kOrderGroup, p.rows - base);
  const uint32_t rank = rel % kOrderGroup;  // < m, since item < rows
  uint32_t len[kOrderPerThread];
#pragma unroll
  for (uint32_t k = 0; k < kOrderPerThread; ++k)
    len[k] = p.hist_len[base + min(k * kBlock + tid, m - 1u)];
  if (tid < 64u) s.count[tid] = 0u;
  __syncthreads();
  uint32_t slot[kOrderPerThread];
#pragma unroll
  for (uint32_t k = 0; k < kOrderPerThread; ++k) {
    const uint32_t l = (size_t)len[k] > p.hist_ld ? (uint32_t)p.hist_ld : len[k];
    slot[k] = k * kBlock + tid < m ? 63u - min(l >> p.order_shift, 63u) : 64u;
    if (slot[k] < 64u) atomicAdd(&s.count[slot[k]], 1u);
  }
  __syncthreads();
  // the slot that holds rank `rank`, and the rank inside it
  if (wave == 0) {
    const uint32_t c = s.count[lane];
    const uint32_t incl = wave_inclusive_sum(c, lane);
    if (rank < incl && rank >= incl - c) {
      s.pick[0] = lane;
      s.pick[1] = rank - (incl - c);
    }
  }
  __syncthreads();
  const uint32_t want = s.pick[0];
  const uint32_t j = s.pick[1];
  // Entry k * kWaves + wave covers rows base + k * 256 + wave * 64 + lane:
  // entries in order are rows in batch order.
#pragma unroll
  for (uint32_t k = 0; k < kOrderPerThread; ++k) {
    const uint64_t hit = __ballot(slot[k] == want);
    if (lane == 0) {
      s.hits[k * kWaves + wave] = (uint32_t)__popcll(hit);
      s.mask[k * kWaves + wave] = hit;
    }
  }
  __syncthreads();
  if (wave == 0) {
    const uint32_t c = s.hits[lane];
    const uint32_t incl = wave_inclusive_sum(c, lane);
    if (j < incl && j >= incl - c)
      s.pick[0] = base + (lane / kWaves) * kBlock + (lane % kWaves) * 64u +
                  nth_set_bit(s.mask[lane], j - (incl - c));
  }
  __syncthreads();
  // exactly one lane wrote the row; the clamp keeps every address in bounds
  return min(__builtin_amdgcn_readfirstlane(s.pick[0]), p.rows - 1u);
}

// Histories are Zipf-like: a few ids recur thousands of times, and atomics
// to one LDS word serialise.  Testing the bit first leaves one atomic per
// distinct id (plus the rare lanes that race on a fresh one).
__device__ __forceinline__ void set_bit_once(uint32_t* word, uint32_t bit) {
  if ((__hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) & bit) == 0u)
    atomicOr(word, bit);
}

typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// Loads float4 base + j*256 + tid, j < F, of a slice ending at f_hi.  Past the
// end the address is clamped to the slice's last float4 (users mask those
// lanes by index): every load is unconditional, so the number of loads in
// flight is the same on every path and a wait for an older load (the
// history's) does not have to wait for all of them.
template <int F>
__device__ __forceinline__ void load_chunk(v4f (&dst)[F], const v4f* __restrict__ rowp,
                                           uint32_t base, uint32_t f_hi, uint32_t tid) {
#pragma unroll
  for (int j = 0; j < F; ++j) {
    const uint32_t f = base + (uint32_t)j * kBlock + tid;
    // Each logit is read exactly once: a non-temporal load keeps the stream
    // from evicting the history and the workspace from the caches.
    dst[j] = __builtin_nontemporal_load(rowp + min(f, f_hi - 1u));
  }
}

template <int F, bool kFinalize>
__global__ __launch_bounds__(kBlock) void segment_kernel(RowParams p) {
  __shared__ __align__(16) uint32_t bm[kRowWords];
  __shared__ uint64_t top[kWaves][kTopK];
  __shared__ uint64_t buf[kWaves][kBufCap];
  __shared__ __align__(16) float stage_x[kWaves][kStageCap][4];
  __shared__ uint32_t stage_f[kWaves][kStageCap];
  __shared__ unsigned long long wg_thr;
  __shared__ uint64_t wave_q[kWaves];  // each wave's kQuota-th best key
  __shared__ uint32_t bad_logit, bad_hist, nonfinite_seen;

  const uint32_t n = p.rows * p.segs;
  uint32_t item = p.segs == 1 ? blockIdx.x : xcd_work_item(blockIdx.x, n);
  if constexpr (kFinalize) {  // one slice per row: the item is the row
    __shared__ RowOrderScratch order_scratch;
    if (p.order_from != 0u && item >= p.order_from) item = ordered_row(p, item, order_scratch);
  }
  const uint32_t row = item / p.segs;
  const uint32_t seg = item - row * p.segs;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  if (row_skipped(p, row)) {  // decode loop: the row has ended or has no room
    if (seg == 0 && tid == 0) skip_row(p, row);
    return;
  }

  const uint32_t f_lo = seg * p.seg_f4;
  const uint32_t f_hi = min(f_lo + p.seg_f4, kRowF4);
  const uint32_t e_lo = f_lo * 4u;  // multiple of 32: seg_f4 % 8 == 0
  const uint32_t e_span = (f_hi - f_lo) * 4u;
  const uint32_t nwords = e_span / 32u;

  const v4f* __restrict__ rowp = reinterpret_cast<const v4f*>(p.logits + (size_t)row * p.ld);
  const uint32_t chunk_f4 = kBlock * (uint32_t)F;
  const uint32_t nchunks = (f_hi - f_lo + chunk_f4 - 1u) / chunk_f4;
  // The first 256 uint4 of the history row and the first chunk of logits are
  // requested before anything else, the history first (the scan needs it
  // first), before the history length is known (ids past the length are
  // padding of the same row and are ignored): the two streams overlap and the
  // scan costs one memory round trip, not two.  The history load is
  // unconditional, from a clamped address (the logits row when the history is
  // not 16-byte aligned; the value is then unused): a load under a branch
  // makes the compiler wait for every outstanding load where the branch joins.
  const v4u* h4 = p.hist_vec4 ? reinterpret_cast<const v4u*>(p.hist + (size_t)row * p.hist_ld)
                              : reinterpret_cast<const v4u*>(rowp);
  const uint32_t h4_last = p.hist_vec4 ? (uint32_t)(p.hist_ld / 4u) - 1u : kBlock - 1u;
  const v4u h_first = __builtin_nontemporal_load(h4 + min(tid, h4_last));
  // The row's uniform, for the finish (S == 1); requested now so that its
  // latency never lands on the row's last step.
  const uint32_t r24 = kFinalize ? p.random_24[row] : 0u;
  v4f cur[F];
  load_chunk<F>(cur, rowp, f_lo, f_hi, tid);
  uint32_t hist_len = 0;
  if (p.hist != nullptr && p.hist_len != nullptr) {
    hist_len = row_word(p.hist_len + row);
    if ((size_t)hist_len > p.hist_ld) hist_len = (uint32_t)p.hist_ld;
  }

  // ---- phase 0: clear LDS state ----
  for (uint32_t i = tid; i < nwords; i += kBlock) bm[i] = 0u;
  if (tid < kWaves * kTopK) (&top[0][0])[tid] = 0u;
  if (tid == 0) {
    wg_thr = 0u;
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w) wave_q[w] = 0u;
    bad_logit = kNone;
    bad_hist = kNone;
    nonfinite_seen = 0u;
  }
  __syncthreads();

  // ---- phase 1: history ids -> bitmap of this slice, first bad position ----
  const uint32_t* __restrict__ hrow = hist_len != 0 ? p.hist + (size_t)row * p.hist_ld : nullptr;
  uint32_t my_bad = kNone;
  // Marks the ids at history positions 4*q4 .. 4*q4+3 in the slice bitmap.
  // The four bitmap words are read first and only bits not yet set are OR-ed
  // in: a wave waits for LDS once per four ids, and repeated ids (most of a
  // long history) cost no atomic.  Lanes with nothing to mark read word 0.
  auto add_ids = [&](const v4u& v, uint32_t q4) {
    const uint32_t ids[4] = {v.x, v.y, v.z, v.w};
    uint32_t word[4], cur_bits[4];
    bool mark[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t q = q4 * 4u + (uint32_t)c;
      const bool valid = q < hist_len;
      my_bad = min(my_bad, valid && ids[c] >= kVocab ? q : kNone);
      const uint32_t rel = ids[c] - e_lo;  // ids >= kVocab fall outside every slice
      mark[c] = valid && rel < e_span;
      word[c] = mark[c] ? rel >> 5 : 0u;
      cur_bits[c] = __hip_atomic_load(&bm[word[c]], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t bit = 1u << (ids[c] & 31u);
      if (mark[c] && (cur_bits[c] & bit) == 0u) atomicOr(&bm[word[c]], bit);
    }
  };
  if (p.hist_vec4) {
    // After the first 256 uint4, kHistBatch uint4 per thread stay in flight:
    // each one consumed is replaced by the load kHistBatch*256 uint4 further
    // on, while there is a further batch.  Loads past the length are clamped
    // to the row's last uint4 (a repeat of it marks nothing new: its
    // positions are past the length).  The scan is bound by HBM latency
    // otherwise.
    constexpr uint32_t kHistBatch = 4;
    constexpr uint32_t kStep = kHistBatch * kBlock;
    const uint32_t n4 = (hist_len + 3u) / 4u;
    add_ids(h_first, tid);
    if (n4 > kBlock) {
      const uint32_t last = n4 - 1u;
      v4u v[kHistBatch];
#pragma unroll
      for (uint32_t u = 0; u < kHistBatch; ++u)
        v[u] = __builtin_nontemporal_load(h4 + min(kBlock + u * kBlock + tid, last));
      uint32_t b4 = kBlock;
      for (; b4 + kStep < n4; b4 += kStep) {
#pragma unroll
        for (uint32_t u = 0; u < kHistBatch; ++u) {
          add_ids(v[u], b4 + u * kBlock + tid);
          // Keeps the ids of v[u] from living past its reload (the empty asm
          // makes my_bad final here, not at the end of the iteration): the
          // reload then lands in v[u]'s own registers, and the loop does not
          // wait for it to copy it back before the next iteration.
          __asm__ volatile("" : "+v"(my_bad));
          __builtin_amdgcn_sched_barrier(0);
          v[u] = __builtin_nontemporal_load(h4 + min(b4 + kStep + u * kBlock + tid, last));
        }
      }
#pragma unroll
      for (uint32_t u = 0; u < kHistBatch; ++u) add_ids(v[u], b4 + u * kBlock + tid);
    }
  } else {
    for (uint32_t q = tid; q < hist_len; q += kBlock) {
      const uint32_t id = hrow[q];
      if (id >= kVocab) {
        my_bad = min(my_bad, q);
      } else if (id - e_lo < e_span) {
        set_bit_once(&bm[(id - e_lo) >> 5], 1u << (id & 31u));
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
  uint64_t* my_top = top[wave];
  uint64_t* my_buf = buf[wave];
  uint64_t thr = 0;      // this wave's current 20th-best key (a lower bound)
  uint32_t cnt = 0;      // pending candidates in my_buf
  float nan_probe = 0.0f;

  // Two chunks are in flight per thread at all times: chunk c sits in
  // cur (c even) or nxt (c odd), and as soon as float4 j of chunk c has been
  // examined its registers are reloaded with float4 j of chunk c + 2.  The
  // reloads are unconditional (clamped past the end of the slice; those lanes
  // are masked by index), so every wait is for the oldest load only.
  v4f nxt[F];
  load_chunk<F>(nxt, rowp, f_lo + chunk_f4, f_hi, tid);

  // Workgroup threshold: the largest of the waves' 20th best keys, and the
  // smallest of their kQuota-th best keys -- the waves' lists then hold at
  // least kWaves * kQuota >= 20 distinct keys at or above it, so the row's
  // 20th best key is never below it.  With the row split over the waves, the
  // second bound is close to the row's own 20th best seen so far; the first
  // is the 20th best of a quarter of it.
  auto publish_quota = [&](uint64_t q) {
    __hip_atomic_store(&wave_q[wave], q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  auto wg_threshold = [&]() -> uint64_t {
    uint64_t t = __hip_atomic_load(&wg_thr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    uint64_t m = __hip_atomic_load(&wave_q[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll
    for (uint32_t w = 1; w < kWaves; ++w) {
      const uint64_t o = __hip_atomic_load(&wave_q[w], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      m = o < m ? o : m;
    }
    return t > m ? t : m;
  };

  {
    // Seed: the best element of each lane in chunk 0 (largest value, lowest
    // id), its penalised key, and the 20th best of those 64 keys.
    float bx = 0.0f;
    uint32_t be = kNone;
#pragma unroll
    for (int j = 0; j < F; ++j) {
      const uint32_t f = f_lo + (uint32_t)j * kBlock + tid;
      const float xs[4] = {cur[j].x, cur[j].y, cur[j].z, cur[j].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (f < f_hi && (be == kNone || xs[k] > bx)) {
          bx = xs[k];
          be = f * 4u + (uint32_t)k;
        }
      }
    }
    // Only the value part is sorted: the smallest key of the 20th best
    // value is reached by 20 distinct elements as well.
    uint32_t lane_ord = 0;
    if (be != kNone) {
      const uint32_t e = be - e_lo;
      const uint32_t xb = b_of(bx);
      const uint32_t yb = ((bm[e >> 5] >> (e & 31u)) & 1u) ? penalize_bits(xb) : xb;
      lane_ord = ord_of(yb);
    }
    const uint32_t sorted = wave_sort_desc_u32(lane_ord, lane);
    thr = (uint64_t)bcast32(sorted, kTopK - 1) << 32;
    if (lane == 0) {
      if (thr != 0) atomicMax(&wg_thr, thr);
      publish_quota((uint64_t)bcast32(sorted, kQuota - 1) << 32);
    }
  }
  // Every wave's seed is in place before any wave filters chunk 0, where the
  // threshold matters most.
  __syncthreads();

  // The exact (penalised) key of a buffered raw key.
  auto exact_key = [&](uint64_t key) -> uint64_t {
    const uint32_t id = key_id(key);
    const uint32_t e = id - e_lo;
    if ((bm[e >> 5] >> (e & 31u)) & 1u) return make_key(penalize_bits(key_value_bits(key)), id);
    return key;
  };

  // Keys the staged float4 (raw values: the penalty only lowers a key, so a
  // raw key below the threshold is below it penalised as well; the penalty is
  // applied when the key is merged), appends those reaching the threshold to
  // the wave's buffer and merges the buffer into the wave's top-20 whenever
  // kMergeAt keys are pending.  Returns the refreshed threshold floor.
  float (*my_stage_x)[4] = stage_x[wave];
  uint32_t* my_stage_f = stage_f[wave];
  uint32_t nst = 0;  // staged float4 (wave-uniform)
  uint64_t thr_eff = 0;
  auto refresh = [&]() -> float {
    const uint64_t shared_thr = wg_threshold();
    thr_eff = thr > shared_thr ? thr : shared_thr;
    return key_floor_value(thr_eff);
  };
  auto flush_stage = [&]() -> float {
    __builtin_amdgcn_wave_barrier();
    float thr_f = refresh();
#pragma unroll 1
    for (uint32_t s0 = 0; s0 < nst; s0 += 64u) {
      const uint32_t i = s0 + lane;
      const bool have = i < nst;
      const v4f x = have ? *reinterpret_cast<const v4f*>(my_stage_x[i]) : v4f{0.f, 0.f, 0.f, 0.f};
      const uint32_t f = have ? my_stage_f[i] : 0u;
      // a runtime loop over the four elements: one copy of the merge code
#pragma unroll 1
      for (uint32_t k = 0; k < 4u; ++k) {
        const float xk = k == 0u ? x.x : k == 1u ? x.y : k == 2u ? x.z : x.w;
        uint64_t key = 0;
        if (have && xk >= thr_f) {
          key = make_key(b_of(xk), f * 4u + k);
          if (key < thr_eff) key = 0;
        }
        const uint64_t mask = __ballot(key != 0);
        if (key != 0) my_buf[cnt + lanes_below(mask)] = key;
        cnt += (uint32_t)__popcll((unsigned long long)mask);
        if (cnt >= kMergeAt) {
          __builtin_amdgcn_wave_barrier();
          while (cnt > 0) {
            const uint32_t take = cnt < kMergeTake ? cnt : kMergeTake;
            const uint64_t t = merge_round(my_top, my_buf + (cnt - take), take, lane, exact_key);
            cnt -= take;
            if (t > thr) thr = t;
          }
          if (lane == 0) {
            if (thr != 0) atomicMax(&wg_thr, thr);
            publish_quota(my_top[kQuota - 1]);
          }
          thr_f = refresh();
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    nst = 0;
    return thr_f;
  };

  // Examines chunk c held in `x4` and reloads each of its float4 with chunk
  // c + 2.  A float4 whose maximum reaches the threshold is staged; the stage
  // is flushed at the end of the chunk, or as soon as it is half full.
  auto stream_chunk = [&](v4f (&x4)[F], uint32_t c) {
    const uint32_t base = f_lo + c * chunk_f4;
    float thr_f = refresh();
#pragma unroll
    for (int j = 0; j < F; ++j) {
      const uint32_t f = base + (uint32_t)j * kBlock + tid;
      const v4f x = x4[j];
      nan_probe = __builtin_fmaf(x.x, 0.0f, nan_probe);
      nan_probe = __builtin_fmaf(x.y, 0.0f, nan_probe);
      nan_probe = __builtin_fmaf(x.z, 0.0f, nan_probe);
      nan_probe = __builtin_fmaf(x.w, 0.0f, nan_probe);
      const float m = fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w));
      const bool pass = f < f_hi && m >= thr_f;
      const uint64_t pmask = __ballot(pass);
      if (pmask) {
        if (pass) {
          const uint32_t slot = nst + lanes_below(pmask);
          *reinterpret_cast<v4f*>(my_stage_x[slot]) = x;
          my_stage_f[slot] = f;
        }
        nst += (uint32_t)__popcll((unsigned long long)pmask);
        if (nst > kStageCap - 64u) thr_f = flush_stage();
      }
      // The empty asm makes nan_probe final here, so nothing reads x4[j]
      // past its reload: the reload lands in x4[j]'s own registers and no
      // copy (and no wait for it) follows.
      __asm__ volatile("" : "+v"(nan_probe));
      __builtin_amdgcn_sched_barrier(0);
      x4[j] = __builtin_nontemporal_load(rowp + min(f + 2u * chunk_f4, f_hi - 1u));
    }
    if (nst >= kFlushAt) flush_stage();
  };
  for (uint32_t c = 0; c < nchunks; c += 2) {
    stream_chunk(cur, c);
    stream_chunk(nxt, c + 1);  // past the last chunk: every lane masked
  }
  // drain the stage and the pending candidates
  if (nst != 0) flush_stage();
  __builtin_amdgcn_wave_barrier();
  while (cnt > 0) {
    const uint32_t take = cnt < kMergeTake ? cnt : kMergeTake;
    merge_round(my_top, my_buf + (cnt - take), take, lane, exact_key);
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

  // ---- phase 3: workgroup top-20 (two levels of bitonic merges) ----
  uint64_t pair = 0;
  if (wave < 2) pair = merge_two_lists(top[2 * wave], top[2 * wave + 1], lane);
  __syncthreads();
  if (wave < 2 && lane < (uint32_t)kTopK) top[wave][lane] = pair;
  __syncthreads();
  if (kFinalize) {
    if (wave == 0) {
      const uint64_t key = merge_two_lists(top[0], top[1], lane);
      const uint32_t bad_bits =
          bad_logit != kNone ? p.logits[(size_t)row * p.ld + bad_logit] : 0u;
      finalize_row(p, row, lane < (uint32_t)kTopK ? key : 0, bad_logit, bad_bits, bad_hist, lane,
                   r24);
    }
    return;
  }

  // S > 1: publish this slice's top-20 and first bad positions; the next
  // launch on the stream (finish_kernel) merges the S lists of each row.  A
  // kernel boundary makes them visible to every XCD; finishing the row in
  // this launch instead needs an agent-scope release per slice, a writeback
  // of the XCD's L2 that serialises across the workgroups.
  if (wave == 0) {
    const uint64_t key = merge_two_lists(top[0], top[1], lane);
    const size_t slot = (size_t)row * p.segs + seg;
    if (lane < (uint32_t)kTopK) p.part_keys[slot * kTopK + lane] = key;
    if (lane == 0) {
      p.part_meta[slot * 2 + 0] = bad_logit;
      p.part_meta[slot * 2 + 1] = bad_hist;
    }
  }
}

// Finishes the rows of a multi-slice launch, one wave per row: the S slice
// lists are merged (merge_lists_by_threshold) and the row finished.
// One row per workgroup: a batch's rows spread over as many CUs as there are
// rows (B = 64: 22.6 against 23.0 us per step with four rows per workgroup).
constexpr uint32_t kFinishWaves = 1;
__global__ __launch_bounds__(64 * kFinishWaves) void finish_kernel(RowParams p) {
  __shared__ __align__(16) uint64_t staged[kFinishWaves][kMaxSegments * kTopK + 64];
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t row = blockIdx.x * kFinishWaves + wave;
  if (row >= p.rows) return;
  if (row_skipped(p, row)) return;  // decode loop: segment_kernel wrote the skipped row
  // every load of the S lists and slice records is issued before the first wait
  constexpr uint32_t kStage = (kMaxSegments * kTopK + 63) / 64;
  uint64_t* st = staged[wave];
  const uint64_t* keys = p.part_keys + (size_t)row * p.segs * kTopK;
  const uint32_t nkeys = p.segs * (uint32_t)kTopK;
  uint64_t v[kStage];
#pragma unroll
  for (uint32_t u = 0; u < kStage; ++u) {
    const uint32_t i = u * 64u + lane;
    v[u] = i < nkeys ? keys[i] : 0;
  }
  const uint32_t r24 = p.random_24[row];  // requested with the lists
  const uint32_t* meta = p.part_meta + (size_t)row * p.segs * 2;
  const uint32_t b = lane < p.segs ? meta[lane * 2] : kNone;
  const uint32_t hist_bad = meta[1];
#pragma unroll
  for (uint32_t u = 0; u < kStage; ++u) {
    const uint32_t i = u * 64u + lane;
    if (i < nkeys) st[i] = v[u];
  }
  __builtin_amdgcn_wave_barrier();
  const uint64_t merged = merge_lists_by_threshold(st, p.segs, st + kMaxSegments * kTopK, lane);
  const uint32_t first_bad = wave_min_u32(b);
  const uint32_t bad_bits = first_bad != kNone ? p.logits[(size_t)row * p.ld + first_bad] : 0u;
  finalize_row(p, row, lane < (uint32_t)kTopK ? merged : 0, first_bad, bad_bits, hist_bad, lane,
               r24);
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
  // Measured on MI355X (HIP events per step, histories of up to 1024 ids):
  //   B=1: 32 slices; B=64: 16 slices (22.4 us; 8: 23.3, 4: 25.3, 1: 30);
  //   B=128: 4 slices (30.1 us; 8: 31.2, 2: 30.4);
  //   B=256: 1 slice (36.2 us; 2: 38.8, 4: 42.0);
  //   B=512: 1 slice (56.3 us; 2: 61.2).
  // Slices stream a row over more CUs, but each slice rescans the history and
  // a second launch merges them; from 256 rows the batch fills the GPU alone.
  if (rows == 0) return 1;
  if (rows >= 256) return 1;
  uint32_t s = rows <= 64 ? 1024u / rows : 512u / rows;
  if (s < 1) s = 1;
  if (s > kMaxSegments) s = kMaxSegments;
  return s;
}

void plan_segments(uint32_t rows, uint32_t forced_segments, uint32_t* segs, uint32_t* seg_f4) {
  uint32_t s = forced_segments ? forced_segments : segments_for_rows(rows);
  if (s > kMaxSegments) s = kMaxSegments;
  uint32_t len = (kRowF4 + s - 1) / s;
  len = (len + 7u) & ~7u;  // slices start on a 32-element bitmap word
  *seg_f4 = len;
  *segs = (kRowF4 + len - 1) / len;
}

hipError_t resident_rows(int device, uint32_t* out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static uint32_t cached[kMaxDevices];
  *out = 0;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[device] == 0) {
    int current = -1, per_cu = 0, cus = 0;
    hipError_t e = hipGetDevice(&current);
    if (e == hipSuccess && current != device) e = hipSetDevice(device);
    if (e == hipSuccess)
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, segment_kernel<kChunkF4, true>,
                                                       kBlock, 0);
    if (e == hipSuccess)
      e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (current >= 0 && current != device) (void)hipSetDevice(current);
    if (e != hipSuccess) return e;
    if (per_cu <= 0 || cus <= 0) return hipErrorInvalidValue;
    cached[device] = (uint32_t)per_cu * (uint32_t)cus;
  }
  *out = cached[device];
  return hipSuccess;
}

void plan_row_order(int device, RowParams* p) {
  p->order_from = 0;
  p->order_shift = 0;
  if (p->segs != 1 || p->hist == nullptr || p->hist_len == nullptr || p->hist_ld == 0) return;
  // The decode loop appends each sampled token to its row, so the lengths
  // the later workgroups would rank change under them: batch order there.
  if (p->row_state != nullptr || p->hist_len_out != nullptr) return;
  uint32_t resident = 0;
  if (resident_rows(device, &resident) != hipSuccess || resident == 0 || p->rows <= resident)
    return;
  // 32 to 63 buckets over the lengths a row can have (lengths are 32-bit)
  const uint64_t top = p->hist_ld < 0xffffffffull ? (uint64_t)p->hist_ld : 0xffffffffull;
  uint32_t shift = 0;
  while ((top >> shift) > 63u) ++shift;
  p->order_from = resident;
  p->order_shift = shift;
}

hipError_t launch_sample(const RowParams& p, hipStream_t stream) {
  (void)hipGetLastError();  // report only this call's launch errors
  const uint32_t blocks = p.rows * p.segs;
  if (p.segs == 1) {
    hipLaunchKernelGGL((segment_kernel<kChunkF4, true>), dim3(blocks), dim3(kBlock), 0, stream, p);
  } else {
    hipLaunchKernelGGL((segment_kernel<kChunkF4, false>), dim3(blocks), dim3(kBlock), 0, stream, p);
    hipLaunchKernelGGL(finish_kernel, dim3((p.rows + kFinishWaves - 1) / kFinishWaves),
                       dim3(64 * kFinishWaves), 0, stream,
                       p);
  }
  return hipGetLastError();
}

// Lane-exchange and wave-reduction self-test (one wave): rows 0-5 hold the
// value seen from lane ^ {1,2,4,8,16,32} for v = 7*lane + 3, rows 6-7 the
// wave maximum of 64 distinct 64-bit keys, rows 8-9 those keys sorted
// descending, row 10 the wave minimum of (13*lane mod 64) + 5.
__global__ __launch_bounds__(64) void wave_selftest_kernel(uint32_t* out) {
  const uint32_t lane = lane_id();
  const uint32_t v = lane * 7u + 3u;
  out[0 * 64 + lane] = lane_xor(v, 1, lane);
  out[1 * 64 + lane] = lane_xor(v, 2, lane);
  out[2 * 64 + lane] = lane_xor(v, 4, lane);
  out[3 * 64 + lane] = lane_xor(v, 8, lane);
  out[4 * 64 + lane] = lane_xor(v, 16, lane);
  out[5 * 64 + lane] = lane_xor(v, 32, lane);
  const uint64_t key = ((uint64_t)(lane * 2654435761u) << 32) | (lane ^ 0x55u);
  const uint64_t m = wave_max64(key);
  out[6 * 64 + lane] = (uint32_t)m;
  out[7 * 64 + lane] = (uint32_t)(m >> 32);
  const uint64_t s = wave_sort_desc(key, lane);
  out[8 * 64 + lane] = (uint32_t)s;
  out[9 * 64 + lane] = (uint32_t)(s >> 32);
  out[10 * 64 + lane] = wave_min_u32((lane * 13u) % 64u + 5u);
}

hipError_t launch_wave_selftest(uint32_t* out, hipStream_t stream) {
  (void)hipGetLastError();  // report only this call's launch errors
  hipLaunchKernelGGL(wave_selftest_kernel, dim3(1), dim3(64), 0, stream, out);
  return hipGetLastError();
}

// Element-wise device arithmetic probe: which == 0 -> expf_ref, else the
// single-logit repetition penalty.
__global__ __launch_bounds__(kBlock) void probe_kernel(int which, const uint32_t* in,
                                                      uint32_t* out, size_t n) {
  const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  out[i] = which == 0 ? b_of(expf_ref(f_of(in[i]))) : penalize_bits(in[i]);
}

hipError_t launch_probe(int which, const uint32_t* in, uint32_t* out, size_t n,
                        hipStream_t stream) {
  (void)hipGetLastError();  // report only this call's launch errors
  if (n == 0) return hipSuccess;
  const size_t blocks = (n + kBlock - 1) / kBlock;
  hipLaunchKernelGGL(probe_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0, stream, which, in,
                     out, n);
  return hipGetLastError();
}

// The XOR of a workgroup's lane values, stored to out[blockIdx.x] by one
// plain store.  (A per-wave atomic XOR at the end of every workgroup made a
// 2.5 GB read 3 % slower than a plain store: a workgroup waits for its atomic
// behind the read traffic before its slot is free.)
__device__ __forceinline__ void store_block_xor(uint32_t acc, uint32_t* out) {
  __shared__ uint32_t part[kWaves];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o);
  if ((threadIdx.x & 63u) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t x = 0;
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w) x ^= part[w];
    out[blockIdx.x] = x;
  }
}

// Read-only stream probe: each workgroup reads a contiguous run of float4
// with the sampler's access pattern (256 threads, kChunkF4 float4 per thread
// in flight, non-temporal loads) and writes one word, the XOR of what it read,
// so the loads cannot be dropped.  Its rate is the read bandwidth the
// sampler's own stream can reach on this device: the ceiling the segment
// kernel is measured against besides the datasheet peak.
__global__ __launch_bounds__(kBlock) void read_probe_kernel(const v4u* __restrict__ in,
                                                            size_t n4, size_t per_block,
                                                            uint32_t* out) {
  const size_t lo = (size_t)blockIdx.x * per_block;
  const size_t hi = lo + per_block < n4 ? lo + per_block : n4;
  uint32_t acc = 0;
  for (size_t base = lo; base < hi; base += (size_t)kBlock * kChunkF4) {
    v4u x[kChunkF4];
#pragma unroll
    for (int j = 0; j < kChunkF4; ++j) {
      const size_t f = base + (size_t)j * kBlock + threadIdx.x;
      x[j] = f < hi ? __builtin_nontemporal_load(in + f) : v4u{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < kChunkF4; ++j) acc ^= x[j].x ^ x[j].y ^ x[j].z ^ x[j].w;
  }
  store_block_xor(acc, out);
}

// The same loads in grid-stride order: the buffer is cut into chunks of
// kBlock x kChunkF4 float4 (32 KiB) and workgroup g reads chunks g,
// g + blocks, g + 2 blocks, ..., so the workgroups resident at once read one
// compact window of the buffer that moves through it.
__global__ __launch_bounds__(kBlock) void read_probe_stride_kernel(const v4u* __restrict__ in,
                                                                   size_t n4, uint32_t* out) {
  constexpr size_t kChunk = (size_t)kBlock * kChunkF4;
  uint32_t acc = 0;
  for (size_t base = (size_t)blockIdx.x * kChunk; base < n4; base += (size_t)gridDim.x * kChunk) {
    v4u x[kChunkF4];
#pragma unroll
    for (int j = 0; j < kChunkF4; ++j) {
      const size_t f = base + (size_t)j * kBlock + threadIdx.x;
      x[j] = f < n4 ? __builtin_nontemporal_load(in + f) : v4u{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < kChunkF4; ++j) acc ^= x[j].x ^ x[j].y ^ x[j].z ^ x[j].w;
  }
  store_block_xor(acc, out);
}

hipError_t launch_read_probe(const uint32_t* in, size_t n_words, uint32_t* out, uint32_t blocks,
                             bool grid_stride, hipStream_t stream) {
  (void)hipGetLastError();  // report only this call's launch errors
  const size_t n4 = n_words / 4;
  if (n4 == 0 || blocks == 0) return hipSuccess;
  if (grid_stride) {
    hipLaunchKernelGGL(read_probe_stride_kernel, dim3(blocks), dim3(kBlock), 0, stream,
                       reinterpret_cast<const v4u*>(in), n4, out);
  } else {
    const size_t per_block = (n4 + blocks - 1) / blocks;
    hipLaunchKernelGGL(read_probe_kernel, dim3(blocks), dim3(kBlock), 0, stream,
                       reinterpret_cast<const v4u*>(in), n4, per_block, out);
  }
  return hipGetLastError();
}

hipError_t launch_writeback(const WritebackParams& p, hipStream_t stream) {
  (void)hipGetLastError();  // report only this call's launch errors
  hipLaunchKernelGGL(writeback_kernel, dim3(p.rows), dim3(kBlock), 0, stream, p);
  return hipGetLastError();
}

}  // namespace pb

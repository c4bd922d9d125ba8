// pb_lmhead.hip -- fused Q4_0 LM head + decode-step sampler for gfx950.
//
// Reference arithmetic (promptboot, crates/promptboot-core/src/fp32_sse2.rs):
//   inference_prepare_q8            :956-983   hidden -> Q8_0 blocks (fp16 scale)
//   promptboot_inference_q4_block_dot :998-1062  exact int32 block dot
//   inference_q4_matvec_rows_prepared :1217-1248
//       total = add(total, mul(mul(f32(dot), w_scale), a_scale)), blocks in order
// followed by the sampler of pb_sampler.hip on the resulting logits rows.
//
// Kernels, in launch order:
//   lm_bitmap_kernel   one workgroup per row: the row's history as a 151,936-bit
//                      bitmap (global), the first bad history position.
//   lm_q8_kernel       one thread per (row, block): the Q8_0 activations and
//                      the fp32 activation scale, rows padded to 64 with zeros.
//   lm_gemm_kernel     one workgroup per (64-id vocabulary tile, 256 rows):
//                      v_mfma_i32_32x32x32_i8 gives each block's exact int32
//                      dot; the reference's per-block binary32 epilogue runs on
//                      the VALU.  Writes the raw logits and, per (row, tile),
//                      the largest penalised 64-bit selection key.
//   lm_select_kernel   one wave per row: the row's top-20 lies inside the 20
//                      tiles with the largest tile keys (each of the 20 best
//                      tile maxima is a distinct element at least as good as
//                      the 20th best of them, so every top-20 element sits in
//                      one of those tiles); it re-reads those 1,280 logits,
//                      selects exactly, and finishes the row (softmax, top-p,
//                      draw) with the sampler's finalize_row.
//
// Weight nibbles are expanded to int8 as (n ^ 8) << 4 = 16 * (n - 8); the
// factor 16 is removed exactly by pre-scaling the fp16 weight scale by 2^-4,
// so f32(16 * dot) * (w_scale / 16) rounds exactly like f32(dot) * w_scale.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pb_device.h"
#include "pb_internal.h"
#include "pb_rows.h"

#pragma clang fp contract(off)

namespace pb {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr uint32_t kBlockThreads = 256;
constexpr uint32_t kTileIds = 64;        // vocabulary ids per tile and per workgroup
constexpr uint32_t kRowsPerWave = 32;   // one 32-row MFMA tile per wave in the head
constexpr uint32_t kGemmThreads = 512;  // eight waves
constexpr uint32_t kRowsPerGroup = 256;
constexpr uint32_t kWordsPerRow = kVocab / 32;
constexpr uint32_t kTilesPerRow = kVocab / kTileIds;  // 2,374
constexpr uint32_t kCandCap = 800;       // >= 20 lanes x 38 tile keys

// cvttss2si semantics (x86 truncation): NaN and out-of-range give INT_MIN.
__device__ __forceinline__ int32_t trunc_i32_x86(float v) {
  return (v >= -2147483648.0f && v < 2147483648.0f) ? (int32_t)v : (int32_t)0x80000000;
}

// half_to_f32_bits (fp32_sse2.rs:362-376).
__device__ __forceinline__ uint32_t half_to_f32_bits(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t exponent = (h >> 10) & 0x1fu;
  const uint32_t fraction = h & 0x03ffu;
  if (exponent == 0 && fraction == 0) return sign;
  if (exponent == 0) {
    const uint32_t shift = (uint32_t)__builtin_clz(fraction) - 21u;
    const uint32_t normalized = fraction << shift;
    return sign | ((113u - shift) << 23) | ((normalized & 0x03ffu) << 13);
  }
  if (exponent == 31) return sign | 0x7f800000u | (fraction << 13);
  return sign | ((exponent + 112u) << 23) | (fraction << 13);
}

// f32_bits_to_half (fp32_sse2.rs:924-943).
__device__ __forceinline__ uint32_t f32_bits_to_half(uint32_t bits) {
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t magnitude = bits & 0x7fffffffu;
  const float scaled = f_of(magnitude) * f_of(0x77800000u);
  const uint32_t base = b_of(scaled * f_of(0x08800000u));
  const uint32_t doubled = bits + bits;
  uint32_t bias = doubled & 0xff000000u;
  if (bias < 0x71000000u) bias = 0x71000000u;
  const uint32_t rounded = b_of(f_of((bias >> 1) + 0x07800000u) + f_of(base));
  const uint32_t exponent = (rounded >> 13) & 0x7c00u;
  const uint32_t mantissa = rounded & 0x0fffu;
  if (doubled > 0xff000000u) return sign | 0x7e00u;
  return sign | (exponent + mantissa);
}

}  // namespace

// ---- repack: promptboot's Q4_0 rows -> block-major nibbles and fp16 scales ----
// in:  vocab rows of `blocks` x 18 bytes (fp16 scale, 16 nibble bytes)
// out: [blocks][vocab][16] nibble bytes, then [blocks][vocab] fp16 scales.
__global__ __launch_bounds__(kBlockThreads) void lm_pack_kernel(const uint8_t* __restrict__ in,
                                                                uint8_t* __restrict__ out,
                                                                uint32_t vocab, uint32_t blocks) {
  const size_t gid = (size_t)blockIdx.x * kBlockThreads + threadIdx.x;
  if (gid >= (size_t)vocab * blocks) return;
  const uint32_t v = (uint32_t)(gid / blocks);
  const uint32_t b = (uint32_t)(gid % blocks);
  const uint8_t* src = in + gid * 18;
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w[i] = (uint32_t)src[2 + 4 * i] | ((uint32_t)src[3 + 4 * i] << 8) |
           ((uint32_t)src[4 + 4 * i] << 16) | ((uint32_t)src[5 + 4 * i] << 24);
  }
  v4u* dst = reinterpret_cast<v4u*>(out + ((size_t)b * vocab + v) * 16);
  *dst = v4u{w[0], w[1], w[2], w[3]};
  uint16_t* scales = reinterpret_cast<uint16_t*>(out + (size_t)blocks * vocab * 16);
  scales[(size_t)b * vocab + v] = (uint16_t)(src[0] | (src[1] << 8));
}

// ---- per-row history bitmap and first bad history position ----
__global__ __launch_bounds__(kBlockThreads) void lm_bitmap_kernel(LmParams p) {
  __shared__ uint32_t bm[kWordsPerRow];
  __shared__ uint32_t bad;
  const uint32_t row = blockIdx.x;
  const uint32_t tid = threadIdx.x;
  for (uint32_t i = tid; i < kWordsPerRow; i += kBlockThreads) bm[i] = 0u;
  if (tid == 0) bad = kNone;
  __syncthreads();
  uint32_t len = 0;
  if (p.hist != nullptr && p.hist_len != nullptr) {
    len = p.hist_len[row];
    if ((size_t)len > p.hist_ld) len = (uint32_t)p.hist_ld;
  }
  const uint32_t* hrow = p.hist + (size_t)row * p.hist_ld;
  uint32_t my_bad = kNone;
  for (uint32_t q = tid; q < len; q += kBlockThreads) {
    const uint32_t id = hrow[q];
    if (id >= kVocab) {
      my_bad = q < my_bad ? q : my_bad;
    } else {
      uint32_t* word = &bm[id >> 5];
      const uint32_t bit = 1u << (id & 31u);
      if ((__hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) & bit) == 0u)
        atomicOr(word, bit);
    }
  }
  if (my_bad != kNone) atomicMin(&bad, my_bad);
  __syncthreads();
  uint32_t* out = p.bitmap + (size_t)row * kWordsPerRow;
  for (uint32_t i = tid; i < kWordsPerRow; i += kBlockThreads) out[i] = bm[i];
  if (tid == 0) {
    p.meta[row * 2 + 0] = kNone;  // first non-finite logit, lowered by the GEMM
    p.meta[row * 2 + 1] = bad;
  }
}

// ---- Q8_0 activations (inference_prepare_q8) ----
// act_q: [blocks][rows_pad][32] int8; act_s: [blocks][rows_pad] fp32 scale as
// the dot uses it (half_to_f32 of the stored fp16).  Pad rows are zero.
__global__ __launch_bounds__(kBlockThreads) void lm_q8_kernel(LmParams p) {
  const uint32_t gid = blockIdx.x * kBlockThreads + threadIdx.x;
  const uint32_t blocks = p.cols / 32u;
  if (gid >= p.rows_pad * blocks) return;
  const uint32_t row = gid / blocks;
  const uint32_t b = gid - row * blocks;
  uint32_t packed[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  float act_scale = 0.0f;
  if (row < p.rows) {
    const uint32_t* x = p.hidden + (size_t)row * p.cols + b * 32u;
    uint32_t maximum = 0u;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const uint32_t magnitude = x[e] & 0x7fffffffu;
      if (f_of(magnitude) > f_of(maximum)) maximum = magnitude;
    }
    const float scale = f_of(maximum) / f_of(0x42fe0000u);  // / 127
    const uint32_t h = f32_bits_to_half(b_of(scale));
    act_scale = f_of(half_to_f32_bits(h));
    const float inverse = b_of(scale) == 0u ? 0.0f : f_of(0x3f800000u) / scale;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const float v = f_of(x[e]) * inverse;
      const float half = (b_of(v) >> 31) == 0u ? f_of(0x3f000000u) : f_of(0xbf000000u);
      const uint32_t q = (uint32_t)trunc_i32_x86(v + half) & 0xffu;
      packed[e >> 2] |= q << (8 * (e & 3));
    }
  }
  v4u* dst = reinterpret_cast<v4u*>(p.act_q + ((size_t)b * p.rows_pad + row) * 32);
  dst[0] = v4u{packed[0], packed[1], packed[2], packed[3]};
  dst[1] = v4u{packed[4], packed[5], packed[6], packed[7]};
  p.act_s[(size_t)b * p.rows_pad + row] = act_scale;
}

// ---- the head: int8 MFMA per block + the reference's binary32 epilogue ----
// Fragment layout of v_mfma_i32_32x32x32_i8 used here (A and B share it, so
// the contraction index only has to agree between them): lane l holds row
// (A) / column (B) l % 32 and contraction elements 16 * (l / 32) + 0..15; the
// result register r of lane l is D[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32].
__global__ __launch_bounds__(kGemmThreads) void lm_gemm_kernel(LmParams p) {
  // Activation scales of every block for this group's rows (the epilogue's
  // per-row multiplier; dynamic LDS of blocks x 256 floats), and this tile's
  // two history bitmap words per row.
  extern __shared__ __align__(16) float act_scale[];
  __shared__ uint32_t hist_words[kRowsPerGroup][2];
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  const uint32_t half = lane >> 5;
  const uint32_t col = lane & 31u;
  const uint32_t tile = blockIdx.x;
  const uint32_t v0 = tile * kTileIds;
  const uint32_t group0 = blockIdx.y * kRowsPerGroup;
  const uint32_t blocks = p.cols / 32u;

  for (uint32_t i = tid; i < kRowsPerGroup * 2; i += kGemmThreads) {
    const uint32_t r = group0 + i / 2;
    (&hist_words[0][0])[i] = r < p.rows ? p.bitmap[(size_t)r * kWordsPerRow + v0 / 32 + i % 2] : 0u;
  }
  for (uint32_t i = tid; i < blocks * kRowsPerGroup; i += kGemmThreads) {
    const uint32_t b = i / kRowsPerGroup;
    const uint32_t r = group0 + (i - b * kRowsPerGroup);
    act_scale[i] = r < p.rows_pad ? p.act_s[(size_t)b * p.rows_pad + r] : 0.0f;
  }
  __syncthreads();

  const uint32_t rw0 = group0 + wave * kRowsPerWave;  // this wave's 32 rows
  if (rw0 >= p.rows_pad) return;  // whole wave idle (no barrier follows)
  const uint32_t lrow0 = wave * kRowsPerWave;       // first row inside the group

  float total[2][16];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) total[c][r] = 0.0f;

  const uint32_t nib_shift = half ? 0u : 4u;  // low nibbles for elements 0..15
  const v16i zero = {};
  const uint16_t* wscale = reinterpret_cast<const uint16_t*>(p.weights + (size_t)blocks * kVocab * 16);
  const int8_t* a_base = p.act_q + ((size_t)rw0 + col) * 32 + 16u * half;
  const uint8_t* w_base = p.weights + ((size_t)v0 + col) * 16;

  // Operands of one block: the activation fragment, both column tiles'
  // packed nibbles and weight scales.  Two sets alternate (the loop is
  // unrolled by two), so the next block's loads are in flight while the
  // current block runs and no registers are copied between iterations.
  struct Operands {
    v4i a;
    v4u raw[2];
    uint16_t wsh[2];
  };
  auto load = [&](uint32_t b, Operands& o) {
    o.a = *reinterpret_cast<const v4i*>(a_base + (size_t)b * p.rows_pad * 32);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const size_t vid = (size_t)b * kVocab + 32u * c;
      o.raw[c] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(w_base + vid * 16));
      o.wsh[c] = wscale[vid + v0 + col];
    }
  };
  auto run = [&](uint32_t b, const Operands& o) {
    // this block's 16 activation scales per lane (rows 8g + 4 * half + 0..3)
    v4f as[4];
#pragma unroll
    for (int g = 0; g < 4; ++g)
      as[g] = *reinterpret_cast<const v4f*>(
          &act_scale[b * kRowsPerGroup + lrow0 + 8u * g + 4u * half]);
    v16i d[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const v4u raw = o.raw[c];
      const v4i w = {(int)((((raw.x << nib_shift) & 0xf0f0f0f0u) ^ 0x80808080u)),
                     (int)((((raw.y << nib_shift) & 0xf0f0f0f0u) ^ 0x80808080u)),
                     (int)((((raw.z << nib_shift) & 0xf0f0f0f0u) ^ 0x80808080u)),
                     (int)((((raw.w << nib_shift) & 0xf0f0f0f0u) ^ 0x80808080u))};
      d[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a, w, zero, 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const float ws = __half2float(__ushort_as_half(o.wsh[c])) * 0.0625f;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float asv[4] = {as[g].x, as[g].y, as[g].z, as[g].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * g + j;
          const float scaled = (float)d[c][r] * ws;
          total[c][r] = total[c][r] + scaled * asv[j];
        }
      }
    }
  };

  // Loads are unconditional (the index is clamped to the last block): a load
  // under a branch makes the compiler wait for every outstanding load at the
  // join, which would serialise each block behind its own prefetch.
  // Both halves of the loop body run unconditionally (an odd last block is a
  // tail), and scheduling barriers keep each prefetch ahead of the compute it
  // overlaps: otherwise the loads are sunk next to their first use.
  const uint32_t last = blocks - 1u;
  Operands even, odd;
  load(0, even);
#pragma unroll 1
  for (uint32_t b = 0; b + 1u < blocks; b += 2) {
    load(b + 1u, odd);
    __builtin_amdgcn_sched_barrier(0);
    run(b, even);
    __builtin_amdgcn_sched_barrier(0);
    load(min(b + 2u, last), even);
    __builtin_amdgcn_sched_barrier(0);
    run(b + 1u, odd);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (blocks & 1u) run(last, even);

  // logits, non-finite check, per-row tile maximum of the penalised keys
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const uint32_t row = rw0 + 8u * (r / 4) + 4u * half + (r % 4);
    const bool live = row < p.rows;
    // The lane's better element of its two columns (the lower id on equal
    // values), kept as (value order, id, sign of zero): the largest key of
    // the row's 64 ids is then a 32-lane maximum of the value order followed
    // by a minimum of the id among the lanes holding it.
    uint32_t best_ord = 0, best_tag = 0;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const uint32_t v = v0 + 32u * c + col;
      const uint32_t xb = b_of(total[c][r]);
      if (live) {
        p.logits[(size_t)row * p.logits_ld + v] = xb;
        if ((xb & 0x7f800000u) == 0x7f800000u) atomicMin(&p.meta[row * 2], v);
      }
      const bool member = live && ((hist_words[row - group0][c] >> col) & 1u) != 0u;
      const uint32_t yb = member ? penalize_bits(xb) : xb;
      const uint32_t ord = ord_of(yb);
      if (c == 0 || ord > best_ord) {
        best_ord = ord;
        best_tag = (v << 1) | (yb == 0x80000000u ? 1u : 0u);
      }
    }
    uint32_t top_ord = best_ord;
#pragma unroll
    for (uint32_t m = 1; m < 32; m <<= 1) {
      const uint32_t o = lane_xor(top_ord, m, lane);
      top_ord = o > top_ord ? o : top_ord;
    }
    uint32_t tag = best_ord == top_ord ? best_tag : 0xffffffffu;
#pragma unroll
    for (uint32_t m = 1; m < 32; m <<= 1) {
      const uint32_t o = lane_xor(tag, m, lane);
      tag = o < tag ? o : tag;
    }
    const uint32_t low = ((0x3ffffu - (tag >> 1)) << 1) | (tag & 1u);  // make_key's low word
    if (live && col == 0) p.tilemax[(size_t)row * kTilesPerRow + tile] = ((uint64_t)top_ord << 32) | low;
  }
}

// Collects into `cand` every key of this lane (keys[0..N)) that reaches thr.
template <int N>
__device__ __forceinline__ uint32_t collect_at_least(uint64_t* cand, const uint64_t (&keys)[N],
                                                     uint64_t thr, uint32_t count) {
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const bool take = keys[j] != 0 && keys[j] >= thr;
    const uint64_t mask = __ballot(take);
    if (take) cand[count + lanes_below(mask)] = keys[j];
    count += (uint32_t)__popcll((unsigned long long)mask);
  }
  return count;
}

// ---- selection: one wave per row ----
__global__ __launch_bounds__(kBlockThreads) void lm_select_kernel(LmParams p, RowParams rp) {
  __shared__ uint64_t cand[kBlockThreads / 64][kCandCap];
  __shared__ uint64_t top[kBlockThreads / 64][kTopK];
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t row = blockIdx.x * (kBlockThreads / 64) + wave;
  if (row >= p.rows) return;
  if (row_skipped(rp, row)) {  // decode loop: the row has ended
    if (lane == 0) rp.token[row] = kNone;
    return;
  }
  const uint32_t bad_logit = p.meta[row * 2 + 0];
  const uint32_t bad_hist = p.meta[row * 2 + 1];
  if (bad_logit != kNone || bad_hist != kNone) {
    // error row: the GEMM lowered meta[0] to the first non-finite logit
    finalize_row(rp, row, 0, bad_logit, bad_hist, lane);
    return;
  }
  uint64_t* my_cand = cand[wave];
  uint64_t* my_top = top[wave];

  // 1. the 20 tiles with the largest maxima
  constexpr int kPerLane = (kTilesPerRow + 63) / 64;  // 38
  const uint64_t* tm = p.tilemax + (size_t)row * kTilesPerRow;
  uint64_t keys[kPerLane];
  uint64_t lane_best = 0;
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const uint32_t i = lane + 64u * j;
    keys[j] = i < kTilesPerRow ? tm[i] : 0;
    lane_best = keys[j] > lane_best ? keys[j] : lane_best;
  }
  uint64_t thr = shfl64(wave_sort_desc(lane_best, lane), kTopK - 1);
  uint32_t count = collect_at_least(my_cand, keys, thr, 0);
  if (lane < (uint32_t)kTopK) my_top[lane] = 0;
  __builtin_amdgcn_wave_barrier();
  merge_all(my_top, my_cand, count, lane);
  const uint64_t tile_key = lane < (uint32_t)kTopK ? my_top[lane] : 0;

  // 2. exact top-20 over those tiles' 1,280 logits
  const uint32_t* lrow = p.logits + (size_t)row * p.logits_ld;
  const uint32_t* brow = p.bitmap + (size_t)row * kWordsPerRow;
  uint64_t ek[kTopK];
  lane_best = 0;
#pragma unroll
  for (int i = 0; i < kTopK; ++i) {
    const uint32_t tile = key_id(shfl64(tile_key, (uint32_t)i)) / kTileIds;
    const uint32_t v = tile * kTileIds + lane;
    const uint32_t xb = lrow[v];
    const uint32_t yb = ((brow[v >> 5] >> (v & 31u)) & 1u) ? penalize_bits(xb) : xb;
    ek[i] = make_key(yb, v);
    lane_best = ek[i] > lane_best ? ek[i] : lane_best;
  }
  thr = shfl64(wave_sort_desc(lane_best, lane), kTopK - 1);
  __builtin_amdgcn_wave_barrier();
  count = collect_at_least(my_cand, ek, thr, 0);
  if (lane < (uint32_t)kTopK) my_top[lane] = 0;
  __builtin_amdgcn_wave_barrier();
  merge_all(my_top, my_cand, count, lane);
  const uint64_t key = lane < (uint32_t)kTopK ? my_top[lane] : 0;
  finalize_row(rp, row, key, kNone, kNone, lane);
}

// MFMA layout self-test (one wave): A[i][k] = (7i + 3k) % 17 - 8,
// B[k][j] = (5k + 11j) % 15 - 7, D written as out[32 * i + j] through the
// fragment mapping the head uses.
__global__ __launch_bounds__(64) void mfma_selftest_kernel(int32_t* out) {
  const uint32_t lane = lane_id();
  const uint32_t half = lane >> 5;
  const uint32_t idx = lane & 31u;
  uint32_t a[4] = {0u, 0u, 0u, 0u}, b[4] = {0u, 0u, 0u, 0u};
  for (uint32_t pos = 0; pos < 16; ++pos) {
    const uint32_t k = 16u * half + pos;
    const int av = (int)((7u * idx + 3u * k) % 17u) - 8;
    const int bv = (int)((5u * k + 11u * idx) % 15u) - 7;
    a[pos >> 2] |= ((uint32_t)av & 0xffu) << (8 * (pos & 3));
    b[pos >> 2] |= ((uint32_t)bv & 0xffu) << (8 * (pos & 3));
  }
  const v4i av = {(int)a[0], (int)a[1], (int)a[2], (int)a[3]};
  const v4i bv = {(int)b[0], (int)b[1], (int)b[2], (int)b[3]};
  const v16i zero = {};
  const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, zero, 0, 0, 0);
  for (int r = 0; r < 16; ++r) {
    const uint32_t i = 8u * (r / 4) + 4u * half + (r % 4);
    out[32 * i + idx] = d[r];
  }
}

hipError_t launch_lm_pack(const uint8_t* in, uint8_t* out, uint32_t vocab, uint32_t blocks,
                          hipStream_t stream) {
  const size_t n = (size_t)vocab * blocks;
  hipLaunchKernelGGL(lm_pack_kernel, dim3((uint32_t)((n + kBlockThreads - 1) / kBlockThreads)),
                     dim3(kBlockThreads), 0, stream, in, out, vocab, blocks);
  return hipGetLastError();
}

hipError_t launch_lm_sample(const LmParams& p, const RowParams& rp, hipStream_t stream) {
  hipLaunchKernelGGL(lm_bitmap_kernel, dim3(p.rows), dim3(kBlockThreads), 0, stream, p);
  const uint32_t q8_threads = p.rows_pad * (p.cols / 32u);
  hipLaunchKernelGGL(lm_q8_kernel, dim3((q8_threads + kBlockThreads - 1) / kBlockThreads),
                     dim3(kBlockThreads), 0, stream, p);
  hipLaunchKernelGGL(lm_gemm_kernel,
                     dim3(kTilesPerRow, (p.rows_pad + kRowsPerGroup - 1) / kRowsPerGroup),
                     dim3(kGemmThreads), (p.cols / 32u) * kRowsPerGroup * sizeof(float), stream,
                     p);
  hipLaunchKernelGGL(lm_select_kernel, dim3((p.rows + 3) / 4), dim3(kBlockThreads), 0, stream,
                     p, rp);
  return hipGetLastError();
}

hipError_t launch_mfma_selftest(int32_t* out, hipStream_t stream) {
  hipLaunchKernelGGL(mfma_selftest_kernel, dim3(1), dim3(64), 0, stream, out);
  return hipGetLastError();
}

}  // namespace pb

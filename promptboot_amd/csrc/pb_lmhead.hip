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
//   lm_quant_kernel    (more than kFusedQuantRows rows) eight lanes per
//                      (row, block): the Q8_0 activations in the head's
//                      contraction order and the fp32 activation scales (for
//                      the Q4_0 head divided by 16), zeros for padding rows.
//   lm_gemm_kernel     one workgroup per (64-id vocabulary tile, 128 rows):
//                      v_mfma_i32_16x16x32_i8 gives each block's exact int32
//                      dot; the reference's per-block binary32 epilogue runs on
//                      the VALU.  With a logits buffer it writes the raw logits
//                      and, per (row, tile), the order word of the largest raw
//                      logit; without one (kLogits false: one pass) it writes
//                      no logits, only that word and the tile's second word (a
//                      bound on its other logits and the maximum's index).
//   lm_gemm_narrow_kernel  the same for up to 64 rows, one wave per tile,
//                      logits always written (to the workspace if the caller
//                      keeps none) with both words; with up to
//                      kFusedQuantRows rows each workgroup quantises the
//                      activations itself (no lm_quant_kernel).
//   lm_select_kernel   one workgroup per row: the history bitmap in LDS, then
//                      the exact top-20 of the penalised logits best-first
//                      over the tiles (the penalty never raises a value, so a
//                      tile's raw maximum bounds its penalised elements), and
//                      the row's finish (softmax, top-p, draw) with the
//                      sampler's finalize_row.  A tile whose second word says
//                      that only its maximum can reach the threshold gives
//                      that element from its words; the other tiles it reads
//                      are read from the logits, or in one pass recomputed from
//                      the packed head with the head's own arithmetic.
//
// Weight nibbles are stored XOR 8 and expanded to int8 by masking them into
// the high half of a byte: (n ^ 8) << 4 = 16 * (n - 8) as a signed byte.  The
// factor 16 is removed exactly in the epilogue (below).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "pb_device.h"
#include "pb_internal.h"
#include "pb_rows.h"

#pragma clang fp contract(off)

namespace pb {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

constexpr uint32_t kBlockThreads = 256;
constexpr uint32_t kTileIds = 64;        // vocabulary ids per tile and per workgroup
constexpr uint32_t kRowsPerWave = 32;   // two 16-row MFMA row tiles per wave in the head
constexpr uint32_t kGemmThreads = 256;  // four waves
// Rows per workgroup of the wide GEMM.  Against 256 rows with eight waves the
// 128-row, four-wave workgroups spread the launch's last workgroups over more
// CUs: B = 256 Q4_0 one-pass GEMM 106.6 -> 103.7 us, Q8_0 116.5 -> 112.7 us
// (same box, traced).  16 or 64 rows per wave were slower (+9 % and +2.5 %:
// the nibble unpacking is shared by a wave's rows; 64 rows need 213 VGPRs).
constexpr uint32_t kRowsPerGroup = 128;
// Batches up to kNarrowRows take lm_gemm_narrow_kernel (measured per step,
// Q4_0 / Q8_0: B = 64 74.8 / 73.7 us against 92.0 / 98.1 with the wide kernel;
// B = 128 119.2 / 121.9 against 103.6 / 108.6).
constexpr uint32_t kWordsPerRow = kVocab / 32;
// Blocks of 32 in Qwen2.5-0.5B's hidden state of 896: the width whose block
// loops are unrolled whole.
constexpr uint32_t kModelBlocks = 28;
constexpr uint32_t kTilesPerRow = kVocab / kTileIds;  // 2,374
constexpr uint32_t kTileBytes = kTileIds * 16;    // packed Q4_0 nibbles of one (block, tile)
constexpr uint32_t kTileBytesQ8 = kTileIds * 32;  // packed Q8_0 weights of one (block, tile)
// M = 1.5 * 2^23: its binade has unit spacing, so M + i is exact for |i| < 2^22.
constexpr uint32_t kMagicBits = 0x4b400000u;
// Word 3 of a buffer resource on gfx9-family parts: 32-bit data format (a
// raw buffer load needs a valid format), no swizzle, no stride.
constexpr int kBufferFlags = 0x00020000;
// Cache policy of a buffer store: non-temporal (the "nt" bit).
constexpr int kNonTemporal = 2;
constexpr float kMagic = 12582912.0f;

// Maximum over the 16 lanes of a DPP row (lanes 16r .. 16r+15), in every
// lane of the row: quad_perm [1,0,3,2] and [2,3,0,1] combine a quad, row
// rotations by 4 and 8 combine the four quads.  The moved value's `old` is 0,
// the identity of an unsigned maximum, so each step folds into one
// v_max_u32 with a DPP operand.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_or_zero(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xF, 0xF, true);
}
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  v = max(v, dpp_or_zero<0xB1>(v));
  v = max(v, dpp_or_zero<0x4E>(v));
  v = max(v, dpp_or_zero<0x124>(v));
  return max(v, dpp_or_zero<0x128>(v));
}
// The same minimum (every source lane of these patterns is in the row).
__device__ __forceinline__ uint32_t row16_min_u32(uint32_t v) {
  v = min(v, dpp_or_zero<0xB1>(v));
  v = min(v, dpp_or_zero<0x4E>(v));
  v = min(v, dpp_or_zero<0x124>(v));
  return min(v, dpp_or_zero<0x128>(v));
}

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

// ---- repack: promptboot's Q4_0 rows -> the head's tile layout ----
// in:  vocab rows of `blocks` x 18 bytes (fp16 scale, 16 nibble bytes: byte j
//      holds element j in the low and element 16 + j in the high nibble).
// out: [blocks][vocab / 64 tiles][1 KB] nibbles, then [blocks][vocab] fp16
//      scales, then one word per tile, non-zero when one of the tile's scales
//      is infinite or NaN (cleared by lm_clear_kernel before the launch).  In the kilobyte of (block b, tile t), lane l = 16 q + n of a
//      head wave reads the 16 bytes at 16 l: word c of them is bytes
//      4q .. 4q+3 of id 64 t + 4 n + c, every nibble XOR 8.  vocab % 64 == 0.
__global__ __launch_bounds__(kBlockThreads) void lm_pack_kernel(const uint8_t* __restrict__ in,
                                                                uint8_t* __restrict__ out,
                                                                uint32_t vocab, uint32_t blocks) {
  const size_t gid = (size_t)blockIdx.x * kBlockThreads + threadIdx.x;
  if (gid >= (size_t)vocab * blocks) return;
  const uint32_t v = (uint32_t)(gid / blocks);
  const uint32_t b = (uint32_t)(gid % blocks);
  const uint8_t* src = in + gid * 18;
  const uint32_t t = v / kTileIds;
  const uint32_t n = (v % kTileIds) / 4u;
  const uint32_t c = v % 4u;
  uint32_t* tile = reinterpret_cast<uint32_t*>(out + ((size_t)b * (vocab / kTileIds) + t) * kTileBytes);
#pragma unroll
  for (uint32_t q = 0; q < 4; ++q) {
    const uint32_t w = (uint32_t)src[2 + 4 * q] | ((uint32_t)src[3 + 4 * q] << 8) |
                       ((uint32_t)src[4 + 4 * q] << 16) | ((uint32_t)src[5 + 4 * q] << 24);
    tile[(q * 16u + n) * 4u + c] = w ^ 0x88888888u;
  }
  uint16_t* scales = reinterpret_cast<uint16_t*>(out + (size_t)blocks * vocab * 16);
  const uint16_t h = (uint16_t)(src[0] | (src[1] << 8));
  scales[(size_t)b * vocab + v] = h;
  // tiles with an infinite or NaN weight scale (the flags start at zero)
  if ((h & 0x7c00u) == 0x7c00u) {
    uint32_t* flags = reinterpret_cast<uint32_t*>(scales + (size_t)blocks * vocab);
    atomicOr(&flags[t], 1u);
  }
}

__global__ __launch_bounds__(kBlockThreads) void lm_clear_kernel(uint32_t* words, uint32_t n) {
  const uint32_t i = blockIdx.x * kBlockThreads + threadIdx.x;
  if (i < n) words[i] = 0u;
}

// ---- repack: promptboot's Q8_0 rows -> the head's tile layout ----
// in:  vocab rows of `blocks` x 34 bytes (fp16 scale, 32 signed weights; the
//      output tensor of model.rs:817-818).
// out: [blocks][vocab / 64 tiles][2 KB] weights, then [blocks][vocab] fp16
//      scales.  In the 2 KB of (block b, tile t), lane l = 16 q + n of a head
//      wave reads the 32 bytes at 32 l: bytes 8c .. 8c+7 of them are weights
//      4q .. 4q+3 and 16+4q .. 16+4q+3 of id 64 t + 4 n + c, the contraction
//      order of the activations.  vocab % 64 == 0.
__global__ __launch_bounds__(kBlockThreads) void lm_pack_q8_kernel(const uint8_t* __restrict__ in,
                                                                   uint8_t* __restrict__ out,
                                                                   uint32_t vocab, uint32_t blocks) {
  const size_t gid = (size_t)blockIdx.x * kBlockThreads + threadIdx.x;
  if (gid >= (size_t)vocab * blocks) return;
  const uint32_t v = (uint32_t)(gid / blocks);
  const uint32_t b = (uint32_t)(gid % blocks);
  const uint8_t* src = in + gid * 34;
  const uint32_t t = v / kTileIds;
  const uint32_t n = (v % kTileIds) / 4u;
  const uint32_t c = v % 4u;
  uint8_t* tile = out + ((size_t)b * (vocab / kTileIds) + t) * kTileBytesQ8;
#pragma unroll
  for (uint32_t q = 0; q < 4; ++q) {
    uint8_t* dst = tile + (q * 16u + n) * 32u + c * 8u;
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e) {
      dst[e] = src[2 + 4 * q + e];
      dst[4 + e] = src[2 + 16 + 4 * q + e];
    }
  }
  uint16_t* scales = reinterpret_cast<uint16_t*>(out + (size_t)blocks * vocab * 32);
  scales[(size_t)b * vocab + v] = (uint16_t)(src[0] | (src[1] << 8));
}

// ---- Q8_0 activations of one block (inference_prepare_q8) ----
// The 32 quants of one block of 32 activations in the head's contraction
// order (bytes 8q .. 8q+7 hold elements 4q .. 4q+3 and 16+4q .. 16+4q+3,
// q = 0..3), and the fp32 scale the dot uses (half_to_f32 of the stored fp16)
// times 2^-4, which is exact.  A padding row (live == false) gives zeros.
__device__ __forceinline__ void quantize_block(const uint32_t (&x)[32], bool live,
                                               uint32_t (&packed)[8], float& scale16) {
#pragma unroll
  for (int k = 0; k < 8; ++k) packed[k] = 0u;
  float act_scale = 0.0f;
  if (live) {
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
      packed[2 * ((e & 15) >> 2) + (e >> 4)] |= q << (8 * (e & 3));
    }
  }
  scale16 = act_scale * 0.0625f;
}

// The 32 activations of (row, block b) as binary32 words, 16-byte loads.
__device__ __forceinline__ void load_block(const LmParams& p, uint32_t row, uint32_t b,
                                           uint32_t (&x)[32]) {
  const v4u* src = reinterpret_cast<const v4u*>(p.hidden + (size_t)row * p.cols + b * 32u);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const v4u v = src[k];
    x[4 * k + 0] = v.x;
    x[4 * k + 1] = v.y;
    x[4 * k + 2] = v.z;
    x[4 * k + 3] = v.w;
  }
}

// ---- Q8_0 activations of every (row, block), batches above kFusedQuantRows ----
// act_q: [blocks][rows_pad][32] int8 in the contraction order; act_s:
// [blocks][rows_pad] scales, a_scale / 16 for the Q4_0 head and a_scale for
// the Q8_0 head (the forms their epilogues take).  Padding rows are zero.  Eight lanes per
// (row, block), four activations each (one 16-byte load): lane l holds
// elements 4l .. 4l+3, which are exactly packed word 2l (l < 4) or 2(l-4)+1 of
// the contraction order.  The block's largest magnitude (NaN ignored, as
// quantize_block does) is a maximum over the eight lanes; the arithmetic per
// element is quantize_block's.
__global__ __launch_bounds__(kBlockThreads) void lm_quant_kernel(LmParams p) {
  const uint32_t blocks = p.cols / 32u;
  const uint32_t g = blockIdx.x * (kBlockThreads / 8u) + threadIdx.x / 8u;  // (row, block)
  const uint32_t l = threadIdx.x & 7u;
  const uint32_t lane = threadIdx.x & 63u;
  const bool in_range = g < p.rows_pad * blocks;
  const uint32_t row = in_range ? g / blocks : 0u;
  const uint32_t b = in_range ? g - row * blocks : 0u;
  const bool live = in_range && row < p.rows;
  v4u v = {0u, 0u, 0u, 0u};
  if (live) v = *reinterpret_cast<const v4u*>(p.hidden + (size_t)row * p.cols + b * 32u + 4u * l);
  const uint32_t x[4] = {v.x, v.y, v.z, v.w};
  // magnitudes as order-preserving integers (non-negative floats), NaN as 0
  uint32_t maximum = 0u;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t magnitude = x[e] & 0x7fffffffu;
    maximum = magnitude > 0x7f800000u ? maximum : max(maximum, magnitude);
  }
  maximum = max(maximum, lane_xor(maximum, 1, lane));
  maximum = max(maximum, lane_xor(maximum, 2, lane));
  maximum = max(maximum, lane_xor(maximum, 4, lane));
  const float scale = f_of(maximum) / f_of(0x42fe0000u);  // / 127
  const uint32_t h = f32_bits_to_half(b_of(scale));
  const float act_scale = f_of(half_to_f32_bits(h));
  const float inverse = b_of(scale) == 0u ? 0.0f : f_of(0x3f800000u) / scale;
  uint32_t word = 0u;
  if (live) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float q = f_of(x[e]) * inverse;
      const float half = (b_of(q) >> 31) == 0u ? f_of(0x3f000000u) : f_of(0xbf000000u);
      word |= ((uint32_t)trunc_i32_x86(q + half) & 0xffu) << (8 * e);
    }
  }
  if (in_range) {
    const uint32_t w = l < 4u ? 2u * l : 2u * (l - 4u) + 1u;
    reinterpret_cast<uint32_t*>(p.act_q + ((size_t)b * p.rows_pad + row) * 32)[w] = word;
    // the Q4_0 epilogue takes a_scale / 16 (exact), the Q8_0 one a_scale
    if (l == 0u)
      p.act_s[(size_t)b * p.rows_pad + row] = live ? (p.q8 ? act_scale : act_scale * 0.0625f) : 0.0f;
  }
}

// Tile word of a row whose 64 logits in the tile include an infinite or NaN
// one (above every finite order word, which is at most 0xff7fffff).
constexpr uint32_t kNonFiniteTile = 0xffffffffu;

// Order word of a finite binary32 value: adding +0 turns -0 into +0, then
// negative values are inverted (so -0 and +0 share 0x80000000).
__device__ __forceinline__ uint32_t order_word(float y) {
  const uint32_t w = b_of(y + 0.0f);
  return w ^ ((uint32_t)((int32_t)w >> 31) | 0x80000000u);
}
// The binary32 bits of a nonzero order word.
__device__ __forceinline__ uint32_t order_word_bits(uint32_t w) {
  return (w & 0x80000000u) ? (w & 0x7fffffffu) : ~w;
}
// Second word of a tile (kSecond): the tile's other logits all have order
// words below (word & ~63), and the maximum is element word & 63 of the tile
// (its lowest, among ties).  A tie at the maximum, or a maximum of zero (whose
// sign the order word does not keep), gives a bound above the maximum.
constexpr uint32_t kSecondIndexMask = 63u;

// The lane's part of a tile word: the order word of the largest of its four
// logits, kNonFiniteTile when one of them is infinite or NaN (y * 0 is NaN
// exactly then).  The tile word is the maximum over the tile's 16 lanes.
// The largest of four values is only used when all four are finite, so it
// is taken with v_max3_f32 and v_max_f32 as they are: fmaxf would first
// quieten a signalling NaN in each two-operand maximum's inputs (one more
// instruction per operand).
__device__ __forceinline__ uint32_t lane_tile_word(const float (&y)[4]) {
  const float probe = __builtin_fmaf(
      y[0], 0.0f, __builtin_fmaf(y[1], 0.0f, __builtin_fmaf(y[2], 0.0f, y[3] * 0.0f)));
  float m;
  __asm__("v_max3_f32 %0, %1, %2, %3\n\tv_max_f32 %0, %0, %4"
          : "=&v"(m)
          : "v"(y[0]), "v"(y[1]), "v"(y[2]), "v"(y[3]));
  return probe != probe ? kNonFiniteTile : order_word(m);
}
// The tile's second word, given the tile word and the lane's four order
// words (ids 4n .. 4n+3 of the tile); every lane of the 16-lane row returns it.
__device__ __forceinline__ uint32_t tile_second_word(const uint32_t (&ow)[4], uint32_t word,
                                                     uint32_t n) {
  // the maximum's lowest index, then the largest word of the others
  uint32_t e = 0xffu;
#pragma unroll
  for (int c = 3; c >= 0; --c) e = ow[c] == word ? 4u * n + (uint32_t)c : e;
  const uint32_t first = row16_min_u32(e);
  uint32_t other = 0;
#pragma unroll
  for (int c = 0; c < 4; ++c) other = max(other, 4u * n + (uint32_t)c != first ? ow[c] : 0u);
  other = row16_max_u32(other);
  if (word == 0x80000000u) other = word;
  return (((other >> 6) + 1u) << 6) | (first & kSecondIndexMask);
}

// ---- a wave's results for one 64-id tile ----
// total[rt][c][i] is row base_row + lane_row + 16 rt + i, id 64 tile + 4n + c,
// where base_row is the first row of the wave's group of group_rows rows and
// lane_row the lane's row of step 0 inside it (lanes 16q .. 16q+15 hold rows
// 4q + i of each row tile, four consecutive ids per lane).  For the real rows among
// result registers i < kI: stores the raw logits and the order word of the
// tile's largest raw logit (kNonFiniteTile when one of them is infinite or
// NaN), and with kSecond the tile's second word.  The repetition penalty is
// not applied here: the selection applies it to the few tiles it reads (it
// never raises a value, so the raw maximum bounds the penalised ones).
// The logits go out as buffer stores over the group's real rows: a padding
// row's store falls outside the buffer and is dropped, so no store needs a
// row test, and each address is the lane's 32-bit offset plus the step's.
// They are non-temporal: the selection reads a few
// tiles of them, and ordinary stores of a 256-row step (155.6 MB) evict the
// packed weights that a workgroup's waves share through the L2.
// Measured per 256-row step: Q8_0 161.3-162.0 -> 142.1-149.8 us, Q4_0 about
// even (128.9-130.0 -> 129.4-134.9 us, HIP events 129.0-131.5 ->
// 129.4-130.4 us).
template <int kRT, int kI, bool kSecond>
__device__ __forceinline__ void write_tile(const LmParams& p, const float (&total)[kRT][4][4],
                                           uint32_t base_row, uint32_t group_rows,
                                           uint32_t lane_row, uint32_t tile, uint32_t n) {
  constexpr int kSteps = kRT * kI;
  const uint32_t v0 = tile * kTileIds;
  // the LM heads' logits are [rows][PB_VOCAB]: a group's rows span at most
  // 256 x 151,936 words
  const uint32_t ld = (uint32_t)p.logits_ld;
  const uint32_t real = p.rows > base_row ? min(p.rows - base_row, group_rows) : 0u;
  const __amdgpu_buffer_rsrc_t logits = __builtin_amdgcn_make_buffer_rsrc(
      p.logits + (size_t)base_row * ld, (short)0, (int)(real * ld * 4u), kBufferFlags);
  const uint32_t lane_off = (lane_row * ld + v0 + 4u * n) * 4u;
  uint32_t o[kSteps];
  uint32_t ow[kSteps][4];
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int rt = s / kI, i = s % kI;
    const float y[4] = {total[rt][0][i], total[rt][1][i], total[rt][2][i], total[rt][3][i]};
    __builtin_amdgcn_raw_buffer_store_b128(v4u{b_of(y[0]), b_of(y[1]), b_of(y[2]), b_of(y[3])},
                                           logits, lane_off + (uint32_t)(16 * rt + i) * ld * 4u, 0,
                                           kNonTemporal);
    o[s] = lane_tile_word(y);
    if constexpr (kSecond) {
#pragma unroll
      for (int c = 0; c < 4; ++c) ow[s][c] = order_word(y[c]);
    }
  }
#pragma unroll
  for (int s = 0; s < kSteps; ++s) o[s] = row16_max_u32(o[s]);
  uint32_t sec[kSteps];
  if constexpr (kSecond) {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) sec[s] = tile_second_word(ow[s], o[s], n);
  }
  if (n != 0u) return;
  if constexpr (kSecond) {
    // the narrow GEMM: plain stores of the real rows' words (its one-row
    // step measured 0.3 us slower with the buffer stores below)
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const uint32_t row = base_row + lane_row + 16u * (uint32_t)(s / kI) + (uint32_t)(s % kI);
      if (row < p.rows) {
        p.tilemax[(size_t)row * kTilesPerRow + tile] = o[s];
        p.tilesec[(size_t)row * kTilesPerRow + tile] = sec[s];
      }
    }
  } else {
    // the tile words through a resource over the same real rows: a store of
    // a padding row falls outside it and is dropped (no row test, 32-bit
    // offsets: 21 fewer VALU instructions per wave of the wide GEMM)
    const __amdgpu_buffer_rsrc_t tm = __builtin_amdgcn_make_buffer_rsrc(
        p.tilemax + (size_t)base_row * kTilesPerRow, (short)0, (int)(real * kTilesPerRow * 4u),
        kBufferFlags);
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const uint32_t row = lane_row + 16u * (uint32_t)(s / kI) + (uint32_t)(s % kI);
      __builtin_amdgcn_raw_buffer_store_b32(o[s], tm, (row * kTilesPerRow + tile) * 4u, 0, 0);
    }
  }
}

// ---- the wide GEMM's tail when the caller keeps no logits (one pass) ----
// Per (row, 64-id tile) the tile word as write_tile gives it and the second
// word (kSecondIndexMask), with no logits written: the selection recomputes
// the few tiles whose second word reaches its threshold from the packed head.
// A lane takes the largest m and second largest s of its four values
// (v_max3 / v_med3), and the index c of m (the lowest, among ties); across
// the 16 lanes the tile word is the largest order word, the maximum's index
// the lowest 4 n + c among the lanes holding it, and the bound on the other
// logits the largest of the other lanes' maxima and that lane's s (a tie at
// the maximum, in a lane or across lanes, makes the bound reach the tile
// word).  The sign of a zero maximum is not kept: the selection reads a tile
// whose word is the order word of zero.  Stores through resources over the
// group's real rows, as write_tile's.
template <int kRT, int kI>
__device__ __forceinline__ void write_tile_words(const LmParams& p,
                                                 const float (&total)[kRT][4][4],
                                                 uint32_t base_row, uint32_t group_rows,
                                                 uint32_t lane_row, uint32_t tile, uint32_t n) {
  constexpr int kSteps = kRT * kI;
  uint32_t o[kSteps], sw[kSteps], at[kSteps];
#pragma unroll
  for (int st = 0; st < kSteps; ++st) {
    const int rt = st / kI, i = st % kI;
    const float y0 = total[rt][0][i], y1 = total[rt][1][i], y2 = total[rt][2][i],
                y3 = total[rt][3][i];
    const float probe = __builtin_fmaf(
        y0, 0.0f, __builtin_fmaf(y1, 0.0f, __builtin_fmaf(y2, 0.0f, y3 * 0.0f)));
    // (the finite case is the only one used: no quietening of NaN operands)
    float m3, md, lo, m, s2;
    __asm__("v_max3_f32 %0, %1, %2, %3" : "=v"(m3) : "v"(y0), "v"(y1), "v"(y2));
    __asm__("v_med3_f32 %0, %1, %2, %3" : "=v"(md) : "v"(y0), "v"(y1), "v"(y2));
    __asm__("v_min_f32 %0, %1, %2" : "=v"(lo) : "v"(m3), "v"(y3));
    __asm__("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(m3), "v"(y3));
    __asm__("v_max_f32 %0, %1, %2" : "=v"(s2) : "v"(md), "v"(lo));
    uint32_t c = y2 == m ? 2u : 3u;
    c = y1 == m ? 1u : c;
    c = y0 == m ? 0u : c;
    o[st] = probe != probe ? kNonFiniteTile : order_word(m);
    sw[st] = order_word(s2);
    at[st] = 4u * n + c;
  }
  uint32_t word[kSteps], sec[kSteps];
#pragma unroll
  for (int st = 0; st < kSteps; ++st) word[st] = row16_max_u32(o[st]);
#pragma unroll
  for (int st = 0; st < kSteps; ++st) {
    const uint32_t idx = row16_min_u32(o[st] == word[st] ? at[st] : 0xffu);
    const uint32_t other = row16_max_u32(at[st] == idx ? sw[st] : o[st]);
    sec[st] = ((other & ~kSecondIndexMask) + 64u) | idx;
  }
  if (n != 0u) return;
  const uint32_t real = p.rows > base_row ? min(p.rows - base_row, group_rows) : 0u;
  const __amdgpu_buffer_rsrc_t tm = __builtin_amdgcn_make_buffer_rsrc(
      p.tilemax + (size_t)base_row * kTilesPerRow, (short)0, (int)(real * kTilesPerRow * 4u),
      kBufferFlags);
  const __amdgpu_buffer_rsrc_t ts = __builtin_amdgcn_make_buffer_rsrc(
      p.tilesec + (size_t)base_row * kTilesPerRow, (short)0, (int)(real * kTilesPerRow * 4u),
      kBufferFlags);
#pragma unroll
  for (int st = 0; st < kSteps; ++st) {
    const uint32_t row = lane_row + 16u * (uint32_t)(st / kI) + (uint32_t)(st % kI);
    __builtin_amdgcn_raw_buffer_store_b32(word[st], tm, (row * kTilesPerRow + tile) * 4u, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b32(sec[st], ts, (row * kTilesPerRow + tile) * 4u, 0, 0);
  }
}

// ---- the head: int8 MFMA per block + the reference's binary32 epilogue ----
// Fragment layout of v_mfma_i32_16x16x32_i8 (A and B alike, so only the
// contraction index has to agree between them): lane l holds row (A) /
// column (B) l % 16 and eight contraction slots 8 (l / 16) + 0..7 as one
// 64-bit operand; result register i of lane l is D[4 (l / 16) + i][l % 16].
// Slots 8q .. 8q+3 carry block elements 4q .. 4q+3 and slots 8q+4 .. 8q+7 the
// elements 16+4q .. 16+4q+3, so one packed weight word gives both halves of a
// lane's B operand: its low nibbles and its high nibbles.  MFMA column n of
// column tile c is vocabulary id v0 + 4n + c: a lane's four columns are four
// consecutive ids.
//
// Epilogue without an int -> float conversion: the accumulator starts at the
// bit pattern of M = 1.5 * 2^23, so each result word read as binary32 is
// exactly M + 16 dot (|16 dot| < 2^19).  fma(M + 16 dot, ws, -M ws) is then
// 16 dot ws rounded once (M ws is exact: ws has at most 11 significant bits),
// which is 16 times the reference's mul(f32(dot), ws); its product with
// a_scale / 16 (from quantize_block) is the reference's
// mul(mul(f32(dot), ws), a_scale) bit for bit.  Scaling by powers of two is
// exact here: |16 dot ws| is 0 or lies in [2^-20, 2^36), far from the
// subnormal and overflow ranges.  A tile with an infinite or NaN fp16 weight
// scale uses (x - M) * ws instead, which gives inf * 0 = NaN as the
// reference does.
//
// The Q8_0 head (kQ8) reads both 4-byte halves of each B operand from the
// packed weights as they are, starts the accumulator at zero and follows
// inference_q8_matvec_rows_prepared (fp32_sse2.rs:1251-1280):
// add(total, mul(f32(dot), mul(ws, a_scale))), four VALU ops per value.  (The
// scales are both fp16 values, so ws * a_scale is exact, with at most 22
// significant bits.  Folding the conversion into an FMA as above would work,
// but it needs -M * ws * a_scale per value: one op either way.)
//
// kNB, when not 0, is the number of blocks (the hidden width / 32) known at
// compile time: the Q4_0 block loop is then unrolled whole, so the LDS
// addresses of the scales are immediate offsets (Q4_0 one-pass GEMM at the
// model's width of 896: 102.5 -> 100.4 us, same box, traced).
template <bool kQ8, bool kLogits, uint32_t kNB = 0>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(4))) void lm_gemm_kernel(LmParams p) {
  // Dynamic LDS: the activation scales / 16 of every block for the group's
  // 128 rows, then this tile's weight scales and -M * weight scales by block.
  extern __shared__ __align__(16) float lds[];
  const uint32_t blocks = kNB != 0 ? kNB : p.cols / 32u;
  float* act_scale = lds;
  float* w_scale = lds + blocks * kRowsPerGroup;
  float* w_neg = w_scale + blocks * kTileIds;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  const uint32_t n = lane & 15u;  // MFMA row (A) / column (B)
  const uint32_t q = lane >> 4;   // contraction quarter; result rows 4q .. 4q+3
  // Consecutive tiles run on the same XCD (xcd_contiguous_item): every
  // (row, tile) gets one or two 4-byte words in row-major arrays, and the
  // words of up to eight neighbouring tiles share a 32-byte sector, which
  // leaves an XCD's L2 whole only when the neighbours were written through
  // that L2.  With tile = block index the neighbours sat on eight different
  // XCDs: 8 x the words' bytes written (39.7 MB instead of 4.9 MB per
  // 256-row one-pass step, WRITE_SIZE).  The row groups of one tile are
  // consecutive items, so they run on one XCD at about the same time and the
  // head leaves HBM once (group-major items read it once per group).
  const uint32_t item = xcd_contiguous_item(blockIdx.x + blockIdx.y * gridDim.x,
                                            gridDim.x * gridDim.y);
  const uint32_t tile = item / gridDim.y;
  const uint32_t v0 = tile * kTileIds;
  const uint32_t group0 = item % gridDim.y * kRowsPerGroup;
  const uint16_t* wscale16 =
      reinterpret_cast<const uint16_t*>(p.weights + (size_t)blocks * kVocab * (kQ8 ? 32 : 16));

  const uint32_t rw0 = group0 + wave * kRowsPerWave;  // this wave's 32 rows
  const bool live = rw0 < p.rows_pad;                 // else the whole wave idles
  const v4i magic = {(int)kMagicBits, (int)kMagicBits, (int)kMagicBits, (int)kMagicBits};
  constexpr uint32_t kWords = kQ8 ? 2u : 1u;  // uint4 of packed weights per lane and block
  constexpr uint32_t kTile = kQ8 ? kTileBytesQ8 : kTileBytes;
  // The operands are buffer loads: a lane's byte offset is fixed, the block's
  // offset is a scalar, so a load costs no VALU address arithmetic (three to
  // five instructions per block otherwise).  Widths of at most 2048 keep the
  // packed head under 330 MB, and the activations of at most
  // PB_LMHEAD_MAX_ROWS rows (the host refuses more) take blocks * rows_pad * 32
  // <= 512 MB, so every offset and resource size fits in 31 bits.
  const uint32_t w_stride = kTilesPerRow * kTile;  // bytes per block
  const uint32_t w_off = tile * kTile + 16u * kWords * lane;
  const uint32_t a_stride = p.rows_pad * 32u;  // bytes per block
  const uint32_t a_off = (rw0 + n) * 32u + 8u * q;
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(p.weights), (short)0, (int)(blocks * w_stride), kBufferFlags);
  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(p.act_q), (short)0, (int)(blocks * a_stride), kBufferFlags);

  // Operands of one block: both row tiles' activation fragments and the
  // lane's packed weight words (one per column tile).  Two sets alternate
  // (the loop is unrolled by two), so the next block's loads are in flight
  // while the current block runs and no registers are copied.
  struct Operands {
    uint64_t a[2];
    v4u raw[kWords];
  };
  auto load = [&](uint32_t b, Operands& o) {
    const uint32_t ab = b * a_stride;
#pragma unroll
    for (uint32_t rt = 0; rt < 2; ++rt) {
      const v2u x = __builtin_amdgcn_raw_buffer_load_b64(a_rsrc, a_off + 16u * 32u * rt, ab, 0);
      o.a[rt] = (uint64_t)x.x | ((uint64_t)x.y << 32);
    }
    const uint32_t wb = b * w_stride;
#pragma unroll
    for (uint32_t k = 0; k < kWords; ++k)
      o.raw[k] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, w_off + 16u * k, wb, 0);
  };
  // The first blocks' operands are requested before the scales are staged,
  // so their latency overlaps the staging and its barrier.
  Operands s0, s1, s2;
  const uint32_t last = blocks - 1u;
  if (live) {
    load(0, s0);
    if (kQ8) load(min(1u, last), s1);
  }

  // Staged four values per thread and load: the weight scales of four
  // consecutive ids (8 bytes), the activation scales of four consecutive rows
  // (16 bytes; rows_pad is a multiple of 64, so four rows are all inside the
  // padded batch or all past it).  lm_quant_kernel stores a_scale / 16 for the
  // Q4_0 epilogue and a_scale for the Q8_0 one.
  for (uint32_t j = tid; j < blocks * (kTileIds / 4u); j += kGemmThreads) {
    const uint32_t b = j / (kTileIds / 4u);
    const uint32_t c = j - b * (kTileIds / 4u);
    const uint64_t h4 = *reinterpret_cast<const uint64_t*>(wscale16 + b * kVocab + v0 + 4u * c);
    v4f ws;
#pragma unroll
    for (int k = 0; k < 4; ++k) ws[k] = __half2float(__ushort_as_half((unsigned short)(h4 >> (16 * k))));
    *reinterpret_cast<v4f*>(&w_scale[4u * j]) = ws;
    if constexpr (!kQ8) *reinterpret_cast<v4f*>(&w_neg[4u * j]) = ws * -kMagic;
  }
  // Activation scales: four 16-byte loads per thread and pass, all requested
  // before any is stored.  Rows past the padded batch (only idle waves use
  // them) read at the end of the resource, which returns zeros.
  const uint32_t as_bytes = blocks * p.rows_pad * 4u;
  const __amdgpu_buffer_rsrc_t s_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      p.act_s, (short)0, (int)as_bytes, kBufferFlags);
  constexpr uint32_t kQuads = kRowsPerGroup / 4u;  // four rows per load
  const uint32_t quads = blocks * kQuads;
  for (uint32_t j0 = tid; j0 < quads; j0 += 4u * kGemmThreads) {
    v4u as[4];
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
      const uint32_t j = j0 + k * kGemmThreads;
      const uint32_t r = group0 + 4u * (j % kQuads);
      const uint32_t off = r < p.rows_pad ? ((j / kQuads) * p.rows_pad + r) * 4u : as_bytes;
      as[k] = __builtin_amdgcn_raw_buffer_load_b128(s_rsrc, off, 0, 0);
    }
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
      const uint32_t j = j0 + k * kGemmThreads;
      if (j < quads) *reinterpret_cast<v4u*>(&act_scale[4u * j]) = as[k];
    }
  }
  __syncthreads();
  // a Q4_0 tile with an infinite or NaN weight scale (flagged at pack time)
  const bool odd_tile =
      !kQ8 && reinterpret_cast<const uint32_t*>(p.weights + (size_t)blocks * kVocab * 18)[tile] != 0u;

  if (!live) return;  // whole wave idle (no barrier follows)
  const uint32_t lrow0 = wave * kRowsPerWave;       // first row inside the group

  // [row tile][column tile][result register]; block 0 starts them (first_tag)
  // as 0 + term, the reference's first add from a zero total, so no register
  // is cleared beforehand
  float total[2][4][4];
  auto sum = [&](int rt, int c, int i, float term, auto first_tag) {
    if constexpr (decltype(first_tag)::value)
      total[rt][c][i] = 0.0f + term;
    else
      total[rt][c][i] = total[rt][c][i] + term;
  };

  auto run = [&](uint32_t b, const Operands& o, auto odd_tag, auto first_tag) {
    constexpr bool kOdd = decltype(odd_tag)::value;
    const v4f ws = *reinterpret_cast<const v4f*>(&w_scale[b * kTileIds + 4u * n]);
    const v4f wn = *reinterpret_cast<const v4f*>(&w_neg[b * kTileIds + 4u * n]);
    v4f as[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
      as[rt] = *reinterpret_cast<const v4f*>(
          &act_scale[b * kRowsPerGroup + lrow0 + 16u * rt + 4u * q]);
    v4i d[2][4];
    if constexpr (kQ8) {
      const uint32_t raw[8] = {o.raw[0].x, o.raw[0].y, o.raw[0].z, o.raw[0].w,
                               o.raw[kWords - 1].x, o.raw[kWords - 1].y, o.raw[kWords - 1].z,
                               o.raw[kWords - 1].w};
      const v4i zero = {0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint64_t w = (uint64_t)raw[2 * c] | ((uint64_t)raw[2 * c + 1] << 32);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
          d[rt][c] = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)o.a[rt], (long)w, zero, 0, 0, 0);
      }
    } else {
      const uint32_t raw[4] = {o.raw[0].x, o.raw[0].y, o.raw[0].z, o.raw[0].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint64_t w = (uint64_t)((raw[c] << 4) & 0xf0f0f0f0u) |
                           ((uint64_t)(raw[c] & 0xf0f0f0f0u) << 32);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
          d[rt][c] = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)o.a[rt], (long)w, magic, 0, 0, 0);
      }
    }
    const float wsv[4] = {ws.x, ws.y, ws.z, ws.w};
    const float wnv[4] = {wn.x, wn.y, wn.z, wn.w};
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const float asv[4] = {as[rt].x, as[rt].y, as[rt].z, as[rt].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (kQ8) {
            const float scale = wsv[c] * asv[i];
            sum(rt, c, i, (float)d[rt][c][i] * scale, first_tag);
          } else {
            const float x = __int_as_float(d[rt][c][i]);
            const float y = kOdd ? (x - kMagic) * wsv[c] : __builtin_fmaf(x, wsv[c], wnv[c]);
            sum(rt, c, i, y * asv[i], first_tag);
          }
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
  // The first round is peeled: its block 0 starts the totals.
  constexpr std::true_type kFirst{};
  constexpr std::false_type kNext{};
  auto gemm = [&](auto odd_tag) {
    Operands& even = s0;
    Operands& odd_ops = s1;
    load(min(1u, last), odd_ops);
    __builtin_amdgcn_sched_barrier(0);
    run(0u, even, odd_tag, kFirst);
    __builtin_amdgcn_sched_barrier(0);
    load(min(2u, last), even);
    __builtin_amdgcn_sched_barrier(0);
    if (blocks > 1u) run(1u, odd_ops, odd_tag, kNext);
    __builtin_amdgcn_sched_barrier(0);
    auto round = [&](uint32_t b) __attribute__((always_inline)) {
      load(b + 1u, odd_ops);
      __builtin_amdgcn_sched_barrier(0);
      run(b, even, odd_tag, kNext);
      __builtin_amdgcn_sched_barrier(0);
      load(min(b + 2u, last), even);
      __builtin_amdgcn_sched_barrier(0);
      run(b + 1u, odd_ops, odd_tag, kNext);
      __builtin_amdgcn_sched_barrier(0);
    };
    if constexpr (kNB != 0) {
#pragma unroll
      for (uint32_t b = 2; b + 1u < kNB; b += 2) round(b);
    } else {
#pragma unroll 1
      for (uint32_t b = 2; b + 1u < blocks; b += 2) round(b);
    }
    if ((blocks & 1u) != 0u && blocks > 1u) run(last, even, odd_tag, kNext);
  };
  // The Q8_0 head reads twice the weight bytes per block: its loads run two
  // blocks ahead (three operand sets in rotation, the same clamped loads).
  auto gemm_ahead2 = [&]() {
    constexpr std::false_type kEven{};
    load(min(2u, last), s2);
    __builtin_amdgcn_sched_barrier(0);
    run(0u, s0, kEven, kFirst);
    __builtin_amdgcn_sched_barrier(0);
    load(min(3u, last), s0);
    __builtin_amdgcn_sched_barrier(0);
    if (blocks > 1u) run(1u, s1, kEven, kNext);
    __builtin_amdgcn_sched_barrier(0);
    load(min(4u, last), s1);
    __builtin_amdgcn_sched_barrier(0);
    if (blocks > 2u) run(2u, s2, kEven, kNext);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t b = 3;
#pragma unroll 1
    for (; b + 2u < blocks; b += 3) {
      load(min(b + 2u, last), s2);
      __builtin_amdgcn_sched_barrier(0);
      run(b, s0, kEven, kNext);
      __builtin_amdgcn_sched_barrier(0);
      load(min(b + 3u, last), s0);
      __builtin_amdgcn_sched_barrier(0);
      run(b + 1u, s1, kEven, kNext);
      __builtin_amdgcn_sched_barrier(0);
      load(min(b + 4u, last), s1);
      __builtin_amdgcn_sched_barrier(0);
      run(b + 2u, s2, kEven, kNext);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (b < blocks) run(b, s0, kEven, kNext);
    if (b + 1u < blocks) run(b + 1u, s1, kEven, kNext);
  };
  if constexpr (kQ8) {
    gemm_ahead2();
  } else if (odd_tile) {
    gemm(std::true_type{});
  } else {
    gemm(std::false_type{});
  }

  if constexpr (kLogits)
    write_tile<2, 4, false>(p, total, group0, kRowsPerGroup, lrow0 + 4u * q, tile, n);
  else
    write_tile_words<2, 4>(p, total, group0, kRowsPerGroup, lrow0 + 4u * q, tile, n);
}

// ---- the head for narrow batches (up to 64 rows) ----
// The wide kernel stages the scales of 128 rows in LDS and gives each wave
// 32 rows of one 64-id tile; with few rows most of that work is padding.
// Here one wave takes one 64-id tile and 16 kRT rows (one MFMA row tile up
// to 32 rows, two above), four waves per workgroup (two for the Q8_0 head
// up to 32 rows) over consecutive tiles, the grid's y over the row groups.
// Each block's weight and activation
// scales are loaded with its operands (four fp16 weight scales and 4 kRT
// activation scales per lane), and the loads run kSets - 1 blocks ahead in
// rotating operand sets: with one wave per tile, the memory in flight per
// wave is what keeps the weights streaming.  The epilogue is the wide
// kernel's, for both formats; a Q4_0 tile flagged at pack time for an
// infinite or NaN weight scale takes the subtract-then-multiply form for all
// its blocks.  The loop body has no branch: at a branch's join the compiler
// waits for every load in flight, which would undo the loads issued ahead.
// For the same reason the Q4_0 block loop is unrolled whole at the model's
// width (kNB = 28): in the loop form the compiler copies the next block's
// operands between registers at the loop edge and waits for every load
// there.  With at most four rows every real row is result register i < kI of lanes
// 0 .. 15, so the epilogue of the other registers (padding rows) is left
// out: kI = 1 for one conversation.
//
// kFused (at most kFusedQuantRows rows): each workgroup quantises the rows'
// activations itself, into LDS, instead of reading them from lm_quant_kernel
// -- one launch less per step.  The first blocks' weights are requested
// before the quantisation, so it overlaps their latency.
constexpr uint32_t kMaxBlocks = 2048 / 32;
template <bool kQ8, int kRT, int kSets, int kI, bool kFused, int kNB, int kNW>
__global__ __launch_bounds__(64 * kNW) void lm_gemm_narrow_kernel(LmParams p) {
  static_assert(kI == 4 || kRT == 1, "partial rows only with one row tile");
  static_assert(!kFused || (kRT == 1 && kI <= (int)kFusedQuantRows), "fused rows fit one row tile");
  // kFused: [block][row] quants (8 words) and scales / 16 of the real rows
  __shared__ __align__(16) uint32_t aq_lds[kFused ? kMaxBlocks : 1][kFused ? kFusedQuantRows : 1][8];
  __shared__ __align__(16) float as_lds[kFused ? kMaxBlocks : 1][kFused ? kFusedQuantRows : 1];
  const uint32_t lane = threadIdx.x & 63u;
  // the tile is wave-uniform: held in scalar registers, so every load below
  // is a scalar base plus a 32-bit lane offset, with no 64-bit address
  // arithmetic per lane
  const uint32_t tile_raw = blockIdx.x * (uint32_t)kNW + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool live_wave = tile_raw < kTilesPerRow;
  // waves past the last tile work on the last one (and store nothing), so
  // that every wave reaches the workgroup barrier of the fused quantisation
  const uint32_t tile = live_wave ? tile_raw : kTilesPerRow - 1u;
  if (!kFused && !live_wave) return;  // whole wave, no barrier follows
  const uint32_t n = lane & 15u;
  const uint32_t q = lane >> 4;
  const uint32_t row0 = blockIdx.y * (16u * kRT);  // first row of the wave's group
  // kNB > 0: the width is 32 kNB, known at compile time (the block loop is
  // unrolled whole, so no loaded register crosses a loop edge)
  const uint32_t blocks = kNB > 0 ? (uint32_t)kNB : p.cols / 32u;
  const uint32_t last = blocks - 1u;
  constexpr uint32_t kWords = kQ8 ? 2u : 1u;  // uint4 of packed weights per lane and block
  constexpr uint32_t kTile = kQ8 ? kTileBytesQ8 : kTileBytes;

  // Each load is a wave-uniform base plus one 32-bit byte offset (the block's
  // uniform part + the lane's part).  The widths of at most 2048 keep the
  // packed head under 330 MB, so every offset fits.
  const uint8_t* a_base = reinterpret_cast<const uint8_t*>(p.act_q);
  const uint32_t a_stride = p.rows_pad * 32u;  // bytes per block
  const uint32_t a_off = (row0 + n) * 32u + 8u * q;
  const uint8_t* w_base = p.weights;
  const uint32_t w_stride = kTilesPerRow * kTile;  // bytes per block
  const uint32_t w_off = tile * kTile + 16u * kWords * lane;
  const uint8_t* ws_base = p.weights;
  const uint32_t ws_off = blocks * kVocab * (kQ8 ? 32u : 16u) + 2u * tile * kTileIds + 8u * n;
  const uint8_t* as_base = reinterpret_cast<const uint8_t*>(p.act_s);
  const uint32_t as_stride = p.rows_pad * 4u;
  const uint32_t as_off = (row0 + 4u * q) * 4u;

  // Only the kI activation scales a lane uses are loaded: a register of a
  // wider load left unused would be taken for a temporary while the load is
  // in flight, and writing it would wait for every load.
  typedef float vIf __attribute__((ext_vector_type(kI)));
  struct Operands {
    uint64_t a[kRT];
    v4u raw[kWords];
    uint64_t ws;    // four fp16 weight scales, ids 4n .. 4n+3
    vIf as[kRT];    // activation scales / 16 of rows 16 rt + 4q .. 4q + kI - 1
  };
  auto load_w = [&](uint32_t b, Operands& o) {
    const uint32_t wo = b * w_stride + w_off;
#pragma unroll
    for (uint32_t k = 0; k < kWords; ++k)
      o.raw[k] = *reinterpret_cast<const v4u*>(w_base + (wo + 16u * k));
    o.ws = *reinterpret_cast<const uint64_t*>(ws_base + (b * (kVocab * 2u) + ws_off));
  };
  auto load_a = [&](uint32_t b, Operands& o) {
    if constexpr (kFused) {
      // real rows only: lanes n < rows (A) and the q == 0 result registers
      const uint64_t a = *reinterpret_cast<const uint64_t*>(&aq_lds[b][n & (kFusedQuantRows - 1u)][2u * q]);
      o.a[0] = n < p.rows ? a : 0ull;
      vIf v;
#pragma unroll
      for (int i = 0; i < kI; ++i) v[i] = q == 0u ? as_lds[b][i] : 0.0f;
      o.as[0] = v;
    } else {
      const uint32_t ao = b * a_stride + a_off;
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt)
        o.a[rt] = *reinterpret_cast<const uint64_t*>(a_base + (ao + 16u * 32u * (uint32_t)rt));
      const uint32_t so = b * as_stride + as_off;
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt)
        o.as[rt] = *reinterpret_cast<const vIf*>(as_base + (so + 64u * (uint32_t)rt));
    }
  };

  float total[kRT][4][4];
#pragma unroll
  for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) total[rt][c][i] = 0.0f;
  const v4i magic = {(int)kMagicBits, (int)kMagicBits, (int)kMagicBits, (int)kMagicBits};
  const v4i zero = {0, 0, 0, 0};

  // run() hands each value's term of the block (the reference's rounded
  // product) to sink(rt, c, i, term); add() adds it to the running total.
  auto add = [&](int rt, int c, int i, float term) { total[rt][c][i] = total[rt][c][i] + term; };
  auto run = [&](const Operands& o, auto odd_tag, auto sink) {
    constexpr bool kOdd = decltype(odd_tag)::value;
    float wsv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
      wsv[c] = __half2float(__ushort_as_half((unsigned short)(o.ws >> (16 * c))));
    v4i d[kRT][4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint64_t w;
      if constexpr (kQ8) {
        const uint32_t raw[8] = {o.raw[0].x, o.raw[0].y, o.raw[0].z, o.raw[0].w,
                                 o.raw[kWords - 1].x, o.raw[kWords - 1].y, o.raw[kWords - 1].z,
                                 o.raw[kWords - 1].w};
        w = (uint64_t)raw[2 * c] | ((uint64_t)raw[2 * c + 1] << 32);
      } else {
        const uint32_t raw[4] = {o.raw[0].x, o.raw[0].y, o.raw[0].z, o.raw[0].w};
        w = (uint64_t)((raw[c] << 4) & 0xf0f0f0f0u) | ((uint64_t)(raw[c] & 0xf0f0f0f0u) << 32);
      }
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt)
        d[rt][c] = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)o.a[rt], (long)w,
                                                         kQ8 ? zero : magic, 0, 0, 0);
    }
    if constexpr (kQ8) {
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        float asv[kI];
#pragma unroll
        for (int i = 0; i < kI; ++i) asv[i] = o.as[rt][i];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int i = 0; i < kI; ++i) {
            const float scale = wsv[c] * asv[i];
            sink(rt, c, i, (float)d[rt][c][i] * scale);
          }
      }
    } else {
      if constexpr (kOdd) {
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
          float asv[kI];
#pragma unroll
          for (int i = 0; i < kI; ++i) asv[i] = o.as[rt][i];
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int i = 0; i < kI; ++i) {
              const float y = (__int_as_float(d[rt][c][i]) - kMagic) * wsv[c];
              sink(rt, c, i, y * asv[i]);
            }
        }
      } else {
        float wnv[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) wnv[c] = wsv[c] * -kMagic;
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
          float asv[kI];
#pragma unroll
          for (int i = 0; i < kI; ++i) asv[i] = o.as[rt][i];
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int i = 0; i < kI; ++i) {
              const float y = __builtin_fmaf(__int_as_float(d[rt][c][i]), wsv[c], wnv[c]);
              sink(rt, c, i, y * asv[i]);
            }
        }
      }
    }
  };

  // Block t sits in set t % kSets.  Loads are unconditional (clamped to the
  // last block).  Whole rounds of kSets blocks run in the loop; the last
  // blocks (fewer than kSets, already loaded) run after it.  The first
  // kSets - 1 blocks are requested before anything else (and, with kFused,
  // before the quantisation and its barrier, which every wave reaches on the
  // same path).
  Operands ops[kSets];
#pragma unroll
  for (int k = 0; k < kSets - 1; ++k) load_w(min((uint32_t)k, last), ops[k]);
  if constexpr (kFused) {
    // the rows' activations, quantised into LDS while those loads fly
    for (uint32_t pair = threadIdx.x; pair < p.rows * blocks; pair += 64u * kNW) {
      const uint32_t r = pair / blocks;
      const uint32_t b = pair - r * blocks;
      uint32_t x[32], packed[8];
      float scale16;
      load_block(p, r, b, x);
      quantize_block(x, true, packed, scale16);
      *reinterpret_cast<v4u*>(&aq_lds[b][r][0]) = v4u{packed[0], packed[1], packed[2], packed[3]};
      *reinterpret_cast<v4u*>(&aq_lds[b][r][4]) = v4u{packed[4], packed[5], packed[6], packed[7]};
      as_lds[b][r] = kQ8 ? scale16 * 16.0f : scale16;  // a_scale for the Q8_0 epilogue
    }
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < kSets - 1; ++k) load_a(min((uint32_t)k, last), ops[k]);
  auto gemm = [&](auto odd_tag) {
    if constexpr (kNB > 0) {
#pragma unroll
      for (int b = 0; b < kNB; ++b) {
        if (b + kSets - 1 < kNB) {
          load_w((uint32_t)(b + kSets - 1), ops[(b + kSets - 1) % kSets]);
          load_a((uint32_t)(b + kSets - 1), ops[(b + kSets - 1) % kSets]);
        }
        __builtin_amdgcn_sched_barrier(0);
        run(ops[b % kSets], odd_tag, add);
        __builtin_amdgcn_sched_barrier(0);
      }
      return;
    }
    const uint32_t whole = blocks / kSets * kSets;
#pragma unroll 1
    for (uint32_t b = 0; b < whole; b += kSets) {
#pragma unroll
      for (int k = 0; k < kSets; ++k) {
        const uint32_t ahead = min(b + (uint32_t)(k + kSets - 1), last);
        load_w(ahead, ops[(k + kSets - 1) % kSets]);
        load_a(ahead, ops[(k + kSets - 1) % kSets]);
        __builtin_amdgcn_sched_barrier(0);
        run(ops[k], odd_tag, add);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int k = 0; k < kSets - 1; ++k)
      if (whole + (uint32_t)k < blocks) run(ops[k], odd_tag, add);
  };
  if constexpr (kQ8) {
    gemm(std::false_type{});
  } else {
    const uint32_t* flags =
        reinterpret_cast<const uint32_t*>(p.weights + (size_t)blocks * kVocab * 18);
    if (flags[tile] != 0u) {
      gemm(std::true_type{});
    } else {
      gemm(std::false_type{});
    }
  }
  if (live_wave) write_tile<kRT, kI, true>(p, total, row0, 16u * kRT, 4u * q, tile, n);
}

// A value every lane holds alike, moved to a scalar register so that the
// compiler branches and selects on it as a wave-uniform value.
__device__ __forceinline__ uint32_t uniform(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}

// Collects into `cand` every key of this lane (keys[0..N)) in [lo, hi);
// `below` receives the lane's largest key under lo.
template <int N>
__device__ __forceinline__ uint32_t collect_range(uint64_t* cand, const uint64_t (&keys)[N],
                                                  uint64_t lo, uint64_t hi, uint64_t& below) {
  uint32_t count = 0;
  below = 0;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const bool take = keys[j] != 0 && keys[j] >= lo && keys[j] < hi;
    const uint64_t mask = __ballot(take);
    if (take) cand[count + lanes_below(mask)] = keys[j];
    count += (uint32_t)__popcll((unsigned long long)mask);
    below = (keys[j] < lo && keys[j] > below) ? keys[j] : below;
  }
  return uniform(count);
}

// ---- tile words of given logits (the batched sampler's small batches) ----
// The same tile and second words as the narrow GEMM writes, from logits in
// memory: one 16-lane row per (row, 64-id tile), lane n reading ids
// 4n .. 4n+3 of the tile (one 16-byte load each, read once).  A workgroup
// takes 16 x kLoads consecutive tiles of one row, each 16-lane row kLoads of
// them (tiles g, g + 16, ...: every load instruction covers 16 whole tiles),
// all loads in flight together; the grid's y runs over the rows.  For a
// single-row drop-in the logits are in mapped pinned host memory: the launch
// also stores them at logits_copy and copies the staged scalars and history,
// so that the selection reads device memory (on MI355X the PCIe read of the
// 608 KB row takes about 15 us, at 128 to 1,024 threads per workgroup alike).
template <uint32_t kLoads>
__global__ __launch_bounds__(256) void tile_words_kernel(LmParams p) {
  constexpr uint32_t kTilesPerGroup = 16u * kLoads;
  const uint32_t n = threadIdx.x & 15u;
  const uint32_t g = threadIdx.x >> 4;
  const uint32_t row = blockIdx.y;
  const uint32_t* lrow = p.logits + (size_t)row * p.logits_ld;
  v4u x[kLoads];
#pragma unroll
  for (uint32_t k = 0; k < kLoads; ++k) {
    // past the last tile the row's last tile is read again (and not stored)
    const uint32_t t = min(blockIdx.x * kTilesPerGroup + g + 16u * k, kTilesPerRow - 1u);
    x[k] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(lrow + t * kTileIds + 4u * n));
  }
  // the staged inputs beside the logits, spread over the whole grid
  const uint32_t stride = gridDim.x * gridDim.y * 256u;
  for (uint32_t i = (blockIdx.y * gridDim.x + blockIdx.x) * 256u + threadIdx.x; i < p.stage_v4;
       i += stride)
    reinterpret_cast<v4u*>(p.stage_dst)[i] = reinterpret_cast<const v4u*>(p.stage_src)[i];
  // Every word is computed before anything is stored: the wait for a load
  // issued before a store also waits for the store (one counter for both on
  // gfx950), and under the stream's read traffic a store's acknowledgement
  // takes microseconds.  Storing the first tile's words before the second
  // load was used made the B = 64 step 0.9 us longer (16.4 against 15.5 us
  // per step cold, wall).
  uint32_t word[kLoads], sec[kLoads];
#pragma unroll
  for (uint32_t k = 0; k < kLoads; ++k) {
    const float y[4] = {f_of(x[k].x), f_of(x[k].y), f_of(x[k].z), f_of(x[k].w)};
    word[k] = row16_max_u32(lane_tile_word(y));
    const uint32_t ow[4] = {order_word(y[0]), order_word(y[1]), order_word(y[2]), order_word(y[3])};
    sec[k] = tile_second_word(ow, word[k], n);
  }
#pragma unroll
  for (uint32_t k = 0; k < kLoads; ++k) {
    const uint32_t tile = blockIdx.x * kTilesPerGroup + g + 16u * k;
    if (p.logits_copy != nullptr && tile < kTilesPerRow)
      *reinterpret_cast<v4u*>(p.logits_copy + (size_t)row * p.logits_ld + tile * kTileIds + 4u * n) =
          x[k];
    if (n == 0u && tile < kTilesPerRow) {
      p.tilemax[(size_t)row * kTilesPerRow + tile] = word[k];
      p.tilesec[(size_t)row * kTilesPerRow + tile] = sec[k];
    }
  }
}

// ---- selection: one workgroup per row ----
// A tile's key is its order word with 0xffff - tile below it: tiles hold
// consecutive ids, so among tiles with equal maxima the lower tile holds the
// lower id, and the keys order the tiles as the keys of their best elements
// would.  No element of a tile can reach a key above its word with the
// lowest low bits any element can have with the tile's lowest id
// (tile_bound): the penalty never raises a value, so the raw maximum bounds
// the penalised ones.
// Where the selection takes the logits of the tiles it reads: from the logits
// the GEMM or tile_words_kernel wrote, or recomputed from the packed Q4_0 or
// Q8_0 head (the wide GEMM's one-pass mode keeps no logits).
constexpr int kFromLogits = 0;
constexpr int kRecomputeQ4 = 1;
constexpr int kRecomputeQ8 = 2;
constexpr uint32_t kTileWaves = 4;                      // waves that read the tile words
constexpr uint32_t kHistWaves = 4;                      // waves that build the history bitmap
constexpr uint32_t kHistGroup = 2;                      // later history batches requested together
constexpr uint32_t kHistShareFrom = 3;                  // batches from which the tile waves take a share
constexpr uint32_t kSelectThreads = 64u * (kTileWaves + kHistWaves);
constexpr int kTileKeys = (kTilesPerRow + 63) / 64;    // 38 tile words per lane
constexpr int kWaveKeys = (kTileKeys + (int)kTileWaves - 1) / (int)kTileWaves;  // 10 per tile wave
constexpr uint32_t kWaveTiles = 16;                     // tiles a tile wave reads in the first round
constexpr uint32_t kFirstElems = 256;                   // a fast round's element slots
constexpr uint32_t kTileCap = 20 * kTileKeys;          // tiles collected per round, at most
constexpr int kChunkTiles = 32;                        // tiles read per pass
constexpr uint32_t kElemCap = 20 * kChunkTiles;        // element keys collected per pass
static_assert(kFirstElems <= kElemCap, "the first round's elements fit the list");
static_assert(kTileWaves * kWaveTiles <= 64, "wave 0 checks the first round's tiles one per lane");

// a[i] for a lane's own i < 16 (N <= 16 entries): a select tree on the bits
// of i, which pass through an empty asm (else the compiler turns the tree back
// into an indexed access through scratch memory).
template <int N>
__device__ __forceinline__ uint32_t pick(const uint32_t (&a)[N], uint32_t i) {
  static_assert(N <= 16, "four select levels");
  uint32_t b0 = i & 1u, b1 = i & 2u, b2 = i & 4u, b3 = i & 8u;
  __asm__ volatile("" : "+v"(b0), "+v"(b1), "+v"(b2), "+v"(b3));
  uint32_t v8[8], v4[4], v2[2];
#pragma unroll
  for (int k = 0; k < 8; ++k) v8[k] = 2 * k >= N ? 0u : (2 * k + 1 < N && b0) ? a[2 * k + 1 < N ? 2 * k + 1 : 0] : a[2 * k < N ? 2 * k : 0];
#pragma unroll
  for (int k = 0; k < 4; ++k) v4[k] = b1 ? v8[2 * k + 1] : v8[2 * k];
#pragma unroll
  for (int k = 0; k < 2; ++k) v2[k] = b2 ? v4[2 * k + 1] : v4[2 * k];
  return b3 ? v2[1] : v2[0];
}

// Descending order of up to 64 distinct nonzero 64-bit keys held by lanes
// 0 .. n-1 (the other lanes hold 0): each lane counts the keys above its own,
// reading them two at a time through broadcast LDS reads, and writes its key
// at that rank.  One wave; buf holds 64 keys.  Lane i returns the i-th best
// key, 0 past n.  (A bitonic sort of 32 keys is 15 dependent exchange stages:
// 0.56 us of a one-row selection; the ranks need no exchange.)
typedef uint64_t v2u64 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint64_t rank_sort_desc64(uint64_t key, uint32_t lane, uint32_t n,
                                                     uint64_t* buf) {
  buf[lane] = key;
  __builtin_amdgcn_wave_barrier();
  uint32_t above0 = 0, above1 = 0;
  for (uint32_t j = 0; j < n; j += 2) {
    const v2u64 two = *reinterpret_cast<const v2u64*>(&buf[j]);
    above0 += two.x > key ? 1u : 0u;
    above1 += two.y > key ? 1u : 0u;
  }
  __builtin_amdgcn_wave_barrier();
  if (lane < n) buf[above0 + above1] = key;
  __builtin_amdgcn_wave_barrier();
  return lane < n ? buf[lane] : 0ull;
}

__device__ __forceinline__ uint64_t tile_key(uint32_t word, uint32_t tile) {
  return ((uint64_t)word << 32) | (0xffffu - tile);
}
// The same bound knowing the tile: its lowest id is 64 tile.
__device__ __forceinline__ uint64_t tile_bound(uint64_t key) {
  const uint32_t tile = 0xffffu - (uint32_t)(key & 0xffffu);
  return (key & 0xffffffff00000000ull) | (uint64_t)(((0x3ffffu - tile * kTileIds) << 1) | 1u);
}

// The first round, in the tile waves: thr_word is the 20th best of the 64
// lanes' best tile words (lane l's best over tiles l + 64 j); every tile whose
// word reaches it is read, and every element of those tiles whose raw value
// reaches thr_word (usually a few more than 20) is keyed, penalised through
// the bitmap, and sorted once.  Every element outside that set has a raw
// word, and so a penalised word (the penalty never raises a value), below
// thr_word: when the 20th best key of the set still reaches thr_word, the
// set's top-20 is the row's.
//
// Waves 0-3 split the tile words (wave w holds words j in [10 w, 10 w + 10)),
// exchange their lanes' best words through LDS, and each reads and filters
// its own tiles that reach thr_word; waves 4-7 build the row's history bitmap
// in LDS (once per unique id) and find the first bad position.  After the
// third barrier wave 0 keys and sorts the candidates.
//
// Any other case -- more than 16 tiles of one wave or more than 64 candidate
// elements, a 20th best key below thr_word -- takes the general selection on
// wave 0: rounds best-first over the 64-bit tile keys, each taking the tiles
// whose keys reach the 20th best of the lanes' best remaining keys, reading
// their logits, penalising them through the bitmap and merging them into the
// row's top-20, until the 20th best key beats tile_bound of the best tile not
// read.  Error rows: the lowest tile flagged kNonFiniteTile holds the first
// non-finite logit (NONFINITE_OUTPUT, which takes precedence), else the first
// history id >= vocab (TOKEN_ID).  The row is finished with finalize_row.
template <int kSrc>
__global__ __launch_bounds__(kSelectThreads) void lm_select_kernel(LmParams p, RowParams rp) {
  constexpr bool kRecompute = kSrc != kFromLogits;
  __shared__ __align__(16) uint32_t bm[kWordsPerRow];
  // recomputing tiles: the row's Q8_0 activations and scales, and the
  // recomputed logits of up to kWaveTiles tiles per tile wave
  __shared__ __align__(16) uint32_t act_row[kRecompute ? kMaxBlocks * 8 : 4];
  __shared__ float act_sc[kRecompute ? kMaxBlocks : 1];
  __shared__ uint32_t xbuf[kRecompute ? kTileWaves * kWaveTiles * 64 : 1];
  __shared__ uint32_t mt_list[kRecompute ? kTileWaves * kWaveTiles : 1];  // tiles to recompute
  __shared__ uint32_t mt_count;
  __shared__ uint32_t mt_thr;  // the threshold word of the round that listed them
  __shared__ uint32_t tcand[kTileCap];
  __shared__ uint64_t ecand[kElemCap];
  __shared__ uint64_t top[kTopK];
  __shared__ __align__(16) uint64_t sortbuf[64];  // wave 0's rank sort
  __shared__ uint32_t lane_best[kTileWaves][64];
  __shared__ uint32_t wave_tiles[kTileWaves][kWaveTiles];
  __shared__ uint32_t first_elems;  // elements the tile waves appended to ecand
  __shared__ uint32_t first_fail;   // a tile wave's tiles overflowed its list
  __shared__ uint32_t round2;       // a second round runs, at round2_thr
  __shared__ uint32_t round2_thr;
  __shared__ uint32_t bad_hist;
  __shared__ uint32_t nf_tile;
  const uint32_t row = blockIdx.x;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = tid >> 6;
  const uint32_t* lrow = kRecompute ? nullptr : p.logits + (size_t)row * p.logits_ld;
  const uint32_t* tm = p.tilemax + (size_t)row * kTilesPerRow;
  const bool tile_wave = wave < kTileWaves;
  const uint32_t blocks = p.cols / 32u;

  // The loads that need only the kernel's arguments go out first, before the
  // row's state and length are read (each of those is a memory round trip
  // that the compiler would otherwise wait for first); a row that turns out
  // to be skipped leaves with them in flight.
  //
  // Tile waves: their tile words (tile lane + 64 (10 w + j) in words[j], 0
  // past the last tile).  The loads are unconditional (the index is clamped
  // to the last tile, the second words read the tile words again when the
  // GEMM wrote none); lanes past the last tile and missing second words are
  // masked after the first barrier, where the values are used.
  uint32_t thr_first = 0;  // the first round's threshold word (tile waves)
  uint32_t words[kWaveKeys];
  uint32_t secs[kWaveKeys];  // their second words, when the GEMM wrote them
  const bool has_sec = p.tilesec != nullptr;
  if (tile_wave) {
    const uint32_t* ts = has_sec ? p.tilesec + (size_t)row * kTilesPerRow : tm;
#pragma unroll
    for (int j = 0; j < kWaveKeys; ++j) {
      const uint32_t t = lane + 64u * (wave * (uint32_t)kWaveKeys + (uint32_t)j);
      words[j] = tm[min(t, kTilesPerRow - 1u)];
      secs[j] = ts[min(t, kTilesPerRow - 1u)];
    }
  }
  // History threads: each requests its first uint4 (or word) of the row,
  // clamped to the row's capacity (hist_ld ids are readable per row); the
  // other three (seven) of its first batch, and its second batch of four,
  // follow once the length shows that the row needs them.
  const uint32_t ht = tid - 64u * kTileWaves;
  constexpr uint32_t kHistThreads = 64u * kHistWaves;
  const bool has_hist = rp.hist != nullptr && rp.hist_len != nullptr && rp.hist_ld != 0;
  const uint32_t* hbase = has_hist ? rp.hist + (size_t)row * rp.hist_ld : nullptr;
  v4u hv[4] = {};
  v4u hb[4] = {};  // the second batch of a history longer than the first
  uint32_t hs[8] = {};
  if (!tile_wave && has_hist) {
    if (rp.hist_vec4)
      hv[0] = reinterpret_cast<const v4u*>(hbase)[min(ht, (uint32_t)(rp.hist_ld / 4u) - 1u)];
    else
      hs[0] = hbase[min(ht, (uint32_t)min(rp.hist_ld, (size_t)kHistThreads) - 1u)];
  }
  // recomputing tiles: the row's activations (one word per thread)
  uint32_t act_word = 0;
  float act_scale = 0.0f;
  if constexpr (kRecompute) {
    if (tid < blocks * 8u)
      act_word = reinterpret_cast<const uint32_t*>(
          p.act_q + ((size_t)(tid >> 3) * p.rows_pad + row) * 32u)[tid & 7u];
    if (tid < blocks) act_scale = p.act_s[(size_t)tid * p.rows_pad + row];
  }
  __builtin_amdgcn_sched_barrier(0);

  if (row_skipped(rp, row)) {  // decode loop: the row has ended or has no room
    if (tid == 0) skip_row(rp, row);
    return;
  }
  uint32_t len = 0;
  if (has_hist) {
    len = row_word(rp.hist_len + row);
    if ((size_t)len > rp.hist_ld) len = (uint32_t)rp.hist_ld;
  }
  // The row's uniform, which wave 0 uses to finish the row, through the
  // scalar cache: a vector load of this wave-uniform word is moved to a
  // scalar register at once, which waits for it.
  const uint32_t r24 = row_word(rp.random_24 + row);
  const uint32_t* hrow = len != 0 ? hbase : nullptr;
  const v4u* h4 = reinterpret_cast<const v4u*>(hrow);
  const uint32_t n4 = (len + 3u) / 4u;
  auto load_hist = [&](uint32_t k0) {
    if (rp.hist_vec4) {
#pragma unroll
      for (uint32_t u = 0; u < 4; ++u) hv[u] = h4[min(k0 + u * kHistThreads, n4 - 1u)];
    } else {
#pragma unroll
      for (uint32_t u = 0; u < 8; ++u) hs[u] = hrow[min(k0 + u * kHistThreads, len - 1u)];
    }
  };
  if (!tile_wave && uniform(rp.hist_vec4 ? n4 : len) > kHistThreads) {
    if (rp.hist_vec4) {
#pragma unroll
      for (uint32_t u = 1; u < 4; ++u) hv[u] = h4[min(ht + u * kHistThreads, n4 - 1u)];
      if (uniform(n4) > 4u * kHistThreads) {
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) hb[u] = h4[min(ht + (4u + u) * kHistThreads, n4 - 1u)];
      }
    } else {
#pragma unroll
      for (uint32_t u = 1; u < 8; ++u) hs[u] = hrow[min(ht + u * kHistThreads, len - 1u)];
    }
  }

  static_assert(kWordsPerRow % 4 == 0, "the bitmap is cleared 16 bytes at a time");
  for (uint32_t i = tid; i < kWordsPerRow / 4; i += kSelectThreads)
    reinterpret_cast<v4u*>(bm)[i] = v4u{0u, 0u, 0u, 0u};
  if (tid == 0) {
    bad_hist = kNone;
    nf_tile = kNone;
    first_elems = 0;
    first_fail = 0;
    mt_count = 0;
  }
  if (tid < (uint32_t)kTopK) top[tid] = 0;
  if constexpr (kRecompute) {
    if (tid < blocks * 8u) act_row[tid] = act_word;
    if (tid < blocks) act_sc[tid] = act_scale;
  }
  __syncthreads();  // (1) the bitmap is clear, the activations staged

  // Recomputing a tile's logits from the packed head and the staged
  // activations, with the head's arithmetic: the exact int32 block dots
  // (v_dot4c_i32_i8 over the nibbles expanded as in the GEMM, so a Q4_0 dot
  // comes out as 16 dot), then the reference's binary32 epilogue over the
  // blocks in order: total + mul(mul(f32(dot), w_scale), a_scale) for Q4_0
  // (a_scale / 16 staged, 16 dot: the same products, scaled by exact powers
  // of two), total + mul(f32(dot), mul(w_scale, a_scale)) for Q8_0.  Lane l
  // takes id 64 tile + l; `tile` is wave-uniform.
  constexpr bool kQ8 = kSrc == kRecomputeQ8;
  constexpr uint32_t kTileB = kQ8 ? kTileBytesQ8 : kTileBytes;
  constexpr uint32_t kWordsB = kQ8 ? 8u : 4u;  // a lane's weight words per block
  // the lane's weight words and fp16 weight scale of (tile, block b)
  auto load_weights = [&](uint32_t tile, uint32_t b, uint32_t(&w)[kWordsB], uint32_t& sc)
      __attribute__((always_inline)) {
    const uint8_t* wb = p.weights + ((size_t)b * kTilesPerRow + tile) * kTileB + kWordsB * lane;
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
      if constexpr (kQ8) {
        const v2u x = *reinterpret_cast<const v2u*>(wb + 512u * q);
        w[2 * q] = x.x;
        w[2 * q + 1] = x.y;
      } else {
        w[q] = *reinterpret_cast<const uint32_t*>(wb + 256u * q);
      }
    }
    sc = reinterpret_cast<const uint16_t*>(p.weights + (size_t)blocks * kVocab * (kQ8 ? 32 : 16))
        [(size_t)b * kVocab + tile * kTileIds + lane];
  };
  // block b's term of the lane's logit
  auto block_term = [&](uint32_t b, const uint32_t(&w)[kWordsB], uint32_t sc)
      __attribute__((always_inline)) -> float {
    const v4u a0 = *reinterpret_cast<const v4u*>(&act_row[b * 8u]);
    const v4u a1 = *reinterpret_cast<const v4u*>(&act_row[b * 8u + 4u]);
    const uint32_t a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    int dot = 0;
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
      const uint32_t lo = kQ8 ? w[2 * q] : (w[q] << 4) & 0xf0f0f0f0u;
      const uint32_t hi = kQ8 ? w[2 * q + 1] : w[q] & 0xf0f0f0f0u;
      dot = __builtin_amdgcn_sdot4((int)lo, (int)a[2 * q], dot, false);
      dot = __builtin_amdgcn_sdot4((int)hi, (int)a[2 * q + 1], dot, false);
    }
    const float ws = __half2float(__ushort_as_half((unsigned short)sc));
    return kQ8 ? (float)dot * (ws * act_sc[b]) : ((float)dot * ws) * act_sc[b];
  };
  // One wave's whole tile, kBatch blocks' loads in flight at a time (the
  // error path's first flagged tile, and the general selection's tiles).
  auto tile_logit = [&](uint32_t tile) __attribute__((always_inline)) -> uint32_t {
    if constexpr (!kRecompute) {
      return lrow[tile * kTileIds + lane];
    } else {
      constexpr uint32_t kBatch = kQ8 ? 7u : 14u;
      const uint32_t last = blocks - 1u;
      float total = 0.0f;
      for (uint32_t b0 = 0; b0 < blocks; b0 += kBatch) {
        uint32_t w[kBatch][kWordsB];
        uint32_t sc[kBatch];
#pragma unroll
        for (uint32_t k = 0; k < kBatch; ++k) load_weights(tile, min(b0 + k, last), w[k], sc[k]);
#pragma unroll
        for (uint32_t k = 0; k < kBatch; ++k)
          if (b0 + k < blocks) total = total + block_term(b0 + k, w[k], sc[k]);
      }
      return b_of(total);
    }
  };

  if (tile_wave) {
#pragma unroll
    for (int j = 0; j < kWaveKeys; ++j) {
      const uint32_t t = lane + 64u * (wave * (uint32_t)kWaveKeys + (uint32_t)j);
      if (t >= kTilesPerRow) words[j] = 0u;
      if (t >= kTilesPerRow || !has_sec) secs[j] = ~0u;
    }
    // the lane's best word, and the wave's lowest tile flagged non-finite
    uint32_t lbw = 0;
#pragma unroll
    for (int j = 0; j < kWaveKeys; ++j) lbw = max(lbw, words[j]);
    if (__ballot(lbw == kNonFiniteTile)) {
      uint32_t nf = kNone;
#pragma unroll
      for (int j = 0; j < kWaveKeys; ++j) {
        const uint32_t t = lane + 64u * (wave * (uint32_t)kWaveKeys + (uint32_t)j);
        if (words[j] == kNonFiniteTile && t < nf) nf = t;
      }
      nf = wave_min_u32(nf);
      if (lane == 0) atomicMin(&nf_tile, nf);
    }
    lane_best[wave][lane] = lbw;
  }
  __syncthreads();  // (2) the lanes' best words are published

  // One round of the tile waves at threshold word `thr`: the wave's tiles whose
  // word reaches it, as masks of the lane's words.  A tile whose second word
  // says that no other logit of it reaches thr gives its maximum directly
  // (element word & 63, the bits of its order word); the others are read
  // (up to kWaveTiles per wave, else first_fail), and their elements whose raw
  // value reaches thr kept.  Every element whose raw word reaches thr ends up
  // in ecand (up to kFirstElems of them; first_elems counts them all).  One
  // pass per bit taken (the lanes' lowest remaining bits).
  // appends a pass's elements (mask: the lanes holding one): one LDS
  // atomic reserves their slots past the other waves' elements
  auto append = [&](uint64_t mask, bool mine, uint64_t e) {
    uint32_t base = 0;
    if (lane == 0) base = atomicAdd(&first_elems, (uint32_t)__popcll((unsigned long long)mask));
    const uint32_t slot = bcast32(base, 0) + lanes_below(mask);
    if (mine && slot < kFirstElems) ecand[slot] = e;
  };
  auto tile_round = [&](uint32_t thr) __attribute__((always_inline)) {
    uint32_t m = 0, d = 0;
#pragma unroll
    for (int j = 0; j < kWaveKeys; ++j) {
      const bool take = words[j] >= thr;
      m |= (take ? 1u : 0u) << j;
      d |= (take && (secs[j] & ~kSecondIndexMask) <= thr && words[j] != 0x80000000u ? 1u : 0u)
           << j;
    }
    m &= ~d;
    for (uint64_t mask = __ballot(d != 0); mask != 0; mask = __ballot(d != 0)) {
      uint64_t e = 0;
      if (d != 0) {
        const uint32_t j = (uint32_t)__builtin_ctz(d);
        const uint32_t t = lane + 64u * (wave * (uint32_t)kWaveKeys + j);
        e = ((uint64_t)(t * kTileIds + (pick(secs, j) & kSecondIndexMask)) << 32) |
            order_word_bits(pick(words, j));
      }
      append(mask, d != 0, e);
      d &= d - 1u;
    }
    uint32_t count = 0;
    for (uint64_t mask = __ballot(m != 0); mask != 0; mask = __ballot(m != 0)) {
      if (m != 0) {
        const uint32_t slot = count + lanes_below(mask);
        const uint32_t j = (uint32_t)__builtin_ctz(m);
        if (slot < kWaveTiles) wave_tiles[wave][slot] = lane + 64u * (wave * (uint32_t)kWaveKeys + j);
        m &= m - 1u;
      }
      count += (uint32_t)__popcll((unsigned long long)mask);
    }
    const uint32_t ntiles = uniform(count);
    if (ntiles > kWaveTiles && lane == 0) first_fail = 1u;
    if constexpr (kRecompute) {
      // listed for recompute_listed, which all waves run after the next barrier
      if (ntiles != 0 && ntiles <= kWaveTiles) {
        __builtin_amdgcn_wave_barrier();
        uint32_t base = 0;
        if (lane == 0) {
          base = atomicAdd(&mt_count, ntiles);
          mt_thr = thr;
        }
        if (lane < ntiles) mt_list[bcast32(base, 0) + lane] = wave_tiles[wave][lane];
      }
    } else if (ntiles != 0 && ntiles <= kWaveTiles) {
      __builtin_amdgcn_wave_barrier();
      // their logits (tile i of the wave is wave-uniform: readlane; past the
      // list the row's tile 0 is read again), then the elements whose raw
      // value reaches thr, as (id, raw bits)
      uint32_t xb[kWaveTiles];
      const uint32_t tl = lane < ntiles ? wave_tiles[wave][lane] : 0u;
#pragma unroll
      for (int i = 0; i < (int)kWaveTiles; ++i) xb[i] = lrow[bcast32(tl, (uint32_t)i) * kTileIds + lane];
      const float floor_value = f_of(key_value_bits((uint64_t)thr << 32));
      uint32_t e = 0;
#pragma unroll
      for (int i = 0; i < (int)kWaveTiles; ++i)
        e |= ((uint32_t)i < ntiles && f_of(xb[i]) >= floor_value ? 1u : 0u) << i;
      for (uint64_t mask = __ballot(e != 0); mask != 0; mask = __ballot(e != 0)) {
        uint64_t x = 0;
        if (e != 0) {
          const uint32_t i = (uint32_t)__builtin_ctz(e);
          x = ((uint64_t)(wave_tiles[wave][i] * kTileIds + lane) << 32) | pick(xb, i);
        }
        append(mask, e != 0, x);
        e &= e - 1u;
      }
    }
  };

  // Recomputing the listed tiles with all eight waves (recompute mode; every
  // thread calls it, after the barrier that follows a round): G tiles at a
  // time, each tile's blocks split over 8 / G waves whose per-block terms
  // go through LDS (xbuf), then one wave per tile adds the terms in block
  // order -- the reference's order -- and appends the elements whose value
  // reaches the round's threshold, as the memory mode's read does.  One
  // memory round trip per group of tiles instead of one per batch of blocks
  // of one tile on one wave.
  auto recompute_listed = [&]() __attribute__((always_inline)) {
    if constexpr (kRecompute) {
      const uint32_t count = uniform(mt_count);
      if (count == 0u) return;
      const float floor_value = f_of(key_value_bits((uint64_t)uniform(mt_thr) << 32));
      constexpr uint32_t kWaves = kSelectThreads / 64u;
      constexpr uint32_t kMaxPart = 8;  // blocks of one wave's part, at most
      const uint32_t G = blocks <= 8u ? 8u : blocks <= 16u ? 4u : blocks <= 32u ? 2u : 1u;
      const uint32_t wpt = kWaves / G;                  // waves per tile
      const uint32_t bpw = (blocks + wpt - 1u) / wpt;   // blocks per wave, <= kMaxPart
      const uint32_t slot = wave / wpt;
      const uint32_t part = wave - slot * wpt;
      const uint32_t b_lo = part * bpw;
      const uint32_t b_hi = min(blocks, b_lo + bpw);
      float* terms = reinterpret_cast<float*>(xbuf) + slot * blocks * 64u;
      static_assert(kMaxBlocks * 64u <= kTileWaves * kWaveTiles * 64u, "the terms fit xbuf");
      for (uint32_t g0 = 0; g0 < count; g0 += G) {
        const uint32_t t = g0 + slot;
        const uint32_t tile = t < count ? uniform(mt_list[t]) : 0u;
        if (t < count && b_lo < b_hi) {
          uint32_t w[kMaxPart][kWordsB];
          uint32_t sc[kMaxPart];
#pragma unroll
          for (uint32_t k = 0; k < kMaxPart; ++k)
            load_weights(tile, min(b_lo + k, b_hi - 1u), w[k], sc[k]);
#pragma unroll
          for (uint32_t k = 0; k < kMaxPart; ++k)
            if (b_lo + k < b_hi) terms[(b_lo + k) * 64u + lane] = block_term(b_lo + k, w[k], sc[k]);
        }
        __syncthreads();
        if (part == 0u && t < count) {
          float total = 0.0f;
          for (uint32_t b = 0; b < blocks; ++b) total = total + terms[b * 64u + lane];
          const uint32_t x = b_of(total);
          const bool take = f_of(x) >= floor_value;
          const uint64_t mask = __ballot(take);
          if (mask != 0) append(mask, take, ((uint64_t)(tile * kTileIds + lane) << 32) | x);
        }
        __syncthreads();
      }
    }
  };

  // ---- the history bitmap: per batch of sixteen ids per thread ----
  uint32_t my_bad = kNone;
  // Sixteen ids (four uint4) per thread per batch: their bitmap words are
  // read together (one LDS round trip), then only the missing bits are
  // set (Zipf histories repeat a few ids thousands of times).  A batch
  // whose last position is inside the row is live throughout and takes
  // no per-element tests; an id >= vocab is looked for once per batch
  // (the largest id), and the rare batch that holds one records the first
  // bad position and sets no bit for it.  Positions past the row read id 0
  // and set nothing.
  auto batch = [&](uint32_t k0, const v4u (&h)[4]) {
    uint32_t id[16], bit[16];
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) {
      id[4 * u] = h[u].x;
      id[4 * u + 1] = h[u].y;
      id[4 * u + 2] = h[u].z;
      id[4 * u + 3] = h[u].w;
    }
    if (4u * (k0 + 3u * kHistThreads) + 3u < len) {
#pragma unroll
      for (int e = 0; e < 16; ++e) bit[e] = 1u << (id[e] & 31u);
    } else {
#pragma unroll
      for (uint32_t e = 0; e < 16; ++e) {
        const bool live = 4u * (k0 + (e >> 2) * kHistThreads) + (e & 3u) < len;
        id[e] = live ? id[e] : 0u;
        bit[e] = live ? 1u << (id[e] & 31u) : 0u;
      }
    }
    uint32_t top_id = 0;
#pragma unroll
    for (int e = 0; e < 16; ++e) top_id = max(top_id, id[e]);
    if (top_id >= kVocab) {
#pragma unroll
      for (uint32_t e = 0; e < 16; ++e) {
        if (id[e] >= kVocab) {
          const uint32_t pos = 4u * (k0 + (e >> 2) * kHistThreads) + (e & 3u);
          my_bad = pos < my_bad ? pos : my_bad;
          id[e] = 0u;
          bit[e] = 0u;
        }
      }
    }
    uint32_t cur[16];
#pragma unroll
    for (int e = 0; e < 16; ++e)
      cur[e] = __hip_atomic_load(&bm[id[e] >> 5], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t need = bit[e] & ~cur[e];
      if (need != 0u) atomicOr(&bm[id[e] >> 5], need);
    }
  };
  auto load4 = [&](uint32_t k0, v4u (&h)[4]) {
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) h[u] = h4[min(k0 + u * kHistThreads, n4 - 1u)];
  };
  // A long history's batches (4,096 ids each) are split: the history waves
  // take the first hist_split, the tile waves the rest once their first
  // round is out.
  constexpr uint32_t kHistStep = 4u * kHistThreads;
  const uint32_t hist_batches = (n4 + kHistStep - 1u) / kHistStep;
  const uint32_t hist_split =
      hist_batches <= kHistShareFrom ? hist_batches : 2u + (hist_batches - 1u) / 2u;

  if (tile_wave) {
    if (nf_tile == kNone) {
      uint32_t best = 0;
#pragma unroll
      for (uint32_t w = 0; w < kTileWaves; ++w) best = max(best, lane_best[w][lane]);
      thr_first = uniform(bcast32(wave_sort_desc_u32(best, lane), kTopK - 1));
      tile_round(thr_first);
    }
    if (rp.hist_vec4 && hist_split < hist_batches) {
      for (uint32_t k0 = tid + hist_split * kHistStep; k0 < n4; k0 += kHistGroup * kHistStep) {
        v4u more[kHistGroup][4];
#pragma unroll
        for (uint32_t s = 0; s < kHistGroup; ++s) load4(k0 + s * kHistStep, more[s]);
#pragma unroll
        for (uint32_t s = 0; s < kHistGroup; ++s)
          if (k0 + s * kHistStep < n4) batch(k0 + s * kHistStep, more[s]);
      }
      my_bad = wave_min_u32(my_bad);
      if (lane == 0 && my_bad != kNone) atomicMin(&bad_hist, my_bad);
    }
  } else {
    // ---- the history bitmap and the first bad position ----
    if (rp.hist_vec4) {
      if (uniform(n4) <= 4u * kHistThreads) {
        // the loads made at entry hold the whole history: no batch is
        // requested ahead (a load nothing uses would still be waited for at
        // the next barrier)
        if (ht < n4) batch(ht, hv);
      } else {
        // Longer histories: the second batch was requested at entry too; the
        // rest come kHistGroup batches at a time (one memory round trip per
        // group, the first group's behind the first two batches).  The loads
        // are clamped inside the row; a batch past the row's end is not used.
        const bool groups = hist_split > 2u;
        const uint32_t lim = min(n4, ht + hist_split * kHistStep);  // past the tile waves' share
        v4u more[kHistGroup][4];
        uint32_t k0 = ht + 2u * kHistStep;
        if (groups) {
#pragma unroll
          for (uint32_t s = 0; s < kHistGroup; ++s) load4(k0 + s * kHistStep, more[s]);
        }
        batch(ht, hv);
        if (ht + kHistStep < n4) batch(ht + kHistStep, hb);
        if (groups) {
          for (;; k0 += kHistGroup * kHistStep) {
#pragma unroll
            for (uint32_t s = 0; s < kHistGroup; ++s)
              if (k0 + s * kHistStep < lim) batch(k0 + s * kHistStep, more[s]);
            if (k0 + kHistGroup * kHistStep >= lim) break;
#pragma unroll
            for (uint32_t s = 0; s < kHistGroup; ++s)
              load4(k0 + (kHistGroup + s) * kHistStep, more[s]);
          }
        }
      }
    } else {
      auto add = [&](uint32_t pos, uint32_t id) {
        if (pos >= len) return;
        if (id >= kVocab) {
          my_bad = pos < my_bad ? pos : my_bad;
        } else {
          uint32_t* word = &bm[id >> 5];
          const uint32_t bit = 1u << (id & 31u);
          if ((__hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) & bit) == 0u)
            atomicOr(word, bit);
        }
      };
      for (uint32_t q0 = ht; q0 < len; q0 += 8u * kHistThreads) {
        uint32_t v[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) v[u] = hs[u];
        if (q0 + 8u * kHistThreads < len) load_hist(q0 + 8u * kHistThreads);
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) add(q0 + u * kHistThreads, v[u]);
      }
    }
    my_bad = wave_min_u32(my_bad);
    if (lane == 0 && my_bad != kNone) atomicMin(&bad_hist, my_bad);
  }
  __syncthreads();  // (3) the bitmap, the first-round lists and the errors are done
  recompute_listed();  // (recompute mode: the first round's listed tiles)

  // ---- wave 0: errors, then the first round's candidates ----
  // (every word read at once: one LDS round trip).  Keys the candidates:
  // lane i < elems keys element i; they are sorted, and the selection is
  // exact when the 20th best penalised key still reaches the threshold word
  // (every element not keyed has a raw word below it).
  enum { kDone, kError, kRound2, kGeneral };
  int action = kDone;
  uint32_t first_bad_hist = kNone, nf = kNone;
  uint64_t sorted = 0;
  // (up to 64 candidates in one sort; more are keyed in place and merged into
  // top, 44 at a time)
  auto key_of = [&](uint64_t cand) {
    const uint32_t id = (uint32_t)(cand >> 32);
    const uint32_t xbits = (uint32_t)cand;
    const bool hit = ((bm[id >> 5] >> (id & 31u)) & 1u) != 0u;
    return make_key(hit ? penalize_bits(xbits) : xbits, id);
  };
  auto key_candidates = [&](uint32_t elems) __attribute__((always_inline)) -> uint64_t {
    if (elems <= 64u) {
      const uint64_t cand = ecand[lane];
      const uint64_t key = lane < elems ? key_of(cand) : 0ull;
      return rank_sort_desc64(key, lane, uniform(elems), sortbuf);
    }
    for (uint32_t i = lane; i < elems; i += 64u) ecand[i] = key_of(ecand[i]);
    if (lane < (uint32_t)kTopK) top[lane] = 0;
    __builtin_amdgcn_wave_barrier();
    merge_all(top, ecand, elems, lane);
    const uint64_t best = top[lane < (uint32_t)kTopK ? lane : 0];
    return lane < (uint32_t)kTopK ? best : 0ull;
  };
  if (wave == 0) {
    first_bad_hist = bad_hist;
    nf = nf_tile;
    const uint32_t elems = uniform(first_elems);
    const bool fits = uniform(first_fail) == 0u && elems <= kFirstElems;
    if (nf != kNone || first_bad_hist != kNone) {
      action = kError;
    } else if (fits) {
      sorted = key_candidates(elems);
      const uint32_t k20_word = uniform((uint32_t)(shfl64(sorted, kTopK - 1) >> 32));
      if (k20_word >= thr_first) {
        action = kDone;
      } else {
        // Penalties took the 20th best below the threshold: a second round
        // at its word.  Every element whose raw word is below it has a key
        // below the 20th best already held, and the new round's elements
        // include this round's, so its top-20 is the row's.
        action = kRound2;
        if (lane == 0) {
          round2_thr = k20_word;
          first_elems = 0;
          first_fail = 0;
          mt_count = 0;
        }
      }
    } else {
      action = kGeneral;
    }
    if (lane == 0) round2 = action == kRound2 ? 1u : 0u;
  }
  __syncthreads();  // (4) the decision
  if (wave == 0 && action == kError) {
    if (nf != kNone) {
      const uint32_t id = nf * kTileIds + lane;
      const uint32_t x = tile_logit(nf);
      const uint32_t first = wave_min_u32((x & 0x7f800000u) == 0x7f800000u ? id : kNone);
      finalize_row(rp, row, 0, first, bcast32(x, first & 63u), first_bad_hist, lane, r24);
    } else {
      finalize_row(rp, row, 0, kNone, 0u, first_bad_hist, lane, r24);
    }
    return;
  }
  if (wave == 0 && action == kDone) {
    finalize_row(rp, row, lane < (uint32_t)kTopK ? sorted : 0, kNone, 0u, kNone, lane, r24);
    return;
  }
  // The penalised logits at the history ids, for a caller that applies the
  // penalty to its own copy of the row when no id is excluded (then every id
  // is penalised once): written by the waves other than wave 0 once they have
  // no other work.  They do not depend on the draw; the caller applies them
  // only when the row succeeded.  Ids out of range are skipped (the row fails).
  // Eight positions per thread go out per batch, their ids and values loaded
  // first (clamped, unconditional): the caller's copy lives in mapped host
  // memory, and each wait for a load also waits for the stores before it, so
  // a store per position made every position wait for a write across PCIe
  // (single-row drop-in with 32,000 history ids: 117 -> 92 us per call).
  auto gather_history = [&]() {
    if (kRecompute || rp.gather == nullptr || len == 0) return;
    uint32_t* out = rp.gather + (size_t)row * rp.hist_ld;
    constexpr uint32_t kThreads = kSelectThreads - 64u;
    constexpr uint32_t kBatch = 8;
    for (uint32_t q0 = tid - 64u; q0 < len; q0 += kBatch * kThreads) {
      uint32_t id[kBatch], x[kBatch];
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) id[u] = hrow[min(q0 + u * kThreads, len - 1u)];
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) x[u] = lrow[min(id[u], kVocab - 1u)];
#pragma unroll
      for (uint32_t u = 0; u < kBatch; ++u) {
        const uint32_t q = q0 + u * kThreads;
        if (q < len && id[u] < kVocab) out[q] = penalize_bits(x[u]);
      }
    }
  };
  if (uniform(round2) != 0u) {
    if (tile_wave) tile_round(uniform(round2_thr));
    __syncthreads();  // (5) the second round's candidates
    recompute_listed();
    if (wave != 0) {
      gather_history();
      return;
    }
    const uint32_t elems = uniform(first_elems);
    if (uniform(first_fail) == 0u && elems <= kFirstElems) {
      sorted = key_candidates(elems);
      finalize_row(rp, row, lane < (uint32_t)kTopK ? sorted : 0, kNone, 0u, kNone, lane, r24);
      return;
    }
  }
  if (wave != 0) {
    gather_history();
    return;
  }

  // ---- wave 0: the general selection, best-first over the 64-bit tile keys ----
  if (lane < (uint32_t)kTopK) top[lane] = 0;
  __builtin_amdgcn_wave_barrier();
  uint32_t all[kTileKeys];  // tile lane + 64 j in all[j], 0 past the last tile
#pragma unroll
  for (int j = 0; j < kTileKeys; ++j) {
    const uint32_t t = lane + 64u * (uint32_t)j;
    all[j] = t < kTilesPerRow ? tm[t] : 0u;
  }
  // Collects the tiles with keys in [lo, hi) into tcand, in lane order per
  // slot; `below` receives the lane's best key under lo.
  auto collect_tiles = [&](uint64_t lo, uint64_t hi, uint64_t& below) -> uint32_t {
    uint32_t count = 0;
    below = 0;
#pragma unroll
    for (int j = 0; j < kTileKeys; ++j) {
      const uint32_t t = lane + 64u * (uint32_t)j;
      const uint64_t k = all[j] != 0u ? tile_key(all[j], t) : 0ull;
      const bool take = k != 0 && k >= lo && k < hi;
      const uint64_t mask = __ballot(take);
      if (mask) {
        if (take) tcand[count + lanes_below(mask)] = t;
        count += (uint32_t)__popcll((unsigned long long)mask);
      }
      below = (k < lo && k > below) ? k : below;
    }
    return uniform(count);
  };
  uint64_t k20 = 0;   // the row's 20th best key so far
  uint64_t hi = ~0ull;
  for (;;) {
    // the next tiles best-first: keys below hi reaching the 20th best of the
    // lanes' best such keys
    uint64_t lb = 0;
#pragma unroll
    for (int j = 0; j < kTileKeys; ++j) {
      const uint64_t k = all[j] != 0u ? tile_key(all[j], lane + 64u * (uint32_t)j) : 0ull;
      lb = (k < hi && k > lb) ? k : lb;
    }
    uint64_t thr = shfl64(wave_sort_desc(lb, lane), kTopK - 1);
    if (thr == 0) thr = 1;  // fewer than 20 lanes hold a tile: take them all
    uint64_t below64;
    const uint32_t ntiles = collect_tiles(thr, hi, below64);
    const uint64_t rem = below64 != 0 ? tile_bound(below64) : 0ull;
    __builtin_amdgcn_wave_barrier();
    for (uint32_t base = 0; base < ntiles; base += (uint32_t)kChunkTiles) {
      const uint32_t nt = uniform(min(ntiles - base, (uint32_t)kChunkTiles));
      // the pass's tiles, one per lane (the first tile again past the end),
      // and their logits: tile i is wave-uniform (readlane), so each load is
      // a scalar base plus the lane's offset
      const uint32_t tl = tcand[base + (lane < nt ? lane : 0u)];
      uint32_t xb[kChunkTiles];
      if constexpr (!kRecompute) {
#pragma unroll
        for (int i = 0; i < kChunkTiles; ++i) xb[i] = lrow[bcast32(tl, (uint32_t)i) * kTileIds + lane];
      } else {
        static_assert(kChunkTiles * 64 <= kTileWaves * kWaveTiles * 64, "a pass fits xbuf");
        for (uint32_t i = 0; i < nt; ++i) xbuf[i * 64u + lane] = tile_logit(uniform(tcand[base + i]));
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < kChunkTiles; ++i) xb[i] = xbuf[(uint32_t)i * 64u + lane];
      }
      // history bits of the lane's element of each tile, all requested first
      // (element 64 t + lane sits in bitmap word 2 t + lane / 32, bit lane % 32)
      uint32_t hw[kChunkTiles];
#pragma unroll
      for (int i = 0; i < kChunkTiles; ++i) hw[i] = bm[2u * bcast32(tl, (uint32_t)i) + (lane >> 5)];
      uint64_t ek[kChunkTiles];
#pragma unroll
      for (int i = 0; i < kChunkTiles; ++i) {
        const uint32_t v = bcast32(tl, (uint32_t)i) * kTileIds + lane;
        const bool hit = ((hw[i] >> (lane & 31u)) & 1u) != 0u;
        uint32_t yb = xb[i];
        // a tile rarely holds a history id: the penalty behind a wave-uniform branch
        if (__ballot(hit)) yb = hit ? penalize_bits(yb) : yb;
        ek[i] = (uint32_t)i < nt ? make_key(yb, v) : 0;
      }
      // Keys below the 20th best of the lanes' best (64 distinct elements)
      // or below the row's 20th best so far cannot enter the top-20.
      uint64_t lbe = 0;
#pragma unroll
      for (int i = 0; i < kChunkTiles; ++i) lbe = ek[i] > lbe ? ek[i] : lbe;
      uint64_t floor = shfl64(wave_sort_desc(lbe, lane), kTopK - 1);
      floor = floor > k20 ? floor : k20;
      uint64_t unused;
      const uint32_t nk = collect_range(ecand, ek, floor, ~0ull, unused);
      __builtin_amdgcn_wave_barrier();
      const uint64_t t20 = merge_all(top, ecand, nk, lane);
      k20 = t20 > k20 ? t20 : k20;
    }
    // stop once no tile left can reach the top-20
    const uint64_t best = wave_max64(rem);
    if (best == 0 || k20 > best) break;
    hi = thr;
  }
  const uint64_t key = top[lane < (uint32_t)kTopK ? lane : 0];
  finalize_row(rp, row, lane < (uint32_t)kTopK ? key : 0, kNone, 0u, kNone, lane, r24);
}

// MFMA layout self-test (one wave): A[i][k] = (7i + 3k) % 17 - 8 and
// B[k][j] = (5k + 11j) % 15 - 7 for i, j, k < 32, multiplied as four 16 x 16
// tiles through the head's fragment mapping, contraction order and
// accumulator start M: out[32 * i + j] = (D[i][j] read as binary32) - M.
__global__ __launch_bounds__(64) void mfma_selftest_kernel(int32_t* out) {
  const uint32_t lane = lane_id();
  const uint32_t n = lane & 15u;
  const uint32_t q = lane >> 4;
  const v4i magic = {(int)kMagicBits, (int)kMagicBits, (int)kMagicBits, (int)kMagicBits};
  for (uint32_t ti = 0; ti < 2; ++ti) {
    for (uint32_t tj = 0; tj < 2; ++tj) {
      uint64_t a = 0, b = 0;
      for (uint32_t slot = 0; slot < 8; ++slot) {
        const uint32_t k = slot < 4 ? 4u * q + slot : 16u + 4u * q + (slot - 4u);
        const uint32_t i = 16u * ti + n;
        const uint32_t j = 16u * tj + n;
        const int av = (int)((7u * i + 3u * k) % 17u) - 8;
        const int bv = (int)((5u * k + 11u * j) % 15u) - 7;
        a |= (uint64_t)((uint32_t)av & 0xffu) << (8 * slot);
        b |= (uint64_t)((uint32_t)bv & 0xffu) << (8 * slot);
      }
      const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)a, (long)b, magic, 0, 0, 0);
      for (int r = 0; r < 4; ++r) {
        const uint32_t i = 16u * ti + 4u * q + (uint32_t)r;
        const uint32_t j = 16u * tj + n;
        out[32 * i + j] = (int32_t)(__int_as_float(d[r]) - kMagic);
      }
    }
  }
}

hipError_t launch_lm_pack(const uint8_t* in, uint8_t* out, uint32_t vocab, uint32_t blocks,
                          hipStream_t stream) {
  (void)hipGetLastError();  // report only this call's launch errors
  const size_t n = (size_t)vocab * blocks;
  // the tile flags start at zero: a fill kernel rather than a memset, which a
  // caller capturing the repack in a graph could not replay reliably
  uint32_t* flags = reinterpret_cast<uint32_t*>(out + n * 18);
  hipLaunchKernelGGL(lm_clear_kernel, dim3((vocab / kTileIds + kBlockThreads - 1) / kBlockThreads),
                     dim3(kBlockThreads), 0, stream, flags, vocab / kTileIds);
  hipLaunchKernelGGL(lm_pack_kernel, dim3((uint32_t)((n + kBlockThreads - 1) / kBlockThreads)),
                     dim3(kBlockThreads), 0, stream, in, out, vocab, blocks);
  return hipGetLastError();
}

hipError_t launch_lm_pack_q8(const uint8_t* in, uint8_t* out, uint32_t vocab, uint32_t blocks,
                             hipStream_t stream) {
  (void)hipGetLastError();  // report only this call's launch errors
  const size_t n = (size_t)vocab * blocks;
  hipLaunchKernelGGL(lm_pack_q8_kernel, dim3((uint32_t)((n + kBlockThreads - 1) / kBlockThreads)),
                     dim3(kBlockThreads), 0, stream, in, out, vocab, blocks);
  return hipGetLastError();
}

size_t gemm_lds_bytes(uint32_t cols) {
  return (size_t)(cols / 32u) * (kRowsPerGroup + 2u * kTileIds) * sizeof(float);
}

// The narrow GEMM for one configuration: the Q4_0 block loop unrolled whole
// at the model's width of 896 (28 blocks), a loop otherwise.  (Unrolled, the
// Q8_0 kernels are scheduled with every block's results live at once: 512
// registers and scratch memory.)  Workgroups of four waves, two for the Q8_0
// head with one row tile.  Measured (whole step, us, Q4_0 / Q8_0), four /
// two / one / eight waves: B = 1 20.2 / 29.9, 21.2 / 29.1, 21.3 / 29.6,
// 21.1 / 32.1; B = 4 26.5 / 33.2, 27.2 / 33.4, 29.0 / 35.2, 27.5 / 36.1;
// B = 16 27.5 / 34.8, 28.2 / 33.8, 27.8 / 34.5, 30.2 / 38.9.
template <bool kQ8, int kRT, int kSets, int kI, bool kFused>
static void launch_narrow(uint32_t rows, hipStream_t stream, const LmParams& p) {
  constexpr int kNW = kQ8 && kRT == 1 ? 2 : 4;
  const dim3 grid((kTilesPerRow + kNW - 1) / kNW, (rows + 16u * kRT - 1) / (16u * kRT));
  if constexpr (!kQ8) {
    if (p.cols == kModelBlocks * 32u) {
      hipLaunchKernelGGL((lm_gemm_narrow_kernel<kQ8, kRT, kSets, kI, kFused, kModelBlocks, kNW>), grid,
                         dim3(64 * kNW), 0, stream, p);
      return;
    }
  }
  hipLaunchKernelGGL((lm_gemm_narrow_kernel<kQ8, kRT, kSets, kI, kFused, 0, kNW>), grid,
                     dim3(64 * kNW), 0, stream, p);
}

hipError_t launch_lm_sample(const LmParams& p, const RowParams& rp, hipStream_t stream) {
  (void)hipGetLastError();  // report only this call's launch errors
  if (!p.fused_quant) {
    const uint32_t pairs = p.rows_pad * (p.cols / 32u);  // eight lanes each
    hipLaunchKernelGGL(lm_quant_kernel, dim3((pairs + kBlockThreads / 8u - 1) / (kBlockThreads / 8u)),
                       dim3(kBlockThreads), 0, stream, p);
  }
  if (p.rows <= kNarrowRows) {
    // Loads one block ahead.  Measured (whole step, HIP events, us) with the
    // Q4_0 block loop unrolled at width 896, one / two / three / five / seven
    // blocks ahead: B = 1 19.5 / 20.5 / 20.7 / 22.8 / 23.0, B = 4 26.3 / 26.3
    // / 27.8 / 28.2 / 36.8, B = 32 39.7 / 40.7 / 42.2 / 43.2 / 51.7; two row
    // tiles (B = 64) 59.2 / 60.2 / 60.4 / 76.4 / 79.2.  Splitting a tile's
    // 28 blocks over two or four waves (each keeping its terms until the
    // previous part's running totals arrive through LDS, so the sums stay in
    // block order) was slower: B = 1 22.6-25.4 us.
    const uint32_t rt = p.rows <= 32u ? 1u : 2u;
    if (p.q8) {
      if (p.rows == 1)
        launch_narrow<true, 1, 2, 1, true>(p.rows, stream, p);
      else if (p.rows == 2)
        launch_narrow<true, 1, 2, 2, true>(p.rows, stream, p);
      else if (p.fused_quant)
        launch_narrow<true, 1, 2, 4, true>(p.rows, stream, p);
      else if (rt == 1)
        launch_narrow<true, 1, 2, 4, false>(p.rows, stream, p);
      else
        launch_narrow<true, 2, 2, 4, false>(p.rows, stream, p);
    } else {
      if (p.rows == 1)
        launch_narrow<false, 1, 2, 1, true>(p.rows, stream, p);
      else if (p.rows == 2)
        launch_narrow<false, 1, 2, 2, true>(p.rows, stream, p);
      else if (p.fused_quant)
        launch_narrow<false, 1, 2, 4, true>(p.rows, stream, p);
      else if (rt == 1)
        launch_narrow<false, 1, 2, 4, false>(p.rows, stream, p);
      else
        launch_narrow<false, 2, 2, 4, false>(p.rows, stream, p);
    }
  } else {
    const dim3 gemm_grid(kTilesPerRow, (p.rows_pad + kRowsPerGroup - 1) / kRowsPerGroup);
    const size_t lds = gemm_lds_bytes(p.cols);
    const bool model_width = p.cols == kModelBlocks * 32u;  // the Q4_0 loop unrolled whole
    if (p.logits == nullptr) {  // one pass: tile and second words, no logits
      if (p.q8)
        hipLaunchKernelGGL((lm_gemm_kernel<true, false>), gemm_grid, dim3(kGemmThreads), lds,
                           stream, p);
      else if (model_width)
        hipLaunchKernelGGL((lm_gemm_kernel<false, false, kModelBlocks>), gemm_grid,
                           dim3(kGemmThreads), lds, stream, p);
      else
        hipLaunchKernelGGL((lm_gemm_kernel<false, false>), gemm_grid, dim3(kGemmThreads), lds,
                           stream, p);
    } else if (p.q8) {
      hipLaunchKernelGGL((lm_gemm_kernel<true, true>), gemm_grid, dim3(kGemmThreads), lds, stream,
                         p);
    } else if (model_width) {
      hipLaunchKernelGGL((lm_gemm_kernel<false, true, kModelBlocks>), gemm_grid,
                         dim3(kGemmThreads), lds, stream, p);
    } else {
      hipLaunchKernelGGL((lm_gemm_kernel<false, true>), gemm_grid, dim3(kGemmThreads), lds,
                         stream, p);
    }
  }
  if (p.logits == nullptr) {  // one pass: no logits kept, the selection recomputes tiles
    if (p.q8)
      hipLaunchKernelGGL(lm_select_kernel<kRecomputeQ8>, dim3(p.rows), dim3(kSelectThreads), 0,
                         stream, p, rp);
    else
      hipLaunchKernelGGL(lm_select_kernel<kRecomputeQ4>, dim3(p.rows), dim3(kSelectThreads), 0,
                         stream, p, rp);
  } else {
    hipLaunchKernelGGL(lm_select_kernel<kFromLogits>, dim3(p.rows), dim3(kSelectThreads), 0,
                       stream, p, rp);
  }
  return hipGetLastError();
}

hipError_t launch_tile_select(const LmParams& p, const RowParams& rp, hipStream_t stream) {
  (void)hipGetLastError();  // report only this call's launch errors
  // Logits in HBM: two loads per thread, 75 workgroups per row (B = 1, 16,
  // 64, 192 steps 0.6, 0.6, 0.4, 0.2 us shorter than with four; one load or
  // eight were slower from 16 rows up).  Up to three rows, where 75
  // workgroups per row leave CUs idle, one load, 149 workgroups per row:
  // B = 1, 2, 3 cold steps 7.8, 8.2, 8.3 -> 7.6, 7.9, 8.1 us (wall, one box;
  // 64 or 128 threads per workgroup measured the same).  Logits in pinned
  // host memory: four, 38 workgroups.
  if (p.logits_copy == nullptr && p.rows <= 3u) {
    constexpr uint32_t kGroupTiles = 16u;
    hipLaunchKernelGGL(tile_words_kernel<1>,
                       dim3((kTilesPerRow + kGroupTiles - 1) / kGroupTiles, p.rows), dim3(256), 0,
                       stream, p);
  } else if (p.logits_copy == nullptr) {
    constexpr uint32_t kGroupTiles = 16u * 2u;
    hipLaunchKernelGGL(tile_words_kernel<2>,
                       dim3((kTilesPerRow + kGroupTiles - 1) / kGroupTiles, p.rows), dim3(256), 0,
                       stream, p);
  } else {
    constexpr uint32_t kGroupTiles = 16u * 4u;
    hipLaunchKernelGGL(tile_words_kernel<4>,
                       dim3((kTilesPerRow + kGroupTiles - 1) / kGroupTiles, p.rows), dim3(256), 0,
                       stream, p);
  }
  // logits read from pinned host memory: the selection reads the device copy
  // the first launch leaves
  LmParams sp = p;
  if (p.logits_copy != nullptr) {
    sp.logits = p.logits_copy;
    sp.logits_copy = nullptr;
  }
  hipLaunchKernelGGL(lm_select_kernel<kFromLogits>, dim3(p.rows), dim3(kSelectThreads), 0, stream,
                     sp, rp);
  return hipGetLastError();
}

hipError_t launch_mfma_selftest(int32_t* out, hipStream_t stream) {
  (void)hipGetLastError();  // report only this call's launch errors
  hipLaunchKernelGGL(mfma_selftest_kernel, dim3(1), dim3(64), 0, stream, out);
  return hipGetLastError();
}

}  // namespace pb

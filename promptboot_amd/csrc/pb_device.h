// pb_device.h -- device-side building blocks of the gfx950 decode-step sampler.
//
// Arithmetic contract: every binary32/binary64 operation here is a single
// IEEE-754 operation rounded to nearest-even with denormals preserved, in the
// same order as promptboot's scalar SSE2 sampler (crates/promptboot-core/src/
// fp32_sse2.rs:147-345 for the ops, :848-867 for the MXCSR 0x1f80 scope).
// The file is compiled with -ffp-contract=off and declares
// `#pragma clang fp contract(off)` so no multiply-add is ever fused, and
// fp32 division uses the correctly rounded expansion (HIP's default).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace pb {

constexpr uint32_t kVocab = 151936u;
constexpr int kTopK = 20;
constexpr uint32_t kNone = 0xffffffffu;

// Sampler constants as binary32 bit patterns (fp32_sse2.rs:1792-1795, 1855).
constexpr uint32_t kTemperatureBits = 0x3f333333u;  // 0.7f
constexpr uint32_t kTopPBits = 0x3f4ccccdu;         // 0.8f
constexpr uint32_t kPenaltyBits = 0x3f8ccccdu;      // 1.1f
constexpr uint32_t kTwoPow24Bits = 0x4b800000u;
// The quiet NaN x86 SSE produces for an invalid operation (inf - inf).
constexpr uint32_t kX86DefaultNaN = 0xffc00000u;

// Row flags (not part of the reference; reported beside each draw).
constexpr uint32_t kFlagDrawBoundary = 1u;
constexpr uint32_t kFlagCutoffBoundary = 2u;

__device__ __forceinline__ float f_of(uint32_t b) { return __uint_as_float(b); }

// Linear workgroup index -> work item, so that each XCD takes one contiguous
// range of the n items: the hardware hands workgroup L of a launch to XCD
// L % 8, and the workgroups that XCD k receives (L = k, k + 8, ...) take the
// items of its range in order.  A bijection of [0, n) for any n.
__device__ __forceinline__ uint32_t xcd_contiguous_item(uint32_t linear, uint32_t n) {
  const uint32_t k = linear & 7u, j = linear >> 3;
  const uint32_t per = n >> 3, extra = n & 7u;
  return k * per + (k < extra ? k : extra) + j;
}
__device__ __forceinline__ uint32_t b_of(float f) { return __float_as_uint(f); }

// ---- scalbnf / expf: FreeBSD e_expf method as adapted in
// fp32_sse2.rs:378-469 (rust-lang/libm 0.2.11), one IEEE op per step. ----
//
// ====================================================
// Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//
// Developed at SunPro, a Sun Microsystems, Inc. business.
// Permission to use, copy, modify, and distribute this
// software is freely granted, provided that this notice
// is preserved.
// ====================================================
__device__ __forceinline__ float scalbnf_ref(float value, int exponent) {
  const float two127 = f_of(0x7f000000u);
  const float two_m102 = f_of(0x0c800000u);  // 2^-126 * 2^24, exact
  if (exponent > 127) {
    value = value * two127;
    exponent -= 127;
    if (exponent > 127) {
      value = value * two127;
      exponent -= 127;
      if (exponent > 127) exponent = 127;
    }
  } else if (exponent < -126) {
    value = value * two_m102;
    exponent += 126 - 24;
    if (exponent < -126) {
      value = value * two_m102;
      exponent += 126 - 24;
      if (exponent < -126) exponent = -126;
    }
  }
  return value * f_of((uint32_t)(0x7f + exponent) << 23);
}

__device__ __forceinline__ float expf_ref(float x) {
  const uint32_t xb = b_of(x);
  const uint32_t magnitude = xb & 0x7fffffffu;
  const uint32_t sign = xb >> 31;
  if (magnitude >= 0x42aeac50u) {
    if (magnitude > 0x7f800000u) return x;
    if (magnitude >= 0x42b17218u && sign == 0) return x * f_of(0x7f000000u);
    if (sign != 0 && magnitude >= 0x42cff1b5u) return 0.0f;
  }
  int k;
  float hi, lo;
  if (magnitude > 0x3eb17218u) {
    if (magnitude > 0x3f851592u) {
      const float half = sign == 0 ? f_of(0x3f000000u) : f_of(0xbf000000u);
      const float scaled = f_of(0x3fb8aa3bu) * x;
      k = (int)(scaled + half);  // v_cvt_i32_f32 truncates toward zero
    } else {
      k = 1 - (int)sign - (int)sign;
    }
    const float kf = (float)k;
    const float khi = kf * f_of(0x3f317200u);
    hi = x - khi;
    lo = kf * f_of(0x35bfbe8eu);
    x = hi - lo;
  } else if (magnitude > 0x39000000u) {
    k = 0;
    hi = x;
    lo = 0.0f;
  } else {
    return f_of(0x3f800000u) + x;
  }
  const float xx = x * x;
  const float poly = f_of(0x3e2aaa8fu) + xx * f_of(0xbb355215u);
  const float c = x - xx * poly;
  const float num = x * c;
  const float den = f_of(0x40000000u) - c;
  const float frac = num / den;
  const float inner = (frac - lo) + hi;
  const float y = f_of(0x3f800000u) + inner;
  return k == 0 ? y : scalbnf_ref(y, k);
}

// Repetition penalty of one logit (fp32_sse2.rs:1860-1866): negative non-zero
// values are multiplied by 1.1f, everything else (positive, +0, -0) divided.
// The result never exceeds the input in IEEE order.
__device__ __forceinline__ uint32_t penalize_bits(uint32_t score) {
  const float p = f_of(kPenaltyBits);
  if ((score & 0x80000000u) != 0 && (score & 0x7fffffffu) != 0) return b_of(f_of(score) * p);
  return b_of(f_of(score) / p);
}

// ---- 64-bit selection keys ----
// key = ord(value) << 32 | (0x3ffff - id) << 1 | negzero.
// ord is the order-preserving map of binary32 with -0 folded onto +0, so a
// larger key means (larger value) or (equal value, smaller id): exactly the
// reference's rank order (strict `>` insertion over an ascending-id scan,
// fp32_sse2.rs:1797-1816).  The low bit keeps -0 recoverable; ids are below
// 2^18, so no two elements share a key and 0 is never a key.
__device__ __forceinline__ uint32_t ord_of(uint32_t bits) {
  if (bits == 0x80000000u) bits = 0u;
  return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}
__device__ __forceinline__ uint64_t make_key(uint32_t value_bits, uint32_t id) {
  const uint32_t low = ((0x3ffffu - id) << 1) | (value_bits == 0x80000000u ? 1u : 0u);
  return ((uint64_t)ord_of(value_bits) << 32) | low;
}
__device__ __forceinline__ uint32_t key_id(uint64_t key) {
  return 0x3ffffu - (((uint32_t)key >> 1) & 0x3ffffu);
}
__device__ __forceinline__ uint32_t key_value_bits(uint64_t key) {
  const uint32_t ord = (uint32_t)(key >> 32);
  uint32_t bits = (ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord;
  if (bits == 0u && (key & 1u)) bits = 0x80000000u;
  return bits;
}
// Lowest float that can still reach `key` (its value, ties included).
__device__ __forceinline__ float key_floor_value(uint64_t key) {
  if (key == 0) return -__builtin_inff();
  return f_of(key_value_bits(key));
}

// ---- wave (64-lane) primitives ----
__device__ __forceinline__ uint32_t lane_id() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}
// Value of lane (lane ^ j) for j in {1, 2, 4, 8, 16, 32}, without the LDS
// crossbar: DPP quad_perm for 1 and 2, DPP row rotations for 4 and 8 (a
// 16-lane row rotated by 8 is lane ^ 8; rotations by 4 and 12 give the two
// halves of lane ^ 4), and gfx950's v_permlane16_swap / v_permlane32_swap
// for 16 and 32.  Every lane of the wave must be active.  `j` must fold to a
// constant at each call site (unrolled loops).
// Every source lane of these patterns is valid, so the DPP `old` operand is
// never selected; passing 0 with bound_ctrl lets the compiler emit a single
// v_mov_b32_dpp (or fold it into the consumer) instead of a copy and a move.
__device__ __forceinline__ uint32_t lane_xor(uint32_t v, uint32_t j, uint32_t lane) {
  const int iv = (int)v;
  switch (j) {
    case 1:
      return (uint32_t)__builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, true);  // [1,0,3,2]
    case 2:
      return (uint32_t)__builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, true);  // [2,3,0,1]
    case 4: {
      const uint32_t from_above = (uint32_t)__builtin_amdgcn_update_dpp(0, iv, 0x12C, 0xF, 0xF, true);
      const uint32_t from_below = (uint32_t)__builtin_amdgcn_update_dpp(0, iv, 0x124, 0xF, 0xF, true);
      return (lane & 4u) ? from_below : from_above;
    }
    case 8:
      return (uint32_t)__builtin_amdgcn_update_dpp(0, iv, 0x128, 0xF, 0xF, true);  // row_ror:8
    case 16: {
      const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
      return (lane & 16u) ? r[0] : r[1];
    }
    default: {
      const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
      return (lane & 32u) ? r[0] : r[1];
    }
  }
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int mask) {
  const uint32_t lane = lane_id();
  const uint32_t lo = lane_xor((uint32_t)v, (uint32_t)mask, lane);
  const uint32_t hi = lane_xor((uint32_t)(v >> 32), (uint32_t)mask, lane);
  return ((uint64_t)hi << 32) | lo;
}
// Broadcast from one lane; `src` must be the same in every lane (v_readlane).
__device__ __forceinline__ uint32_t bcast32(uint32_t v, uint32_t src) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)src);
}
__device__ __forceinline__ uint64_t shfl64(uint64_t v, uint32_t src) {
  const uint32_t lo = bcast32((uint32_t)v, src);
  const uint32_t hi = bcast32((uint32_t)(v >> 32), src);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ float bcast_f32(float v, uint32_t src) {
  return __uint_as_float(bcast32(__float_as_uint(v), src));
}
__device__ __forceinline__ double bcast_f64(double v, uint32_t src) {
  return __builtin_bit_cast(double, shfl64(__builtin_bit_cast(uint64_t, v), src));
}

// Bitonic sort of one key per lane, descending (lane 0 holds the maximum),
// over groups of kLanes lanes (32 or 64; with 32 each half of the wave is
// sorted on its own).
template <uint32_t kLanes = 64>
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t key, uint32_t lane) {
#pragma unroll
  for (uint32_t k = 2; k <= kLanes; k <<= 1) {
#pragma unroll
    for (uint32_t j = k >> 1; j > 0; j >>= 1) {
      const uint64_t other = shfl_xor64(key, (int)j);
      const bool lower = (lane & j) == 0;
      const bool desc = (lane & k) == 0;
      const bool take_max = lower == desc;
      const uint64_t hi = key > other ? key : other;
      const uint64_t lo = key > other ? other : key;
      key = take_max ? hi : lo;
    }
  }
  return key;
}

// Bitonic sort of one 32-bit value per lane, descending, over groups of
// kLanes lanes (32 or 64; with 32 each half of the wave is sorted on its own).
template <uint32_t kLanes = 64>
__device__ __forceinline__ uint32_t wave_sort_desc_u32(uint32_t v, uint32_t lane) {
#pragma unroll
  for (uint32_t k = 2; k <= kLanes; k <<= 1) {
#pragma unroll
    for (uint32_t j = k >> 1; j > 0; j >>= 1) {
      const uint32_t other = lane_xor(v, j, lane);
      const bool take_max = ((lane & j) == 0) == ((lane & k) == 0);
      const uint32_t hi = v > other ? v : other;
      const uint32_t lo = v > other ? other : v;
      v = take_max ? hi : lo;
    }
  }
  return v;
}

struct KeepKey {
  __device__ uint64_t operator()(uint64_t key) const { return key; }
};

// One merge round: the wave's current top-20 (LDS, sorted, 0 = empty) plus up
// to 44 new keys from `src` are sorted; the best 20 become the new top.  Each
// new key passes through `fix` first (the sampler applies the history penalty
// there).  Returns the new 20th key (0 while fewer than 20 real keys are held).
template <typename SrcPtr, typename Fix = KeepKey>
__device__ __forceinline__ uint64_t merge_round(uint64_t* top, SrcPtr src, uint32_t n,
                                                uint32_t lane, Fix fix = Fix()) {
  uint64_t key = 0;
  if (lane < (uint32_t)kTopK) {
    key = top[lane];
  } else if (lane - kTopK < n) {
    key = fix(src[lane - kTopK]);
  }
  key = wave_sort_desc(key, lane);
  __builtin_amdgcn_wave_barrier();
  if (lane < (uint32_t)kTopK) top[lane] = key;
  __builtin_amdgcn_wave_barrier();
  return shfl64(key, kTopK - 1);
}

constexpr uint32_t kMergeTake = 64 - kTopK;  // 44 new keys per round

// Top-20 of two sorted (descending, 20 keys, 0 = empty) lists with one
// bitonic merge: lanes 0..31 hold `a` descending (zero-padded), lanes 32..63
// hold `b` ascending, so the 64 keys form a bitonic sequence and six
// compare-exchange stages sort them.  Lane i < 20 returns the i-th best key.
__device__ __forceinline__ uint64_t merge_two_lists(const uint64_t* a, const uint64_t* b,
                                                    uint32_t lane) {
  uint64_t key = 0;
  if (lane < (uint32_t)kTopK) {
    key = a[lane];
  } else if (lane >= 64u - kTopK) {
    key = b[63u - lane];
  }
#pragma unroll
  for (uint32_t j = 32; j > 0; j >>= 1) {
    const uint64_t other = shfl_xor64(key, (int)j);
    const bool lower = (lane & j) == 0;
    const uint64_t hi = key > other ? key : other;
    const uint64_t lo = key > other ? other : key;
    key = lower ? hi : lo;
  }
  return key;
}

// Merge `n` keys from src into top (any n), in rounds of 44.
template <typename SrcPtr>
__device__ __forceinline__ uint64_t merge_all(uint64_t* top, SrcPtr src, uint32_t n,
                                              uint32_t lane) {
  uint64_t thr = 0;
  uint32_t done = 0;
  while (done < n) {
    const uint32_t take = (n - done) < kMergeTake ? (n - done) : kMergeTake;
    thr = merge_round(top, src + done, take, lane);
    done += take;
  }
  return thr;
}

__device__ __forceinline__ uint64_t wave_max64(uint64_t v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const uint64_t o = shfl_xor64(v, m);
    v = o > v ? o : v;
  }
  return v;
}

// Top-20 of up to 64 lists, each sorted descending with 20 keys (0 = empty),
// list l at lists[l * 20].  One list per lane; 20 steps of "take the largest
// head".  Lane i < 20 returns the i-th best key.  Keys are unique, so exactly
// one lane owns each maximum.
__device__ __forceinline__ uint64_t merge_sorted_lists(const uint64_t* lists, uint32_t nlists,
                                                       uint32_t lane) {
  uint32_t pos = 0;
  uint64_t head = lane < nlists ? lists[lane * kTopK] : 0;
  uint64_t mine = 0;
#pragma unroll 1
  for (int i = 0; i < kTopK; ++i) {
    const uint64_t m = wave_max64(head);
    if (lane == (uint32_t)i) mine = m;
    if (m != 0 && head == m) {
      ++pos;
      head = pos < (uint32_t)kTopK ? lists[lane * kTopK + pos] : 0;
    }
  }
  return mine;
}

// Top-20 of `nlists` (1..32) sorted lists as merge_sorted_lists, with two
// wave sorts instead of 20 dependent wave maxima.  With m = ceil(20 / n) and
// r = ceil(20 / m), take the r-th best value among the lists' m-th keys: the
// smallest key of that value, T, is reached by at least r * m >= 20 keys, so
// the top-20 lies among the keys >= T.  Those are a prefix of each list,
// gathered into `scratch` (64 keys of LDS) and sorted once.  Above 64 such
// keys it falls back to merge_sorted_lists.  Lane i < 20 returns the i-th
// best key.
__device__ __forceinline__ uint64_t merge_lists_by_threshold(const uint64_t* lists,
                                                             uint32_t nlists, uint64_t* scratch,
                                                             uint32_t lane) {
  const uint32_t m = ((uint32_t)kTopK + nlists - 1u) / nlists;
  const uint32_t r = ((uint32_t)kTopK + m - 1u) / m;
  const bool own = lane < nlists;
  const uint64_t* mine = lists + lane * kTopK;
  const uint32_t c = own ? (uint32_t)(mine[m - 1u] >> 32) : 0u;
  const uint64_t t = (uint64_t)bcast32(wave_sort_desc_u32<32>(c, lane), r - 1u) << 32;
  // The lane's list stays in registers for the gather below: a loop that
  // re-reads each key from LDS before storing it waits once per key.
  uint64_t kk[kTopK];
  uint32_t n = 0;
#pragma unroll
  for (int q = 0; q < kTopK; ++q) {
    kk[q] = own ? mine[q] : 0;
    n += (kk[q] != 0 && kk[q] >= t) ? 1u : 0u;
  }
  // exclusive prefix of n (< 32) over the lanes, one ballot per bit
  const uint64_t below = (1ull << lane) - 1ull;
  uint32_t before = 0, total = 0;
#pragma unroll
  for (int b = 0; b < 5; ++b) {
    const uint64_t bits = __ballot((n >> b) & 1u);
    before += (uint32_t)__popcll((unsigned long long)(bits & below)) << b;
    total += (uint32_t)__popcll((unsigned long long)bits) << b;
  }
  if (total > 64u) return merge_sorted_lists(lists, nlists, lane);
#pragma unroll
  for (uint32_t q = 0; q < (uint32_t)kTopK; ++q) {
    if (q < n) scratch[before + q] = kk[q];
  }
  __builtin_amdgcn_wave_barrier();
  uint64_t key = lane < total ? scratch[lane] : 0;
  __builtin_amdgcn_wave_barrier();
  return wave_sort_desc(key, lane);
}

}  // namespace pb

// pb_rows.h -- per-row epilogue shared by the sampler and the fused LM head:
// softmax weights, top-p cutoff and the categorical draw over a row's top-20,
// plus the per-row error records.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pb_device.h"
#include "pb_internal.h"

#pragma clang fp contract(off)

namespace pb {

constexpr uint64_t kErrDetailFinite = (uint64_t)7 << 32;
constexpr uint64_t kErrDetailToken = (uint64_t)2 << 32;

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const uint32_t o = lane_xor(v, (uint32_t)m, lane_id());
    v = o < v ? o : v;
  }
  return v;
}

// A per-row word read through the scalar cache (s_load, counted apart from
// vector loads, so that waiting for it does not wait for a row's streams).
// Only for words that no wave of the launch writes before this read: the
// row's own state and length, which its own workgroup updates at the end.
__device__ __forceinline__ uint32_t row_word(const uint32_t* ptr) {
  return *(const __attribute__((address_space(4))) uint32_t*)ptr;
}

// Context cap of a row in decode-loop mode: max_len[row], at most hist_ld.
__device__ __forceinline__ uint32_t row_cap(const RowParams& p, uint32_t row) {
  uint32_t cap = (uint32_t)p.hist_ld;
  if (p.max_len != nullptr) {
    const uint32_t m = row_word(p.max_len + row);
    cap = m < cap ? m : cap;
  }
  return cap;
}

// True when a launch in decode-loop mode must skip `row`: the row has ended,
// or its context is already at its cap (the REPL never samples without room).
__device__ __forceinline__ bool row_skipped(const RowParams& p, uint32_t row) {
  if (p.row_state == nullptr) return false;
  if (row_word(p.row_state + row) != PB_ROW_ACTIVE) return true;
  return row_word(p.hist_len_out + row) >= row_cap(p, row);
}

// Outputs of a skipped row (one lane): no token; a row that was still active
// (its context is full) ends at its limit.  Its detail and error records are
// not written.
__device__ __forceinline__ void skip_row(const RowParams& p, uint32_t row) {
  p.token[row] = kNone;
  if (row_word(p.row_state + row) == PB_ROW_ACTIVE) p.row_state[row] = PB_ROW_LIMIT;
}

// Decode-loop bookkeeping after a row's sample (one lane): the working
// context receives the token, an end-of-sequence piece as <|im_end|>
// (model_repl.rs:1099-1103), and the row ends on end-of-sequence
// (:1119-1150), on its length limit, or on an error (no append).
__device__ __forceinline__ void decode_commit(const RowParams& p, uint32_t row, uint32_t token) {
  if (p.row_state == nullptr) return;
  if (token == kNone) {
    p.row_state[row] = PB_ROW_ERROR;
    return;
  }
  uint32_t cap = (uint32_t)p.hist_ld;
  if (p.max_len != nullptr && p.max_len[row] < cap) cap = p.max_len[row];
  const uint32_t len = p.hist_len_out[row];
  const bool eos = token == PB_IM_END || token == PB_END_OF_TEXT;
  uint32_t state = PB_ROW_LIMIT;
  if (len < cap) {
    p.hist_out[(size_t)row * p.hist_ld + len] = eos ? PB_IM_END : token;
    p.hist_len_out[row] = len + 1u;
    state = eos ? PB_ROW_EOS : (len + 1u == cap ? PB_ROW_LIMIT : PB_ROW_ACTIVE);
  }
  p.row_state[row] = state;
}

// Finishes one row on one wave: lanes 0..19 hold the row's top-20 keys in
// rank order.  Softmax weights, top-p cutoff and the categorical draw follow
// fp32_sse2.rs:1818-1845 operation for operation; the binary64 sums run as a
// lane-serial chain in rank order, so every partial sum is the reference's.
// `r24` is the row's uniform (random_24[row]), which callers request early.
// An error row: bad_logit is the first non-finite index (bad_bits its bits)
// or kNone, bad_hist the first history position holding an id >= vocab.
__device__ __forceinline__ void finalize_row(const RowParams& p, uint32_t row, uint64_t key,
                                             uint32_t bad_logit, uint32_t bad_bits,
                                             uint32_t bad_hist, uint32_t lane, uint32_t r24) {
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
      e.available = bad_bits;
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
      decode_commit(p, row, kNone);
    }
    if (p.detail) {
      uint32_t* d = reinterpret_cast<uint32_t*>(p.detail + row);
      for (uint32_t i = lane; i < sizeof(pb_sample_detail) / 4; i += 64) d[i] = 0xffffffffu;
    }
    return;
  }

  const uint32_t id = key_id(key);
  const uint32_t vbits = key_value_bits(key);
  const float maximum = f_of(bcast32(vbits, 0));
  float w = 0.0f;
  if (lane < (uint32_t)kTopK) {
    const float shifted = f_of(vbits) - maximum;
    w = expf_ref(shifted / f_of(kTemperatureBits));
    // The only NaN here is -inf - -inf (every top-20 value penalised to
    // -inf): x86 SSE returns its default NaN 0xffc00000 for that invalid
    // operation and passes it through the divide and expf unchanged, while
    // the GPU's default NaN is positive.  The weights and probabilities
    // reported carry the reference's bits.
    if (w != w) w = f_of(kX86DefaultNaN);
  }
  double running = 0.0, mine = 0.0;
#pragma unroll
  for (int i = 0; i < kTopK; ++i) {
    const float wi = bcast_f32(w, (uint32_t)i);
    running = running + (double)wi;
    if (lane == (uint32_t)i) mine = running;
  }
  const double total = running;
  const float cutoff = (float)total * f_of(kTopPBits);
  const uint64_t stop = __ballot(lane < (uint32_t)kTopK && !(cutoff > (float)mine));
  const uint32_t kept = stop ? (uint32_t)__ffsll((unsigned long long)stop) : (uint32_t)kTopK;
  const double kept_total = bcast_f64(mine, kept - 1);
  const float unit = (float)(r24 & 0x00ffffffu) / f_of(kTwoPow24Bits);
  const float target = (float)kept_total * unit;
  const uint64_t hit = __ballot(lane < kept && (float)mine > target);
  const uint32_t rank = hit ? (uint32_t)__ffsll((unsigned long long)hit) - 1 : kept - 1;
  const uint32_t token = bcast32(id, rank);

  if (lane == 0) {
    p.token[row] = token;
    decode_commit(p, row, token);
  }
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
      float prob = lane < kept ? (float)((double)w / kept_total) : 0.0f;
      if (prob != prob) prob = f_of(kX86DefaultNaN);  // NaN weights: x86's NaN, as above
      d->probs[lane] = prob;
    }
    if (lane == 0) {
      d->kept = kept;
      d->rank = rank;
      d->flags = flags;
      d->token = token;
    }
  }
}

}  // namespace pb

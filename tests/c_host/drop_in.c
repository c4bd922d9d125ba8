/* A plain C host of the sampler library: the calls a non-Python caller (a
 * Rust FFI crate, the REPL's decode loop) makes through include/pbsample.h,
 * with no Python or PyTorch in the process.
 *
 * Usage: drop_in <golden dir> <output dir>
 *
 * On the real Qwen "hello" row (tests/golden) it runs, in order:
 *   1. pb_sample_token_with_repetition with one word too few: the error tuple,
 *      and the row, `seen` and the state left untouched (transactional);
 *   2. the same call on the whole row: token, state, `seen` cleared, and the
 *      penalised row written to <output dir>/hello_penalised.u32le;
 *   3. pb_greedy_token and pb_top_logits_8 on the original row;
 *   4. pb_sample_batch on device copies of the three real rows
 *      (hello, arithmetic, color) with their prompts as histories.
 * It prints one `key value...` line per result; the Python test compares them
 * with the oracle. */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pbsample.h"

static uint32_t *read_words(const char *dir, const char *name, size_t *n) {
  char path[1024];
  snprintf(path, sizeof path, "%s/%s", dir, name);
  FILE *f = fopen(path, "rb");
  if (!f) {
    fprintf(stderr, "cannot open %s\n", path);
    exit(2);
  }
  fseek(f, 0, SEEK_END);
  long bytes = ftell(f);
  fseek(f, 0, SEEK_SET);
  uint32_t *w = malloc((size_t)bytes);
  if (!w || fread(w, 1, (size_t)bytes, f) != (size_t)bytes) exit(2);
  fclose(f);
  *n = (size_t)bytes / 4;
  return w;
}

static void print_error(const char *key, const pb_inference_error *e) {
  printf("%s %u %u %u %u %u %llu %llu %llu\n", key, e->status, e->domain, e->layer, e->position,
         e->tensor_id, (unsigned long long)e->needed, (unsigned long long)e->available,
         (unsigned long long)e->detail);
}

#define HIP_OK(x)                                                    \
  do {                                                               \
    hipError_t rc_ = (x);                                            \
    if (rc_ != hipSuccess) {                                         \
      fprintf(stderr, "%s failed: %d\n", #x, (int)rc_);              \
      exit(3);                                                       \
    }                                                                \
  } while (0)

int main(int argc, char **argv) {
  if (argc != 3) {
    fprintf(stderr, "usage: drop_in <golden dir> <output dir>\n");
    return 2;
  }
  const char *golden = argv[1];
  size_t n_logits, n_prompt;
  uint32_t *logits = read_words(golden, "qwen_hello_logits.f32le", &n_logits);
  uint32_t *prompt = read_words(golden, "qwen_hello_prompt.u32le", &n_prompt);
  uint32_t *original = malloc(n_logits * 4);
  memcpy(original, logits, n_logits * 4);
  static uint8_t seen[PB_SEEN_BYTES];
  pb_sampling_state state;
  pb_sampling_state_new(&state, 0x0123456789abcdefull);
  pb_inference_error err;
  uint32_t token = 0;

  /* 1. one word too few: nothing changes */
  uint32_t st = pb_sample_token_with_repetition(logits, n_logits - 1, prompt, n_prompt, seen,
                                                sizeof seen, &state, &token, &err);
  print_error("short_error", &err);
  int seen_zero = 1;
  for (size_t i = 0; i < sizeof seen; ++i) seen_zero &= seen[i] == 0;
  printf("short_status %u unchanged %d seen_zero %d draws %llu\n", st,
         memcmp(logits, original, n_logits * 4) == 0, seen_zero,
         (unsigned long long)state.draws);

  /* 2. the whole row */
  st = pb_sample_token_with_repetition(logits, n_logits, prompt, n_prompt, seen, sizeof seen,
                                       &state, &token, &err);
  seen_zero = 1;
  for (size_t i = 0; i < sizeof seen; ++i) seen_zero &= seen[i] == 0;
  printf("sample_status %u token %u state %llu draws %llu seen_zero %d\n", st, token,
         (unsigned long long)state.state, (unsigned long long)state.draws, seen_zero);
  char path[1024];
  snprintf(path, sizeof path, "%s/hello_penalised.u32le", argv[2]);
  FILE *out = fopen(path, "wb");
  if (!out || fwrite(logits, 4, n_logits, out) != n_logits) return 2;
  fclose(out);

  /* 3. greedy and top-8 of the original row */
  st = pb_greedy_token(original, n_logits, &token, &err);
  printf("greedy_status %u token %u\n", st, token);
  pb_top_logit top[8];
  st = pb_top_logits_8(original, n_logits, top, &err);
  printf("top8_status %u", st);
  for (int i = 0; i < 8; ++i) printf(" %u %u", top[i].token, top[i].logit_bits);
  printf("\n");

  /* 4. the batched device entry point on the three real rows */
  const char *cases[3] = {"hello", "arithmetic", "color"};
  const uint32_t rows = 3;
  const size_t hist_ld = 64;
  uint32_t *h_logits = calloc((size_t)rows * PB_VOCAB, 4);
  uint32_t *h_hist = calloc((size_t)rows * hist_ld, 4);
  uint32_t h_len[3], h_r24[3], h_token[3];
  pb_sampling_state states[3];
  for (uint32_t r = 0; r < rows; ++r) {
    char name[256];
    size_t n, m;
    snprintf(name, sizeof name, "qwen_%s_logits.f32le", cases[r]);
    uint32_t *row = read_words(golden, name, &n);
    snprintf(name, sizeof name, "qwen_%s_prompt.u32le", cases[r]);
    uint32_t *ids = read_words(golden, name, &m);
    if (n != PB_VOCAB || m > hist_ld) return 2;
    memcpy(h_logits + (size_t)r * PB_VOCAB, row, n * 4);
    memcpy(h_hist + (size_t)r * hist_ld, ids, m * 4);
    h_len[r] = (uint32_t)m;
    pb_sampling_state_new(&states[r], 42u + r);
    free(row);
    free(ids);
  }
  pb_fill_random_24(states, rows, h_r24);
  pb_context *ctx = NULL;
  st = pb_context_create(0, &ctx);
  if (st != 0) {
    fprintf(stderr, "pb_context_create: %u\n", st);
    return 3;
  }
  uint32_t *d_logits, *d_hist, *d_len, *d_r24, *d_token;
  HIP_OK(hipMalloc((void **)&d_logits, (size_t)rows * PB_VOCAB * 4));
  HIP_OK(hipMalloc((void **)&d_hist, (size_t)rows * hist_ld * 4));
  HIP_OK(hipMalloc((void **)&d_len, rows * 4));
  HIP_OK(hipMalloc((void **)&d_r24, rows * 4));
  HIP_OK(hipMalloc((void **)&d_token, rows * 4));
  HIP_OK(hipMemcpy(d_logits, h_logits, (size_t)rows * PB_VOCAB * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_hist, h_hist, (size_t)rows * hist_ld * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_len, h_len, rows * 4, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(d_r24, h_r24, rows * 4, hipMemcpyHostToDevice));
  st = pb_sample_batch(ctx, d_logits, PB_VOCAB, PB_VOCAB, rows, d_hist, hist_ld, d_len, d_r24,
                       d_token, NULL, NULL, NULL, &err);
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(h_token, d_token, rows * 4, hipMemcpyDeviceToHost));
  printf("batch_status %u tokens %u %u %u r24 %u %u %u\n", st, h_token[0], h_token[1],
         h_token[2], h_r24[0], h_r24[1], h_r24[2]);
  HIP_OK(hipFree(d_logits));
  HIP_OK(hipFree(d_hist));
  HIP_OK(hipFree(d_len));
  HIP_OK(hipFree(d_r24));
  HIP_OK(hipFree(d_token));
  pb_context_destroy(ctx);
  free(h_logits);
  free(h_hist);
  free(logits);
  free(prompt);
  free(original);
  printf("done\n");
  return 0;
}

/*
 * A plain C host of the C ABI (include/ferric_hip.h), doing what the Rust
 * binding in INTEGRATION.md does on the reference's side of the boundary:
 * create a context, make weights and KV prefixes, run greedy decode steps
 * through fh_execute_batch with caller-owned page lists, hit a validation
 * failure (which must not poison the context), run a prefill batch larger
 * than row_capacity, destroy. It prints one line per step; the GPU test
 * tests/test_gpu_c_abi.py runs the same scenario through the Python runner
 * and compares every choice.
 *
 * Model: Qwen3-0.6B shape with 2 layers; 4 sequences with KV prefixes of 5,
 * 17, 40 and 100 tokens; pages from a fixed permutation of the pool.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ferric_hip.h"

#define SEQS 4
#define STEPS 6
#define STRIDE 16
#define POOL 96
#define PREFILL 20

static uint32_t perm[POOL];
static uint32_t pages[SEQS + 1][STRIDE];

static int check(fh_status st, fh_ctx* ctx, const char* what) {
  if (st != FH_OK) {
    printf("error %s: status %d: %s\n", what, (int)st, fh_last_error(ctx));
    return 1;
  }
  return 0;
}

int main(void) {
  /* A fixed permutation of the physical pages (LCG-driven Fisher-Yates). */
  uint64_t lcg = 0x9e3779b97f4a7c15ull;
  for (uint32_t i = 0; i < POOL; ++i) perm[i] = i;
  for (uint32_t i = POOL - 1; i > 0; --i) {
    lcg = lcg * 6364136223846793005ull + 1442695040888963407ull;
    const uint32_t j = (uint32_t)((lcg >> 33) % (i + 1));
    const uint32_t t = perm[i];
    perm[i] = perm[j];
    perm[j] = t;
  }
  for (uint32_t s = 0; s <= SEQS; ++s)
    for (uint32_t p = 0; p < STRIDE; ++p) pages[s][p] = perm[s * STRIDE + p];

  const fh_model_desc model = {2, 1024, 16, 8, 128, 3072, 151936, 1, 1000000, 1e-6f};
  const fh_ctx_options opts = {8, POOL, STRIDE, STRIDE * 16, 1, 0, 0, 64};
  fh_ctx* ctx = NULL;
  if (check(fh_create(&model, &opts, &ctx), NULL, "create")) return 1;
  printf("row_capacity %u\n", fh_row_capacity(ctx));
  if (check(fh_synthesize_weights(ctx, 7, 0.02f), ctx, "synthesize")) return 1;

  const uint32_t prefix[SEQS] = {5, 17, 40, 100};
  const uint64_t keys[SEQS] = {11, 12, 13, 14};
  fh_row rows[PREFILL];
  for (uint32_t s = 0; s < SEQS; ++s) {
    rows[s].sequence = s + 1;
    rows[s].token = 0;
    rows[s].position = prefix[s];
    rows[s].pages = pages[s];
    rows[s].page_count = STRIDE;
    rows[s].writable_page = pages[s][prefix[s] / 16];
  }
  if (check(fh_kv_fill_synthetic(ctx, 5, 1.0f, rows, keys, SEQS, STRIDE * 16), ctx, "kv fill")) return 1;

  uint32_t tokens[SEQS] = {1000, 2000, 3000, 4000};
  uint32_t out_rows[PREFILL];
  uint32_t choices[PREFILL];
  for (uint32_t i = 0; i < PREFILL; ++i) out_rows[i] = i;
  uint64_t batch = 1;
  for (uint32_t step = 0; step < STEPS; ++step) {
    for (uint32_t s = 0; s < SEQS; ++s) {
      const uint32_t pos = prefix[s] + step;
      rows[s].token = tokens[s];
      rows[s].position = pos;
      rows[s].writable_page = pages[s][pos / 16];
    }
    if (check(fh_execute_batch(ctx, batch++, rows, SEQS, out_rows, SEQS, choices), ctx, "decode")) return 1;
    printf("decode %u:", step);
    for (uint32_t s = 0; s < SEQS; ++s) {
      printf(" %u", choices[s]);
      tokens[s] = choices[s];
    }
    printf("\n");
  }

  /* A row whose writable page is not pages[position / 16]: rejected before
     anything runs, and the context stays usable. */
  rows[0].position = prefix[0] + STEPS; /* page 0 of its list */
  rows[0].writable_page = pages[0][1];   /* a different page: pages are distinct */
  const fh_status bad = fh_execute_batch(ctx, batch++, rows, 1, out_rows, 1, choices);
  printf("invalid row: status %d, message %s\n", (int)bad, fh_last_error(ctx)[0] ? "set" : "empty");

  /* Prefill: a new sequence's 20-token prompt from position 0 (more rows than
     row_capacity), then one decode step of it. */
  for (uint32_t i = 0; i < PREFILL; ++i) {
    rows[i].sequence = SEQS + 1;
    rows[i].token = 100 + 37 * i;
    rows[i].position = i;
    rows[i].pages = pages[SEQS];
    rows[i].page_count = STRIDE;
    rows[i].writable_page = pages[SEQS][i / 16];
  }
  const uint32_t last = PREFILL - 1;
  if (check(fh_execute_batch(ctx, batch++, rows, PREFILL, &last, 1, choices), ctx, "prefill")) return 1;
  printf("prefill: %u\n", choices[0]);
  rows[0].token = choices[0];
  rows[0].position = PREFILL;
  rows[0].writable_page = pages[SEQS][PREFILL / 16];
  if (check(fh_execute_batch(ctx, batch++, rows, 1, out_rows, 1, choices), ctx, "decode after prefill")) return 1;
  printf("after prefill: %u\n", choices[0]);
  printf("dispatches %llu\n", (unsigned long long)fh_dispatch_count(ctx));
  fh_destroy(ctx);
  printf("done\n");
  return 0;
}

/* CPU oracle, C restatement of the integer part of the MoE hot path (router logits, top-k, layout).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ and the checker in __graft_entry__.smoke(); the product
 * path never links it.  It exists because the numpy restatement (oracle/moe_oracle.py) is too slow at
 * the full benchmark sizes; tests pin this file against the numpy one bit for bit.
 *
 *  oracle_router_logits  logits[t,e] = sum_i x[t,i] * w[i,e], summed sequentially over i in float32,
 *                        then + bias[e] (MaxText RoutedMoE gate; numerics contract of moe_oracle.py).
 *  oracle_topk           k largest logits per token, descending, ties -> lower expert index
 *                        (argsort(-logits)[:, :k] as in modal/test_moe_permute.py:23-26).
 *  oracle_layout         stable counting sort of the flat slots by expert (modal/moe_permute.py:240-264)
 *                        plus the 128-row padded block layout.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float bf16f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void oracle_router_logits(const uint16_t* x, const uint16_t* w, const float* bias, int64_t T, int64_t d,
                          int64_t E, float* logits) {
  float* wf = (float*)malloc(sizeof(float) * d * E);
  for (int64_t i = 0; i < d * E; ++i) wf[i] = bf16f(w[i]);
  for (int64_t t = 0; t < T; ++t) {
    float* acc = logits + t * E;
    for (int64_t e = 0; e < E; ++e) acc[e] = 0.0f;
    for (int64_t i = 0; i < d; ++i) {
      const float xv = bf16f(x[t * d + i]);
      const float* wr = wf + i * E;
      for (int64_t e = 0; e < E; ++e) {
        const float prod = xv * wr[e]; /* exact: both factors are bf16 */
        acc[e] = acc[e] + prod;
      }
    }
    if (bias)
      for (int64_t e = 0; e < E; ++e) acc[e] = acc[e] + bias[e];
  }
  free(wf);
}

void oracle_topk(const float* logits, int64_t T, int64_t E, int64_t k, int32_t* sel) {
  unsigned char* taken = (unsigned char*)malloc((size_t)E);
  for (int64_t t = 0; t < T; ++t) {
    const float* l = logits + t * E;
    memset(taken, 0, (size_t)E);
    for (int64_t j = 0; j < k; ++j) {
      int64_t best = -1;
      for (int64_t e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || l[e] > l[best]) best = e; /* strict '>' keeps the lower index on ties */
      }
      taken[best] = 1;
      sel[t * k + j] = (int32_t)best;
    }
  }
  free(taken);
}

/* gs, offsets, block_off: [E]; order, pos, slot: [M]; returns the number of blocks. */
int64_t oracle_layout(const int32_t* flat, int64_t M, int64_t E, int64_t block, int32_t* gs, int32_t* offsets,
                      int32_t* block_off, int32_t* order, int32_t* pos, int32_t* slot) {
  int64_t* cursor = (int64_t*)calloc((size_t)E, sizeof(int64_t));
  for (int64_t e = 0; e < E; ++e) gs[e] = 0;
  for (int64_t i = 0; i < M; ++i) gs[flat[i]]++;
  int64_t run = 0, brun = 0;
  for (int64_t e = 0; e < E; ++e) {
    offsets[e] = (int32_t)run;
    block_off[e] = (int32_t)brun;
    cursor[e] = run;
    run += gs[e];
    brun += (gs[e] + block - 1) / block;
  }
  for (int64_t i = 0; i < M; ++i) { /* ascending i: stable */
    const int32_t e = flat[i];
    const int64_t p = cursor[e]++;
    pos[i] = (int32_t)p;
    order[p] = (int32_t)i;
    slot[i] = (int32_t)(block * block_off[e] + (p - offsets[e]));
  }
  free(cursor);
  return brun;
}

/*
 * pkv_oracle.c — CPU restatement of the PersistentKV paged decode algorithm.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP engine: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and never as the
 * product path.  Plain C, single-threaded, fp32 arithmetic in the order the reference
 * kernel uses.
 *
 * Functions and the reference code they restate (ahmed123hds/persistentkv-attention):
 *   pkv_oracle_paged_row_offset  kernels/persistentkv_attention.cuh:191-199 (paged index)
 *   pkv_oracle_split_partial     cuh:330-363 (row-local split bounds, empty-split neutral
 *                                state) and :398-632 (32-token online softmax, partial
 *                                (m, l, acc) in natural-log units of the scaled score)
 *   pkv_oracle_lse_merge         cuh:719-751 / :753-784 (max, rescale, sum, O = A / L)
 *   pkv_oracle_paged_decode      cuh:929-974 (split grid + merge) for one query row
 *   pkv_oracle_cpu_gqa_attention tests/smoke_test.cu:35-74 (exact fp32 reference with
 *                                the +1e-8 denominator guard)
 *   pkv_oracle_smoke_inputs      tests/smoke_test.cu:77-81, :438, :486-493 (glibc
 *                                srand(42)/rand() inputs of the eight smoke cases)
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define PKV_D 128
#define PKV_TILE 32

/* Element offset of (token, dim 0) of KV head kvh in a [pages, Hkv, ps, D] pool. */
int64_t pkv_oracle_paged_row_offset(const int32_t* table_row, int32_t token, int32_t kvh,
                                    int32_t num_kv_heads, int32_t page_size) {
  const int32_t logical = token / page_size;
  const int32_t in_page = token - logical * page_size;
  const int64_t physical = table_row[logical];
  return ((physical * num_kv_heads + kvh) * page_size + in_page) * PKV_D;
}

/* Partial state of one (row, query head, split) over tiles [tile_begin, tile_end) of a
 * row with `length` tokens.  K and V are fp32 copies of the paged pool.  Writes
 * m (natural-log units of score*scale), l and acc[128]. */
void pkv_oracle_split_partial(const float* q_head, const float* k_pool, const float* v_pool,
                              const int32_t* table_row, int32_t num_kv_heads, int32_t page_size,
                              int32_t kvh, int32_t length, int32_t tile_begin, int32_t tile_end,
                              float* out_m, float* out_l, float* out_acc) {
  const float scale = 1.0f / sqrtf((float)PKV_D);
  float m = -FLT_MAX, l = 0.0f;
  float acc[PKV_D];
  memset(acc, 0, sizeof(acc));
  for (int32_t tile = tile_begin; tile < tile_end; ++tile) {
    const int32_t t0 = tile * PKV_TILE;
    int32_t tile_size = length - t0;
    if (tile_size > PKV_TILE) tile_size = PKV_TILE;
    if (tile_size <= 0) break;
    float score[PKV_TILE];
    float tile_m = -FLT_MAX;
    for (int32_t t = 0; t < tile_size; ++t) {
      const float* k = k_pool + pkv_oracle_paged_row_offset(table_row, t0 + t, kvh, num_kv_heads, page_size);
      float s = 0.0f;
      for (int d = 0; d < PKV_D; ++d) s = fmaf(q_head[d], k[d], s);
      score[t] = s * scale;
      if (score[t] > tile_m) tile_m = score[t];
    }
    const float new_m = m > tile_m ? m : tile_m;
    const float corr = expf(m - new_m);
    float tile_l = 0.0f;
    float tile_acc[PKV_D];
    memset(tile_acc, 0, sizeof(tile_acc));
    for (int32_t t = 0; t < tile_size; ++t) {
      const float w = expf(score[t] - new_m);
      tile_l += w;
      const float* v = v_pool + pkv_oracle_paged_row_offset(table_row, t0 + t, kvh, num_kv_heads, page_size);
      for (int d = 0; d < PKV_D; ++d) tile_acc[d] = fmaf(w, v[d], tile_acc[d]);
    }
    l = corr * l + tile_l;
    for (int d = 0; d < PKV_D; ++d) acc[d] = corr * acc[d] + tile_acc[d];
    m = new_m;
  }
  *out_m = m;
  *out_l = l;
  memcpy(out_acc, acc, sizeof(acc));
}

/* LSE merge of n partial states; writes the normalised output (0 when L == 0). */
void pkv_oracle_lse_merge(const float* m, const float* l, const float* acc, int32_t n,
                          float* out) {
  float M = -FLT_MAX;
  for (int32_t s = 0; s < n; ++s) M = m[s] > M ? m[s] : M;
  float L = 0.0f;
  float A[PKV_D];
  memset(A, 0, sizeof(A));
  for (int32_t s = 0; s < n; ++s) {
    const float c = expf(m[s] - M);
    L += c * l[s];
    for (int d = 0; d < PKV_D; ++d) A[d] += c * acc[(int64_t)s * PKV_D + d];
  }
  for (int d = 0; d < PKV_D; ++d) out[d] = L > 0.0f ? A[d] / L : 0.0f;
}

/* One query row of the paged decode with `num_splits` row-local splits (1 = direct).
 * q_row is [Hq, 128]; out is [Hq, 128]. */
void pkv_oracle_paged_decode(const float* q_row, const float* k_pool, const float* v_pool,
                             const int32_t* table_row, int32_t num_q_heads, int32_t num_kv_heads,
                             int32_t page_size, int32_t length, int32_t num_splits, float* out) {
  const int32_t G = num_q_heads / num_kv_heads;
  const int32_t total_tiles = (length + PKV_TILE - 1) / PKV_TILE;
  float* m = (float*)malloc(sizeof(float) * (size_t)num_splits);
  float* l = (float*)malloc(sizeof(float) * (size_t)num_splits);
  float* acc = (float*)malloc(sizeof(float) * (size_t)num_splits * PKV_D);
  for (int32_t qh = 0; qh < num_q_heads; ++qh) {
    const int32_t kvh = qh / G;
    for (int32_t s = 0; s < num_splits; ++s) {
      const int32_t tb = (int32_t)(((int64_t)total_tiles * s) / num_splits);
      const int32_t te = (int32_t)(((int64_t)total_tiles * (s + 1)) / num_splits);
      pkv_oracle_split_partial(q_row + (int64_t)qh * PKV_D, k_pool, v_pool, table_row, num_kv_heads,
                               page_size, kvh, length, tb, te, &m[s], &l[s], acc + (int64_t)s * PKV_D);
    }
    pkv_oracle_lse_merge(m, l, acc, num_splits, out + (int64_t)qh * PKV_D);
  }
  free(m);
  free(l);
  free(acc);
}

/* tests/smoke_test.cu:35-74, contiguous K/V [B, Hkv, N, d]. */
void pkv_oracle_cpu_gqa_attention(const float* Q, const float* K, const float* V, float* O,
                                  int B, int Hq, int Hkv, int N, int d) {
  const int G = Hq / Hkv;
  const float scale = 1.0f / sqrtf((float)d);
  float* scores = (float*)malloc(sizeof(float) * (size_t)N);
  for (int b = 0; b < B; b++) {
    for (int qh = 0; qh < Hq; qh++) {
      const int kvh = qh / G;
      const float* q = Q + (int64_t)b * Hq * d + (int64_t)qh * d;
      const float* Kh = K + (int64_t)b * Hkv * N * d + (int64_t)kvh * N * d;
      const float* Vh = V + (int64_t)b * Hkv * N * d + (int64_t)kvh * N * d;
      float* o = O + (int64_t)b * Hq * d + (int64_t)qh * d;
      float m = -FLT_MAX, l = 0.f;
      for (int t = 0; t < N; t++) {
        float s = 0.f;
        for (int dd = 0; dd < d; dd++) s += q[dd] * Kh[(int64_t)t * d + dd];
        s *= scale;
        scores[t] = s;
        m = fmaxf(m, s);
      }
      memset(o, 0, sizeof(float) * (size_t)d);
      for (int t = 0; t < N; t++) {
        const float w = expf(scores[t] - m);
        l += w;
        for (int dd = 0; dd < d; dd++) o[dd] += w * Vh[(int64_t)t * d + dd];
      }
      for (int dd = 0; dd < d; dd++) o[dd] /= (l + 1e-8f);
    }
  }
  free(scores);
}

/* The eight correctness cases of tests/smoke_test.cu:486-493, in order:
 * {B, Hq, Hkv, N, splits, page_size (0 = contiguous)}. */
static const int kSmokeCases[8][6] = {
    {1, 4, 1, 257, 1, 0},  {1, 8, 2, 257, 4, 0},  {1, 32, 8, 512, 4, 0}, {2, 32, 8, 259, 3, 0},
    {1, 32, 4, 511, 4, 0}, {1, 8, 8, 256, 2, 0},  {1, 8, 2, 257, 4, 16}, {2, 8, 2, 259, 3, 32}};

int pkv_oracle_smoke_case(int index, int* shape6) {
  if (index < 0 || index >= 8) return -1;
  memcpy(shape6, kSmokeCases[index], sizeof(int) * 6);
  return 0;
}

static float smoke_rand(void) { return (float)rand() / RAND_MAX * 2.0f - 1.0f; } /* :77 */

/* Fills Q [B,Hq,128], K and V [B,Hkv,N,128] with the values smoke_test draws for case
 * `index` after srand(42): every earlier case consumes Q, K, V in that order (:119-121,
 * :228-230).  Values are returned as drawn (before the fp16 quantisation). */
int pkv_oracle_smoke_inputs(int index, float* q, float* k, float* v) {
  if (index < 0 || index >= 8) return -1;
  srand(42);
  for (int c = 0; c <= index; ++c) {
    const int* s = kSmokeCases[c];
    const int64_t qn = (int64_t)s[0] * s[1] * PKV_D, kvn = (int64_t)s[0] * s[2] * s[3] * PKV_D;
    for (int64_t i = 0; i < qn; ++i) { const float x = smoke_rand(); if (c == index) q[i] = x; }
    for (int64_t i = 0; i < kvn; ++i) { const float x = smoke_rand(); if (c == index) k[i] = x; }
    for (int64_t i = 0; i < kvn; ++i) { const float x = smoke_rand(); if (c == index) v[i] = x; }
  }
  return 0;
}

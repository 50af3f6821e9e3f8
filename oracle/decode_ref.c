/*
 * decode_ref.c -- CPU oracle for the paged decode path, TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's CPU baseline may load
 * this library, and only as the checker. The product path never calls it.
 *
 * Functions:
 *   oracle_paged_decode_f64    fp64 attention over a paged cache: the textbook
 *                              softmax(q K^T * scale) V per (sequence, query head),
 *                              gathering token t of sequence b from page
 *                              block_table[b, t / PS], row t % PS; query head h
 *                              reads kv head h / (HQ / HKV). Follows
 *                              mxflashattn/reference.py:88-139 (gather) and
 *                              :8-40 (attention), in the fp64 host style of
 *                              gate1/gate1b.cpp:111-142. A sequence of length 0
 *                              gives zeros (the reference raises instead,
 *                              reference.py:21-22).
 *   oracle_append_kv_u16       block-table append of new rows at positions
 *                              seqlens[b] + t (reference.py:117-122), bitwise.
 *   oracle_reshape_and_cache_u16  slot-mapping append, slot < 0 skipped
 *                              (vLLM reshape_and_cache_flash semantics), bitwise.
 *
 * Element arrays for the fp64 path are float32 copies of the fp16/bf16 inputs
 * (exact widening), laid out densely: q [B,HQ,HD], caches [P,PS,HKV,HD].
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

int oracle_paged_decode_f64(const float *q, const float *k_cache, const float *v_cache,
                            const int32_t *block_table, int btw, const int32_t *seqlens,
                            int B, int HQ, int HKV, int HD, int PS, int P, double scale,
                            double *out) {
  if (B < 0 || HQ <= 0 || HKV <= 0 || HD <= 0 || PS <= 0 || P <= 0 || btw <= 0) return -2;
  if (HQ % HKV != 0) return -1;
  const int gq = HQ / HKV;
  int maxlen = 0;
  for (int b = 0; b < B; ++b) {
    if (seqlens[b] < 0 || seqlens[b] > btw * PS) return -3;
    if (seqlens[b] > maxlen) maxlen = seqlens[b];
  }
  double *score = (double *)malloc(sizeof(double) * (size_t)(maxlen > 0 ? maxlen : 1));
  const float **krow = (const float **)malloc(sizeof(float *) * (size_t)(maxlen > 0 ? maxlen : 1));
  const float **vrow = (const float **)malloc(sizeof(float *) * (size_t)(maxlen > 0 ? maxlen : 1));
  if (!score || !krow || !vrow) {
    free(score);
    free(krow);
    free(vrow);
    return -4;
  }
  for (int b = 0; b < B; ++b) {
    const int L = seqlens[b];
    for (int h = 0; h < HQ; ++h) {
      const int kvh = h / gq;
      double *o = out + ((size_t)b * HQ + h) * HD;
      for (int d = 0; d < HD; ++d) o[d] = 0.0;
      if (L == 0) continue;
      const float *qv = q + ((size_t)b * HQ + h) * HD;
      double mx = -INFINITY;
      for (int t = 0; t < L; ++t) {
        const int page = block_table[(size_t)b * btw + t / PS];
        if (page < 0 || page >= P) {
          free(score);
          free(krow);
          free(vrow);
          return -3;
        }
        const size_t row = (((size_t)page * PS + (size_t)(t % PS)) * HKV + kvh) * HD;
        krow[t] = k_cache + row;
        vrow[t] = v_cache + row;
        double acc = 0.0;
        for (int d = 0; d < HD; ++d) acc += (double)qv[d] * (double)krow[t][d];
        score[t] = acc * scale;
        if (score[t] > mx) mx = score[t];
      }
      double sum = 0.0;
      for (int t = 0; t < L; ++t) {
        score[t] = exp(score[t] - mx);
        sum += score[t];
      }
      for (int t = 0; t < L; ++t) {
        const double w = score[t] / sum;
        for (int d = 0; d < HD; ++d) o[d] += w * (double)vrow[t][d];
      }
    }
  }
  free(score);
  free(krow);
  free(vrow);
  return 0;
}

int oracle_append_kv_u16(const uint16_t *k, const uint16_t *v, uint16_t *k_cache,
                         uint16_t *v_cache, const int32_t *block_table, int btw,
                         const int32_t *seqlens, int B, int S, int HKV, int HD, int PS, int P) {
  const size_t row = (size_t)HKV * HD;
  for (int b = 0; b < B; ++b) {
    for (int t = 0; t < S; ++t) {
      const long pos = (long)seqlens[b] + t;
      if (pos < 0 || pos / PS >= btw) continue;
      const int page = block_table[(size_t)b * btw + pos / PS];
      if (page < 0 || page >= P) continue;
      const size_t dst = ((size_t)page * PS + (size_t)(pos % PS)) * row;
      const size_t src = ((size_t)b * S + t) * row;
      memcpy(k_cache + dst, k + src, row * sizeof(uint16_t));
      memcpy(v_cache + dst, v + src, row * sizeof(uint16_t));
    }
  }
  return 0;
}

int oracle_reshape_and_cache_u16(const uint16_t *key, const uint16_t *value, uint16_t *k_cache,
                                 uint16_t *v_cache, const int64_t *slots, int T, int HKV,
                                 int HD, int PS, int P) {
  const size_t row = (size_t)HKV * HD;
  for (int t = 0; t < T; ++t) {
    const int64_t slot = slots[t];
    if (slot < 0) continue;
    const int64_t page = slot / PS;
    if (page >= P) continue;
    const size_t dst = ((size_t)page * PS + (size_t)(slot % PS)) * row;
    memcpy(k_cache + dst, key + (size_t)t * row, row * sizeof(uint16_t));
    memcpy(v_cache + dst, value + (size_t)t * row, row * sizeof(uint16_t));
  }
  return 0;
}

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
 *   oracle_e4m3fn_decode       OCP fp8 e4m3fn bytes to float32 (exact): bias 7,
 *                              subnormals m/8 * 2^-6, S.1111.111 = NaN, no inf.
 *   oracle_e4m3fn_encode       float32 to e4m3fn: saturate to +-448 (inf too),
 *                              round to nearest even, NaN -> S.1111.111.
 *   oracle_reshape_and_cache_fp8  slot-mapping append into an fp8 cache:
 *                              e4m3fn(x / scale), x widened exactly from fp16 or
 *                              bf16, the division in fp32 (IEEE, correctly
 *                              rounded). No reference counterpart (the
 *                              reference has no fp8 cache); the fp8 semantics
 *                              follow the OCP 8-bit floating point spec and
 *                              vLLM's saturating cache conversion.
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

/* ---- fp8 (OCP e4m3fn) ---------------------------------------------------- */

static float f16_bits_to_f32(uint16_t h) {
  const int sign = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(1024 + m), e - 25);
  return sign ? -v : v;
}

static float bf16_bits_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float e4m3fn_to_f32(uint8_t c) {
  const int sign = c >> 7, e = (c >> 3) & 15, m = c & 7;
  float v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf((float)(8 + m), e - 10);
  return sign ? -v : v;
}

static uint8_t f32_to_e4m3fn(float x) {
  if (x != x) return (uint8_t)(signbit(x) ? 0xff : 0x7f);
  const uint8_t sign = signbit(x) ? 0x80 : 0;
  const double a = fabs((double)x);
  if (a >= 448.0) return sign | 0x7e;
  if (a < ldexp(1.0, -6)) { /* subnormal: units of 2^-9, 8 units = 2^-6 */
    const double q = nearbyint(a * 512.0);
    return sign | (uint8_t)q;
  }
  int e;
  frexp(a, &e); /* a = f * 2^e, f in [0.5, 1) */
  e -= 1;       /* a = g * 2^e, g in [1, 2) */
  double r = nearbyint(ldexp(a, -e) * 8.0); /* in [8, 16] */
  if (r >= 16.0) {
    r = 8.0;
    e += 1;
  }
  return sign | (uint8_t)(((e + 7) << 3) | ((int)r - 8));
}

int oracle_e4m3fn_decode(const uint8_t *in, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = e4m3fn_to_f32(in[i]);
  return 0;
}

int oracle_e4m3fn_encode(const float *in, uint8_t *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = f32_to_e4m3fn(in[i]);
  return 0;
}

int oracle_reshape_and_cache_fp8(const uint16_t *key, const uint16_t *value, int is_bf16,
                                 float k_scale, float v_scale, uint8_t *k_cache,
                                 uint8_t *v_cache, const int64_t *slots, int T, int HKV, int HD,
                                 int PS, int P) {
  const size_t row = (size_t)HKV * HD;
  for (int t = 0; t < T; ++t) {
    const int64_t slot = slots[t];
    if (slot < 0) continue;
    const int64_t page = slot / PS;
    if (page >= P) continue;
    const size_t dst = ((size_t)page * PS + (size_t)(slot % PS)) * row;
    for (size_t i = 0; i < row; ++i) {
      const uint16_t kb = key[(size_t)t * row + i], vb = value[(size_t)t * row + i];
      const float kx = is_bf16 ? bf16_bits_to_f32(kb) : f16_bits_to_f32(kb);
      const float vx = is_bf16 ? bf16_bits_to_f32(vb) : f16_bits_to_f32(vb);
      volatile float kq = kx / k_scale, vq = vx / v_scale; /* fp32 division */
      k_cache[dst + i] = f32_to_e4m3fn(kq);
      v_cache[dst + i] = f32_to_e4m3fn(vq);
    }
  }
  return 0;
}

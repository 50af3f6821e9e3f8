// Split-KV paged decode attention for MI355X (gfx950, wave64).
//
// Partial kernel: one workgroup per (kv head, split, sequence). A split covers
// chunk_len consecutive token positions of one sequence. Four waves share the
// split; each wave streams its own tiles of TT tokens straight from HBM into
// VGPRs with 128-bit loads (LPR = HD/8 lanes per 256/128-byte token row, so a
// wave load covers 4 (HD128) or 8 (HD64) whole rows), keeps an online softmax
// per 16-lane row and merges rows and waves once at the end. The page id of
// each token is looked up in the block table one tile ahead of its K/V loads,
// and the K/V loads of tile i+1 are in flight while tile i is computed.
//
// Softmax runs in the base-2 domain: x = q.k * scale * log2(e) - m, p = 2^x.
// The reference m of a row only moves when a score exceeds it by more than
// kRescaleLog2 (so p <= 2^kRescaleLog2), which keeps the rescale branch rare.
//
// Workspace (num_splits > 1), fp32:
//   ws_o  [B, HQ, NS, HD]  normalised partial output of each split
//   ws_lse[B, HQ, NS]      base-2 log-sum-exp of each split (-inf when empty)
// Only splits s < ceil(L_b / chunk_len) are written; the combine reads no more.
// With num_splits == 1 the partial kernel writes the final output directly.
//
// Reference counterpart: paged_decode_v3 split mode and split_combine
// (csrc_native/m1_kernel.cpp:553-888); the algorithm (split partials + LSE
// merge) is the same, the data path and numerics are this file's own.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "mxfa_device.h"
#include "mxfa_mi355x.h"

namespace mxfa {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleLog2 = 8.0f;

struct DecodeParams {
  const uint16_t *q;
  int64_t q_sb, q_sh;
  const uint16_t *k;
  const uint16_t *v;
  int64_t c_sp, c_st, c_sh;
  const int32_t *bt;
  int64_t bt_stride;
  const int32_t *seqlens;
  uint16_t *out;
  int64_t o_sb, o_sh;
  float *ws_o;
  float *ws_lse;
  float scale_log2;
  int seqlen_add;
  int hq;
  int ps_log2;
  int max_len;  // block_table_width * page_size
  int num_pages;
  int num_splits;
  int chunk_len;
};

struct CombineParams {
  const float *ws_o;
  const float *ws_lse;
  const int32_t *seqlens;
  uint16_t *out;
  int64_t o_sb, o_sh;
  int seqlen_add;
  int batch;
  int hq;
  int max_len;
  int num_splits;
  int chunk_len;
};

__device__ __forceinline__ int seq_len_of(const int32_t *seqlens, int b, int add, int max_len) {
  int L = seqlens[b] + add;
  L = L < 0 ? 0 : L;
  return L > max_len ? max_len : L;
}

// Scores of the U x GQ (token row, head) pairs of one wave load group: dot
// products of the 8-element fragments, then the LPR-lane row sums. The steps
// run across all pairs so consecutive DPP ops touch independent registers.
template <int U, int GQ, int LPR, typename T>
__device__ __forceinline__ void tile_scores(const uint4 (&kr)[U], const uint32_t (&qv)[GQ][4],
                                            float (&s)[U][GQ]) {
  using E = Elem<T>;
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int g = 0; g < GQ; ++g) s[u][g] = E::dot2(kr[u].x, qv[g][0], 0.f);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int g = 0; g < GQ; ++g) s[u][g] = E::dot2(kr[u].y, qv[g][1], s[u][g]);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int g = 0; g < GQ; ++g) s[u][g] = E::dot2(kr[u].z, qv[g][2], s[u][g]);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int g = 0; g < GQ; ++g) s[u][g] = E::dot2(kr[u].w, qv[g][3], s[u][g]);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int g = 0; g < GQ; ++g) s[u][g] += dpp_f<kDppQuadXor1>(s[u][g]);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int g = 0; g < GQ; ++g) s[u][g] += dpp_f<kDppQuadXor2>(s[u][g]);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int g = 0; g < GQ; ++g) s[u][g] += dpp_f<kDppRowHalfMirror>(s[u][g]);
  if constexpr (LPR == 16) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int g = 0; g < GQ; ++g) s[u][g] += dpp_f<kDppRowMirror>(s[u][g]);
  }
}

// kLanePages: the block-table lookup is done per lane (page size smaller than
// the RPW rows of one wave load). Otherwise the RPW rows of each load lie in
// one page, so each load needs one wave-uniform (scalar) lookup.
template <int HD, int GQ, typename T, bool kLanePages>
__global__ __launch_bounds__(kThreads) void split_partial_kernel(DecodeParams p) {
  using E = Elem<T>;
  constexpr int LPR = HD / 8;    // lanes per token row (16 B per lane)
  constexpr int RPW = 64 / LPR;  // token rows per wave load
  constexpr int U = 4;           // loads per tile per tensor
  constexpr int TT = U * RPW;    // tokens per wave tile

  const int kvh = blockIdx.x;
  const int split = blockIdx.y;
  const int b = blockIdx.z;
  const int L = seq_len_of(p.seqlens, b, p.seqlen_add, p.max_len);
  const int c_start = split * p.chunk_len;
  int sl = L - c_start;
  sl = sl > p.chunk_len ? p.chunk_len : sl;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = lane / LPR;
  const int col = lane % LPR;
  const int h0 = kvh * GQ;
  const bool direct = p.num_splits == 1;

  if (sl <= 0) {
    // Empty split. In direct mode split 0 of an empty sequence owns the zero output.
    if (direct) {
      for (int idx = threadIdx.x; idx < GQ * HD; idx += kThreads) {
        const int g = idx / HD, dim = idx % HD;
        p.out[b * p.o_sb + (int64_t)(h0 + g) * p.o_sh + dim] = 0;
      }
    }
    return;
  }

  // Query fragment of every head of this group: 8 elements per lane.
  uint32_t qv[GQ][4];
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    const uint4 t = *reinterpret_cast<const uint4 *>(p.q + b * p.q_sb + (int64_t)(h0 + g) * p.q_sh +
                                                      col * 8);
    qv[g][0] = t.x;
    qv[g][1] = t.y;
    qv[g][2] = t.z;
    qv[g][3] = t.w;
  }

  float m[GQ], d[GQ], o[GQ][8];
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    m[g] = -INFINITY;
    d[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[g][i] = 0.f;
  }

  const int32_t *__restrict__ btrow = p.bt + (int64_t)b * p.bt_stride;
  const char *__restrict__ kbase = reinterpret_cast<const char *>(p.k);
  const char *__restrict__ vbase = reinterpret_cast<const char *>(p.v);
  const int ps_mask = (1 << p.ps_log2) - 1;
  const uint32_t st_bytes = (uint32_t)p.c_st * 2u;
  const uint64_t sp_bytes = (uint64_t)p.c_sp * 2u;
  const uint32_t lane_bytes = (uint32_t)kvh * ((uint32_t)p.c_sh * 2u) + (uint32_t)col * 16u;
  const int ntiles = (sl + TT - 1) / TT;
  const float c = p.scale_log2;

  auto clamp_page = [&](int pg) -> int {
    pg = pg < 0 ? 0 : pg;
    return pg >= p.num_pages ? p.num_pages - 1 : pg;
  };
  // Position of this lane's row in load u of a tile, clamped to the last valid
  // token so every address is a real row of this sequence.
  auto lane_pos = [&](int tile, int u) -> int {
    int t = tile * TT + u * RPW + row;
    t = t < sl ? t : sl - 1;
    return c_start + t;
  };

  int pg_a[U], pg_b[U];  // raw block-table entries (clamped at use)
  uint4 ka[U], va[U], kb[U], vb[U];

  // Loads are issued unconditionally (also for the tile after the wave's last
  // one): positions clamp to the last valid token, so the extra loads hit the
  // cache lines of that row, and the straight-line code lets the compiler wait
  // for exactly the tile being computed.
  auto load_pages = [&](int tile, int (&pg)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (kLanePages) {
        pg[u] = btrow[lane_pos(tile, u) >> p.ps_log2];
      } else {
        int t = tile * TT + u * RPW;
        t = t < sl ? t : sl - 1;
        pg[u] = btrow[__builtin_amdgcn_readfirstlane((c_start + t) >> p.ps_log2)];
      }
    }
  };
  auto load_kv = [&](int tile, const int (&pg)[U], uint4 (&kr)[U], uint4 (&vr)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t off = (uint32_t)(lane_pos(tile, u) & ps_mask) * st_bytes + lane_bytes;
      const uint64_t page_off = (uint64_t)(uint32_t)clamp_page(pg[u]) * sp_bytes;
      kr[u] = *reinterpret_cast<const uint4 *>(kbase + page_off + off);
      vr[u] = *reinterpret_cast<const uint4 *>(vbase + page_off + off);
    }
  };
  // Scalar page ids (SMEM, returns out of order) are fetched after the K/V
  // loads that need the previous ids; per-lane ids (VMEM, in order) before
  // them, so that waiting for an id never waits for K/V data.
  auto advance = [&](int tile, const int (&pg_next)[U], int (&pg_after)[U], uint4 (&kr)[U],
                     uint4 (&vr)[U]) {
    if constexpr (kLanePages) {
      load_pages(tile + 2 * kWaves, pg_after);
      load_kv(tile + kWaves, pg_next, kr, vr);
    } else {
      load_kv(tile + kWaves, pg_next, kr, vr);
      load_pages(tile + 2 * kWaves, pg_after);
    }
  };
  auto compute = [&](int tile, const uint4 (&kr)[U], const uint4 (&vr)[U]) {
    float s[U][GQ];
    tile_scores<U, GQ, LPR, T>(kr, qv, s);
    // Scaled scores (base 2); rows past the end of the split get -inf.
    float mt[GQ];
#pragma unroll
    for (int g = 0; g < GQ; ++g) mt[g] = -INFINITY;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool valid = tile * TT + u * RPW + row < sl;
#pragma unroll
      for (int g = 0; g < GQ; ++g) {
        const float sc = valid ? s[u][g] * c : -INFINITY;
        s[u][g] = sc;
        mt[g] = fmaxf(mt[g], sc);
      }
    }
    bool need = false;
#pragma unroll
    for (int g = 0; g < GQ; ++g) need |= mt[g] > m[g] + kRescaleLog2;
    if (need) {
      // Rare: a score passed the row's reference by more than kRescaleLog2.
      // Move the reference to the tile maximum and rescale the accumulators
      // (m = -inf: nothing accumulated yet, the factor is 0).
#pragma unroll
      for (int g = 0; g < GQ; ++g) {
        if (mt[g] > m[g] + kRescaleLog2) {
          const float f = fast_exp2(m[g] - mt[g]);
          d[g] *= f;
#pragma unroll
          for (int i = 0; i < 8; ++i) o[g][i] *= f;
          m[g] = mt[g];
        }
      }
    }
    // m = -inf here means this row has seen no valid token, so every score of
    // the row in this tile is -inf as well; a zero reference keeps 2^x = 0.
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      const float mr = m[g] == -INFINITY ? 0.f : m[g];
#pragma unroll
      for (int u = 0; u < U; ++u) s[u][g] = fast_exp2(s[u][g] - mr);
    }
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      float acc = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u) acc += s[u][g];
      d[g] += acc;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float vf[8];
      vf[0] = E::lo(vr[u].x);
      vf[1] = E::hi(vr[u].x);
      vf[2] = E::lo(vr[u].y);
      vf[3] = E::hi(vr[u].y);
      vf[4] = E::lo(vr[u].z);
      vf[5] = E::hi(vr[u].z);
      vf[6] = E::lo(vr[u].w);
      vf[7] = E::hi(vr[u].w);
#pragma unroll
      for (int g = 0; g < GQ; ++g) {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[g][i] = fmaf(s[u][g], vf[i], o[g][i]);
      }
    }
  };

  // Software pipeline over this wave's tiles: wave, wave + kWaves, ...
  // Page ids run two tiles ahead of the math and K/V loads one tile ahead; two
  // register sets (a/b) alternate so no copies are needed. The loop body runs
  // two tiles and exits only at its latch, so the loads crossing the back edge
  // are always the a-set of the next tile and the compiler never has to drain
  // the load queue at the loop head.
  const int ntw = wave < ntiles ? (ntiles - wave + kWaves - 1) / kWaves : 0;
  if (ntw > 0) {
    int tile = wave;
    load_pages(tile, pg_a);
    load_kv(tile, pg_a, ka, va);
    load_pages(tile + kWaves, pg_b);
    for (int i = 0; i + 1 < ntw; i += 2) {
      advance(tile, pg_b, pg_a, kb, vb);
      compute(tile, ka, va);
      tile += kWaves;
      advance(tile, pg_a, pg_b, ka, va);
      compute(tile, kb, vb);
      tile += kWaves;
    }
    if (ntw & 1) compute(tile, ka, va);
  }

  // Merge the RPW token rows of the wave (rows sit LPR lanes apart).
  __shared__ float sm_m[kWaves][GQ];
  __shared__ float sm_d[kWaves][GQ];
  __shared__ float sm_o[kWaves][GQ][HD];
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    float M = m[g];
#pragma unroll
    for (int mask = LPR; mask < 64; mask <<= 1) M = fmaxf(M, xor_shfl(M, mask));
    const float f = (m[g] == -INFINITY) ? 0.f : fast_exp2(m[g] - M);
    float dd = d[g] * f;
    float oo[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) oo[i] = o[g][i] * f;
#pragma unroll
    for (int mask = LPR; mask < 64; mask <<= 1) {
      dd += xor_shfl(dd, mask);
#pragma unroll
      for (int i = 0; i < 8; ++i) oo[i] += xor_shfl(oo[i], mask);
    }
    if (row == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) sm_o[wave][g][col * 8 + i] = oo[i];
      if (col == 0) {
        sm_m[wave][g] = M;
        sm_d[wave][g] = dd;
      }
    }
  }
  __syncthreads();

  // Merge the waves and write either the final output or the split partial.
  for (int idx = threadIdx.x; idx < GQ * HD; idx += kThreads) {
    const int g = idx / HD, dim = idx % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][g]);
    float D = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = sm_m[w][g];
      const float f = (mw == -INFINITY) ? 0.f : fast_exp2(mw - M);
      D = fmaf(sm_d[w][g], f, D);
      O = fmaf(sm_o[w][g][dim], f, O);
    }
    const float r = D > 0.f ? O / D : 0.f;
    const int h = h0 + g;
    if (direct) {
      p.out[b * p.o_sb + (int64_t)h * p.o_sh + dim] = E::narrow(r);
    } else {
      const int64_t slot = ((int64_t)b * p.hq + h) * p.num_splits + split;
      p.ws_o[slot * HD + dim] = r;
      if (dim == 0) p.ws_lse[slot] = D > 0.f ? M + __log2f(D) : -INFINITY;
    }
  }
}

// LSE combine: HD/4 threads per (sequence, head), float4 per thread.
template <int HD, typename T>
__global__ __launch_bounds__(256) void split_combine_kernel(CombineParams p) {
  using E = Elem<T>;
  constexpr int TPH = HD / 4;
  constexpr int HPB = 256 / TPH;
  const int hid = blockIdx.x * HPB + threadIdx.x / TPH;
  if (hid >= p.batch * p.hq) return;
  const int t = threadIdx.x % TPH;
  const int b = hid / p.hq, h = hid % p.hq;
  const int L = seq_len_of(p.seqlens, b, p.seqlen_add, p.max_len);
  int ns = (L + p.chunk_len - 1) / p.chunk_len;
  ns = ns > p.num_splits ? p.num_splits : ns;

  const float *lse = p.ws_lse + (int64_t)hid * p.num_splits;
  const float4 *po = reinterpret_cast<const float4 *>(p.ws_o + (int64_t)hid * p.num_splits * HD) + t;
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, lse[s]);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float wsum = 0.f;
  if (M != -INFINITY) {
#pragma unroll 4
    for (int s = 0; s < ns; ++s) {
      const float l = lse[s];
      const float w = (l == -INFINITY) ? 0.f : fast_exp2(l - M);
      const float4 v = po[s * TPH];
      acc.x = fmaf(w, v.x, acc.x);
      acc.y = fmaf(w, v.y, acc.y);
      acc.z = fmaf(w, v.z, acc.z);
      acc.w = fmaf(w, v.w, acc.w);
      wsum += w;
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  uint16_t r[4] = {E::narrow(acc.x * inv), E::narrow(acc.y * inv), E::narrow(acc.z * inv),
                   E::narrow(acc.w * inv)};
  uint2 packed;
  packed.x = (uint32_t)r[0] | ((uint32_t)r[1] << 16);
  packed.y = (uint32_t)r[2] | ((uint32_t)r[3] << 16);
  *reinterpret_cast<uint2 *>(p.out + b * p.o_sb + (int64_t)h * p.o_sh + t * 4) = packed;
}

// ---------------------------------------------------------------------------
// Host side: argument checks, template selection, launches.

static bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15u) == 0; }

static int ilog2_exact(int v) {
  if (v <= 0 || (v & (v - 1)) != 0) return -1;
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}

struct SplitArgs {
  const void *q;
  int64_t q_sb, q_sh;
  const void *k, *v;
  int64_t c_sp, c_st, c_sh;
  const int32_t *bt;
  int64_t bt_stride;
  const int32_t *seqlens;
  int seqlen_add;
  void *out;
  int64_t o_sb, o_sh;
  void *ws;
  size_t ws_bytes;
  float scale;
  int batch, hq, hkv, hd, ps, btw, num_pages, dtype, num_splits, chunk_len;
};

static size_t workspace_bytes(int batch, int hq, int hd, int ns) {
  if (ns <= 1) return 0;
  const size_t slots = (size_t)batch * hq * ns;
  return slots * hd * sizeof(float) + slots * sizeof(float);
}

static int check_split_args(const SplitArgs &a, bool need_out, bool need_ws) {
  if (!a.q || !a.k || !a.v || !a.bt || !a.seqlens) return MXFA_EINVAL;
  if (need_out && !a.out) return MXFA_EINVAL;
  if (a.batch <= 0 || a.hq <= 0 || a.hkv <= 0 || a.btw <= 0 || a.num_pages <= 0)
    return MXFA_EINVAL;
  if (a.num_splits <= 0 || a.chunk_len <= 0 || a.seqlen_add < 0) return MXFA_EINVAL;
  if (!(a.scale == a.scale) || a.scale == INFINITY || a.scale == -INFINITY) return MXFA_EINVAL;
  if (a.hd != 64 && a.hd != 128) return MXFA_EUNSUPPORTED;
  if (a.hq % a.hkv != 0) return MXFA_EUNSUPPORTED;
  const int gq = a.hq / a.hkv;
  if (gq != 2 && gq != 4 && gq != 8) return MXFA_EUNSUPPORTED;
  if (a.dtype != MXFA_DTYPE_F16 && a.dtype != MXFA_DTYPE_BF16) return MXFA_EUNSUPPORTED;
  if (ilog2_exact(a.ps) < 0 || a.ps > 4096) return MXFA_EUNSUPPORTED;
  if (a.num_splits > 65535 || a.batch > 65535) return MXFA_EUNSUPPORTED;
  const int64_t max_len = (int64_t)a.btw * a.ps;
  if (max_len > (int64_t)1 << 30) return MXFA_EUNSUPPORTED;
  if ((int64_t)a.num_splits * a.chunk_len < max_len) return MXFA_EINVAL;
  // 16-byte fragments: pointers and every stride must keep 8-element alignment.
  if (!aligned16(a.q) || !aligned16(a.k) || !aligned16(a.v)) return MXFA_EINVAL;
  if (need_out && ((uintptr_t)a.out & 7u)) return MXFA_EINVAL;
  if ((a.q_sb | a.q_sh | a.c_sp | a.c_st | a.c_sh) & 7) return MXFA_EINVAL;
  // In-page byte offsets are 32-bit: (PS-1)*token + (HKV-1)*head + HD elements.
  if (((int64_t)(a.ps - 1) * a.c_st + (int64_t)(a.hkv - 1) * a.c_sh + a.hd) * 2 >=
      ((int64_t)1 << 32))
    return MXFA_EUNSUPPORTED;
  if (a.q_sb < 0 || a.q_sh < 0 || a.c_sp < 0 || a.c_st < 0 || a.c_sh < 0 || a.bt_stride < 0)
    return MXFA_EINVAL;
  if (need_out && ((a.o_sb | a.o_sh) & 3)) return MXFA_EINVAL;
  if (need_ws && a.num_splits > 1) {
    if (!a.ws || !aligned16(a.ws)) return MXFA_EWORKSPACE;
    if (a.ws_bytes < workspace_bytes(a.batch, a.hq, a.hd, a.num_splits)) return MXFA_EWORKSPACE;
  }
  return MXFA_OK;
}

static DecodeParams make_params(const SplitArgs &a) {
  DecodeParams p;
  p.q = (const uint16_t *)a.q;
  p.q_sb = a.q_sb;
  p.q_sh = a.q_sh;
  p.k = (const uint16_t *)a.k;
  p.v = (const uint16_t *)a.v;
  p.c_sp = a.c_sp;
  p.c_st = a.c_st;
  p.c_sh = a.c_sh;
  p.bt = a.bt;
  p.bt_stride = a.bt_stride;
  p.seqlens = a.seqlens;
  p.out = (uint16_t *)a.out;
  p.o_sb = a.o_sb;
  p.o_sh = a.o_sh;
  const size_t slots = (size_t)a.batch * a.hq * a.num_splits;
  p.ws_o = a.num_splits > 1 ? (float *)a.ws : nullptr;
  p.ws_lse = a.num_splits > 1 ? (float *)a.ws + slots * a.hd : nullptr;
  p.scale_log2 = a.scale * kLog2e;
  p.seqlen_add = a.seqlen_add;
  p.hq = a.hq;
  p.ps_log2 = ilog2_exact(a.ps);
  p.max_len = a.btw * a.ps;
  p.num_pages = a.num_pages;
  p.num_splits = a.num_splits;
  p.chunk_len = a.chunk_len;
  return p;
}

template <int HD, int GQ, typename T>
static int launch_partial_t(const DecodeParams &p, int hkv, int batch, hipStream_t st) {
  constexpr int RPW = 64 / (HD / 8);
  dim3 grid(hkv, p.num_splits, batch);
  if ((1 << p.ps_log2) >= RPW)
    hipLaunchKernelGGL((split_partial_kernel<HD, GQ, T, false>), grid, dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL((split_partial_kernel<HD, GQ, T, true>), grid, dim3(kThreads), 0, st, p);
  return hipGetLastError() == hipSuccess ? MXFA_OK : MXFA_ELAUNCH;
}

template <int HD, typename T>
static int launch_partial_gq(const DecodeParams &p, int gq, int hkv, int batch, hipStream_t st) {
  switch (gq) {
    case 2: return launch_partial_t<HD, 2, T>(p, hkv, batch, st);
    case 4: return launch_partial_t<HD, 4, T>(p, hkv, batch, st);
    case 8: return launch_partial_t<HD, 8, T>(p, hkv, batch, st);
  }
  return MXFA_EUNSUPPORTED;
}

static int launch_partial(const SplitArgs &a, hipStream_t st) {
  const DecodeParams p = make_params(a);
  const int gq = a.hq / a.hkv;
  if (a.dtype == MXFA_DTYPE_BF16) {
    return a.hd == 128 ? launch_partial_gq<128, BF16>(p, gq, a.hkv, a.batch, st)
                       : launch_partial_gq<64, BF16>(p, gq, a.hkv, a.batch, st);
  }
  return a.hd == 128 ? launch_partial_gq<128, F16>(p, gq, a.hkv, a.batch, st)
                     : launch_partial_gq<64, F16>(p, gq, a.hkv, a.batch, st);
}

template <int HD, typename T>
static int launch_combine_t(const CombineParams &c, hipStream_t st) {
  constexpr int HPB = 256 / (HD / 4);
  const int heads = c.batch * c.hq;
  dim3 grid((heads + HPB - 1) / HPB);
  hipLaunchKernelGGL((split_combine_kernel<HD, T>), grid, dim3(256), 0, st, c);
  return hipGetLastError() == hipSuccess ? MXFA_OK : MXFA_ELAUNCH;
}

static int launch_combine(const float *ws, const int32_t *seqlens, int seqlen_add, void *out,
                          int64_t o_sb, int64_t o_sh, int batch, int hq, int hd, int dtype,
                          int ns, int chunk_len, int max_len, hipStream_t st) {
  CombineParams c;
  const size_t slots = (size_t)batch * hq * ns;
  c.ws_o = ws;
  c.ws_lse = ws + slots * hd;
  c.seqlens = seqlens;
  c.out = (uint16_t *)out;
  c.o_sb = o_sb;
  c.o_sh = o_sh;
  c.seqlen_add = seqlen_add;
  c.batch = batch;
  c.hq = hq;
  c.max_len = max_len;
  c.num_splits = ns;
  c.chunk_len = chunk_len;
  if (dtype == MXFA_DTYPE_BF16)
    return hd == 128 ? launch_combine_t<128, BF16>(c, st) : launch_combine_t<64, BF16>(c, st);
  return hd == 128 ? launch_combine_t<128, F16>(c, st) : launch_combine_t<64, F16>(c, st);
}

}  // namespace mxfa

using namespace mxfa;

extern "C" {

int mxfa_abi_version(void) { return MXFA_ABI_VERSION; }

const char *mxfa_strerror(int code) {
  switch (code) {
    case MXFA_OK: return "ok";
    case MXFA_EUNSUPPORTED: return "unsupported configuration (head dim, GQA ratio, dtype or page size)";
    case MXFA_EINVAL: return "invalid argument (null pointer, size, alignment or stride)";
    case MXFA_EWORKSPACE: return "workspace missing or too small";
    case MXFA_ELAUNCH: return "kernel launch failed";
  }
  return "unknown error";
}

int mxfa_split_heuristic(int batch, int kv_heads, int page_size, int block_table_width,
                         int num_cus, int *num_splits, int *chunk_len) {
  if (!num_splits || !chunk_len) return MXFA_EINVAL;
  if (batch <= 0 || kv_heads <= 0 || page_size <= 0 || block_table_width <= 0 || num_cus <= 0)
    return MXFA_EINVAL;
  const int64_t cap = (int64_t)block_table_width * page_size;
  if (cap > (int64_t)1 << 30) return MXFA_EUNSUPPORTED;
  // Aim for about eight (sequence, kv head, split) workgroups per CU when the
  // sequences fill their block tables, with splits of at least kMinChunk tokens.
  const int64_t kMinChunk = 256;
  const int64_t kMaxSplits = 1024;
  const int64_t target = (int64_t)num_cus * 8;
  const int64_t base = (int64_t)batch * kv_heads;
  int64_t want = (target + base - 1) / base;
  if (want < 1) want = 1;
  int64_t c = (cap + want - 1) / want;
  if (c < kMinChunk) c = kMinChunk;
  c = (c + 63) / 64 * 64;
  int64_t n = (cap + c - 1) / c;
  if (n > kMaxSplits) {
    n = kMaxSplits;
    c = ((cap + n - 1) / n + 63) / 64 * 64;
    n = (cap + c - 1) / c;
  }
  if (n <= 1) {
    n = 1;
    c = (cap + 63) / 64 * 64;
  }
  *num_splits = (int)n;
  *chunk_len = (int)c;
  return MXFA_OK;
}

int mxfa_split_decode_workspace_size(int batch, int q_heads, int head_dim, int num_splits,
                                     size_t *bytes) {
  if (!bytes || batch <= 0 || q_heads <= 0 || head_dim <= 0 || num_splits <= 0)
    return MXFA_EINVAL;
  *bytes = workspace_bytes(batch, q_heads, head_dim, num_splits);
  return MXFA_OK;
}

int mxfa_split_decode_launch(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                             const void *k_cache, const void *v_cache,
                             int64_t cache_stride_page, int64_t cache_stride_token,
                             int64_t cache_stride_head, const int32_t *block_table,
                             int64_t bt_stride, const int32_t *seqlens, int seqlen_add,
                             void *out, int64_t out_stride_b, int64_t out_stride_h,
                             void *workspace, size_t workspace_bytes_, float scale, int batch,
                             int q_heads, int kv_heads, int head_dim, int page_size,
                             int block_table_width, int num_pages, int dtype, int num_splits,
                             int chunk_len, void *stream) {
  SplitArgs a{q,         q_stride_b,       q_stride_h,   k_cache,      v_cache,
              cache_stride_page, cache_stride_token, cache_stride_head, block_table, bt_stride,
              seqlens,   seqlen_add,       out,          out_stride_b, out_stride_h,
              workspace, workspace_bytes_, scale,        batch,        q_heads,
              kv_heads,  head_dim,         page_size,    block_table_width, num_pages,
              dtype,     num_splits,       chunk_len};
  int rc = check_split_args(a, true, true);
  if (rc != MXFA_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  rc = launch_partial(a, st);
  if (rc != MXFA_OK || num_splits == 1) return rc;
  return launch_combine((const float *)workspace, seqlens, seqlen_add, out, out_stride_b,
                        out_stride_h, batch, q_heads, head_dim, dtype, num_splits, chunk_len,
                        block_table_width * page_size, st);
}

int mxfa_split_decode_partial_launch(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                                     const void *k_cache, const void *v_cache,
                                     int64_t cache_stride_page, int64_t cache_stride_token,
                                     int64_t cache_stride_head, const int32_t *block_table,
                                     int64_t bt_stride, const int32_t *seqlens, int seqlen_add,
                                     void *workspace, size_t workspace_bytes_, float scale,
                                     int batch, int q_heads, int kv_heads, int head_dim,
                                     int page_size, int block_table_width, int num_pages,
                                     int dtype, int num_splits, int chunk_len, void *stream) {
  if (num_splits < 2) return MXFA_EINVAL;  // the partial stage exists only with splits
  SplitArgs a{q,         q_stride_b,       q_stride_h,   k_cache,      v_cache,
              cache_stride_page, cache_stride_token, cache_stride_head, block_table, bt_stride,
              seqlens,   seqlen_add,       nullptr,      0,            0,
              workspace, workspace_bytes_, scale,        batch,        q_heads,
              kv_heads,  head_dim,         page_size,    block_table_width, num_pages,
              dtype,     num_splits,       chunk_len};
  int rc = check_split_args(a, false, true);
  if (rc != MXFA_OK) return rc;
  return launch_partial(a, (hipStream_t)stream);
}

int mxfa_split_decode_combine_launch(const void *workspace, size_t workspace_bytes_,
                                     const int32_t *seqlens, int seqlen_add, void *out,
                                     int64_t out_stride_b, int64_t out_stride_h, int batch,
                                     int q_heads, int head_dim, int dtype, int num_splits,
                                     int chunk_len, void *stream) {
  if (!workspace || !seqlens || !out) return MXFA_EINVAL;
  if (batch <= 0 || q_heads <= 0 || num_splits < 2 || chunk_len <= 0 || seqlen_add < 0)
    return MXFA_EINVAL;
  if (head_dim != 64 && head_dim != 128) return MXFA_EUNSUPPORTED;
  if (dtype != MXFA_DTYPE_F16 && dtype != MXFA_DTYPE_BF16) return MXFA_EUNSUPPORTED;
  if (!aligned16(workspace) || ((uintptr_t)out & 7u) || ((out_stride_b | out_stride_h) & 3))
    return MXFA_EINVAL;
  if (workspace_bytes_ < workspace_bytes(batch, q_heads, head_dim, num_splits))
    return MXFA_EWORKSPACE;
  const int64_t max_len = (int64_t)num_splits * chunk_len;
  return launch_combine((const float *)workspace, seqlens, seqlen_add, out, out_stride_b,
                        out_stride_h, batch, q_heads, head_dim, dtype, num_splits, chunk_len,
                        (int)(max_len > (1 << 30) ? (1 << 30) : max_len), (hipStream_t)stream);
}

}  // extern "C"

// Split-KV paged decode attention for MI355X (gfx950, wave64).
//
// Work split (sized on the device, no host sync). Every sequence b is cut into
// ceil(L_b / 16) tiles of 16 tokens; for each kv head the tiles of all
// sequences are laid end to end (tile index t = S_b + j, S = exclusive prefix
// sum) and cut into `num_splits` equal ranges. Workgroup (kv head, r) streams
// range r: [floor(r*NT/R), floor((r+1)*NT/R)). A range covers whole sequences
// and at most two pieces of sequences that cross its ends. Every workgroup
// therefore gets the same number of tiles whatever the length mix, which is
// what keeps all 256 CUs busy to the end of the call.
//
// Partial kernel, per workgroup (4 waves) and per sequence piece of its range:
//   waves take the piece's tiles round-robin; per tile of 16 tokens
//   QK   on the matrix cores: S^T[16 tokens x 16 heads] = K[16 x HD] . Q^T[HD x 16]
//        (v_mfma_f32_16x16x32, HD/32 steps; query heads >= GQ are zero columns).
//        K is loaded token-per-lane for the A operand: lane l reads 64
//        contiguous bytes of token l%16 per step. Result layout: lane
//        (r = l/16, h = l%16) holds the scores of tokens 4r+i, i = 0..3, head h.
//   softmax on that layout in the base-2 domain: one exp per (token, head).
//        The reference max m of each head is shared by the wave and only moves
//        (wave-uniform branch) when a score passes it by kRescaleLog2, so
//        p = 2^(x - m) <= 2^kRescaleLog2 and rescales are rare.
//   PV   on the VALU: V is loaded row-per-DPP-row (lane (r, c) holds dims
//        [c*VD, c*VD+VD) of token 4r+u for load u), so the probability of
//        token 4r+u and head h sits in lane (r, h), register u, of the same DPP
//        row and reaches every lane through a row_newbcast:h operand.
//   Rows, then waves (through LDS) are merged per piece. A piece that is a
//   whole sequence writes the final output; a piece of a longer sequence
//   writes its normalised output and base-2 log-sum-exp to the workspace.
//
// Combine kernel: for every sequence that crosses a range end, merge its pieces
// with the LSE weights; it also writes the zero output of empty sequences.
//
// Workspace (fp32 unless noted), R = num_splits:
//   ws_o   [HQ, R, 2, HD]  piece outputs; slot 0 = first piece of the range,
//                          slot 1 = last piece (when it differs)
//   ws_lse [HQ, R, 2]      piece log-sum-exp (base 2)
//   ws_s   int32 [B + 1]   tile prefix sums S (written by workgroup (0, 0))
//
// Reference counterpart: paged_decode_v3 split mode and split_combine
// (csrc_native/m1_kernel.cpp:553-888) with the split count of
// integrations/vllm/vllm_plugin.py:271-276; the algorithm (split partials +
// LSE merge) is the same, the work split, data path and numerics are this
// file's own.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "mxfa_device.h"
#include "mxfa_mi355x.h"

namespace mxfa {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kTile = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleLog2 = 8.0f;
constexpr int kMaxBatch = 16384;  // tile prefix sums live in LDS

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
  int32_t *ws_s;
  float scale_log2;
  int seqlen_add;
  int batch;
  int hq;
  int ps_log2;
  int max_len;  // block_table_width * page_size
  int num_pages;
  int num_ranges;
};

struct CombineParams {
  const float *ws_o;
  const float *ws_lse;
  const int32_t *ws_s;
  uint16_t *out;
  int64_t o_sb, o_sh;
  int batch;
  int hq;
  int num_ranges;
};

// Block tables and lengths are read-only for the whole call; reading them
// through the constant address space lets wave-uniform lookups use scalar
// (SMEM) loads even inside loops that also store results.
typedef const __attribute__((address_space(4))) int32_t *ConstI32;

__device__ __forceinline__ ConstI32 as_const(const int32_t *p) { return (ConstI32)p; }

__device__ __forceinline__ int seq_len_of(const int32_t *seqlens, int b, int add, int max_len) {
  int L = as_const(seqlens)[b] + add;
  L = L < 0 ? 0 : L;
  return L > max_len ? max_len : L;
}

// First tile of range r out of R over NT tiles, and the range holding tile t.
__device__ __forceinline__ int range_lo(int r, int R, int NT) {
  return (int)(((int64_t)r * NT) / R);
}
__device__ __forceinline__ int range_of(int t, int R, int NT) {
  return (int)((((int64_t)t + 1) * R - 1) / NT);
}

template <typename T>
struct Mfma;
template <>
struct Mfma<F16> {
  static __device__ __forceinline__ f32x4 run(const uint4 &a, const uint4 &b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma<BF16> {
  static __device__ __forceinline__ f32x4 run(const uint4 &a, const uint4 &b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

// V fragment of one lane: 8 elements (HD128, 16 B) or 4 elements (HD64, 8 B).
template <int VD>
struct VFrag;
template <>
struct VFrag<8> {
  uint4 w;
  static __device__ __forceinline__ VFrag load(const char *ptr) {
    VFrag f;
    f.w = *reinterpret_cast<const uint4 *>(ptr);
    return f;
  }
  template <typename E>
  __device__ __forceinline__ void widen(float (&v)[8]) const {
    v[0] = E::lo(w.x);
    v[1] = E::hi(w.x);
    v[2] = E::lo(w.y);
    v[3] = E::hi(w.y);
    v[4] = E::lo(w.z);
    v[5] = E::hi(w.z);
    v[6] = E::lo(w.w);
    v[7] = E::hi(w.w);
  }
};
template <>
struct VFrag<4> {
  uint2 w;
  static __device__ __forceinline__ VFrag load(const char *ptr) {
    VFrag f;
    f.w = *reinterpret_cast<const uint2 *>(ptr);
    return f;
  }
  template <typename E>
  __device__ __forceinline__ void widen(float (&v)[4]) const {
    v[0] = E::lo(w.x);
    v[1] = E::hi(w.x);
    v[2] = E::lo(w.y);
    v[3] = E::hi(w.y);
  }
};

template <int H>
__device__ __forceinline__ float row_bcast(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), kDppRowNewBcast0 + H, 0xf, 0xf, false));
}

// o[h][j] += p(token of this lane's row, head h) * v[j] for every head of the group.
template <int GQ, int VD, int H = 0>
__device__ __forceinline__ void pv_accumulate(float (&o)[GQ][VD], float p, const float (&v)[VD]) {
  if constexpr (H < GQ) {
    const float ph = row_bcast<H>(p);
#pragma unroll
    for (int j = 0; j < VD; ++j) o[H][j] = fmaf(ph, v[j], o[H][j]);
    pv_accumulate<GQ, VD, H + 1>(o, p, v);
  }
}

template <int GQ, int VD, int H = 0>
__device__ __forceinline__ void rescale_rows(float (&o)[GQ][VD], float f) {
  if constexpr (H < GQ) {
    const float fh = row_bcast<H>(f);
#pragma unroll
    for (int j = 0; j < VD; ++j) o[H][j] *= fh;
    rescale_rows<GQ, VD, H + 1>(o, f);
  }
}

// Exclusive prefix sum of per-sequence tile counts into s[0..B] (LDS), all threads.
__device__ __forceinline__ void tile_prefix(const DecodeParams &p, int32_t *s, int *wave_tot) {
  const int B = p.batch;
  const int per = (B + kThreads - 1) / kThreads;
  const int b0 = threadIdx.x * per;
  int local = 0;
  for (int i = 0; i < per; ++i) {
    const int b = b0 + i;
    if (b < B) local += (seq_len_of(p.seqlens, b, p.seqlen_add, p.max_len) + kTile - 1) / kTile;
  }
  // Inclusive scan of `local` across the workgroup.
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) wave_tot[wave] = x;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += wave_tot[w];
  int run = base + x - local;  // exclusive prefix of this thread's first element
  for (int i = 0; i < per; ++i) {
    const int b = b0 + i;
    if (b < B) {
      s[b] = run;
      run += (seq_len_of(p.seqlens, b, p.seqlen_add, p.max_len) + kTile - 1) / kTile;
    }
  }
  if (threadIdx.x == kThreads - 1) s[B] = base + x;
  __syncthreads();
}

// kLanePages: page size below the 16-token tile, so every lane looks up its own
// tokens' pages. Otherwise a tile lies in one page: one scalar lookup per tile.
template <int HD, int GQ, typename T, bool kLanePages>
__global__ __launch_bounds__(kThreads) void split_partial_kernel(DecodeParams p) {
  using E = Elem<T>;
  constexpr int NCH = HD / 32;  // MFMA steps over the head dim
  constexpr int VD = HD / 16;   // V elements per lane
  constexpr int U = 4;          // V loads per tile (token 4r+u in DPP row r)

  extern __shared__ int32_t s_tiles[];  // [B + 1]
  __shared__ int s_wave_tot[kWaves];
  __shared__ float sm_m[kWaves][GQ];
  __shared__ float sm_d[kWaves][GQ];
  __shared__ float sm_o[kWaves][GQ][HD];

  const int kvh = blockIdx.x;
  const int r = blockIdx.y;
  const int R = p.num_ranges;
  tile_prefix(p, s_tiles, s_wave_tot);
  const int B = p.batch;
  const int NT = s_tiles[B];
  if (kvh == 0 && r == 0) {
    for (int i = threadIdx.x; i <= B; i += kThreads) p.ws_s[i] = s_tiles[i];
  }
  const int lo = range_lo(r, R, NT), hi = range_lo(r + 1, R, NT);
  if (lo >= hi) return;

  // Sequence holding tile lo: largest b with s[b] <= lo (then s[b+1] > lo).
  int b;
  {
    int a = 0, z = B - 1;
    while (a < z) {
      const int mid = (a + z + 1) >> 1;
      if (s_tiles[mid] <= lo) a = mid;
      else z = mid - 1;
    }
    b = __builtin_amdgcn_readfirstlane(a);
  }

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = lane >> 4;  // DPP row
  const int col = lane & 15;  // head (score layout) / V column
  const int h0 = kvh * GQ;

  const char *__restrict__ kbase = reinterpret_cast<const char *>(p.k);
  const char *__restrict__ vbase = reinterpret_cast<const char *>(p.v);
  const int ps_mask = (1 << p.ps_log2) - 1;
  const uint32_t st_bytes = (uint32_t)p.c_st * 2u;
  const uint64_t sp_bytes = (uint64_t)p.c_sp * 2u;
  const uint32_t head_bytes = (uint32_t)kvh * ((uint32_t)p.c_sh * 2u);
  const uint32_t k_lane_bytes = head_bytes + (uint32_t)row * 16u;  // + 64c
  const uint32_t v_lane_bytes = head_bytes + (uint32_t)col * (VD * 2u);
  const float c = p.scale_log2;

  bool first_piece = true;
  for (; b < B && s_tiles[b] < hi; ++b) {
    const int sb = s_tiles[b], se = s_tiles[b + 1];
    const int t0 = (lo > sb ? lo : sb) - sb;  // piece = tiles [t0, t1) of sequence b
    const int t1 = (hi < se ? hi : se) - sb;
    if (t1 <= t0) continue;
    const int L = seq_len_of(p.seqlens, b, p.seqlen_add, p.max_len);
    const int c_start = t0 * kTile;
    const int sl = (t1 * kTile < L ? t1 * kTile : L) - c_start;  // tokens in the piece
    const int ntiles = t1 - t0;
    const ConstI32 btrow = as_const(p.bt + (int64_t)b * p.bt_stride);

    // B operand of the QK MFMA: lane (row, col) holds q[head col][32c + 8row, +8).
    uint4 qf[NCH];
#pragma unroll
    for (int cc = 0; cc < NCH; ++cc) {
      qf[cc] = make_uint4(0u, 0u, 0u, 0u);
      if (col < GQ)
        qf[cc] = *reinterpret_cast<const uint4 *>(p.q + b * p.q_sb + (int64_t)(h0 + col) * p.q_sh +
                                                   cc * 32 + row * 8);
    }

    float m = -INFINITY;  // reference max (base 2) of head `col`, same in every row
    float d = 0.f;        // partial denominator of head `col` over this row's tokens
    float o[GQ][VD];
#pragma unroll
    for (int g = 0; g < GQ; ++g)
#pragma unroll
      for (int j = 0; j < VD; ++j) o[g][j] = 0.f;

    auto clamp_page = [&](int pg) -> int {
      pg = pg < 0 ? 0 : pg;
      return pg >= p.num_pages ? p.num_pages - 1 : pg;
    };
    // Token positions clamp to the last valid token, so every address is a
    // real row of this sequence (and in the tile's own page).
    auto pos_of = [&](int tile, int t) -> int {
      t += tile * kTile;
      return c_start + (t < sl ? t : sl - 1);
    };

    // Per tile: page ids (scalar: [0] for the whole tile; lane: [0] K, [1+u] V).
    constexpr int NPG = kLanePages ? 1 + U : 1;
    int pg_a[NPG], pg_b[NPG];
    uint4 ka[NCH], kb[NCH];
    VFrag<VD> va[U], vb[U];

    auto load_pages = [&](int tile, int (&pg)[NPG]) {
      if constexpr (kLanePages) {
        pg[0] = btrow[pos_of(tile, col) >> p.ps_log2];
#pragma unroll
        for (int u = 0; u < U; ++u) pg[1 + u] = btrow[pos_of(tile, 4 * row + u) >> p.ps_log2];
      } else {
        pg[0] = btrow[__builtin_amdgcn_readfirstlane(pos_of(tile, 0) >> p.ps_log2)];
      }
    };
    auto load_kv = [&](int tile, const int (&pg)[NPG], uint4 (&kr)[NCH], VFrag<VD> (&vr)[U]) {
      {
        const int pos = pos_of(tile, col);
        const uint64_t page_off = (uint64_t)(uint32_t)clamp_page(pg[0]) * sp_bytes;
        const uint32_t off = (uint32_t)(pos & ps_mask) * st_bytes + k_lane_bytes;
#pragma unroll
        for (int cc = 0; cc < NCH; ++cc)
          kr[cc] = *reinterpret_cast<const uint4 *>(kbase + page_off + off + cc * 64u);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int pos = pos_of(tile, 4 * row + u);
        const int pgv = kLanePages ? pg[kLanePages ? 1 + u : 0] : pg[0];
        const uint64_t page_off = (uint64_t)(uint32_t)clamp_page(pgv) * sp_bytes;
        const uint32_t off = (uint32_t)(pos & ps_mask) * st_bytes + v_lane_bytes;
        vr[u] = VFrag<VD>::load(vbase + page_off + off);
      }
    };
    // Lane-page ids (VMEM) are fetched before the K/V loads that follow them so
    // waiting for an id never waits for K/V data; scalar ids (SMEM, unordered)
    // after the K/V loads that consume the previous ids.
    auto advance = [&](int tile, const int (&pg_next)[NPG], int (&pg_after)[NPG],
                       uint4 (&kr)[NCH], VFrag<VD> (&vr)[U]) {
      if constexpr (kLanePages) {
        load_pages(tile + 2 * kWaves, pg_after);
        load_kv(tile + kWaves, pg_next, kr, vr);
      } else {
        load_kv(tile + kWaves, pg_next, kr, vr);
        load_pages(tile + 2 * kWaves, pg_after);
      }
    };
    auto compute = [&](int tile, const uint4 (&kr)[NCH], const VFrag<VD> (&vr)[U]) {
      // QK on the matrix cores; two accumulators halve the MFMA dependency chain.
      f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cc = 0; cc < NCH; cc += 2) {
        acc0 = Mfma<T>::run(kr[cc], qf[cc], acc0);
        acc1 = Mfma<T>::run(kr[cc + 1], qf[cc + 1], acc1);
      }
      float x[4];
      bool need = false;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool valid = (col < GQ) & (tile * kTile + 4 * row + i < sl);
        x[i] = valid ? (acc0[i] + acc1[i]) * c : -INFINITY;
        need |= x[i] > m + kRescaleLog2;
      }
      if (__builtin_amdgcn_ballot_w64(need) != 0) {
        // Rare, wave-uniform: move the reference of each head to the wave's
        // tile maximum when it passed the reference by more than kRescaleLog2.
        float mt = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
        mt = fmaxf(mt, xor_shfl(mt, 16));
        mt = fmaxf(mt, xor_shfl(mt, 32));
        const float mn = mt > m + kRescaleLog2 ? mt : m;
        const float f = (mn == m) ? 1.f : fast_exp2(m - mn);  // m = -inf: f = 0
        d *= f;
        rescale_rows<GQ, VD>(o, f);
        m = mn;
      }
      // m = -inf: this head has seen no valid token, its scores here are -inf too.
      const float mr = m == -INFINITY ? 0.f : m;
      float pr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pr[i] = fast_exp2(x[i] - mr);
      d += (pr[0] + pr[1]) + (pr[2] + pr[3]);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float v[VD];
        vr[u].template widen<E>(v);
        pv_accumulate<GQ, VD>(o, pr[u], v);
      }
    };

    // Software pipeline over this wave's tiles of the piece: wave, wave +
    // kWaves, ... Page ids run two tiles ahead of the math and K/V loads one
    // tile ahead; two register sets (a/b) alternate so no copies are needed.
    // The loop body runs two tiles and exits only at its latch, so the loads
    // crossing the back edge are always the a-set of the next tile and the
    // compiler never has to drain the load queue at the loop head. Loads past
    // the wave's last tile clamp to the last valid token (cache hits).
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

    // Merge the four DPP rows of the wave (same reference max, different tokens).
    d += xor_shfl(d, 16);
    d += xor_shfl(d, 32);
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
#pragma unroll
      for (int j = 0; j < VD; ++j) {
        float t = o[g][j];
        t += xor_shfl(t, 16);
        t += xor_shfl(t, 32);
        o[g][j] = t;
      }
    }
    if (row == 0) {
#pragma unroll
      for (int g = 0; g < GQ; ++g)
#pragma unroll
        for (int j = 0; j < VD; ++j) sm_o[wave][g][col * VD + j] = o[g][j];
      if (col < GQ) {
        sm_m[wave][col] = m;
        sm_d[wave][col] = d;
      }
    }
    __syncthreads();

    // Merge the waves; a whole sequence writes its output, a piece its partial.
    const bool whole = (t0 == 0) && (t1 == se - sb);
    const int slot = first_piece ? 0 : 1;
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
      const float res = D > 0.f ? O / D : 0.f;
      const int h = h0 + g;
      if (whole) {
        p.out[b * p.o_sb + (int64_t)h * p.o_sh + dim] = E::narrow(res);
      } else {
        const int64_t ps = ((int64_t)h * R + r) * 2 + slot;
        p.ws_o[ps * HD + dim] = res;
        if (dim == 0) p.ws_lse[ps] = D > 0.f ? M + __log2f(D) : -INFINITY;
      }
    }
    first_piece = false;
    __syncthreads();  // sm_* are reused by the next piece
  }
}

// LSE combine: HD/4 threads per (sequence, head), float4 per thread. Sequences
// that lie inside one range were written by the partial kernel and are skipped.
template <int HD, typename T>
__global__ __launch_bounds__(256) void split_combine_kernel(CombineParams p) {
  using E = Elem<T>;
  constexpr int TPH = HD / 4;
  constexpr int HPB = 256 / TPH;
  const int hid = blockIdx.x * HPB + threadIdx.x / TPH;
  if (hid >= p.batch * p.hq) return;
  const int t = threadIdx.x % TPH;
  const int b = hid / p.hq, h = hid % p.hq;
  const int R = p.num_ranges;
  const int NT = p.ws_s[p.batch];
  const int sb = p.ws_s[b], nt = p.ws_s[b + 1] - sb;
  uint2 *dst = reinterpret_cast<uint2 *>(p.out + b * p.o_sb + (int64_t)h * p.o_sh + t * 4);
  // The prefix sums come from the partial launch; prefix sums that do not
  // describe tiles inside [0, NT) (a workspace the partial stage did not fill)
  // give zeros, so every range index below stays in [0, R).
  if (nt <= 0 || sb < 0 || NT <= 0 || sb + nt > NT) {
    *dst = make_uint2(0u, 0u);  // empty sequence: zero output
    return;
  }
  const int ra = range_of(sb, R, NT), rb = range_of(sb + nt - 1, R, NT);
  if (ra == rb) return;  // whole sequence inside one range: already written

  // Pieces, walked range by range over the sequence's tiles: range ra holds
  // slot 0 when the sequence starts that range (else slot 1); every later
  // range holds slot 0. Two passes: the LSE maximum, then the weighted sum.
  const int slot_a = (range_lo(ra, R, NT) == sb) ? 0 : 1;
  const int tend = sb + nt;
  float M = -INFINITY;
  for (int tt = sb; tt < tend;) {
    const int q = range_of(tt, R, NT);
    const int64_t ps = ((int64_t)h * R + q) * 2 + (q == ra ? slot_a : 0);
    M = fmaxf(M, p.ws_lse[ps]);
    tt = range_lo(q + 1, R, NT);
  }
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float wsum = 0.f;
  if (M != -INFINITY) {
    for (int tt = sb; tt < tend;) {
      const int q = range_of(tt, R, NT);
      const int64_t ps = ((int64_t)h * R + q) * 2 + (q == ra ? slot_a : 0);
      const float l = p.ws_lse[ps];
      const float w = (l == -INFINITY) ? 0.f : fast_exp2(l - M);
      const float4 v = reinterpret_cast<const float4 *>(p.ws_o + ps * HD)[t];
      acc.x = fmaf(w, v.x, acc.x);
      acc.y = fmaf(w, v.y, acc.y);
      acc.z = fmaf(w, v.z, acc.z);
      acc.w = fmaf(w, v.w, acc.w);
      wsum += w;
      tt = range_lo(q + 1, R, NT);
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  const uint16_t r0 = E::narrow(acc.x * inv), r1 = E::narrow(acc.y * inv);
  const uint16_t r2 = E::narrow(acc.z * inv), r3 = E::narrow(acc.w * inv);
  *dst = make_uint2((uint32_t)r0 | ((uint32_t)r1 << 16), (uint32_t)r2 | ((uint32_t)r3 << 16));
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
  int batch, hq, hkv, hd, ps, btw, num_pages, dtype, num_splits;
};

struct WsLayout {
  size_t o_floats, lse_floats, s_ints, bytes;
};

static WsLayout ws_layout(int batch, int hq, int hd, int ns) {
  WsLayout w;
  w.o_floats = (size_t)hq * ns * 2 * hd;
  w.lse_floats = (size_t)hq * ns * 2;
  w.s_ints = (size_t)batch + 1;
  w.bytes = (w.o_floats + w.lse_floats + w.s_ints) * 4;
  return w;
}

static int check_split_args(const SplitArgs &a) {
  if (!a.q || !a.k || !a.v || !a.bt || !a.seqlens || !a.out) return MXFA_EINVAL;
  if (a.batch <= 0 || a.hq <= 0 || a.hkv <= 0 || a.btw <= 0 || a.num_pages <= 0)
    return MXFA_EINVAL;
  if (a.num_splits <= 0 || a.seqlen_add < 0) return MXFA_EINVAL;
  if (!(a.scale == a.scale) || a.scale == INFINITY || a.scale == -INFINITY) return MXFA_EINVAL;
  if (a.hd != 64 && a.hd != 128) return MXFA_EUNSUPPORTED;
  if (a.hq % a.hkv != 0) return MXFA_EUNSUPPORTED;
  const int gq = a.hq / a.hkv;
  if (gq != 2 && gq != 4 && gq != 8) return MXFA_EUNSUPPORTED;
  if (a.dtype != MXFA_DTYPE_F16 && a.dtype != MXFA_DTYPE_BF16) return MXFA_EUNSUPPORTED;
  if (ilog2_exact(a.ps) < 0 || a.ps > 4096) return MXFA_EUNSUPPORTED;
  if (a.num_splits > 65535 || a.batch > kMaxBatch || a.hkv > 65535) return MXFA_EUNSUPPORTED;
  const int64_t max_len = (int64_t)a.btw * a.ps;
  if (max_len > (int64_t)1 << 30) return MXFA_EUNSUPPORTED;
  // Total tiles per kv head must fit int32: B * ceil(max_len / 16).
  if ((int64_t)a.batch * ((max_len + kTile - 1) / kTile) >= ((int64_t)1 << 31))
    return MXFA_EUNSUPPORTED;
  // 16-byte fragments: pointers and every stride must keep 8-element alignment.
  if (!aligned16(a.q) || !aligned16(a.k) || !aligned16(a.v)) return MXFA_EINVAL;
  if ((a.q_sb | a.q_sh | a.c_sp | a.c_st | a.c_sh) & 7) return MXFA_EINVAL;
  if (a.q_sb < 0 || a.q_sh < 0 || a.c_sp < 0 || a.c_st < 0 || a.c_sh < 0 || a.bt_stride < 0)
    return MXFA_EINVAL;
  // In-page byte offsets are 32-bit: (PS-1)*token + (HKV-1)*head + HD elements.
  if (((int64_t)(a.ps - 1) * a.c_st + (int64_t)(a.hkv - 1) * a.c_sh + a.hd) * 2 >=
      ((int64_t)1 << 32))
    return MXFA_EUNSUPPORTED;
  if (((uintptr_t)a.out & 7u) || ((a.o_sb | a.o_sh) & 3) || a.o_sb < 0 || a.o_sh < 0)
    return MXFA_EINVAL;
  if (!a.ws || !aligned16(a.ws)) return MXFA_EWORKSPACE;
  if (a.ws_bytes < ws_layout(a.batch, a.hq, a.hd, a.num_splits).bytes) return MXFA_EWORKSPACE;
  return MXFA_OK;
}

static DecodeParams make_params(const SplitArgs &a) {
  const WsLayout w = ws_layout(a.batch, a.hq, a.hd, a.num_splits);
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
  p.ws_o = (float *)a.ws;
  p.ws_lse = (float *)a.ws + w.o_floats;
  p.ws_s = (int32_t *)((float *)a.ws + w.o_floats + w.lse_floats);
  p.scale_log2 = a.scale * kLog2e;
  p.seqlen_add = a.seqlen_add;
  p.batch = a.batch;
  p.hq = a.hq;
  p.ps_log2 = ilog2_exact(a.ps);
  p.max_len = a.btw * a.ps;
  p.num_pages = a.num_pages;
  p.num_ranges = a.num_splits;
  return p;
}

template <int HD, int GQ, typename T>
static int launch_partial_t(const DecodeParams &p, int hkv, hipStream_t st) {
  dim3 grid(hkv, p.num_ranges);
  const size_t lds = (size_t)(p.batch + 1) * sizeof(int32_t);
  if ((1 << p.ps_log2) >= kTile)
    hipLaunchKernelGGL((split_partial_kernel<HD, GQ, T, false>), grid, dim3(kThreads), lds, st, p);
  else
    hipLaunchKernelGGL((split_partial_kernel<HD, GQ, T, true>), grid, dim3(kThreads), lds, st, p);
  return hipGetLastError() == hipSuccess ? MXFA_OK : MXFA_ELAUNCH;
}

template <int HD, typename T>
static int launch_partial_gq(const DecodeParams &p, int gq, int hkv, hipStream_t st) {
  switch (gq) {
    case 2: return launch_partial_t<HD, 2, T>(p, hkv, st);
    case 4: return launch_partial_t<HD, 4, T>(p, hkv, st);
    case 8: return launch_partial_t<HD, 8, T>(p, hkv, st);
  }
  return MXFA_EUNSUPPORTED;
}

static int launch_partial(const SplitArgs &a, hipStream_t st) {
  const DecodeParams p = make_params(a);
  const int gq = a.hq / a.hkv;
  if (a.dtype == MXFA_DTYPE_BF16) {
    return a.hd == 128 ? launch_partial_gq<128, BF16>(p, gq, a.hkv, st)
                       : launch_partial_gq<64, BF16>(p, gq, a.hkv, st);
  }
  return a.hd == 128 ? launch_partial_gq<128, F16>(p, gq, a.hkv, st)
                     : launch_partial_gq<64, F16>(p, gq, a.hkv, st);
}

template <int HD, typename T>
static int launch_combine_t(const CombineParams &c, hipStream_t st) {
  constexpr int HPB = 256 / (HD / 4);
  const int heads = c.batch * c.hq;
  dim3 grid((heads + HPB - 1) / HPB);
  hipLaunchKernelGGL((split_combine_kernel<HD, T>), grid, dim3(256), 0, st, c);
  return hipGetLastError() == hipSuccess ? MXFA_OK : MXFA_ELAUNCH;
}

static int launch_combine(void *ws, void *out, int64_t o_sb, int64_t o_sh, int batch, int hq,
                          int hd, int dtype, int ns, hipStream_t st) {
  const WsLayout w = ws_layout(batch, hq, hd, ns);
  CombineParams c;
  c.ws_o = (const float *)ws;
  c.ws_lse = (const float *)ws + w.o_floats;
  c.ws_s = (const int32_t *)((const float *)ws + w.o_floats + w.lse_floats);
  c.out = (uint16_t *)out;
  c.o_sb = o_sb;
  c.o_sh = o_sh;
  c.batch = batch;
  c.hq = hq;
  c.num_ranges = ns;
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

int mxfa_split_heuristic(int batch, int q_heads, int kv_heads, int head_dim, int page_size,
                         int block_table_width, int num_cus, int *num_splits) {
  if (!num_splits) return MXFA_EINVAL;
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || page_size <= 0 ||
      block_table_width <= 0 || num_cus <= 0)
    return MXFA_EINVAL;
  // One workgroup (one wave per SIMD) per CU streams fastest (measured on
  // MI355X across the GQ x HD cells); a second one per CU pays where the math
  // per byte is highest (HD 64 with GQ 8) and where block tables are short
  // (many short sequences, so more pieces to merge per range).
  const int64_t cap = (int64_t)block_table_width * page_size;
  const int gq = q_heads / kv_heads;
  const int64_t per_cu = ((head_dim == 64 && gq >= 8) || cap < 2048) ? 2 : 1;
  const int64_t kMinTiles = 4;
  const int64_t cap_tiles = (int64_t)batch * ((cap + kTile - 1) / kTile);
  int64_t n = ((int64_t)num_cus * per_cu + kv_heads - 1) / kv_heads;
  const int64_t by_tiles = (cap_tiles + kMinTiles - 1) / kMinTiles;
  if (n > by_tiles) n = by_tiles;
  if (n < 1) n = 1;
  if (n > 65535) n = 65535;
  *num_splits = (int)n;
  return MXFA_OK;
}

int mxfa_split_decode_workspace_size(int batch, int q_heads, int head_dim, int num_splits,
                                     size_t *bytes) {
  if (!bytes || batch <= 0 || q_heads <= 0 || head_dim <= 0 || num_splits <= 0)
    return MXFA_EINVAL;
  *bytes = ws_layout(batch, q_heads, head_dim, num_splits).bytes;
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
                             void *stream) {
  SplitArgs a{q,         q_stride_b,       q_stride_h,   k_cache,      v_cache,
              cache_stride_page, cache_stride_token, cache_stride_head, block_table, bt_stride,
              seqlens,   seqlen_add,       out,          out_stride_b, out_stride_h,
              workspace, workspace_bytes_, scale,        batch,        q_heads,
              kv_heads,  head_dim,         page_size,    block_table_width, num_pages,
              dtype,     num_splits};
  int rc = check_split_args(a);
  if (rc != MXFA_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  rc = launch_partial(a, st);
  if (rc != MXFA_OK) return rc;
  return launch_combine(workspace, out, out_stride_b, out_stride_h, batch, q_heads, head_dim,
                        dtype, num_splits, st);
}

int mxfa_split_decode_partial_launch(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                                     const void *k_cache, const void *v_cache,
                                     int64_t cache_stride_page, int64_t cache_stride_token,
                                     int64_t cache_stride_head, const int32_t *block_table,
                                     int64_t bt_stride, const int32_t *seqlens, int seqlen_add,
                                     void *out, int64_t out_stride_b, int64_t out_stride_h,
                                     void *workspace, size_t workspace_bytes_, float scale,
                                     int batch, int q_heads, int kv_heads, int head_dim,
                                     int page_size, int block_table_width, int num_pages,
                                     int dtype, int num_splits, void *stream) {
  SplitArgs a{q,         q_stride_b,       q_stride_h,   k_cache,      v_cache,
              cache_stride_page, cache_stride_token, cache_stride_head, block_table, bt_stride,
              seqlens,   seqlen_add,       out,          out_stride_b, out_stride_h,
              workspace, workspace_bytes_, scale,        batch,        q_heads,
              kv_heads,  head_dim,         page_size,    block_table_width, num_pages,
              dtype,     num_splits};
  int rc = check_split_args(a);
  if (rc != MXFA_OK) return rc;
  return launch_partial(a, (hipStream_t)stream);
}

int mxfa_split_decode_combine_launch(void *workspace, size_t workspace_bytes_, void *out,
                                     int64_t out_stride_b, int64_t out_stride_h, int batch,
                                     int q_heads, int head_dim, int dtype, int num_splits,
                                     void *stream) {
  if (!workspace || !out) return MXFA_EINVAL;
  if (batch <= 0 || q_heads <= 0 || num_splits <= 0) return MXFA_EINVAL;
  if (head_dim != 64 && head_dim != 128) return MXFA_EUNSUPPORTED;
  if (dtype != MXFA_DTYPE_F16 && dtype != MXFA_DTYPE_BF16) return MXFA_EUNSUPPORTED;
  if (batch > kMaxBatch || num_splits > 65535) return MXFA_EUNSUPPORTED;
  if (!aligned16(workspace) || ((uintptr_t)out & 7u) || ((out_stride_b | out_stride_h) & 3) ||
      out_stride_b < 0 || out_stride_h < 0)
    return MXFA_EINVAL;
  if (workspace_bytes_ < ws_layout(batch, q_heads, head_dim, num_splits).bytes)
    return MXFA_EWORKSPACE;
  return launch_combine(workspace, out, out_stride_b, out_stride_h, batch, q_heads, head_dim,
                        dtype, num_splits, (hipStream_t)stream);
}

}  // extern "C"

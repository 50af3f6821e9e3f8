// Split-KV paged decode attention for MI355X (gfx950, wave64): device code.
//
// Work split (sized on the device, no host sync). Every sequence b is cut into
// ceil(L_b / 16) tiles of 16 tokens; the tiles of all sequences are laid end to
// end (tile index t = S_b + j, S = exclusive prefix sum) and cut into R equal
// ranges [floor(r*NT/R), floor((r+1)*NT/R)), R = min(num_splits, NT). Every
// (kv head, range) pair is the work of one wave, so every wave streams the same
// number of tiles whatever the length mix.
//
// Workgroups: WAVES waves = KH kv heads x S sub-ranges (KH = min(HKV, WAVES),
// S = WAVES/KH). The waves of a workgroup read the same pages at the same
// time, all their kv heads of each token row together, so the HBM sees whole
// pages instead of 128/256-byte slivers spread over the run.
//
// Per wave, over the tiles of its range in order, with no break between
// sequences (the load pipeline runs straight across sequence ends):
//   loads  per tile, a buffer descriptor whose base is the tile's first row in
//          its page (head offset folded in) and whose size covers exactly the
//          valid rows, so rows past the sequence end and the padding tile past
//          the range end read as zeros and cost no memory traffic. K and V
//          carry the nontemporal hint (read once per call). With 128-byte
//          head rows, lanes c and c^8 of a DPP row load 16 V bytes of two
//          tokens each and swap halves (one DPP move per word).
//   QK     on the matrix cores: S^T[16 tokens x 16 columns] = K[16 x HD].Q^T[HD x 16]
//          (v_mfma_f32_16x16x32, HD/32 steps). Column c = t*GQ + g is query
//          token t (of QL new tokens per sequence) and query head g of the
//          group; columns >= GQ*QL are zero. 16-bit caches: lane l holds K
//          bytes [64c + 16(l/16), +16) of token l%16 for step c. fp8 caches:
//          lane l loads K bytes [64m + 16(l/16), +16) (16 elements) and widens
//          them exactly to the element type for steps 2m and 2m+1; q is read
//          in the same order.
//          Result: lane (r = l/16, h = l%16) holds tokens 4r+i, i = 0..3, head h.
//   softmax base 2; the reference max m of each head is shared by the wave and
//          only moves (wave-uniform branch) when a score passes it by
//          kRescaleLog2, so p = 2^(x - m) <= 2^kRescaleLog2 and rescales are rare.
//   PV     on the matrix cores (v_mfma_f32_16x16x16): A = P[head][token] is the
//          QK result layout itself, rounded to the element type; B pairs the
//          16-bit halves of the V rows the lane holds (lane (r, c) holds dims
//          [c*VD, c*VD + VD) of tokens 4r..4r+3). D = O[head][dim]: lane (r, c)
//          holds heads 4r..4r+3, dim c*VD + jb in block jb.
//   piece end: the 4 DPP rows are summed (permlane swaps). A sequence that lies
//          whole inside the range writes its output. A piece of a longer
//          sequence writes its normalised output and base-2 log-sum-exp to the
//          workspace.
// fp8 (OCP e4m3fn) caches: k_scale folds into the score scale and v_scale into
// the output normalisation, both read from device memory once per wave.
//
// Combine kernel (second launch; the kernel boundary makes the pieces visible
// across the XCDs' separate L2s): sequences that cross a range end fold their
// pieces with base-2 LSE weights.
//
// Per-sequence kernel (one launch, for batches of short sequences): one
// workgroup per (sequence, kv head); its waves take every S-th tile of the
// sequence through the same per-wave loop and merge their pieces in LDS, so
// there is no tile scan, no workspace and no second launch.
//
// Several query tokens per sequence (QL, decode with draft tokens): token t
// sits at position L - QL + t and, with the causal mask, sees keys
// [0, L - QL + t] (the bottom-right alignment of the reference's mask).
//
// Workspace (fp32 unless noted), R = num_splits, C = GQ*QL: ws_o [HKV, R, 2, C, HD]
// piece outputs (slot 0 = first piece of a range, slot 1 = last piece when it
// differs), ws_lse [HKV, R, 2, C], ws_s int32 [B + 1] tile prefix sums.
//
// Reference counterpart: paged_decode_v3 split mode and split_combine
// (csrc_native/m1_kernel.cpp:553-888) with the split count of
// integrations/vllm/vllm_plugin.py:271-276; the algorithm (split partials +
// LSE merge) is the same, the work split, data path and numerics are this
// file's own.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "mxfa_device.h"
#include "mxfa_mi355x.h"

namespace mxfa {

constexpr int kTile = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleLog2 = 8.0f;
// Tile prefix sums live in LDS, (B + 1) int32 next to a few bytes of static
// LDS: 16000 sequences keep a workgroup within 64 KB.
constexpr int kMaxBatch = 16000;
constexpr int kMaxCols = 16;      // query tokens x heads per kv head: the 16 MFMA columns
constexpr int kOffOut = 0x40000000;          // a lane offset no descriptor covers

// Tile flags.
constexpr int kFirst = 1;        // first tile of a piece (range start or sequence start)
constexpr int kLast = 2;         // last tile of a piece (range end or sequence end)
constexpr int kSeqStart = 4;     // first tile of its sequence
constexpr int kSeqEnd = 8;       // last tile of its sequence
constexpr int kRangeStart = 16;  // first tile of the range

struct DecodeParams {
  const char *q;
  int64_t q_sb, q_st, q_sh;  // bytes (batch, query token, head)
  const char *k;
  const char *v;
  int64_t sp_bytes;   // page stride
  uint32_t st_bytes;  // token stride
  uint32_t sh_bytes;  // head stride
  const int32_t *bt;
  int64_t bt_stride;
  const int32_t *seqlens;
  char *out;
  int64_t o_sb, o_st, o_sh;  // bytes
  float *ws_o;
  float *ws_lse;
  int32_t *ws_s;
  const float *k_scale;  // fp8 caches: dequantisation scales (nullptr: 1)
  const float *v_scale;
  const float *sinks;    // per query head logit added once to each denominator (nullptr: none)
  float scale_log2;
  float softcap;         // logit soft-capping: s -> softcap * tanh(s / softcap) (0: none)
  const float *alibi;    // per query head ALiBi slope: s -= slope * |query pos - key pos| (nullptr: none)
  int seqlen_add;
  int batch;
  int hkv;
  int gq;
  int ql;      // query tokens per sequence
  int causal;  // mask keys after each query token's position
  int window_left;  // sliding window: token at position i sees keys >= i - window_left (-1: none)
  int heads_per_wg;
  int subs;
  int ps_log2;
  int max_len;  // block_table_width * page_size
  int num_pages;
  int num_ranges;
  int grid_y;  // workgroups along y of the split kernel's grid (gridDim.y, read from here
               // with the other fields rather than from the dispatch's own arguments)
#ifdef MXFA_WAVE_STAMPS
  unsigned long long *stamps;  // profiling builds: kStampWords words per wave (see wave_stamp)
#endif
};

// Launch shape: workgroups of `waves` waves (a kernel instantiation), of which
// heads_per_wg x subs are used (kv head, sub-range); gx x gy workgroups.
struct Grid {
  int waves, heads_per_wg, subs, gx, gy;
  bool short_ranges = false;  // host's bound on tiles per range <= kShortRangeTiles
};

struct CombineParams {
  const float *ws_o;
  const float *ws_lse;
  const int32_t *ws_s;
  char *out;
  int64_t o_sb, o_st, o_sh;  // bytes
  int batch;
  int hq;
  int gq;
  int ql;
  int num_ranges;
  int heads_per_block;  // a power of two; heads_per_block * HD / 4 <= kCombineThreads
  int chunk_parts;      // a power of two <= HD / 32; heads_per_block is 1 when above 1
  const float *sinks;   // as DecodeParams::sinks
#ifdef MXFA_WAVE_STAMPS
  unsigned long long *stamps;  // profiling builds: kStampCombineWords words per block
#endif
};

// Profiling builds (-DMXFA_WAVE_STAMPS) record, per wave (kStampWords words
// each), the real-time clock (100 MHz) at kernel entry [0], after the tile
// scan [1], when the first tiles' loads are issued [2] and at the end [3],
// with the tiles [4], a valid flag [5], the workgroup [6] and the kv head [7];
// then when the lengths have arrived [8], when the range's first sequence is
// known [9], when the first page id has arrived [10] and when the first
// tile's data has arrived [11]. The combine kernel records per block, after
// the waves' words, entry [0], prefix sums read [1], pieces folded [2] and
// end [3]. Other builds compile none of it.
constexpr int kStampWords = 16;
constexpr int kStampWaves = 65536;
constexpr int kStampCombineWords = 4;
constexpr long kStampCombineBase = (long)kStampWaves * kStampWords;
constexpr int kStampCombineBlocks = 65536;

__device__ __forceinline__ unsigned long long wave_clock() {
#ifdef MXFA_WAVE_STAMPS
  return __builtin_amdgcn_s_memrealtime();
#else
  return 0;
#endif
}

__device__ __forceinline__ void wave_stamp(const DecodeParams &p, int slot,
                                           unsigned long long value) {
#ifdef MXFA_WAVE_STAMPS
  const unsigned wave = ((blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  if (p.stamps && (threadIdx.x & 63) == 0 && wave < kStampWaves)
    p.stamps[wave * kStampWords + slot] = value;
#endif
}

// The clock once `dep` exists (profiling builds): the empty asm statement
// uses the value, so the clock read cannot move ahead of its computation.
template <typename V>
__device__ __forceinline__ void wave_stamp_after(const DecodeParams &p, int slot, V dep) {
#ifdef MXFA_WAVE_STAMPS
  asm volatile("" ::"v"(dep));
  wave_stamp(p, slot, wave_clock());
#endif
}

// Combine-kernel stamps (profiling builds): thread 0 of each block, once `dep` exists.
template <typename V>
__device__ __forceinline__ void block_stamp_after(const CombineParams &c, int slot, V dep) {
#ifdef MXFA_WAVE_STAMPS
  asm volatile("" ::"v"(dep));
  if (c.stamps && threadIdx.x == 0 && blockIdx.x < kStampCombineBlocks)
    c.stamps[blockIdx.x * kStampCombineWords + slot] = wave_clock();
#endif
}

// Block tables and lengths are read-only for the whole call; reading them
// through the constant address space lets wave-uniform lookups use scalar
// (SMEM) loads even inside loops that also store results.
typedef const __attribute__((address_space(4))) int32_t *ConstI32;
typedef const __attribute__((address_space(4))) float *ConstF32;

__device__ __forceinline__ ConstI32 as_const(const int32_t *p) { return (ConstI32)p; }

__device__ __forceinline__ int rfl(int x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ __forceinline__ int seq_len_of(const int32_t *seqlens, int b, int add, int max_len) {
  int L = as_const(seqlens)[b] + add;
  L = L < 0 ? 0 : L;
  return L > max_len ? max_len : L;
}

// First tile of a sequence of L keys that any of its QL query tokens sees: the
// earliest token (position L - QL) sees keys >= L - QL - window_left. Tiles are
// aligned to the sequence start; with no window this is tile 0.
__device__ __forceinline__ int first_tile_of(int L, int ql, int window_left) {
  if (window_left < 0) return 0;
  const int first_key = L - ql - window_left;
  return first_key > 0 ? first_key / kTile : 0;
}

// Tiles of a sequence of L keys inside the window (L > 0: at least one).
__device__ __forceinline__ int tiles_of(int L, int ql, int window_left) {
  return (L + kTile - 1) / kTile - first_tile_of(L, ql, window_left);
}

// First tile of range r out of R over NT tiles, and the range holding tile t.
// Both stay in 32-bit unsigned division while the product fits (every
// benchmark shape: r * NT < 2^31), which is a few instructions where the
// 64-bit division is a long software sequence on the prologue's critical path.
__device__ __forceinline__ int range_lo(int r, int R, int NT) {
  const int64_t x = (int64_t)r * NT;
  if (x < 0x7fffffff) return (int)((uint32_t)x / (uint32_t)R);
  return (int)(x / R);
}
__device__ __forceinline__ int range_of(int t, int R, int NT) {
  const int64_t x = ((int64_t)t + 1) * R - 1;
  if (x < 0x7fffffff) return (int)((uint32_t)x / (uint32_t)NT);
  return (int)(x / NT);
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

// PV on the matrix cores, v_mfma_f32_16x16x16: A = P[head][token] is the QK
// result layout itself (lane (r, h) holds tokens 4r..4r+3 of head h), packed to
// the element type; B = V[token][dim], lane (r, c) supplying tokens 4r..4r+3 of
// one dim per block; D = O[head][dim]. Element packing keeps k order: the low
// half of the first register is token 4r.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Dot product of two packed pairs of the element type, accumulated in fp32
// (v_dot2c_f32_bf16 / v_dot2c_f32_f16).
template <typename T>
struct Dot2;
template <>
struct Dot2<BF16> {
  static __device__ __forceinline__ float run(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
  }
};
template <>
struct Dot2<F16> {
  static __device__ __forceinline__ float run(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                  false);
  }
};
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct PvMfma;
template <>
struct PvMfma<BF16> {
  static __device__ __forceinline__ f32x4 run(uint2 a, uint2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                      __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t round(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
  static __device__ __forceinline__ float widen(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
  }
};
template <>
struct PvMfma<F16> {
  static __device__ __forceinline__ f32x4 run(uint2 a, uint2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint16_t round(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
  static __device__ __forceinline__ float widen(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
  }
};

// Two OCP e4m3fn values (bytes 2*Hi, 2*Hi+1 of w) to a packed pair of the
// element type. Exact: every e4m3fn value is representable in fp16 and bf16
// (scale 1 leaves the exponent alone).
template <typename T>
struct Fp8Widen;
template <>
struct Fp8Widen<BF16> {
  template <bool Hi>
  static __device__ __forceinline__ uint32_t pair(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, Hi));
  }
};
template <>
struct Fp8Widen<F16> {
  template <bool Hi>
  static __device__ __forceinline__ uint32_t pair(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, Hi));
  }
};

// 8 e4m3fn bytes (two words) to 8 elements (one MFMA operand), in byte order.
template <typename T>
__device__ __forceinline__ uint4 widen8(uint32_t w0, uint32_t w1) {
  return make_uint4(Fp8Widen<T>::template pair<false>(w0), Fp8Widen<T>::template pair<true>(w0),
                    Fp8Widen<T>::template pair<false>(w1), Fp8Widen<T>::template pair<true>(w1));
}

// 16-bit element j of a V fragment word list, paired from two tokens.
__device__ __forceinline__ uint32_t pair_halves(uint32_t lo_tok, uint32_t hi_tok, int odd) {
  return __builtin_amdgcn_perm(hi_tok, lo_tok, odd ? 0x07060302u : 0x05040100u);
}

// BYTES contiguous bytes of one lane (4, 8, 16 or 32), as words.
template <int BYTES>
struct Frag {
  static constexpr int W = BYTES / 4;
  uint32_t w[W];
  template <int Aux>
  __device__ __forceinline__ void load_buf(__amdgpu_buffer_rsrc_t r, int off) {
    if constexpr (BYTES == 4) {
      w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, Aux);
    } else if constexpr (BYTES == 8) {
      const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, Aux);
      w[0] = v.x;
      w[1] = v.y;
    } else {
#pragma unroll
      for (int i = 0; i < W / 4; ++i) {
        const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, Aux);
        w[4 * i] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
      }
    }
  }
  __device__ __forceinline__ void load_ptr(const char *ptr) {
    if constexpr (BYTES == 4) {
      w[0] = load_stream4(ptr);
    } else if constexpr (BYTES == 8) {
      const uint2 v = load_stream8(ptr);
      w[0] = v.x;
      w[1] = v.y;
    } else {
#pragma unroll
      for (int i = 0; i < W / 4; ++i) {
        const uint4 v = load_stream16(ptr + 16 * i);
        w[4 * i] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
      }
    }
  }
};

// f(std::integral_constant<int, I>) for I = 0 .. N-1, unrolled at compile time.
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Lane c of each 16-lane row takes the value of lane c ^ 8 (row_ror:8).
__device__ __forceinline__ uint32_t row_swap8(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xf, 0xf, false);
}

// tanh(y) = 1 - 2 / (e^(2y) + 1) from the hardware exp2 and reciprocal; exact
// saturation to +-1 for large |y|, absolute error ~1e-7 near 0.
__device__ __forceinline__ float tanh_exp2(float y) {
  return 1.f - 2.f * __builtin_amdgcn_rcpf(fast_exp2(2.f * kLog2e * y) + 1.f);
}

// Every lane takes the value of lane H of its own 16-lane row (row_newbcast:H).
template <int H>
__device__ __forceinline__ float row_bcast(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), kDppRowNewBcast0 + H, 0xf, 0xf, false));
}

// Value of head 4*row + I from a per-head quantity held by column h of every
// DPP row (the score layout), for HR head rows (GQ <= 4 HR). Rows past HR get
// the value of row 0's head (unused). DPP moves only: no LDS round trip, so no
// wait on the scalar page-id loads in flight.
template <int HR, int I>
__device__ __forceinline__ float head_of_row(float x, int row) {
  float v = row_bcast<I>(x);
  if constexpr (HR > 1) v = row == 1 ? row_bcast<4 + I>(x) : v;
  if constexpr (HR > 2) {
    v = row == 2 ? row_bcast<8 + I>(x) : v;
    v = row == 3 ? row_bcast<12 + I>(x) : v;
  }
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves only (no
// LDS permutes): a Hillis-Steele scan inside each 16-lane row (row_shr 1, 2,
// 4, 8), then the row totals carried across rows (row_bcast:15 into rows 1
// and 3, row_bcast:31 into rows 2 and 3). Lanes a move leaves unwritten add 0.
__device__ __forceinline__ int wave_scan_incl(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, kDppRowShr0 + 1, 0xf, 0xf, true);
  x += __builtin_amdgcn_update_dpp(0, x, kDppRowShr0 + 2, 0xf, 0xf, true);
  x += __builtin_amdgcn_update_dpp(0, x, kDppRowShr0 + 4, 0xf, 0xf, true);
  x += __builtin_amdgcn_update_dpp(0, x, kDppRowShr0 + 8, 0xf, 0xf, true);
  x += __builtin_amdgcn_update_dpp(0, x, kDppRowBcast15, 0xa, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, kDppRowBcast31, 0xc, 0xf, false);
  return x;
}

// Exclusive prefix sum of per-sequence tile counts into s[0..B] (LDS), all
// threads (seqlens and B are the kernel's preloaded leading arguments, equal
// to p.seqlens and p.batch). The lengths are read from memory once, eight loads in flight per
// thread: the first pass parks each tile count in s[b], the second turns them
// into prefix sums in place (up to one sequence per thread, the count stays in a
// register instead). Without a window (kWindow false) every sequence starts at
// its tile 0. Returns the tile total s[B] (from the wave totals, so no thread
// reads s[B] back).
template <int kThreads, bool kWindow>
__device__ __forceinline__ int tile_prefix(const DecodeParams &p, const int32_t *seqlens, int B,
                                           int32_t *s, int *wave_tot) {
  constexpr int kWaves = kThreads / 64;
  constexpr int kBatchLoads = 8;
  const int per = (B + kThreads - 1) / kThreads;
  const int b0 = threadIdx.x * per;
  int local = 0;
  if (per == 1) {  // up to one sequence per thread (B <= kThreads): one load
    const int b = b0;
    if (b < B) {
      const int L = seq_len_of(seqlens, b, p.seqlen_add, p.max_len);
      local = kWindow ? tiles_of(L, p.ql, p.window_left) : (L + kTile - 1) / kTile;
    }
  }
  for (int i0 = 0; per > 1 && i0 < per; i0 += kBatchLoads) {
    // Branch-free, so a thread's loads all go out together (entries past the
    // batch read sequence 0 and count nothing).
    int n[kBatchLoads];
#pragma unroll
    for (int j = 0; j < kBatchLoads; ++j) {
      const int b = b0 + i0 + j;
      const bool live = i0 + j < per && b < B;
      const int L = seq_len_of(seqlens, live ? b : 0, p.seqlen_add, p.max_len);
      const int t = kWindow ? (L > 0 ? tiles_of(L, p.ql, p.window_left) : 0)
                            : (L + kTile - 1) / kTile;
      n[j] = live ? t : 0;
    }
#pragma unroll
    for (int j = 0; j < kBatchLoads; ++j) {
      const int b = b0 + i0 + j;
      if (i0 + j < per && b < B) {
        s[b] = n[j];
        local += n[j];
      }
    }
  }
  wave_stamp_after(p, 8, local);
  // Inclusive scan of `local` across the workgroup.
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int x = wave_scan_incl(local);
  if (lane == 63) wave_tot[wave] = x;
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int t = wave_tot[w];
    base += w < wave ? t : 0;
    total += t;
  }
  int run = base + x - local;  // exclusive prefix of this thread's first element
  if (per == 1) {
    if (b0 < B) s[b0] = run;
  } else {
    for (int i = 0; i < per; ++i) {  // each thread rewrites only its own entries
      const int b = b0 + i;
      if (b < B) {
        const int n = s[b];
        s[b] = run;
        run += n;
      }
    }
  }
  if (threadIdx.x == kThreads - 1) s[B] = total;
  __syncthreads();
  return total;
}

// Zero output rows of sequence b for this workgroup's kv heads [kv0, kv1):
// thread i writes 8-byte piece i % F of rows i / F, i / F + kThreads / F, ...
// of every query token (F = HD / 4 pieces per row; no run-time division, so
// nothing is set up before the caller knows a sequence is empty).
template <int HD, int kThreads>
__device__ __forceinline__ void zero_rows(const DecodeParams &p, int b, int kv0, int nh) {
  constexpr int F = HD / 4;
  static_assert(kThreads % F == 0, "whole rows per pass");
  char *row = p.out + b * p.o_sb + (int64_t)kv0 * p.gq * p.o_sh + (threadIdx.x % F) * 8;
  for (int t = 0; t < p.ql; ++t)
    for (int h = threadIdx.x / F; h < nh; h += kThreads / F)
      *reinterpret_cast<uint2 *>(row + t * p.o_st + h * p.o_sh) = make_uint2(0u, 0u);
}

// Empty sequences (no tiles) get zero output; sequence b is cleared by the
// workgroups with blockIdx.y == b % grid_y, each for its own kv heads.
template <int HD, int kThreads>
__device__ __forceinline__ void zero_empty(const DecodeParams &p, const int32_t *s) {
  const int kv0 = blockIdx.x * p.heads_per_wg;
  const int nh = (min(kv0 + p.heads_per_wg, p.hkv) - kv0) * p.gq;
  for (int b = blockIdx.y; b < p.batch; b += p.grid_y)
    if (s[b + 1] == s[b]) zero_rows<HD, kThreads>(p, b, kv0, nh);
}

// Batches of up to kWaveScanMax sequences skip the LDS tile scan: every wave
// loads the lengths itself, kPer consecutive sequences per lane, and scans the
// tile counts with DPP (wave_tile_scan), so no wave waits on a barrier or an
// LDS round trip before it looks for its range's first sequence. One sequence
// per lane up to 64 sequences, four up to 256: the four-per-lane scan costs
// 0.2 us more per call at B <= 64 (measured on MI355X), so each batch size
// takes the smaller one. kWaveScan template arguments: 0 (the LDS scan), 1, 4.
constexpr int kWaveScanMax1 = 64;
constexpr int kWaveScanMax = 4 * 64;
inline int wave_scan_per_lane(int batch) {
  return batch <= kWaveScanMax1 ? 1 : batch <= kWaveScanMax ? 4 : 0;
}

// The wave-local scan state. Lane l holds sequences b = kPer * l + j (j <
// kPer): the clamped lengths len0.., the exclusive tile prefix sums pre0..
// (S_b), and incl = S_{b+1} of its last one. Sequences past the batch count
// length 0, so their S is the tile total. Every query takes a wave-uniform
// sequence b < B. Named fields rather than arrays: an array indexed by j is
// kept in memory (private, or LDS by promotion), not in registers.
template <int kPer>
struct WaveScan;

template <>
struct WaveScan<1> {
  int len0 = 0, pre0 = 0, incl = 0;
  __device__ __forceinline__ int start(int b) const { return __builtin_amdgcn_readlane(pre0, b); }
  __device__ __forceinline__ int end(int b) const { return __builtin_amdgcn_readlane(incl, b); }
  __device__ __forceinline__ int length(int b) const { return __builtin_amdgcn_readlane(len0, b); }
  // The sequence holding tile t (0 <= t < tile total): the largest b < B with
  // S_b <= t; the lanes that pass form a prefix (S is nondecreasing).
  __device__ __forceinline__ int find(int t, int B) const {
    const int lane = threadIdx.x & 63;
    return __builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < B && pre0 <= t)) - 1;
  }
};

template <>
struct WaveScan<4> {
  int len0 = 0, len1 = 0, len2 = 0, len3 = 0;
  int pre0 = 0, pre1 = 0, pre2 = 0, pre3 = 0;
  int incl = 0;

  __device__ __forceinline__ static int sel(int j, int a0, int a1, int a2, int a3) {
    return j == 0 ? a0 : j == 1 ? a1 : j == 2 ? a2 : a3;
  }
  __device__ __forceinline__ int start(int b) const {
    return __builtin_amdgcn_readlane(sel(b & 3, pre0, pre1, pre2, pre3), b >> 2);
  }
  __device__ __forceinline__ int end(int b) const {
    return __builtin_amdgcn_readlane(sel(b & 3, pre1, pre2, pre3, incl), b >> 2);
  }
  __device__ __forceinline__ int length(int b) const {
    return __builtin_amdgcn_readlane(sel(b & 3, len0, len1, len2, len3), b >> 2);
  }
  // As above: the last lane whose first S passes holds b, and of its own S
  // those that pass form a prefix too (entries past the batch hold the total,
  // which none do).
  __device__ __forceinline__ int find(int t, int B) const {
    const int lane = threadIdx.x & 63;
    const int l =
        __builtin_popcountll(__builtin_amdgcn_ballot_w64(4 * lane < B && pre0 <= t)) - 1;
    const int j = (__builtin_amdgcn_readlane(pre1, l) <= t ? 1 : 0) +
                  (__builtin_amdgcn_readlane(pre2, l) <= t ? 1 : 0) +
                  (__builtin_amdgcn_readlane(pre3, l) <= t ? 1 : 0);
    return 4 * l + j;
  }
};

// Clamped length of sequence b (0 past the batch), and the tile count of a length.
__device__ __forceinline__ int clamp_len(const DecodeParams &p, int raw, int b, int B) {
  int L = raw + p.seqlen_add;
  L = L < 0 ? 0 : (L > p.max_len ? p.max_len : L);
  return b < B ? L : 0;
}
template <bool kWindow>
__device__ __forceinline__ int tile_count(const DecodeParams &p, int L) {
  return kWindow ? (L > 0 ? tiles_of(L, p.ql, p.window_left) : 0) : (L + kTile - 1) / kTile;
}

// Fills `w` for the batch and returns the tile total. The length loads need
// only the preloaded leading arguments, so they are issued (together) before
// any wait on the parameter struct.
template <bool kWindow>
__device__ __forceinline__ int wave_tile_scan(const DecodeParams &p, const int32_t *seqlens, int B,
                                              WaveScan<1> &w) {
  const int b = threadIdx.x & 63;
  w.len0 = clamp_len(p, as_const(seqlens)[b < B ? b : B - 1], b, B);
  const int n = tile_count<kWindow>(p, w.len0);
  wave_stamp_after(p, 8, n);
  w.incl = wave_scan_incl(n);
  w.pre0 = w.incl - n;
  return __builtin_amdgcn_readlane(w.incl, 63);
}
template <bool kWindow>
__device__ __forceinline__ int wave_tile_scan(const DecodeParams &p, const int32_t *seqlens, int B,
                                              WaveScan<4> &w) {
  const int b0 = 4 * (threadIdx.x & 63);
  const int r0 = as_const(seqlens)[b0 < B ? b0 : B - 1];
  const int r1 = as_const(seqlens)[b0 + 1 < B ? b0 + 1 : B - 1];
  const int r2 = as_const(seqlens)[b0 + 2 < B ? b0 + 2 : B - 1];
  const int r3 = as_const(seqlens)[b0 + 3 < B ? b0 + 3 : B - 1];
  w.len0 = clamp_len(p, r0, b0, B);
  w.len1 = clamp_len(p, r1, b0 + 1, B);
  w.len2 = clamp_len(p, r2, b0 + 2, B);
  w.len3 = clamp_len(p, r3, b0 + 3, B);
  const int n0 = tile_count<kWindow>(p, w.len0), n1 = tile_count<kWindow>(p, w.len1);
  const int n2 = tile_count<kWindow>(p, w.len2), n3 = tile_count<kWindow>(p, w.len3);
  const int run = n0 + n1 + n2 + n3;  // this lane's tiles
  wave_stamp_after(p, 8, run);
  w.incl = wave_scan_incl(run);
  w.pre0 = w.incl - run;
  w.pre1 = w.pre0 + n0;
  w.pre2 = w.pre1 + n1;
  w.pre3 = w.pre2 + n2;
  return __builtin_amdgcn_readlane(w.incl, 63);
}

// zero_empty for the wave-local scan (every wave holds the whole scan).
template <int HD, int kThreads, int kPer>
__device__ __forceinline__ void zero_empty_wave(const DecodeParams &p, const WaveScan<kPer> &w) {
  const int kv0 = blockIdx.x * p.heads_per_wg;
  const int nh = (min(kv0 + p.heads_per_wg, p.hkv) - kv0) * p.gq;
  for (int b = blockIdx.y; b < p.batch; b += p.grid_y)
    if (w.end(b) == w.start(b)) zero_rows<HD, kThreads>(p, b, kv0, nh);
}

// The prefix sums s[0..B] into the workspace (workgroup (0, 0), first wave).
__device__ __forceinline__ void store_prefix_wave(const DecodeParams &p, const WaveScan<1> &w,
                                                  int B, int NT) {
  const int b = threadIdx.x & 63;
  if (b < B) p.ws_s[b] = w.pre0;
  if (b == 0) p.ws_s[B] = NT;
}
__device__ __forceinline__ void store_prefix_wave(const DecodeParams &p, const WaveScan<4> &w,
                                                  int B, int NT) {
  const int b0 = 4 * (threadIdx.x & 63);
  if (b0 < B) p.ws_s[b0] = w.pre0;
  if (b0 + 1 < B) p.ws_s[b0 + 1] = w.pre1;
  if (b0 + 2 < B) p.ws_s[b0 + 2] = w.pre2;
  if (b0 + 3 < B) p.ws_s[b0 + 3] = w.pre3;
  if (b0 == 0) p.ws_s[B] = NT;
}

// Sum / max over the 4 DPP rows of the wave (lanes l, l^16, l^32, l^48); every
// lane receives the result.
__device__ __forceinline__ float rows_sum(float x) {
  const auto a =
      __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto c =
      __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}
__device__ __forceinline__ float rows_max(float x) {
  const auto a =
      __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto c =
      __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
}

// VD fp32 values times `scale`, rounded once to the element type, to 8-byte aligned dst.
template <int VD, typename E>
__device__ __forceinline__ void store_row(char *dst, const float (&v)[VD], float scale) {
  uint32_t w[VD / 2];
#pragma unroll
  for (int j = 0; j < VD / 2; ++j)
    w[j] = (uint32_t)E::narrow(v[2 * j] * scale) |
           ((uint32_t)E::narrow(v[2 * j + 1] * scale) << 16);
#pragma unroll
  for (int j = 0; j < VD / 4; ++j)
    *reinterpret_cast<uint2 *>(dst + 8 * j) = make_uint2(w[2 * j], w[2 * j + 1]);
}

// Scalar description of one tile, built NBUF tiles ahead of the math.
struct Tile {
  int b;      // sequence
  int tok0;   // first token of the tile within the sequence
  int valid;  // tokens of the tile that exist (0: padding past the range end)
  int rem;    // keys from the tile start to the sequence end (0: padding)
  int flags;
  int pg;  // page id (block-table entry), page-uniform tiles only
};

// One wave: the tiles [lo, hi) of kv head kvh, range rr. HR = DPP rows
// holding used columns (GQ*QL <= 4 HR), T = element type of q, out and the MFMA
// operands, kF8 = e4m3fn caches. Accumulator lane (r, c) holds columns
// 4r..4r+3, dims c*VD + jb in block jb.
//
// kSeq (per-sequence workgroups): p describes one sequence (batch 1), the wave
// takes its tiles lo, lo + stride, ... below hi = the sequence's tile count,
// and writes its one piece (normalised output, base-2 LSE) to LDS at lds_o
// [C][HD] and lds_lse [C] for the workgroup to merge; s_tiles is not read.
// Without a window and with page-uniform tiles, pg_first is the page id of
// tile lo, already read by the caller.
//
// kProbe (the streaming probe): the same tile walk and loads, but each tile
// only XORs the words it loaded into the returned value, with no attention
// math and no output; other instantiations return 0.
template <int HD, int HR, typename T, bool kF8, bool kLanePages, int NBUF, bool kExtras,
          bool kSeq, bool kBalance = false, bool kProbe = false, int kWaveLocal = 0,
          int kValuG = 0>
__device__ __forceinline__ uint32_t run_range(const DecodeParams &p, const int32_t *s_tiles,
                                              int kvh, int rr, int lo, int hi, int stride,
                                              float *lds_o, float *lds_lse, int pg_first = 0,
                                              WaveScan<kWaveLocal == 4 ? 4 : 1> wsc = {}) {
  const int tstep = kSeq ? stride : 1;  // tile index step between the wave's tiles
  using E = Elem<T>;
  constexpr int NCH = HD / 32;               // MFMA steps over the head dim
  constexpr int NKL = kF8 ? HD / 64 : NCH;   // 16-byte K loads per lane and tile
  constexpr int VD = HD / 16;                // V elements per lane
  constexpr int VB = kF8 ? VD : 2 * VD;      // V bytes per lane and token
  constexpr int U = 4;                       // V tokens per lane (token 4r+u in DPP row r)
  constexpr int NPG = kLanePages ? 1 + U : 1;
  // 8-byte V slots (128-byte rows): lanes c and c^8 of a row load 16 bytes
  // (slots 2(c&7), 2(c&7)+1) of two tokens each and swap halves, so a tile
  // takes two 16-byte loads per lane instead of four 8-byte ones. Lane c then
  // holds slot 2(c&7) + (c>>3).
  constexpr bool kShareV = VB == 8 && !kLanePages;
  const int B = p.batch;
  const int gq = p.gq;
  const int nc = gq * p.ql;  // used columns

  const int lane = threadIdx.x & 63;
  const int row = lane >> 4;  // DPP row
  const int col = lane & 15;  // column (score layout) / V column
  const int ps_mask = (1 << p.ps_log2) - 1;
  const uint32_t st = p.st_bytes;
  const uint64_t head_off = (uint64_t)kvh * p.sh_bytes;
  float c = p.scale_log2;
  float v_scale = 1.f;
  if constexpr (kF8) {
    if (p.k_scale) c *= ((ConstF32)p.k_scale)[0];
    if (p.v_scale) v_scale = ((ConstF32)p.v_scale)[0];
  }
  const int ns = p.num_ranges;  // workspace stride
  // kExtras: a sliding window, soft-capping, ALiBi and/or sinks are on (the
  // loop without them carries no trace of any). Soft-capping of the scaled score s = acc * scale *
  // k_scale: the base-2 score becomes cap_out * tanh(acc * cap_in) (no
  // division by the scale, so scale 0 stays 0).
  const bool capped = kExtras && p.softcap > 0.f;
  const float cap_in = capped ? c / (kLog2e * p.softcap) : 0.f;
  const float cap_out = p.softcap * kLog2e;

  // Lane offsets inside a tile: K in the MFMA A layout, V row-contiguous, q as
  // the MFMA B operand (columns >= GQ*QL read nothing). For fp8 caches step
  // 2m + s of lane row r covers dims 64m + 16r + 8s .. +7; q follows it.
  // kValuG > 0: QK on the VALU for the first kValuG columns (the rest are
  // unused). Lane (r, c) then holds token 4r + c/4, 16-byte chunk c%4 of each
  // 64-byte step: the same addresses per load instruction as the MFMA
  // layout's token c, chunk r.
  constexpr bool kValu = kValuG > 0 && !kF8 && !kLanePages && !kProbe;
  const int k_off = kValu ? (4 * row + (col >> 2)) * (int)st + (col & 3) * 16
                          : col * (int)st + row * 16;
  int v_off[U];
#pragma unroll
  for (int u = 0; u < U; ++u) v_off[u] = (4 * row + u) * (int)st + col * VB;
  // Column col = query token ct, group head cg; the causal mask hides the
  // last c_hide keys of the sequence from it, and the window all keys more
  // than c_reach from the sequence end. Key k of a sequence of L keys is seen
  // when c_hide < L - k <= c_reach.
  const int ct = col / gq, cg = col - (col / gq) * gq;
  const int c_hide = p.causal ? p.ql - 1 - ct : 0;
  const int c_reach = p.window_left >= 0 ? p.ql - ct + p.window_left : 0x3fffffff;
  // ALiBi: base-2 slope of this lane's column; the query of column (ct, cg)
  // sits QL - ct keys before the sequence end, so key k (L - k = rel) is
  // |rel - (QL - ct)| positions away from it.
  const bool alibi = kExtras && p.alibi != nullptr;
  const float slope2 =
      alibi && col < nc ? ((ConstF32)p.alibi)[kvh * gq + cg] * kLog2e : 0.f;
  const int qdist = p.ql - ct;
  const int q_off =
      col < nc ? ct * (int)p.q_st + cg * (int)p.q_sh + row * (kF8 ? 32 : 16) : kOffOut;
  const int q_bytes = (p.ql - 1) * (int)p.q_st + (gq - 1) * (int)p.q_sh + HD * 2;
  auto q_step = [](int cc) { return kF8 ? (cc >> 1) * 128 + (cc & 1) * 16 : cc * 64; };

  // Sequence holding tile lo: the largest b < B with s[b] <= lo (then
  // s[b+1] > lo). s is nondecreasing and s[0] = 0 <= lo, so the lanes whose
  // probe passes form a prefix: each round narrows [a, a + n) to one of 64
  // steps, down to at most 63 candidates, which one last round settles (one
  // round for B < 64, two up to B = 4032, three up to 16000).
  // Cursor of the tile builder (runs NBUF tiles ahead of the math): the
  // sequence pb and its tiles [p_start, p_end). Without a window every
  // sequence starts at its tile 0, so the first page id does not wait for the
  // length.
  int pb = 0, p_start = 0, p_end = hi;
  // kWaveLocal (split kernel, 1 or 4 sequences per lane): the wave-local scan wsc
  // gives the prefix sums and lengths; s_tiles is not read.
  constexpr bool wave_local = kWaveLocal != 0 && !kSeq;
  if constexpr (wave_local) {
    pb = wsc.find(lo, B);
    p_start = wsc.start(pb);
    p_end = wsc.end(pb);
    wave_stamp_after(p, 9, pb);
  } else if constexpr (!kSeq) {
    int a = 0, n = B;  // s[a] <= lo < s[a + n]
    while (n > 63) {
      const int step = (n + 63) >> 6;
      const int idx = a + lane * step;
      const bool ok = idx < a + n && s_tiles[idx] <= lo;
      const int cnt = __builtin_popcountll(__builtin_amdgcn_ballot_w64(ok));
      const int na = a + (cnt - 1) * step;
      n = min(step, a + n - na);
      a = na;
    }
    // Last round, n <= 63: lane l holds s[min(a + l, B)], so s[pb] and
    // s[pb + 1] come from two lanes rather than from another LDS read.
    a = rfl(a);
    n = rfl(n);
    const int v = s_tiles[min(a + lane, B)];
    const int c = __builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < n && v <= lo));
    pb = a + c - 1;
    p_start = __builtin_amdgcn_readlane(v, c - 1);
    p_end = __builtin_amdgcn_readlane(v, c);
    wave_stamp_after(p, 9, pb);
  }
  ConstI32 p_bt = as_const(p.bt + (int64_t)pb * p.bt_stride);
  // Split kernel without a window: the first tile's page id needs only
  // p_start, so its load goes out before the length's (the scheduling barrier
  // keeps that order) and the two share one round trip. Issued after, it
  // would wait for the length: the compiler uses the length at once. Tile lo
  // lies inside sequence pb (lo < p_end), so the position is in the table row;
  // the clamp keeps the read there whatever the lengths say.
  if constexpr (!kSeq && !kLanePages && !kExtras) {
    pg_first = p_bt[min((lo - p_start) * kTile, p.max_len - 1) >> p.ps_log2];
    __builtin_amdgcn_sched_barrier(0);
  }
  int p_len = wave_local ? wsc.length(pb) : seq_len_of(p.seqlens, pb, p.seqlen_add, p.max_len);
  int p_first = kExtras ? first_tile_of(p_len, p.ql, p.window_left) : 0;  // tile at p_start

  // Per-lane page ids are computed into a local array and copied to `lpg` at
  // one point that both the padding and the real tile reach: stores to `lpg`
  // from two branches were merged by the compiler into a store through a
  // selected address, which kept the register sets in private memory.
  auto make_tile = [&](int t, Tile &d, int (&lpg)[NPG]) {
    // kSeq: the page id is read before the range test, clamped into the
    // table row, so without a window it does not wait for the length.
    int pg_early = 0;
    if constexpr (kSeq && !kLanePages)
      pg_early = p_bt[min((t - p_start + p_first) * kTile, p.max_len - 1) >> p.ps_log2];
    int lp[NPG];
#pragma unroll
    for (int i = 0; i < NPG; ++i) lp[i] = 0;
    if (t >= hi) {
      d.b = pb;
      d.tok0 = 0;
      d.valid = 0;
      d.rem = 0;
      d.flags = 0;
      d.pg = 0;
#pragma unroll
      for (int i = 0; i < NPG; ++i) lpg[i] = lp[i];
      return;
    }
    if constexpr (!kSeq) {
      if (t >= p_end) {  // next sequence with tiles (rare, wave-uniform)
        do {
          ++pb;
          p_start = p_end;
          p_end = wave_local ? wsc.end(pb) : rfl(s_tiles[pb + 1]);
        } while (t >= p_end);
        p_len = wave_local ? wsc.length(pb) : seq_len_of(p.seqlens, pb, p.seqlen_add, p.max_len);
        p_first = kExtras ? first_tile_of(p_len, p.ql, p.window_left) : 0;
        p_bt = as_const(p.bt + (int64_t)pb * p.bt_stride);
      }
    }
    d.b = pb;
    d.tok0 = (t - p_start + p_first) * kTile;
    d.rem = p_len - d.tok0;
    d.valid = min(kTile, d.rem);
    if constexpr (kSeq) {  // one piece per wave, merged in LDS
      d.flags = (t == lo ? kFirst : 0) | (t + tstep >= hi ? kLast : 0);
    } else {
      const bool seq_start = t == p_start, seq_end = d.tok0 + kTile >= p_len;
      d.flags = ((t == lo || seq_start) ? kFirst : 0) | ((t == hi - 1 || seq_end) ? kLast : 0) |
                (seq_start ? kSeqStart : 0) | (seq_end ? kSeqEnd : 0) |
                (t == lo ? kRangeStart : 0);
    }
    if constexpr (kLanePages) {
      // Per-lane page ids: [0] for this lane's K token, [1+u] for its V tokens.
      // Token positions clamp to the last valid token.
      const int last = d.valid - 1;
      lp[0] = p_bt[(d.tok0 + min(col, last)) >> p.ps_log2];
#pragma unroll
      for (int u = 0; u < U; ++u)
        lp[1 + u] = p_bt[(d.tok0 + min(4 * row + u, last)) >> p.ps_log2];
      d.pg = 0;
    } else {
      d.pg = kSeq ? pg_early : p_bt[d.tok0 >> p.ps_log2];
    }
#pragma unroll
    for (int i = 0; i < NPG; ++i) lpg[i] = lp[i];
  };

  // In the split kernel the page id is read one pipeline step before issue()
  // uses it; the empty asm keeps the clamp (and so the wait for that read)
  // here instead of letting the compiler clamp it right after the read and
  // stall there. (The per-sequence kernel measured better without it.)
  auto clamp_page = [&](int pg) -> int {
    if constexpr (!kSeq) {
      if constexpr (kLanePages)
        asm volatile("" : "+v"(pg));  // per-lane page ids
      else
        asm volatile("" : "+s"(pg));
    }
    pg = pg < 0 ? 0 : pg;
    return pg >= p.num_pages ? p.num_pages - 1 : pg;
  };

  struct Set {
    uint4 k[NKL];
    Frag<VB> v[kShareV ? 1 : U];  // kShareV: unused
    uint4 vr[kShareV ? 2 : 1];    // kShareV: tokens 4r+2h, 4r+2h+1, 16 bytes each
    uint4 q[NCH];
    int lpg[NPG];
    Tile d;
  };

  auto issue = [&](Set &s) {
    const Tile &d = s.d;
    // rfl: the size is wave-uniform; without it the compiler may keep it in a
    // VGPR and wrap the q loads in a loop over distinct descriptors.
    const __amdgpu_buffer_rsrc_t rq =
        make_srd(p.q + (int64_t)d.b * p.q_sb + (int64_t)kvh * gq * p.q_sh,
                 rfl((d.flags & kFirst) ? q_bytes : 0));
    if (d.flags & kFirst) {  // wave-uniform; q is loaded once per piece
#pragma unroll
      for (int cc = 0; cc < NCH; ++cc) s.q[cc] = buf_load16<0>(rq, q_off + q_step(cc));
    }
    if constexpr (!kLanePages) {
      const uint64_t tile_off = (uint64_t)(uint32_t)clamp_page(d.pg) * (uint64_t)p.sp_bytes +
                                (uint64_t)(d.tok0 & ps_mask) * st + head_off;
      const int bytes = d.valid > 0 ? (d.valid - 1) * (int)st + HD * (kF8 ? 1 : 2) : 0;
      const __amdgpu_buffer_rsrc_t rk = make_srd(p.k + tile_off, bytes);
      const __amdgpu_buffer_rsrc_t rv = make_srd(p.v + tile_off, bytes);
#pragma unroll
      for (int cc = 0; cc < NKL; ++cc) s.k[cc] = buf_load16<kAuxStream>(rk, k_off + cc * 64);
      if constexpr (kShareV) {
        const int t0 = 4 * row + 2 * (col >> 3);
        const int vo = (col & 7) * 16;
        s.vr[0] = buf_load16<kAuxStream>(rv, t0 * (int)st + vo);
        s.vr[1] = buf_load16<kAuxStream>(rv, (t0 + 1) * (int)st + vo);
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u) s.v[u].template load_buf<kAuxStream>(rv, v_off[u]);
      }
    } else {
      // Lane pages: every lane addresses its own page; positions past the
      // sequence end were clamped to its last token (their scores are masked).
      const int last = d.valid > 0 ? d.valid - 1 : 0;
      {
        const int pos = d.tok0 + min(col, last);
        const uint64_t off = (uint64_t)(uint32_t)clamp_page(s.lpg[0]) * (uint64_t)p.sp_bytes +
                             (uint64_t)(pos & ps_mask) * st + head_off + row * 16;
#pragma unroll
        for (int cc = 0; cc < NKL; ++cc) s.k[cc] = load_stream16(p.k + off + cc * 64);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int pos = d.tok0 + min(4 * row + u, last);
        const uint64_t off = (uint64_t)(uint32_t)clamp_page(s.lpg[1 + u]) * (uint64_t)p.sp_bytes +
                             (uint64_t)(pos & ps_mask) * st + head_off + col * VB;
        s.v[u].load_ptr(p.v + off);
      }
    }
  };

  // Running state of the current piece.
  float m = -INFINITY;  // reference max (base 2) of column `col`, same in every row
  float dsum = 0.f;     // partial denominator of column `col` over this row's tokens
  f32x4 oacc[VD];       // PV accumulators
  uint4 qf[NCH];
  uint4 qv[kValu ? kValuG : 1][NCH];  // kValu: column g's chunk c%4 of each step, lane (r, c)
  auto clear_acc = [&]() {
#pragma unroll
    for (int j = 0; j < VD; ++j) oacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  clear_acc();
#pragma unroll
  for (int cc = 0; cc < NCH; ++cc) qf[cc] = make_uint4(0u, 0u, 0u, 0u);
  bool piece_from_start = false;
  bool piece_first_in_range = false;
#ifdef MXFA_WAVE_STAMPS
  bool stamp_data = true;  // the first tile's data not yet stamped
#endif
  // V slot of this lane: the VD dims it holds (and writes) start at vslot*VD.
  const int vslot = kShareV ? 2 * (col & 7) + (col >> 3) : col;

  auto finalize = [&](const Tile &d) {
    const float dt = rows_sum(dsum);  // lane (any row, h): denominator of head h
    const int b = d.b;
    const bool whole = !kSeq && piece_from_start && (d.flags & kSeqEnd);
    const int slot = piece_first_in_range ? 0 : 1;
    const int64_t pbase = ((int64_t)(kvh * ns + rr) * 2 + slot) * nc;
    static_for<4>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      const int hh = 4 * row + i;  // column of accumulator element i in this lane
      const float Dh = head_of_row<HR, i>(dt, row);
      const float Mh = head_of_row<HR, i>(m, row);
      if (hh >= nc) return;
      const int ht = hh / gq, hg = hh - (hh / gq) * gq;
      // A sink joins the denominator once per (sequence, head): here for a
      // sequence whole in the range, in the combine for a split one. With no
      // key seen (Mh = -inf) the term is +inf and the output 0.
      float Dw = Dh;
      if constexpr (kExtras) {
        if (whole && p.sinks) Dw += fast_exp2(p.sinks[kvh * gq + hg] * kLog2e - Mh);
      }
      const float inv = Dw > 0.f ? v_scale / Dw : 0.f;
      float v[VD];
#pragma unroll
      for (int j = 0; j < VD; ++j) v[j] = oacc[j][i];
      if (whole) {
        store_row<VD, E>(p.out + b * p.o_sb + ht * p.o_st + (kvh * gq + hg) * p.o_sh +
                             vslot * (VD * 2),
                         v, inv);
      } else {
        float4 *dst = reinterpret_cast<float4 *>(
            (kSeq ? lds_o + hh * HD : p.ws_o + (pbase + hh) * HD) + vslot * VD);
#pragma unroll
        for (int j = 0; j < VD / 4; ++j)
          dst[j] = make_float4(v[4 * j] * inv, v[4 * j + 1] * inv, v[4 * j + 2] * inv,
                               v[4 * j + 3] * inv);
        if (col == 0)
          (kSeq ? lds_lse[hh] : p.ws_lse[pbase + hh]) = Dh > 0.f ? Mh + __log2f(Dh) : -INFINITY;
      }
    });
  };

  uint32_t probe = 0;
  auto compute = [&](Set &s) {
    const Tile &d = s.d;
    if constexpr (kProbe) {
#pragma unroll
      for (int cc = 0; cc < NKL; ++cc) probe ^= s.k[cc].x ^ s.k[cc].y ^ s.k[cc].z ^ s.k[cc].w;
      if constexpr (kShareV) {
        probe ^= s.vr[0].x ^ s.vr[0].y ^ s.vr[0].z ^ s.vr[0].w;
        probe ^= s.vr[1].x ^ s.vr[1].y ^ s.vr[1].z ^ s.vr[1].w;
      } else {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int w = 0; w < VB / 4; ++w) probe ^= s.v[u].w[w];
      }
      if (d.flags & kFirst) {
#pragma unroll
        for (int cc = 0; cc < NCH; ++cc) probe ^= s.q[cc].x ^ s.q[cc].y ^ s.q[cc].z ^ s.q[cc].w;
      }
      return;
    }
    if (d.flags & kFirst) {
      m = -INFINITY;
      dsum = 0.f;
      clear_acc();
#pragma unroll
      for (int cc = 0; cc < NCH; ++cc) qf[cc] = s.q[cc];
      if constexpr (kValu) {
        // qf: lane (r', c') holds column c' chunk r'; column g chunk k sits in
        // lane 16k + g (the LDS crossbar moves it; no LDS memory is used).
#pragma unroll
        for (int g = 0; g < kValuG; ++g) {
          const int src = ((col & 3) * 16 + g) * 4;
#pragma unroll
          for (int cc = 0; cc < NCH; ++cc) {
            qv[g][cc].x = __builtin_amdgcn_ds_bpermute(src, qf[cc].x);
            qv[g][cc].y = __builtin_amdgcn_ds_bpermute(src, qf[cc].y);
            qv[g][cc].z = __builtin_amdgcn_ds_bpermute(src, qf[cc].z);
            qv[g][cc].w = __builtin_amdgcn_ds_bpermute(src, qf[cc].w);
          }
        }
      }
      piece_from_start = (d.flags & kSeqStart) != 0;
      piece_first_in_range = (d.flags & kRangeStart) != 0;
    }
    // QK on the matrix cores; two accumulators halve the MFMA dependency chain.
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    if constexpr (kValu) {
      // QK on the VALU: per column g, the lane's 4 * NCH dot2 over its chunks
      // of its token, summed over the four chunk lanes of the token (quad_perm
      // [1,0,3,2] then [2,3,0,1]); lane (r, c) then holds the score of token
      // 4r + c/4. Score element i of lane (r, h) (token 4r + i, column h) is
      // lane (r, 4i)'s score of column h (row_newbcast:4i). The result is the
      // MFMA layout, so the softmax and PV below are the same code.
      float sg[kValuG];
#pragma unroll
      for (int g = 0; g < kValuG; ++g) {
        float a = 0.f;
#pragma unroll
        for (int cc = 0; cc < NCH; ++cc) {
          a = Dot2<T>::run(s.k[cc].x, qv[g][cc].x, a);
          a = Dot2<T>::run(s.k[cc].y, qv[g][cc].y, a);
          a = Dot2<T>::run(s.k[cc].z, qv[g][cc].z, a);
          a = Dot2<T>::run(s.k[cc].w, qv[g][cc].w, a);
        }
        a += __int_as_float(
            __builtin_amdgcn_update_dpp(0, __float_as_int(a), kDppQuadSwap1, 0xf, 0xf, false));
        a += __int_as_float(
            __builtin_amdgcn_update_dpp(0, __float_as_int(a), kDppQuadSwap2, 0xf, 0xf, false));
        sg[g] = a;
      }
      static_for<4>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        float v = 0.f;
#pragma unroll
        for (int g = 0; g < kValuG; ++g) {
          const float b = row_bcast<4 * i>(sg[g]);
          v = col == g ? b : v;
        }
        acc0[i] = v;
      });
    } else if constexpr (kF8) {
#pragma unroll
      for (int mm = 0; mm < NKL; ++mm) {
        acc0 = Mfma<T>::run(widen8<T>(s.k[mm].x, s.k[mm].y), qf[2 * mm], acc0);
        acc1 = Mfma<T>::run(widen8<T>(s.k[mm].z, s.k[mm].w), qf[2 * mm + 1], acc1);
      }
    } else {
#pragma unroll
      for (int cc = 0; cc < NCH; cc += 2) {
        acc0 = Mfma<T>::run(s.k[cc], qf[cc], acc0);
        acc1 = Mfma<T>::run(s.k[cc + 1], qf[cc + 1], acc1);
      }
    }
    float x[4];
    bool need = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = (acc0[i] + acc1[i]) * c;
    if constexpr (kExtras) {
      if (capped) {  // wave-uniform
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = cap_out * tanh_exp2((acc0[i] + acc1[i]) * cap_in);
      }
      if (alibi) {  // wave-uniform; after the cap, as FlashAttention applies it
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int dist = abs(d.rem - (4 * row + i) - qdist);
          x[i] -= slope2 * (float)dist;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * row + i;
      bool valid = (col < nc) & (r < d.rem - c_hide);
      if constexpr (kExtras) valid &= r >= d.rem - c_reach;
      x[i] = valid ? x[i] : -INFINITY;
      need |= x[i] > m + kRescaleLog2;
    }
#ifdef MXFA_WAVE_STAMPS
    if (stamp_data) {
      wave_stamp_after(p, 11, x[0]);
      stamp_data = false;
    }
#endif
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
      // Rare, wave-uniform: move the reference of each head to the wave's
      // tile maximum when it passed the reference by more than kRescaleLog2.
      const float mt = rows_max(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
      const float mn = mt > m + kRescaleLog2 ? mt : m;
      const float f = (mn == m) ? 1.f : fast_exp2(m - mn);  // m = -inf: f = 0
      dsum *= f;
      static_for<4>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        const float fi = head_of_row<HR, i>(f, row);
#pragma unroll
        for (int j = 0; j < VD; ++j) oacc[j][i] *= fi;
      });
      m = mn;
    }
    // m = -inf: this column has seen no valid token, its scores here are -inf too.
    const float mr = m == -INFINITY ? 0.f : m;
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pr[i] = fast_exp2(x[i] - mr);
    // P rounded to the element type once; the denominator sums the same
    // rounded weights, so the output stays a convex combination of V rows.
    uint16_t ph[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ph[i] = PvMfma<T>::round(pr[i]);
    dsum += (PvMfma<T>::widen(ph[0]) + PvMfma<T>::widen(ph[1])) +
            (PvMfma<T>::widen(ph[2]) + PvMfma<T>::widen(ph[3]));
    const uint2 a = make_uint2((uint32_t)ph[0] | ((uint32_t)ph[1] << 16),
                               (uint32_t)ph[2] | ((uint32_t)ph[3] << 16));
    // The lane's V bytes of its four tokens (kShareV: halves swapped with lane
    // c^8 first), then as element pairs (fp8: widened here, once).
    constexpr int VW = VB / 4;  // words per token
    uint32_t vt[U][VW];
    if constexpr (kShareV) {
      const bool hi = col >= 8;
      const uint4 a = s.vr[0], bq = s.vr[1];
      const uint32_t r0 = row_swap8(hi ? a.x : a.z), r1 = row_swap8(hi ? a.y : a.w);
      const uint32_t r2 = row_swap8(hi ? bq.x : bq.z), r3 = row_swap8(hi ? bq.y : bq.w);
      vt[0][0] = hi ? r0 : a.x;
      vt[0][1] = hi ? r1 : a.y;
      vt[1][0] = hi ? r2 : bq.x;
      vt[1][1] = hi ? r3 : bq.y;
      vt[2][0] = hi ? a.z : r0;
      vt[2][1] = hi ? a.w : r1;
      vt[3][0] = hi ? bq.z : r2;
      vt[3][1] = hi ? bq.w : r3;
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int w = 0; w < VW; ++w) vt[u][w] = s.v[u].w[w];
    }
    uint32_t vw[U][VD / 2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int wi = 0; wi < VD / 2; ++wi) {
        if constexpr (kF8)
          vw[u][wi] = (wi & 1) ? Fp8Widen<T>::template pair<true>(vt[u][wi >> 1])
                               : Fp8Widen<T>::template pair<false>(vt[u][wi >> 1]);
        else
          vw[u][wi] = vt[u][wi];
      }
    }
#pragma unroll
    for (int jb = 0; jb < VD; ++jb) {
      const int wi = jb >> 1, odd = jb & 1;
      const uint2 bv = make_uint2(pair_halves(vw[0][wi], vw[1][wi], odd),
                                  pair_halves(vw[2][wi], vw[3][wi], odd));
      oacc[jb] = PvMfma<T>::run(a, bv, oacc[jb]);
    }
    if (d.flags & kLast) finalize(d);
  };

  // Software pipeline over the range with NBUF register sets: tile
  // descriptors (and page ids) are built NBUF tiles ahead of the math, K/V/q
  // loads issued NBUF-1 tiles ahead. The body runs NBUF tiles and exits only at
  // its latch, so the loads crossing the back edge always land in the same
  // sets. The descriptor of a padding tile past the range end covers no
  // bytes, so its loads cost nothing.
  Set sets[NBUF];
  Tile dn;
  int lpg_n[NPG];
  static_for<NBUF>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    make_tile(lo + i * tstep, sets[i].d, sets[i].lpg);
    // The page id of the first tile read above (or by the caller) replaces
    // make_tile's read, which is then dead code.
    if constexpr (i == 0 && !kLanePages && !kExtras) sets[0].d.pg = pg_first;
    if constexpr (i < NBUF - 1) issue(sets[i]);
  });
  wave_stamp_after(p, 10, sets[0].d.pg);
  const int ntiles = kSeq ? (hi - lo + tstep - 1) / tstep : hi - lo;
  int t = lo;
  wave_stamp(p, 2, wave_clock());
  auto step = [&](auto kc) {
    constexpr int k = decltype(kc)::value;
    constexpr int kn = (k + NBUF - 1) % NBUF;  // holds tile t + NBUF - 1
    if constexpr (kLanePages) {
      make_tile(t + NBUF * tstep, dn, lpg_n);
      issue(sets[kn]);
    } else {
      issue(sets[kn]);
      make_tile(t + NBUF * tstep, dn, lpg_n);
    }
    compute(sets[k]);
    sets[k].d = dn;
#pragma unroll
    for (int i = 0; i < NPG; ++i) sets[k].lpg[i] = lpg_n[i];
    t += tstep;
  };
  int done = 0;
  for (; done + NBUF <= ntiles; done += NBUF) {
    if constexpr (kBalance) {
      // Two waves per SIMD: the older one runs ahead of its partner and the
      // CU ends on one wave per SIMD. Each wave lowers its priority as its
      // range shrinks (3 in the first quarter, 0 in the last), so the one
      // behind issues first.
      const int q = ((ntiles - done) * 4 - 1) / ntiles;
      if (q >= 3)
        __builtin_amdgcn_s_setprio(3);
      else if (q == 2)
        __builtin_amdgcn_s_setprio(2);
      else if (q == 1)
        __builtin_amdgcn_s_setprio(1);
      else
        __builtin_amdgcn_s_setprio(0);
    }
    static_for<NBUF>(step);
  }
  const int rest = ntiles - done;  // < NBUF tiles, already issued into sets[0 .. rest-1]
  static_for<NBUF - 1>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    if (j < rest) compute(sets[j]);
  });
  return probe;
}

// kExtras: the call has a sliding window, soft-capping, ALiBi or sinks (the host
// picks the instantiation; without them the kernel is the plain one).
template <int HD, int HR, typename T, bool kF8, bool kLanePages, int NBUF, int WAVES,
          bool kExtras, int kWaveScan, int kValuG>
__global__ __launch_bounds__(WAVES * 64, 1) void split_partial_kernel(const int32_t *seqlens,
                                                                        int batch,
                                                                        DecodeParams p) {
  constexpr int kThreads = WAVES * 64;
  extern __shared__ int32_t s_tiles[];  // [B + 1]
  __shared__ int s_wave_tot[WAVES];

  const unsigned long long t_entry = wave_clock();
  const int B = batch;
  // kWaveScan: the launcher's choice, sequences per lane of the wave-local
  // scan (wave_scan_per_lane), or 0 for the LDS scan.
  WaveScan<kWaveScan == 4 ? 4 : 1> wsc;
  int NT;
  if constexpr (kWaveScan != 0) {
    NT = rfl(wave_tile_scan<kExtras>(p, seqlens, B, wsc));
    zero_empty_wave<HD, kThreads>(p, wsc);
  } else {
    NT = rfl(tile_prefix<kThreads, kExtras>(p, seqlens, B, s_tiles, s_wave_tot));
    zero_empty<HD, kThreads>(p, s_tiles);
    if (blockIdx.x == 0 && blockIdx.y == 0) {
      for (int i = threadIdx.x; i <= B; i += kThreads) p.ws_s[i] = s_tiles[i];
    }
  }

  const int wave = rfl(threadIdx.x >> 6);
  const int KH = p.heads_per_wg;
  const int kh = wave % KH, sub = wave / KH;
  const int kvh = blockIdx.x * KH + kh;
  const int R = min(p.num_ranges, NT);  // every range holds >= 1 tile
  const int rr = blockIdx.y * p.subs + sub;
  if (sub >= p.subs || kvh >= p.hkv || rr >= R) return;
  const int lo = range_lo(rr, R, NT), hi = range_lo(rr + 1, R, NT);
  wave_stamp(p, 0, t_entry);
  wave_stamp(p, 1, wave_clock());
  run_range<HD, HR, T, kF8, kLanePages, NBUF, kExtras, false, WAVES == 8, false, kWaveScan,
            kValuG>(p, s_tiles, kvh, rr, lo, hi, 1, nullptr, nullptr, 0, wsc);
  // The prefix sums for the combine, by the first wave of workgroup (0, 0)
  // (which always has a range) once its own range is done: the pointer is
  // read from the parameter block only here, off the prologue.
  if constexpr (kWaveScan != 0) {
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < 64) store_prefix_wave(p, wsc, B, NT);
  }
  wave_stamp(p, 3, wave_clock());
  wave_stamp(p, 4, hi - lo);
  wave_stamp(p, 5, 1);
  wave_stamp(p, 6, blockIdx.y * gridDim.x + blockIdx.x);
  wave_stamp(p, 7, kvh);
}

// Streaming probe: split_partial_kernel's tile scan, ranges, launch shape and
// per-tile loads (16-bit caches, page-uniform tiles, NBUF register sets) with
// no attention math: each lane XORs the words it loads and writes that to
// sink[(kvh * num_ranges + rr) * 64 + lane]. Its time is the ceiling the tile loop's
// access pattern allows; it writes no output, workspace or prefix sums.
template <int HD, typename T, int NBUF, int WAVES, int kWaveScan>
__global__ __launch_bounds__(WAVES * 64, 1) void stream_probe_kernel(const int32_t *seqlens,
                                                                       int batch, DecodeParams p,
                                                                       uint32_t *sink) {
  constexpr int kThreads = WAVES * 64;
  extern __shared__ int32_t s_tiles[];  // [B + 1]
  __shared__ int s_wave_tot[WAVES];
  WaveScan<kWaveScan == 4 ? 4 : 1> wsc;
  int NT;
  if constexpr (kWaveScan != 0)
    NT = rfl(wave_tile_scan<false>(p, seqlens, batch, wsc));
  else
    NT = rfl(tile_prefix<kThreads, false>(p, seqlens, batch, s_tiles, s_wave_tot));
  const int wave = rfl(threadIdx.x >> 6);
  const int KH = p.heads_per_wg;
  const int kh = wave % KH, sub = wave / KH;
  const int kvh = blockIdx.x * KH + kh;
  const int R = min(p.num_ranges, NT);
  const int rr = blockIdx.y * p.subs + sub;
  if (sub >= p.subs || kvh >= p.hkv || rr >= R) return;
  const int lo = range_lo(rr, R, NT), hi = range_lo(rr + 1, R, NT);
  const uint32_t x =
      run_range<HD, 1, T, false, false, NBUF, false, false, WAVES == 8, true, kWaveScan>(
          p, s_tiles, kvh, rr, lo, hi, 1, nullptr, nullptr, 0, wsc);
  sink[((int64_t)kvh * p.num_ranges + rr) * 64 + (threadIdx.x & 63)] = x;
}

// Merge of two partial states (max, weight, accumulator) in the base-2 domain.
__device__ __forceinline__ void lse_fold(float &M, float &W, float4 &A, float m2, float w2,
                                         const float4 &a2) {
  const float Mn = fmaxf(M, m2);
  if (Mn == -INFINITY) return;
  const float f1 = (M == -INFINITY) ? 0.f : fast_exp2(M - Mn);
  const float f2 = (m2 == -INFINITY) ? 0.f : fast_exp2(m2 - Mn);
  W = W * f1 + w2 * f2;
  A.x = A.x * f1 + a2.x * f2;
  A.y = A.y * f1 + a2.y * f2;
  A.z = A.z * f1 + a2.z * f2;
  A.w = A.w * f1 + a2.w * f2;
  M = Mn;
}

// LSE combine: one block of kCombineThreads per (sequence b, H consecutive
// query heads), H = heads_per_block (host choice), or, with X = chunk_parts > 1
// (then H = 1), per (sequence, head, 1/X of the head's HD/4 float4 chunks).
// The block's CB = H * HD/4 / X chunks are split over G = kCombineThreads / CB
// piece groups: thread (g, c) folds pieces ra+g, ra+g+G, ... of chunk c, eight
// loads in flight per step; the G groups then merge through an LDS tree and
// the output is rounded once. Splitting a head's chunks over X blocks gives a
// sequence of many pieces (few sequences, many ranges) X times the groups, so
// its pieces come in one step. The fold order depends on H and X only (host
// choices), never on timing. Blocks whose sequence lies inside one range
// (written by the partial kernel) or is empty (zero-filled there) leave at once.
constexpr int kCombineThreads = 256;

template <int HD, typename T>
__global__ __launch_bounds__(kCombineThreads) void split_combine_kernel(
    const int32_t *ws_s, const float *ws_o, const float *ws_lse, int batch, int nblk, int H,
    int X, int hq, int ql, int gq, int ns, CombineParams p) {
  using E = Elem<T>;
  constexpr int CH = HD / 4;  // float4 chunks per head
  constexpr int kUnroll = 8;
  __shared__ float s_red[kCombineThreads * 6];
  // Everything up to the piece loads comes from the leading arguments (the
  // CombineParams fields of the same names, preloaded into SGPRs): the
  // prefix sums are read at once and the pieces right after them.
  const int b = blockIdx.x / nblk;  // nblk = ceil(nv / H) * X blocks per sequence
  const int NT = ws_s[batch];
  const int sb = ws_s[b], se = ws_s[b + 1];
  const int CC = CH / X;  // chunks of a head in this block
  const int CB = H * CC;
  const int groups = kCombineThreads / CB;
  const int nv = hq * ql;  // (query token, head) rows per sequence
  const int hb = blockIdx.x % nblk;
  const int vh = (hb / X) * H + (threadIdx.x % CB) / CC;
  const int cc = (hb % X) * CC + threadIdx.x % CC;
  const int g = threadIdx.x / CB;
  block_stamp_after(p, 0, g);
  block_stamp_after(p, 1, NT + sb + se);
  // Prefix sums that do not describe tiles inside [0, NT) (a workspace the
  // partial kernel did not fill) are skipped, so every index stays in range.
  if (se <= sb || sb < 0 || se > NT) {
    block_stamp_after(p, 3, sb);
    return;
  }
  const int R = min(ns, NT);
  const int ra = range_of(sb, R, NT), rb = range_of(se - 1, R, NT);
  if (ra == rb) {
    block_stamp_after(p, 3, ra);
    return;
  }
  const int slot_a = (range_lo(ra, R, NT) == sb) ? 0 : 1;
  const bool live = vh < nv;  // the last block of a sequence may run past the rows
  const int t = live ? vh / hq : 0, h = live ? vh - t * hq : 0;
  const int kvh = h / gq, hh = t * gq + (h - kvh * gq);  // piece column
  const int nc = gq * ql;
  float M = -INFINITY, W = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (live) {
    for (int q0 = ra + g; q0 <= rb; q0 += kUnroll * groups) {
      float l[kUnroll];
      float4 ov[kUnroll];
#pragma unroll
      for (int i = 0; i < kUnroll; ++i) {
        const int q = min(q0 + i * groups, rb);
        const int64_t ps = ((int64_t)(kvh * ns + q) * 2 + (q == ra ? slot_a : 0)) * nc + hh;
        l[i] = (q0 + i * groups <= rb) ? ws_lse[ps] : -INFINITY;
        ov[i] = reinterpret_cast<const float4 *>(ws_o + ps * HD)[cc];
      }
#pragma unroll
      for (int i = 0; i < kUnroll; ++i) lse_fold(M, W, acc, l[i], 1.f, ov[i]);
    }
  }
  block_stamp_after(p, 2, M);
  float *red = s_red + threadIdx.x * 6;
  red[0] = M;
  red[1] = W;
  red[2] = acc.x;
  red[3] = acc.y;
  red[4] = acc.z;
  red[5] = acc.w;
  __syncthreads();
  for (int stride = groups / 2; stride >= 1; stride >>= 1) {  // groups is a power of two
    if (g < stride) {
      const float *o2 = s_red + (threadIdx.x + stride * CB) * 6;
      lse_fold(M, W, acc, o2[0], o2[1], make_float4(o2[2], o2[3], o2[4], o2[5]));
      red[0] = M;
      red[1] = W;
      red[2] = acc.x;
      red[3] = acc.y;
      red[4] = acc.z;
      red[5] = acc.w;
    }
    __syncthreads();
  }
  if (g == 0 && live) {
    if (p.sinks) W += fast_exp2(p.sinks[h] * kLog2e - M);  // M = -inf: W = inf, out 0
    const float inv = W > 0.f ? 1.f / W : 0.f;
    const uint32_t w0 =
        (uint32_t)E::narrow(acc.x * inv) | ((uint32_t)E::narrow(acc.y * inv) << 16);
    const uint32_t w1 =
        (uint32_t)E::narrow(acc.z * inv) | ((uint32_t)E::narrow(acc.w * inv) << 16);
    *reinterpret_cast<uint2 *>(p.out + b * p.o_sb + t * p.o_st + h * p.o_sh + cc * 8) =
        make_uint2(w0, w1);
  }
  block_stamp_after(p, 3, W);
}

// Per-sequence workgroups (one launch, no workspace, no tile scan): workgroup
// (x, b) takes sequence b for kv heads x*KH .. x*KH + KH - 1, KH =
// heads_per_wg. Wave (kh, s), s < S = subs, takes tiles s, s + S, s + 2S, ...
// of the sequence for its kv head, so its first page id is read together with
// the length. Each wave leaves one piece (normalised output and base-2 LSE)
// in LDS; after a barrier the workgroup folds the S pieces of every (kv head,
// column) in wave order and rounds the output once. Waves past the sequence's
// tiles leave an LSE of -inf and are skipped; an empty sequence gets zeros.
// LDS: WAVES * C * (HD + 1) floats, C = GQ * QL.
template <int HD, int HR, typename T, bool kF8, bool kLanePages, int NBUF, int WAVES, int OCC,
          bool kExtras>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(OCC)))
void seq_decode_kernel(const int32_t *seqlens, const int32_t *bt, int64_t bt_stride, int max_len,
                       int seqlen_add, int ps_log2, DecodeParams p) {
  using E = Elem<T>;
  constexpr int CH = HD / 4;  // float4 chunks per head row
  extern __shared__ float s_piece[];
  // One kv head per workgroup (the launcher's shape): wave s takes tiles s,
  // s + WAVES, ... of the sequence.
  constexpr int KH = 1, S = WAVES;
  const int wave = rfl(threadIdx.x >> 6);
  const int sub = wave;
  const int kvh = blockIdx.x;
  const int b = blockIdx.y;
  const unsigned long long t_entry = wave_clock();
  // The length and (no window, page-uniform tiles) the first tile's page id
  // first: their addresses need only the preloaded leading arguments, so
  // both loads go out with the kernel-argument loads.
  const int len_raw = as_const(seqlens)[b];
  int pg_first = 0;
  if constexpr (!kExtras && !kLanePages)
    pg_first = as_const(bt + (int64_t)b * bt_stride)[min(sub * kTile, max_len - 1) >> ps_log2];
  // One wait for all of them and for the arguments the first K/V loads need
  // (otherwise each is read where first used, one round trip after another).
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::"s"(len_raw), "s"(pg_first), "s"(p.q), "s"(p.k), "s"(p.v), "s"(p.sp_bytes),
               "s"(p.st_bytes), "s"(p.hkv));
  const int nc = p.gq * p.ql;
  float *const lse_base = s_piece + WAVES * nc * HD;
  int L = len_raw + seqlen_add;
  L = L < 0 ? 0 : (L > max_len ? max_len : L);
  const int n = L > 0 ? (kExtras ? tiles_of(L, p.ql, p.window_left) : (L + kTile - 1) / kTile)
                      : 0;
  if ((threadIdx.x & 63) < nc) lse_base[wave * nc + (threadIdx.x & 63)] = -INFINITY;
  if (kvh < p.hkv && sub < n) {
    DecodeParams v = p;  // the one sequence, as a batch of 1
    v.q += b * p.q_sb;
    v.bt = bt + b * bt_stride;  // the preloaded copies: the first page id waits on no kernarg load
    v.seqlens = seqlens + b;
    v.max_len = max_len;
    v.seqlen_add = seqlen_add;
    v.ps_log2 = ps_log2;
    v.out += b * p.o_sb;
    v.batch = 1;
    wave_stamp(p, 0, t_entry);
    wave_stamp(p, 1, wave_clock());
    run_range<HD, HR, T, kF8, kLanePages, NBUF, kExtras, true>(
        v, nullptr, kvh, 0, sub, n, S, s_piece + wave * nc * HD, lse_base + wave * nc, pg_first);
    wave_stamp(p, 3, wave_clock());
    wave_stamp(p, 4, (n - sub + S - 1) / S);
    wave_stamp(p, 5, 1);
    wave_stamp(p, 6, blockIdx.y * gridDim.x + blockIdx.x);
    wave_stamp(p, 7, kvh);
  }
  __syncthreads();
  for (int it = threadIdx.x; it < KH * nc * CH; it += WAVES * 64) {
    const int cc = it % CH, r = it / CH;
    const int hh = r % nc, kk = r / nc;
    const int kv = blockIdx.x * KH + kk;
    if (kv >= p.hkv) continue;
    float M = -INFINITY, W = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s2 = 0; s2 < S; ++s2) {
      const int w = s2 * KH + kk;
      const float l = lse_base[w * nc + hh];
      if (l == -INFINITY) continue;  // no piece (or no key seen): its output is not read
      lse_fold(M, W, acc, l, 1.f, reinterpret_cast<const float4 *>(s_piece + (w * nc + hh) * HD)[cc]);
    }
    const int t = hh / p.gq, h = kv * p.gq + (hh - t * p.gq);
    if (p.sinks) W += fast_exp2(p.sinks[h] * kLog2e - M);  // M = -inf: W = inf, out 0
    const float inv = W > 0.f ? 1.f / W : 0.f;
    const uint32_t w0 =
        (uint32_t)E::narrow(acc.x * inv) | ((uint32_t)E::narrow(acc.y * inv) << 16);
    const uint32_t w1 =
        (uint32_t)E::narrow(acc.z * inv) | ((uint32_t)E::narrow(acc.w * inv) << 16);
    *reinterpret_cast<uint2 *>(p.out + b * p.o_sb + t * p.o_st + h * p.o_sh + cc * 8) =
        make_uint2(w0, w1);
  }
}

// ---------------------------------------------------------------------------
// Launch shapes (host side, shared by the per-head-dim compilation units).

// Launch shape by the bytes of one K (or V) head row, RB = HD * element size:
// 64 (fp8 HD 64), 128 (16-bit HD 64, fp8 HD 128), 256 (16-bit HD 128, fp8
// HD 256) or 512 (16-bit HD 256).
template <int HD, bool kF8>
constexpr int kRowBytes = HD * (kF8 ? 1 : 2);

// Waves per workgroup: one wave per kv head (KH = min(HKV, waves) kv heads per
// workgroup, S = waves / KH sub-ranges when HKV < 4); 4 waves for HKV <= 4,
// else 8 for rows of up to 128 bytes and 4 for longer rows; one workgroup per
// CU. Waves past KH x S (HKV 3, 5, 6, 7) leave at once.
// Measured on MI355X (one call, config-2 lengths): with 256-byte rows
// eight-wave workgroups run as two generations of four waves per CU (the
// second wave on each SIMD issues its first loads only when the first
// finishes, since four waves already fill the CU's vector-memory queue), which
// leaves a drain tail: four-wave workgroups are 3% (GQ4) to 10% (GQ8) faster.
// With 128-byte rows all eight waves run together: eight beat four by 2-3%
// (16-bit HD 64) and 15% (fp8 HD 128) at 8 kv heads; four beat two sub-ranges
// of eight by 10% at 4 kv heads; two workgroups per CU lose 2-15% everywhere.
constexpr int kMinWaves = 4;
template <int HD, bool kF8>
constexpr int kMaxWaves = kRowBytes<HD, kF8> <= 128 ? 8 : 4;

inline int waves_for(int row_bytes, int hkv) {
  const int most = row_bytes <= 128 ? 8 : 4;
  return hkv > kMinWaves ? most : kMinWaves;
}

// Workgroups of `waves` waves: min(HKV, waves) kv heads x waves / that sub-ranges.
inline Grid grid_for(int hkv, int num_splits, int waves) {
  Grid g;
  g.waves = waves;
  g.heads_per_wg = hkv < waves ? hkv : waves;
  g.subs = waves / g.heads_per_wg;
  g.gx = (hkv + g.heads_per_wg - 1) / g.heads_per_wg;
  g.gy = (num_splits + g.subs - 1) / g.subs;
  return g;
}

// Register sets of the tile pipeline: tiles of 128-byte rows are half the
// bytes of 256-byte ones, so a third set keeps as many bytes in flight per
// wave; 64-byte rows (fp8 HD 64) take a fourth.
template <int HD, bool kF8>
constexpr int kNbuf = kRowBytes<HD, kF8> <= 64 ? 4 : kRowBytes<HD, kF8> <= 128 ? 3 : 2;

// Eight-wave workgroups of 128-byte rows (two waves per SIMD) take two
// register sets instead of three when the host's bound on tiles per range is
// small: the shorter pipeline fill and drain pay more than the third set's
// bytes in flight there, and less over long ranges. Graph replays on MI355X,
// three sets against two: config 3 (B 128, 8 tiles per range) 17.56 / 17.35
// us, B 32 GQ4 HD64 with L <= 2048 19.59 / 19.14, the GQ4 HD64 cell (42 tiles)
// 60.13 / 59.88, fp8 HD128 at config 2 (42 tiles) 61.65 / 61.37; the GQ2 HD64
// cell (84 tiles) 108.62 / 109.19. Four-wave workgroups (one wave per SIMD)
// keep three sets everywhere (GQ8 HD64 33.76 / 34.26 with two).
constexpr int kShortRangeTiles = 64;
template <int HD, bool kF8, int WAVES>
constexpr bool kTwoSetsShort = kRowBytes<HD, kF8> == 128 && WAVES == 8;

// Rows of the MFMA layout that hold used columns (4 columns per row).
inline int head_rows(int cols) { return cols <= 4 ? 1 : cols <= 8 ? 2 : 4; }

template <int HD, int HR, typename T, bool kF8, int WAVES, bool kExtras, int kWaveScan,
          int kValuG>
static int launch_partial_s(const DecodeParams &p, const Grid &g, hipStream_t st) {
  dim3 grid(g.gx, g.gy);
  // The wave-local scan keeps nothing in LDS.
  const size_t lds = kWaveScan ? 0 : (size_t)(p.batch + 1) * sizeof(int32_t);
  if (p.ps_log2 >= 4) {
    if constexpr (kTwoSetsShort<HD, kF8, WAVES>) {
      if (g.short_ranges) {
        hipLaunchKernelGGL((split_partial_kernel<HD, HR, T, kF8, false, 2, WAVES, kExtras,
                                                 kWaveScan, kValuG>),
                           grid, dim3(WAVES * 64), lds, st, p.seqlens, p.batch, p);
        return hipGetLastError() == hipSuccess ? MXFA_OK : MXFA_ELAUNCH;
      }
    }
    hipLaunchKernelGGL((split_partial_kernel<HD, HR, T, kF8, false, kNbuf<HD, kF8>, WAVES, kExtras,
                                             kWaveScan, kValuG>),
                       grid, dim3(WAVES * 64), lds, st, p.seqlens, p.batch, p);
  } else {  // per-lane page ids: QK stays on the matrix cores
    if constexpr (kWaveScan == 4)
      return MXFA_EUNSUPPORTED;  // not instantiated (plain_call)
    else
      hipLaunchKernelGGL(
          (split_partial_kernel<HD, HR, T, kF8, true, 2, WAVES, kExtras, kWaveScan, 0>), grid,
          dim3(WAVES * 64), lds, st, p.seqlens, p.batch, p);
  }
  return hipGetLastError() == hipSuccess ? MXFA_OK : MXFA_ELAUNCH;
}

// A call with no window, cap, sinks or ALiBi on page-uniform tiles: the only
// calls the four-sequences-per-lane scan is built for (the others, past 64
// sequences, keep the LDS scan), so its instantiations stay few.
inline bool plain_call(const DecodeParams &p) {
  return p.window_left < 0 && !(p.softcap > 0.f) && !p.sinks && !p.alibi && p.ps_log2 >= 4;
}

// kWaveScan (the wave-local tile scan, 1 or 4 sequences per lane, or 0) is
// the caller's choice (wave_scan_per_lane, plain_call); the three compile in
// separate units.
template <int HD, int HR, typename T, bool kF8, int WAVES, int kWaveScan, int kValuG>
static int launch_partial_w(const DecodeParams &p, const Grid &g, hipStream_t st) {
  const bool extras = p.window_left >= 0 || p.softcap > 0.f || p.sinks || p.alibi;
  if constexpr (kWaveScan == 4) {
    if (extras) return MXFA_EUNSUPPORTED;  // not instantiated (plain_call)
    return launch_partial_s<HD, HR, T, kF8, WAVES, false, kWaveScan, kValuG>(p, g, st);
  } else {
    return extras ? launch_partial_s<HD, HR, T, kF8, WAVES, true, kWaveScan, kValuG>(p, g, st)
                  : launch_partial_s<HD, HR, T, kF8, WAVES, false, kWaveScan, kValuG>(p, g, st);
  }
}

// The kernel is the grid's wave count; a grid the instantiations cannot run
// (more waves than the row size has, or its heads and sub-ranges past the
// waves) is refused: its extra kv heads would go uncomputed.
template <int HD, int HR, typename T, bool kF8, int kWaveScan, int kValuG = 0>
static int launch_partial_t(const DecodeParams &p, const Grid &g, hipStream_t st) {
  if (g.heads_per_wg * g.subs > g.waves) return MXFA_ELAUNCH;
  if constexpr (kMaxWaves<HD, kF8> == 8) {
    if (g.waves == 8) return launch_partial_w<HD, HR, T, kF8, 8, kWaveScan, kValuG>(p, g, st);
  }
  if (g.waves != 4) return MXFA_ELAUNCH;
  return launch_partial_w<HD, HR, T, kF8, 4, kWaveScan, kValuG>(p, g, st);
}

// Columns (query tokens x heads per kv head) whose QK runs on the VALU in
// the split kernel: 0 for the matrix cores. Measured on MI355X (config-2
// lengths, B 32, bf16, partial kernel under rocprof, VALU against MFMA): GQ 1
// HD 128 423.0 / 427.9 us, GQ 2 HD 128 202.2 / 204.4, GQ 4 HD 128 103.5 /
// 103.9; graph replays: GQ 1 HD 64 208.8 / 210.8, GQ 2 HD 256 218.1 / 223.2,
// GQ 2 HD 64 109.0 / 109.1, GQ 4 HD 64 60.8 / 59.9, GQ 8 HD 128 61.8 / 59.5,
// GQ 8 HD 64 42.8 / 33.7; as built here, config 3 (B 128, GQ 2 HD 64, fp16,
// L <= 512) 18.67 / 17.82 and GQ 2 HD 64 109.3 / 109.1. With few columns the
// MFMA computes 16 columns for one or two; with more, its few instructions per
// tile beat the VALU's 4 x HD/32 dot2 per column; with 128-byte rows (eight
// waves per CU, short pieces) the per-piece q exchange does not pay. 16-bit
// caches with page-uniform tiles and head dims of 128 or more only.
inline int valu_qk_columns(int cols, int hd) {
#ifdef MXFA_QK_ON_MFMA
  // Comparison build (python -m mxflashattn_amd._build --qk-mfma): QK always
  // on the matrix cores.
  return 0;
#endif
  if (hd < 128) return 0;
  if (cols <= 1) return 1;
  if (cols <= 2) return 2;
  if (cols <= 4 && hd == 128) return 4;
  return 0;
}

template <int HD, typename T, bool kF8, int kWaveScan>
static int launch_partial_hr(const DecodeParams &p, const Grid &g, hipStream_t st) {
  const int cols = p.gq * p.ql;
  switch (head_rows(cols)) {
    case 1:
      if constexpr (!kF8 && HD >= 128) {
        if (p.ps_log2 >= 4) {
          switch (valu_qk_columns(cols, HD)) {
            case 1: return launch_partial_t<HD, 1, T, kF8, kWaveScan, 1>(p, g, st);
            case 2: return launch_partial_t<HD, 1, T, kF8, kWaveScan, 2>(p, g, st);
            case 4:
              if constexpr (HD == 128) return launch_partial_t<HD, 1, T, kF8, kWaveScan, 4>(p, g, st);
              break;
            default: break;
          }
        }
      }
      return launch_partial_t<HD, 1, T, kF8, kWaveScan>(p, g, st);
    case 2: return launch_partial_t<HD, 2, T, kF8, kWaveScan>(p, g, st);
    default: return launch_partial_t<HD, 4, T, kF8, kWaveScan>(p, g, st);
  }
}

// Partial kernel for one head dim: dtype of q/out (MXFA_DTYPE_F16/BF16), fp8
// caches or caches of that dtype; kWaveScan the sequences per lane of the
// wave-local scan, or 0 (the caller's choice).
template <int HD, int kWaveScan>
int launch_partial_hd(const DecodeParams &p, const Grid &g, int dtype, bool fp8,
                      hipStream_t st) {
  if (dtype == MXFA_DTYPE_BF16)
    return fp8 ? launch_partial_hr<HD, BF16, true, kWaveScan>(p, g, st)
               : launch_partial_hr<HD, BF16, false, kWaveScan>(p, g, st);
  return fp8 ? launch_partial_hr<HD, F16, true, kWaveScan>(p, g, st)
             : launch_partial_hr<HD, F16, false, kWaveScan>(p, g, st);
}

// Per-sequence kernel (seq_decode_kernel): grid (ceil(HKV / KH), B) of
// kSeqWaves = KH * S waves, KH = p.heads_per_wg, S = p.subs. Four waves of one
// kv head beat eight (one or two kv heads) on every short-context shape
// measured. Register budget for two waves per SIMD: four per SIMD spill and
// measured 3-7 % slower at 16-bit HD 64 (19 % at B 128, 8 kv heads, L <= 512).
// Head dim 256 gets one wave per SIMD: its two-wave builds spilled 65-200
// VGPRs and returned wrong outputs (max error 0.6-1.9 on a seeded case, the
// same case right with one wave per SIMD); nothing spills with one.
constexpr int kSeqWaves = 4;
template <int HD>
constexpr int kSeqOcc = HD >= 256 ? 1 : 2;

// LDS bytes of the per-sequence kernel's pieces, and the most it takes.
inline size_t seq_lds_bytes(int hd, int cols) {
  return (size_t)kSeqWaves * cols * (hd + 1) * sizeof(float);
}
constexpr size_t kSeqLdsMax = (size_t)64 << 10;

template <int HD, int HR, typename T, bool kF8, bool kExtras>
static void launch_seq_x(const DecodeParams &p, hipStream_t st) {
  // The kernel assumes one kv head per workgroup and kSeqWaves waves on it.
  dim3 grid(p.hkv, p.batch);
  const size_t lds = seq_lds_bytes(HD, p.gq * p.ql);
  if (p.ps_log2 >= 4)
    hipLaunchKernelGGL((seq_decode_kernel<HD, HR, T, kF8, false, kNbuf<HD, kF8>, kSeqWaves,
                                          kSeqOcc<HD>, kExtras>),
                       grid, dim3(kSeqWaves * 64), lds, st, p.seqlens, p.bt, p.bt_stride,
                       p.max_len, p.seqlen_add, p.ps_log2, p);
  else
    hipLaunchKernelGGL((seq_decode_kernel<HD, HR, T, kF8, true, 2, kSeqWaves, kSeqOcc<HD>,
                                          kExtras>),
                       grid, dim3(kSeqWaves * 64), lds, st, p.seqlens, p.bt, p.bt_stride,
                       p.max_len, p.seqlen_add, p.ps_log2, p);
}

template <int HD, int HR, typename T, bool kF8>
static int launch_seq_t(const DecodeParams &p, hipStream_t st) {
  if (p.window_left >= 0 || p.softcap > 0.f || p.sinks || p.alibi)
    launch_seq_x<HD, HR, T, kF8, true>(p, st);
  else
    launch_seq_x<HD, HR, T, kF8, false>(p, st);
  return hipGetLastError() == hipSuccess ? MXFA_OK : MXFA_ELAUNCH;
}

template <int HD, typename T, bool kF8>
static int launch_seq_hr(const DecodeParams &p, hipStream_t st) {
  switch (head_rows(p.gq * p.ql)) {
    case 1: return launch_seq_t<HD, 1, T, kF8>(p, st);
    case 2: return launch_seq_t<HD, 2, T, kF8>(p, st);
    default: return launch_seq_t<HD, 4, T, kF8>(p, st);
  }
}

template <int HD>
int launch_seq_hd(const DecodeParams &p, int dtype, bool fp8, hipStream_t st) {
  if (p.heads_per_wg != 1 || p.subs != kSeqWaves) return MXFA_ELAUNCH;  // the kernel's shape
  if (dtype == MXFA_DTYPE_BF16)
    return fp8 ? launch_seq_hr<HD, BF16, true>(p, st) : launch_seq_hr<HD, BF16, false>(p, st);
  return fp8 ? launch_seq_hr<HD, F16, true>(p, st) : launch_seq_hr<HD, F16, false>(p, st);
}

// Streaming probe launch (16-bit caches, page size >= 16): the decode
// kernel's grid and waves; nbuf 0 takes the decode kernel's register sets.
template <int HD, int WAVES, int kWaveScan>
static int launch_probe_s(const DecodeParams &p, const Grid &g, int nbuf, uint32_t *sink,
                          hipStream_t st) {
  dim3 grid(g.gx, g.gy);
  const size_t lds = kWaveScan ? 0 : (size_t)(p.batch + 1) * sizeof(int32_t);
  switch (nbuf == 0 ? kNbuf<HD, false> : nbuf) {
    case 2:
      hipLaunchKernelGGL((stream_probe_kernel<HD, BF16, 2, WAVES, kWaveScan>), grid,
                         dim3(WAVES * 64), lds, st, p.seqlens, p.batch, p, sink);
      break;
    case 3:
      hipLaunchKernelGGL((stream_probe_kernel<HD, BF16, 3, WAVES, kWaveScan>), grid,
                         dim3(WAVES * 64), lds, st, p.seqlens, p.batch, p, sink);
      break;
    case 4:
      hipLaunchKernelGGL((stream_probe_kernel<HD, BF16, 4, WAVES, kWaveScan>), grid,
                         dim3(WAVES * 64), lds, st, p.seqlens, p.batch, p, sink);
      break;
    default: return MXFA_EUNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? MXFA_OK : MXFA_ELAUNCH;
}

template <int HD, int WAVES>
static int launch_probe_w(const DecodeParams &p, const Grid &g, int nbuf, uint32_t *sink,
                          hipStream_t st) {
  switch (wave_scan_per_lane(p.batch)) {
    case 1: return launch_probe_s<HD, WAVES, 1>(p, g, nbuf, sink, st);
    case 4: return launch_probe_s<HD, WAVES, 4>(p, g, nbuf, sink, st);
    default: return launch_probe_s<HD, WAVES, 0>(p, g, nbuf, sink, st);
  }
}

template <int HD>
int launch_probe_hd(const DecodeParams &p, const Grid &g, int nbuf, uint32_t *sink,
                    hipStream_t st) {
  if (g.heads_per_wg * g.subs > g.waves || p.ps_log2 < 4) return MXFA_ELAUNCH;
  if constexpr (kMaxWaves<HD, false> == 8) {
    if (g.waves == 8) return launch_probe_w<HD, 8>(p, g, nbuf, sink, st);
  }
  if (g.waves != 4) return MXFA_ELAUNCH;
  return launch_probe_w<HD, 4>(p, g, nbuf, sink, st);
}

template <int HD>
int launch_combine_hd(const CombineParams &c, int dtype, hipStream_t st) {
  // One block per (sequence, heads_per_block rows of (query token, head),
  // 1/chunk_parts of the head dim).
  if (c.chunk_parts < 1 || (HD / 32) % c.chunk_parts || (c.chunk_parts > 1 && c.heads_per_block != 1))
    return MXFA_ELAUNCH;
  const int nblk =
      (c.hq * c.ql + c.heads_per_block - 1) / c.heads_per_block * c.chunk_parts;
  dim3 grid(c.batch * nblk);
  if (dtype == MXFA_DTYPE_BF16)
    hipLaunchKernelGGL((split_combine_kernel<HD, BF16>), grid, dim3(kCombineThreads), 0, st,
                       c.ws_s, c.ws_o, c.ws_lse, c.batch, nblk, c.heads_per_block,
                       c.chunk_parts, c.hq, c.ql, c.gq, c.num_ranges, c);
  else
    hipLaunchKernelGGL((split_combine_kernel<HD, F16>), grid, dim3(kCombineThreads), 0, st,
                       c.ws_s, c.ws_o, c.ws_lse, c.batch, nblk, c.heads_per_block,
                       c.chunk_parts, c.hq, c.ql, c.gq, c.num_ranges, c);
  return hipGetLastError() == hipSuccess ? MXFA_OK : MXFA_ELAUNCH;
}

}  // namespace mxfa

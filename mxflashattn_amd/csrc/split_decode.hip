// C ABI of the split-KV paged decode kernels (include/mxfa_mi355x.h): argument
// checks, launch shapes, workspace layout and the split-count heuristic. The
// kernels live in split_kernels.h and are compiled per head dim
// (split_hd64.hip, split_hd128.hip, split_hd256.hip).
//
// Reference counterpart: the C launcher mxfa_paged_decode_split_launch and
// launch_split (csrc_native/m1_kernel.cpp:970-1003,1206-1222), the binding's
// workspace allocation (csrc_native/m1_binding.cpp:94-97) and the split count
// of integrations/vllm/vllm_plugin.py:271-276.

#include <mutex>

#include "split_kernels.h"

namespace mxfa {

// Workspace of mxfa_split_decode_noalloc_launch: one array per GPU (each
// device holds its own copy at its own address), alive until the process
// ends. Host code never passes `scratch` itself to a kernel: its host-side
// name is a stand-in, not a device address. scratch_address() looks the
// address up once per device, with that device current.
static __device__ __align__(256) unsigned char scratch[MXFA_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mutex;
static void *g_scratch_ptr[kMaxScratchDevices];

// The lookup enqueues no work on any stream. When a device's first call comes
// while this thread captures a graph, the lookup runs with the thread's
// capture mode relaxed for its duration (a global-mode capture would count a
// first-use module load as an unsafe call), then the mode is restored.
static int scratch_address(void **ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return MXFA_ELAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const bool swapped = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
    void *p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (swapped) hipThreadExchangeStreamCaptureMode(&mode);
    if (err != hipSuccess || !p) return MXFA_ELAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return MXFA_OK;
}

int launch_partial_64(const DecodeParams &p, const Grid &g, int dtype, bool fp8, hipStream_t st);
int launch_partial_128(const DecodeParams &p, const Grid &g, int dtype, bool fp8, hipStream_t st);
int launch_partial_256(const DecodeParams &p, const Grid &g, int dtype, bool fp8, hipStream_t st);
int launch_partial_64_ws(const DecodeParams &p, const Grid &g, int dtype, bool fp8,
                         hipStream_t st);
int launch_partial_128_ws(const DecodeParams &p, const Grid &g, int dtype, bool fp8,
                          hipStream_t st);
int launch_partial_256_ws(const DecodeParams &p, const Grid &g, int dtype, bool fp8,
                          hipStream_t st);
int launch_partial_64_ws4(const DecodeParams &p, const Grid &g, int dtype, bool fp8,
                          hipStream_t st);
int launch_partial_128_ws4(const DecodeParams &p, const Grid &g, int dtype, bool fp8,
                           hipStream_t st);
int launch_partial_256_ws4(const DecodeParams &p, const Grid &g, int dtype, bool fp8,
                           hipStream_t st);
int launch_combine_64(const CombineParams &c, int dtype, hipStream_t st);
int launch_combine_128(const CombineParams &c, int dtype, hipStream_t st);
int launch_combine_256(const CombineParams &c, int dtype, hipStream_t st);
int launch_seq_64(const DecodeParams &p, int dtype, bool fp8, hipStream_t st);
int launch_seq_128(const DecodeParams &p, int dtype, bool fp8, hipStream_t st);
int launch_seq_256(const DecodeParams &p, int dtype, bool fp8, hipStream_t st);
int launch_probe_64(const DecodeParams &p, const Grid &g, int nbuf, uint32_t *sink,
                    hipStream_t st);
int launch_probe_128(const DecodeParams &p, const Grid &g, int nbuf, uint32_t *sink,
                     hipStream_t st);

static bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15u) == 0; }

static int ilog2_exact(int v) {
  if (v <= 0 || (v & (v - 1)) != 0) return -1;
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}

static bool supported_hd(int hd) { return hd == 64 || hd == 128 || hd == 256; }

// Output rows (batch, query token, head) of `hd` contiguous elements never
// share an element: with the dims of more than one entry sorted by stride,
// each stride covers the whole extent of the dims below it (the innermost
// covers a row). Different workgroups write different rows, so rows that
// overlap (an expand()ed view, a head stride below the head dim) would race.
static bool rows_disjoint(const int64_t (&size)[3], const int64_t (&stride)[3], int64_t hd) {
  int64_t sz[3], sd[3];
  int n = 0;
  for (int i = 0; i < 3; ++i) {
    if (size[i] <= 1) continue;
    int j = n++;
    for (; j > 0 && sd[j - 1] > stride[i]; --j) {
      sz[j] = sz[j - 1];
      sd[j] = sd[j - 1];
    }
    sz[j] = size[i];
    sd[j] = stride[i];
  }
  int64_t extent = hd;  // elements spanned by the dims below the current one
  for (int i = 0; i < n; ++i) {
    if (sd[i] < extent) return false;
    extent = sd[i] * (sz[i] - 1) + extent;
  }
  return true;
}

struct SplitArgs {
  const void *q;
  int64_t q_sb, q_st, q_sh;
  const void *k, *v;
  int64_t c_sp, c_st, c_sh;  // cache strides in elements (bytes for fp8 caches)
  const int32_t *bt;
  int64_t bt_stride;
  const int32_t *seqlens;
  int seqlen_add;
  void *out;
  int64_t o_sb, o_st, o_sh;
  void *ws;
  size_t ws_bytes;
  float scale;
  int batch, hq, hkv, hd, ps, btw, num_pages, dtype, num_splits;
  bool fp8;  // caches hold OCP e4m3fn
  const float *k_scale, *v_scale;
  int ql;      // query tokens per sequence
  int causal;  // bottom-right aligned causal mask
  int window_left;  // sliding window (keys >= position - window_left), -1: none
  const float *sinks;  // per query head softmax sink logits, nullptr: none
  float softcap;       // logit soft-capping (0: none)
  const float *alibi;  // per query head ALiBi slopes, nullptr: none
  int min_seqlen_add;  // 0, or -2^30 where lengths below zero count as 0
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

// Checks common to every decode launch; the workspace is checked by the caller.
static int check_call_args(const SplitArgs &a) {
  if (!a.q || !a.k || !a.v || !a.bt || !a.seqlens || !a.out) return MXFA_EINVAL;
  if (a.batch <= 0 || a.hq <= 0 || a.hkv <= 0 || a.btw <= 0 || a.num_pages <= 0)
    return MXFA_EINVAL;
  if ((a.num_splits <= 0 && a.num_splits != MXFA_SPLITS_PER_SEQUENCE) ||
      a.seqlen_add < a.min_seqlen_add)
    return MXFA_EINVAL;
  if (!(a.scale == a.scale) || a.scale == INFINITY || a.scale == -INFINITY) return MXFA_EINVAL;
  if (!supported_hd(a.hd)) return MXFA_EUNSUPPORTED;
  if (a.hq % a.hkv != 0) return MXFA_EUNSUPPORTED;
  const int gq = a.hq / a.hkv;
  if (a.ql <= 0 || a.window_left < -1) return MXFA_EINVAL;
  if (!(a.softcap >= 0.f) || a.softcap == INFINITY) return MXFA_EINVAL;
  if (a.window_left > (1 << 30)) return MXFA_EUNSUPPORTED;
  if (gq * a.ql > kMaxCols) return MXFA_EUNSUPPORTED;
  if (a.dtype != MXFA_DTYPE_F16 && a.dtype != MXFA_DTYPE_BF16) return MXFA_EUNSUPPORTED;
  if (ilog2_exact(a.ps) < 0 || a.ps > 4096) return MXFA_EUNSUPPORTED;
  if (a.num_splits > 65535 || a.batch > kMaxBatch || a.hkv > 65535) return MXFA_EUNSUPPORTED;
  const int64_t max_len = (int64_t)a.btw * a.ps;
  if (max_len > (int64_t)1 << 30) return MXFA_EUNSUPPORTED;
  // Total tiles must fit int32: B * ceil(max_len / 16).
  if ((int64_t)a.batch * ((max_len + kTile - 1) / kTile) >= ((int64_t)1 << 31))
    return MXFA_EUNSUPPORTED;
  // 16-byte fragments: pointers and every byte stride must keep 16-byte
  // alignment (8 elements of 16 bits, 16 fp8 elements).
  const int64_t esz = a.fp8 ? 1 : 2;
  if (!aligned16(a.q) || !aligned16(a.k) || !aligned16(a.v)) return MXFA_EINVAL;
  if ((a.q_sb | a.q_st | a.q_sh) & 7) return MXFA_EINVAL;
  if (((a.c_sp | a.c_st | a.c_sh) * esz) & 15) return MXFA_EINVAL;
  if (a.q_sb < 0 || a.q_st < 0 || a.q_sh < 0 || a.c_sp < 0 || a.c_st < 0 || a.c_sh < 0 ||
      a.bt_stride < 0)
    return MXFA_EINVAL;
  // Rows must not overlap: the per-tile descriptors cover whole rows.
  if ((a.ps > 1 && a.c_st < a.hd) || (gq > 1 && a.q_sh < a.hd)) return MXFA_EINVAL;
  // Byte offsets inside a tile and inside a q group are 32-bit.
  if (((int64_t)(kTile - 1) * a.c_st + a.hd) * esz >= ((int64_t)1 << 30))
    return MXFA_EUNSUPPORTED;
  if ((int64_t)(a.ps - 1) * a.c_st * esz >= ((int64_t)1 << 32) ||
      a.c_sh * esz >= ((int64_t)1 << 32))
    return MXFA_EUNSUPPORTED;
  if (((int64_t)(a.ql - 1) * a.q_st + (int64_t)(gq - 1) * a.q_sh + a.hd) * 2 >=
      ((int64_t)1 << 30))
    return MXFA_EUNSUPPORTED;
  if (((uintptr_t)a.out & 7u) || ((a.o_sb | a.o_st | a.o_sh) & 3) || a.o_sb < 0 ||
      a.o_st < 0 || a.o_sh < 0)
    return MXFA_EINVAL;
  // Output rows of different (sequence, query token, head) triples must not overlap.
  if (!rows_disjoint({a.batch, a.ql, a.hq}, {a.o_sb, a.o_st, a.o_sh}, a.hd)) return MXFA_EINVAL;
  if (((uintptr_t)a.k_scale & 3u) || ((uintptr_t)a.v_scale & 3u) || ((uintptr_t)a.sinks & 3u) ||
      ((uintptr_t)a.alibi & 3u))
    return MXFA_EINVAL;
  return MXFA_OK;
}

static int check_split_args(const SplitArgs &a) {
  const int rc = check_call_args(a);
  if (rc != MXFA_OK) return rc;
  if (a.num_splits == MXFA_SPLITS_PER_SEQUENCE) return MXFA_OK;  // no workspace
  if (!a.ws || !aligned16(a.ws)) return MXFA_EWORKSPACE;
  if (a.ws_bytes < ws_layout(a.batch, a.hq * a.ql, a.hd, a.num_splits).bytes)
    return MXFA_EWORKSPACE;
  return MXFA_OK;
}

#ifdef MXFA_WAVE_STAMPS
static unsigned long long *g_wave_stamps = nullptr;
#endif

static DecodeParams make_params(const SplitArgs &a, const Grid &g) {
  // The per-sequence kernel has no workspace, and the streaming probe none either.
  const bool ws = a.num_splits > 0 && a.ws != nullptr;
  const WsLayout w = ws_layout(a.batch, a.hq * a.ql, a.hd, ws ? a.num_splits : 1);
  const int64_t esz = a.fp8 ? 1 : 2;
  DecodeParams p;
  p.q = (const char *)a.q;
  p.q_sb = a.q_sb * 2;
  p.q_st = a.q_st * 2;
  p.q_sh = a.q_sh * 2;
  p.k = (const char *)a.k;
  p.v = (const char *)a.v;
  p.sp_bytes = a.c_sp * esz;
  p.st_bytes = (uint32_t)(a.c_st * esz);
  p.sh_bytes = (uint32_t)(a.c_sh * esz);
  p.bt = a.bt;
  p.bt_stride = a.bt_stride;
  p.seqlens = a.seqlens;
  p.out = (char *)a.out;
  p.o_sb = a.o_sb * 2;
  p.o_st = a.o_st * 2;
  p.o_sh = a.o_sh * 2;
  p.ws_o = ws ? (float *)a.ws : nullptr;
  p.ws_lse = ws ? (float *)a.ws + w.o_floats : nullptr;
  p.ws_s = ws ? (int32_t *)((float *)a.ws + w.o_floats + w.lse_floats) : nullptr;
  p.k_scale = a.fp8 ? a.k_scale : nullptr;
  p.v_scale = a.fp8 ? a.v_scale : nullptr;
  p.scale_log2 = a.scale * kLog2e;
  p.seqlen_add = a.seqlen_add;
  p.batch = a.batch;
  p.hkv = a.hkv;
  p.gq = a.hq / a.hkv;
  p.ql = a.ql;
  p.causal = a.causal ? 1 : 0;
  p.window_left = a.window_left;
  p.sinks = a.sinks;
  p.softcap = a.softcap;
  p.alibi = a.alibi;
  p.heads_per_wg = g.heads_per_wg;
  p.subs = g.subs;
  p.ps_log2 = ilog2_exact(a.ps);
  p.max_len = a.btw * a.ps;
  p.num_pages = a.num_pages;
  p.num_ranges = a.num_splits;
  p.grid_y = g.gy;
#ifdef MXFA_WAVE_STAMPS
  p.stamps = g_wave_stamps;
#endif
  return p;
}

static int launch_partial(const SplitArgs &a, hipStream_t st) {
  Grid g = grid_for(a.hkv, a.num_splits, waves_for(a.hd * (a.fp8 ? 1 : 2), a.hkv));
  // The host's bound on tiles per range: every sequence at the table's
  // capacity (the lengths are on the device).
  const int64_t cap_tiles = ((int64_t)a.btw * a.ps + kTile - 1) / kTile;
  g.short_ranges = (int64_t)a.batch * cap_tiles <= (int64_t)kShortRangeTiles * a.num_splits;
  const DecodeParams p = make_params(a, g);
  // The tile scan: inside each wave, one or four sequences per lane, or
  // through LDS; four per lane is built for plain calls only.
  int ws = wave_scan_per_lane(a.batch);
  if (ws == 4 && !plain_call(p)) ws = 0;
  switch (a.hd) {
    case 64:
      return ws == 1   ? launch_partial_64_ws(p, g, a.dtype, a.fp8, st)
             : ws == 4 ? launch_partial_64_ws4(p, g, a.dtype, a.fp8, st)
                       : launch_partial_64(p, g, a.dtype, a.fp8, st);
    case 128:
      return ws == 1   ? launch_partial_128_ws(p, g, a.dtype, a.fp8, st)
             : ws == 4 ? launch_partial_128_ws4(p, g, a.dtype, a.fp8, st)
                       : launch_partial_128(p, g, a.dtype, a.fp8, st);
    default:
      return ws == 1   ? launch_partial_256_ws(p, g, a.dtype, a.fp8, st)
             : ws == 4 ? launch_partial_256_ws4(p, g, a.dtype, a.fp8, st)
                       : launch_partial_256(p, g, a.dtype, a.fp8, st);
  }
}

// Rows (query token, head) per combine block: a typical crossing sequence has
// about num_splits / batch + 1 pieces; enough piece groups G (a power of two)
// that they fold in one step of eight loads, then as many rows as fit in the
// block's kCombineThreads / G chunk threads (at most the next power of two of
// the rows per sequence). Where one row's chunks leave too few groups for
// that (few sequences, many ranges), each row's chunks are split over up to
// HD/32 chunk_parts blocks.
static void combine_shape(int batch, int hq, int hd, int num_splits, CombineParams &c) {
  const int ch = hd / 4;
  const int pieces = (num_splits + batch - 1) / batch + 1;
  int groups = 1;
  while (groups * ch < kCombineThreads && groups * 8 < pieces) groups *= 2;
  int h = kCombineThreads / (groups * ch);
  if (h < 1) h = 1;
  // One head per block and still more than eight pieces per thread: split
  // the head's chunks over more blocks, each with more piece groups, down to
  // eight chunks (a whole 128-byte line of a piece) per group: finer splits
  // were slower (two chunks per group at head dim 256: 39.1 against 36.1 µs
  // for one sequence over 512 ranges).
  int parts = 1;
  while (h == 1 && parts < ch / 8 && kCombineThreads / (ch / parts) * 8 < pieces) parts *= 2;
  while (h > 1 && h / 2 >= hq) h /= 2;
  c.heads_per_block = h;
  c.chunk_parts = parts;
}

static int launch_combine(void *ws, void *out, const float *sinks, int64_t o_sb, int64_t o_st,
                          int64_t o_sh,
                          int batch, int hq, int hkv, int ql, int hd, int dtype, int ns,
                          hipStream_t st) {
  const WsLayout w = ws_layout(batch, hq * ql, hd, ns);
  CombineParams c;
  c.ws_o = (const float *)ws;
  c.ws_lse = (const float *)ws + w.o_floats;
  c.ws_s = (const int32_t *)((const float *)ws + w.o_floats + w.lse_floats);
  c.out = (char *)out;
  c.o_sb = o_sb * 2;
  c.o_st = o_st * 2;
  c.o_sh = o_sh * 2;
  c.batch = batch;
  c.hq = hq;
  c.gq = hq / hkv;
  c.ql = ql;
  c.num_ranges = ns;
  combine_shape(batch, hq * ql, hd, ns, c);
  c.sinks = sinks;
#ifdef MXFA_WAVE_STAMPS
  c.stamps = g_wave_stamps ? g_wave_stamps + kStampCombineBase : nullptr;
#endif
  switch (hd) {
    case 64: return launch_combine_64(c, dtype, st);
    case 128: return launch_combine_128(c, dtype, st);
    default: return launch_combine_256(c, dtype, st);
  }
}

static SplitArgs split_args(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                            const void *k_cache, const void *v_cache, int64_t cache_stride_page,
                            int64_t cache_stride_token, int64_t cache_stride_head,
                            const int32_t *block_table, int64_t bt_stride, const int32_t *seqlens,
                            int seqlen_add, void *out, int64_t out_stride_b, int64_t out_stride_h,
                            void *workspace, size_t workspace_bytes, float scale, int batch,
                            int q_heads, int kv_heads, int head_dim, int page_size,
                            int block_table_width, int num_pages, int dtype, int num_splits) {
  SplitArgs a;
  a.q = q;
  a.q_sb = q_stride_b;
  a.q_st = 0;
  a.q_sh = q_stride_h;
  a.k = k_cache;
  a.v = v_cache;
  a.c_sp = cache_stride_page;
  a.c_st = cache_stride_token;
  a.c_sh = cache_stride_head;
  a.bt = block_table;
  a.bt_stride = bt_stride;
  a.seqlens = seqlens;
  a.seqlen_add = seqlen_add;
  a.out = out;
  a.o_sb = out_stride_b;
  a.o_st = 0;
  a.o_sh = out_stride_h;
  a.ws = workspace;
  a.ws_bytes = workspace_bytes;
  a.scale = scale;
  a.batch = batch;
  a.hq = q_heads;
  a.hkv = kv_heads;
  a.hd = head_dim;
  a.ps = page_size;
  a.btw = block_table_width;
  a.num_pages = num_pages;
  a.dtype = dtype;
  a.num_splits = num_splits;
  a.fp8 = false;
  a.k_scale = nullptr;
  a.v_scale = nullptr;
  a.ql = 1;
  a.causal = 0;
  a.window_left = -1;
  a.sinks = nullptr;
  a.softcap = 0.f;
  a.alibi = nullptr;
  a.min_seqlen_add = 0;
  return a;
}

// Per-sequence launch shape: one kv head per workgroup, kSeqWaves waves on it.
static Grid seq_grid(int hkv, int batch) {
  Grid g;
  g.waves = kSeqWaves;
  g.heads_per_wg = 1;
  g.subs = kSeqWaves;
  g.gx = hkv;
  g.gy = batch;
  return g;
}

static int launch_seq(const SplitArgs &a, hipStream_t st) {
  // The pieces live in LDS: at most 64 KB per workgroup (HD 256 with 16 columns needs more).
  if (seq_lds_bytes(a.hd, a.hq / a.hkv * a.ql) > kSeqLdsMax) return MXFA_EUNSUPPORTED;
  const Grid g = seq_grid(a.hkv, a.batch);
  DecodeParams p = make_params(a, g);
  p.num_ranges = 0;
  switch (a.hd) {
    case 64: return launch_seq_64(p, a.dtype, a.fp8, st);
    case 128: return launch_seq_128(p, a.dtype, a.fp8, st);
    default: return launch_seq_256(p, a.dtype, a.fp8, st);
  }
}

static int run_split(const SplitArgs &a, bool with_combine, hipStream_t st) {
  int rc = check_split_args(a);
  if (rc != MXFA_OK) return rc;
  if (a.num_splits == MXFA_SPLITS_PER_SEQUENCE) return launch_seq(a, st);
  rc = launch_partial(a, st);
  if (rc != MXFA_OK || !with_combine) return rc;
  return launch_combine(a.ws, a.out, a.sinks, a.o_sb, a.o_st, a.o_sh, a.batch, a.hq, a.hkv,
                        a.ql, a.hd, a.dtype, a.num_splits, st);
}

static SplitArgs fp8_args(SplitArgs a, const float *k_scale, const float *v_scale) {
  a.fp8 = true;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  return a;
}

static int split_heuristic(int batch, int q_heads, int kv_heads, int head_dim, int elem_bytes,
                           int page_size, int block_table_width, int num_cus, int *num_splits) {
  if (!num_splits) return MXFA_EINVAL;
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || page_size <= 0 ||
      block_table_width <= 0 || num_cus <= 0)
    return MXFA_EINVAL;
  const int row_bytes = head_dim * elem_bytes;
  const int64_t cap = (int64_t)block_table_width * page_size;
  // Short sequences (by the table's capacity C, the one bound known without
  // reading the lengths): the per-sequence kernel, whose four waves per (b,
  // kv head) finish a few tiles each sooner than the split path's tile scan
  // and second launch. Bounds from MI355X sweeps (lengths U[C/2, C], B 1..128,
  // 1, 2 or 8 kv heads, GQ 4): inside them 0.99-1.9x the split path's speed;
  // past them it loses (128-byte rows at C 1024 for most batches, B * HKV >=
  // 512 at C 768; 256-byte rows at C 768, or C 512 with B * HKV < 64; head
  // dim 256, one wave per SIMD, at B * HKV = 1024).
  const int64_t seq_tiles = (cap + kTile - 1) / kTile;
  const int64_t units = (int64_t)batch * kv_heads;
  const int64_t seq_work = units * seq_tiles;
  const bool short_rows = row_bytes <= 128 && cap <= 768;
  const bool mid_rows = row_bytes <= 256 && (cap <= 384 || (cap <= 512 && units >= 64)) &&
                        (head_dim < 256 || seq_work <= 8192);
  // q_heads / kv_heads columns per launch (q_heads * q_len for the multi-token
  // entry point) must fit the kernel's LDS.
  const bool fits = seq_lds_bytes(head_dim, (q_heads + kv_heads - 1) / kv_heads) <= kSeqLdsMax;
  if (page_size >= kTile && seq_work <= 16384 && fits && (short_rows || mid_rows)) {
    *num_splits = MXFA_SPLITS_PER_SEQUENCE;
    return MXFA_OK;
  }
  // One range per wave: one workgroup (waves_for waves) fills every CU, and
  // each wave streams one (kv head, range). The kernel lowers the count to the
  // real tile total on the device.
  const Grid g = grid_for(kv_heads, 1, waves_for(row_bytes, kv_heads));
  int64_t n = (int64_t)num_cus * g.subs / g.gx;
  const int64_t cap_tiles = (int64_t)batch * seq_tiles;
  if (n > cap_tiles) n = cap_tiles;
  if (n < 1) n = 1;
  if (n > 65535) n = 65535;
  *num_splits = (int)n;
  return MXFA_OK;
}

}  // namespace mxfa

using namespace mxfa;

extern "C" {

int mxfa_abi_version(void) { return MXFA_ABI_VERSION; }

#ifdef MXFA_WAVE_STAMPS
// Profiling builds only (not part of the C ABI): device buffer of
// kStampWaves x kStampWords words for the partial and per-sequence kernels'
// waves, then kStampCombineBlocks x kStampCombineWords for the combine
// kernel's blocks, that later launches stamp; nullptr stops.
void mxfa_wave_stamps_set(void *device_buffer) {
  g_wave_stamps = (unsigned long long *)device_buffer;
}
#endif

const char *mxfa_strerror(int code) {
  switch (code) {
    case MXFA_OK: return "ok";
    case MXFA_EUNSUPPORTED:
      return "unsupported configuration (head dim, GQA ratio, dtype or page size)";
    case MXFA_EINVAL: return "invalid argument (null pointer, size, alignment or stride)";
    case MXFA_EWORKSPACE: return "workspace missing or too small";
    case MXFA_ELAUNCH: return "kernel launch failed";
    case MXFA_ESCRATCH:
      return "the call needs more workspace than the no-allocation entry point's 8 MiB "
             "(use mxfa_split_decode_launch with a workspace)";
  }
  return "unknown error";
}

int mxfa_split_heuristic(int batch, int q_heads, int kv_heads, int head_dim, int page_size,
                         int block_table_width, int num_cus, int *num_splits) {
  return split_heuristic(batch, q_heads, kv_heads, head_dim, 2, page_size, block_table_width,
                         num_cus, num_splits);
}

int mxfa_split_heuristic_fp8(int batch, int q_heads, int kv_heads, int head_dim, int page_size,
                             int block_table_width, int num_cus, int *num_splits) {
  return split_heuristic(batch, q_heads, kv_heads, head_dim, 1, page_size, block_table_width,
                         num_cus, num_splits);
}

int mxfa_split_decode_workspace_size(int batch, int q_heads, int head_dim, int num_splits,
                                     size_t *bytes) {
  if (!bytes || batch <= 0 || q_heads <= 0 || head_dim <= 0 ||
      (num_splits <= 0 && num_splits != MXFA_SPLITS_PER_SEQUENCE))
    return MXFA_EINVAL;
  *bytes = num_splits > 0 ? ws_layout(batch, q_heads, head_dim, num_splits).bytes : 0;
  return MXFA_OK;
}

#define MXFA_SPLIT_PARAMS                                                                    \
  const void *q, int64_t q_stride_b, int64_t q_stride_h, const void *k_cache,               \
      const void *v_cache, int64_t cache_stride_page, int64_t cache_stride_token,           \
      int64_t cache_stride_head, const int32_t *block_table, int64_t bt_stride,             \
      const int32_t *seqlens, int seqlen_add, void *out, int64_t out_stride_b,              \
      int64_t out_stride_h, void *workspace, size_t workspace_bytes, float scale, int batch, \
      int q_heads, int kv_heads, int head_dim, int page_size, int block_table_width,        \
      int num_pages, int dtype, int num_splits
#define MXFA_SPLIT_ARGS                                                                      \
  q, q_stride_b, q_stride_h, k_cache, v_cache, cache_stride_page, cache_stride_token,       \
      cache_stride_head, block_table, bt_stride, seqlens, seqlen_add, out, out_stride_b,    \
      out_stride_h, workspace, workspace_bytes, scale, batch, q_heads, kv_heads, head_dim,  \
      page_size, block_table_width, num_pages, dtype, num_splits

int mxfa_split_decode_launch(MXFA_SPLIT_PARAMS, void *stream) {
  return run_split(split_args(MXFA_SPLIT_ARGS), true, (hipStream_t)stream);
}

int mxfa_split_decode_noalloc_launch(
    const void *q, int64_t q_stride_b, int64_t q_stride_h, const void *k_cache,
    const void *v_cache, int64_t cache_stride_page, int64_t cache_stride_token,
    int64_t cache_stride_head, const int32_t *block_table, int64_t bt_stride,
    const int32_t *seqlens, int seqlen_add, void *out, int64_t out_stride_b,
    int64_t out_stride_h, float scale, int batch, int q_heads, int kv_heads, int head_dim,
    int page_size, int block_table_width, int num_pages, int dtype, int num_splits,
    void *stream) {
  if (batch <= 0 || q_heads <= 0 || head_dim <= 0 ||
      (num_splits <= 0 && num_splits != MXFA_SPLITS_PER_SEQUENCE))
    return MXFA_EINVAL;
  const size_t need =
      num_splits > 0 ? ws_layout(batch, q_heads, head_dim, num_splits).bytes : 0;
  if (need > MXFA_SCRATCH_BYTES) return MXFA_ESCRATCH;
  void *ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != MXFA_OK) return rc;
  return run_split(split_args(q, q_stride_b, q_stride_h, k_cache, v_cache, cache_stride_page,
                              cache_stride_token, cache_stride_head, block_table, bt_stride,
                              seqlens, seqlen_add, out, out_stride_b, out_stride_h, ws,
                              MXFA_SCRATCH_BYTES, scale, batch, q_heads, kv_heads, head_dim,
                              page_size, block_table_width, num_pages, dtype, num_splits),
                   true, (hipStream_t)stream);
}

int mxfa_stream_probe_launch(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                             const void *k_cache, const void *v_cache,
                             int64_t cache_stride_page, int64_t cache_stride_token,
                             int64_t cache_stride_head, const int32_t *block_table,
                             int64_t bt_stride, const int32_t *seqlens, int seqlen_add,
                             uint32_t *sink, size_t sink_bytes, int batch, int q_heads,
                             int kv_heads, int head_dim, int page_size, int block_table_width,
                             int num_pages, int dtype, int num_splits, int tiles_in_flight,
                             void *stream) {
  // The probe writes no output; `out` is checked as q (same shape and strides).
  SplitArgs a = split_args(q, q_stride_b, q_stride_h, k_cache, v_cache, cache_stride_page,
                           cache_stride_token, cache_stride_head, block_table, bt_stride,
                           seqlens, seqlen_add, const_cast<void *>(q), q_stride_b, q_stride_h,
                           nullptr, 0, 1.f, batch, q_heads, kv_heads, head_dim, page_size,
                           block_table_width, num_pages, dtype, num_splits);
  int rc = check_call_args(a);
  if (rc != MXFA_OK) return rc;
  if (num_splits <= 0 || (head_dim != 64 && head_dim != 128) || page_size < kTile ||
      (tiles_in_flight != 0 && (tiles_in_flight < 2 || tiles_in_flight > 4)))
    return MXFA_EUNSUPPORTED;
  if (!sink || ((uintptr_t)sink & 3u) || sink_bytes < (size_t)kv_heads * num_splits * 64 * 4)
    return MXFA_EWORKSPACE;
  const Grid g = grid_for(kv_heads, num_splits, waves_for(head_dim * 2, kv_heads));
  const DecodeParams p = make_params(a, g);
  return head_dim == 64 ? launch_probe_64(p, g, tiles_in_flight, sink, (hipStream_t)stream)
                        : launch_probe_128(p, g, tiles_in_flight, sink, (hipStream_t)stream);
}

int mxfa_split_decode_partial_launch(MXFA_SPLIT_PARAMS, void *stream) {
  return run_split(split_args(MXFA_SPLIT_ARGS), false, (hipStream_t)stream);
}

int mxfa_split_decode_fp8_launch(MXFA_SPLIT_PARAMS, const float *k_scale, const float *v_scale,
                                 void *stream) {
  return run_split(fp8_args(split_args(MXFA_SPLIT_ARGS), k_scale, v_scale), true,
                   (hipStream_t)stream);
}

int mxfa_split_decode_fp8_partial_launch(MXFA_SPLIT_PARAMS, const float *k_scale,
                                         const float *v_scale, void *stream) {
  return run_split(fp8_args(split_args(MXFA_SPLIT_ARGS), k_scale, v_scale), false,
                   (hipStream_t)stream);
}

int mxfa_split_decode_combine_launch(void *workspace, size_t workspace_bytes, void *out,
                                     int64_t out_stride_b, int64_t out_stride_h, int batch,
                                     int q_heads, int kv_heads, int head_dim, int dtype,
                                     int num_splits, void *stream) {
  if (num_splits == MXFA_SPLITS_PER_SEQUENCE) return MXFA_OK;  // the one launch merged already
  if (!workspace || !out) return MXFA_EINVAL;
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || num_splits <= 0) return MXFA_EINVAL;
  if (!supported_hd(head_dim)) return MXFA_EUNSUPPORTED;
  if (q_heads % kv_heads != 0 || q_heads / kv_heads > kMaxCols) return MXFA_EUNSUPPORTED;
  if (dtype != MXFA_DTYPE_F16 && dtype != MXFA_DTYPE_BF16) return MXFA_EUNSUPPORTED;
  if (batch > kMaxBatch || num_splits > 65535) return MXFA_EUNSUPPORTED;
  if (!aligned16(workspace) || ((uintptr_t)out & 7u) || ((out_stride_b | out_stride_h) & 3) ||
      out_stride_b < 0 || out_stride_h < 0)
    return MXFA_EINVAL;
  if (!rows_disjoint({batch, 1, q_heads}, {out_stride_b, 0, out_stride_h}, head_dim))
    return MXFA_EINVAL;
  if (workspace_bytes < ws_layout(batch, q_heads, head_dim, num_splits).bytes)
    return MXFA_EWORKSPACE;
  return launch_combine(workspace, out, nullptr, out_stride_b, 0, out_stride_h, batch, q_heads,
                        kv_heads,
                        1, head_dim, dtype, num_splits, (hipStream_t)stream);
}

int mxfa_split_decode_multi_launch(
    const void *q, int64_t q_stride_b, int64_t q_stride_t, int64_t q_stride_h, int q_len,
    int causal, int window_left, const float *sinks, float softcap, const float *alibi_slopes,
    const void *k_cache, const void *v_cache, int64_t cache_stride_page,
    int64_t cache_stride_token, int64_t cache_stride_head, const int32_t *block_table,
    int64_t bt_stride, const int32_t *seqlens, int seqlen_add, void *out, int64_t out_stride_b,
    int64_t out_stride_t, int64_t out_stride_h, void *workspace, size_t workspace_bytes,
    float scale, int batch, int q_heads, int kv_heads, int head_dim, int page_size,
    int block_table_width, int num_pages, int dtype, int kv_dtype, const float *k_scale,
    const float *v_scale, int num_splits, void *stream) {
  SplitArgs a = split_args(q, q_stride_b, q_stride_h, k_cache, v_cache, cache_stride_page,
                           cache_stride_token, cache_stride_head, block_table, bt_stride,
                           seqlens, seqlen_add, out, out_stride_b, out_stride_h, workspace,
                           workspace_bytes, scale, batch, q_heads, kv_heads, head_dim, page_size,
                           block_table_width, num_pages, dtype, num_splits);
  if (kv_dtype == MXFA_DTYPE_FP8_E4M3) a = fp8_args(a, k_scale, v_scale);
  else if (kv_dtype != dtype) return MXFA_EUNSUPPORTED;
  a.q_st = q_stride_t;
  a.o_st = out_stride_t;
  a.ql = q_len;
  a.causal = causal;
  a.window_left = window_left;
  a.sinks = sinks;
  a.softcap = softcap;
  a.alibi = alibi_slopes;
  a.min_seqlen_add = -(1 << 30);  // a window on the tokens before the cache end
  return run_split(a, true, (hipStream_t)stream);
}

}  // extern "C"

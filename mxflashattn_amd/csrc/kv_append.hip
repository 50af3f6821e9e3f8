// Paged KV append for MI355X: bit-exact 16-byte copies of new K/V rows into
// their pages. One thread moves one 16-byte fragment of K and the matching one
// of V, so a wave writes four (HD128) or eight (HD64) whole head rows.
//
// Two index forms share the copy:
//   slot form (vLLM reshape_and_cache): row t goes to slot_mapping[t], skipped if < 0;
//   table form (flash_attn_with_kvcache k=/v=): token t of sequence b goes to
//     logical position seqlens[b] + t, page block_table[b, pos / PS].
// Destinations outside the cache (page id out of range, position beyond the
// block table) are skipped, never written.
//
// fp8 caches (slot form): each element is divided by its tensor's scale in
// fp32 (correctly rounded), saturated to the finite e4m3fn range [-448, 448]
// (NaN stays NaN) and rounded to nearest-even OCP e4m3fn by v_cvt_pk_fp8_f32;
// a thread turns 16 bytes of K (and of V) into 8.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mxfa_device.h"
#include "mxfa_mi355x.h"

namespace mxfa {

struct AppendParams {
  const uint16_t *k;
  const uint16_t *v;
  int64_t s_b, s_t, s_h;  // source strides (batch, token, head); s_b unused in slot form
  uint16_t *kc;
  uint16_t *vc;
  int64_t c_sp, c_st, c_sh;
  const int64_t *slots;    // slot form
  const int32_t *bt;       // table form
  int64_t bt_stride;
  const int32_t *seqlens;  // table form
  int rows;                // slot form: num_tokens; table form: batch * new_tokens
  int new_tokens;
  int hkv;
  int frags;  // 16-byte fragments per head row (HD / 8)
  int ps;
  int btw;
  int num_pages;
};

template <bool kTable>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendParams p) {
  const int64_t total = (int64_t)p.rows * p.hkv * p.frags;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int f = (int)(i % p.frags);
    const int64_t rh = i / p.frags;
    const int h = (int)(rh % p.hkv);
    const int r = (int)(rh / p.hkv);
    int64_t page, off, src;
    if (kTable) {
      const int b = r / p.new_tokens, t = r % p.new_tokens;
      const int64_t pos = (int64_t)p.seqlens[b] + t;
      if (pos < 0) continue;
      const int64_t pidx = pos / p.ps;
      if (pidx >= p.btw) continue;
      page = p.bt[(int64_t)b * p.bt_stride + pidx];
      off = pos % p.ps;
      src = (int64_t)b * p.s_b + (int64_t)t * p.s_t;
    } else {
      const int64_t slot = p.slots[r];
      if (slot < 0) continue;
      page = slot / p.ps;
      off = slot % p.ps;
      src = (int64_t)r * p.s_t;
    }
    if (page < 0 || page >= p.num_pages) continue;
    src += (int64_t)h * p.s_h + f * 8;
    const int64_t dst = page * p.c_sp + off * p.c_st + (int64_t)h * p.c_sh + f * 8;
    *reinterpret_cast<uint4 *>(p.kc + dst) = *reinterpret_cast<const uint4 *>(p.k + src);
    *reinterpret_cast<uint4 *>(p.vc + dst) = *reinterpret_cast<const uint4 *>(p.v + src);
  }
}

struct QuantAppendParams {
  const uint16_t *k;
  const uint16_t *v;
  int64_t s_t, s_h;  // source strides (token, head), elements
  uint8_t *kc;
  uint8_t *vc;
  int64_t c_sp, c_st, c_sh;  // cache strides, bytes
  const int64_t *slots;
  const float *k_scale;
  const float *v_scale;
  int rows;
  int hkv;
  int frags;  // 8-element fragments per head row (HD / 8)
  int ps;
  int num_pages;
};

__device__ __forceinline__ float fp8_saturate(float y) {
  return y != y ? y : fminf(fmaxf(y, -448.f), 448.f);
}

// Eight 16-bit elements divided by s, as eight e4m3fn bytes (byte i = element i).
template <typename T>
__device__ __forceinline__ uint2 quantize8(const uint4 w, float s) {
  using E = Elem<T>;
  const uint32_t in[4] = {w.x, w.y, w.z, w.w};
  uint32_t out[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float a = fp8_saturate(__fdiv_rn(E::lo(in[2 * j]), s));
    const float b = fp8_saturate(__fdiv_rn(E::hi(in[2 * j]), s));
    const float c = fp8_saturate(__fdiv_rn(E::lo(in[2 * j + 1]), s));
    const float d = fp8_saturate(__fdiv_rn(E::hi(in[2 * j + 1]), s));
    int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
    out[j] = (uint32_t)r;
  }
  return make_uint2(out[0], out[1]);
}

template <typename T>
__global__ __launch_bounds__(256) void kv_quant_append_kernel(QuantAppendParams p) {
  const float ks = p.k_scale ? p.k_scale[0] : 1.f;
  const float vs = p.v_scale ? p.v_scale[0] : 1.f;
  const int64_t total = (int64_t)p.rows * p.hkv * p.frags;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int f = (int)(i % p.frags);
    const int64_t rh = i / p.frags;
    const int h = (int)(rh % p.hkv);
    const int r = (int)(rh / p.hkv);
    const int64_t slot = p.slots[r];
    if (slot < 0) continue;
    const int64_t page = slot / p.ps, off = slot % p.ps;
    if (page >= p.num_pages) continue;
    const int64_t src = (int64_t)r * p.s_t + (int64_t)h * p.s_h + f * 8;
    const int64_t dst = page * p.c_sp + off * p.c_st + (int64_t)h * p.c_sh + f * 8;
    *reinterpret_cast<uint2 *>(p.kc + dst) =
        quantize8<T>(*reinterpret_cast<const uint4 *>(p.k + src), ks);
    *reinterpret_cast<uint2 *>(p.vc + dst) =
        quantize8<T>(*reinterpret_cast<const uint4 *>(p.v + src), vs);
  }
}

static bool al16(const void *ptr) { return ((uintptr_t)ptr & 15u) == 0; }

template <bool kTable>
static int launch_append(const AppendParams &p, hipStream_t st) {
  const int64_t total = (int64_t)p.rows * p.hkv * p.frags;
  if (total == 0) return MXFA_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL((kv_append_kernel<kTable>), dim3((unsigned)blocks), dim3(256), 0, st, p);
  return hipGetLastError() == hipSuccess ? MXFA_OK : MXFA_ELAUNCH;
}

static int check_common(const void *k, const void *v, const void *kc, const void *vc,
                        int64_t s_t, int64_t s_h, int64_t c_sp, int64_t c_st, int64_t c_sh,
                        int hkv, int hd, int ps, int num_pages, int dtype) {
  if (!k || !v || !kc || !vc) return MXFA_EINVAL;
  if (hkv <= 0 || ps <= 0 || num_pages <= 0) return MXFA_EINVAL;
  if (hd <= 0 || hd % 8 != 0 || hd > 4096) return MXFA_EUNSUPPORTED;
  if (dtype != MXFA_DTYPE_F16 && dtype != MXFA_DTYPE_BF16) return MXFA_EUNSUPPORTED;
  if (!al16(k) || !al16(v) || !al16(kc) || !al16(vc)) return MXFA_EINVAL;
  if ((s_t | s_h | c_sp | c_st | c_sh) & 7) return MXFA_EINVAL;
  if (s_t < 0 || s_h < 0 || c_sp < 0 || c_st < 0 || c_sh < 0) return MXFA_EINVAL;
  return MXFA_OK;
}

}  // namespace mxfa

using namespace mxfa;

extern "C" {

int mxfa_reshape_and_cache_launch(const void *key, const void *value, int64_t kv_stride_token,
                                  int64_t kv_stride_head, void *k_cache, void *v_cache,
                                  int64_t cache_stride_page, int64_t cache_stride_token,
                                  int64_t cache_stride_head, const int64_t *slot_mapping,
                                  int num_tokens, int kv_heads, int head_dim, int page_size,
                                  int num_pages, int dtype, void *stream) {
  if (num_tokens < 0) return MXFA_EINVAL;
  if (num_tokens > 0 && !slot_mapping) return MXFA_EINVAL;
  int rc = check_common(key, value, k_cache, v_cache, kv_stride_token, kv_stride_head,
                        cache_stride_page, cache_stride_token, cache_stride_head, kv_heads,
                        head_dim, page_size, num_pages, dtype);
  if (rc != MXFA_OK) return rc;
  AppendParams p{};
  p.k = (const uint16_t *)key;
  p.v = (const uint16_t *)value;
  p.s_b = 0;
  p.s_t = kv_stride_token;
  p.s_h = kv_stride_head;
  p.kc = (uint16_t *)k_cache;
  p.vc = (uint16_t *)v_cache;
  p.c_sp = cache_stride_page;
  p.c_st = cache_stride_token;
  p.c_sh = cache_stride_head;
  p.slots = slot_mapping;
  p.rows = num_tokens;
  p.new_tokens = 1;
  p.hkv = kv_heads;
  p.frags = head_dim / 8;
  p.ps = page_size;
  p.num_pages = num_pages;
  return launch_append<false>(p, (hipStream_t)stream);
}

int mxfa_reshape_and_cache_fp8_launch(const void *key, const void *value,
                                      int64_t kv_stride_token, int64_t kv_stride_head,
                                      void *k_cache, void *v_cache, int64_t cache_stride_page,
                                      int64_t cache_stride_token, int64_t cache_stride_head,
                                      const int64_t *slot_mapping, int num_tokens, int kv_heads,
                                      int head_dim, int page_size, int num_pages, int dtype,
                                      const float *k_scale, const float *v_scale, void *stream) {
  if (num_tokens < 0) return MXFA_EINVAL;
  if (num_tokens > 0 && !slot_mapping) return MXFA_EINVAL;
  if (!key || !value || !k_cache || !v_cache) return MXFA_EINVAL;
  if (kv_heads <= 0 || page_size <= 0 || num_pages <= 0) return MXFA_EINVAL;
  if (head_dim <= 0 || head_dim % 16 != 0 || head_dim > 4096) return MXFA_EUNSUPPORTED;
  if (dtype != MXFA_DTYPE_F16 && dtype != MXFA_DTYPE_BF16) return MXFA_EUNSUPPORTED;
  if (!al16(key) || !al16(value) || !al16(k_cache) || !al16(v_cache)) return MXFA_EINVAL;
  if (((uintptr_t)k_scale & 3u) || ((uintptr_t)v_scale & 3u)) return MXFA_EINVAL;
  if ((kv_stride_token | kv_stride_head) & 7) return MXFA_EINVAL;
  if ((cache_stride_page | cache_stride_token | cache_stride_head) & 15) return MXFA_EINVAL;
  if (kv_stride_token < 0 || kv_stride_head < 0 || cache_stride_page < 0 ||
      cache_stride_token < 0 || cache_stride_head < 0)
    return MXFA_EINVAL;
  QuantAppendParams p{};
  p.k = (const uint16_t *)key;
  p.v = (const uint16_t *)value;
  p.s_t = kv_stride_token;
  p.s_h = kv_stride_head;
  p.kc = (uint8_t *)k_cache;
  p.vc = (uint8_t *)v_cache;
  p.c_sp = cache_stride_page;
  p.c_st = cache_stride_token;
  p.c_sh = cache_stride_head;
  p.slots = slot_mapping;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.rows = num_tokens;
  p.hkv = kv_heads;
  p.frags = head_dim / 8;
  p.ps = page_size;
  p.num_pages = num_pages;
  const int64_t total = (int64_t)p.rows * p.hkv * p.frags;
  if (total == 0) return MXFA_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MXFA_DTYPE_BF16)
    hipLaunchKernelGGL((kv_quant_append_kernel<BF16>), dim3((unsigned)blocks), dim3(256), 0, st,
                       p);
  else
    hipLaunchKernelGGL((kv_quant_append_kernel<F16>), dim3((unsigned)blocks), dim3(256), 0, st,
                       p);
  return hipGetLastError() == hipSuccess ? MXFA_OK : MXFA_ELAUNCH;
}

int mxfa_append_kv_launch(const void *k, const void *v, int64_t kv_stride_b,
                          int64_t kv_stride_token, int64_t kv_stride_head, void *k_cache,
                          void *v_cache, int64_t cache_stride_page, int64_t cache_stride_token,
                          int64_t cache_stride_head, const int32_t *block_table,
                          int64_t bt_stride, const int32_t *seqlens, int batch, int new_tokens,
                          int kv_heads, int head_dim, int page_size, int block_table_width,
                          int num_pages, int dtype, void *stream) {
  if (batch < 0 || new_tokens < 0 || block_table_width <= 0 || bt_stride < 0) return MXFA_EINVAL;
  if (batch > 0 && new_tokens > 0 && (!block_table || !seqlens)) return MXFA_EINVAL;
  if ((kv_stride_b & 7) || kv_stride_b < 0) return MXFA_EINVAL;
  int rc = check_common(k, v, k_cache, v_cache, kv_stride_token, kv_stride_head,
                        cache_stride_page, cache_stride_token, cache_stride_head, kv_heads,
                        head_dim, page_size, num_pages, dtype);
  if (rc != MXFA_OK) return rc;
  if ((int64_t)batch * new_tokens > (int64_t)1 << 30) return MXFA_EUNSUPPORTED;
  AppendParams p{};
  p.k = (const uint16_t *)k;
  p.v = (const uint16_t *)v;
  p.s_b = kv_stride_b;
  p.s_t = kv_stride_token;
  p.s_h = kv_stride_head;
  p.kc = (uint16_t *)k_cache;
  p.vc = (uint16_t *)v_cache;
  p.c_sp = cache_stride_page;
  p.c_st = cache_stride_token;
  p.c_sh = cache_stride_head;
  p.bt = block_table;
  p.bt_stride = bt_stride;
  p.seqlens = seqlens;
  p.rows = batch * new_tokens;
  p.new_tokens = new_tokens > 0 ? new_tokens : 1;
  p.hkv = kv_heads;
  p.frags = head_dim / 8;
  p.ps = page_size;
  p.btw = block_table_width;
  p.num_pages = num_pages;
  return launch_append<true>(p, (hipStream_t)stream);
}

}  // extern "C"

// Device helpers shared by the gfx950 kernels: element types (exact widening
// of 16-bit halves, fp32 -> fp16/bf16 rounding), the DPP row broadcast,
// nontemporal loads and raw buffer descriptors.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxfa {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct F16 {};
struct BF16 {};

template <typename T>
struct Elem;

// fp16: widening by v_cvt_f32_f16, RNE narrowing.
template <>
struct Elem<F16> {
  static __device__ __forceinline__ float lo(uint32_t x) {
    return (float)__builtin_bit_cast(half2_t, x).x;
  }
  static __device__ __forceinline__ float hi(uint32_t x) {
    return (float)__builtin_bit_cast(half2_t, x).y;
  }
  static __device__ __forceinline__ uint16_t narrow(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
};

// bf16: widening is a 16-bit shift (exact); RNE narrowing.
template <>
struct Elem<BF16> {
  static __device__ __forceinline__ float lo(uint32_t x) { return __uint_as_float(x << 16); }
  static __device__ __forceinline__ float hi(uint32_t x) {
    return __uint_as_float(x & 0xffff0000u);
  }
  static __device__ __forceinline__ uint16_t narrow(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
  }
};

// DPP control row_newbcast:n = 0x150 + n (lane n of each 16-lane row to the row).
constexpr int kDppRowNewBcast0 = 0x150;
// row_shr:n = 0x110 + n (lane i of a row takes lane i - n of the same row);
// row_bcast:15 / row_bcast:31 (lane 15 of each row to the next row / lane 31
// to rows 2 and 3).
constexpr int kDppRowShr0 = 0x110;
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;
// quad_perm:[1,0,3,2] and quad_perm:[2,3,0,1] (lane i of each group of four
// takes lane i^1, then lane i^2).
constexpr int kDppQuadSwap1 = 0xB1;
constexpr int kDppQuadSwap2 = 0x4E;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Streaming loads of KV rows: every byte is read once per call, so the loads
// carry the nontemporal hint and do not displace reusable lines from the
// caches (measured on MI355X: about +10% read bandwidth on paged gathers).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t load_stream4(const void *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
}
__device__ __forceinline__ uint4 load_stream16(const void *p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 load_stream8(const void *p) {
  const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(p));
  return make_uint2(v.x, v.y);
}

// Raw buffer descriptors: loads at byte offsets at or past `bytes` return
// zeros and touch no memory.
constexpr uint32_t kSrdWord3 = 0x00020000u;  // raw 32-bit buffer, gfx9 family
constexpr int kAuxStream = 2;                // nt: no temporal reuse expected

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_srd(const char *base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(base), (short)0, bytes, kSrdWord3);
}

template <int Aux>
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, int off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, Aux);
  return make_uint4(v.x, v.y, v.z, v.w);
}

}  // namespace mxfa

// Plain streaming read for MI355X (a measurement aid): one pass over a buffer
// with 16-byte non-temporal buffer loads and no other work, the device's read
// ceiling against which the decode gather (stream_probe_kernel) and the decode
// kernels are compared at the same byte counts.
//
// A launch of G workgroups of four waves; each wave reads, per step, one
// chunk of kDepth KB (lane l loads bytes [16 l + 1024 i, +16) of it for
// i < kDepth, all issued before any is used) and folds the words into an XOR.
// Layout 0: wave w reads the w-th of 4G equal contiguous slices, chunk after
// chunk. Layout 1: the waves take consecutive chunks in turn (chunk c by wave
// c mod 4G), so the whole launch sweeps one window of the buffer. Each chunk
// gets its own descriptor sized to the bytes left, so loads past the end read
// zeros and touch no memory. Lane l of wave w writes its XOR to
// sink[64 w + l]: the XOR of the sink is the XOR of the buffer's words when
// every word was read once.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mxfa_device.h"
#include "mxfa_mi355x.h"

namespace mxfa {

template <int kDepth>
__global__ __launch_bounds__(256) void stream_read_kernel(const char *buf, uint64_t bytes,
                                                          uint64_t slice, int layout,
                                                          uint32_t *sink) {
  constexpr uint32_t kChunk = 64u * 16u * kDepth;  // bytes a wave reads per step
  const int lane = threadIdx.x & 63;
  const uint64_t waves = (uint64_t)gridDim.x * 4;
  // The wave index through readfirstlane: the compiler then knows it is the
  // same in every lane, so each chunk's descriptor is built in scalar
  // registers (a per-lane one would wrap every load in a loop over lanes).
  const uint64_t w = (uint64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint32_t x = 0;
  auto step = [&](uint64_t off, uint64_t end) {
    const uint64_t left = end - off;
    const __amdgpu_buffer_rsrc_t r = make_srd(buf + off, (int)(left < kChunk ? left : kChunk));
    uint4 v[kDepth];
#pragma unroll
    for (int i = 0; i < kDepth; ++i) v[i] = buf_load16<kAuxStream>(r, lane * 16 + i * 1024);
#pragma unroll
    for (int i = 0; i < kDepth; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  };
  if (layout == 0) {  // slice: bytes per wave, a multiple of 16 (host)
    const uint64_t lo = w * slice < bytes ? w * slice : bytes;
    const uint64_t hi = bytes - lo < slice ? bytes : lo + slice;
    for (uint64_t off = lo; off < hi; off += kChunk) step(off, hi);
  } else {
    for (uint64_t off = w * kChunk; off < bytes; off += waves * kChunk) step(off, bytes);
  }
  sink[w * 64 + lane] = x;
}

}  // namespace mxfa

using namespace mxfa;

extern "C" int mxfa_stream_read_launch(const void *buf, uint64_t bytes, int layout, int depth,
                                       int workgroups, uint32_t *sink, size_t sink_bytes,
                                       void *stream) {
  if (!buf || ((uintptr_t)buf & 15u) || bytes == 0 || (bytes & 15u) || workgroups <= 0 ||
      (layout != 0 && layout != 1))
    return MXFA_EINVAL;
  if (depth != 4 && depth != 8 && depth != 16) return MXFA_EUNSUPPORTED;
  if (!sink || ((uintptr_t)sink & 3u) || sink_bytes / 1024 < (size_t)workgroups)
    return MXFA_EWORKSPACE;
  const char *b = static_cast<const char *>(buf);
  const uint64_t waves = (uint64_t)workgroups * 4;
  const uint64_t slice = ((bytes + waves - 1) / waves + 15) & ~(uint64_t)15;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(workgroups), block(256);
  if (depth == 4)
    hipLaunchKernelGGL(stream_read_kernel<4>, grid, block, 0, st, b, bytes, slice, layout, sink);
  else if (depth == 8)
    hipLaunchKernelGGL(stream_read_kernel<8>, grid, block, 0, st, b, bytes, slice, layout, sink);
  else
    hipLaunchKernelGGL(stream_read_kernel<16>, grid, block, 0, st, b, bytes, slice, layout, sink);
  return hipGetLastError() == hipSuccess ? MXFA_OK : MXFA_ELAUNCH;
}

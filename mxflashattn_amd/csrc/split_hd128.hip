// Instantiation unit of the split decode kernels for head dim 128: the partial
// kernel with the LDS tile scan, the per-sequence, combine and probe kernels
// (the units compile in parallel; the C ABI in split_decode.hip calls these).
#include "split_kernels.h"

namespace mxfa {

int launch_partial_128(const DecodeParams &p, const Grid &g, int dtype, bool fp8,
                       hipStream_t st) {
  return launch_partial_hd<128, 0>(p, g, dtype, fp8, st);
}

int launch_combine_128(const CombineParams &c, int dtype, hipStream_t st) {
  return launch_combine_hd<128>(c, dtype, st);
}

int launch_seq_128(const DecodeParams &p, int dtype, bool fp8, hipStream_t st) {
  return launch_seq_hd<128>(p, dtype, fp8, st);
}

int launch_probe_128(const DecodeParams &p, const Grid &g, int nbuf, uint32_t *sink,
                    hipStream_t st) {
  return launch_probe_hd<128>(p, g, nbuf, sink, st);
}

}  // namespace mxfa

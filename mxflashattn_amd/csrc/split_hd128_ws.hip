// Instantiation unit of the split partial kernel for head dim 128 with the
// wave-local tile scan, one sequence per lane (batches of up to
// kWaveScanMax1 sequences); a unit of its own so it compiles in parallel
// with split_hd128.hip.
#include "split_kernels.h"

namespace mxfa {

int launch_partial_128_ws(const DecodeParams &p, const Grid &g, int dtype, bool fp8,
                          hipStream_t st) {
  return launch_partial_hd<128, 1>(p, g, dtype, fp8, st);
}

}  // namespace mxfa

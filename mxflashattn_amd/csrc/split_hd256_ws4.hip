// Instantiation unit of the split partial kernel for head dim 256 with the
// wave-local tile scan, four sequences per lane (batches of up to
// kWaveScanMax sequences; plain calls only, plain_call); a unit of its own
// so it compiles in parallel with split_hd256.hip.
#include "split_kernels.h"

namespace mxfa {

int launch_partial_256_ws4(const DecodeParams &p, const Grid &g, int dtype, bool fp8,
                           hipStream_t st) {
  return launch_partial_hd<256, 4>(p, g, dtype, fp8, st);
}

}  // namespace mxfa

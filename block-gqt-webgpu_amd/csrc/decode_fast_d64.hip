// Fused decode instances: structured layouts and FP16 K at d=64.
#include "decode_fast_kernel.h"

namespace bgtq {

// Structured layouts (NN nibble K-steps, SG K-steps in group 0) and FP16 K.
hipError_t launch_decode_fast_d64(const DecodeParams &p, const FastLayout &fl, int nn, int sg, hipStream_t stream) {
  if (p.key_format == 0) return launch_one<64, 0, 0, 2>(p, fl, stream);
  if (nn == 1 && sg == 1) return launch_one<64, 1, 1, 1>(p, fl, stream);
  if (nn == 2 && sg == 2) return launch_one<64, 1, 2, 2>(p, fl, stream);
  if (nn == 0 && sg == 2) return launch_one<64, 1, 0, 2>(p, fl, stream);
  if (nn == 2 && sg == 1) return launch_one<64, 1, 2, 1>(p, fl, stream);
  if (nn == 0 && sg == 1) return launch_one<64, 1, 0, 1>(p, fl, stream);
  return hipErrorInvalidValue;
}

}  // namespace bgtq

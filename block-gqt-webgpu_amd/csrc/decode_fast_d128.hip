// Fused decode instances: structured layouts and FP16 K at d=128.
#include "decode_fast_kernel.h"

namespace bgtq {

// Structured layouts (NN nibble K-steps, SG K-steps in group 0) and FP16 K.
hipError_t launch_decode_fast_d128(const DecodeParams &p, const FastLayout &fl, int nn, int sg, hipStream_t stream) {
  if (p.key_format == 0) return launch_one<128, 0, 0, 4>(p, fl, stream);
  if (nn == 2 && sg == 2) return launch_one<128, 1, 2, 2>(p, fl, stream);
  if (nn == 4 && sg == 4) return launch_one<128, 1, 4, 4>(p, fl, stream);
  if (nn == 0 && sg == 4) return launch_one<128, 1, 0, 4>(p, fl, stream);
  if (nn == 4 && sg == 2) return launch_one<128, 1, 4, 2>(p, fl, stream);
  if (nn == 0 && sg == 2) return launch_one<128, 1, 0, 2>(p, fl, stream);
  return hipErrorInvalidValue;
}

}  // namespace bgtq

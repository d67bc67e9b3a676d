// Fused decode instances: structured layouts and FP16 K at d=128, every kind
// of launch.
#include "decode_fast_kernel.h"

namespace bgtq {

hipError_t launch_decode_fast_d128(const DecodeParams &p, const FastLayout &fl, int nn, int sg, hipStream_t stream) {
  return launch_family_d128<kKindAll>(p, fl, nn, sg, stream);
}

}  // namespace bgtq

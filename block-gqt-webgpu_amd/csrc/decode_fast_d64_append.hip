// Fused decode instances: structured layouts and FP16 K at d=64, decode with
// an appended token.
#include "decode_fast_kernel.h"

namespace bgtq {

hipError_t launch_decode_fast_d64_append(const DecodeParams &p, const FastLayout &fl, int nn, int sg,
                                         hipStream_t stream) {
  return launch_family_d64<kKindAppend>(p, fl, nn, sg, stream);
}

}  // namespace bgtq

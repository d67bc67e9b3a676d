// Fused decode instances: any packed layout at d=64, decode with an appended
// token.
#include "decode_fast_kernel.h"

namespace bgtq {

hipError_t launch_decode_fast_any64_append(const DecodeParams &p, const FastLayout &fl, hipStream_t stream) {
  return launch_family_any<kKindAppend, 64>(p, fl, stream);
}

}  // namespace bgtq

// Fused decode instances: any packed layout at d=128, every kind of launch.
#include "decode_fast_kernel.h"

namespace bgtq {

hipError_t launch_decode_fast_any128(const DecodeParams &p, const FastLayout &fl, hipStream_t stream) {
  return launch_family_any<kKindAll, 128>(p, fl, stream);
}

}  // namespace bgtq

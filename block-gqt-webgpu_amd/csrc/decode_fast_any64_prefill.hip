// Fused decode instances: any packed layout at d=64, row-wise prefill.
#include "decode_fast_kernel.h"

namespace bgtq {

hipError_t launch_decode_fast_any64_prefill(const DecodeParams &p, const FastLayout &fl, hipStream_t stream) {
  return launch_family_any<kKindPrefill, 64>(p, fl, stream);
}

}  // namespace bgtq

// Fused decode instances: any packed layout at d=128.
#include "decode_fast_kernel.h"

namespace bgtq {

// Any packed layout: one or two scale DMAs per chunk (the largest norm stride
// of the launch's heads), pair lookups for K-step 0 when every head's K-step
// 0 is a pair K-step.
hipError_t launch_decode_fast_any128(const DecodeParams &p, const FastLayout &fl, hipStream_t stream) {
  int ns = 0;
  for (int h = 0; h < p.kv_heads; ++h) ns = fl.gns[h] > ns ? fl.gns[h] : ns;
  const bool pk = fl.gpair_lead >= 1;
  if (ns <= 4) return pk ? launch_one<128, 2, 1, 1, 1>(p, fl, stream) : launch_one<128, 2, 1, 1>(p, fl, stream);
  return pk ? launch_one<128, 2, 2, 1, 1>(p, fl, stream) : launch_one<128, 2, 2, 1>(p, fl, stream);
}

}  // namespace bgtq

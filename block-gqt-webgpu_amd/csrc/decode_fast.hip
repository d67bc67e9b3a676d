// Fused single-launch decode attention: layout queries and the launch
// dispatch (the kernel is in decode_fast_kernel.h).
#include "decode_fast_kernel.h"

namespace bgtq {

int decode_fast_row_bytes(int dim, int nn) { return nn * 16 + (dim / 32 - nn) * 32; }

int decode_fast_enc_capacity(int dim, int nn) {
  if (nn < 0) return dim == 64 ? Slot<64, 2, 1>::ENC_DMAS * 1024 : Slot<128, 2, 1>::ENC_DMAS * 1024;
  if (dim == 64) {
    if (nn == 0) return Slot<64, 1, 0>::ENC_DMAS * 1024;
    if (nn == 1) return Slot<64, 1, 1>::ENC_DMAS * 1024;
    return Slot<64, 1, 2>::ENC_DMAS * 1024;
  }
  if (nn == 0) return Slot<128, 1, 0>::ENC_DMAS * 1024;
  if (nn == 2) return Slot<128, 1, 2>::ENC_DMAS * 1024;
  return Slot<128, 1, 4>::ENC_DMAS * 1024;
}

bool decode_fast_supported(int dim, int key_format, int nn, int sg) {
  if (dim != 64 && dim != 128) return false;
  if (key_format == 0) return true;
  const int ks = dim / 32, h = ks / 2;
  return (nn == h && sg == h) || (nn == ks && sg == ks) || (nn == 0 && sg == ks) || (nn == ks && sg == h) ||
         (nn == 0 && sg == h);
}

int decode_general_table_bytes(int dim) { return dim == 64 ? Slot<64, 2, 1>::CTABLES : Slot<128, 2, 1>::CTABLES; }

int decode_general_max_norm_stride(int dim) {
  return dim == 64 ? Slot<64, 2, 2>::NBYTES / 64 : Slot<128, 2, 2>::NBYTES / 64;
}

// Instances by family and kind of launch, each in a translation unit of its own.
hipError_t launch_decode_fast_any64(const DecodeParams &p, const FastLayout &fl, hipStream_t stream);
hipError_t launch_decode_fast_any64_append(const DecodeParams &p, const FastLayout &fl, hipStream_t stream);
hipError_t launch_decode_fast_any64_prefill(const DecodeParams &p, const FastLayout &fl, hipStream_t stream);
hipError_t launch_decode_fast_any128(const DecodeParams &p, const FastLayout &fl, hipStream_t stream);
hipError_t launch_decode_fast_d64(const DecodeParams &p, const FastLayout &fl, int nn, int sg, hipStream_t stream);
hipError_t launch_decode_fast_d64_append(const DecodeParams &p, const FastLayout &fl, int nn, int sg,
                                         hipStream_t stream);
hipError_t launch_decode_fast_d64_prefill(const DecodeParams &p, const FastLayout &fl, int nn, int sg,
                                          hipStream_t stream);
hipError_t launch_decode_fast_d128(const DecodeParams &p, const FastLayout &fl, int nn, int sg, hipStream_t stream);

hipError_t launch_decode_fast(const DecodeParams &p, const FastLayout &fl, int nn, int sg, hipStream_t stream) {
  const int kind = decode_fast_launch_kind(p);
  if (nn < 0) {  // any packed layout
    if (p.dim != 64) return launch_decode_fast_any128(p, fl, stream);
    return kind == kKindAppend    ? launch_decode_fast_any64_append(p, fl, stream)
           : kind == kKindPrefill ? launch_decode_fast_any64_prefill(p, fl, stream)
                                  : launch_decode_fast_any64(p, fl, stream);
  }
  if (p.dim != 64) return launch_decode_fast_d128(p, fl, nn, sg, stream);
  return kind == kKindAppend    ? launch_decode_fast_d64_append(p, fl, nn, sg, stream)
         : kind == kKindPrefill ? launch_decode_fast_d64_prefill(p, fl, nn, sg, stream)
                                : launch_decode_fast_d64(p, fl, nn, sg, stream);
}

}  // namespace bgtq

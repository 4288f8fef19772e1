// Decode attention kernel instances for f32 K/V (templates in hc_decode_kernels.h).
#include "hc_decode_kernels.h"

namespace hc {
int decode_dispatch_f32(int64_t D, const DecodeArgs& a, int nw, hipStream_t st) {
  return dispatch_d<float>(D, a, nw, st);
}
}  // namespace hc

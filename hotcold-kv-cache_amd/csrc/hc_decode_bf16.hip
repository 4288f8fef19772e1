// Decode attention kernel instances for bf16 K/V (templates in hc_decode_kernels.h).
#include "hc_decode_kernels.h"

namespace hc {
int decode_dispatch_bf16(int64_t D, const DecodeArgs& a, int nw, hipStream_t st) {
  return dispatch_d<bf16_t>(D, a, nw, st);
}
}  // namespace hc

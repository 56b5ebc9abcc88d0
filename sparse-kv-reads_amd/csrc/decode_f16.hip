// The decode-attention kernels (decode.h) for f16 KV caches.
#include "decode.h"

namespace ssa {

hipError_t launch_decode_f16(const DecodeParams& p, int d, int mode, hipStream_t st) {
  return launch_decode_ty<__half>(p, d, mode, st);
}

}  // namespace ssa

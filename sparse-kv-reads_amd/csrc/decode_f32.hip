// The decode-attention kernels (decode.h) for f32 KV caches.
#include "decode.h"

namespace ssa {

hipError_t launch_decode_f32(const DecodeParams& p, int d, int mode, hipStream_t st) {
  return launch_decode_ty<float>(p, d, mode, st);
}

}  // namespace ssa

// The decode-attention kernels (decode.h) for bf16 KV caches.
#include "decode.h"

namespace ssa {

hipError_t launch_decode_bf16(const DecodeParams& p, int d, int mode, hipStream_t st) {
  return launch_decode_ty<__hip_bfloat16>(p, d, mode, st);
}

}  // namespace ssa

// Chunked DGDA prefill on MFMA (scalar per-token decay, dk = dv = 64, bf16 q/k/v).
// Placeholder until the segment-scan kernels land: reports "unsupported" so the
// dispatcher entry point uses the sequential kernel.
#include "maba_common.h"

namespace maba {

bool dgda_chunk_supported(const maba_tensor*, const maba_tensor*, const maba_tensor*,
                          const maba_tensor*, const maba_tensor*) {
  return false;
}

size_t dgda_chunk_workspace(int64_t, int64_t) { return 0; }

int launch_dgda_chunk(const maba_tensor*, const maba_tensor*, const maba_tensor*, const maba_tensor*, int,
                      const maba_tensor*, const maba_tensor*, const maba_tensor*, maba_tensor*,
                      maba_tensor*, void*, size_t, hipStream_t) {
  return fail(MABA_ERR_UNSUPPORTED, "dgda_prefill: chunked path not built");
}

}  // namespace maba

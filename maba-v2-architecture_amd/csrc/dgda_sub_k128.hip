// Kernels of the sub-chunk DGDA prefill (dgda_sub.h) for d_k = 128.
#include "dgda_sub.h"

namespace maba {

int run_sub_k128(SubArgs& a, int dv, bool f32in, bool g16, bool obf, hipStream_t stream) {
  return dv == 32 ? run_sub_passes<false, 128, 32>(a, f32in, g16, obf, stream)
                  : run_sub_passes<false, 128, 64>(a, f32in, g16, obf, stream);
}

}  // namespace maba

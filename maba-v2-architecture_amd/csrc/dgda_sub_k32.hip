// Kernels of the sub-chunk DGDA prefill (dgda_sub.h) for d_k = 32.
#include "dgda_sub.h"

namespace maba {

int run_sub_k32(SubArgs& a, int dv, bool f32in, bool g16, bool obf, hipStream_t stream) {
  return dv == 32 ? run_sub_passes<false, 32, 32>(a, f32in, g16, obf, stream)
                  : run_sub_passes<false, 32, 64>(a, f32in, g16, obf, stream);
}

}  // namespace maba

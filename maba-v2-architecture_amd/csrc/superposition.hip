// Three-stream gate superposition (reference: maba_sparse/kernels/common.py:406-438,
// cpu_indexer.py:115-150):  out = g0*o_local + g1*o_sparse + g2*o_hca with
// g = softmax(gate_logits) (fp32) or given gate_weights; a [B,L,3] gate is
// broadcast over heads, a [B,H,L,3] gate is per head.
//
// One thread per output element; the three gate values of a (b,h,t) row are
// recomputed per element (3 exps), which is free next to the 4 streamed
// tensors.  Elementwise, HBM-bound.
#include "maba_common.h"

namespace maba {

struct SupArgs {
  View4 ol, os, oh;
  const void* g;
  int gdt;
  int64_t gsb, gsh, gsl, gsm;  // gsh = 0 for a 3-D gate
  MView4 out;
  int64_t H, L, D, total;
  int is_weights;
};

__global__ __launch_bounds__(256) void superposition_kernel(SupArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.total) return;
  const int64_t d = i % a.D;
  const int64_t t = (i / a.D) % a.L;
  const int64_t h = (i / (a.D * a.L)) % a.H;
  const int64_t b = i / (a.D * a.L * a.H);
  const int64_t gb = b * a.gsb + h * a.gsh + t * a.gsl;
  float z0 = load_elem(a.g, a.gdt, gb), z1 = load_elem(a.g, a.gdt, gb + a.gsm),
        z2 = load_elem(a.g, a.gdt, gb + 2 * a.gsm);
  if (!a.is_weights) {
    const float m = fmaxf(z0, fmaxf(z1, z2));
    z0 = __expf(z0 - m);
    z1 = __expf(z1 - m);
    z2 = __expf(z2 - m);
    const float inv = 1.0f / (z0 + z1 + z2);
    z0 *= inv;
    z1 *= inv;
    z2 *= inv;
  }
  const float r = z0 * a.ol.at(b, h, t, d) + z1 * a.os.at(b, h, t, d) + z2 * a.oh.at(b, h, t, d);
  a.out.put(b, h, t, d, r);
}

}  // namespace maba

using namespace maba;

extern "C" int maba_hip_stream_superposition(const maba_tensor* o_local, const maba_tensor* o_sparse,
                                             const maba_tensor* o_hca, const maba_tensor* gate,
                                             int is_weights, maba_tensor* out, void* stream) {
  if (!o_local || o_local->ndim != 4) return fail(MABA_ERR_INVALID, "stream_superposition: o_local must be [B,H,L,D]");
  const int64_t B = o_local->shape[0], H = o_local->shape[1], L = o_local->shape[2], D = o_local->shape[3];
  const int64_t so[4] = {B, H, L, D};
  if (!expect_shape(o_sparse, "o_sparse", 4, so) || !expect_shape(o_hca, "o_hca", 4, so) ||
      !expect_shape(out, "out", 4, so))
    return MABA_ERR_INVALID;
  if (!gate || (gate->ndim != 3 && gate->ndim != 4)) return fail(MABA_ERR_INVALID, "stream_superposition: gate must be 3D or 4D");
  if (gate->shape[gate->ndim - 1] != 3) return fail(MABA_ERR_INVALID, "stream_superposition: gate last dim must be 3");
  if (gate->shape[0] != B) return fail(MABA_ERR_INVALID, "stream_superposition: gate batch must be %lld", (long long)B);
  if (gate->ndim == 3 && gate->shape[1] != L) return fail(MABA_ERR_INVALID, "stream_superposition: 3D gate must be [B,L,3]");
  if (gate->ndim == 4 && (gate->shape[1] != H || gate->shape[2] != L))
    return fail(MABA_ERR_INVALID, "stream_superposition: 4D gate must be [B,H,L,3]");
  const maba_tensor* all[] = {o_local, o_sparse, o_hca, gate, out};
  for (const maba_tensor* t : all)
    if (!expect_float(t, "stream_superposition")) return MABA_ERR_DTYPE;
  SupArgs a;
  a.ol = view4(o_local); a.os = view4(o_sparse); a.oh = view4(o_hca);
  a.g = gate->data; a.gdt = gate->dtype;
  a.gsb = gate->stride[0];
  if (gate->ndim == 3) { a.gsh = 0; a.gsl = gate->stride[1]; a.gsm = gate->stride[2]; }
  else { a.gsh = gate->stride[1]; a.gsl = gate->stride[2]; a.gsm = gate->stride[3]; }
  a.out = mview4(out);
  a.H = H; a.L = L; a.D = D; a.total = B * H * L * D;
  a.is_weights = is_weights;
  if (a.total == 0) return MABA_OK;
  hipLaunchKernelGGL(superposition_kernel, dim3((unsigned)ceil_div(a.total, 256)), dim3(256), 0,
                     (hipStream_t)stream, a);
  return check_launch("stream_superposition");
}

// Three-stream gate superposition (reference: maba_sparse/kernels/common.py:406-438,
// cpu_indexer.py:115-150):  out = g0*o_local + g1*o_sparse + g2*o_hca with
// g = softmax(gate_logits) (fp32) or given gate_weights; a [B,L,3] gate is
// broadcast over heads, a [B,H,L,3] gate is per head.
//
// Contiguous tensors of one dtype (bf16 or fp32) take the vector kernel: one
// 16-byte vector of a (b,h,t) row per thread, its gate softmax computed once for
// the vector, 32-bit index arithmetic.  Anything else takes the generic kernel, one
// thread per element.  Elementwise, HBM-bound.
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

template <typename T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
};

struct SupVecArgs {
  const void* ol; const void* os; const void* oh; void* out;
  const void* g; int gdt;
  int gsb, gsh, gsl, gsm;        // element strides of the gate (gsh = 0 for [B,L,3])
  int H, L, dvec, nvec;          // vectors per row, vectors in all
  int is_weights;
};

template <typename T>
__global__ __launch_bounds__(256) void superposition_vec_kernel(SupVecArgs a) {
  constexpr int N = Vec16<T>::N;
  const int v = blockIdx.x * 256 + threadIdx.x;
  if (v >= a.nvec) return;
  const int row = v / a.dvec;              // (b, h, t) row
  const int t = row % a.L;
  const int bh = row / a.L;
  const int h = bh % a.H, b = bh / a.H;
  const int gb = b * a.gsb + h * a.gsh + t * a.gsl;
  // all loads first: the three stream vectors and the gate
  typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
  const u32x4 xl = ((const u32x4*)a.ol)[v], xs = ((const u32x4*)a.os)[v], xh = ((const u32x4*)a.oh)[v];
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
  u32x4 r;
  if constexpr (N == 8) {   // bf16 pairs per 32-bit word
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float o[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int sh = 16 * e;
        const float fl = bf16_bits_to_f32((uint16_t)(xl[w] >> sh));
        const float fs = bf16_bits_to_f32((uint16_t)(xs[w] >> sh));
        const float fh = bf16_bits_to_f32((uint16_t)(xh[w] >> sh));
        o[e] = fmaf(z0, fl, fmaf(z1, fs, z2 * fh));
      }
      r[w] = (uint32_t)f32_to_bf16_bits(o[0]) | ((uint32_t)f32_to_bf16_bits(o[1]) << 16);
    }
  } else {
#pragma unroll
    for (int w = 0; w < 4; ++w)
      r[w] = __float_as_uint(fmaf(z0, __uint_as_float(xl[w]), fmaf(z1, __uint_as_float(xs[w]),
                                                                      z2 * __uint_as_float(xh[w]))));
  }
  ((u32x4*)a.out)[v] = r;
}

static bool contiguous4(const maba_tensor* t) {
  return t->stride[3] == 1 && t->stride[2] == t->shape[3] && t->stride[1] == t->shape[2] * t->shape[3] &&
         t->stride[0] == t->shape[1] * t->shape[2] * t->shape[3];
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
  const int dt = o_local->dtype;
  const int vn = dt == MABA_BF16 ? 8 : 4;
  const bool vec_ok = (dt == MABA_BF16 || dt == MABA_F32) && o_sparse->dtype == dt && o_hca->dtype == dt &&
                      out->dtype == dt && contiguous4(o_local) && contiguous4(o_sparse) && contiguous4(o_hca) &&
                      contiguous4(out) && D % vn == 0 && a.total / vn < (1ll << 31) &&
                      a.gsb < (1ll << 31) && a.gsl < (1ll << 31) && a.gsh < (1ll << 31) && a.gsm < (1ll << 31) &&
                      (B - 1) * a.gsb + (H - 1) * a.gsh + (L - 1) * a.gsl + 2 * a.gsm < (1ll << 31) &&
                      (uintptr_t)o_local->data % 16 == 0 && (uintptr_t)o_sparse->data % 16 == 0 &&
                      (uintptr_t)o_hca->data % 16 == 0 && (uintptr_t)out->data % 16 == 0;
  if (vec_ok) {
    SupVecArgs v;
    v.ol = o_local->data; v.os = o_sparse->data; v.oh = o_hca->data; v.out = out->data;
    v.g = gate->data; v.gdt = gate->dtype;
    v.gsb = (int)a.gsb; v.gsh = (int)a.gsh; v.gsl = (int)a.gsl; v.gsm = (int)a.gsm;
    v.H = (int)H; v.L = (int)L; v.dvec = (int)(D / vn); v.nvec = (int)(a.total / vn);
    v.is_weights = is_weights;
    const dim3 grid((unsigned)ceil_div(v.nvec, 256));
    if (dt == MABA_BF16) hipLaunchKernelGGL(superposition_vec_kernel<uint16_t>, grid, dim3(256), 0, (hipStream_t)stream, v);
    else hipLaunchKernelGGL(superposition_vec_kernel<float>, grid, dim3(256), 0, (hipStream_t)stream, v);
    return check_launch("stream_superposition/vec");
  }
  hipLaunchKernelGGL(superposition_kernel, dim3((unsigned)ceil_div(a.total, 256)), dim3(256), 0,
                     (hipStream_t)stream, a);
  return check_launch("stream_superposition");
}

// DGDA layer prologue: the op inputs of dgda_prefill / dgda_step from the layer's
// six projection outputs, in one pass.
//
// Reference: maba_sparse/layers/dgda.py
//   :103-121  q, k, v = silu(causal depthwise conv, kernel 4, over [history, x]),
//             new history = the last kernel_size - 1 conv inputs
//   :193-197  b = sigmoid(x_b), w = sigmoid(x_w),
//             log_alpha = max(-softplus(x_a), -14), alpha = exp(log_alpha)
//   :207      k = k / (||k||_head + eps)
//
// One workgroup per run of PRO_TOK tokens of one batch element, one thread per pair of
// channels (C = 64 H channels, 32 threads per head).  A thread walks its run keeping the
// three previous conv inputs of each stream in registers, so every projection row is read
// once (plus a three-row halo per run).  The per-head norm of k is a reduction over the
// head's 32 threads (half a wave).  Arithmetic in fp32; each output is rounded once.
// Bound: HBM (six input rows in, seven output rows out per token).
#include "dgda_common.h"

namespace maba {

constexpr int PRO_TOK = 64;   // tokens per workgroup
constexpr int PRO_GRP = 4;    // tokens whose loads are issued together
constexpr int PRO_KH = 3;     // conv history (kernel 4)

struct ProArgs {
  const void* x[6]; int64_t xsb[6], xsl[6];   // q, k, v, alpha, erase, write projections [B,L,C]
  const void* cw[3]; int cwdt; int64_t cwsc[3], cwst[3];   // conv weights [C,1,4]: channel / tap strides
  const void* hist[3]; int hdt; int64_t hsb[3], hsc[3], hst[3];   // [B,C,3] or null
  void* y[7]; int64_t ysb[7], ysl[7];         // q, k, v, log_alpha, alpha (may be null), b, w
  void* nh[3]; int nhdt; int64_t nhsb[3], nhsc[3], nhst[3];   // new history [B,C,3]
  int64_t L;
  float eps;
};

// Two consecutive channels (element index i even, 4- or 8-byte aligned).
template <class T> struct Pair;
template <> struct Pair<float> {
  static __device__ __forceinline__ float2 ld(const void* p, int64_t i) { return *(const float2*)((const float*)p + i); }
  static __device__ __forceinline__ void st(void* p, int64_t i, float x0, float x1) {
    *(float2*)((float*)p + i) = make_float2(x0, x1);
  }
};
template <> struct Pair<uint16_t> {   // bf16 bits
  static __device__ __forceinline__ float2 ld(const void* p, int64_t i) {
    const uint32_t u = *(const uint32_t*)((const uint16_t*)p + i);
    return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
  }
  static __device__ __forceinline__ void st(void* p, int64_t i, float x0, float x1) {
    *(uint32_t*)((uint16_t*)p + i) = (uint32_t)f32_to_bf16_bits(x0) | ((uint32_t)f32_to_bf16_bits(x1) << 16);
  }
};

// Conv input of stream s, channel ch, at token t (t >= -3): the projection for t >= 0,
// the carried history for t < 0 (zeros without one).
template <class XT>
__device__ __forceinline__ float pro_input(const ProArgs& a, int s, int64_t b, int ch, int64_t t) {
  if (t >= 0) {
    const float2 v = Pair<XT>::ld(a.x[s], b * a.xsb[s] + t * a.xsl[s] + (ch & ~1));
    return (ch & 1) ? v.y : v.x;
  }
  if (!a.hist[s]) return 0.f;
  return load_elem(a.hist[s], a.hdt, b * a.hsb[s] + ch * a.hsc[s] + (PRO_KH + t) * a.hst[s]);
}

template <class XT, class QT, class GT>
__global__ __launch_bounds__(512) void dgda_prologue_kernel(ProArgs a) {
  const int tid = threadIdx.x;
  const int c = 2 * tid;
  const int64_t b = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * PRO_TOK;
  const int64_t t1 = min(t0 + (int64_t)PRO_TOK, a.L);

  // the run holding the last token writes the new history: inputs L-3 .. L-1
  if (t1 == a.L) {
#pragma unroll
    for (int s = 0; s < 3; ++s)
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int j = 0; j < PRO_KH; ++j)
          store_elem(a.nh[s], a.nhdt, b * a.nhsb[s] + (c + e) * a.nhsc[s] + j * a.nhst[s],
                     pro_input<XT>(a, s, b, c + e, a.L - PRO_KH + j));
  }

  float w[3][2][4];     // conv taps per stream and channel
  float win[3][2][3];   // the three previous conv inputs, oldest first
#pragma unroll
  for (int s = 0; s < 3; ++s)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
#pragma unroll
      for (int j = 0; j < 4; ++j) w[s][e][j] = load_elem(a.cw[s], a.cwdt, (c + e) * a.cwsc[s] + j * a.cwst[s]);
#pragma unroll
      for (int j = 0; j < PRO_KH; ++j) win[s][e][j] = pro_input<XT>(a, s, b, c + e, t0 - PRO_KH + j);
    }

  // Tokens go in groups of PRO_GRP whose 6 PRO_GRP loads are all issued before the first
  // token of the group is computed (the stores of one token could alias the loads of the
  // next as far as the compiler knows, so it would not hoist them itself).  Loads past the
  // sequence end re-read the last token (in bounds) and are not used.
  for (int64_t tg = t0; tg < t1; tg += PRO_GRP) {   // block-uniform: every lane joins the shuffles
    float2 xg[PRO_GRP][6];
#pragma unroll
    for (int u = 0; u < PRO_GRP; ++u) {
      const int64_t tl = min(tg + u, a.L - 1);
#pragma unroll
      for (int s = 0; s < 6; ++s) xg[u][s] = Pair<XT>::ld(a.x[s], b * a.xsb[s] + tl * a.xsl[s] + c);
    }
#pragma unroll
    for (int u = 0; u < PRO_GRP; ++u) {
      const int64_t t = tg + u;
        if (t >= t1) break;   // block-uniform
      const float2* xv = xg[u];
      float y[3][2];
#pragma unroll
      for (int s = 0; s < 3; ++s)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float xn = e ? xv[s].y : xv[s].x;
          float acc = w[s][e][3] * xn;
          acc = fmaf(w[s][e][2], win[s][e][2], acc);
          acc = fmaf(w[s][e][1], win[s][e][1], acc);
          acc = fmaf(w[s][e][0], win[s][e][0], acc);
          y[s][e] = pro_silu(acc);
          win[s][e][0] = win[s][e][1];
          win[s][e][1] = win[s][e][2];
          win[s][e][2] = xn;
        }
      // ||k|| over the head's 64 channels: 32 threads, xor offsets below 32 stay in the half wave
      float ss = y[1][0] * y[1][0] + y[1][1] * y[1][1];
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) ss += __shfl_xor(ss, off);
      const float kinv = pro_knorm_inv(ss, a.eps);
      const float la0 = pro_log_decay(xv[3].x), la1 = pro_log_decay(xv[3].y);
      Pair<QT>::st(a.y[0], b * a.ysb[0] + t * a.ysl[0] + c, y[0][0], y[0][1]);
      Pair<QT>::st(a.y[1], b * a.ysb[1] + t * a.ysl[1] + c, y[1][0] * kinv, y[1][1] * kinv);
      Pair<QT>::st(a.y[2], b * a.ysb[2] + t * a.ysl[2] + c, y[2][0], y[2][1]);
      Pair<GT>::st(a.y[3], b * a.ysb[3] + t * a.ysl[3] + c, la0, la1);
      if (a.y[4]) Pair<GT>::st(a.y[4], b * a.ysb[4] + t * a.ysl[4] + c, __expf(la0), __expf(la1));
      Pair<GT>::st(a.y[5], b * a.ysb[5] + t * a.ysl[5] + c, pro_sigmoid(xv[4].x), pro_sigmoid(xv[4].y));
      Pair<GT>::st(a.y[6], b * a.ysb[6] + t * a.ysl[6] + c, pro_sigmoid(xv[5].x), pro_sigmoid(xv[5].y));
    }
  }
}

// One element of a projection / output row.
template <class T> __device__ __forceinline__ float pro_ld1(const void* p, int64_t i);
template <> __device__ __forceinline__ float pro_ld1<float>(const void* p, int64_t i) { return ((const float*)p)[i]; }
template <> __device__ __forceinline__ float pro_ld1<uint16_t>(const void* p, int64_t i) {
  return bf16_bits_to_f32(((const uint16_t*)p)[i]);
}
template <class T> __device__ __forceinline__ void pro_st1(void* p, int64_t i, float x);
template <> __device__ __forceinline__ void pro_st1<float>(void* p, int64_t i, float x) { ((float*)p)[i] = x; }
template <> __device__ __forceinline__ void pro_st1<uint16_t>(void* p, int64_t i, float x) {
  ((uint16_t*)p)[i] = f32_to_bf16_bits(x);
}

// One token (a decode step): one wave per (head, batch element), one lane per channel.
// Every input, the carried history included, is read before the first store, so the new
// history may overwrite the old one in place.  Same arithmetic as the run kernel.
template <class XT, class QT, class GT>
__global__ __launch_bounds__(64) void dgda_prologue_step_kernel(ProArgs a) {
  const int lane = threadIdx.x;
  const int c = 64 * blockIdx.x + lane;
  const int64_t b = blockIdx.y;
  float x[6], w[3][4], h[3][PRO_KH];
#pragma unroll
  for (int s = 0; s < 6; ++s) x[s] = pro_ld1<XT>(a.x[s], b * a.xsb[s] + c);
#pragma unroll
  for (int s = 0; s < 3; ++s) {
#pragma unroll
    for (int j = 0; j < 4; ++j) w[s][j] = load_elem(a.cw[s], a.cwdt, c * a.cwsc[s] + j * a.cwst[s]);
#pragma unroll
    for (int j = 0; j < PRO_KH; ++j)
      h[s][j] = a.hist[s] ? load_elem(a.hist[s], a.hdt, b * a.hsb[s] + c * a.hsc[s] + j * a.hst[s]) : 0.f;
  }
  float y[3];
#pragma unroll
  for (int s = 0; s < 3; ++s) {
    float acc = w[s][3] * x[s];
    acc = fmaf(w[s][2], h[s][2], acc);
    acc = fmaf(w[s][1], h[s][1], acc);
    acc = fmaf(w[s][0], h[s][0], acc);
    y[s] = pro_silu(acc);
  }
#pragma unroll
  for (int s = 0; s < 3; ++s) {   // new history: the inputs of tokens -2, -1, 0
    const int64_t o = b * a.nhsb[s] + c * a.nhsc[s];
    store_elem(a.nh[s], a.nhdt, o, h[s][1]);
    store_elem(a.nh[s], a.nhdt, o + a.nhst[s], h[s][2]);
    store_elem(a.nh[s], a.nhdt, o + 2 * a.nhst[s], x[s]);
  }
  float ss = y[1] * y[1];
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) ss += __shfl_xor(ss, off);
  const float kinv = pro_knorm_inv(ss, a.eps);
  const float la = pro_log_decay(x[3]);
  pro_st1<QT>(a.y[0], b * a.ysb[0] + c, y[0]);
  pro_st1<QT>(a.y[1], b * a.ysb[1] + c, y[1] * kinv);
  pro_st1<QT>(a.y[2], b * a.ysb[2] + c, y[2]);
  pro_st1<GT>(a.y[3], b * a.ysb[3] + c, la);
  if (a.y[4]) pro_st1<GT>(a.y[4], b * a.ysb[4] + c, __expf(la));
  pro_st1<GT>(a.y[5], b * a.ysb[5] + c, pro_sigmoid(x[4]));
  pro_st1<GT>(a.y[6], b * a.ysb[6] + c, pro_sigmoid(x[5]));
}

static bool pro_pair_ok(const maba_tensor* t, int64_t B, int64_t L, int64_t C) {
  if (!t || t->ndim != 3 || t->shape[0] != B || t->shape[1] != L || t->shape[2] != C) return false;
  if (t->dtype != MABA_F32 && t->dtype != MABA_BF16) return false;
  const int64_t el = t->dtype == MABA_F32 ? 4 : 2;
  return t->stride[2] == 1 && t->stride[0] % 2 == 0 && t->stride[1] % 2 == 0 &&
         (uintptr_t)t->data % (2 * el) == 0;
}

template <class XT, class QT>
static void pro_launch_g(const ProArgs& a, int gdt, dim3 grid, dim3 block, hipStream_t s) {
  const bool step = a.L == 1;   // grid (H, B) of 64-lane waves for a single token
  if (gdt == MABA_F32) {
    if (step) hipLaunchKernelGGL((dgda_prologue_step_kernel<XT, QT, float>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((dgda_prologue_kernel<XT, QT, float>), grid, block, 0, s, a);
  } else {
    if (step) hipLaunchKernelGGL((dgda_prologue_step_kernel<XT, QT, uint16_t>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((dgda_prologue_kernel<XT, QT, uint16_t>), grid, block, 0, s, a);
  }
}

// New conv history of a prefill whose conv runs inside the DGDA kernels (the fused layer
// prefill): the conv inputs of tokens L-3 .. L-1 per stream and channel, from the
// projections or, for L < 3, the old history.  One thread per channel reads its three
// inputs before writing, so the new history may overwrite the old one in place.
template <class XT>
__global__ __launch_bounds__(256) void dgda_history_kernel(ProArgs a, int C) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (c >= C) return;
  float v[3][PRO_KH];
#pragma unroll
  for (int s = 0; s < 3; ++s)
#pragma unroll
    for (int j = 0; j < PRO_KH; ++j) v[s][j] = pro_input<XT>(a, s, b, c, a.L - PRO_KH + j);
#pragma unroll
  for (int s = 0; s < 3; ++s)
#pragma unroll
    for (int j = 0; j < PRO_KH; ++j)
      store_elem(a.nh[s], a.nhdt, b * a.nhsb[s] + c * a.nhsc[s] + j * a.nhst[s], v[s][j]);
}

// Host side of the above for the fused layer prefill, whose entry point has validated the
// shapes ([B,L,C] projections with unit channel stride, [B,C,3] histories).
int launch_dgda_new_history(const maba_tensor* const* xs, const maba_tensor* const* hist,
                            maba_tensor* const* new_hist, hipStream_t stream) {
  const int64_t B = xs[0]->shape[0], L = xs[0]->shape[1], C = xs[0]->shape[2];
  if (B == 0) return MABA_OK;
  ProArgs a = {};
  for (int s = 0; s < 3; ++s) {
    a.x[s] = xs[s]->data; a.xsb[s] = xs[s]->stride[0]; a.xsl[s] = xs[s]->stride[1];
    a.hist[s] = hist ? hist[s]->data : nullptr;
    a.hsb[s] = hist ? hist[s]->stride[0] : 0; a.hsc[s] = hist ? hist[s]->stride[1] : 0;
    a.hst[s] = hist ? hist[s]->stride[2] : 0;
    a.nh[s] = new_hist[s]->data; a.nhsb[s] = new_hist[s]->stride[0]; a.nhsc[s] = new_hist[s]->stride[1];
    a.nhst[s] = new_hist[s]->stride[2];
  }
  a.hdt = hist ? hist[0]->dtype : MABA_F32;
  a.nhdt = new_hist[0]->dtype;
  a.L = L;
  const dim3 grid((unsigned)ceil_div(C, 256), (unsigned)B);
  if (xs[0]->dtype == MABA_F32) hipLaunchKernelGGL(dgda_history_kernel<float>, grid, dim3(256), 0, stream, a, (int)C);
  else hipLaunchKernelGGL(dgda_history_kernel<uint16_t>, grid, dim3(256), 0, stream, a, (int)C);
  return check_launch("dgda_layer_prefill/history");
}

}  // namespace maba

using namespace maba;

extern "C" int maba_hip_dgda_prologue(const maba_tensor* const* xs, const maba_tensor* const* conv_w,
                                      const maba_tensor* const* hist, float eps, maba_tensor* const* ys,
                                      maba_tensor* const* new_hist, void* stream) {
  if (!xs || !conv_w || !ys || !new_hist) return fail(MABA_ERR_INVALID, "dgda_prologue: null argument array");
  for (int s = 0; s < 6; ++s)
    if (!xs[s] || xs[s]->ndim != 3) return fail(MABA_ERR_INVALID, "dgda_prologue: projection %d must be [B,L,C]", s);
  const int64_t B = xs[0]->shape[0], L = xs[0]->shape[1], C = xs[0]->shape[2];
  if (C % 64 != 0 || C / 2 > 512)
    return fail(MABA_ERR_UNSUPPORTED, "dgda_prologue: C must be 64 * H with H <= 16, got C = %lld", (long long)C);
  const int xdt = xs[0]->dtype;
  for (int s = 0; s < 6; ++s) {
    if (!pro_pair_ok(xs[s], B, L, C) || xs[s]->dtype != xdt)
      return fail(MABA_ERR_UNSUPPORTED,
                  "dgda_prologue: projections must share one f32/bf16 dtype, [B,L,C] with unit channel stride");
  }
  const int qdt = ys[0] ? ys[0]->dtype : -1, gdt = ys[3] ? ys[3]->dtype : -1;
  for (int s = 0; s < 7; ++s) {
    if (s == 4 && !ys[s]) continue;   // alpha is optional
    if (!pro_pair_ok(ys[s], B, L, C) || ys[s]->dtype != (s < 3 ? qdt : gdt))
      return fail(MABA_ERR_UNSUPPORTED, "dgda_prologue: output %d must be [B,L,C] f32/bf16 with unit channel "
                  "stride (q, k, v share one dtype, the gates another)", s);
  }
  const int64_t sw[3] = {C, 1, 4}, sh[3] = {B, C, PRO_KH};
  for (int s = 0; s < 3; ++s) {
    if (!expect_shape(conv_w[s], "conv weight", 3, sw) || !expect_float(conv_w[s], "conv weight"))
      return MABA_ERR_INVALID;
    if (conv_w[s]->dtype != conv_w[0]->dtype) return fail(MABA_ERR_DTYPE, "dgda_prologue: conv weights differ in dtype");
    if (hist) {
      if (!expect_shape(hist[s], "conv history", 3, sh) || !expect_float(hist[s], "conv history"))
        return MABA_ERR_INVALID;
      if (hist[s]->dtype != hist[0]->dtype) return fail(MABA_ERR_DTYPE, "dgda_prologue: histories differ in dtype");
    }
    if (!expect_shape(new_hist[s], "new conv history", 3, sh) || !expect_float(new_hist[s], "new conv history"))
      return MABA_ERR_INVALID;
    if (new_hist[s]->dtype != new_hist[0]->dtype)
      return fail(MABA_ERR_DTYPE, "dgda_prologue: new histories differ in dtype");
  }
  // with several tokens the new history is written while other workgroups still read the
  // old one; a single token reads each channel's history before writing it (in place is fine)
  for (int s = 0; hist && L > 1 && s < 3; ++s)
    for (int r = 0; r < 3; ++r)
      if (new_hist[s]->data == hist[r]->data)
        return fail(MABA_ERR_INVALID, "dgda_prologue: the new conv history must not alias the old one");
  if (B == 0 || L == 0) return MABA_OK;
  ProArgs a;
  for (int s = 0; s < 6; ++s) { a.x[s] = xs[s]->data; a.xsb[s] = xs[s]->stride[0]; a.xsl[s] = xs[s]->stride[1]; }
  a.cwdt = conv_w[0]->dtype;
  a.hdt = hist ? hist[0]->dtype : MABA_F32;
  a.nhdt = new_hist[0]->dtype;
  for (int s = 0; s < 3; ++s) {
    a.cw[s] = conv_w[s]->data; a.cwsc[s] = conv_w[s]->stride[0]; a.cwst[s] = conv_w[s]->stride[2];
    a.hist[s] = hist ? hist[s]->data : nullptr;
    a.hsb[s] = hist ? hist[s]->stride[0] : 0; a.hsc[s] = hist ? hist[s]->stride[1] : 0;
    a.hst[s] = hist ? hist[s]->stride[2] : 0;
    a.nh[s] = new_hist[s]->data; a.nhsb[s] = new_hist[s]->stride[0]; a.nhsc[s] = new_hist[s]->stride[1];
    a.nhst[s] = new_hist[s]->stride[2];
  }
  for (int s = 0; s < 7; ++s) {
    a.y[s] = ys[s] ? ys[s]->data : nullptr;
    a.ysb[s] = ys[s] ? ys[s]->stride[0] : 0;
    a.ysl[s] = ys[s] ? ys[s]->stride[1] : 0;
  }
  a.L = L;
  a.eps = eps;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = L == 1 ? dim3((unsigned)(C / 64), (unsigned)B) : dim3((unsigned)ceil_div(L, PRO_TOK), (unsigned)B);
  const dim3 block = L == 1 ? dim3(64) : dim3((unsigned)(C / 2));
  if (xdt == MABA_F32) {
    if (qdt == MABA_F32) pro_launch_g<float, float>(a, gdt, grid, block, st);
    else pro_launch_g<float, uint16_t>(a, gdt, grid, block, st);
  } else {
    if (qdt == MABA_F32) pro_launch_g<uint16_t, float>(a, gdt, grid, block, st);
    else pro_launch_g<uint16_t, uint16_t>(a, gdt, grid, block, st);
  }
  return check_launch("dgda_prologue");
}

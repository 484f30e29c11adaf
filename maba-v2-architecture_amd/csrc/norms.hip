// The full-model harness's elementwise kernels (reference maba_sparse/model.py):
//   RMSNorm                 :11-22    h = x / sqrt(mean(x^2) + eps) * w
//   gated residual + norm   :92-128   x' = x + g * mo (MabaBlock's sigmoid-gated residual),
//                                     then h = RMSNorm(x') for the next sub-layer
//   SwiGLU activation       :25-38    a = silu(x W_gate^T) * (x W_up^T), from the one GEMM over
//                                     the stacked [W_gate; W_up] ([.., 2I] -> [.., I])
// One wave per row (token); arithmetic in fp32, each output rounded once to its dtype.
// Bound: HBM (a few row reads and writes per token).
#include <algorithm>

#include "maba_common.h"

namespace maba {

constexpr int NRM_MAXP = 16;   // channel pairs per lane: C <= 2048

struct NormArgs {
  const void* x; int64_t xs;        // [R, C] rows (row stride xs, unit channel stride)
  const void* mo; int64_t ms;       // residual input rows (null: plain RMSNorm)
  const void* g;                    // [C] residual gate (fp32 or the row dtype)
  int gdt;
  const void* w; int wdt;           // [C] norm weight
  void* xo; int64_t xos;            // x' rows (null: not written)
  void* h; int64_t hs;              // normalised rows
  int64_t R;
  int C;
  float eps;
};

template <class T> struct P2;
template <> struct P2<float> {
  typedef float2 raw;   // the bits of a channel pair as loaded
  static __device__ __forceinline__ raw ldr(const void* p, int64_t i) { return *(const float2*)((const float*)p + i); }
  static __device__ __forceinline__ float2 cvt(raw u) { return u; }
  static __device__ __forceinline__ raw zero(uint32_t z) { return make_float2(__uint_as_float(z), __uint_as_float(z)); }
  static __device__ __forceinline__ float2 ld(const void* p, int64_t i) { return ldr(p, i); }
  static __device__ __forceinline__ void st(void* p, int64_t i, float2 v) { *(float2*)((float*)p + i) = v; }
};
template <> struct P2<uint16_t> {
  typedef uint32_t raw;
  static __device__ __forceinline__ raw ldr(const void* p, int64_t i) { return *(const uint32_t*)((const uint16_t*)p + i); }
  static __device__ __forceinline__ float2 cvt(raw u) {
    return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
  }
  static __device__ __forceinline__ raw zero(uint32_t z) { return z; }
  static __device__ __forceinline__ float2 ld(const void* p, int64_t i) { return cvt(ldr(p, i)); }
  static __device__ __forceinline__ void st(void* p, int64_t i, float2 v) {
    *(uint32_t*)((uint16_t*)p + i) = (uint32_t)f32_to_bf16_bits(v.x) | ((uint32_t)f32_to_bf16_bits(v.y) << 16);
  }
};

// v as the row dtype stores it (the residual stream is normalised as stored).
template <class T> __device__ __forceinline__ float2 as_stored(float2 v);
template <> __device__ __forceinline__ float2 as_stored<float>(float2 v) { return v; }
template <> __device__ __forceinline__ float2 as_stored<uint16_t>(float2 v) {
  return make_float2(bf16_bits_to_f32(f32_to_bf16_bits(v.x)), bf16_bits_to_f32(f32_to_bf16_bits(v.y)));
}

// T: row dtype; TG, TW: dtype of the residual gate and the norm weight; MODE 0: h = norm(x),
// 1: x' = x + g * mo and h = norm(x'), 2: as 1 with x' written to xo in T and normalised as
// written.  The wave first issues every load of its row as raw bits (channel indices clamped
// into the row) and only then converts and computes, every chunk without a branch on the
// chunk count.  A value used under the same test as its load, or converted inside a run-time
// dtype switch, is waited for on its own, one memory round trip per chunk; the fill of the
// chunks past the row comes from an instruction the optimiser cannot see through, which
// keeps it from moving the conversions up into the loads' branches.
// MAXP: channel pairs per lane the arrays hold (4, 8 or NRM_MAXP, the smallest that covers C:
// fewer registers, more waves per SIMD, more rows in flight).
template <class T, class TG, class TW, int MODE, int MAXP>
__global__ __launch_bounds__(256) void rmsnorm_kernel(NormArgs a) {
  const int lane = threadIdx.x & 63;
  // a wave past the last row reads that row and stores nothing: with an early return the
  // compiler reads the row count, waits and branches before it loads the other arguments
  asm volatile("" ::"s"(a.x), "s"(a.xs), "s"(a.mo), "s"(a.ms), "s"(a.g), "s"(a.w), "s"(a.xo), "s"(a.xos),
               "s"(a.h), "s"(a.hs), "s"(a.R), "s"(a.C), "s"(a.eps));   // every argument loaded at once
  const int64_t r0 = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const bool live = r0 < a.R;
  const int64_t r = live ? r0 : a.R - 1;
  const int np = live ? a.C / 2 : 0, nit = (a.C / 2 + 63) >> 6;
  uint32_t zr;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zr));
  typename P2<T>::raw v[MAXP], m[MAXP];
  typename P2<TG>::raw g[MAXP];
  typename P2<TW>::raw w[MAXP];
#pragma unroll
  for (int i = 0; i < MAXP; ++i) {
    v[i] = P2<T>::zero(zr); m[i] = P2<T>::zero(zr); g[i] = P2<TG>::zero(zr); w[i] = P2<TW>::zero(zr);
    if (i < nit) {
      const int j = min(lane + 64 * i, a.C / 2 - 1);
      v[i] = P2<T>::ldr(a.x, r * a.xs + 2 * j);
      if constexpr (MODE > 0) {
        m[i] = P2<T>::ldr(a.mo, r * a.ms + 2 * j);
        g[i] = P2<TG>::ldr(a.g, 2 * j);
      }
      w[i] = P2<TW>::ldr(a.w, 2 * j);
    }
  }
  float2 xs[MAXP];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXP; ++i) {
    const int j = lane + 64 * i;
    float2 x = P2<T>::cvt(v[i]);
    if constexpr (MODE > 0) {
      const float2 mm = P2<T>::cvt(m[i]), gg = P2<TG>::cvt(g[i]);
      x.x = fmaf(gg.x, mm.x, x.x);
      x.y = fmaf(gg.y, mm.y, x.y);
      if constexpr (MODE == 2) {
        x = as_stored<T>(x);
        if (j < np) P2<T>::st(a.xo, r * a.xos + 2 * j, x);
      }
    }
    const bool in = j < np;
    x.x = in ? x.x : 0.f;
    x.y = in ? x.y : 0.f;
    xs[i] = x;
    ss = fmaf(x.x, x.x, fmaf(x.y, x.y, ss));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  const float inv = rsqrtf(ss / (float)a.C + a.eps);   // (np = 0 on a dead wave: no stores)
#pragma unroll
  for (int i = 0; i < MAXP; ++i) {
    const int j = lane + 64 * i;
    const float2 ww = P2<TW>::cvt(w[i]);
    if (j < np) P2<T>::st(a.h, r * a.hs + 2 * j, make_float2(xs[i].x * inv * ww.x, xs[i].y * inv * ww.y));
  }
}

struct SwigluArgs {
  const void* gu; int64_t gus;      // [R, 2I]: gate columns [0, I), up columns [I, 2I)
  void* out; int64_t os;            // [R, I]
  int64_t R;
  int I;
};

template <class T>
__global__ __launch_bounds__(256) void swiglu_kernel(SwigluArgs a) {
  const int np = a.I / 2;
  const int64_t total = a.R * np;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
    const int64_t r = e / np;
    const int j = (int)(e - r * np);
    const float2 g = P2<T>::ld(a.gu, r * a.gus + 2 * j);
    const float2 u = P2<T>::ld(a.gu, r * a.gus + a.I + 2 * j);
    const float s0 = g.x * fast_rcp(1.f + fast_exp(-g.x)), s1 = g.y * fast_rcp(1.f + fast_exp(-g.y));
    P2<T>::st(a.out, r * a.os + 2 * j, make_float2(s0 * u.x, s1 * u.y));
  }
}

// bf16 rows with I % 8 == 0 and 16-byte aligned rows: one wave per row, 16-byte loads of
// eight gate and eight up channels per lane and chunk, no index division; the same
// per-element arithmetic as swiglu_kernel.
constexpr int SW_MAXQ = 4;   // 16-byte chunks per lane: I <= 64 * 8 * SW_MAXQ
__global__ __launch_bounds__(256) void swiglu_rows_kernel(SwigluArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.R) return;   // whole wave
  const int nq = a.I / 8;
  const uint16_t* gp = (const uint16_t*)a.gu + r * a.gus;
  uint16_t* op = (uint16_t*)a.out + r * a.os;
  uint4 g[SW_MAXQ], u[SW_MAXQ];
#pragma unroll
  for (int q = 0; q < SW_MAXQ; ++q) {
    const int c = lane + 64 * q;
    if (c < nq) {
      g[q] = *(const uint4*)(gp + 8 * c);
      u[q] = *(const uint4*)(gp + a.I + 8 * c);
    }
  }
#pragma unroll
  for (int q = 0; q < SW_MAXQ; ++q) {
    const int c = lane + 64 * q;
    if (c < nq) {
      const uint32_t gw[4] = {g[q].x, g[q].y, g[q].z, g[q].w}, uw[4] = {u[q].x, u[q].y, u[q].z, u[q].w};
      uint32_t ow[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float2 gg = P2<uint16_t>::cvt(gw[e]), uu = P2<uint16_t>::cvt(uw[e]);
        const float s0 = gg.x * fast_rcp(1.f + fast_exp(-gg.x)), s1 = gg.y * fast_rcp(1.f + fast_exp(-gg.y));
        ow[e] = (uint32_t)f32_to_bf16_bits(s0 * uu.x) | ((uint32_t)f32_to_bf16_bits(s1 * uu.y) << 16);
      }
      *(uint4*)(op + 8 * c) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
  }
}

// Greedy pick (model.py:279-313, torch.argmax over the vocabulary): one workgroup per row.
// Each thread loads AM_BATCH 16-byte vectors of the row before it reads the first, then keeps
// the largest key: the value mapped to an unsigned integer in float order (NaN above
// everything, -0 as +0) in the high word, the complement of the index in the low word, so the
// largest key of a row is its first maximum.
constexpr int AM_T = 1024, AM_BATCH = 4;

struct ArgmaxArgs {
  const void* x; int64_t xs;   // rows [M, V]
  int64_t* out; int64_t os;
  int V;
};

__device__ __forceinline__ uint64_t am_key(float v, int idx) {
  uint32_t o;
  if (v != v) {
    o = 0xffffffffu;
  } else {
    const uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
    o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
  return ((uint64_t)o << 32) | (uint32_t)(0xffffffffu - (uint32_t)idx);
}

template <class T>
__global__ __launch_bounds__(AM_T) void argmax_rows_kernel(ArgmaxArgs a) {
  __shared__ uint64_t s_best[AM_T / 64];
  typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
  constexpr int E = 16 / sizeof(T);   // elements per vector
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nv = a.V / E;
  const char* base = (const char*)a.x + (int64_t)blockIdx.x * a.xs * (int64_t)sizeof(T);
  uint64_t best = 0;
  for (int v0 = 0; v0 < nv; v0 += AM_T * AM_BATCH) {
    u32x4 raw[AM_BATCH];
#pragma unroll
    for (int b = 0; b < AM_BATCH; ++b) raw[b] = *(const u32x4*)(base + (int64_t)min(v0 + b * AM_T + tid, nv - 1) * 16);
#pragma unroll
    for (int b = 0; b < AM_BATCH; ++b) {
      const int v = v0 + b * AM_T + tid;
      if (v < nv) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          float f;
          if constexpr (sizeof(T) == 2) f = __uint_as_float(e & 1 ? raw[b][e / 2] & 0xffff0000u : raw[b][e / 2] << 16);
          else f = __uint_as_float(raw[b][e]);
          const uint64_t k = am_key(f, v * E + e);
          best = k > best ? k : best;
        }
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t o = __shfl_xor(best, off);
    best = o > best ? o : best;
  }
  if (lane == 0) s_best[wave] = best;
  __syncthreads();
  if (tid == 0) {
    uint64_t b = s_best[0];
#pragma unroll
    for (int w = 1; w < AM_T / 64; ++w) b = s_best[w] > b ? s_best[w] : b;
    a.out[(int64_t)blockIdx.x * a.os] = (int64_t)(0xffffffffu - (uint32_t)b);
  }
}

// Rows of a [..., C] tensor: leading dims collapse into one when they are contiguous.
static bool rows_of(const maba_tensor* t, int C, int64_t& R, int64_t& rs) {
  if (!t || t->ndim < 1 || t->ndim > 3 || t->shape[t->ndim - 1] != C || t->stride[t->ndim - 1] != 1) return false;
  R = 1;
  for (int d = 0; d < t->ndim - 1; ++d) R *= t->shape[d];
  rs = C;
  if (t->ndim == 2) {
    rs = t->stride[0];
  } else if (t->ndim == 3) {
    if (t->shape[1] == 1) rs = t->stride[0];                   // [B, 1, C]: rows over the batch
    else if (t->shape[0] == 1) rs = t->stride[1];
    else if (t->stride[0] == t->shape[1] * t->stride[1]) rs = t->stride[1];
    else return false;
  }
  return R <= 1 || (rs % 2 == 0 && (uintptr_t)t->data % 4 == 0);
}

}  // namespace maba

using namespace maba;

extern "C" int maba_hip_rmsnorm(const maba_tensor* x, const maba_tensor* mo, const maba_tensor* gate,
                                const maba_tensor* weight, float eps, maba_tensor* x_out, maba_tensor* h,
                                void* stream) {
  if (!x || !weight || !h) return fail(MABA_ERR_INVALID, "rmsnorm: x, weight and h required");
  const int C = (int)x->shape[x->ndim - 1];
  if (C < 2) return fail(MABA_ERR_INVALID, "rmsnorm: the last dimension must hold at least 2 channels");
  if (C % 2 != 0 || C > 2 * 64 * NRM_MAXP) return fail(MABA_ERR_UNSUPPORTED, "rmsnorm: C even and <= %d", 128 * NRM_MAXP);
  if (x->dtype != MABA_F32 && x->dtype != MABA_BF16) return fail(MABA_ERR_DTYPE, "rmsnorm: f32 or bf16 rows");
  NormArgs a;
  int64_t R, R2;
  if (!rows_of(x, C, R, a.xs)) return fail(MABA_ERR_UNSUPPORTED, "rmsnorm: x rows must be [.., C] with unit channel stride");
  if (!rows_of(h, C, R2, a.hs) || R2 != R || h->dtype != x->dtype)
    return fail(MABA_ERR_INVALID, "rmsnorm: h must match x");
  if (weight->ndim != 1 || weight->shape[0] != C || weight->stride[0] != 1 ||
      (weight->dtype != MABA_F32 && weight->dtype != MABA_BF16) || (uintptr_t)weight->data % 4)
    return fail(MABA_ERR_INVALID, "rmsnorm: weight must be [C] f32/bf16");
  a.mo = nullptr; a.ms = 0; a.g = nullptr; a.gdt = MABA_F32; a.xo = nullptr; a.xos = 0;
  if (mo) {
    if (!rows_of(mo, C, R2, a.ms) || R2 != R || mo->dtype != x->dtype)
      return fail(MABA_ERR_INVALID, "rmsnorm: mo must match x");
    if (!gate || gate->ndim != 1 || gate->shape[0] != C || gate->stride[0] != 1 ||
        (gate->dtype != MABA_F32 && gate->dtype != MABA_BF16) || (uintptr_t)gate->data % 4)
      return fail(MABA_ERR_INVALID, "rmsnorm: gate must be [C] f32/bf16");
    a.mo = mo->data; a.g = gate->data; a.gdt = gate->dtype;
    if (x_out) {
      if (!rows_of(x_out, C, R2, a.xos) || R2 != R || x_out->dtype != x->dtype)
        return fail(MABA_ERR_INVALID, "rmsnorm: x_out must match x");
      a.xo = x_out->data;
    }
  }
  a.x = x->data; a.w = weight->data; a.wdt = weight->dtype; a.h = h->data;
  a.R = R; a.C = C; a.eps = eps;
  if (R == 0) return MABA_OK;
  const dim3 grid((unsigned)ceil_div(R, 4));
  const int mode = !a.mo ? 0 : !a.xo ? 1 : 2;
  const bool tb = x->dtype == MABA_BF16, gb = a.gdt == MABA_BF16, wb = a.wdt == MABA_BF16;
  void (*k)(NormArgs) = nullptr;
  const int nit = (C / 2 + 63) / 64;
#define MABA_NRM_PICKP(T, TW, P)                                                                       \
  k = mode == 0 ? rmsnorm_kernel<T, float, TW, 0, P>                                                    \
    : mode == 1 ? (gb ? rmsnorm_kernel<T, uint16_t, TW, 1, P> : rmsnorm_kernel<T, float, TW, 1, P>)    \
                : (gb ? rmsnorm_kernel<T, uint16_t, TW, 2, P> : rmsnorm_kernel<T, float, TW, 2, P>)
#define MABA_NRM_PICK(T, TW)                                                                           \
  if (nit <= 4) { MABA_NRM_PICKP(T, TW, 4); }                                                          \
  else if (nit <= 8) { MABA_NRM_PICKP(T, TW, 8); }                                                     \
  else { MABA_NRM_PICKP(T, TW, NRM_MAXP); }
  if (tb) { if (wb) { MABA_NRM_PICK(uint16_t, uint16_t); } else { MABA_NRM_PICK(uint16_t, float); } }
  else { if (wb) { MABA_NRM_PICK(float, uint16_t); } else { MABA_NRM_PICK(float, float); } }
#undef MABA_NRM_PICK
#undef MABA_NRM_PICKP
  hipLaunchKernelGGL(k, grid, dim3(256), 0, (hipStream_t)stream, a);
  return check_launch("rmsnorm");
}

extern "C" int maba_hip_swiglu(const maba_tensor* gate_up, maba_tensor* out, void* stream) {
  if (!gate_up || !out) return fail(MABA_ERR_INVALID, "swiglu: gate_up and out required");
  const int I = (int)out->shape[out->ndim - 1];
  if (gate_up->shape[gate_up->ndim - 1] != 2 * (int64_t)I || I % 2 != 0)
    return fail(MABA_ERR_INVALID, "swiglu: gate_up [.., 2I] and out [.., I] with I even");
  if (gate_up->dtype != out->dtype || (out->dtype != MABA_F32 && out->dtype != MABA_BF16))
    return fail(MABA_ERR_DTYPE, "swiglu: f32 or bf16, one dtype");
  SwigluArgs a;
  int64_t R, R2;
  if (!rows_of(gate_up, 2 * I, R, a.gus) || !rows_of(out, I, R2, a.os) || R2 != R)
    return fail(MABA_ERR_UNSUPPORTED, "swiglu: rows with unit channel stride required");
  a.gu = gate_up->data; a.out = out->data; a.R = R; a.I = I;
  if (R == 0) return MABA_OK;
  const bool rows16 = out->dtype == MABA_BF16 && I % 8 == 0 && I <= 64 * 8 * SW_MAXQ &&
                      (uintptr_t)a.gu % 16 == 0 && (uintptr_t)a.out % 16 == 0 &&
                      (R == 1 || (a.gus % 8 == 0 && a.os % 8 == 0)) && ceil_div(R, 4) <= 0x7fffffff;
  if (rows16) {
    hipLaunchKernelGGL(swiglu_rows_kernel, dim3((unsigned)ceil_div(R, 4)), dim3(256), 0, (hipStream_t)stream, a);
    return check_launch("swiglu");
  }
  const int64_t total = R * (I / 2);
  const unsigned blocks = (unsigned)std::min<int64_t>(ceil_div(total, 256), 65536);
  if (out->dtype == MABA_F32) hipLaunchKernelGGL(swiglu_kernel<float>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, a);
  else hipLaunchKernelGGL(swiglu_kernel<uint16_t>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, a);
  return check_launch("swiglu");
}

extern "C" int maba_hip_argmax_rows(const maba_tensor* x, maba_tensor* out, void* stream) {
  if (!x || !out) return fail(MABA_ERR_INVALID, "argmax_rows: x and out required");
  if (x->dtype != MABA_F32 && x->dtype != MABA_BF16) return fail(MABA_ERR_DTYPE, "argmax_rows: f32 or bf16 rows");
  const int64_t V = x->shape[x->ndim - 1], E = x->dtype == MABA_F32 ? 4 : 8;
  ArgmaxArgs a;
  int64_t R;
  if (V < 1 || V > (int64_t)INT32_MAX - 16 || V % E != 0 || !rows_of(x, (int)V, R, a.xs) ||
      (a.xs * (16 / E)) % 16 != 0 || (uintptr_t)x->data % 16 != 0 || (x->ndim == 3 && x->shape[1] != 1))
    return fail(MABA_ERR_UNSUPPORTED, "argmax_rows: rows [M,V] or [M,1,V] with unit stride, 16-byte aligned, "
                "V a multiple of %d", (int)E);
  if (out->dtype != MABA_I64 || out->shape[0] != R || out->ndim < 1 || out->ndim > 2 ||
      (out->ndim == 2 && out->shape[1] != 1))
    return fail(MABA_ERR_INVALID, "argmax_rows: out must be int64 [M] or [M,1]");
  a.x = x->data; a.out = (int64_t*)out->data; a.os = out->stride[0]; a.V = (int)V;
  if (R == 0) return MABA_OK;
  if (R > 0x7fffffff) return fail(MABA_ERR_UNSUPPORTED, "argmax_rows: too many rows");
  if (x->dtype == MABA_F32) hipLaunchKernelGGL(argmax_rows_kernel<float>, dim3((unsigned)R), dim3(AM_T), 0, (hipStream_t)stream, a);
  else hipLaunchKernelGGL(argmax_rows_kernel<uint16_t>, dim3((unsigned)R), dim3(AM_T), 0, (hipStream_t)stream, a);
  return check_launch("argmax_rows");
}

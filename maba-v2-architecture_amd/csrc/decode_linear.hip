// Decode-time linear layers of the full-model harness: y = A W^T for one token per sequence
// (M rows, one per sequence; W [N, K] bf16 in nn.Linear's layout), with the layer input stage
// that feeds A done inside the same launch:
//   PLAIN    A = a                                      rows [M, K]
//   GATHER   A = a[rows[m]]                             rows of a table (an embedding lookup,
//            model.py:95-102's in_emb before its projection)
//   NORM     A = RMSNorm(a) * nw                        reference model.py:11-22
//   NORMRES  A = RMSNorm(x') * nw, x' = a + g * mo      model.py:92-128 (MabaBlock's gated
//            residual; x' is stored to xo in bf16 and normalised as stored, like the separate
//            gated-residual RMSNorm kernel)
//   SWIGLU   A = silu(a[:, :K]) * a[:, K:2K]            model.py:25-38 (the stacked gate/up
//            GEMM's output)
// A is rounded to bf16 before the product, as the separate input kernel stores it; the product
// accumulates in fp32 on v_mfma_f32_16x16x32_bf16 and y is rounded to bf16.
//
// Work split: a workgroup of four waves makes one 16 x 16 tile of y (16 rows, 16 columns); the
// waves split K into four runs of 32-wide chunks and add their partial tiles through LDS in a
// fixed order.  Every wave issues all of its loads (the weight slice, the input rows and the
// gate and norm vectors) before it uses the first, with chunk indices clamped into K, so a
// launch costs about one memory round trip; the chunks a wave has past K enter the product as
// zeros.  The norm's sum of squares is per row: over the lane's elements, the four lanes of
// the row in the wave, then the four waves through LDS.  Decode M is small (the batch), so
// the weight read dominates: bound HBM at 2 N K bytes per launch.
#include <algorithm>

#include "maba_common.h"

namespace maba {

constexpr int DL_PLAIN = 0, DL_NORM = 1, DL_NORMRES = 2, DL_SWIGLU = 3, DL_GATHER = 4;

struct DlArgs {
  const uint16_t* a; int64_t as;      // input rows (SWIGLU: [M, 2K]; GATHER: the table)
  const int64_t* rows; int64_t rs;    // GATHER: table row of each output row (clamped into the table)
  int64_t nrows;                      // GATHER: rows of the table
  const uint16_t* mo; int64_t ms;     // NORMRES: residual branch rows [M, K]
  const uint16_t* g;                  // NORMRES: residual gate [K]
  const uint16_t* nw;                 // NORM, NORMRES: norm weight [K]
  uint16_t* xo; int64_t xos;          // NORMRES: x' rows [M, K], written by the column-tile 0 groups
  const uint16_t* w; int64_t ws;      // [N, K]
  uint16_t* y; int64_t ys;            // [M, N]
  int M, N, K;
  float eps;
};

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

__device__ __forceinline__ void unpack8(u32x4 u, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(u[i] << 16);
    f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
}

// Round to bf16 (v_cvt_pk_bf16_f32: round to nearest even, as f32_to_bf16_bits).
__device__ __forceinline__ uint32_t bf16_bits_hw(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 u;
#pragma unroll
  for (int i = 0; i < 4; ++i) u[i] = bf16_bits_hw(f[2 * i]) | (bf16_bits_hw(f[2 * i + 1]) << 16);
  return u;
}

// NW: waves of the workgroup (they split K); CPW: chunk slots per wave (>= ceil(K / (32 NW))).
template <int MODE, int NW, int CPW>
__global__ __launch_bounds__(64 * NW) void decode_linear_kernel(DlArgs a) {
  __shared__ float s_ss[NW][16];
  __shared__ __attribute__((aligned(16))) float s_acc[NW][64][4];
  asm volatile("" ::"s"(a.a), "s"(a.as), "s"(a.rows), "s"(a.rs), "s"(a.nrows), "s"(a.mo), "s"(a.ms), "s"(a.g), "s"(a.nw), "s"(a.xo), "s"(a.xos),
               "s"(a.w), "s"(a.ws), "s"(a.y), "s"(a.ys), "s"(a.M), "s"(a.N), "s"(a.K), "s"(a.eps));
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 15, q = lane >> 4;   // A row / W row (y column) of the lane, K quarter of the chunk
  const int m0 = blockIdx.y * 16, n0 = blockIdx.x * 16;
  int64_t m = min(m0 + r, a.M - 1);
  const int64_t n = min(n0 + r, a.N - 1);
  if constexpr (MODE == DL_GATHER) m = min(max(a.rows[m * a.rs], (int64_t)0), a.nrows - 1);   // ahead of the weight loads
  const int KC = a.K >> 5, c0 = wave * CPW;
  uint32_t zr;
  asm volatile("v_mov_b32 %0, 0" : "=v"(zr));   // an opaque zero: keeps every conversion out of the loads
  const u32x4 z4 = {zr, zr, zr, zr};
  u32x4 wb[CPW], xa[CPW], xm[CPW], xg[CPW], xn[CPW];
#pragma unroll
  for (int j = 0; j < CPW; ++j) wb[j] = *(const u32x4*)(a.w + n * a.ws + 32 * min(c0 + j, KC - 1) + 8 * q);
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int k = 32 * min(c0 + j, KC - 1) + 8 * q;
    xa[j] = *(const u32x4*)(a.a + m * a.as + k);
    xm[j] = z4; xg[j] = z4; xn[j] = z4;
    if constexpr (MODE == DL_NORMRES) {
      xm[j] = *(const u32x4*)(a.mo + m * a.ms + k);
      xg[j] = *(const u32x4*)(a.g + k);
    }
    if constexpr (MODE == DL_SWIGLU) xm[j] = *(const u32x4*)(a.a + m * a.as + a.K + k);
    if constexpr (MODE == DL_NORM || MODE == DL_NORMRES) xn[j] = *(const u32x4*)(a.nw + k);
  }
  __builtin_amdgcn_sched_barrier(0);   // no use of a load ahead of the last load's issue
  // input stage: the bf16 A operand of every chunk slot (zero past K)
  u32x4 av[CPW];
  if constexpr (MODE == DL_NORM || MODE == DL_NORMRES) {
    float v[CPW][8];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      const bool in = c0 + j < KC;   // wave-uniform
      unpack8(xa[j], v[j]);
      if constexpr (MODE == DL_NORMRES) {
        float mm[8], gg[8];
        unpack8(xm[j], mm);
        unpack8(xg[j], gg);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[j][i] = __uint_as_float(bf16_bits_hw(fmaf(gg[i], mm[i], v[j][i])) << 16);
        if (blockIdx.x == 0 && in && m0 + r < a.M)
          *(u32x4*)(a.xo + (int64_t)(m0 + r) * a.xos + 32 * (c0 + j) + 8 * q) = pack8(v[j]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v[j][i] = in ? v[j][i] : 0.f;
        ss = fmaf(v[j][i], v[j][i], ss);
      }
    }
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    if (q == 0) s_ss[wave][r] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += s_ss[w][r];
    const float inv = rsqrtf(tot / (float)a.K + a.eps);
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      float nn[8], h[8];
      unpack8(xn[j], nn);
#pragma unroll
      for (int i = 0; i < 8; ++i) h[i] = v[j][i] * inv * nn[i];
      av[j] = pack8(h);
    }
  } else if constexpr (MODE == DL_SWIGLU) {
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      float gg[8], uu[8], h[8];
      unpack8(xa[j], gg);
      unpack8(xm[j], uu);
#pragma unroll
      for (int i = 0; i < 8; ++i) h[i] = gg[i] * fast_rcp(1.f + fast_exp(-gg[i])) * uu[i];
      av[j] = pack8(h);
    }
  } else {
#pragma unroll
    for (int j = 0; j < CPW; ++j) av[j] = xa[j];
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const bool in = c0 + j < KC;
    const u32x4 A = in ? av[j] : z4, B = in ? wb[j] : z4;
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, A), __builtin_bit_cast(bf16x8, B), acc,
                                                  0, 0, 0);
  }
  *(f32x4*)s_acc[wave][lane] = acc;
  __syncthreads();
  // lane l holds y[m0 + 4 (l / 16) + i][n0 + l % 16], i < 4; wave w < 4 stores i = w
  if (wave < 4) {
    float val = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) val += s_acc[w][lane][wave];
    const int row = m0 + 4 * q + wave, col = n0 + r;
    if (row < a.M && col < a.N) a.y[(int64_t)row * a.ys + col] = (uint16_t)bf16_bits_hw(val);
  }
}

// Rows of a [M, C] / [M, 1, C] bf16 tensor with unit channel stride: the row stride.
static bool dl_rows(const maba_tensor* t, int64_t M, int64_t C, int64_t& rs) {
  if (!t || t->dtype != MABA_BF16 || t->shape[0] != M || t->shape[t->ndim - 1] != C || t->stride[t->ndim - 1] != 1)
    return false;
  if (t->ndim == 3) {
    if (t->shape[1] != 1) return false;
  } else if (t->ndim != 2) {
    return false;
  }
  rs = t->stride[0];
  return rs % 8 == 0 && (uintptr_t)t->data % 16 == 0;
}

// Whether the byte spans of the rows of two [M, ..] bf16 tensors (row strides rs, row lengths C) meet.
static bool overlaps(const maba_tensor* t, int64_t trs, int64_t tc, const maba_tensor* u, int64_t urs, int64_t uc) {
  const int64_t M = t->shape[0];
  if (M <= 0) return false;
  const char *t0 = (const char*)t->data, *u0 = (const char*)u->data;
  const char *t1 = t0 + 2 * ((M - 1) * trs + tc), *u1 = u0 + 2 * ((M - 1) * urs + uc);
  return t0 < u1 && u0 < t1;
}

static bool dl_vec(const maba_tensor* t, int64_t C) {
  return t && t->dtype == MABA_BF16 && t->ndim == 1 && t->shape[0] == C && t->stride[0] == 1 &&
         (uintptr_t)t->data % 16 == 0;
}

// The kernel for NW waves of `need` chunk slots each (the norm modes stop at 8 slots: their
// per-slot registers for more would spill).
template <int MODE, int NW, int CPW>
static void (*dl_fit())(DlArgs) {
  if constexpr ((MODE == DL_NORM || MODE == DL_NORMRES) && CPW > 8) return nullptr;
  else return decode_linear_kernel<MODE, NW, CPW>;
}

template <int MODE, int NW>
static void (*dl_pick(int need))(DlArgs) {
  if (need <= 1) return dl_fit<MODE, NW, 1>();
  if (need <= 2) return dl_fit<MODE, NW, 2>();
  if (need <= 3) return dl_fit<MODE, NW, 3>();
  if (need <= 4) return dl_fit<MODE, NW, 4>();
  if (need <= 5) return dl_fit<MODE, NW, 5>();
  if (need <= 6) return dl_fit<MODE, NW, 6>();
  if (need <= 8) return dl_fit<MODE, NW, 8>();
  if (need <= 10) return dl_fit<MODE, NW, 10>();
  if (need <= 12) return dl_fit<MODE, NW, 12>();
  if (need <= 16) return dl_fit<MODE, NW, 16>();
  return nullptr;
}

template <int NW>
static void (*dl_pick_mode(int mode, int need))(DlArgs) {
  return mode == DL_PLAIN ? dl_pick<DL_PLAIN, NW>(need)
       : mode == DL_GATHER ? dl_pick<DL_GATHER, NW>(need)
       : mode == DL_NORM ? dl_pick<DL_NORM, NW>(need)
       : mode == DL_NORMRES ? dl_pick<DL_NORMRES, NW>(need) : dl_pick<DL_SWIGLU, NW>(need);
}

// Waves per workgroup: eight from K = 1024 (measured on the config-5 widths: K = 1248 with
// SwiGLU input 5.7 -> 4.6 us per launch; at K <= 640 eight waves cost 0.3-0.5 us more).
static int dl_waves(int64_t K) { return K >= 1024 ? 8 : 4; }

}  // namespace maba

using namespace maba;

extern "C" int maba_hip_decode_linear(const maba_tensor* a, const maba_tensor* rows, const maba_tensor* mo,
                                      const maba_tensor* gate, const maba_tensor* norm_w, float eps, int act,
                                      const maba_tensor* weight, maba_tensor* x_out, maba_tensor* y, void* stream) {
  const char* who = "decode_linear";
  if (!a || !weight || !y) return fail(MABA_ERR_INVALID, "%s: a, weight and y required", who);
  if (rows && (act != 0 || norm_w || mo || gate || x_out))
    return fail(MABA_ERR_INVALID, "%s: rows take a plain table input", who);
  if (weight->ndim != 2 || weight->dtype != MABA_BF16 || weight->stride[1] != 1 || weight->stride[0] % 8 != 0 ||
      (uintptr_t)weight->data % 16 != 0)
    return fail(MABA_ERR_INVALID, "%s: weight must be bf16 [N,K], unit K stride, 16-byte aligned rows", who);
  const int64_t N = weight->shape[0], K = weight->shape[1];
  int64_t M = a->shape[0];
  if (rows) {   // rows [M] or [M, 1] int64: table rows
    if (rows->dtype != MABA_I64 || rows->ndim < 1 || rows->ndim > 2 || (rows->ndim == 2 && rows->shape[1] != 1))
      return fail(MABA_ERR_INVALID, "%s: rows must be int64 [M] or [M,1]", who);
    M = rows->shape[0];
  }
  if (K < 32 || K % 32 != 0) return fail(MABA_ERR_UNSUPPORTED, "%s: K must be a positive multiple of 32", who);
  if (N < 1 || N > (int64_t)INT32_MAX || M > (int64_t)16 * 65535)
    return fail(MABA_ERR_UNSUPPORTED, "%s: N or M out of range", who);
  if (act != 0 && act != 1) return fail(MABA_ERR_INVALID, "%s: act 0 (none) or 1 (swiglu)", who);
  if (act == 1 && norm_w) return fail(MABA_ERR_INVALID, "%s: swiglu input takes no norm", who);
  if ((mo || gate || x_out) && !(mo && gate && x_out && norm_w))
    return fail(MABA_ERR_INVALID, "%s: the gated residual needs mo, gate, x_out and norm_w", who);
  DlArgs d = {};
  if (rows) {
    if (a->ndim != 2 || a->dtype != MABA_BF16 || a->shape[1] != K || a->stride[1] != 1 || a->stride[0] % 8 != 0 ||
        (uintptr_t)a->data % 16 != 0 || a->shape[0] < 1)
      return fail(MABA_ERR_INVALID, "%s: the table must be bf16 [V,K], unit K stride, 16-byte aligned rows", who);
    d.as = a->stride[0];
    d.rows = (const int64_t*)rows->data; d.rs = rows->stride[0]; d.nrows = a->shape[0];
  } else if (!dl_rows(a, M, act == 1 ? 2 * K : K, d.as))
    return fail(MABA_ERR_INVALID, "%s: a must be bf16 [M,%s] or [M,1,%s] rows, unit channel stride, 16-byte aligned",
                who, act == 1 ? "2K" : "K", act == 1 ? "2K" : "K");
  if (y->dtype != MABA_BF16 || y->shape[0] != M || y->shape[y->ndim - 1] != N || y->stride[y->ndim - 1] != 1 ||
      !(y->ndim == 2 || (y->ndim == 3 && y->shape[1] == 1)))
    return fail(MABA_ERR_INVALID, "%s: y must be bf16 [M,N] or [M,1,N] with unit column stride", who);
  const int64_t ys = y->stride[0];
  int mode = act == 1 ? DL_SWIGLU : rows ? DL_GATHER : DL_PLAIN;
  if (norm_w) {
    if (!dl_vec(norm_w, K)) return fail(MABA_ERR_INVALID, "%s: norm_w must be bf16 [K], 16-byte aligned", who);
    mode = DL_NORM;
    d.nw = (const uint16_t*)norm_w->data;
  }
  if (mo) {
    if (!dl_rows(mo, M, K, d.ms)) return fail(MABA_ERR_INVALID, "%s: mo must match a", who);
    if (!dl_vec(gate, K)) return fail(MABA_ERR_INVALID, "%s: gate must be bf16 [K], 16-byte aligned", who);
    if (!dl_rows(x_out, M, K, d.xos)) return fail(MABA_ERR_INVALID, "%s: x_out must match a", who);
    // x_out is written while other workgroups read a and mo: it may overlap neither
    if (overlaps(x_out, d.xos, K, a, d.as, K) || overlaps(x_out, d.xos, K, mo, d.ms, K))
      return fail(MABA_ERR_INVALID, "%s: x_out may not overlap a or mo", who);
    // every workgroup reads mo and the first column of workgroups writes x_out while others
    // write y: y may overlap neither
    if (M > 0 && (overlaps(y, ys, N, mo, d.ms, K) || overlaps(y, ys, N, x_out, d.xos, K)))
      return fail(MABA_ERR_INVALID, "%s: y may not overlap mo or x_out", who);
    mode = DL_NORMRES;
    d.mo = (const uint16_t*)mo->data; d.g = (const uint16_t*)gate->data; d.xo = (uint16_t*)x_out->data;
  }
  if (M > 0 && !rows && overlaps(y, ys, N, a, d.as, act == 1 ? 2 * K : K))
    return fail(MABA_ERR_INVALID, "%s: y may not overlap a", who);
  const int nw = dl_waves(K);
  const int need = (int)((K / 32 + nw - 1) / nw);   // chunk slots per wave
  void (*k)(DlArgs) = nw == 8 ? dl_pick_mode<8>(mode, need) : dl_pick_mode<4>(mode, need);
  if (!k) return fail(MABA_ERR_UNSUPPORTED, "%s: K <= 4096 (2048 with a norm)", who);
  d.a = (const uint16_t*)a->data; d.w = (const uint16_t*)weight->data; d.ws = weight->stride[0];
  d.y = (uint16_t*)y->data; d.ys = ys;
  d.M = (int)M; d.N = (int)N; d.K = (int)K; d.eps = eps;
  if (M == 0) return MABA_OK;
  const dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16));
  hipLaunchKernelGGL(k, grid, dim3(64 * nw), 0, (hipStream_t)stream, d);
  return check_launch(who);
}

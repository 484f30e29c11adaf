// Block pooling kernels over token-major [B, L, d] tensors.
//
//  * compute_centroids: c_n = 0.5*(mean + max) over a block of block_size
//    tokens; the tail block is zero-padded and the padding takes part in both
//    the mean (divide by block_size) and the max
//    (reference: maba_sparse/kernels/common.py:343-350, cpu_indexer.py:38-50).
//  * hca_pool: mean of each complete pool-token block of the MLA latent cache
//    (reference: layers/sparse_attention.py:206).
//
// Both are pure streaming reductions (HBM-bound, ~2 flop per element read).
// One wave reduces one block: each lane loads VEC consecutive channels (16 B),
// LPR lanes cover one token row, so a wave instruction reads 64/LPR rows
// (1 KiB) fully coalesced; partial sums/maxima are combined across the lane
// groups with cross-lane shuffles.
#include "maba_common.h"

namespace maba {

struct PoolArgs {
  const void* x;
  int dt;
  int64_t sb, sl;    // element strides of x (channel stride is 1)
  void* out;
  int odt;
  int64_t ob, on;    // element strides of out (channel stride is 1)
  int64_t L, nblk, d;
  int bs;
  int mode;          // 0 = centroid (0.5*(mean+max)), 1 = mean of complete blocks
  int64_t total;     // B * nblk
};

template <typename T>
struct Vec16;
template <> struct Vec16<float> { static constexpr int N = 4; };
template <> struct Vec16<uint16_t> { static constexpr int N = 8; };

template <typename T>
__device__ __forceinline__ float to_f32(T v, int dt);
template <> __device__ __forceinline__ float to_f32<float>(float v, int) { return v; }
template <> __device__ __forceinline__ float to_f32<uint16_t>(uint16_t v, int dt) {
  if (dt == MABA_BF16) return bf16_bits_to_f32(v);
  __half h;
  __builtin_memcpy(&h, &v, 2);
  return __half2float(h);
}

// Vectorised path: d*sizeof(T) is a multiple of 16 and LPR = d/VEC divides 64.
template <typename T, int LPR>
__global__ __launch_bounds__(256) void pool_vec_kernel(PoolArgs a) {
  constexpr int VEC = Vec16<T>::N;
  constexpr int RPI = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= a.total) return;
  const int64_t bi = item / a.nblk, n = item % a.nblk;
  const int cg = lane % LPR, r = lane / LPR;
  float sum[VEC], mx[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) { sum[j] = 0.f; mx[j] = -INFINITY; }
  const T* base = (const T*)a.x + bi * a.sb + (int64_t)cg * VEC;
  const int64_t t0 = n * a.bs;
  for (int t = r; t < a.bs; t += RPI) {
    const int64_t tok = t0 + t;
    T v[VEC];
    if (tok < a.L) {
      *(uint4*)v = *(const uint4*)(base + tok * a.sl);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = (T)0;
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float f = to_f32<T>(v[j], a.dt);
      sum[j] += f;
      mx[j] = fmaxf(mx[j], f);
    }
  }
#pragma unroll
  for (int off = LPR; off < 64; off <<= 1) {
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      sum[j] += __shfl_xor(sum[j], off);
      mx[j] = fmaxf(mx[j], __shfl_xor(mx[j], off));
    }
  }
  if (r == 0) {
    const float inv = 1.0f / (float)a.bs;
    const int64_t obase = bi * a.ob + n * a.on + (int64_t)cg * VEC;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float res = a.mode == 0 ? 0.5f * (sum[j] * inv + mx[j]) : sum[j] * inv;
      store_elem(a.out, a.odt, obase + j, res);
    }
  }
}

// Scalar path for any d: one thread per channel, one workgroup per block.
__global__ __launch_bounds__(256) void pool_scalar_kernel(PoolArgs a, int64_t xsd) {
  const int64_t item = blockIdx.x;
  const int64_t bi = item / a.nblk, n = item % a.nblk;
  for (int64_t c = threadIdx.x; c < a.d; c += blockDim.x) {
    float sum = 0.f, mx = -INFINITY;
    for (int t = 0; t < a.bs; ++t) {
      const int64_t tok = n * a.bs + t;
      const float f = tok < a.L ? load_elem(a.x, a.dt, bi * a.sb + tok * a.sl + c * xsd) : 0.f;
      sum += f;
      mx = fmaxf(mx, f);
    }
    const float inv = 1.0f / (float)a.bs;
    const float res = a.mode == 0 ? 0.5f * (sum * inv + mx) : sum * inv;
    store_elem(a.out, a.odt, bi * a.ob + n * a.on + c, res);
  }
}

static int launch_pool(const maba_tensor* x, maba_tensor* out, int bs, int mode, int64_t nblk,
                       hipStream_t s, const char* what) {
  const int64_t B = x->shape[0], L = x->shape[1], d = x->shape[2];
  if (out->stride[2] != 1) return fail(MABA_ERR_UNSUPPORTED, "%s: out must be contiguous in the channel dim", what);
  PoolArgs a;
  a.x = x->data; a.dt = x->dtype; a.sb = x->stride[0]; a.sl = x->stride[1];
  a.out = out->data; a.odt = out->dtype; a.ob = out->stride[0]; a.on = out->stride[1];
  a.L = L; a.nblk = nblk; a.d = d; a.bs = bs; a.mode = mode; a.total = B * nblk;
  if (a.total == 0 || d == 0) return MABA_OK;
  const int es = x->dtype == MABA_F32 ? 4 : 2;
  const int vec = 16 / es;
  const bool aligned = ((uintptr_t)x->data % 16 == 0) && ((a.sb * es) % 16 == 0) && ((a.sl * es) % 16 == 0);
  const int64_t lpr = d / vec;
  const bool vec_ok = x->stride[2] == 1 && aligned && d % vec == 0 && lpr >= 1 && lpr <= 64 && (64 % lpr) == 0;
  dim3 block(256);
  if (vec_ok) {
    dim3 grid((unsigned)ceil_div(a.total, 4));
#define MABA_POOL_LAUNCH(T, LPRV) hipLaunchKernelGGL((pool_vec_kernel<T, LPRV>), grid, block, 0, s, a)
#define MABA_POOL_SWITCH(T)                                  \
  switch (lpr) {                                             \
    case 1: MABA_POOL_LAUNCH(T, 1); break;                   \
    case 2: MABA_POOL_LAUNCH(T, 2); break;                   \
    case 4: MABA_POOL_LAUNCH(T, 4); break;                   \
    case 8: MABA_POOL_LAUNCH(T, 8); break;                   \
    case 16: MABA_POOL_LAUNCH(T, 16); break;                 \
    case 32: MABA_POOL_LAUNCH(T, 32); break;                 \
    default: MABA_POOL_LAUNCH(T, 64); break;                 \
  }
    if (es == 4) { MABA_POOL_SWITCH(float) } else { MABA_POOL_SWITCH(uint16_t) }
#undef MABA_POOL_SWITCH
#undef MABA_POOL_LAUNCH
  } else {
    dim3 grid((unsigned)a.total);
    hipLaunchKernelGGL(pool_scalar_kernel, grid, block, 0, s, a, x->stride[2]);
  }
  return check_launch(what);
}

}  // namespace maba

using namespace maba;

extern "C" int maba_hip_compute_centroids(const maba_tensor* k_idx, maba_tensor* out, int block_size,
                                         void* stream) {
  if (!k_idx || k_idx->ndim != 3) return fail(MABA_ERR_INVALID, "compute_centroids: k_idx must be [B,L,d]");
  if (block_size <= 0) return fail(MABA_ERR_INVALID, "compute_centroids: block_size must be positive, got %d", block_size);
  const int64_t B = k_idx->shape[0], L = k_idx->shape[1], d = k_idx->shape[2];
  const int64_t nb = ceil_div(L, block_size);
  const int64_t so[3] = {B, nb, d};
  if (!expect_shape(out, "out", 3, so)) return MABA_ERR_INVALID;
  if (!expect_float(k_idx, "k_idx") || !expect_float(out, "out")) return MABA_ERR_DTYPE;
  return launch_pool(k_idx, out, block_size, 0, nb, (hipStream_t)stream, "compute_centroids");
}

extern "C" int maba_hip_hca_pool(const maba_tensor* c_kv, maba_tensor* out, int pool, void* stream) {
  if (!c_kv || c_kv->ndim != 3) return fail(MABA_ERR_INVALID, "hca_pool: c_kv must be [B,L,dc]");
  if (pool <= 0) return fail(MABA_ERR_INVALID, "hca_pool: pool must be positive");
  const int64_t B = c_kv->shape[0], L = c_kv->shape[1], d = c_kv->shape[2];
  const int64_t nc = L / pool;
  const int64_t so[3] = {B, nc, d};
  if (!expect_shape(out, "out", 3, so)) return MABA_ERR_INVALID;
  if (!expect_float(c_kv, "c_kv") || !expect_float(out, "out")) return MABA_ERR_DTYPE;
  return launch_pool(c_kv, out, pool, 1, nc, (hipStream_t)stream, "hca_pool");
}

// Decode-time cache append: one launch per decode token and MABA-SA layer.
//
// Reference semantics:
//   layers/indexer.py:62-82          the new indexer key joins the key cache; a completed
//                                    block adds its centroid 0.5 (mean + max); otherwise the
//                                    zero-padded tail block's centroid stands in for the last
//                                    block (the padding counts in the mean and the max)
//   layers/sparse_attention.py:206   the HCA stream attends to the means of complete
//                                    pool-token blocks of the latent cache
//   (the latent row itself is the reference's per-step concatenation, :241-251)
//
// Cache format (device memory, all bf16, rows of one sequence contiguous):
//   c     [B, Lmax, dc]        latent rows; rows [0, n) valid
//   keys  [B, Lmax, di]        indexer keys; rows [0, n) valid
//   hca   [B, Lmax/pool, dc]   means of the complete pool-blocks: entries [0, n/pool) valid
//   cent  [B, ceil(Lmax/bs), di]  centroids: entries [0, ceil(n/bs)) valid, the last one the
//                              zero-padded tail centroid while its block is incomplete
// The new row goes to index p = *pos (a device scalar, so that one captured launch serves
// every position); the caller advances *pos after the step.  One workgroup per sequence:
// it reduces the block that holds row p, taking row p from the inputs and rows before it
// from the caches (written by earlier launches), then writes the two rows.
//
// The same launch can also form the token's absorbed queries and gate logits, which the
// decode streams read next (layers/sparse_attention.py:79-219 with the latent absorption
// <q_h, W_k,h c> = <W_k,h^T q_h, c>, and :274, W_g x + b): B * H more workgroups, one per
// (b, h), write q_lat[b, h, :] = W_k,h^T q_h in fp32 (bf16 products, exact in fp32, summed
// in fp32), and the first of each sequence writes the gate logits plus bias, rounded to bf16
// as the bf16 addition of the two would be.
#include "maba_common.h"

namespace maba {

constexpr int AP_T = 256;
constexpr int AP_MAXD = 256;

struct AppendArgs {
  const uint16_t* cn; int64_t cnsb, cnsd;   // new latent rows [B, dc]
  const uint16_t* kn; int64_t knsb, knsd;   // new keys [B, di]
  uint16_t* c; int64_t csb, csl;            // latent cache, channel stride 1
  uint16_t* k; int64_t ksb, ksl;            // key cache, channel stride 1
  uint16_t* hca; int64_t hsb, hsn;          // block means, channel stride 1
  uint16_t* cent; int64_t esb, esn;         // centroids, channel stride 1
  const int64_t* pos;
  int64_t Lmax, nh_max, nc_max;
  int dc, di, pool, bs;
  // absorbed queries and gate logits (qh null: not formed)
  const uint16_t* qh; int64_t qhsb, qhsd;   // q projection [B, H * dh] bf16
  const uint16_t* wk; int64_t wks;          // W_k [H * dh, dc] bf16, unit column stride
  float* ql; int64_t qlsb, qlsh;            // q_lat [B, H, dc] fp32, unit channel stride
  const uint16_t* gin; int64_t ginsb, ginsd;   // gate logits [B, 3] bf16
  const uint16_t* gbias; int64_t gbsd;         // gate bias [3] bf16
  uint16_t* gout; int64_t goutsb, goutsd;      // gate logits + bias [B, 3] bf16
  int H, dh;
};

// Column reduction of rows [r0, p) of a cache plus the new row (newrow[col * nsd]): sum
// (and max when WITH_MAX) per column; the threads split the rows in AP_T / d parts, and
// thread `col` of the result holds column col.  Each thread loads AP_BATCH of its rows
// before it adds the first (rows past p reread row rb, which is < p, and add nothing), so
// a block costs one or two memory round trips rather than one per row; the rows are still
// added in ascending order, one at a time.
constexpr int AP_BATCH = 16;

template <bool WITH_MAX>
__device__ void ap_reduce(const uint16_t* base, int64_t rstride, int64_t r0, int64_t p, int d,
                          const uint16_t* newrow, int64_t nsd, float* s_sum, float* s_max, float& sum, float& mx) {
  const int tid = threadIdx.x;
  const int parts = AP_T / d;
  const int col = tid % d, part = tid / d;
  float s = 0.f, m = -INFINITY;
  if (part < parts) {
    const float xn = bf16_bits_to_f32(newrow[col * nsd]);   // added by the last part only
    for (int64_t rb = r0 + part; rb < p; rb += (int64_t)AP_BATCH * parts) {
      uint16_t x[AP_BATCH];
#pragma unroll
      for (int k = 0; k < AP_BATCH; ++k) {
        const int64_t r = rb + (int64_t)k * parts;
        x[k] = base[(r < p ? r : rb) * rstride + col];
      }
#pragma unroll
      for (int k = 0; k < AP_BATCH; ++k) {
        const bool in = rb + (int64_t)k * parts < p;
        const float v = bf16_bits_to_f32(x[k]);
        s += in ? v : 0.f;   // s is never -0, so adding +0 leaves it unchanged
        if (WITH_MAX) m = in ? fmaxf(m, v) : m;
      }
    }
    if (part == parts - 1) {
      s += xn;
      if (WITH_MAX) m = fmaxf(m, xn);
    }
    s_sum[part * d + col] = s;
    if (WITH_MAX) s_max[part * d + col] = m;
  }
  __syncthreads();
  sum = 0.f;
  mx = -INFINITY;
  if (tid < d) {
    for (int q = 0; q < parts; ++q) {   // fixed order: deterministic
      sum += s_sum[q * d + tid];
      if (WITH_MAX) mx = fmaxf(mx, s_max[q * d + tid]);
    }
  }
  __syncthreads();
}

// q_lat[b, h, c] = sum_d q[b, h dh + d] W_k[h dh + d, c]: thread (part, c) sums its part of
// the d range in ascending order, the parts are added in a fixed order (deterministic).
__device__ void ap_absorbed_query(const AppendArgs& a, int64_t b, int h, float* s_part) {
  const int tid = threadIdx.x;
  const int parts = AP_T / a.dc;
  const int c = tid % a.dc, part = tid / a.dc;
  const int per = (a.dh + parts - 1) / parts;
  float acc = 0.f;
  if (part < parts) {
    const int d0 = part * per, d1 = min(a.dh, d0 + per);
    const uint16_t* q = a.qh + b * a.qhsb + (int64_t)h * a.dh * a.qhsd;
    const uint16_t* w = a.wk + (int64_t)h * a.dh * a.wks + c;
    for (int d = d0; d < d1; d += AP_BATCH) {   // a batch of loads in flight, then its products in order
      uint16_t qv[AP_BATCH], wv[AP_BATCH];
#pragma unroll
      for (int k = 0; k < AP_BATCH; ++k) {
        const int dd = min(d + k, d1 - 1);
        qv[k] = q[dd * a.qhsd];
        wv[k] = w[dd * a.wks];
      }
#pragma unroll
      for (int k = 0; k < AP_BATCH; ++k)
        if (d + k < d1) acc = fmaf(bf16_bits_to_f32(qv[k]), bf16_bits_to_f32(wv[k]), acc);
    }
    s_part[part * a.dc + c] = acc;
  }
  __syncthreads();
  if (tid < a.dc) {
    float r = 0.f;
    for (int q = 0; q < parts; ++q) r += s_part[q * a.dc + tid];
    a.ql[b * a.qlsb + (int64_t)h * a.qlsh + tid] = r;
  }
  if (h == 0 && tid < 3) {
    const float g = bf16_bits_to_f32(a.gin[b * a.ginsb + tid * a.ginsd]) + bf16_bits_to_f32(a.gbias[tid * a.gbsd]);
    a.gout[b * a.goutsb + tid * a.goutsd] = f32_to_bf16_bits(g);
  }
}

__global__ __launch_bounds__(AP_T) void cache_append_kernel(AppendArgs a, int64_t B) {
  __shared__ float s_sum[AP_T], s_max[AP_T];
  if ((int64_t)blockIdx.x >= B) {   // absorbed query of one (b, h)
    const int64_t j = blockIdx.x - B;
    ap_absorbed_query(a, j / a.H, (int)(j % a.H), s_sum);
    return;
  }
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  // the new rows, loaded together with the position; they are stored last, so that no
  // load of the reductions (rows before p only) waits behind their stores
  const uint16_t xc = a.cn[b * a.cnsb + min(tid, a.dc - 1) * a.cnsd];
  const uint16_t xk = a.kn[b * a.knsb + min(tid, a.di - 1) * a.knsd];
  const int64_t p = *a.pos;
  if (p < 0 || p >= a.Lmax) return;   // the host checks capacity; never write out of bounds
  // centroid of the block holding row p: complete, or the zero-padded tail
  const int64_t blk = p / a.bs;
  const int64_t r0 = blk * a.bs;
  float sum, mx;
  ap_reduce<true>(a.k + b * a.ksb, a.ksl, r0, p, a.di, a.kn + b * a.knsb, a.knsd, s_sum, s_max, sum, mx);
  if (tid < a.di && blk < a.nc_max) {
    if (p - r0 + 1 < a.bs) mx = fmaxf(mx, 0.f);   // the zero padding takes part in the max
    const float c = 0.5f * (sum * (1.0f / (float)a.bs) + mx);
    a.cent[b * a.esb + blk * a.esn + tid] = f32_to_bf16_bits(c);
  }
  // HCA mean of the pool-block that row p completes
  if ((p + 1) % a.pool == 0) {
    const int64_t e = (p + 1) / a.pool - 1;
    ap_reduce<false>(a.c + b * a.csb, a.csl, p + 1 - a.pool, p, a.dc, a.cn + b * a.cnsb, a.cnsd, s_sum, s_max,
                     sum, mx);
    if (tid < a.dc && e < a.nh_max) a.hca[b * a.hsb + e * a.hsn + tid] = f32_to_bf16_bits(sum * (1.0f / (float)a.pool));
  }
  if (tid < a.dc) a.c[b * a.csb + p * a.csl + tid] = xc;
  if (tid < a.di) a.k[b * a.ksb + p * a.ksl + tid] = xk;
}

}  // namespace maba

using namespace maba;

static int cache_append(const maba_tensor* c_new, const maba_tensor* k_new, const int64_t* pos,
                        maba_tensor* c_cache, maba_tensor* k_cache, maba_tensor* hca, maba_tensor* centroids,
                        int pool, int block_size, const maba_tensor* q_heads, const maba_tensor* w_k,
                        const maba_tensor* gate_in, const maba_tensor* gate_bias, maba_tensor* q_lat,
                        maba_tensor* gate_out, void* stream) {
  if (!c_new || c_new->ndim != 2 || !k_new || k_new->ndim != 2)
    return fail(MABA_ERR_INVALID, "cache_append: c_new must be [B,dc] and k_new [B,di]");
  const int64_t B = c_new->shape[0], dc = c_new->shape[1], di = k_new->shape[1];
  if (k_new->shape[0] != B) return fail(MABA_ERR_INVALID, "cache_append: batch mismatch");
  if (!pos) return fail(MABA_ERR_INVALID, "cache_append: pos (device int64) required");
  if (pool <= 0 || block_size <= 0) return fail(MABA_ERR_INVALID, "cache_append: bad pool / block size");
  if (!c_cache || c_cache->ndim != 3 || c_cache->shape[0] != B || c_cache->shape[2] != dc)
    return fail(MABA_ERR_INVALID, "cache_append: c_cache must be [B,Lmax,dc]");
  const int64_t Lmax = c_cache->shape[1];
  const int64_t sk[3] = {B, Lmax, di};
  if (!expect_shape(k_cache, "k_cache", 3, sk)) return MABA_ERR_INVALID;
  if (!hca || hca->ndim != 3 || hca->shape[0] != B || hca->shape[2] != dc || hca->shape[1] < Lmax / pool)
    return fail(MABA_ERR_INVALID, "cache_append: hca must be [B,>=Lmax/pool,dc]");
  if (!centroids || centroids->ndim != 3 || centroids->shape[0] != B || centroids->shape[2] != di ||
      centroids->shape[1] < ceil_div(Lmax, block_size))
    return fail(MABA_ERR_INVALID, "cache_append: centroids must be [B,>=ceil(Lmax/block),di]");
  const maba_tensor* all[] = {c_new, k_new, c_cache, k_cache, hca, centroids};
  for (const maba_tensor* t : all)
    if (t->dtype != MABA_BF16) return fail(MABA_ERR_DTYPE, "cache_append: bf16 tensors only");
  if (dc > AP_MAXD || di > AP_MAXD || dc < 1 || di < 1)
    return fail(MABA_ERR_UNSUPPORTED, "cache_append: dc and di in [1, %d]", AP_MAXD);
  for (const maba_tensor* t : {c_cache, k_cache, hca, centroids})
    if (t->stride[2] != 1) return fail(MABA_ERR_UNSUPPORTED, "cache_append: caches need unit channel stride");
  if (B == 0) return MABA_OK;
  AppendArgs a;
  a.cn = (const uint16_t*)c_new->data; a.cnsb = c_new->stride[0]; a.cnsd = c_new->stride[1];
  a.kn = (const uint16_t*)k_new->data; a.knsb = k_new->stride[0]; a.knsd = k_new->stride[1];
  a.c = (uint16_t*)c_cache->data; a.csb = c_cache->stride[0]; a.csl = c_cache->stride[1];
  a.k = (uint16_t*)k_cache->data; a.ksb = k_cache->stride[0]; a.ksl = k_cache->stride[1];
  a.hca = (uint16_t*)hca->data; a.hsb = hca->stride[0]; a.hsn = hca->stride[1];
  a.cent = (uint16_t*)centroids->data; a.esb = centroids->stride[0]; a.esn = centroids->stride[1];
  a.pos = pos;
  a.Lmax = Lmax; a.nh_max = hca->shape[1]; a.nc_max = centroids->shape[1];
  a.dc = (int)dc; a.di = (int)di; a.pool = pool; a.bs = block_size;
  a.qh = nullptr; a.H = 0; a.dh = 0;
  int64_t nq = 0;
  if (q_heads) {   // absorbed queries and gate logits in the same launch
    // q_lat's head count is checked positive before it divides anything
    if (q_heads->ndim != 2 || q_heads->shape[0] != B || !w_k || w_k->ndim != 2 || w_k->shape[1] != dc ||
        w_k->shape[0] != q_heads->shape[1] || !q_lat || q_lat->ndim != 3 || q_lat->shape[0] != B ||
        q_lat->shape[2] != dc || q_lat->shape[1] < 1 || w_k->shape[0] < q_lat->shape[1] ||
        w_k->shape[0] % q_lat->shape[1] != 0)
      return fail(MABA_ERR_INVALID, "cache_append: q_heads [B,H*dh], w_k [H*dh,dc], q_lat [B,H,dc] required");
    const int64_t so[2] = {B, 3}, sb[1] = {3};
    if (!expect_shape(gate_in, "gate_in", 2, so) || !expect_shape(gate_out, "gate_out", 2, so) ||
        !expect_shape(gate_bias, "gate_bias", 1, sb))
      return MABA_ERR_INVALID;
    for (const maba_tensor* t : {q_heads, w_k, gate_in, gate_bias, (const maba_tensor*)gate_out})
      if (t->dtype != MABA_BF16) return fail(MABA_ERR_DTYPE, "cache_append: bf16 q_heads, w_k and gate tensors");
    if (q_lat->dtype != MABA_F32 || q_lat->stride[2] != 1 || w_k->stride[1] != 1)
      return fail(MABA_ERR_DTYPE, "cache_append: q_lat f32 and w_k with unit channel strides");
    a.qh = (const uint16_t*)q_heads->data; a.qhsb = q_heads->stride[0]; a.qhsd = q_heads->stride[1];
    a.wk = (const uint16_t*)w_k->data; a.wks = w_k->stride[0];
    a.ql = (float*)q_lat->data; a.qlsb = q_lat->stride[0]; a.qlsh = q_lat->stride[1];
    a.gin = (const uint16_t*)gate_in->data; a.ginsb = gate_in->stride[0]; a.ginsd = gate_in->stride[1];
    a.gbias = (const uint16_t*)gate_bias->data; a.gbsd = gate_bias->stride[0];
    a.gout = (uint16_t*)gate_out->data; a.goutsb = gate_out->stride[0]; a.goutsd = gate_out->stride[1];
    a.H = (int)q_lat->shape[1];
    a.dh = (int)(w_k->shape[0] / a.H);
    nq = B * a.H;
  }
  hipLaunchKernelGGL(cache_append_kernel, dim3((unsigned)(B + nq)), dim3(AP_T), 0, (hipStream_t)stream, a, B);
  return check_launch("cache_append");
}

extern "C" int maba_hip_cache_append(const maba_tensor* c_new, const maba_tensor* k_new, const int64_t* pos,
                                     maba_tensor* c_cache, maba_tensor* k_cache, maba_tensor* hca,
                                     maba_tensor* centroids, int pool, int block_size, void* stream) {
  return cache_append(c_new, k_new, pos, c_cache, k_cache, hca, centroids, pool, block_size, nullptr, nullptr,
                      nullptr, nullptr, nullptr, nullptr, stream);
}

extern "C" int maba_hip_cache_append_heads(const maba_tensor* c_new, const maba_tensor* k_new, const int64_t* pos,
                                           maba_tensor* c_cache, maba_tensor* k_cache, maba_tensor* hca,
                                           maba_tensor* centroids, int pool, int block_size,
                                           const maba_tensor* q_heads, const maba_tensor* w_k,
                                           const maba_tensor* gate_in, const maba_tensor* gate_bias,
                                           maba_tensor* q_lat, maba_tensor* gate_out, void* stream) {
  if (!q_heads) return fail(MABA_ERR_INVALID, "cache_append_heads: q_heads required");
  return cache_append(c_new, k_new, pos, c_cache, k_cache, hca, centroids, pool, block_size, q_heads, w_k,
                      gate_in, gate_bias, q_lat, gate_out, stream);
}

// Fused MABA-SA decode step over an MLA latent cache.
//
// Reference semantics (maba_sparse/layers/sparse_attention.py):
//   local  (:84-93)   keys {0..min(4,L)-1} U [max(min(4,L), L-128), L)
//   sparse (:129-143) the 64-token blocks in idx[b, :] with position < L; one
//                     index set per batch element shared by all heads, or one
//                     per head
//   HCA    (:173-219) for pos = L-1 >= 63: attention over the means of all
//                     complete 64-blocks; for pos < 63 the running mean of
//                     c[0..pos]
//   gate   (:274-275) out = sum_s softmax(logits)_s * o_s
// With the latent absorption <q_h, W_k,h c> = <W_k,h^T q_h, c> and
// sum_j p_j W_v,h c_j = W_v,h sum_j p_j c_j, every stream is softmax attention
// of q_lat[b,h] against latent rows c_j with the latent rows as values, and the
// kernel returns z[b,h] = sum_s g_s z_s (fp32, [B,H,dc]).
//
// Kernel 1 splits every stream of every batch element into 64-key tiles (one
// workgroup per tile) and writes a flash-decoding partial (max, sum, weighted
// latent sum) per head.  Kernel 2 merges the partials of each (b, h, stream),
// applies the gate softmax and writes z.  Traffic is one read of the selected
// latent rows (bf16) plus small partials: HBM-bound.
#include "maba_common.h"

namespace maba {

constexpr int SA_MAXH = 16;
constexpr int SA_MAXDC = 256;

struct SaArgs {
  const void* q; int qdt; int64_t qsb, qsh, qsd;
  const void* c; int cdt; int64_t csb, csl, csd;
  const void* hca; int hdt; int64_t hsb, hsn, hsd;
  const int64_t* idx; int64_t isb, ish, isk;
  const void* gate; int gdt; int64_t gsb, gsh, gsm;  // gsh = 0 for [B,3]
  float* out; int64_t osb, osh, osd;
  float* ws;
  int64_t L;
  int H, dc, Hi, K, window, n_sink, bs, pool;
  int ns, loc_start, nloc, nc;           // local / hca geometry
  int t_loc, t_sp, t_hca, ntiles;        // tile counts per batch element
  float scale;
};

__device__ __forceinline__ int64_t sa_part_off(const SaArgs& a, int64_t b, int tile, int h) {
  return (((b * a.ntiles + tile) * a.H) + h) * (int64_t)(a.dc + 2);
}

__global__ __launch_bounds__(256) void maba_sa_tile_kernel(SaArgs a) {
  __shared__ float s_c[64][SA_MAXDC + 1];
  __shared__ float s_q[SA_MAXH][SA_MAXDC];
  __shared__ float s_p[SA_MAXH][64];
  __shared__ float s_red[2][SA_MAXH][SA_MAXDC];
  const int tile = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int H = a.H, dc = a.dc;

  // Which stream / keys does this tile cover?
  int stream, head_only = -1;
  int64_t base = 0;  // local: list offset; sparse: block; hca: entry offset
  if (tile < a.t_loc) {
    stream = 0;
    base = (int64_t)tile * 64;
  } else if (tile < a.t_loc + a.t_sp) {
    stream = 1;
    const int r = tile - a.t_loc;
    const int hs = r / a.K, kk = r % a.K;
    base = a.idx[b * a.isb + hs * a.ish + kk * a.isk];
    if (a.Hi > 1) head_only = hs;
  } else {
    stream = 2;
    base = (int64_t)(tile - a.t_loc - a.t_sp) * 64;
  }
  // Key position / validity of row j.
  auto key_of = [&](int j, int64_t& pos) -> bool {
    if (stream == 0) {
      const int64_t li = base + j;
      if (li >= a.nloc) return false;
      pos = li < a.ns ? li : a.loc_start + (li - a.ns);
      return true;
    } else if (stream == 1) {
      const int64_t nblk = (a.L + a.bs - 1) / a.bs;
      if (base < 0 || base >= nblk || j >= a.bs) return false;
      pos = base * a.bs + j;
      return pos < a.L;
    } else {
      const int64_t e = base + j;
      pos = e;
      return e < a.nc;
    }
  };
  // Stage the 64 key rows (fp32) and the queries.
  for (int i = tid; i < 64 * dc; i += 256) {
    const int j = i / dc, d = i % dc;
    int64_t pos = 0;
    float x = 0.f;
    if (key_of(j, pos)) {
      x = stream == 2 ? load_elem(a.hca, a.hdt, b * a.hsb + pos * a.hsn + d * a.hsd)
                      : load_elem(a.c, a.cdt, b * a.csb + pos * a.csl + d * a.csd);
    }
    s_c[j][d] = x;
  }
  for (int i = tid; i < H * dc; i += 256) {
    const int h = i / dc, d = i % dc;
    s_q[h][d] = load_elem(a.q, a.qdt, b * a.qsb + h * a.qsh + d * a.qsd) * a.scale;
  }
  __syncthreads();

  // Scores: wave w handles heads w, w+4, ...; lane = key.
  int64_t mypos = 0;
  const bool kvalid = key_of(lane, mypos);
  for (int h = wave; h < H; h += 4) {
    const bool active = head_only < 0 || head_only == h;
    float s = -INFINITY;
    if (active && kvalid) {
      float acc = 0.f;
      for (int d = 0; d < dc; ++d) acc = fmaf(s_q[h][d], s_c[lane][d], acc);
      s = acc;
    }
    float m = s;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    const float p = (m == -INFINITY) ? 0.f : __expf(s - m);
    float l = p;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
    s_p[h][lane] = p;
    if (lane == 0) {
      const int64_t o = sa_part_off(a, b, tile, h);
      a.ws[o] = m;
      a.ws[o + 1] = l;
    }
  }
  __syncthreads();
  // Weighted latent sums: thread -> (channel d, half of the keys).
  const int half = tid / 128;
  for (int h = 0; h < H; ++h) {
    for (int d = tid % 128; d < dc; d += 128) {
      float z = 0.f;
      for (int j = half * 32; j < half * 32 + 32; ++j) z = fmaf(s_p[h][j], s_c[j][d], z);
      s_red[half][h][d] = z;
    }
  }
  __syncthreads();
  for (int i = tid; i < H * dc; i += 256) {
    const int h = i / dc, d = i % dc;
    a.ws[sa_part_off(a, b, tile, h) + 2 + d] = s_red[0][h][d] + s_red[1][h][d];
  }
}

// One workgroup per (b, h): merge partials per stream, apply the gate.
__global__ __launch_bounds__(256) void maba_sa_combine_kernel(SaArgs a) {
  const int64_t b = blockIdx.x / a.H;
  const int h = blockIdx.x % a.H;
  const int dc = a.dc;
  // gate softmax
  const int64_t gb = b * a.gsb + h * a.gsh;
  float z0 = load_elem(a.gate, a.gdt, gb), z1 = load_elem(a.gate, a.gdt, gb + a.gsm),
        z2 = load_elem(a.gate, a.gdt, gb + 2 * a.gsm);
  const float gm = fmaxf(z0, fmaxf(z1, z2));
  z0 = __expf(z0 - gm); z1 = __expf(z1 - gm); z2 = __expf(z2 - gm);
  const float gi = 1.f / (z0 + z1 + z2);
  const float g[3] = {z0 * gi, z1 * gi, z2 * gi};
  const int t_begin[3] = {0, a.t_loc, a.t_loc + a.t_sp};
  const int t_end[3] = {a.t_loc, a.t_loc + a.t_sp, a.t_loc + a.t_sp + a.t_hca};
  for (int d = threadIdx.x; d < dc; d += blockDim.x) {
    float res = 0.f;
    for (int st = 0; st < 3; ++st) {
      float zs = 0.f;
      if (st == 2 && a.L - 1 < a.pool - 1) {
        // early HCA: running mean of c[0..L-1] (sparse_attention.py:189-199)
        for (int64_t t = 0; t < a.L; ++t) zs += load_elem(a.c, a.cdt, b * a.csb + t * a.csl + d * a.csd);
        zs /= (float)a.L;
      } else {
        float M = -INFINITY;
        for (int t = t_begin[st]; t < t_end[st]; ++t) M = fmaxf(M, a.ws[sa_part_off(a, b, t, h)]);
        if (M != -INFINITY) {
          float Ls = 0.f, Z = 0.f;
          for (int t = t_begin[st]; t < t_end[st]; ++t) {
            const int64_t o = sa_part_off(a, b, t, h);
            const float m = a.ws[o];
            if (m == -INFINITY) continue;
            const float e = __expf(m - M);
            Ls = fmaf(a.ws[o + 1], e, Ls);
            Z = fmaf(a.ws[o + 2 + d], e, Z);
          }
          zs = Ls > 0.f ? Z / Ls : 0.f;
        }
      }
      res = fmaf(g[st], zs, res);
    }
    a.out[b * a.osb + h * a.osh + d * a.osd] = res;
  }
}

static void sa_geometry(SaArgs& a, int64_t L, int window, int n_sink, int pool, int Hi, int K) {
  const int64_t ns = L < n_sink ? L : n_sink;
  const int64_t st = (L - window) > ns ? (L - window) : ns;
  a.ns = (int)ns;
  a.loc_start = (int)st;
  a.nloc = (int)(ns + (L - st));
  a.nc = (int)(L / pool);
  a.t_loc = (int)ceil_div(a.nloc, 64);
  a.t_sp = Hi * K;
  a.t_hca = (L - 1 >= pool - 1) ? (int)ceil_div(a.nc, 64) : 0;
  a.ntiles = a.t_loc + a.t_sp + a.t_hca;
}

}  // namespace maba

using namespace maba;

extern "C" size_t maba_hip_maba_sa_decode_workspace_size(int64_t B, int64_t H, int64_t dc, int64_t L,
                                                         int64_t K, int window, int n_sink, int pool) {
  SaArgs a;
  sa_geometry(a, L, window, n_sink, pool > 0 ? pool : 64, (int)H, (int)K);  // upper bound: Hi = H
  return (size_t)(B * (int64_t)(a.ntiles > 0 ? a.ntiles : 1) * H * (dc + 2)) * sizeof(float);
}

extern "C" int maba_hip_maba_sa_decode(const maba_tensor* q_lat, const maba_tensor* c_kv,
                                       const maba_tensor* hca, const maba_tensor* idx,
                                       const maba_tensor* gate, int64_t L, float scale, int window,
                                       int n_sink, int block_size, int pool, maba_tensor* out_lat,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  if (!q_lat || q_lat->ndim != 3) return fail(MABA_ERR_INVALID, "maba_sa_decode: q_lat must be [B,H,dc]");
  const int64_t B = q_lat->shape[0], H = q_lat->shape[1], dc = q_lat->shape[2];
  if (!c_kv || c_kv->ndim != 3 || c_kv->shape[0] != B || c_kv->shape[2] != dc)
    return fail(MABA_ERR_INVALID, "maba_sa_decode: c_kv must be [B,Lmax,dc]");
  if (L <= 0 || L > c_kv->shape[1]) return fail(MABA_ERR_INVALID, "maba_sa_decode: L out of range");
  if (window < 0 || n_sink < 0 || block_size <= 0 || pool <= 0)
    return fail(MABA_ERR_INVALID, "maba_sa_decode: bad window/sink/block/pool");
  if (!hca || hca->ndim != 3 || hca->shape[0] != B || hca->shape[2] != dc || hca->shape[1] < L / pool)
    return fail(MABA_ERR_INVALID, "maba_sa_decode: hca must be [B,>=L/pool,dc]");
  if (!idx || idx->ndim != 3 || idx->shape[0] != B || (idx->shape[1] != 1 && idx->shape[1] != H))
    return fail(MABA_ERR_INVALID, "maba_sa_decode: idx must be [B,1|H,K]");
  if (idx->dtype != MABA_I64) return fail(MABA_ERR_DTYPE, "maba_sa_decode: idx must be int64");
  if (!gate || !((gate->ndim == 2 && gate->shape[0] == B && gate->shape[1] == 3) ||
                 (gate->ndim == 3 && gate->shape[0] == B && gate->shape[1] == H && gate->shape[2] == 3)))
    return fail(MABA_ERR_INVALID, "maba_sa_decode: gate must be [B,3] or [B,H,3]");
  const int64_t so[3] = {B, H, dc};
  if (!expect_shape(out_lat, "out_lat", 3, so)) return MABA_ERR_INVALID;
  if (out_lat->dtype != MABA_F32) return fail(MABA_ERR_DTYPE, "maba_sa_decode: out_lat must be f32");
  const maba_tensor* fl[] = {q_lat, c_kv, hca, gate};
  for (const maba_tensor* t : fl)
    if (!expect_float(t, "maba_sa_decode")) return MABA_ERR_DTYPE;
  if (H > SA_MAXH || dc > SA_MAXDC || block_size > 64)
    return fail(MABA_ERR_UNSUPPORTED, "maba_sa_decode: H <= %d, dc <= %d, block_size <= 64 required",
                SA_MAXH, SA_MAXDC);
  if (B * H == 0) return MABA_OK;
  SaArgs a;
  a.q = q_lat->data; a.qdt = q_lat->dtype; a.qsb = q_lat->stride[0]; a.qsh = q_lat->stride[1]; a.qsd = q_lat->stride[2];
  a.c = c_kv->data; a.cdt = c_kv->dtype; a.csb = c_kv->stride[0]; a.csl = c_kv->stride[1]; a.csd = c_kv->stride[2];
  a.hca = hca->data; a.hdt = hca->dtype; a.hsb = hca->stride[0]; a.hsn = hca->stride[1]; a.hsd = hca->stride[2];
  a.idx = (const int64_t*)idx->data; a.isb = idx->stride[0]; a.ish = idx->stride[1]; a.isk = idx->stride[2];
  a.gate = gate->data; a.gdt = gate->dtype; a.gsb = gate->stride[0];
  if (gate->ndim == 2) { a.gsh = 0; a.gsm = gate->stride[1]; } else { a.gsh = gate->stride[1]; a.gsm = gate->stride[2]; }
  a.out = (float*)out_lat->data; a.osb = out_lat->stride[0]; a.osh = out_lat->stride[1]; a.osd = out_lat->stride[2];
  a.ws = (float*)workspace;
  a.L = L; a.H = (int)H; a.dc = (int)dc; a.Hi = (int)idx->shape[1]; a.K = (int)idx->shape[2];
  a.window = window; a.n_sink = n_sink; a.bs = block_size; a.pool = pool; a.scale = scale;
  sa_geometry(a, L, window, n_sink, pool, a.Hi, a.K);
  const size_t need = (size_t)(B * (int64_t)(a.ntiles > 0 ? a.ntiles : 1) * H * (dc + 2)) * sizeof(float);
  if (!workspace || workspace_bytes < need)
    return fail(MABA_ERR_WORKSPACE, "maba_sa_decode: workspace of %zu bytes required", need);
  hipStream_t s = (hipStream_t)stream;
  if (a.ntiles > 0) {
    hipLaunchKernelGGL(maba_sa_tile_kernel, dim3((unsigned)a.ntiles, (unsigned)B), dim3(256), 0, s, a);
    int rc = check_launch("maba_sa_decode/tiles");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(maba_sa_combine_kernel, dim3((unsigned)(B * H)), dim3(128), 0, s, a);
  return check_launch("maba_sa_decode/combine");
}

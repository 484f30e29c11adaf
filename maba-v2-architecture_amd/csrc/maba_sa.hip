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
#include <algorithm>

#include "maba_common.h"

namespace maba {

constexpr int SA_MAXH = 16;
constexpr int SA_MAXDC = 256;

struct SaArgs {
  const void* q; int qdt; int64_t qsb, qsh, qsd;
  int qvec;  // q is fp32 with unit channel stride and 16-byte aligned rows
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

// One workgroup per (b, h): merge the partials of each stream, apply the gate.
// Partials [0, p1) are the local stream, [p1, p2) sparse, [p2, p3) HCA.  Waves
// 0-2 reduce the (max, sum) pairs of one stream each; then, in chunks of 256
// partials, every partial's weight g_s exp(m - M_s) / L_s goes to LDS and the
// threads (dim d, sub-slice) accumulate the weighted latent sums.
__global__ __launch_bounds__(256) void maba_sa_combine_kernel(SaArgs a, int p1, int p2, int p3) {
  __shared__ float s_w[256];
  __shared__ float s_M[3], s_S[3];
  __shared__ float s_acc[256];
  const int64_t b = blockIdx.x / a.H;
  const int h = blockIdx.x % a.H;
  const int dc = a.dc;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t gb = b * a.gsb + h * a.gsh;
  float z0 = load_elem(a.gate, a.gdt, gb), z1 = load_elem(a.gate, a.gdt, gb + a.gsm),
        z2 = load_elem(a.gate, a.gdt, gb + 2 * a.gsm);
  const float gm = fmaxf(z0, fmaxf(z1, z2));
  z0 = __expf(z0 - gm); z1 = __expf(z1 - gm); z2 = __expf(z2 - gm);
  const float gi = 1.f / (z0 + z1 + z2);
  const float gate[3] = {z0 * gi, z1 * gi, z2 * gi};
  const int t_begin[3] = {0, p1, p2};
  const int t_end[3] = {p1, p2, p3};
  // partial headers of the first chunk, loaded alongside the stream reductions
  float m_first = -INFINITY;
  if (tid < p3) m_first = a.ws[sa_part_off(a, b, tid, h)];
  if (wave < 3) {  // online (max, sum) over the stream's partials, one pass
    float M = -INFINITY, S = 0.f;
    for (int t = t_begin[wave] + lane; t < t_end[wave]; t += 64) {
      const int64_t o = sa_part_off(a, b, t, h);
      const float m = a.ws[o], l = a.ws[o + 1];
      if (m != -INFINITY) {
        if (m > M) {
          S = S * __expf(M - m) + l;
          M = m;
        } else {
          S = fmaf(l, __expf(m - M), S);
        }
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float M2 = __shfl_xor(M, o), S2 = __shfl_xor(S, o);
      const float Mn = fmaxf(M, M2);
      S = (M == -INFINITY ? 0.f : S * __expf(M - Mn)) + (M2 == -INFINITY ? 0.f : S2 * __expf(M2 - Mn));
      M = Mn;
    }
    if (lane == 0) {
      s_M[wave] = M;
      s_S[wave] = S;
    }
  }
  __syncthreads();
  const int nsub = 256 / dc;  // threads per latent dim
  const int d = tid % dc, sub = tid / dc;
  const bool active = sub < nsub;
  float acc = 0.f;
  for (int c0 = 0; c0 < p3; c0 += 256) {
    const int t = c0 + tid;
    float w = 0.f;
    if (t < p3) {
      const int st = t < p1 ? 0 : (t < p2 ? 1 : 2);
      const float m = c0 == 0 ? m_first : a.ws[sa_part_off(a, b, t, h)];
      if (m != -INFINITY && s_S[st] > 0.f) w = gate[st] * __expf(m - s_M[st]) / s_S[st];
    }
    s_w[tid] = w;
    __syncthreads();
    const int cn = (p3 - c0) < 256 ? (p3 - c0) : 256;
    // every partial slot is written by the segment kernel, so the loads need no guard
    if (active) {
#pragma unroll 8
      for (int j = sub; j < cn; j += nsub) acc = fmaf(s_w[j], a.ws[sa_part_off(a, b, c0 + j, h) + 2 + d], acc);
    }
    __syncthreads();
  }
  s_acc[tid] = active ? acc : 0.f;
  __syncthreads();
  if (tid < dc) {
    float r = 0.f;
    for (int k = 0; k < nsub; ++k) r += s_acc[k * dc + tid];
    if (a.L - 1 < a.pool - 1) {
      // early HCA: running mean of c[0..L-1] (sparse_attention.py:189-199)
      float zs = 0.f;
      for (int64_t t = 0; t < a.L; ++t) zs += load_elem(a.c, a.cdt, b * a.csb + t * a.csl + tid * a.csd);
      r = fmaf(gate[2], zs / (float)a.L, r);
    }
    a.out[b * a.osb + h * a.osh + tid * a.osd] = r;
  }
}

// ------------------------------------------------------------------ MFMA path
// Used when c_kv / hca are bf16 rows with unit channel stride, d_c <= 128 (a
// multiple of 32) and H <= 16.  Every stream of every batch element is cut into
// segments of up to 4 * tpw 64-key tiles, one workgroup per segment.  Each wave
// runs tpw consecutive tiles with an online softmax, loading tile t+1 into
// registers while it computes tile t; the four wave partials are merged in LDS
// and the workgroup writes one partial (max, sum, weighted latent sum) per head.
//   scores  D[key][head] = C Q^T   (A: key rows straight from global memory,
//                                   B: the queries, bf16 hi + lo, in registers)
//   values  Z[dim][head] += C^T P  (A: C^T fragments read with ds_read_b64_tr_b16
//                                   from the tile kept row-major in per-wave LDS,
//                                   B: the probabilities, bf16 hi + lo, used in
//                                   place from the score accumulators)
typedef __attribute__((ext_vector_type(8))) short s16x8;
typedef __attribute__((ext_vector_type(4))) short s16x4;

// Transposed read: within each 16-lane group, lane i receives src[4r + i/4][i%4]
// (r = 0..3) where src[j] are the four bf16 at lane j's address.  Lane j of group g
// addressing row r0 + 4g + j/4, column c0 + 4(j%4) of a row-major tile gets the
// column fragment tile[r0 + 4g + r][c0 + c16], r = 0..3.
__device__ __forceinline__ s16x4 sa_ldsT4(const short* tile, int pitch, int r0, int c0, int c16, int g) {
  const short* p = tile + (r0 + 4 * g + (c16 >> 2)) * pitch + c0 + 4 * (c16 & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
}

struct SaSeg {
  int stream, head_only;
  int64_t t_begin, t_end;  // tile range within the stream (sparse: index slots)
  int hs;                  // sparse index row
};

__device__ __forceinline__ SaSeg sa_segment(const SaArgs& a, int sid, int s_sp1, int span) {
  SaSeg g;
  g.head_only = -1;
  g.hs = 0;
  const int s_sp = (a.Hi == 1) ? s_sp1 : a.H * s_sp1;
  if (sid == 0) {
    g.stream = 0; g.t_begin = 0; g.t_end = a.t_loc;
  } else if (sid < 1 + s_sp) {
    const int r = sid - 1;
    g.stream = 1;
    g.hs = (a.Hi == 1) ? 0 : r / s_sp1;
    const int rr = (a.Hi == 1) ? r : r % s_sp1;
    if (a.Hi > 1) g.head_only = g.hs;
    g.t_begin = (int64_t)rr * span;
    g.t_end = min((int64_t)a.K, g.t_begin + span);
  } else {
    const int r = sid - 1 - s_sp;
    g.stream = 2;
    g.t_begin = (int64_t)r * span;
    g.t_end = min((int64_t)a.t_hca, g.t_begin + span);
  }
  return g;
}

// Key rows 16 rb + c16 of tile tix of a segment, dims 32 p + 8 g .. +7; invalid rows read as zeros.
// blk is the tile's block index for the sparse stream.
template <int NP>
__device__ __forceinline__ void sa_load_tile(const SaArgs& a, const SaSeg& sg, int64_t b, int64_t tix, int64_t blk,
                                             int c16, int g, s16x8 (&cv)[4][NP], bool (&ok)[4]) {
  const uint16_t* base;
  int64_t rstride;
  if (sg.stream == 2) {
    base = (const uint16_t*)a.hca + b * a.hsb;
    rstride = a.hsn;
  } else {
    base = (const uint16_t*)a.c + b * a.csb;
    rstride = a.csl;
  }
  const int64_t nblk = (a.L + a.bs - 1) / a.bs;
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int j = 16 * rb + c16;
    int64_t pos;
    if (sg.stream == 0) {
      const int64_t li = tix * 64 + j;
      ok[rb] = li < a.nloc;
      pos = li < a.ns ? li : a.loc_start + (li - a.ns);
    } else if (sg.stream == 1) {
      pos = blk * a.bs + j;
      ok[rb] = blk >= 0 && blk < nblk && j < a.bs && pos < a.L;
    } else {
      pos = tix * 64 + j;
      ok[rb] = pos < a.nc;
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      s16x8 v = {0, 0, 0, 0, 0, 0, 0, 0};
      if (ok[rb]) v = *(const s16x8*)(base + pos * rstride + 32 * p + 8 * g);
      cv[rb][p] = v;
    }
  }
}

template <int NP>  // d_c = 32 * NP
__global__ __launch_bounds__(256, 2) void maba_sa_mfma_kernel(SaArgs a, int nseg, int s_sp1, int tpw) {
  constexpr int DC = 32 * NP;
  constexpr int TP = DC + 8;  // row pitch (bf16) of the per-wave key tile: 16-B aligned, rows shift 4 banks
  __shared__ __attribute__((aligned(16))) short s_tile[4][64 * TP];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int sid = blockIdx.x;
  const int64_t b = blockIdx.y;
  if (sid >= nseg) return;  // uniform per workgroup
  const SaSeg sg = sa_segment(a, sid, s_sp1, 4 * tpw);
  const int64_t t0 = sg.t_begin + (int64_t)wave * tpw;
  const int64_t t1 = min(sg.t_end, t0 + tpw);
  short* tile = s_tile[wave];

  // queries (B operand of the scores): head c16, dims 32p + 8g .. +7, split hi/lo
  s16x8 qh[NP], ql[NP];
  float qv[NP][8];
  if (a.qvec) {  // fp32 rows, 16-byte aligned: all of the lane's query loads in flight at once
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      f32x4 x0 = {0.f, 0.f, 0.f, 0.f}, x1 = {0.f, 0.f, 0.f, 0.f};
      if (c16 < a.H) {
        const float* qp = (const float*)a.q + b * a.qsb + c16 * a.qsh + 32 * p + 8 * g;
        x0 = *(const f32x4*)qp;
        x1 = *(const f32x4*)(qp + 4);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        qv[p][j] = x0[j];
        qv[p][4 + j] = x1[j];
      }
    }
  } else {
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        qv[p][j] = (c16 < a.H) ? load_elem(a.q, a.qdt, b * a.qsb + c16 * a.qsh + (32 * p + 8 * g + j) * a.qsd) : 0.f;
  }
#pragma unroll
  for (int p = 0; p < NP; ++p) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = qv[p][j];
      const short h = __builtin_bit_cast(short, (__bf16)x);
      qh[p][j] = h;
      ql[p][j] = __builtin_bit_cast(short, (__bf16)(x - bf16_bits_to_f32((uint16_t)h)));
    }
  }
  const bool head_on = c16 < a.H && (sg.head_only < 0 || sg.head_only == c16);
  float m_run = -INFINITY, l_run = 0.f;
  f32x4 z[DC / 16];
#pragma unroll
  for (int dt = 0; dt < DC / 16; ++dt) z[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // sparse block indices of this wave's tiles, one per lane, fetched up front so that
  // the tile loads do not wait on a dependent index load
  int64_t blk_l = 0;
  if (sg.stream == 1 && lane < t1 - t0) blk_l = a.idx[b * a.isb + sg.hs * a.ish + (t0 + lane) * a.isk];
  s16x8 cv[4][NP];
  bool ok[4];
  if (t0 < t1) sa_load_tile<NP>(a, sg, b, t0, __shfl(blk_l, 0), c16, g, cv, ok);
  for (int64_t tix = t0; tix < t1; ++tix) {
    // prefetch the next tile (the current one is re-read when there is none: in bounds, unused)
    s16x8 nv[4][NP];
    bool nok[4];
    const int64_t tn = tix + 1 < t1 ? tix + 1 : tix;
    sa_load_tile<NP>(a, sg, b, tn, __shfl(blk_l, (int)(tn - t0)), c16, g, nv, nok);
    f32x4 sc[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        // row-major copy for the value product (read back transposed)
        *(s16x8*)(tile + (16 * rb + c16) * TP + 32 * p + 8 * g) = cv[rb][p];
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, cv[rb][p]),
                                                      __builtin_bit_cast(bf16x8, qh[p]), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, cv[rb][p]),
                                                      __builtin_bit_cast(bf16x8, ql[p]), acc, 0, 0, 0);
      }
      sc[rb] = acc;
    }
    // lane (head c16, group g) holds scores of keys 16 rb + 4g + i
    float tmax = -INFINITY;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // key row 16 rb + 4g + i is valid iff the loading lane c16' = 4g + i had ok[rb]
        const bool kv = __shfl(ok[rb] ? 1 : 0, 4 * g + i) != 0;
        const float x = (kv && head_on) ? sc[rb][i] * a.scale : -INFINITY;
        sc[rb][i] = x;
        tmax = fmaxf(tmax, x);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const float corr = (m_new == -INFINITY) ? 1.f : __expf(m_run - m_new);
    float psum = 0.f;
    s16x4 ph[4], pl[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      f32x4 pv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pe = (sc[rb][i] == -INFINITY) ? 0.f : __expf(sc[rb][i] - m_new);
        pv[i] = pe;
        psum += pe;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const short h = __builtin_bit_cast(short, (__bf16)pv[i]);
        ph[rb][i] = h;
        pl[rb][i] = __builtin_bit_cast(short, (__bf16)(pv[i] - bf16_bits_to_f32((uint16_t)h)));
      }
    }
    psum += __shfl_xor(psum, 16);
    psum += __shfl_xor(psum, 32);
    l_run = l_run * corr + psum;
    m_run = m_new;
    // z[dim][head] = corr * z + C^T P  (K = 64 keys as two permuted 32-steps)
#pragma unroll
    for (int dt = 0; dt < DC / 16; ++dt) {
      f32x4 acc = z[dt] * corr;
#pragma unroll
      for (int p2 = 0; p2 < 2; ++p2) {
        const s16x4 a0 = sa_ldsT4(tile, TP, 32 * p2, 16 * dt, c16, g);
        const s16x4 a1 = sa_ldsT4(tile, TP, 32 * p2 + 16, 16 * dt, c16, g);
        const s16x8 av = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        const s16x8 bh = {ph[2 * p2][0], ph[2 * p2][1], ph[2 * p2][2], ph[2 * p2][3],
                          ph[2 * p2 + 1][0], ph[2 * p2 + 1][1], ph[2 * p2 + 1][2], ph[2 * p2 + 1][3]};
        const s16x8 bl = {pl[2 * p2][0], pl[2 * p2][1], pl[2 * p2][2], pl[2 * p2][3],
                          pl[2 * p2 + 1][0], pl[2 * p2 + 1][1], pl[2 * p2 + 1][2], pl[2 * p2 + 1][3]};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bh),
                                                      acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bl),
                                                      acc, 0, 0, 0);
      }
      z[dt] = acc;
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      ok[rb] = nok[rb];
#pragma unroll
      for (int p = 0; p < NP; ++p) cv[rb][p] = nv[rb][p];
    }
  }
  // merge the four wave partials: s_z[wave][head][dim], s_m / s_l[wave][head]
  __syncthreads();
  float* s_z = (float*)&s_tile[0][0];
  float* s_m = s_z + 4 * 16 * DC;
  float* s_l = s_m + 64;
#pragma unroll
  for (int dt = 0; dt < DC / 16; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_z[(wave * 16 + c16) * DC + 16 * dt + 4 * g + i] = z[dt][i];
  if (g == 0) {
    s_m[wave * 16 + c16] = m_run;
    s_l[wave * 16 + c16] = l_run;
  }
  __syncthreads();
  const int h = threadIdx.x >> 4, part = threadIdx.x & 15;  // 16 threads per head
  if (h < a.H) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, s_m[w * 16 + h]);
    float e[4], Ls = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float m = s_m[w * 16 + h];
      e[w] = (m == -INFINITY) ? 0.f : __expf(m - M);
      Ls = fmaf(e[w], s_l[w * 16 + h], Ls);
    }
    const int64_t o = (((b * a.ntiles) + sid) * a.H + h) * (int64_t)(a.dc + 2);
    if (part == 0) {
      a.ws[o] = M;
      a.ws[o + 1] = Ls;
    }
#pragma unroll
    for (int j = 0; j < DC / 16; ++j) {
      const int dd = part * (DC / 16) + j;
      float zz = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) zz = fmaf(e[w], s_z[(w * 16 + h) * DC + dd], zz);
      a.ws[o + 2 + dd] = zz;
    }
  }
}

// Compute units of the current device (queried once per device).
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
  a.qvec = q_lat->dtype == MABA_F32 && q_lat->stride[2] == 1 && (uintptr_t)q_lat->data % 16 == 0 &&
           q_lat->stride[0] % 4 == 0 && q_lat->stride[1] % 4 == 0;
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
  const bool mfma_ok = c_kv->dtype == MABA_BF16 && hca->dtype == MABA_BF16 && c_kv->stride[2] == 1 &&
                       hca->stride[2] == 1 && dc % 32 == 0 && dc <= 128 && (uintptr_t)c_kv->data % 16 == 0 &&
                       (uintptr_t)hca->data % 16 == 0 && c_kv->stride[0] % 8 == 0 && c_kv->stride[1] % 8 == 0 &&
                       hca->stride[0] % 8 == 0 && hca->stride[1] % 8 == 0 && block_size <= 64;
  if (mfma_ok) {
    // tiles per wave: the fewest that still fit one workgroup per CU (every workgroup
    // pays a fixed start-up, and one round of workgroups covers the machine), at most 8
    const int ncu = device_cu_count();
    int tpw = 1, span = 4, s_sp1 = 0, s_sp = 0, s_hca = 0, nseg = 0;
    for (tpw = 1; tpw <= 8; ++tpw) {
      span = 4 * tpw;
      s_sp1 = (int)ceil_div(a.K, span);
      s_sp = a.Hi == 1 ? s_sp1 : (int)H * s_sp1;
      s_hca = (int)ceil_div(a.t_hca, span);
      nseg = 1 + s_sp + s_hca;
      if (B * nseg <= ncu || tpw == 8) break;
    }
    a.ntiles = nseg;  // partial slots are segments
    const dim3 grid((unsigned)nseg, (unsigned)B);
    switch (dc / 32) {
      case 1: hipLaunchKernelGGL(maba_sa_mfma_kernel<1>, grid, dim3(256), 0, s, a, nseg, s_sp1, tpw); break;
      case 2: hipLaunchKernelGGL(maba_sa_mfma_kernel<2>, grid, dim3(256), 0, s, a, nseg, s_sp1, tpw); break;
      case 3: hipLaunchKernelGGL(maba_sa_mfma_kernel<3>, grid, dim3(256), 0, s, a, nseg, s_sp1, tpw); break;
      default: hipLaunchKernelGGL(maba_sa_mfma_kernel<4>, grid, dim3(256), 0, s, a, nseg, s_sp1, tpw); break;
    }
    int rc = check_launch("maba_sa_decode/segments");
    if (rc) return rc;
    hipLaunchKernelGGL(maba_sa_combine_kernel, dim3((unsigned)(B * H)), dim3(256), 0, s, a, 1, 1 + s_sp, nseg);
    return check_launch("maba_sa_decode/combine");
  }
  if (a.ntiles > 0) {
    hipLaunchKernelGGL(maba_sa_tile_kernel, dim3((unsigned)a.ntiles, (unsigned)B), dim3(256), 0, s, a);
    int rc = check_launch("maba_sa_decode/tiles");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(maba_sa_combine_kernel, dim3((unsigned)(B * H)), dim3(256), 0, s, a, a.t_loc,
                     a.t_loc + a.t_sp, a.t_loc + a.t_sp + a.t_hca);
  return check_launch("maba_sa_decode/combine");
}

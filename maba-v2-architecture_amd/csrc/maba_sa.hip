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
// Each stream of each batch element is cut into segments; a workgroup writes one
// flash-decoding partial (max, sum, weighted latent sum) per head for its segment,
// and a merge of the partials of each (b, h) applies the gate softmax and writes z.
// Traffic is one read of the selected latent rows (bf16) plus small partials:
// HBM-bound.
#include <algorithm>
#include <mutex>

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
  float* ws;    // partials, slot-major: [slot][b][h][dc + 2]
  int64_t L, B;
  int H, dc, Hi, K, window, n_sink, bs, pool;
  int ns, loc_start, nloc, nc;           // local / hca geometry
  int t_loc, t_sp, t_hca, ntiles;        // tile counts per batch element
  // segment path: tiles per wave and the segment counts; partial slots [0, s_loc)
  // local, [s_loc, s_loc + s_hca) HCA, then the sparse ones (s_sp1 per index row)
  int tpw, s_loc, s_hca, s_sp1, s_sp;
  float scale;
  const int64_t* dlen;   // device sequence length (null: L as given); the geometry above is then re-derived
  // value up-projection in the merge (wv null: not applied): oh[b, h dh + d] = bf16(sum_c W_v[h dh + d, c] z[b, h, c])
  const uint16_t* wv; int64_t wvs;    // W_v [H * dh, dc] bf16, unit column stride
  uint16_t* oh; int64_t ohsb, ohsd;   // [B, H * dh] bf16
  int dh;
};

// Tile geometry of the three streams (per batch element).
__host__ __device__ inline void sa_geometry(SaArgs& a, int64_t L, int window, int n_sink, int pool, int Hi, int K) {
  const int64_t ns = L < n_sink ? L : n_sink;
  const int64_t st = (L - window) > ns ? (L - window) : ns;
  a.ns = (int)ns;
  a.loc_start = (int)st;
  a.nloc = (int)(ns + (L - st));
  a.nc = (int)(L / pool);
  a.t_loc = (int)((a.nloc + 63) / 64);
  a.t_sp = Hi * K;
  a.t_hca = (L - 1 >= pool - 1) ? (int)((a.nc + 63) / 64) : 0;
  a.ntiles = a.t_loc + a.t_sp + a.t_hca;
}

// The arguments of a launch with a device-resident sequence length: the stream geometry
// of the current length (the partial-slot layout stays that of the capacity the host
// planned for, so slots past the current length hold empty partials).
__device__ __forceinline__ SaArgs sa_live(const SaArgs& in) {
  SaArgs a = in;
  if (a.dlen) {   // a.L holds the capacity the buffers were checked against
    const int64_t L = *a.dlen;
    a.L = L < 1 ? 1 : (L < a.L ? L : a.L);
    sa_geometry(a, a.L, a.window, a.n_sink, a.pool, a.Hi, a.K);
  }
  return a;
}

__device__ __forceinline__ int64_t sa_part_off(const SaArgs& a, int64_t b, int slot, int h) {
  return (((int64_t)slot * a.B + b) * a.H + h) * (int64_t)(a.dc + 2);
}

// Partials merged for one (b, h): n virtual partials t = 0 .. n-1 at slots t (t < na)
// and sp0 + sp_step * h + (t - na) (t >= na).  Virtual partials [0, e1) belong to stream
// st0, [e1, e2) to st1 and [e2, n) to st2 (streams: 0 local, 1 sparse, 2 HCA).
struct SaMerge {
  int n, na, sp0, sp_step, e1, e2, st0, st1, st2;
};

// Generic path: one workgroup per 64-key tile, one partial slot per tile.
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

// Merge of the n virtual partials of (b, h) (streams as in SaMerge), NT threads.
// src.m(t), src.l(t) and src.z(t, d) read partial t's max, sum and latent sum.
// Thread (dim d, sub-slice) issues the loads of its latent sums of the first SA_PRE
// partials together with the partial headers, so that the merge waits on one round of
// loads; waves 0-2 then reduce the (max, sum) pairs of one stream each, every
// partial's weight g_s exp(m - M_s) / L_s goes to LDS and the threads accumulate their
// weighted sums.  lds holds at least 2 NT + 8 floats.
constexpr int SA_PRE = 16;   // partials per thread whose latent sums are loaded up front
template <int NT, class Src>
__device__ void sa_merge(const SaArgs& a, const SaMerge& mg, int64_t b, int h, float* lds, const Src& src,
                         float* zkeep = nullptr) {
  float* s_w = lds;
  float* s_acc = lds + NT;
  float* s_M = lds + 2 * NT;
  float* s_S = lds + 2 * NT + 4;
  const int dc = a.dc;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n = mg.n;
  const int nsub = NT / dc;  // threads per latent dim
  const int d = tid % dc, sub = tid / dc;
  const bool active = sub < nsub;
  float zpre[SA_PRE];
#pragma unroll
  for (int i = 0; i < SA_PRE; ++i) {
    const int t = sub + i * nsub;
    zpre[i] = (active && t < n) ? src.z(t, d) : 0.f;
  }
  const float m_first = tid < n ? src.m(tid) : -INFINITY;
  const int64_t gb = b * a.gsb + h * a.gsh;
  float z0 = load_elem(a.gate, a.gdt, gb), z1 = load_elem(a.gate, a.gdt, gb + a.gsm),
        z2 = load_elem(a.gate, a.gdt, gb + 2 * a.gsm);
  if (wave < 3) {  // online (max, sum) over one stream's partials, one pass
    const int t0 = wave == 0 ? 0 : (wave == 1 ? mg.e1 : mg.e2);
    const int t1 = wave == 0 ? mg.e1 : (wave == 1 ? mg.e2 : n);
    float M = -INFINITY, S = 0.f;
    for (int t = t0 + lane; t < t1; t += 64) {
      const float m = src.m(t), l = src.l(t);
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
  const float gm = fmaxf(z0, fmaxf(z1, z2));
  z0 = __expf(z0 - gm); z1 = __expf(z1 - gm); z2 = __expf(z2 - gm);
  const float gi = 1.f / (z0 + z1 + z2);
  auto gate_of = [&](int st) { return (st == 0 ? z0 : (st == 1 ? z1 : z2)) * gi; };
  const float g0 = gate_of(mg.st0), g1 = gate_of(mg.st1), g2 = gate_of(mg.st2);
  __syncthreads();
  float acc = 0.f;
  for (int c0 = 0; c0 < n; c0 += NT) {
    const int t = c0 + tid;
    float w = 0.f;
    if (t < n) {
      const int k = t < mg.e1 ? 0 : (t < mg.e2 ? 1 : 2);
      const float m = c0 == 0 ? m_first : src.m(t);
      const float Sk = s_S[k];
      if (m != -INFINITY && Sk > 0.f) w = (k == 0 ? g0 : (k == 1 ? g1 : g2)) * __expf(m - s_M[k]) / Sk;
    }
    s_w[tid] = w;
    __syncthreads();
    const int cn = (n - c0) < NT ? (n - c0) : NT;
    if (active) {
      int j = sub;
      if (c0 == 0) {
#pragma unroll
        for (int i = 0; i < SA_PRE; ++i)
          if (sub + i * nsub < cn) acc = fmaf(s_w[sub + i * nsub], zpre[i], acc);
        j = sub + SA_PRE * nsub;
      }
#pragma unroll 4
      for (; j < cn; j += nsub) acc = fmaf(s_w[j], src.z(c0 + j, d), acc);
    }
    __syncthreads();
  }
  s_acc[tid] = active ? acc : 0.f;
  __syncthreads();
  if (tid < dc) {
    float res = 0.f;
    for (int k = 0; k < nsub; ++k) res += s_acc[k * dc + tid];
    if (a.L - 1 < a.pool - 1) {
      // early HCA: running mean of c[0..L-1] (sparse_attention.py:189-199)
      float zs = 0.f;
      for (int64_t t = 0; t < a.L; ++t) zs += load_elem(a.c, a.cdt, b * a.csb + t * a.csl + tid * a.csd);
      res = fmaf(gate_of(2), zs / (float)a.L, res);
    }
    a.out[b * a.osb + h * a.osh + tid * a.osd] = res;
    if (zkeep) zkeep[tid] = res;
  }
}

// o[b, h dh + d] = bf16(sum_c W_v[h dh + d, c] z[c]) for the merged z of (b, h) in LDS (the
// caller's sa_merge left it in zk): four threads per output, eight bf16 weights per load,
// the four partial sums added by shuffles (layers/sparse_attention.py:208, absorbed:
// sum_j p_j W_v,h c_j = W_v,h z_h).
template <int NT>
__device__ __forceinline__ void sa_value_up(const SaArgs& a, int64_t b, int h, const float* zk) {
  const int tid = threadIdx.x;
  const int d = tid >> 2, part = tid & 3;
  const int per = a.dc / 4;   // a multiple of 8 (dc a multiple of 32)
  float acc = 0.f;
  if (d < a.dh) {
    const uint16_t* w = a.wv + ((int64_t)h * a.dh + d) * a.wvs + part * per;
    for (int c = 0; c < per; c += 8) {
      const i16x4 lo4 = *(const i16x4*)(w + c), hi4 = *(const i16x4*)(w + c + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = fmaf(bf16_bits_to_f32((uint16_t)lo4[j]), zk[part * per + c + j], acc);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc = fmaf(bf16_bits_to_f32((uint16_t)hi4[j]), zk[part * per + c + 4 + j], acc);
    }
  }
  acc += __shfl_xor(acc, 1);
  acc += __shfl_xor(acc, 2);
  if (d < a.dh && part == 0) a.oh[b * a.ohsb + ((int64_t)h * a.dh + d) * a.ohsd] = f32_to_bf16_bits(acc);
}

// Partials of (b, h) in the workspace: virtual partial t at slot t (t < na), else at
// slot sp0 + sp_step * h + (t - na).  Every slot read is written by a segment kernel.
struct SaWsSrc {
  const float* base;   // partial (slot 0, b, h)
  int64_t row;         // floats per slot
  int na, spb;
  __device__ const float* p(int t) const { return base + (int64_t)(t < na ? t : spb + t) * row; }
  __device__ float m(int t) const { return p(t)[0]; }
  __device__ float l(int t) const { return p(t)[1]; }
  __device__ float z(int t, int d) const { return p(t)[2 + d]; }
};

__device__ __forceinline__ SaWsSrc sa_ws_src(const SaArgs& a, const SaMerge& mg, int64_t b, int h) {
  SaWsSrc s;
  s.base = a.ws + (b * a.H + h) * (int64_t)(a.dc + 2);
  s.row = (int64_t)a.B * a.H * (a.dc + 2);
  s.na = mg.na;
  s.spb = mg.sp0 + mg.sp_step * h - mg.na;
  return s;
}

// One workgroup per (b, h) over the per-tile partials of the generic path.
__global__ __launch_bounds__(256) void maba_sa_combine_kernel(SaArgs a_in, SaMerge mg) {
  __shared__ float lds[2 * 256 + 8];
  __shared__ float zk[SA_MAXDC];
  const SaArgs a = sa_live(a_in);
  const int64_t b = blockIdx.x / a.H;
  const int h = blockIdx.x % a.H;
  sa_merge<256>(a, mg, b, h, lds, sa_ws_src(a, mg, b, h), a.wv ? zk : nullptr);
  if (a.wv) {
    __syncthreads();
    sa_value_up<256>(a, b, h, zk);
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

// Segment of partial slot sid (segment path): up to 4 tpw tiles (sparse: index slots
// of one index row).
__device__ __forceinline__ SaSeg sa_segment(const SaArgs& a, int sid) {
  SaSeg g;
  g.head_only = -1;
  g.hs = 0;
  const int span = 4 * a.tpw;
  if (sid < a.s_loc) {
    g.stream = 0;
    g.t_begin = (int64_t)sid * span;
    g.t_end = min((int64_t)a.t_loc, g.t_begin + span);
  } else if (sid < a.s_loc + a.s_hca) {
    g.stream = 2;
    g.t_begin = (int64_t)(sid - a.s_loc) * span;
    g.t_end = min((int64_t)a.t_hca, g.t_begin + span);
  } else {
    const int r = sid - a.s_loc - a.s_hca;
    g.stream = 1;
    g.hs = (a.Hi == 1) ? 0 : r / a.s_sp1;
    const int rr = (a.Hi == 1) ? r : r % a.s_sp1;
    if (a.Hi > 1) g.head_only = g.hs;
    g.t_begin = (int64_t)rr * span;
    g.t_end = min((int64_t)a.K, g.t_begin + span);
  }
  return g;
}

// Where the key rows of the three streams of one query live: the latent rows c[0, L) and the
// complete-block means hca[0, nc), with the local stream's geometry.
struct SaRows {
  const uint16_t* c; int64_t cs;     // latent rows of the sequence, row stride (unit channel stride)
  const uint16_t* hca; int64_t hs;   // block means of the sequence
  int64_t L, nblk;                   // nblk = ceil(L / bs), formed once per workgroup
  int bs, ns, loc_start, nloc, nc;
};

__device__ __forceinline__ SaRows sa_rows(const SaArgs& a, int64_t b) {
  SaRows r;
  r.c = (const uint16_t*)a.c + b * a.csb; r.cs = a.csl;
  r.hca = (const uint16_t*)a.hca + b * a.hsb; r.hs = a.hsn;
  r.L = a.L; r.bs = a.bs; r.ns = a.ns; r.loc_start = a.loc_start; r.nloc = a.nloc; r.nc = a.nc;
  r.nblk = (a.L + a.bs - 1) / a.bs;
  return r;
}

// Key rows 16 rb + c16 (rb < RB: tiles of 16 RB keys) of tile tix of a stream (0 local,
// 1 sparse, 2 HCA; wave-uniform), dims 32 p + 8 g .. +7, without branches: a tile's first
// row and the row limits are uniform, and a local row past the sinks shifts to the window.
// A sparse block spans ceil(block_size / (16 RB)) tiles: tile tix is part tix % that of
// its block.  Invalid rows read row 0 of
// the stream (in bounds: L >= 1, and the HCA stream is only walked when it has entries);
// their scores are masked to -inf, so they get zero weight.  blk is the tile's block index
// for the sparse stream.  Bit 4 rb + i of okb says whether key row 16 rb + 4 g + i (a row of
// this lane's score accumulators) is valid.  Row offsets are 32-bit (the hosts check that a
// sequence's rows span fewer than 2^31 elements).
template <int NP, int RB = 4>
__device__ __forceinline__ void sa_load_rows(const SaRows& r, int stream, int64_t tix, int64_t blk, int c16, int g,
                                             s16x8 (&cv)[RB][NP], uint32_t& okb) {
  constexpr int TK = 16 * RB;
  const uint16_t* base = stream == 2 ? r.hca : r.c;
  const int rstride = (int)(stream == 2 ? r.hs : r.cs);
  const bool blk_ok = blk >= 0 && blk < r.nblk;
  int part = 0;   // the tile's part of its sparse block (block_size <= 64: one part of a 64-key tile)
  if constexpr (RB < 4) part = (int)(tix % ((r.bs + TK - 1) / TK));
  const int first = (int)(stream == 1 ? (blk_ok ? blk * r.bs + part * TK : 0) : tix * TK);
  // rows [first, lim) are valid; local rows at or past the sinks move by `shift`
  const int lim = stream == 0 ? r.nloc : stream == 2 ? r.nc : (blk_ok ? (int)min(r.L, (int64_t)first + r.bs) : 0);
  const int thr = stream == 0 ? r.ns : INT32_MAX;
  const int shift = stream == 0 ? r.loc_start - r.ns : 0;
  okb = 0;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int p0 = first + 16 * rb + c16;
    const bool ok = p0 < lim;
    const int pos = ok ? p0 + (p0 >= thr ? shift : 0) : 0;
    const uint16_t* row = base + (uint32_t)(pos * rstride + 8 * g);
#pragma unroll
    for (int p = 0; p < NP; ++p) cv[rb][p] = *(const s16x8*)(row + 32 * p);
    // lanes 0-15 load rows 16 rb + c16: bits 4g .. 4g+3 of their ballot are this lane's rows
    okb |= (uint32_t)((__ballot(ok) >> (4 * g)) & 0xfu) << (4 * rb);
  }
}

// Online-softmax state of one stream for the lane's MFMA column (head c16): running max,
// running sum and Z[dim][head] as accumulator tiles (lane holds dims 16 dt + 4 g + i).
template <int NP>
struct SaAcc {
  float m, l;
  f32x4 z[2 * NP];
};

template <int NP>
__device__ __forceinline__ void sa_acc_init(SaAcc<NP>& st) {
  st.m = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int dt = 0; dt < 2 * NP; ++dt) st.z[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// After a stream's tiles: a column whose head does not attend to the stream (heads >= H, or
// other heads of a per-head sparse segment) leaves as no valid key (m = -inf, l = 0); every
// merge gives such a partial zero weight without reading its Z.
template <int NP>
__device__ __forceinline__ void sa_acc_close(SaAcc<NP>& st, bool head_on) {
  if (!head_on) {
    st.m = -INFINITY;
    st.l = 0.f;
  }
}

// The tiles [t0, t1) of a stream through two register sets in turn: the next tile's
// loads are in flight while a tile computes, and no set is copied into the other (a copy
// would wait for the loads).  Loads past the last tile re-read it (in bounds, unused);
// unconditional loads keep the register pressure at that of straight-line code.  blk_of(t)
// is the sparse block index of tile t (wave-uniform).
template <int NP, int RB = 4, class BlkOf, class Prep>
__device__ __forceinline__ void sa_stream_tiles(const SaRows& rows, int stream, int64_t t0, int64_t t1, BlkOf blk_of,
                                                const s16x8 (&qh)[NP], const s16x8 (&ql)[NP], short* tile,
                                                int c16, int g, SaAcc<NP>& st, Prep prep);

// One 64-key tile: scores D[key][head] = C Q^T with the scaled query in bf16 hi + lo (B
// operand), online softmax, values Z[dim][head] += C^T P with the tile copied row-major into
// the wave's LDS and read transposed, P in bf16 hi + lo.  Every column runs the softmax (a
// column of a head that does not attend to the stream is discarded by the caller, see
// sa_acc_close); a tile whose 64 keys are all valid skips the masking, and the rescale of
// Z is skipped when no column's running max moved (both tests wave-uniform).
template <int NP, int RB = 4>
__device__ __forceinline__ void sa_tile_step(const s16x8 (&cv)[RB][NP], uint32_t okb,
                                             const s16x8 (&qh)[NP], const s16x8 (&ql)[NP], short* tile, int c16,
                                             int g, SaAcc<NP>& st) {
  static_assert(RB == 2 || RB == 4, "tiles of 32 or 64 keys");
  constexpr int DC = 32 * NP;
  constexpr int TP = DC + 8;
  f32x4 sc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < NP; ++p) {
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
  if (__ballot(okb != (1u << (4 * RB)) - 1u) != 0ull) {   // some key of the tile is invalid
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = ((okb >> (4 * rb + i)) & 1u) ? sc[rb][i] : -INFINITY;
        sc[rb][i] = x;
        tmax = fmaxf(tmax, x);
      }
    }
  } else {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      tmax = fmaxf(fmaxf(tmax, fmaxf(sc[rb][0], sc[rb][1])), fmaxf(sc[rb][2], sc[rb][3]));
  }
  tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
  tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
  const float m_new = fmaxf(st.m, tmax);
  const bool grow = __ballot(m_new != st.m) != 0ull;   // wave-uniform: some column's max moved
  const float corr = (m_new == -INFINITY || !grow) ? 1.f : __expf(st.m - m_new);
  const float m_sub = (m_new == -INFINITY) ? 0.f : m_new;   // exp(-inf - m_sub) = 0 for masked keys
  float psum = 0.f;
  s16x4 ph[RB], pl[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    f32x4 pv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float pe = __expf(sc[rb][i] - m_sub);
      pv[i] = pe;
      psum += pe;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const short hb = __builtin_bit_cast(short, (__bf16)pv[i]);
      ph[rb][i] = hb;
      pl[rb][i] = __builtin_bit_cast(short, (__bf16)(pv[i] - bf16_bits_to_f32((uint16_t)hb)));
    }
  }
  psum += __shfl_xor(psum, 16);
  psum += __shfl_xor(psum, 32);
  st.l = st.l * corr + psum;
  st.m = m_new;
  // z[dim][head] = corr * z + C^T P  (the tile's keys as permuted 32-steps)
#pragma unroll
  for (int dt = 0; dt < DC / 16; ++dt) {
    f32x4 acc = grow ? st.z[dt] * corr : st.z[dt];
#pragma unroll
    for (int p2 = 0; p2 < RB / 2; ++p2) {
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
    st.z[dt] = acc;
  }
}

// prep() runs once the first tile's loads are issued (or at once when the wave has no tile):
// the caller's work that waits on earlier loads (the query conversion) then overlaps them.
template <int NP, int RB, class BlkOf, class Prep>
__device__ __forceinline__ void sa_stream_tiles(const SaRows& rows, int stream, int64_t t0, int64_t t1, BlkOf blk_of,
                                                const s16x8 (&qh)[NP], const s16x8 (&ql)[NP], short* tile,
                                                int c16, int g, SaAcc<NP>& st, Prep prep) {
  if (t0 >= t1) {
    prep();
    return;
  }
  s16x8 cvA[RB][NP], cvB[RB][NP];
  uint32_t okA = 0, okB = 0;
  sa_load_rows<NP, RB>(rows, stream, t0, blk_of(t0), c16, g, cvA, okA);
  prep();
  for (int64_t tix = t0; tix < t1; tix += 2) {
    const int64_t n1 = tix + 1 < t1 ? tix + 1 : tix;
    sa_load_rows<NP, RB>(rows, stream, n1, blk_of(n1), c16, g, cvB, okB);
    sa_tile_step<NP, RB>(cvA, okA, qh, ql, tile, c16, g, st);
    if (tix + 1 >= t1) break;
    const int64_t n2 = tix + 2 < t1 ? tix + 2 : tix + 1;
    sa_load_rows<NP, RB>(rows, stream, n2, blk_of(n2), c16, g, cvA, okA);
    sa_tile_step<NP, RB>(cvB, okB, qh, ql, tile, c16, g, st);
  }
}

// The lane's query fragment for MFMA column c16 (head c16, dims 32 p + 8 g .. +7), loaded as
// stored (sa_query_load) and then, once the first key tile's loads are in flight, times the
// score scale and split bf16 hi + lo (sa_query_cvt); heads >= H are zero.  q + qoff: the fp32
// query rows of the sequence (head stride qsh, unit channel stride when vec).
template <int NP, bool VEC>
__device__ __forceinline__ void sa_query_load(const void* q, int qdt, int64_t qoff, int64_t qsh, int64_t qsd,
                                              int H, int c16, int g, float (&qv)[NP][8]) {
  if constexpr (VEC) {  // fp32 rows, 16-byte aligned: all of the lane's query loads in flight at once
    // unconditional loads (columns past H read head H - 1; sa_query_cvt zeroes them), so that
    // the compiler can count them and later waits need not drain every load
    const float* qp = (const float*)q + qoff + (c16 < H ? c16 : H - 1) * qsh + 8 * g;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const f32x4 x0 = *(const f32x4*)(qp + 32 * p);
      const f32x4 x1 = *(const f32x4*)(qp + 32 * p + 4);
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
        qv[p][j] = (c16 < H) ? load_elem(q, qdt, qoff + c16 * qsh + (32 * p + 8 * g + j) * qsd) : 0.f;
  }
}

template <int NP>
__device__ __forceinline__ void sa_query_cvt(const float (&qv)[NP][8], float scale, bool on, s16x8 (&qh)[NP],
                                             s16x8 (&ql)[NP]) {
#pragma unroll
  for (int p = 0; p < NP; ++p) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float x = on ? qv[p][j] * scale : 0.f;   // scores come out scaled; heads >= H are zero
      const short h = __builtin_bit_cast(short, (__bf16)x);
      qh[p][j] = h;
      ql[p][j] = __builtin_bit_cast(short, (__bf16)(x - bf16_bits_to_f32((uint16_t)h)));
    }
  }
}

template <int NP, bool QV>  // d_c = 32 * NP; QV: fp32 queries with 16-byte aligned rows
__global__ __launch_bounds__(256, 2) void maba_sa_mfma_kernel(SaArgs a_in) {
  const SaArgs a = sa_live(a_in);
  constexpr int DC = 32 * NP;
  constexpr int TP = DC + 8;  // row pitch (bf16) of the per-wave key tile: 16-B aligned, rows shift 4 banks
  __shared__ __attribute__((aligned(16))) short s_tile[4][64 * TP];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int sid = (int)blockIdx.x;
  const int64_t b = blockIdx.y;
  const SaSeg sg = sa_segment(a, sid);
  const int tpw = a.tpw;
  const int64_t t0 = sg.t_begin + (int64_t)wave * tpw;
  const int64_t t1 = min(sg.t_end, t0 + tpw);
  short* tile = s_tile[wave];

  // Loads in the order they are needed: the sparse block indices of the wave's tiles (one per
  // lane), the query rows, then the first tile (which waits for the indices only); the query's
  // scaling and hi/lo split (the scores' B operand, head c16) wait for it only after that.
  int64_t blk_l = 0;
  if (sg.stream == 1 && lane < t1 - t0) blk_l = a.idx[b * a.isb + sg.hs * a.ish + (t0 + lane) * a.isk];
  float qv[NP][8];
  sa_query_load<NP, QV>(a.q, a.qdt, b * a.qsb, a.qsh, a.qsd, a.H, c16, g, qv);
  s16x8 qh[NP], ql[NP];
  const bool head_on = c16 < a.H && (sg.head_only < 0 || sg.head_only == c16);
  SaAcc<NP> st;
  sa_acc_init(st);
  const SaRows rows = sa_rows(a, b);
  auto blk_of = [&](int64_t tix) {   // wave-uniform lane index
    const int src = (int)(tix - t0);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)blk_l, src);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)blk_l >> 32), src);
    return (int64_t)(((uint64_t)hi << 32) | lo);
  };
  sa_stream_tiles<NP>(rows, sg.stream, t0, t1, blk_of, qh, ql, tile, c16, g, st,
                      [&] { sa_query_cvt<NP>(qv, a.scale, c16 < a.H, qh, ql); });
  sa_acc_close(st, head_on);
  const float m_run = st.m, l_run = st.l;
  const f32x4* z = st.z;
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
    const int64_t o = sa_part_off(a, b, sid, h);
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

// ------------------------------------------------------------------ prefill, latent form
// Every query t of a prefill (position pos = Lkv - Lq + t) attends, per head, to the three
// streams of a decode step at length L = pos + 1 (layers/sparse_attention.py:95-105,
// 145-171, 173-219, 275: the local window and sinks with j <= pos, the listed blocks'
// tokens <= pos with multiplicity, the complete means with (e+1) pool - 1 <= pos or the
// running mean before pool - 1), in latent space with the heads in the MFMA columns: the
// key rows of a tile serve every head of the query, and no query of another position
// shares the wave.  One workgroup of PL_W waves per query; the waves are split over the
// streams in proportion to their tile counts (each wave one stream, one online softmax),
// then the partials of each stream are merged in LDS, gated and written as
// z[b, t, h] = sum_s g_s sum_j p_sj c_j (fp32); the caller applies W_v,h.
// Eight waves (two per SIMD) on 64-key tiles.  Twelve waves on 32-key tiles (three per SIMD
// within 168 VGPRs, a few spilled) measured 4.84 ms against 4.02 ms at the 32k bench row: the
// per-tile reductions and rescale are paid twice as often, and the third wave does not win
// that back.
constexpr int PL_W = 8;
constexpr int PL_RB = 4;
constexpr int PL_TK = 16 * PL_RB;

struct PlArgs {
  const void* q; int qdt; int64_t qsb, qst, qsh, qsd; int qvec;   // q_lat [B, Lq, H, dc]
  const uint16_t* c; int64_t csb, csl;                            // [B, Lkv, dc] bf16
  const uint16_t* hca; int64_t hsb, hsn;                          // [B, >= Lkv/pool, dc] bf16
  const int64_t* idx; int64_t isb, ist, isk;                      // [B, Lq | 1, K]
  const void* gate; int gdt; int64_t gsb, gsh, gst, gsm;          // [B, Lq, 3] (gsh = 0) or [B, H, Lq, 3]
  float* out; int64_t osb, ost, osh;                              // [B, Lq, H, dc] fp32, unit channel stride
  int64_t Lq, Lkv;
  int H, K, window, n_sink, bs, pool;
  float scale;
};

template <int NP, bool QV>
__global__ __launch_bounds__(PL_W * 64, 1) void maba_sa_prefill_latent_kernel(PlArgs a) {
  constexpr int DC = 32 * NP;
  constexpr int TP = DC + 8;
  __shared__ __attribute__((aligned(16))) short s_tile[PL_W][PL_TK * TP];
  static_assert(PL_W * 16 * DC * sizeof(float) <= sizeof(s_tile), "the merge reuses the tiles' LDS");
  __shared__ float s_ml[PL_W][2][16];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int64_t b = blockIdx.x / a.Lq, t = blockIdx.x % a.Lq;
  const int64_t L = a.Lkv - a.Lq + t + 1;
  // the three streams of a decode step at length L (as sa_geometry)
  SaRows rows;
  rows.c = a.c + b * a.csb; rows.cs = a.csl;
  rows.hca = a.hca + b * a.hsb; rows.hs = a.hsn;
  rows.L = L; rows.bs = a.bs; rows.nblk = (L + a.bs - 1) / a.bs;
  const int64_t ns = L < a.n_sink ? L : a.n_sink;
  const int64_t lst = (L - a.window) > ns ? (L - a.window) : ns;
  rows.ns = (int)ns; rows.loc_start = (int)lst; rows.nloc = (int)(ns + (L - lst)); rows.nc = (int)(L / a.pool);
  // tiles per stream (a sparse block is tpb tiles; the sparse waves split the K slots)
  const int tpb = (a.bs + PL_TK - 1) / PL_TK;
  const int tc0 = (rows.nloc + PL_TK - 1) / PL_TK, tc1 = a.K * tpb;
  const int tc2 = (L - 1 >= a.pool - 1) ? (rows.nc + PL_TK - 1) / PL_TK : 0;
  // waves per stream: in proportion to the tile counts, at least one per nonempty stream
  // (scalars throughout: a small array indexed by the stream would go to scratch memory)
  const int T = tc0 + tc1 + tc2;
  const int Tm = T > 0 ? T : 1;
  int n0 = tc0 > 0 ? max(1, PL_W * tc0 / Tm) : 0;
  int n1 = tc1 > 0 ? max(1, PL_W * tc1 / Tm) : 0;
  int n2 = tc2 > 0 ? max(1, PL_W * tc2 / Tm) : 0;
  while (n0 + n1 + n2 > PL_W) {   // take a wave from the stream with the most waves
    if (n1 >= n0 && n1 >= n2 && n1 > 1) --n1;
    else if (n2 >= n0 && n2 > 1) --n2;
    else --n0;
  }
  while (n0 + n1 + n2 < PL_W) {   // give a wave to the stream with the most tiles per wave
    const int p0 = n0 ? (tc0 + n0 - 1) / n0 : 0, p1 = n1 ? (tc1 + n1 - 1) / n1 : 0, p2 = n2 ? (tc2 + n2 - 1) / n2 : 0;
    const int best = max(p0, max(p1, p2));
    if (best <= 1) break;
    if (p1 == best) ++n1; else if (p2 == best) ++n2; else ++n0;
  }
  const int wb1 = n0, wb2 = n0 + n1, wend = n0 + n1 + n2;   // waves [0,wb1) local, [wb1,wb2) sparse, [wb2,wend) HCA
  const int stream = wave < wb1 ? 0 : (wave < wb2 ? 1 : (wave < wend ? 2 : -1));
  const int j = stream == 0 ? wave : (stream == 1 ? wave - wb1 : wave - wb2);
  // units a wave's range is counted in: tiles, or K slots for the sparse stream
  const int tcs = stream == 0 ? tc0 : (stream == 1 ? a.K : tc2);
  const int nws = stream == 0 ? n0 : (stream == 1 ? n1 : n2);
  int64_t u0 = 0, u1 = 0;
  if (stream >= 0) {
    const int per = (tcs + nws - 1) / nws;
    u0 = (int64_t)j * per;
    u1 = min((int64_t)tcs, u0 + per);
  }
  const int64_t t0 = stream == 1 ? u0 * tpb : u0, t1 = stream == 1 ? u1 * tpb : u1;
  short* tile = s_tile[wave];
  // the wave's sparse slots [u0, u1) (at most 64: K <= 64), one block index per lane, then the
  // query rows (converted once the first tile's loads are issued)
  int64_t blk_l = 0;
  if (stream == 1 && lane < u1 - u0) blk_l = a.idx[b * a.isb + t * a.ist + (u0 + lane) * a.isk];
  float qv[NP][8];
  sa_query_load<NP, QV>(a.q, a.qdt, b * a.qsb + t * a.qst, a.qsh, a.qsd, a.H, c16, g, qv);
  s16x8 qh[NP], ql[NP];
  const bool head_on = c16 < a.H;
  SaAcc<NP> st;
  sa_acc_init(st);
  auto blk_of = [&](int64_t tix) {
    const int src = (int)(tix / tpb - u0);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)blk_l, src);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)blk_l >> 32), src);
    return (int64_t)(((uint64_t)hi << 32) | lo);
  };
  if (stream >= 0)
    sa_stream_tiles<NP, PL_RB>(rows, stream, t0, t1, blk_of, qh, ql, tile, c16, g, st,
                               [&] { sa_query_cvt<NP>(qv, a.scale, c16 < a.H, qh, ql); });
  sa_acc_close(st, head_on);
  // wave partials to LDS (the tiles are free once every wave is past its loop)
  __syncthreads();
  float* s_z = (float*)&s_tile[0][0];   // [PL_W][16][DC]
#pragma unroll
  for (int dt = 0; dt < DC / 16; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) s_z[(wave * 16 + c16) * DC + 16 * dt + 4 * g + i] = st.z[dt][i];
  if (g == 0) {
    s_ml[wave][0][c16] = stream >= 0 ? st.m : -INFINITY;
    s_ml[wave][1][c16] = stream >= 0 ? st.l : 0.f;
  }
  __syncthreads();
  const bool early = L - 1 < a.pool - 1;
  const int wr[4] = {0, wb1, wb2, wend};
  for (int e = threadIdx.x; e < a.H * DC; e += PL_W * 64) {
    const int h = e / DC, d = e % DC;
    const int64_t gb = b * a.gsb + h * a.gsh + t * a.gst;
    float z0 = load_elem(a.gate, a.gdt, gb), z1 = load_elem(a.gate, a.gdt, gb + a.gsm),
          z2 = load_elem(a.gate, a.gdt, gb + 2 * a.gsm);
    const float gm = fmaxf(z0, fmaxf(z1, z2));
    z0 = __expf(z0 - gm); z1 = __expf(z1 - gm); z2 = __expf(z2 - gm);
    const float gi = 1.f / (z0 + z1 + z2);
    const float gs[3] = {z0 * gi, z1 * gi, z2 * gi};
    float res = 0.f;
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      if (s == 2 && early) continue;
      float M = -INFINITY;
      for (int w = wr[s]; w < wr[s + 1]; ++w) M = fmaxf(M, s_ml[w][0][h]);
      if (M == -INFINITY) continue;   // no valid key: the stream gives 0
      float Ls = 0.f, Zs = 0.f;
      for (int w = wr[s]; w < wr[s + 1]; ++w) {
        const float m = s_ml[w][0][h];
        if (m == -INFINITY) continue;
        const float f = __expf(m - M);
        Ls = fmaf(f, s_ml[w][1][h], Ls);
        Zs = fmaf(f, s_z[(w * 16 + h) * DC + d], Zs);
      }
      if (Ls > 0.f) res = fmaf(gs[s], Zs / Ls, res);
    }
    if (early) {   // HCA before the first complete block: running mean of c[0..pos]
      float zs = 0.f;
      for (int64_t r = 0; r < L; ++r) zs += bf16_bits_to_f32(rows.c[r * rows.cs + d]);
      res = fmaf(gs[2], zs / (float)L, res);
    }
    a.out[b * a.osb + t * a.ost + h * a.osh + d] = res;
  }
}

// Segment path geometry: the fewest tiles per wave (at most 8) for which the segments
// of all streams fit one workgroup per compute unit (every workgroup pays a fixed
// start-up; one round of workgroups covers the machine).
static void sa_segments(SaArgs& a, int ncu) {
  for (a.tpw = 1;; ++a.tpw) {
    const int span = 4 * a.tpw;
    a.s_loc = (int)ceil_div(a.t_loc, span);
    a.s_hca = (int)ceil_div(a.t_hca, span);
    a.s_sp1 = (int)ceil_div(a.K, span);
    a.s_sp = a.Hi == 1 ? a.s_sp1 : a.H * a.s_sp1;
    if (a.B * (a.s_loc + a.s_hca + a.s_sp) <= ncu || a.tpw == 8) break;
  }
}

static size_t sa_part_bytes(int64_t slots, int64_t B, int64_t H, int64_t dc) {
  return (size_t)((slots > 0 ? slots : 1) * B * H * (dc + 2)) * sizeof(float);
}

// Validation and argument set-up.
static int sa_setup(const maba_tensor* q_lat, const maba_tensor* c_kv, const maba_tensor* hca,
                    const maba_tensor* idx, const maba_tensor* gate, const maba_tensor* out_lat, int64_t L,
                    float scale, int window, int n_sink, int block_size, int pool, void* workspace,
                    size_t workspace_bytes, SaArgs& a, bool& seg, bool& empty, size_t& need) {
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
  empty = B * H == 0;
  if (empty) return MABA_OK;
  a = SaArgs{};
  a.dlen = nullptr;
  a.q = q_lat->data; a.qdt = q_lat->dtype; a.qsb = q_lat->stride[0]; a.qsh = q_lat->stride[1]; a.qsd = q_lat->stride[2];
  a.qvec = q_lat->dtype == MABA_F32 && q_lat->stride[2] == 1 && (uintptr_t)q_lat->data % 16 == 0 &&
           q_lat->stride[0] % 4 == 0 && q_lat->stride[1] % 4 == 0;
  a.c = c_kv->data; a.cdt = c_kv->dtype; a.csb = c_kv->stride[0]; a.csl = c_kv->stride[1]; a.csd = c_kv->stride[2];
  a.hca = hca->data; a.hdt = hca->dtype; a.hsb = hca->stride[0]; a.hsn = hca->stride[1]; a.hsd = hca->stride[2];
  a.idx = (const int64_t*)idx->data; a.isb = idx->stride[0]; a.ish = idx->stride[1]; a.isk = idx->stride[2];
  a.gate = gate->data; a.gdt = gate->dtype; a.gsb = gate->stride[0];
  if (gate->ndim == 2) { a.gsh = 0; a.gsm = gate->stride[1]; } else { a.gsh = gate->stride[1]; a.gsm = gate->stride[2]; }
  a.out = (float*)out_lat->data; a.osb = out_lat->stride[0]; a.osh = out_lat->stride[1]; a.osd = out_lat->stride[2];
  a.L = L; a.B = B; a.H = (int)H; a.dc = (int)dc; a.Hi = (int)idx->shape[1]; a.K = (int)idx->shape[2];
  a.window = window; a.n_sink = n_sink; a.bs = block_size; a.pool = pool; a.scale = scale;
  sa_geometry(a, L, window, n_sink, pool, a.Hi, a.K);
  seg = c_kv->dtype == MABA_BF16 && hca->dtype == MABA_BF16 && c_kv->stride[2] == 1 && hca->stride[2] == 1 &&
        dc % 32 == 0 && dc <= 128 && (uintptr_t)c_kv->data % 16 == 0 && (uintptr_t)hca->data % 16 == 0 &&
        c_kv->stride[0] % 8 == 0 && c_kv->stride[1] % 8 == 0 && hca->stride[0] % 8 == 0 && hca->stride[1] % 8 == 0 &&
        c_kv->shape[1] * c_kv->stride[1] <= INT32_MAX && hca->shape[1] * hca->stride[1] <= INT32_MAX;
  int64_t slots = a.ntiles;
  if (seg) {
    sa_segments(a, device_cu_count());
    slots = a.s_loc + a.s_hca + a.s_sp;
  }
  need = sa_part_bytes(slots, B, H, dc);
  if (!workspace || workspace_bytes < need)
    return fail(MABA_ERR_WORKSPACE, "maba_sa_decode: workspace of %zu bytes required", need);
  a.ws = (float*)workspace;
  return MABA_OK;
}

// Merge of every (b, h): one workgroup each.
static int sa_launch_combine(const SaArgs& a, bool seg, hipStream_t s) {
  SaMerge mg;
  if (seg) {   // slots: local, HCA, then the sparse ones (per index row)
    const int nsp = a.Hi == 1 ? a.s_sp : a.s_sp1;
    mg = SaMerge{a.s_loc + a.s_hca + nsp, a.s_loc + a.s_hca, a.s_loc + a.s_hca, a.Hi == 1 ? 0 : a.s_sp1,
                 a.s_loc, a.s_loc + a.s_hca, 0, 2, 1};
  } else {     // per-tile slots: local, sparse, HCA
    mg = SaMerge{a.ntiles, a.ntiles, 0, 0, a.t_loc, a.t_loc + a.t_sp, 0, 1, 2};
  }
  hipLaunchKernelGGL(maba_sa_combine_kernel, dim3((unsigned)(a.B * a.H)), dim3(256), 0, s, a, mg);
  return check_launch("maba_sa_decode/combine");
}

// The segment (or per-tile) launch and the merge, once sa_setup has filled the arguments.
static int sa_run(const SaArgs& a, bool seg, hipStream_t s) {
  const unsigned nslot = (unsigned)(seg ? a.s_loc + a.s_hca + a.s_sp : a.ntiles);
  if (nslot > 0) {
    const dim3 grid(nslot, (unsigned)a.B);
    if (seg) {
      switch (a.dc / 32) {
        case 1: hipLaunchKernelGGL((a.qvec ? maba_sa_mfma_kernel<1, true> : maba_sa_mfma_kernel<1, false>), grid, dim3(256), 0, s, a); break;
        case 2: hipLaunchKernelGGL((a.qvec ? maba_sa_mfma_kernel<2, true> : maba_sa_mfma_kernel<2, false>), grid, dim3(256), 0, s, a); break;
        case 3: hipLaunchKernelGGL((a.qvec ? maba_sa_mfma_kernel<3, true> : maba_sa_mfma_kernel<3, false>), grid, dim3(256), 0, s, a); break;
        default: hipLaunchKernelGGL((a.qvec ? maba_sa_mfma_kernel<4, true> : maba_sa_mfma_kernel<4, false>), grid, dim3(256), 0, s, a); break;
      }
    } else {
      hipLaunchKernelGGL(maba_sa_tile_kernel, grid, dim3(256), 0, s, a);
    }
    const int rc = check_launch(seg ? "maba_sa_decode/segments" : "maba_sa_decode/tiles");
    if (rc) return rc;
  }
  return sa_launch_combine(a, seg, s);
}

// Scratch of maba_hip_maba_sa_decode_static: the partial slots of one decode step, held by
// every GPU the library runs on until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not a device address); it passes
// the device address hipGetSymbolAddress returns for the current device, kept per device.
static __device__ __align__(256) float scratch[MABA_SA_STATIC_SCRATCH_BYTES / sizeof(float)];

constexpr int SA_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[SA_MAX_DEVICES];

// Device address of the current device's scratch, queried on the first call per device.
static int sa_static_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MABA_ERR_HIP, "maba_sa_decode_static: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= SA_MAX_DEVICES)
    return fail(MABA_ERR_UNSUPPORTED, "maba_sa_decode_static: device %d beyond %d", dev, SA_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(MABA_ERR_HIP, "maba_sa_decode_static: hipGetSymbolAddress: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MABA_OK;
}

}  // namespace maba

using namespace maba;

extern "C" size_t maba_hip_maba_sa_decode_workspace_size(int64_t B, int64_t H, int64_t dc, int64_t L,
                                                         int64_t K, int window, int n_sink, int pool) {
  // upper bound over both paths and index-row counts: the generic path's per-tile slots with Hi = H
  SaArgs a;
  sa_geometry(a, L, window, n_sink, pool > 0 ? pool : 64, (int)H, (int)K);
  return sa_part_bytes(a.ntiles, B, H, dc);
}

extern "C" int maba_hip_maba_sa_decode(const maba_tensor* q_lat, const maba_tensor* c_kv,
                                       const maba_tensor* hca, const maba_tensor* idx,
                                       const maba_tensor* gate, int64_t L, float scale, int window,
                                       int n_sink, int block_size, int pool, maba_tensor* out_lat,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  SaArgs a;
  bool seg = false, empty = false;
  size_t need = 0;
  int rc = sa_setup(q_lat, c_kv, hca, idx, gate, out_lat, L, scale, window, n_sink, block_size, pool, workspace,
                    workspace_bytes, a, seg, empty, need);
  if (rc || empty) return rc;
  return sa_run(a, seg, (hipStream_t)stream);
}

extern "C" int maba_hip_maba_sa_decode_static(const maba_tensor* q_lat, const maba_tensor* c_kv,
                                              const maba_tensor* hca, const maba_tensor* idx,
                                              const maba_tensor* gate, int64_t L, float scale, int window,
                                              int n_sink, int block_size, int pool, maba_tensor* out_lat,
                                              void* stream) {
  void* ws = nullptr;
  int rc = sa_static_scratch(&ws);
  if (rc) return rc;
  SaArgs a;
  bool seg = false, empty = false;
  size_t need = 0;
  rc = sa_setup(q_lat, c_kv, hca, idx, gate, out_lat, L, scale, window, n_sink, block_size, pool, ws,
                MABA_SA_STATIC_SCRATCH_BYTES, a, seg, empty, need);
  if (rc == MABA_ERR_WORKSPACE)
    return fail(MABA_ERR_WORKSPACE,
                "maba_sa_decode_static: this call needs %zu bytes of scratch; the static scratch holds %zu "
                "(use maba_hip_maba_sa_decode with a workspace)", need, (size_t)MABA_SA_STATIC_SCRATCH_BYTES);
  if (rc || empty) return rc;
  // every partial slot the merge reads is written by this call's first launch, so nothing
  // left in the scratch by an earlier call is read
  return sa_run(a, seg, (hipStream_t)stream);
}

extern "C" int maba_hip_maba_sa_decode_dev(const maba_tensor* q_lat, const maba_tensor* c_kv,
                                           const maba_tensor* hca, const maba_tensor* idx,
                                           const maba_tensor* gate, const int64_t* d_len, int64_t L_cap,
                                           float scale, int window, int n_sink, int block_size, int pool,
                                           maba_tensor* out_lat, void* workspace, size_t workspace_bytes,
                                           void* stream) {
  if (!d_len) return fail(MABA_ERR_INVALID, "maba_sa_decode_dev: d_len (device int64) required");
  SaArgs a;
  bool seg = false, empty = false;
  size_t need = 0;
  int rc = sa_setup(q_lat, c_kv, hca, idx, gate, out_lat, L_cap, scale, window, n_sink, block_size, pool,
                    workspace, workspace_bytes, a, seg, empty, need);
  if (rc || empty) return rc;
  if (!seg)
    return fail(MABA_ERR_UNSUPPORTED, "maba_sa_decode_dev: bf16 caches with 16-byte aligned rows and d_c a "
                                      "multiple of 32 up to 128 required");
  if (L_cap < pool) return fail(MABA_ERR_UNSUPPORTED, "maba_sa_decode_dev: L_cap must be at least pool");
  a.dlen = d_len;
  return sa_run(a, seg, (hipStream_t)stream);
}

extern "C" int maba_hip_maba_sa_decode_dev_heads(const maba_tensor* q_lat, const maba_tensor* c_kv,
                                                 const maba_tensor* hca, const maba_tensor* idx,
                                                 const maba_tensor* gate, const int64_t* d_len, int64_t L_cap,
                                                 float scale, int window, int n_sink, int block_size, int pool,
                                                 const maba_tensor* w_v, maba_tensor* out_heads,
                                                 maba_tensor* out_lat, void* workspace, size_t workspace_bytes,
                                                 void* stream) {
  if (!d_len) return fail(MABA_ERR_INVALID, "maba_sa_decode_dev_heads: d_len (device int64) required");
  SaArgs a;
  bool seg = false, empty = false;
  size_t need = 0;
  int rc = sa_setup(q_lat, c_kv, hca, idx, gate, out_lat, L_cap, scale, window, n_sink, block_size, pool,
                    workspace, workspace_bytes, a, seg, empty, need);
  if (rc || empty) return rc;
  if (!seg)
    return fail(MABA_ERR_UNSUPPORTED, "maba_sa_decode_dev_heads: bf16 caches with 16-byte aligned rows and d_c a "
                                      "multiple of 32 up to 128 required");
  if (L_cap < pool) return fail(MABA_ERR_UNSUPPORTED, "maba_sa_decode_dev_heads: L_cap must be at least pool");
  const int64_t B = a.B, H = a.H, dc = a.dc;
  if (!w_v || w_v->ndim != 2 || w_v->shape[1] != dc || w_v->shape[0] % H != 0 || w_v->shape[0] / H > 64 ||
      !out_heads || out_heads->ndim != 2 || out_heads->shape[0] != B || out_heads->shape[1] != w_v->shape[0])
    return fail(MABA_ERR_INVALID, "maba_sa_decode_dev_heads: w_v [H*dh,dc] (dh <= 64) and out_heads [B,H*dh] required");
  if (w_v->dtype != MABA_BF16 || out_heads->dtype != MABA_BF16)
    return fail(MABA_ERR_DTYPE, "maba_sa_decode_dev_heads: bf16 w_v and out_heads");
  if (w_v->stride[1] != 1 || (uintptr_t)w_v->data % 8 != 0 || w_v->stride[0] % 4 != 0)
    return fail(MABA_ERR_UNSUPPORTED, "maba_sa_decode_dev_heads: w_v rows 8-byte aligned with unit column stride");
  a.wv = (const uint16_t*)w_v->data; a.wvs = w_v->stride[0];
  a.oh = (uint16_t*)out_heads->data; a.ohsb = out_heads->stride[0]; a.ohsd = out_heads->stride[1];
  a.dh = (int)(w_v->shape[0] / H);
  a.dlen = d_len;
  return sa_run(a, seg, (hipStream_t)stream);
}

extern "C" int maba_hip_maba_sa_prefill_latent(const maba_tensor* q_lat, const maba_tensor* c_kv,
                                               const maba_tensor* hca, const maba_tensor* idx,
                                               const maba_tensor* gate, float scale, int window, int n_sink,
                                               int block_size, int pool, maba_tensor* out_lat, void* stream) {
  if (!q_lat || q_lat->ndim != 4) return fail(MABA_ERR_INVALID, "maba_sa_prefill_latent: q_lat must be [B,Lq,H,dc]");
  const int64_t B = q_lat->shape[0], Lq = q_lat->shape[1], H = q_lat->shape[2], dc = q_lat->shape[3];
  if (!c_kv || c_kv->ndim != 3 || c_kv->shape[0] != B || c_kv->shape[2] != dc || c_kv->shape[1] < Lq)
    return fail(MABA_ERR_INVALID, "maba_sa_prefill_latent: c_kv must be [B,Lkv>=Lq,dc]");
  const int64_t Lkv = c_kv->shape[1];
  if (window < 0 || n_sink < 0 || block_size <= 0 || pool <= 0)
    return fail(MABA_ERR_INVALID, "maba_sa_prefill_latent: bad window/sink/block/pool");
  if (!hca || hca->ndim != 3 || hca->shape[0] != B || hca->shape[2] != dc || hca->shape[1] < Lkv / pool)
    return fail(MABA_ERR_INVALID, "maba_sa_prefill_latent: hca must be [B,>=Lkv/pool,dc]");
  if (!idx || idx->ndim != 3 || idx->shape[0] != B || (idx->shape[1] != Lq && idx->shape[1] != 1))
    return fail(MABA_ERR_INVALID, "maba_sa_prefill_latent: idx must be [B,Lq|1,K]");
  if (idx->dtype != MABA_I64) return fail(MABA_ERR_DTYPE, "maba_sa_prefill_latent: idx must be int64");
  if (!gate || !((gate->ndim == 3 && gate->shape[0] == B && gate->shape[1] == Lq && gate->shape[2] == 3) ||
                 (gate->ndim == 4 && gate->shape[0] == B && gate->shape[1] == H && gate->shape[2] == Lq &&
                  gate->shape[3] == 3)))
    return fail(MABA_ERR_INVALID, "maba_sa_prefill_latent: gate must be [B,Lq,3] or [B,H,Lq,3]");
  const int64_t so[4] = {B, Lq, H, dc};
  if (!expect_shape(out_lat, "out_lat", 4, so)) return MABA_ERR_INVALID;
  if (out_lat->dtype != MABA_F32 || out_lat->stride[3] != 1)
    return fail(MABA_ERR_DTYPE, "maba_sa_prefill_latent: out_lat must be f32 with unit channel stride");
  if (!expect_float(q_lat, "q_lat") || !expect_float(gate, "gate")) return MABA_ERR_DTYPE;
  if (c_kv->dtype != MABA_BF16 || hca->dtype != MABA_BF16)
    return fail(MABA_ERR_UNSUPPORTED, "maba_sa_prefill_latent: bf16 c_kv and hca");
  if (H > SA_MAXH || dc % 32 != 0 || dc > 128 || block_size > 64 || idx->shape[2] > 64)
    return fail(MABA_ERR_UNSUPPORTED, "maba_sa_prefill_latent: H <= %d, d_c a multiple of 32 up to 128, "
                "block_size <= 64 and K <= 64", SA_MAXH);
  if (B * Lq > INT32_MAX) return fail(MABA_ERR_UNSUPPORTED, "maba_sa_prefill_latent: B * Lq beyond one grid");
  if (c_kv->stride[2] != 1 || hca->stride[2] != 1 || (uintptr_t)c_kv->data % 16 || (uintptr_t)hca->data % 16 ||
      c_kv->stride[0] % 8 || c_kv->stride[1] % 8 || hca->stride[0] % 8 || hca->stride[1] % 8)
    return fail(MABA_ERR_UNSUPPORTED, "maba_sa_prefill_latent: 16-byte aligned bf16 rows with unit channel stride");
  if (Lkv * c_kv->stride[1] > INT32_MAX || hca->shape[1] * hca->stride[1] > INT32_MAX)
    return fail(MABA_ERR_UNSUPPORTED, "maba_sa_prefill_latent: a sequence's rows must span fewer than 2^31 elements");
  if (B * Lq * H == 0) return MABA_OK;
  PlArgs a;
  a.q = q_lat->data; a.qdt = q_lat->dtype; a.qsb = q_lat->stride[0]; a.qst = q_lat->stride[1];
  a.qsh = q_lat->stride[2]; a.qsd = q_lat->stride[3];
  a.qvec = q_lat->dtype == MABA_F32 && q_lat->stride[3] == 1 && (uintptr_t)q_lat->data % 16 == 0 &&
           q_lat->stride[0] % 4 == 0 && q_lat->stride[1] % 4 == 0 && q_lat->stride[2] % 4 == 0;
  a.c = (const uint16_t*)c_kv->data; a.csb = c_kv->stride[0]; a.csl = c_kv->stride[1];
  a.hca = (const uint16_t*)hca->data; a.hsb = hca->stride[0]; a.hsn = hca->stride[1];
  a.idx = (const int64_t*)idx->data; a.isb = idx->stride[0]; a.ist = idx->shape[1] == 1 ? 0 : idx->stride[1];
  a.isk = idx->stride[2];
  a.gate = gate->data; a.gdt = gate->dtype;
  if (gate->ndim == 3) { a.gsb = gate->stride[0]; a.gsh = 0; a.gst = gate->stride[1]; a.gsm = gate->stride[2]; }
  else { a.gsb = gate->stride[0]; a.gsh = gate->stride[1]; a.gst = gate->stride[2]; a.gsm = gate->stride[3]; }
  a.out = (float*)out_lat->data; a.osb = out_lat->stride[0]; a.ost = out_lat->stride[1]; a.osh = out_lat->stride[2];
  a.Lq = Lq; a.Lkv = Lkv; a.H = (int)H; a.K = (int)idx->shape[2];
  a.window = window; a.n_sink = n_sink; a.bs = block_size; a.pool = pool; a.scale = scale;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)(B * Lq));
  switch (dc / 32) {
    case 1: hipLaunchKernelGGL((a.qvec ? maba_sa_prefill_latent_kernel<1, true> : maba_sa_prefill_latent_kernel<1, false>), grid, dim3(PL_W * 64), 0, s, a); break;
    case 2: hipLaunchKernelGGL((a.qvec ? maba_sa_prefill_latent_kernel<2, true> : maba_sa_prefill_latent_kernel<2, false>), grid, dim3(PL_W * 64), 0, s, a); break;
    case 3: hipLaunchKernelGGL((a.qvec ? maba_sa_prefill_latent_kernel<3, true> : maba_sa_prefill_latent_kernel<3, false>), grid, dim3(PL_W * 64), 0, s, a); break;
    default: hipLaunchKernelGGL((a.qvec ? maba_sa_prefill_latent_kernel<4, true> : maba_sa_prefill_latent_kernel<4, false>), grid, dim3(PL_W * 64), 0, s, a); break;
  }
  return check_launch("maba_sa_prefill_latent");
}

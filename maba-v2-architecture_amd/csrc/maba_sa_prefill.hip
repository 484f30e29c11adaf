// MABA-SA prefill: the three attention streams for every query of a sequence and their
// gate superposition, without the reference's dense [Lq, Lkv] masks.
//
// Reference semantics (maba_sparse/layers/sparse_attention.py), per batch b, head h and
// query t at position pos = (Lkv - Lq) + t, with per-head keys/values k, v [Lkv, dh]:
//   local  (:95-105)  keys j <= pos with pos - j < window or j < min(n_sink, Lkv)
//   sparse (:145-171) the tokens of the blocks idx[b, t, :] that are < Lkv and <= pos
//                     (a block listed twice counts twice, as the reference's gather does)
//   HCA    (:173-219) pos >= pool - 1: the complete-block means e with (e+1) pool - 1 <= pos,
//                     keys kh / values vh (up-projected means); pos < pool - 1: the caller's
//                     running-mean row early[t]
//   gate   (:275)     out = sum_s softmax(logits)_s o_s; a stream with no valid key gives 0
//
// One workgroup per 64 consecutive queries of one (b, h), one wave per 16 of them.  The
// workgroup walks one list of 64-key tiles -- local (sinks, then the window of all 64
// queries), sparse (the union of the 64 queries' blocks, from an LDS bitmap compacted in
// ascending block order), HCA (the means any of them sees) -- staging each key and value tile
// once into double-buffered LDS, the next tile's loads in flight while the current one
// computes, one barrier per tile.  Per tile and wave, on bf16 MFMA with fp32 accumulation:
//   scores  S^T[key][query] = K Q^T     (A: key rows from the LDS tile, B: the wave's
//                                        16 queries in registers)
//   values  O^T[dim][query] += V^T P    (A: V^T fragments read transposed from the LDS
//                                        tile, B: the probabilities in bf16 hi + lo)
// with an online softmax per query and stream; each sparse key is weighted by how often the
// lane's query lists its block.  A wave skips the tiles none of its queries weights.
#include <algorithm>

#include "dgda_common.h"

namespace maba {

constexpr int PF_MAXK = 64;          // index slots per query
constexpr int PF_WORDS = 512;        // bitmap words per workgroup: blocks below 16384
constexpr int PF_LIST = 64 * PF_MAXK;   // the union of a workgroup's 64 queries' slots

typedef __attribute__((ext_vector_type(8))) short pf16x8;
typedef __attribute__((ext_vector_type(4))) short pf16x4;

struct PfArgs {
  const uint16_t* q; int64_t qsb, qsh, qst;       // [B,H,Lq,dh] bf16, unit channel stride
  const uint16_t* k; int64_t ksb, ksh, kst;       // [B,H,Lkv,dh]
  const uint16_t* v; int64_t vsb, vsh, vst;
  const uint16_t* kh; int64_t khb, khh, khe;      // [B,H,nc,dh] (unused when nc == 0)
  const uint16_t* vh; int64_t vhb, vhh, vhe;
  const void* early; int edt; int64_t esb, esh, est, esd;   // [B,H,n_early,dh] or null
  const int64_t* idx; int64_t isb, ist, isk;      // [B,Lq,K] (ist = 0 for one shared row)
  const void* gate; int gdt; int64_t gsb, gsh, gst, gsm;    // [B,Lq,3] (gsh = 0) or [B,H,Lq,3]
  void* out; int odt; int64_t osb, osh, ost;      // [B,H,Lq,dh], unit channel stride
  int64_t Lq, Lkv, nc, n_early, nb;
  int K, window, n_sink, pool;
  float scale;
};

// Transposed LDS read: lane j of 16-lane group g addressing row r0 + 4g + j/4, column
// c0 + 4(j%4) of a row-major tile receives the column fragment tile[r0 + 4g + r][c0 + j],
// r = 0..3.
__device__ __forceinline__ pf16x4 pf_ldsT4(const short* tile, int pitch, int r0, int c0, int c16, int g) {
  const short* p = tile + (r0 + 4 * g + (c16 >> 2)) * pitch + c0 + 4 * (c16 & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) pf16x4*)p);
}

// Bits 4 rb + i of the lane's 16 tile rows j = 16 rb + 4 g + i that lie in [lo, hi]
// (tile-relative, either bound may fall outside [0, 63]).
__device__ __forceinline__ uint32_t pf_range_bits(int lo, int hi, int g) {
  auto lowmask = [](int n) -> uint32_t { return n <= 0 ? 0u : n >= 32 ? 0xffffffffu : (1u << n) - 1u; };
  const uint32_t m0 = lowmask(hi + 1) & ~lowmask(lo);
  const uint32_t m1 = lowmask(hi - 31) & ~lowmask(lo - 32);
  const int sh = 4 * g;
  return ((m0 >> sh) & 0xfu) | (((m0 >> (16 + sh)) & 0xfu) << 4) | (((m1 >> sh) & 0xfu) << 8) |
         (((m1 >> (16 + sh)) & 0xfu) << 12);
}

// Running softmax state of one stream for the lane's query (m in log2 units).
template <int NDT>
struct PfAcc {
  float m, l;
  f32x4 z[NDT];   // O^T[16 dt + 4g + i][query c16]
};

template <int NP>   // dh = 32 NP
__global__ __launch_bounds__(256, NP == 4 ? 2 : 3) void maba_sa_prefill_kernel(PfArgs a) {
  constexpr int DH = 32 * NP;
  constexpr int TP = DH + 8;      // row pitch (bf16) of the LDS key and value tiles
  constexpr int NDT = DH / 16;
  constexpr int TE = 64 * TP;
  __shared__ __attribute__((aligned(16))) short s_k[2][TE];
  __shared__ __attribute__((aligned(16))) short s_v[2][TE];
  __shared__ uint32_t s_bits[PF_WORDS];
  __shared__ uint16_t s_list[PF_LIST];
  __shared__ uint32_t s_need[4][PF_LIST / 32];    // per wave: the list entries its queries list
  // Set-up only, in value buffer 1 (first written by the first tile's prefetch, after the
  // set-up's last barrier): the list position of each bitmap word's first block, the list length.
  int* s_wpre = (int*)&s_v[1][0];
  int* s_nlist = s_wpre + PF_WORDS;
  static_assert((PF_WORDS + 1) * 4 <= TE * 2, "set-up tables fit one value buffer");
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int64_t b = blockIdx.z;
  const int h = blockIdx.y;
  const int64_t tw0 = (int64_t)blockIdx.x * 64;                // the workgroup's first query (< Lq)
  const int64_t tq0 = tw0 + wave * 16;                         // the wave's first query
  const bool qvalid = tq0 + c16 < a.Lq;
  const int64_t tq = qvalid ? tq0 + c16 : a.Lq - 1;            // extra columns repeat the last query
  const int64_t off = a.Lkv - a.Lq;
  const int pos = (int)(off + tq);   // key positions fit 32 bits: Lkv <= PF_WORDS * 32 * 64
  const int64_t wpos_lo = off + tw0;
  const int64_t wpos_hi = off + min(tw0 + 63, a.Lq - 1);

  pf16x8 qb[NP];   // lane (query c16, group g): dims 32 p + 8 g .. +7
#pragma unroll
  for (int p = 0; p < NP; ++p) qb[p] = *(const pf16x8*)(a.q + b * a.qsb + h * a.qsh + tq * a.qst + 32 * p + 8 * g);

  // gate weights of the lane's query
  const int64_t gb = b * a.gsb + h * a.gsh + tq * a.gst;
  float g0 = load_elem(a.gate, a.gdt, gb), g1 = load_elem(a.gate, a.gdt, gb + a.gsm),
        g2 = load_elem(a.gate, a.gdt, gb + 2 * a.gsm);
  {
    const float gm = fmaxf(g0, fmaxf(g1, g2));
    g0 = __expf(g0 - gm); g1 = __expf(g1 - gm); g2 = __expf(g2 - gm);
    const float gi = 1.f / (g0 + g1 + g2);
    g0 *= gi; g1 *= gi; g2 *= gi;
  }
  f32x4 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- the workgroup's tiles, in stream order: local (sink tiles below the first window
  // tile, then the window tiles of all 64 queries), sparse (the union of the 64 queries'
  // blocks, ascending), HCA (the means any of the 64 queries can see).
  const int64_t ns = min((int64_t)a.n_sink, a.Lkv);
  const int64_t lo = max((int64_t)0, wpos_lo - a.window + 1);
  const int64_t wt0 = (lo / 64) * 64;
  const int64_t sink_end = min(ns, wt0);
  const int n_st = (int)((sink_end + 63) / 64);
  const int n_loc = n_st + (wpos_hi >= wt0 ? (int)((wpos_hi - wt0) / 64 + 1) : 0);

  // this lane's share of its query's index slots, k = g + 4 r, two per register (slot 2 m in
  // the low half): the block, or 0xffff for an empty or out-of-range slot (blocks are below
  // PF_WORDS * 32 = 16384)
  uint32_t myblk[PF_MAXK / 8];
#pragma unroll
  for (int m = 0; m < PF_MAXK / 8; ++m) {
    uint32_t pr = 0u;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int kk = g + 4 * (2 * m + hf);
      const int64_t v = kk < a.K ? a.idx[b * a.isb + tq * a.ist + kk * a.isk] : -1;
      pr |= (uint32_t)((v >= 0 && v < a.nb) ? (int)v : 0xffff) << (16 * hf);
    }
    myblk[m] = pr;
  }
  const int64_t nbl = min(a.nb, wpos_hi / 64 + 1);   // blocks that hold a key <= wpos_hi
  const int nwords = (int)((nbl + 31) / 32);
  for (int wd = tid; wd < nwords; wd += 256) s_bits[wd] = 0u;
  __syncthreads();
  if (qvalid) {
#pragma unroll
    for (int r = 0; r < PF_MAXK / 4; ++r) {
      const int bk = (int)((myblk[r >> 1] >> (16 * (r & 1))) & 0xffffu);
      if (bk < nbl) atomicOr(&s_bits[bk >> 5], 1u << (bk & 31));
    }
  }
  __syncthreads();
  if (wave == 0) {   // compaction in ascending block order: word wd's set bits at base + (bits before it)
    int nlist = 0;
    for (int w0 = 0; w0 < nwords; w0 += 64) {
      const int wd = w0 + lane;
      const uint32_t word = wd < nwords ? s_bits[wd] : 0u;
      const int cnt = __popc(word);
      int incl = cnt;
#pragma unroll
      for (int o2 = 1; o2 < 64; o2 <<= 1) {
        const int y = __shfl_up(incl, o2);
        if (lane >= o2) incl += y;
      }
      int at = nlist + incl - cnt;
      if (wd < nwords) s_wpre[wd] = at;
      uint32_t rest = word;
      while (rest) {
        const int bit = __ffs(rest) - 1;
        s_list[at++] = (uint16_t)(wd * 32 + bit);
        rest &= rest - 1;
      }
      nlist += __shfl(incl, 63);
    }
    if (lane == 0) *s_nlist = nlist;
  }
  const int64_t e_hi = min(a.nc - 1, (wpos_hi + 1) / a.pool - 1);
  const int n_hca = e_hi >= 0 ? (int)(e_hi / 64 + 1) : 0;
  for (int wd = tid; wd < 4 * (PF_LIST / 32); wd += 256) (&s_need[0][0])[wd] = 0u;
  __syncthreads();
  const int n_sp = *s_nlist;
  if (qvalid) {   // mark the list entries of the lane's slots for its wave
#pragma unroll
    for (int r = 0; r < PF_MAXK / 4; ++r) {
      const int bk = (int)((myblk[r >> 1] >> (16 * (r & 1))) & 0xffffu);
      if (bk < nbl) {
        const int u = s_wpre[bk >> 5] + __popc(s_bits[bk >> 5] & ((1u << (bk & 31)) - 1u));
        atomicOr(&s_need[wave][u >> 5], 1u << (u & 31));
      }
    }
  }
  __syncthreads();
  const int n_ls = n_loc + n_sp;
  const int nt = n_ls + n_hca;

  // ---- tile staging: thread tid copies row tid / 4, 16-byte chunks (tid % 4) + 4 p, of the
  // key and value tiles; the next tile's loads are in flight while the current one computes.
  const uint16_t* kbase = a.k + b * a.ksb + h * a.ksh;
  const uint16_t* vbase = a.v + b * a.vsb + h * a.vsh;
  const uint16_t* khbase = a.kh ? a.kh + b * a.khb + h * a.khh : nullptr;
  const uint16_t* vhbase = a.vh ? a.vh + b * a.vhb + h * a.vhh : nullptr;
  const int srow = tid >> 2, spart = tid & 3;
  pf16x8 pk[NP], pv[NP];
  auto fetch = [&](int i) {
    const uint16_t* kr;
    const uint16_t* vr;
    if (i < n_ls) {
      const int64_t tb = i < n_st ? 64 * (int64_t)i
                       : i < n_loc ? wt0 + 64 * (int64_t)(i - n_st) : 64 * (int64_t)s_list[i - n_loc];
      const int64_t j = min(tb + srow, a.Lkv - 1);
      kr = kbase + j * a.kst;
      vr = vbase + j * a.vst;
    } else {
      const int64_t e = min(64 * (int64_t)(i - n_ls) + srow, a.nc - 1);
      kr = khbase + e * a.khe;
      vr = vhbase + e * a.vhe;
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      pk[p] = *(const pf16x8*)(kr + 8 * (spart + 4 * p));
      pv[p] = *(const pf16x8*)(vr + 8 * (spart + 4 * p));
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      *(pf16x8*)(s_k[buf] + srow * TP + 8 * (spart + 4 * p)) = pk[p];
      *(pf16x8*)(s_v[buf] + srow * TP + 8 * (spart + 4 * p)) = pv[p];
    }
  };

  // One 64-key tile from LDS buffer buf: the lane's rows with bit 4 rb + i of vmask set
  // (row 16 rb + 4 g + i) have weight fc, the others 0.  A wave none of whose queries weights
  // any row skips the tile: for such a lane the tile would leave (m, l, z) exactly as they
  // are.  Scores are scaled to log2 units (scale * log2 e) so that each probability is one
  // exp2; a tile whose 64 rows are valid for every lane of the wave skips the masking.
  const float sl2 = a.scale * 1.4426950408889634f;
  auto tile = [&](PfAcc<NDT>& st, int buf, float fc, uint32_t vmask) {
    if (!qvalid || !(fc > 0.f)) vmask = 0u;
    if (__ballot(vmask != 0u) == 0ull) return;   // wave-uniform
    const bool full = __ballot(qvalid && vmask != 0xffffu) == 0ull;
    const short* ks = s_k[buf];
    const short* vt = s_v[buf];
    f32x4 sc[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const pf16x8 kv = *(const pf16x8*)(ks + (16 * rb + c16) * TP + 32 * p + 8 * g);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kv),
                                                      __builtin_bit_cast(bf16x8, qb[p]), acc, 0, 0, 0);
      }
      sc[rb] = acc;
    }
    // lane (query c16, g) holds the scores of keys 16 rb + 4 g + i
    float tmax = -INFINITY;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = (full || ((vmask >> (4 * rb + i)) & 1u)) ? sc[rb][i] * sl2 : -INFINITY;
        sc[rb][i] = x;
        tmax = fmaxf(tmax, x);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(st.m, tmax);
    const float corr = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(st.m - m_new);
    const float m_sub = (m_new == -INFINITY) ? 0.f : m_new;
    float psum = 0.f;
    i16x4 ph[4], pl[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      f32x4 pe;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pe[i] = fc * __builtin_amdgcn_exp2f(sc[rb][i] - m_sub);   // exp2(-inf) = 0 for masked keys
        psum += pe[i];
      }
      split4(pe, ph[rb], pl[rb]);
    }
    psum += __shfl_xor(psum, 16);
    psum += __shfl_xor(psum, 32);
    st.l = st.l * corr + psum;
    st.m = m_new;
    // O^T[dim][query] = corr O^T + V^T P over the 64 keys as two 32-key steps whose key order
    // (16 rb + 4 g + i, rb in {2 p2, 2 p2 + 1}) matches the probabilities this lane holds
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      f32x4 acc = st.z[dt] * corr;
#pragma unroll
      for (int p2 = 0; p2 < 2; ++p2) {
        const pf16x4 a0 = pf_ldsT4(vt, TP, 32 * p2, 16 * dt, c16, g);
        const pf16x4 a1 = pf_ldsT4(vt, TP, 32 * p2 + 16, 16 * dt, c16, g);
        const pf16x8 av = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        const i16x8 bh = cat8(ph[2 * p2], ph[2 * p2 + 1]), bl = cat8(pl[2 * p2], pl[2 * p2 + 1]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bh),
                                                      acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bl),
                                                      acc, 0, 0, 0);
      }
      st.z[dt] = acc;
    }
  };
  auto reset = [&](PfAcc<NDT>& st) {
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) st.z[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  auto fold = [&](const PfAcc<NDT>& st, float gs) {   // o += g_s z_s / l_s
    const float w = st.l > 0.f ? gs / st.l : 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] += st.z[dt] * w;
  };
  // tiles [i, i_end): prefetch tile i + 1 (of whichever stream), compute tile i, stage the
  // prefetched tile into the other buffer, one barrier per tile.  weight_of(i) gives tile i's
  // weight for the lane's query and mask_of(i) its row mask (pf_range_bits).
  int i = 0;
  auto run = [&](PfAcc<NDT>& st, int i_end, auto weight_of, auto mask_of) {
    for (; i < i_end; ++i) {
      if (i + 1 < nt) fetch(i + 1);
      const float fc = weight_of(i);
      tile(st, i & 1, fc, fc > 0.f ? mask_of(i) : 0u);
      if (i + 1 < nt) stash((i + 1) & 1);
      __syncthreads();
    }
  };
  if (nt > 0) {
    fetch(0);
    stash(0);
  }
  __syncthreads();
  PfAcc<NDT> st;

  // ---- local stream: sink tiles hold keys [0, min(sink_end, pos + 1)); window tiles the keys
  // in (pos - window, pos] and the sinks below min(ns, pos + 1)
  reset(st);
  run(st, n_loc, [](int) { return 1.f; }, [&](int ti) {
    if (ti < n_st) return pf_range_bits(-64 * ti, min((int)sink_end - 1, pos) - 64 * ti, g);
    const int tb = (int)wt0 + 64 * (ti - n_st);
    return pf_range_bits(pos - a.window + 1 - tb, pos - tb, g) |
           pf_range_bits(-tb, min((int)ns - 1, pos) - tb, g);
  });
  fold(st, g0);

  // ---- sparse stream: each key weighted by how often the lane's query lists its block; a
  // wave skips the entries none of its queries lists without counting
  reset(st);
  run(st, n_ls, [&](int ti) {
    const int u = ti - n_loc;
    if (((s_need[wave][u >> 5] >> (u & 31)) & 1u) == 0u) return 0.f;   // wave-uniform
    const int blk = s_list[u];
    int cnt = 0;
#pragma unroll
    for (int m = 0; m < PF_MAXK / 8; ++m)
      cnt += (int)((myblk[m] & 0xffffu) == (uint32_t)blk) + (int)((myblk[m] >> 16) == (uint32_t)blk);
    cnt += __shfl_xor(cnt, 16);
    cnt += __shfl_xor(cnt, 32);
    return (float)cnt;
  }, [&](int ti) { return pf_range_bits(0, pos - 64 * (int)s_list[ti - n_loc], g); });
  fold(st, g1);

  // ---- HCA stream: means e <= e_max, the last complete block's mean before the lane's query;
  // early queries take their row
  reset(st);
  const int e_max = (int)min(a.nc - 1, (int64_t)((pos + 1) / a.pool) - 1);
  run(st, nt, [](int) { return 1.f; }, [&](int ti) { return pf_range_bits(0, e_max - 64 * (ti - n_ls), g); });
  if (pos < a.pool - 1) {   // running mean of c[0..pos] through W_v (the caller's row)
    const bool have = a.early && tq < a.n_early;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int i2 = 0; i2 < 4; ++i2) {
        const int d = 16 * dt + 4 * g + i2;
        const float x = have ? load_elem(a.early, a.edt, b * a.esb + h * a.esh + tq * a.est + d * a.esd) : 0.f;
        o[dt][i2] += g2 * x;
      }
  } else {
    fold(st, g2);
  }

  if (!qvalid) return;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    const int64_t oo = b * a.osb + h * a.osh + tq * a.ost + 16 * dt + 4 * g;
    if (a.odt == MABA_F32) {
      *(f32x4*)((float*)a.out + oo) = o[dt];
    } else {
      uint2 u;
      u.x = (uint32_t)f32_to_bf16_bits(o[dt][0]) | ((uint32_t)f32_to_bf16_bits(o[dt][1]) << 16);
      u.y = (uint32_t)f32_to_bf16_bits(o[dt][2]) | ((uint32_t)f32_to_bf16_bits(o[dt][3]) << 16);
      *(uint2*)((uint16_t*)a.out + oo) = u;
    }
  }
}

static bool pf_rows_ok(const maba_tensor* t, int64_t B, int64_t H, int64_t n, int64_t dh) {
  if (!t || t->ndim != 4 || t->dtype != MABA_BF16) return false;
  if (t->shape[0] != B || t->shape[1] != H || t->shape[2] != n || t->shape[3] != dh) return false;
  if (t->stride[3] != 1 || (uintptr_t)t->data % 16 != 0) return false;
  for (int d = 0; d < 3; ++d)
    if (t->shape[d] > 1 && t->stride[d] % 8 != 0) return false;
  return true;
}

}  // namespace maba

using namespace maba;

extern "C" int maba_hip_maba_sa_prefill(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                                        const maba_tensor* kh, const maba_tensor* vh,
                                        const maba_tensor* early, const maba_tensor* idx,
                                        const maba_tensor* gate, float scale, int window, int n_sink,
                                        int block_size, int pool, maba_tensor* out, void* stream) {
  if (!q || q->ndim != 4) return fail(MABA_ERR_INVALID, "maba_sa_prefill: q must be [B,H,Lq,dh]");
  const int64_t B = q->shape[0], H = q->shape[1], Lq = q->shape[2], dh = q->shape[3];
  if (!k || k->ndim != 4 || !v || v->ndim != 4)
    return fail(MABA_ERR_INVALID, "maba_sa_prefill: k and v must be [B,H,Lkv,dh]");
  const int64_t Lkv = k->shape[2];
  if (Lq > Lkv) return fail(MABA_ERR_INVALID, "maba_sa_prefill: more queries than keys");
  if (window < 0 || n_sink < 0 || pool <= 0) return fail(MABA_ERR_INVALID, "maba_sa_prefill: bad window/sink/pool");
  if (block_size != 64) return fail(MABA_ERR_UNSUPPORTED, "maba_sa_prefill: block_size 64 only");
  if (dh != 32 && dh != 64 && dh != 128) return fail(MABA_ERR_UNSUPPORTED, "maba_sa_prefill: dh in {32, 64, 128}");
  if (!pf_rows_ok(q, B, H, Lq, dh) || !pf_rows_ok(k, B, H, Lkv, dh) || !pf_rows_ok(v, B, H, Lkv, dh))
    return fail(MABA_ERR_UNSUPPORTED, "maba_sa_prefill: q, k, v must be bf16 with unit channel stride and "
                "16-byte aligned rows");
  const int64_t nc = Lkv / pool;
  if (nc > 0 && (!pf_rows_ok(kh, B, H, nc, dh) || !pf_rows_ok(vh, B, H, nc, dh)))
    return fail(MABA_ERR_UNSUPPORTED, "maba_sa_prefill: kh, vh must be bf16 [B,H,Lkv/pool,dh], unit channel stride");
  const int64_t off = Lkv - Lq;
  const int64_t n_early = off < pool - 1 ? std::min(Lq, (int64_t)(pool - 1) - off) : 0;
  if (n_early > 0) {
    const int64_t se[4] = {B, H, n_early, dh};
    if (!expect_shape(early, "early", 4, se) || !expect_float(early, "early")) return MABA_ERR_INVALID;
  }
  if (!idx || idx->ndim != 3 || idx->shape[0] != B || (idx->shape[1] != Lq && idx->shape[1] != 1))
    return fail(MABA_ERR_INVALID, "maba_sa_prefill: idx must be [B,Lq|1,K]");
  if (idx->dtype != MABA_I64) return fail(MABA_ERR_DTYPE, "maba_sa_prefill: idx must be int64");
  const int64_t K = idx->shape[2];
  if (K > PF_MAXK) return fail(MABA_ERR_UNSUPPORTED, "maba_sa_prefill: at most %d index slots", PF_MAXK);
  const int64_t nb = (Lkv + 63) / 64;
  if (nb > (int64_t)PF_WORDS * 32) return fail(MABA_ERR_UNSUPPORTED, "maba_sa_prefill: Lkv up to %d", PF_WORDS * 32 * 64);
  if (!gate || !((gate->ndim == 3 && gate->shape[0] == B && gate->shape[1] == Lq && gate->shape[2] == 3) ||
                 (gate->ndim == 4 && gate->shape[0] == B && gate->shape[1] == H && gate->shape[2] == Lq &&
                  gate->shape[3] == 3)))
    return fail(MABA_ERR_INVALID, "maba_sa_prefill: gate must be [B,Lq,3] or [B,H,Lq,3]");
  if (!expect_float(gate, "gate")) return MABA_ERR_DTYPE;
  const int64_t so[4] = {B, H, Lq, dh};
  if (!expect_shape(out, "out", 4, so)) return MABA_ERR_INVALID;
  if ((out->dtype != MABA_F32 && out->dtype != MABA_BF16) || out->stride[3] != 1 ||
      (uintptr_t)out->data % 16 != 0 || out->stride[0] % 4 != 0 || out->stride[1] % 4 != 0 ||
      out->stride[2] % 4 != 0)
    return fail(MABA_ERR_UNSUPPORTED, "maba_sa_prefill: out must be f32/bf16 with unit channel stride");
  if (B * H * Lq == 0) return MABA_OK;
  PfArgs a;
  a.q = (const uint16_t*)q->data; a.qsb = q->stride[0]; a.qsh = q->stride[1]; a.qst = q->stride[2];
  a.k = (const uint16_t*)k->data; a.ksb = k->stride[0]; a.ksh = k->stride[1]; a.kst = k->stride[2];
  a.v = (const uint16_t*)v->data; a.vsb = v->stride[0]; a.vsh = v->stride[1]; a.vst = v->stride[2];
  a.kh = nc > 0 ? (const uint16_t*)kh->data : nullptr;
  a.khb = nc > 0 ? kh->stride[0] : 0; a.khh = nc > 0 ? kh->stride[1] : 0; a.khe = nc > 0 ? kh->stride[2] : 0;
  a.vh = nc > 0 ? (const uint16_t*)vh->data : nullptr;
  a.vhb = nc > 0 ? vh->stride[0] : 0; a.vhh = nc > 0 ? vh->stride[1] : 0; a.vhe = nc > 0 ? vh->stride[2] : 0;
  a.early = n_early > 0 ? early->data : nullptr; a.edt = n_early > 0 ? early->dtype : MABA_F32;
  a.esb = n_early > 0 ? early->stride[0] : 0; a.esh = n_early > 0 ? early->stride[1] : 0;
  a.est = n_early > 0 ? early->stride[2] : 0; a.esd = n_early > 0 ? early->stride[3] : 0;
  a.idx = (const int64_t*)idx->data; a.isb = idx->stride[0];
  a.ist = idx->shape[1] == 1 ? 0 : idx->stride[1]; a.isk = idx->stride[2];
  a.gate = gate->data; a.gdt = gate->dtype; a.gsb = gate->stride[0];
  if (gate->ndim == 3) { a.gsh = 0; a.gst = gate->stride[1]; a.gsm = gate->stride[2]; }
  else { a.gsh = gate->stride[1]; a.gst = gate->stride[2]; a.gsm = gate->stride[3]; }
  a.out = out->data; a.odt = out->dtype; a.osb = out->stride[0]; a.osh = out->stride[1]; a.ost = out->stride[2];
  a.Lq = Lq; a.Lkv = Lkv; a.nc = nc; a.n_early = n_early; a.nb = nb;
  a.K = (int)K; a.window = window; a.n_sink = n_sink; a.pool = pool; a.scale = scale;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)ceil_div(Lq, 64), (unsigned)H, (unsigned)B);
  switch (dh) {
    case 32: hipLaunchKernelGGL(maba_sa_prefill_kernel<1>, grid, dim3(256), 0, s, a); break;
    case 64: hipLaunchKernelGGL(maba_sa_prefill_kernel<2>, grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(maba_sa_prefill_kernel<4>, grid, dim3(256), 0, s, a); break;
  }
  return check_launch("maba_sa_prefill");
}

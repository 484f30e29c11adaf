// DG-Indexer scoring + top-k.
//
// Decode (reference: maba_sparse/layers/indexer.py:101-112):
//   s[h,n] = (q_h / sqrt(d)) . c_n - lam * log1p(max(nb-1-n, 0))   (no mask)
//   idx[h] = top min(K, nb) of s[h,:], score descending, ties -> lower index
// Prefill (reference: maba_sparse/kernels/cpu_indexer.py:91-108):
//   s[t,n] = (q_t / sqrt(d)) . c_n - lam * log1p(|t//bs - n|), -inf if n > t//bs
//
// Scores are fp32 dots of the stored inputs (bf16/f16/f32 converted exactly
// to fp32).  The decode path streams the centroid set once per batch element:
// each wave scores a 64-centroid tile for every query head (lane = centroid)
// and folds it into per-head running top-64 lists (topk_wave.h); workgroup
// results go to a workspace and a second kernel merges the splits.
#include "maba_common.h"
#include "topk_wave.h"
#include <type_traits>

namespace maba {

constexpr int IDX_MAX_HEADS = 16;   // query heads per decode launch
constexpr int IDX_MAX_D = 256;      // channels

struct DecArgs {
  const void* q; int qdt; int64_t qsb, qsh, qsd;
  const void* c; int cdt; int64_t csb, csn, csd;
  int64_t nb, d;
  int Hq, K, nsplit, tiles_per_wave;
  float scale, lam;
  key64* ws;                           // [B, nsplit, Hq, 64]
  float* scores; int64_t ssb, ssh, ssn; // optional fp32 scores
};

__global__ __launch_bounds__(256) void index_decode_score_kernel(DecArgs a) {
  __shared__ float s_q[IDX_MAX_HEADS * IDX_MAX_D];
  __shared__ key64 s_lists[4][64];
  const int split = blockIdx.x;
  const int64_t bi = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int Hq = a.Hq;
  const int64_t d = a.d;
  for (int64_t i = threadIdx.x; i < (int64_t)Hq * d; i += 256) {
    const int h = (int)(i / d);
    const int64_t c = i % d;
    s_q[h * IDX_MAX_D + c] = load_elem(a.q, a.qdt, bi * a.qsb + h * a.qsh + c * a.qsd) * a.scale;
  }
  __syncthreads();

  key64 list[IDX_MAX_HEADS];
#pragma unroll
  for (int h = 0; h < IDX_MAX_HEADS; ++h) list[h] = KEY_NONE;

  const int64_t tile0 = ((int64_t)split * 4 + wave) * a.tiles_per_wave;
  for (int tt = 0; tt < a.tiles_per_wave; ++tt) {
    const int64_t n = (tile0 + tt) * 64 + lane;
    const bool valid = n < a.nb;
    float acc[IDX_MAX_HEADS];
#pragma unroll
    for (int h = 0; h < IDX_MAX_HEADS; ++h) acc[h] = 0.f;
    if (valid) {
      const int64_t cb = bi * a.csb + n * a.csn;
      for (int64_t c = 0; c < d; ++c) {
        const float x = load_elem(a.c, a.cdt, cb + c * a.csd);
#pragma unroll
        for (int h = 0; h < IDX_MAX_HEADS; ++h)
          if (h < Hq) acc[h] = fmaf(s_q[h * IDX_MAX_D + c], x, acc[h]);
      }
    }
    const float pen = valid ? a.lam * fast_log(1.f + (float)(a.nb - 1 - n)) : 0.f;
    if (__ballot(valid) == 0ull) break;
#pragma unroll
    for (int h = 0; h < IDX_MAX_HEADS; ++h) {
      if (h < Hq) {
        const float s = acc[h] - pen;
        if (a.scores && valid) a.scores[bi * a.ssb + h * a.ssh + n * a.ssn] = s;
        const key64 key = valid ? make_key(s, (uint32_t)n) : KEY_NONE;
        list[h] = wave_merge_topk(list[h], key, a.K);
      }
    }
  }
  // merge the 4 wave lists per head, write the workgroup's top-64
#pragma unroll
  for (int h = 0; h < IDX_MAX_HEADS; ++h) {
    if (h < Hq) {  // uniform across the workgroup
      s_lists[wave][lane] = list[h];
      __syncthreads();
      if (wave == 0) {
        key64 m = s_lists[0][lane];
        for (int w = 1; w < 4; ++w) m = wave_merge_topk(m, s_lists[w][lane], a.K);
        a.ws[(((int64_t)bi * a.nsplit + split) * Hq + h) * 64 + lane] = m;
      }
      __syncthreads();
    }
  }
}

__global__ __launch_bounds__(64) void index_decode_merge_kernel(const key64* ws, int nsplit, int Hq, int K,
                                                                int ak, int64_t* out, int64_t osb,
                                                                int64_t osh, int64_t osk) {
  const int64_t bi = blockIdx.x / Hq;
  const int h = blockIdx.x % Hq;
  const int lane = threadIdx.x;
  key64 m = KEY_NONE;
  for (int s = 0; s < nsplit; ++s) m = wave_merge_topk(m, ws[((bi * nsplit + s) * Hq + h) * 64 + lane], K);
  if (lane < ak) out[bi * osb + h * osh + lane * osk] = (int64_t)key_index(m);
}

// Decode on MFMA (bf16 q and centroids, d a multiple of 32, <= 256), two launches.
//
// index_decode_tile_kernel -- one wave per 64-centroid tile: D = C x Q^T with
//   v_mfma_f32_16x16x32_bf16 (A: centroid rows straight from global memory, B:
//   the queries, heads padded to 16, in registers).  bf16 x bf16 products are
//   exact and accumulate in fp32.  Writes every score to a workspace row per
//   (b, head) and the tile's best key per head.
// index_decode_select_kernel -- one 1024-thread workgroup per (b, head).  The tile
//   maxima are folded into 64 groups; tau = the K-th largest group maximum bounds
//   the K-th largest key from below (K groups each hold a key >= tau), so the top
//   K are among the keys >= tau: collect those (typically a few dozen to a few
//   hundred) into one list, rank them by counting, write ranks < K.  With more than
//   SEL_CAP of them (heavily tied scores) the workgroup falls back to wave top-k
//   merges over the whole row.
typedef __attribute__((ext_vector_type(8))) short i16x8_t;
constexpr int SEL_CAP = 1024;     // candidate slots of the select kernel
constexpr int SEL_GROUPS = 64;    // tile maxima are folded into this many groups
constexpr int SEL_T = 1024;       // threads of the select kernel (16 waves)
constexpr int SEL_W = SEL_T / 64;
constexpr int SEL_V = 4;          // float4 score loads in flight per thread in the select kernel
constexpr int SEL_PASS = SEL_T * SEL_V * 4;   // scores per pass

struct DecTileArgs {
  const uint16_t* q; int64_t qsb, qsh;   // [B, Hq, d] bf16, channel stride 1
  const uint16_t* c; int64_t csb, csn;   // [B, nb, d] bf16, channel stride 1
  int64_t nb;
  int ntiles, Hq;                         // ntiles: the workspace rows' tile capacity
  const int64_t* dlen; int bs;            // device sequence length: nb = ceil(*dlen / bs) (null: nb as given)
  float scale, lam;
  float* sc;                              // [B, Hq, ntiles * 64] workspace scores
  key64* tmax;                            // [B, Hq, ntiles] best key per tile
  float* scores; int64_t ssb, ssh, ssn;   // optional caller scores [B, Hq, nb]
};

template <int NP>  // NP = d / 32
__global__ __launch_bounds__(256) void index_decode_tile_kernel(DecTileArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int tile = blockIdx.x * 4 + wave;
  const int64_t bi = blockIdx.y;
  // a device length never reaches past the capacity the buffers were sized for
  const int64_t nb = a.dlen ? min((*a.dlen + a.bs - 1) / a.bs, a.nb) : a.nb;
  if ((int64_t)tile * 64 >= nb) return;  // wave-uniform; the kernel has no barrier
  const int64_t n0 = (int64_t)tile * 64;
  const uint16_t* cb = a.c + bi * a.csb;
  // all centroid loads of the tile first: lane (c16, g) reads row 16 rb + c16, dims 32 p + 8 g .. +7
  i16x8_t av[4][NP];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int64_t n = n0 + 16 * rb + c16;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      i16x8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
      if (n < nb) z = *(const i16x8_t*)(cb + n * a.csn + 32 * p + 8 * g);
      av[rb][p] = z;
    }
  }
  i16x8_t qb[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    i16x8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
    if (c16 < a.Hq) z = *(const i16x8_t*)(a.q + bi * a.qsb + c16 * a.qsh + 32 * p + 8 * g);
    qb[p] = z;
  }
  const bool hv = c16 < a.Hq;
  float* srow = a.sc + (bi * a.Hq + c16) * (int64_t)a.ntiles * 64 + n0;
  key64 best = KEY_NONE;
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < NP; ++p)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[rb][p]),
                                                    __builtin_bit_cast(bf16x8, qb[p]), acc, 0, 0, 0);
    // lane holds D[centroid n0 + 16 rb + 4 g + i][head c16]
    f32x4 sv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t n = n0 + 16 * rb + 4 * g + i;
      float sc = -INFINITY;
      if (n < nb) {
        // log1p(m) = log(1 + m) with 1 + m exact for integer block distances m < 2^24
        sc = acc[i] * a.scale - a.lam * fast_log(1.f + (float)(nb - 1 - n));
        best = kmax(best, make_key(sc, (uint32_t)n));
        if (hv && a.scores) a.scores[bi * a.ssb + c16 * a.ssh + n * a.ssn] = sc;
      }
      sv[i] = sc;
    }
    if (hv) *(f32x4*)(srow + 16 * rb + 4 * g) = sv;
  }
  best = kmax(best, __shfl_xor(best, 16));
  best = kmax(best, __shfl_xor(best, 32));
  if (hv && g == 0) a.tmax[(bi * a.Hq + c16) * a.ntiles + tile] = best;
}

// Number of keys in s[0, n8) greater than k; n8 is a multiple of 8 and s 16-byte
// aligned.  Eight keys per step through 128-bit LDS reads, all lanes reading the
// same address (broadcast).
__device__ __forceinline__ int count_greater(const key64* s, int n8, key64 k) {
  typedef __attribute__((ext_vector_type(2))) unsigned long long u64x2;
  int r = 0;
  for (int i = 0; i < n8; i += 8) {
    const u64x2 x0 = *(const u64x2*)(s + i), x1 = *(const u64x2*)(s + i + 2);
    const u64x2 x2 = *(const u64x2*)(s + i + 4), x3 = *(const u64x2*)(s + i + 6);
    r += (x0.x > k) + (x0.y > k) + (x1.x > k) + (x1.y > k) + (x2.x > k) + (x2.y > k) + (x3.x > k) + (x3.y > k);
  }
  return r;
}

struct DecSelArgs {
  const float* sc; const key64* tmax;
  int64_t nb;
  int ntiles, Hq, K, ak;                  // ntiles: the workspace rows' tile capacity
  const int64_t* dlen; int bs;            // as in DecTileArgs
  int64_t* out; int64_t osb, osh, osk;
};

__device__ __forceinline__ key64 readlane64(key64 x, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), lane);
  return ((key64)hi << 32) | lo;
}

// Number of keys in s[0, 16) greater than k (s 16-byte aligned; broadcast reads, unrolled).
__device__ __forceinline__ int count_greater16(const key64* s, key64 k) {
  typedef __attribute__((ext_vector_type(2))) unsigned long long u64x2;
  int r = 0;
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    const u64x2 x = *(const u64x2*)(s + i);
    r += (x.x > k) + (x.y > k);
  }
  return r;
}

__device__ __forceinline__ int lane_rank(unsigned long long m) {   // set bits of m below this lane
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__global__ __launch_bounds__(SEL_T) void index_decode_select_kernel(DecSelArgs a) {
  __shared__ __attribute__((aligned(16))) key64 s_c[SEL_T];          // the fallback's wave lists
  __shared__ __attribute__((aligned(16))) key64 s_k[SEL_CAP + 8];   // the candidate list
  __shared__ __attribute__((aligned(16))) key64 s_g[SEL_GROUPS];
  __shared__ key64 s_part[SEL_T];
  __shared__ int s_rank[4][64];
  __shared__ int s_cnt;
  __shared__ key64 s_tau;
  const int64_t row = blockIdx.x;  // b * Hq + h
  const int64_t bi = row / a.Hq;
  const int h = (int)(row % a.Hq);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t nb = a.dlen ? min((*a.dlen + a.bs - 1) / a.bs, a.nb) : a.nb;   // clamped to the capacity
  const int ntl = (int)((nb + 63) / 64);                 // tiles holding centroids
  const int ak = (int)(a.K < nb ? a.K : nb);
  const key64* tm = a.tmax + row * a.ntiles;
  const float* sc = a.sc + row * (int64_t)a.ntiles * 64;
  // first pass of score loads, issued before the tile maxima so that both are in flight
  // together.  Vectors past the row's end read as -inf, like the row's padding.
  f32x4 v[SEL_V];
#pragma unroll
  for (int j = 0; j < SEL_V; ++j) {
    const int64_t n = 4 * (SEL_T * j + tid);
    f32x4 z = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    if (n < nb) z = *(const f32x4*)(sc + n);
    v[j] = z;
  }
  if (tid < 64) s_k[tid] = KEY_NONE;   // list slots the final rank reads past cnt
  if (tid == 0) s_cnt = 0;
  // tile maxima: thread t folds tiles t, t + SEL_T, ...; group j < 64 is the tiles
  // t = j (mod 64), i.e. lane j of every wave (any partition of the tiles gives a valid bound)
  key64 m = KEY_NONE;
  for (int t = tid; t < ntl; t += SEL_T) m = kmax(m, tm[t]);
  s_part[tid] = m;
  __syncthreads();
  // tau = K-th largest group maximum (keys are distinct; empty groups hold KEY_NONE):
  // wave w < 4 counts the group maxima in slots [16 w, 16 w + 16) above group `lane`'s
  if (wave == 0) {
    key64 gm = s_part[lane];
#pragma unroll
    for (int w = 1; w < SEL_W; ++w) gm = kmax(gm, s_part[64 * w + lane]);
    s_g[lane] = gm;
  }
  __syncthreads();
  const key64 gm = s_g[lane];
  if (wave < 4) s_rank[wave][lane] = count_greater16(s_g + 16 * wave, gm);
  __syncthreads();
  if (wave == 0) {
    const int G = ntl < SEL_GROUPS ? ntl : SEL_GROUPS;   // groups j < G hold a tile
    key64 tau = KEY_NONE;
    if (G >= a.K) {
      const int rank = s_rank[0][lane] + s_rank[1][lane] + s_rank[2][lane] + s_rank[3][lane];
      const unsigned long long bal = __ballot(lane < G && rank == a.K - 1);
      tau = readlane64(gm, __builtin_ctzll(bal));
    }
    if (lane == 0) s_tau = tau;
  }
  __syncthreads();
  const key64 tau = s_tau;
  // Candidates: keys whose score is not below tau's score.  They include every key >= tau
  // (key order is score order first); the extra ones (equal score, larger index) rank
  // below all K keys >= tau and are never written.  With fewer groups than K
  // (tau = KEY_NONE) every key n < nb is a candidate.  A wave appends a batch of taken
  // keys to the shared list at an offset reserved with one LDS atomic (the list order
  // does not matter: ranking is by counting), so candidates clustered in one part of the
  // row (the distance penalty favours the newest blocks) fill the list like spread ones.
  // A vector no lane of the wave takes costs one max and one compare.
  const bool all = tau == KEY_NONE;
  const float tau_s = key_score(tau);
  auto scan = [&](auto all_c) {
    constexpr bool ALL = decltype(all_c)::value;
    for (int64_t base = 0; base < nb; base += SEL_PASS) {
      if (base > 0) {
#pragma unroll
        for (int j = 0; j < SEL_V; ++j) {
          const int64_t n = base + 4 * (SEL_T * j + tid);
          f32x4 z = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
          if (n < nb) z = *(const f32x4*)(sc + n);
          v[j] = z;
        }
      }
      const int64_t n0 = base + 4 * tid;
#pragma unroll
      for (int j = 0; j < SEL_V; ++j) {
        const f32x4 x = v[j];
        if (ALL) {
          if (__ballot(n0 + 4 * SEL_T * j < nb) == 0ull) continue;
        } else {
          const float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
          if (__ballot(!(mx < tau_s)) == 0ull) continue;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t n = n0 + 4 * SEL_T * j + i;
          const bool t = ALL ? n < nb : !(x[i] < tau_s);
          const unsigned long long b = __ballot(t);
          if (b == 0ull) continue;
          int at = 0;
          if (lane == 0) at = atomicAdd(&s_cnt, __builtin_popcountll(b));
          at = __builtin_amdgcn_readfirstlane(at);
          const int p = at + lane_rank(b);
          if (t && p < SEL_CAP) s_k[p] = make_key(x[i], (uint32_t)n);
        }
      }
    }
  };
  if (all) scan(std::true_type{}); else scan(std::false_type{});
  __syncthreads();
  const int cnt = s_cnt;
  int64_t* orow = a.out + bi * a.osb + h * a.osh;
  if (cnt <= SEL_CAP && cnt >= ak) {
    if (cnt <= 64) {  // rank across the four waves; slots past cnt hold KEY_NONE
      const key64 kj = s_k[lane];
      if (wave < 4) s_rank[wave][lane] = count_greater16(s_k + 16 * wave, kj);
      __syncthreads();
      if (wave == 0) {
        const int rank = s_rank[0][lane] + s_rank[1][lane] + s_rank[2][lane] + s_rank[3][lane];
        if (lane < cnt && rank < ak) orow[rank * a.osk] = (int64_t)key_index(kj);
      }
      return;
    }
    const int c8 = (cnt + 7) & ~7;
    if (tid < c8 - cnt) s_k[cnt + tid] = KEY_NONE;   // pad to whole groups of 8
    __syncthreads();
    for (int j = tid; j < cnt; j += SEL_T) {
      const key64 kj = s_k[j];
      const int rank = count_greater(s_k, c8, kj);
      if (rank < ak) orow[rank * a.osk] = (int64_t)key_index(kj);
    }
    return;
  }
  // fallback: each wave merges every SEL_W-th 64-key slice of the row, newest slice first
  // (the distance penalty favours recent blocks, so the list fills with its best keys at
  // once and older slices are rejected by the merge's K-th-key test), then wave 0 merges
  // the SEL_W lists
  key64 list = KEY_NONE;
  const int64_t nsl = (nb + 63) / 64;
  for (int64_t sl = nsl - 1 - wave; sl >= 0; sl -= SEL_W) {
    const int64_t n = sl * 64 + lane;
    const key64 key = n < nb ? make_key(sc[n], (uint32_t)n) : KEY_NONE;
    list = wave_merge_topk(list, key >= tau ? key : KEY_NONE, a.K);
  }
  __syncthreads();
  s_c[wave * 64 + lane] = list;
  __syncthreads();
  if (wave == 0) {
    key64 m = s_c[lane];
    for (int w = 1; w < SEL_W; ++w) m = wave_merge_topk(m, s_c[w * 64 + lane], a.K);
    if (lane < ak) orow[lane * a.osk] = (int64_t)key_index(m);
  }
}

// Prefill on MFMA (bf16 q and centroids, d = 32 NP, unit channel stride, no score
// output): one workgroup per 16 consecutive query rows of one sequence.  Wave w
// scores 64-centroid tiles for all 16 rows with v_mfma_f32_16x16x32_bf16 (A: the
// centroid rows from global memory, B: the 16 query rows in registers), round by
// round, newest tiles first, and the scores pass through LDS to the owners of the
// per-row top-K lists: wave w keeps rows 4w..4w+3 (one key per lane each) and merges
// each tile into them with wave_merge_topk, whose early exit skips tiles that cannot
// beat the K-th key.  Scores and causal mask as index_prefill_kernel.
struct PreMfmaArgs {
  const uint16_t* q; int64_t qsb, qsl;    // [B, L, d] bf16, channel stride 1
  const uint16_t* c; int64_t csb, csn;    // [B, nb, d] bf16, channel stride 1
  int64_t L, nb;
  int K, ak, bs;
  float scale, lam;
  int64_t* out; int64_t osb, osl, osk;
};

template <int NP>
__global__ __launch_bounds__(256) void index_prefill_mfma_kernel(PreMfmaArgs a) {
  constexpr int SP = 68;                                   // float pitch of a tile row in LDS
  __shared__ __attribute__((aligned(16))) float s_sc[4][16][SP];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int64_t bi = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * 16;
  const uint16_t* cb = a.c + bi * a.csb;
  // query rows t0 + c16 as the B operand (rows past L read as zero)
  i16x8_t qb[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    i16x8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
    if (t0 + c16 < a.L) z = *(const i16x8_t*)(a.q + bi * a.qsb + (t0 + c16) * a.qsl + 32 * p + 8 * g);
    qb[p] = z;
  }
  // causal limits: row t sees blocks n < nvalid(t) = min(t / bs + 1, nb)
  auto nvalid = [&](int64_t t) { const int64_t v = t / a.bs + 1; return v < a.nb ? v : a.nb; };
  const int64_t tlast = (t0 + 15 < a.L ? t0 + 15 : a.L - 1);
  const int ntiles = (int)((nvalid(tlast) + 63) / 64);
  key64 list[4] = {KEY_NONE, KEY_NONE, KEY_NONE, KEY_NONE};   // rows 4 wave + r
  for (int r0 = ntiles - 1; r0 >= 0; r0 -= 4) {                // tiles r0, r0-1, r0-2, r0-3
    const int tile = r0 - wave;
    if (tile >= 0) {
      const int64_t n0 = (int64_t)tile * 64;
      f32x4 acc[4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        const int64_t n = n0 + 16 * rb + c16;
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          i16x8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
          if (n < a.nb) z = *(const i16x8_t*)(cb + n * a.csn + 32 * p + 8 * g);
          s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, z), __builtin_bit_cast(bf16x8, qb[p]),
                                                       s, 0, 0, 0);
        }
        acc[rb] = s;
      }
      // lane holds D[centroid n0 + 16 rb + 4 g + i][row t0 + c16]
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) *(f32x4*)&s_sc[wave][c16][16 * rb + 4 * g] = acc[rb] * a.scale;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t t = t0 + 4 * wave + r;
      const int64_t nv = nvalid(t < a.L ? t : a.L - 1);
      const int64_t qblk = (t < a.L ? t : a.L - 1) / a.bs;
      for (int j = 0; j < 4 && r0 - j >= 0; ++j) {
        const int64_t n = (int64_t)(r0 - j) * 64 + lane;
        key64 key = KEY_NONE;
        if (n < nv) key = make_key(s_sc[j][4 * wave + r][lane] - a.lam * fast_log(1.f + (float)(qblk - n)), (uint32_t)n);
        list[r] = wave_merge_topk(list[r], key, a.K);
      }
    }
    __syncthreads();   // the next round overwrites the score tiles
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t t = t0 + 4 * wave + r;
    if (t >= a.L) break;
    // fewer valid blocks than ak: the remaining slots hold -inf blocks, lowest index first
    const int64_t nv = nvalid(t);
    if (lane < a.ak) a.out[bi * a.osb + t * a.osl + lane * a.osk] = lane < nv ? (int64_t)key_index(list[r]) : lane;
  }
}

// Prefill: one wave per query row; lane = centroid within a 64-wide tile.
struct PreArgs {
  const void* q; int qdt; int64_t qsb, qsl, qsd;
  const void* c; int cdt; int64_t csb, csn, csd;
  int64_t B, L, nb, d;
  int K, ak, bs;
  float scale, lam;
  int64_t* out; int64_t osb, osl, osk;
  void* scores; int sdt; int64_t ssb, ssl, ssn;
};

__global__ __launch_bounds__(256) void index_prefill_kernel(PreArgs a) {
  __shared__ float s_q[4][IDX_MAX_D];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;  // over B*L
  const bool row_ok = row < a.B * a.L;
  const int64_t bi = row_ok ? row / a.L : 0;
  const int64_t t = row_ok ? row % a.L : 0;
  for (int64_t c = lane; c < a.d; c += 64)
    s_q[wave][c] = row_ok ? load_elem(a.q, a.qdt, bi * a.qsb + t * a.qsl + c * a.qsd) * a.scale : 0.f;
  __syncthreads();
  if (!row_ok) return;
  const int64_t qblk = t / a.bs;
  const int64_t nvalid = (qblk + 1 < a.nb) ? qblk + 1 : a.nb;  // blocks n <= qblk
  key64 list = KEY_NONE;
  for (int64_t n0 = 0; n0 < a.nb; n0 += 64) {
    const int64_t n = n0 + lane;
    float s = -INFINITY;
    if (n < nvalid) {
      float acc = 0.f;
      const int64_t cb = bi * a.csb + n * a.csn;
      for (int64_t c = 0; c < a.d; ++c) acc = fmaf(s_q[wave][c], load_elem(a.c, a.cdt, cb + c * a.csd), acc);
      s = acc - a.lam * fast_log(1.f + (float)(qblk - n));
    }
    if (a.scores && n < a.nb) store_elem(a.scores, a.sdt, bi * a.ssb + t * a.ssl + n * a.ssn, s);
    if (n0 < nvalid) list = wave_merge_topk(list, n < nvalid ? make_key(s, (uint32_t)n) : KEY_NONE, a.K);
  }
  // Fewer valid blocks than ak: the remaining slots hold -inf blocks, lowest index first.
  const int64_t nv = nvalid;
  if (lane < a.ak) {
    const int64_t idx = lane < nv ? (int64_t)key_index(list) : lane;  // masked blocks nv, nv+1, ...
    a.out[bi * a.osb + t * a.osl + lane * a.osk] = idx;
  }
}

// Any top_k (the reference accepts every K, cpu_indexer.py:53-112, layers/indexer.py:101-112):
// one 256-thread workgroup per query row scores all the row's blocks itself (fp32 dots of the
// stored inputs, any float dtypes), keeps their keys in LDS and sorts them descending with a
// bitonic network, then writes the first ak indices.  Decode rows score every block with the
// distance nb - 1 - n (no mask); prefill rows are causal (blocks n > t / bs score -inf, so they
// follow every live block, lowest index first, as index_prefill_kernel leaves them).  Rows of
// at most SORT_MAX_N blocks; the taken path for top_k > 64, where the wave lists above stop.
constexpr int SORT_MAX_N = 16384;   // 128 KB of keys in LDS

struct SortArgs {
  const void* q; int qdt; int64_t qsb, qsr, qsd;   // decode: [B, Hq, d]; prefill: [B, L, d]
  const void* c; int cdt; int64_t csb, csn, csd;   // [B, nb, d]
  int64_t R, nb, d;          // R: query rows per batch element (Hq or L)
  int np, ak, bs, prefill;   // np: keys sorted per row (a power of two >= nb)
  float scale, lam;
  int64_t* out; int64_t osb, osr, osk;
  void* scores; int sdt; int64_t ssb, ssr, ssn;    // optional [B, R, nb] score output
};

__global__ __launch_bounds__(256) void index_sort_topk_kernel(SortArgs a) {
  extern __shared__ key64 s_key[];   // a.np keys
  __shared__ float s_q[IDX_MAX_D];
  const int tid = threadIdx.x;
  const int64_t bi = blockIdx.y, r = blockIdx.x;
  for (int64_t c = tid; c < a.d; c += 256) s_q[c] = load_elem(a.q, a.qdt, bi * a.qsb + r * a.qsr + c * a.qsd) * a.scale;
  __syncthreads();
  const int64_t qblk = a.prefill ? r / a.bs : a.nb - 1;
  for (int n = tid; n < a.np; n += 256) {
    key64 key = KEY_NONE;
    if (n < a.nb) {
      float sc = -INFINITY;
      if (n <= qblk) {
        float acc = 0.f;
        const int64_t cb = bi * a.csb + n * a.csn;
        for (int64_t c = 0; c < a.d; ++c) acc = fmaf(s_q[c], load_elem(a.c, a.cdt, cb + c * a.csd), acc);
        sc = acc - a.lam * fast_log(1.f + (float)(qblk - n));
      }
      if (a.scores) store_elem(a.scores, a.sdt, bi * a.ssb + r * a.ssr + n * a.ssn, sc);
      key = make_key(sc, (uint32_t)n);
    }
    s_key[n] = key;
  }
  __syncthreads();
  for (int k = 2; k <= a.np; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < a.np; i += 256) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const key64 x = s_key[i], y = s_key[ixj];
          const bool desc = (i & k) == 0;   // descending runs where bit k of i is clear
          if (desc ? x < y : x > y) {
            s_key[i] = y;
            s_key[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int i = tid; i < a.ak; i += 256) a.out[bi * a.osb + r * a.osr + i * a.osk] = (int64_t)key_index(s_key[i]);
}

static int launch_sort_topk(const maba_tensor* q, const maba_tensor* centroids, int prefill, int block_size,
                            float lambda_dist, int ak, maba_tensor* out_idx, maba_tensor* out_scores,
                            hipStream_t s, const char* who) {
  const int64_t B = q->shape[0], R = q->shape[1], d = q->shape[2], nb = centroids->shape[1];
  if (nb > SORT_MAX_N) return fail(MABA_ERR_UNSUPPORTED, "%s: top_k > 64 needs at most %d blocks", who, SORT_MAX_N);
  if (R > 0xffffffffLL || B > 65535) return fail(MABA_ERR_UNSUPPORTED, "%s: too many query rows", who);
  SortArgs a;
  a.q = q->data; a.qdt = q->dtype; a.qsb = q->stride[0]; a.qsr = q->stride[1]; a.qsd = q->stride[2];
  a.c = centroids->data; a.cdt = centroids->dtype;
  a.csb = centroids->stride[0]; a.csn = centroids->stride[1]; a.csd = centroids->stride[2];
  a.R = R; a.nb = nb; a.d = d;
  int np = 64;
  while (np < nb) np <<= 1;
  a.np = np; a.ak = ak; a.bs = block_size; a.prefill = prefill;
  a.scale = 1.0f / sqrtf((float)d);
  a.lam = lambda_dist;
  a.out = (int64_t*)out_idx->data; a.osb = out_idx->stride[0]; a.osr = out_idx->stride[1]; a.osk = out_idx->stride[2];
  a.scores = out_scores ? out_scores->data : nullptr;
  a.sdt = out_scores ? out_scores->dtype : MABA_F32;
  a.ssb = out_scores ? out_scores->stride[0] : 0;
  a.ssr = out_scores ? out_scores->stride[1] : 0;
  a.ssn = out_scores ? out_scores->stride[2] : 0;
  hipLaunchKernelGGL(index_sort_topk_kernel, dim3((unsigned)R, (unsigned)B), dim3(256), (size_t)np * sizeof(key64), s, a);
  return check_launch(who);
}

}  // namespace maba

using namespace maba;

static size_t decode_scores_bytes(int64_t B, int64_t Hq, int64_t nb) {
  return (size_t)(B * Hq * ceil_div(nb, 64) * 64) * sizeof(float);
}

extern "C" size_t maba_hip_index_topk_decode_workspace_size(int64_t B, int64_t Hq, int64_t nb, int top_k) {
  (void)top_k;
  const int64_t tiles = ceil_div(nb, 64);
  // MFMA path: scores + per-tile maxima; scalar path: per-split top-64 lists
  const size_t mfma = decode_scores_bytes(B, Hq, nb) + (size_t)(B * Hq * tiles) * sizeof(key64);
  const int64_t nsplit = ceil_div(tiles, 4);
  const size_t scalar = (size_t)(B * (nsplit > 0 ? nsplit : 1) * Hq * 64) * sizeof(key64);
  return mfma > scalar ? mfma : scalar;
}

// The MFMA decode (tile + select launches).  nb_cap: centroid capacity of the workspace
// rows; dlen (device) holds the sequence length when the centroid count is device-resident
// (nb = ceil(*dlen / block_size), at most nb_cap), else null and nb_cap is the count.
static int launch_decode_mfma(const maba_tensor* q, const maba_tensor* centroids, int64_t nb_cap,
                              const int64_t* dlen, int block_size, float lambda_dist, int top_k, int ak,
                              maba_tensor* out_idx, maba_tensor* out_scores, void* workspace, hipStream_t s) {
  const int64_t B = q->shape[0], Hq = q->shape[1], d = q->shape[2];
  DecTileArgs m;
  m.q = (const uint16_t*)q->data; m.qsb = q->stride[0]; m.qsh = q->stride[1];
  m.c = (const uint16_t*)centroids->data; m.csb = centroids->stride[0]; m.csn = centroids->stride[1];
  m.nb = nb_cap; m.ntiles = (int)ceil_div(nb_cap, 64); m.Hq = (int)Hq;
  m.dlen = dlen; m.bs = block_size;
  m.scale = 1.0f / sqrtf((float)d);
  m.lam = lambda_dist;
  m.sc = (float*)workspace;
  m.tmax = (key64*)((char*)workspace + decode_scores_bytes(B, Hq, nb_cap));
  m.scores = out_scores ? (float*)out_scores->data : nullptr;
  m.ssb = out_scores ? out_scores->stride[0] : 0;
  m.ssh = out_scores ? out_scores->stride[1] : 0;
  m.ssn = out_scores ? out_scores->stride[2] : 0;
  const dim3 grid((unsigned)ceil_div(m.ntiles, 4), (unsigned)B);
  switch (d / 32) {
    case 1: hipLaunchKernelGGL(index_decode_tile_kernel<1>, grid, dim3(256), 0, s, m); break;
    case 2: hipLaunchKernelGGL(index_decode_tile_kernel<2>, grid, dim3(256), 0, s, m); break;
    case 3: hipLaunchKernelGGL(index_decode_tile_kernel<3>, grid, dim3(256), 0, s, m); break;
    case 4: hipLaunchKernelGGL(index_decode_tile_kernel<4>, grid, dim3(256), 0, s, m); break;
    case 5: hipLaunchKernelGGL(index_decode_tile_kernel<5>, grid, dim3(256), 0, s, m); break;
    case 6: hipLaunchKernelGGL(index_decode_tile_kernel<6>, grid, dim3(256), 0, s, m); break;
    case 7: hipLaunchKernelGGL(index_decode_tile_kernel<7>, grid, dim3(256), 0, s, m); break;
    default: hipLaunchKernelGGL(index_decode_tile_kernel<8>, grid, dim3(256), 0, s, m); break;
  }
  int rc = check_launch("index_topk_decode/tiles");
  if (rc) return rc;
  DecSelArgs e;
  e.sc = m.sc; e.tmax = m.tmax; e.nb = nb_cap; e.ntiles = m.ntiles; e.Hq = (int)Hq; e.K = top_k; e.ak = ak;
  e.dlen = dlen; e.bs = block_size;
  e.out = (int64_t*)out_idx->data; e.osb = out_idx->stride[0]; e.osh = out_idx->stride[1];
  e.osk = out_idx->stride[2];
  hipLaunchKernelGGL(index_decode_select_kernel, dim3((unsigned)(B * Hq)), dim3(SEL_T), 0, s, e);
  return check_launch("index_topk_decode/select");
}

// Whether the MFMA decode takes q / centroids (bf16 rows, 16-byte aligned, d a multiple of 32).
static bool decode_mfma_ok(const maba_tensor* q, const maba_tensor* centroids) {
  const int64_t B = q->shape[0], Hq = q->shape[1], d = q->shape[2];
  return q->dtype == MABA_BF16 && centroids->dtype == MABA_BF16 && q->stride[2] == 1 && centroids->stride[2] == 1 &&
         d % 32 == 0 && d <= 256 && (uintptr_t)q->data % 16 == 0 && (uintptr_t)centroids->data % 16 == 0 &&
         (B == 1 || q->stride[0] % 8 == 0) && (Hq == 1 || q->stride[1] % 8 == 0) &&
         (B == 1 || centroids->stride[0] % 8 == 0) && centroids->stride[1] % 8 == 0;
}

extern "C" int maba_hip_index_topk_decode(const maba_tensor* q, const maba_tensor* centroids,
                                          float lambda_dist, int top_k, maba_tensor* out_idx,
                                          maba_tensor* out_scores, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  if (!q || q->ndim != 3) return fail(MABA_ERR_INVALID, "index_topk_decode: q must be [B,Hq,d]");
  if (!centroids || centroids->ndim != 3) return fail(MABA_ERR_INVALID, "index_topk_decode: centroids must be [B,nb,d]");
  const int64_t B = q->shape[0], Hq = q->shape[1], d = q->shape[2], nb = centroids->shape[1];
  if (centroids->shape[0] != B || centroids->shape[2] != d)
    return fail(MABA_ERR_INVALID, "index_topk_decode: centroids shape mismatch");
  if (top_k <= 0) return fail(MABA_ERR_INVALID, "index_topk_decode: top_k must be positive, got %d", top_k);
  const int64_t ak = top_k < nb ? top_k : nb;
  const int64_t so[3] = {B, Hq, ak};
  if (!expect_shape(out_idx, "out_idx", 3, so)) return MABA_ERR_INVALID;
  if (out_idx->dtype != MABA_I64) return fail(MABA_ERR_DTYPE, "index_topk_decode: out_idx must be int64");
  if (!expect_float(q, "q") || !expect_float(centroids, "centroids")) return MABA_ERR_DTYPE;
  if (d > IDX_MAX_D) return fail(MABA_ERR_UNSUPPORTED, "index_topk_decode: d <= %d required", IDX_MAX_D);
  if (top_k > 64) {   // the general path: per-row scores sorted in LDS (no workspace)
    if (out_scores) {
      const int64_t ss[3] = {B, Hq, nb};
      if (!expect_shape(out_scores, "out_scores", 3, ss)) return MABA_ERR_INVALID;
      if (out_scores->dtype != MABA_F32) return fail(MABA_ERR_DTYPE, "index_topk_decode: out_scores must be f32");
    }
    if (B * Hq == 0 || nb == 0) return MABA_OK;
    return launch_sort_topk(q, centroids, 0, 64, lambda_dist, (int)ak, out_idx, out_scores, (hipStream_t)stream,
                            "index_topk_decode");
  }
  if (Hq > IDX_MAX_HEADS || d > IDX_MAX_D)
    return fail(MABA_ERR_UNSUPPORTED, "index_topk_decode: Hq <= %d and d <= %d required", IDX_MAX_HEADS, IDX_MAX_D);
  if (out_scores) {
    const int64_t ss[3] = {B, Hq, nb};
    if (!expect_shape(out_scores, "out_scores", 3, ss)) return MABA_ERR_INVALID;
    if (out_scores->dtype != MABA_F32) return fail(MABA_ERR_DTYPE, "index_topk_decode: out_scores must be f32");
  }
  if (B * Hq == 0 || nb == 0) return MABA_OK;
  const size_t need = maba_hip_index_topk_decode_workspace_size(B, Hq, nb, top_k);
  if (!workspace || workspace_bytes < need)
    return fail(MABA_ERR_WORKSPACE, "index_topk_decode: workspace of %zu bytes required", need);
  hipStream_t s = (hipStream_t)stream;
  const bool mfma_ok = decode_mfma_ok(q, centroids);
  if (mfma_ok)
    return launch_decode_mfma(q, centroids, nb, nullptr, 0, lambda_dist, top_k, (int)ak, out_idx, out_scores,
                              workspace, s);
  DecArgs a;
  a.q = q->data; a.qdt = q->dtype; a.qsb = q->stride[0]; a.qsh = q->stride[1]; a.qsd = q->stride[2];
  a.c = centroids->data; a.cdt = centroids->dtype;
  a.csb = centroids->stride[0]; a.csn = centroids->stride[1]; a.csd = centroids->stride[2];
  a.nb = nb; a.d = d; a.Hq = (int)Hq; a.K = top_k;
  a.tiles_per_wave = 1;
  a.nsplit = (int)ceil_div(ceil_div(nb, 64), 4);
  a.scale = 1.0f / sqrtf((float)d);
  a.lam = lambda_dist;
  a.ws = (key64*)workspace;
  a.scores = out_scores ? (float*)out_scores->data : nullptr;
  a.ssb = out_scores ? out_scores->stride[0] : 0;
  a.ssh = out_scores ? out_scores->stride[1] : 0;
  a.ssn = out_scores ? out_scores->stride[2] : 0;
  hipLaunchKernelGGL(index_decode_score_kernel, dim3((unsigned)a.nsplit, (unsigned)B), dim3(256), 0, s, a);
  int rc = check_launch("index_topk_decode/score");
  if (rc) return rc;
  hipLaunchKernelGGL(index_decode_merge_kernel, dim3((unsigned)(B * Hq)), dim3(64), 0, s, a.ws, a.nsplit,
                     (int)Hq, top_k, (int)ak, (int64_t*)out_idx->data, out_idx->stride[0],
                     out_idx->stride[1], out_idx->stride[2]);
  return check_launch("index_topk_decode/merge");
}

extern "C" int maba_hip_index_topk_decode_dev(const maba_tensor* q, const maba_tensor* centroids,
                                              const int64_t* d_len, int block_size, float lambda_dist,
                                              int top_k, maba_tensor* out_idx, void* workspace,
                                              size_t workspace_bytes, void* stream) {
  if (!q || q->ndim != 3) return fail(MABA_ERR_INVALID, "index_topk_decode_dev: q must be [B,Hq,d]");
  if (!centroids || centroids->ndim != 3)
    return fail(MABA_ERR_INVALID, "index_topk_decode_dev: centroids must be [B,Ncap,d]");
  if (!d_len) return fail(MABA_ERR_INVALID, "index_topk_decode_dev: d_len (device int64) required");
  const int64_t B = q->shape[0], Hq = q->shape[1], d = q->shape[2], ncap = centroids->shape[1];
  if (centroids->shape[0] != B || centroids->shape[2] != d)
    return fail(MABA_ERR_INVALID, "index_topk_decode_dev: centroids shape mismatch");
  if (top_k <= 0 || top_k > 64) return fail(MABA_ERR_INVALID, "index_topk_decode_dev: top_k in [1, 64]");
  if (block_size <= 0) return fail(MABA_ERR_INVALID, "index_topk_decode_dev: block_size must be positive");
  const int64_t so[3] = {B, Hq, top_k};
  if (!expect_shape(out_idx, "out_idx", 3, so)) return MABA_ERR_INVALID;
  if (out_idx->dtype != MABA_I64) return fail(MABA_ERR_DTYPE, "index_topk_decode_dev: out_idx must be int64");
  if (Hq > IDX_MAX_HEADS) return fail(MABA_ERR_UNSUPPORTED, "index_topk_decode_dev: Hq <= %d", IDX_MAX_HEADS);
  if (!decode_mfma_ok(q, centroids))
    return fail(MABA_ERR_UNSUPPORTED, "index_topk_decode_dev: bf16 q and centroids, 16-byte aligned rows, d a "
                                      "multiple of 32 up to 256");
  if (B * Hq == 0 || ncap == 0) return MABA_OK;
  const size_t need = maba_hip_index_topk_decode_workspace_size(B, Hq, ncap, top_k);
  if (!workspace || workspace_bytes < need)
    return fail(MABA_ERR_WORKSPACE, "index_topk_decode_dev: workspace of %zu bytes required", need);
  return launch_decode_mfma(q, centroids, ncap, d_len, block_size, lambda_dist, top_k, top_k, out_idx, nullptr,
                            workspace, (hipStream_t)stream);
}

extern "C" int maba_hip_index_topk(const maba_tensor* q_idx, const maba_tensor* centroids,
                                   float lambda_dist, int top_k, int block_size, maba_tensor* out_idx,
                                   maba_tensor* out_scores, void* stream) {
  if (!q_idx || q_idx->ndim != 3 || !centroids || centroids->ndim != 3)
    return fail(MABA_ERR_INVALID, "index_topk: q_idx and centroids must be 3D");
  const int64_t B = q_idx->shape[0], L = q_idx->shape[1], d = q_idx->shape[2], nb = centroids->shape[1];
  if (centroids->shape[0] != B || centroids->shape[2] != d)
    return fail(MABA_ERR_INVALID, "index_topk: dimension mismatch between q_idx and centroids");
  if (top_k <= 0) return fail(MABA_ERR_INVALID, "index_topk: top_k must be positive, got %d", top_k);
  if (block_size <= 0) return fail(MABA_ERR_INVALID, "index_topk: block_size must be positive, got %d", block_size);
  const int64_t ak = top_k < nb ? top_k : nb;
  const int64_t so[3] = {B, L, ak};
  if (!expect_shape(out_idx, "out_idx", 3, so)) return MABA_ERR_INVALID;
  if (out_idx->dtype != MABA_I64) return fail(MABA_ERR_DTYPE, "index_topk: out_idx must be int64");
  if (!expect_float(q_idx, "q_idx") || !expect_float(centroids, "centroids")) return MABA_ERR_DTYPE;
  if (d > IDX_MAX_D) return fail(MABA_ERR_UNSUPPORTED, "index_topk: d <= %d required", IDX_MAX_D);
  if (out_scores) {
    const int64_t ss[3] = {B, L, nb};
    if (!expect_shape(out_scores, "out_scores", 3, ss)) return MABA_ERR_INVALID;
    if (!expect_float(out_scores, "out_scores")) return MABA_ERR_DTYPE;
  }
  if (B * L == 0 || nb == 0) return MABA_OK;
  if (top_k > 64 && nb > 64)   // the general path: per-row scores sorted in LDS
    return launch_sort_topk(q_idx, centroids, 1, block_size, lambda_dist, (int)ak, out_idx, out_scores,
                            (hipStream_t)stream, "index_topk");
  // MFMA path: bf16 rows with unit channel stride, 16-byte aligned, d a multiple of 32
  const bool mfma = !out_scores && q_idx->dtype == MABA_BF16 && centroids->dtype == MABA_BF16 && d % 32 == 0 &&
                    q_idx->stride[2] == 1 && centroids->stride[2] == 1 && (uintptr_t)q_idx->data % 16 == 0 &&
                    (uintptr_t)centroids->data % 16 == 0 && q_idx->stride[0] % 8 == 0 && q_idx->stride[1] % 8 == 0 &&
                    centroids->stride[0] % 8 == 0 && centroids->stride[1] % 8 == 0 && nb < ((int64_t)1 << 31);
  if (mfma) {
    PreMfmaArgs m;
    m.q = (const uint16_t*)q_idx->data; m.qsb = q_idx->stride[0]; m.qsl = q_idx->stride[1];
    m.c = (const uint16_t*)centroids->data; m.csb = centroids->stride[0]; m.csn = centroids->stride[1];
    m.L = L; m.nb = nb;
    m.K = (int)(top_k < 64 ? top_k : 64); m.ak = (int)ak; m.bs = block_size;
    m.scale = 1.0f / sqrtf((float)d);
    m.lam = lambda_dist;
    m.out = (int64_t*)out_idx->data; m.osb = out_idx->stride[0]; m.osl = out_idx->stride[1];
    m.osk = out_idx->stride[2];
    const dim3 grid((unsigned)ceil_div(L, 16), (unsigned)B);
    hipStream_t st = (hipStream_t)stream;
    switch (d / 32) {
      case 1: hipLaunchKernelGGL(index_prefill_mfma_kernel<1>, grid, dim3(256), 0, st, m); break;
      case 2: hipLaunchKernelGGL(index_prefill_mfma_kernel<2>, grid, dim3(256), 0, st, m); break;
      case 3: hipLaunchKernelGGL(index_prefill_mfma_kernel<3>, grid, dim3(256), 0, st, m); break;
      case 4: hipLaunchKernelGGL(index_prefill_mfma_kernel<4>, grid, dim3(256), 0, st, m); break;
      case 5: hipLaunchKernelGGL(index_prefill_mfma_kernel<5>, grid, dim3(256), 0, st, m); break;
      case 6: hipLaunchKernelGGL(index_prefill_mfma_kernel<6>, grid, dim3(256), 0, st, m); break;
      case 7: hipLaunchKernelGGL(index_prefill_mfma_kernel<7>, grid, dim3(256), 0, st, m); break;
      default: hipLaunchKernelGGL(index_prefill_mfma_kernel<8>, grid, dim3(256), 0, st, m); break;
    }
    return check_launch("index_topk");
  }
  PreArgs a;
  a.q = q_idx->data; a.qdt = q_idx->dtype; a.qsb = q_idx->stride[0]; a.qsl = q_idx->stride[1]; a.qsd = q_idx->stride[2];
  a.c = centroids->data; a.cdt = centroids->dtype;
  a.csb = centroids->stride[0]; a.csn = centroids->stride[1]; a.csd = centroids->stride[2];
  a.B = B; a.L = L; a.nb = nb; a.d = d;
  a.K = (int)(top_k < 64 ? top_k : 64); a.ak = (int)ak; a.bs = block_size;
  a.scale = 1.0f / sqrtf((float)d);
  a.lam = lambda_dist;
  a.out = (int64_t*)out_idx->data; a.osb = out_idx->stride[0]; a.osl = out_idx->stride[1]; a.osk = out_idx->stride[2];
  a.scores = out_scores ? out_scores->data : nullptr;
  a.sdt = out_scores ? out_scores->dtype : MABA_F32;
  a.ssb = out_scores ? out_scores->stride[0] : 0;
  a.ssl = out_scores ? out_scores->stride[1] : 0;
  a.ssn = out_scores ? out_scores->stride[2] : 0;
  hipLaunchKernelGGL(index_prefill_kernel, dim3((unsigned)ceil_div(B * L, 4)), dim3(256), 0,
                     (hipStream_t)stream, a);
  return check_launch("index_topk");
}

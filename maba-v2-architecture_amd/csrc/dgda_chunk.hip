// Chunked DGDA prefill on MFMA for per-token (scalar) decay and erase gates,
// dk = dv = 64, bf16 q/k/v -- the BASELINE prefill configuration.
//
// Math per 64-token chunk (reference: maba_sparse/kernels/cpu_dgda.py:101-146,
// here with Lam_i the inclusive cumulative log-decay of token i, a scalar):
//   L_ij = beta_i (k_i . k_j) exp(Lam_i - Lam_j)         i > j
//   A_ij =        (q_i . k_j) exp(Lam_i - Lam_j)         i >= j
//   v_e  = w*v - diag(beta e^Lam) (k S0)
//   u    = (I + L)^-1 v_e
//   o    = diag(e^Lam) (q S0) + A u
//   S    = e^{Lam_63} S0 + k^T diag(e^{Lam_63 - Lam}) u
// All decay factors are <= 1, so nothing overflows for any gate values.
//
// Sequence parallelism (only B*H = 40 recurrences at the BASELINE shape, but
// 256 CUs): the sequence of each (b,h) is cut into segments of CPS chunks.
//   pass 1 (dgda_chunk_kernel<AGG>) runs every segment but the last from a zero
//          state, carrying X = [N | M] (64 x 128): N is the segment's state from
//          S0 = 0, M its state transition (X starts as [0 | I], the M half gets
//          no input), so S_end = M S_start + N.
//   pass 2 (dgda_segment_scan_kernel) walks the segments of each (b,h):
//          S_{s+1} = M_s S_s + N_s, writing every segment's start state.
//   pass 3 (dgda_chunk_kernel<OUT>) re-runs each segment from its start state and
//          writes the outputs (and the final state from the last segment).
//
// Workgroup layout: wave w owns 16 columns of the carried state (pass 1: 8 waves
// over the 128 columns of [N | M]; pass 3: 4 waves over the 64 columns of S).
// Per chunk the workgroup stages k (and k^T, q) in LDS, builds L, A and the 16x16
// diagonal-block inverses T_II = (I + L_II)^-1 cooperatively, then each wave runs
// its columns through v_e, the blocked triangular solve, the output and the state
// update with register-resident accumulator tiles.
//
// MFMA usage (gfx950): v_mfma_f32_16x16x32_bf16 for every product with K >= 32 and
// v_mfma_f32_16x16x16_bf16 for the K = 16 steps of the solve.  An accumulator tile
// (lane l holds rows 4(l/16)..+3 of column l%16) is used directly as a B operand by
// permuting K: lane group g supplies the rows 4g..4g+3 of two stacked tiles, and the
// A operand is read from LDS at the matching two column groups.  Raw bf16 inputs
// are exact MFMA operands; fp32 operands (S, u, L, A, T) are split into bf16
// hi + lo parts (two or three MFMAs) so products carry ~16 mantissa bits.
#include "maba_common.h"

namespace maba {

typedef __attribute__((ext_vector_type(8))) short i16x8;

constexpr int CH = 64;        // chunk length (tokens)
constexpr int DK = 64;        // key / value head size
constexpr int PITCH = 72;     // bf16 row pitch of LDS matrices (144 B: 16-B aligned, conflict-light)
constexpr int TPITCH = 20;    // bf16 row pitch of the 16x16 inverse blocks
constexpr int CPS = 16;       // chunks per segment

struct ChunkArgs {
  const uint16_t* q; int64_t qs0, qs1, qs2;   // bf16 [B,H,L,64], channel stride 1
  const uint16_t* k; int64_t ks0, ks1, ks2;
  View4 v, gate, b, w, s0;                    // gate: log_alpha (use_log) or alpha
  MView4 out, sf;
  float* agg;      // [BH, nseg, 64, 128]
  float* sstart;   // [BH, nseg, 64, 64]
  int H, L, nseg, nchunks, use_log, has_s0;
};

// ------------------------------------------------------------------ MFMA helpers

__device__ __forceinline__ f32x4 mma32(f32x4 c, i16x8 a, i16x8 b) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mma16(f32x4 c, i16x4 a, i16x4 b) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ short bf16_rn(float f) { return (short)f32_to_bf16_bits(f); }
__device__ __forceinline__ float bf16_val(short h) { return bf16_bits_to_f32((uint16_t)h); }

// Split four fp32 values into bf16 hi and lo parts (x ~= hi + lo).
__device__ __forceinline__ void split4(f32x4 x, i16x4& hi, i16x4& lo) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const short h = bf16_rn(x[i]);
    hi[i] = h;
    lo[i] = bf16_rn(x[i] - bf16_val(h));
  }
}

__device__ __forceinline__ i16x8 cat8(i16x4 a, i16x4 b) {
  i16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

__device__ __forceinline__ i16x4 lds4(const short* base, int row, int col, int pitch) {
  return *(const i16x4*)(base + row * pitch + col);
}
__device__ __forceinline__ i16x8 lds8(const short* base, int row, int col, int pitch) {
  return *(const i16x8*)(base + row * pitch + col);
}
// Permuted-K A operand: columns c0..c0+3 and c0+16..c0+19 of one row.
__device__ __forceinline__ i16x8 lds4x2(const short* base, int row, int c0, int pitch) {
  return cat8(lds4(base, row, c0, pitch), lds4(base, row, c0 + 16, pitch));
}

// ------------------------------------------------------------------ shared memory

template <bool AGG>
struct ChunkSmem {
  short K[CH * PITCH];        // k rows (token-major)
  short KT[DK * PITCH];       // k^T (channel-major)
  short Q[AGG ? 1 : CH * PITCH];
  short LH[CH * PITCH], LL[CH * PITCH];              // L hi/lo, strictly lower
  short AH[AGG ? 1 : CH * PITCH], AL[AGG ? 1 : CH * PITCH];  // A hi/lo, lower incl. diagonal
  short TH[4 * 16 * TPITCH], TL[4 * 16 * TPITCH];   // (I + L_II)^-1 hi/lo
  float LD[4][16][17];                               // diagonal blocks of L, fp32
  float lam[CH], elam[CH], eend[CH], beta[CH];
};

// ------------------------------------------------------------------ the chunk kernel

template <bool AGG>
__global__ __launch_bounds__(AGG ? 512 : 256) void dgda_chunk_kernel(ChunkArgs a) {
  constexpr int NW = AGG ? 8 : 4;
  __shared__ ChunkSmem<AGG> sm;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int seg = blockIdx.x % a.nseg;
  const int bh = blockIdx.x / a.nseg;
  const int bi = bh / a.H, hi = bh % a.H;
  if (AGG && seg == a.nseg - 1) return;  // the last segment's aggregate is never needed

  // Carried state slab: S[16kt + 4g + i][col0 + c16] in Sr[kt][i].
  f32x4 Sr[4];
  const int col0 = (wave & 3) * 16;
  const bool is_m = AGG && wave >= 4;  // pass 1: M half of [N | M]
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * kt + 4 * g + i;
      float x = 0.f;
      if (AGG) {
        x = (is_m && r == col0 + c16) ? 1.f : 0.f;
      } else if (seg == 0) {
        x = a.has_s0 ? a.s0.at(bi, hi, r, col0 + c16) : 0.f;
      } else {
        x = a.sstart[(((int64_t)bh * a.nseg + seg) * 64 + r) * 64 + col0 + c16];
      }
      Sr[kt][i] = x;
    }
  }

  const int c_begin = seg * CPS;
  const int c_end = min(a.nchunks, c_begin + CPS);
  const uint16_t* qb = a.q + bi * a.qs0 + hi * a.qs1;
  const uint16_t* kb = a.k + bi * a.ks0 + hi * a.ks1;

  for (int c = c_begin; c < c_end; ++c) {
    const int t0 = c * CH;
    __syncthreads();  // previous chunk is done with the shared buffers
    // ---- stage k (and q) rows, k^T, gates
    for (int i = tid; i < CH * 8; i += NW * 64) {
      const int t = i >> 3, c8 = (i & 7) * 8;
      i16x8 kv = {0, 0, 0, 0, 0, 0, 0, 0}, qv = {0, 0, 0, 0, 0, 0, 0, 0};
      if (t0 + t < a.L) {
        kv = *(const i16x8*)(kb + (int64_t)(t0 + t) * a.ks2 + c8);
        if (!AGG) qv = *(const i16x8*)(qb + (int64_t)(t0 + t) * a.qs2 + c8);
      }
      *(i16x8*)(sm.K + t * PITCH + c8) = kv;
      if (!AGG) *(i16x8*)(sm.Q + t * PITCH + c8) = qv;
#pragma unroll
      for (int j = 0; j < 8; ++j) sm.KT[(c8 + j) * PITCH + t] = kv[j];
    }
    if (tid < CH) {
      const int t = t0 + tid;
      float la = 0.f, be = 0.f;
      if (t < a.L) {
        const float gv = a.gate.at(bi, hi, t, 0);
        la = a.use_log ? gv : __logf(fmaxf(gv, 1e-20f));
        la = fminf(la, 0.f);
        be = a.b.at(bi, hi, t, 0);
      }
      // inclusive prefix sum of the log decay across the wave
      float s = la;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float o = __shfl_up(s, off);
        if (tid >= off) s += o;
      }
      const float last = __shfl(s, 63);
      sm.lam[tid] = s;
      sm.elam[tid] = __expf(s);
      sm.eend[tid] = __expf(last - s);
      sm.beta[tid] = be;
    }
    __syncthreads();

    // ---- L = beta_i (k k^T) decay (strict lower) and A = (q k^T) decay (lower)
    // Tile (I,J) is computed as D = k_J x k_I^T (or k_J x q_I^T) so each lane holds
    // row i = 16I + c16 and columns 16J + 4g..+3: a contiguous 8-byte store.
    {
      constexpr int NT = AGG ? 10 : 20;
      for (int tix = wave; tix < NT; tix += NW) {
        const bool isA = tix >= 10;
        int tt = isA ? tix - 10 : tix;
        int I = 0;
        while (tt > I) { tt -= I + 1; ++I; }
        const int J = tt;  // J <= I
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const short* Bsrc = isA ? sm.Q : sm.K;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const i16x8 av = lds8(sm.K, 16 * J + c16, 32 * p + 8 * g, PITCH);
          const i16x8 bv = lds8(Bsrc, 16 * I + c16, 32 * p + 8 * g, PITCH);
          acc = mma32(acc, av, bv);
        }
        const int i = 16 * I + c16;
        const float li = sm.lam[i];
        const float be = sm.beta[i];
        i16x4 h, l;
        f32x4 val;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * J + 4 * g + r;
          const float dec = __expf(fminf(li - sm.lam[j], 0.f));
          float x = acc[r] * dec;
          if (isA) {
            x = (j <= i) ? x : 0.f;
          } else {
            x = (j < i) ? x * be : 0.f;
          }
          val[r] = x;
        }
        split4(val, h, l);
        short* dh = isA ? sm.AH : sm.LH;
        short* dl = isA ? sm.AL : sm.LL;
        *(i16x4*)(dh + i * PITCH + 16 * J + 4 * g) = h;
        *(i16x4*)(dl + i * PITCH + 16 * J + 4 * g) = l;
        if (!isA && I == J) {
#pragma unroll
          for (int r = 0; r < 4; ++r) sm.LD[I][c16][4 * g + r] = bf16_val(h[r]) + bf16_val(l[r]);
        }
      }
    }
    __syncthreads();

    // ---- T_II = (I + L_II)^-1 by forward substitution, one column per lane.
    if (wave < 4 && lane < 16) {
      const int I = wave, j = lane;
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float s = (i == j) ? 1.f : 0.f;
#pragma unroll
        for (int m = 0; m < i; ++m) s = fmaf(-sm.LD[I][i][m], x[m], s);
        x[i] = s;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const short h = bf16_rn(x[i]);
        sm.TH[(I * 16 + i) * TPITCH + j] = h;
        sm.TL[(I * 16 + i) * TPITCH + j] = bf16_rn(x[i] - bf16_val(h));
      }
    }
    __syncthreads();

    // ---- per-wave column slab: v_e = w*v - diag(beta e^Lam) (k S)
    i16x4 Sh[4], Sl[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) split4(Sr[kt], Sh[kt], Sl[kt]);
    f32x4 u[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const i16x8 av = lds4x2(sm.K, 16 * tt + c16, 32 * p + 4 * g, PITCH);
        acc = mma32(acc, av, cat8(Sh[2 * p], Sh[2 * p + 1]));
        acc = mma32(acc, av, cat8(Sl[2 * p], Sl[2 * p + 1]));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tl = 16 * tt + 4 * g + i;
        const int t = t0 + tl;
        float y = 0.f;
        if (!is_m && t < a.L) y = a.w.at(bi, hi, t, col0 + c16) * a.v.at(bi, hi, t, col0 + c16);
        u[tt][i] = y - sm.beta[tl] * sm.elam[tl] * acc[i];
      }
    }

    // ---- blocked forward substitution, u_I = T_II (v_e_I - sum_{J<I} L_IJ u_J)
    i16x4 uh[4], ul[4];
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 rhs = u[I];
      if (I >= 1) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if (I >= 2) {  // J = 0,1 as one K = 32 step
          const int row = 16 * I + c16;
          const i16x8 ah = lds4x2(sm.LH, row, 4 * g, PITCH), al = lds4x2(sm.LL, row, 4 * g, PITCH);
          const i16x8 bh8 = cat8(uh[0], uh[1]), bl8 = cat8(ul[0], ul[1]);
          acc = mma32(acc, ah, bh8);
          acc = mma32(acc, ah, bl8);
          acc = mma32(acc, al, bh8);
        }
        if (I == 1 || I == 3) {  // the remaining single 16-wide step J = I-1 (I=3: J=2)
          const int J = I == 1 ? 0 : 2;
          const int row = 16 * I + c16;
          const i16x4 ah = lds4(sm.LH, row, 16 * J + 4 * g, PITCH), al = lds4(sm.LL, row, 16 * J + 4 * g, PITCH);
          acc = mma16(acc, ah, uh[J]);
          acc = mma16(acc, ah, ul[J]);
          acc = mma16(acc, al, uh[J]);
        }
        rhs = rhs - acc;
      }
      i16x4 rh, rl;
      split4(rhs, rh, rl);
      const i16x4 th = lds4(sm.TH, I * 16 + c16, 4 * g, TPITCH), tl = lds4(sm.TL, I * 16 + c16, 4 * g, TPITCH);
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      x = mma16(x, th, rh);
      x = mma16(x, th, rl);
      x = mma16(x, tl, rh);
      u[I] = x;
      split4(x, uh[I], ul[I]);
    }

    // ---- outputs: o = diag(e^Lam) (q S) + A u
    if (!AGG) {
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        f32x4 qs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const i16x8 av = lds4x2(sm.Q, 16 * I + c16, 32 * p + 4 * g, PITCH);
          qs = mma32(qs, av, cat8(Sh[2 * p], Sh[2 * p + 1]));
          qs = mma32(qs, av, cat8(Sl[2 * p], Sl[2 * p + 1]));
        }
        f32x4 au = {0.f, 0.f, 0.f, 0.f};
        const int row = 16 * I + c16;
#pragma unroll
        for (int P = 0; P < 2; ++P) {  // J pairs (0,1), (2,3)
          if (2 * P + 1 <= I) {
            const i16x8 ah = lds4x2(sm.AH, row, 32 * P + 4 * g, PITCH), al = lds4x2(sm.AL, row, 32 * P + 4 * g, PITCH);
            const i16x8 bh8 = cat8(uh[2 * P], uh[2 * P + 1]), bl8 = cat8(ul[2 * P], ul[2 * P + 1]);
            au = mma32(au, ah, bh8);
            au = mma32(au, ah, bl8);
            au = mma32(au, al, bh8);
          }
        }
        if ((I & 1) == 0) {  // single J = I
          const i16x4 ah = lds4(sm.AH, row, 16 * I + 4 * g, PITCH), al = lds4(sm.AL, row, 16 * I + 4 * g, PITCH);
          au = mma16(au, ah, uh[I]);
          au = mma16(au, ah, ul[I]);
          au = mma16(au, al, uh[I]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tl = 16 * I + 4 * g + i;
          const int t = t0 + tl;
          if (t < a.L) a.out.put(bi, hi, t, col0 + c16, sm.elam[tl] * qs[i] + au[i]);
        }
      }
    }

    // ---- state update: S = e^{Lam_63} S + k^T diag(e^{Lam_63 - Lam}) u
    i16x4 wh[4], wl[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      f32x4 x;
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = u[tt][i] * sm.eend[16 * tt + 4 * g + i];
      split4(x, wh[tt], wl[tt]);
    }
    const float gdec = sm.elam[CH - 1];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      f32x4 acc = Sr[kt] * gdec;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const i16x8 av = lds4x2(sm.KT, 16 * kt + c16, 32 * p + 4 * g, PITCH);
        acc = mma32(acc, av, cat8(wh[2 * p], wh[2 * p + 1]));
        acc = mma32(acc, av, cat8(wl[2 * p], wl[2 * p + 1]));
      }
      Sr[kt] = acc;
    }
  }

  // ---- segment results
  if (AGG) {
    float* dst = a.agg + ((int64_t)bh * a.nseg + seg) * 64 * 128;
    const int cc = (is_m ? 64 : 0) + col0 + c16;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[(16 * kt + 4 * g + i) * 128 + cc] = Sr[kt][i];
  } else if (seg == a.nseg - 1) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) a.sf.put(bi, hi, 16 * kt + 4 * g + i, col0 + c16, Sr[kt][i]);
  }
}

// ------------------------------------------------------------------ pass 2: segment scan
// One wave per (b,h, 16-column slab): S_{s+1} = M_s S_s + N_s with fp32 accuracy
// (M and S both split into bf16 hi/lo).  Writes the start state of segments 1..nseg-1.
__global__ __launch_bounds__(64) void dgda_segment_scan_kernel(ChunkArgs a) {
  const int bh = blockIdx.x >> 2;
  const int col0 = (blockIdx.x & 3) * 16;
  const int bi = bh / a.H, hi = bh % a.H;
  const int lane = threadIdx.x, g = lane >> 4, c16 = lane & 15;
  f32x4 Sr[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      Sr[kt][i] = a.has_s0 ? a.s0.at(bi, hi, 16 * kt + 4 * g + i, col0 + c16) : 0.f;
  for (int s = 0; s + 1 < a.nseg; ++s) {
    const float* X = a.agg + ((int64_t)bh * a.nseg + s) * 64 * 128;
    i16x4 Sh[4], Sl[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) split4(Sr[kt], Sh[kt], Sl[kt]);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      f32x4 acc;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = X[(16 * mt + 4 * g + i) * 128 + col0 + c16];  // N_s
      const int row = 16 * mt + c16;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        // A operand: M_s[row][32p + 4g..+3] and [32p + 16 + 4g..+3]  (M lives in columns 64..127)
        const float4 m0 = *(const float4*)(X + row * 128 + 64 + 32 * p + 4 * g);
        const float4 m1 = *(const float4*)(X + row * 128 + 64 + 32 * p + 16 + 4 * g);
        f32x4 mlo = {m0.x, m0.y, m0.z, m0.w}, mhi = {m1.x, m1.y, m1.z, m1.w};
        i16x4 h0, l0, h1, l1;
        split4(mlo, h0, l0);
        split4(mhi, h1, l1);
        const i16x8 ah = cat8(h0, h1), al = cat8(l0, l1);
        const i16x8 bh8 = cat8(Sh[2 * p], Sh[2 * p + 1]), bl8 = cat8(Sl[2 * p], Sl[2 * p + 1]);
        acc = mma32(acc, ah, bh8);
        acc = mma32(acc, ah, bl8);
        acc = mma32(acc, al, bh8);
      }
      Sr[mt] = acc;
    }
    float* dst = a.sstart + ((int64_t)bh * a.nseg + s + 1) * 64 * 64;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[(16 * kt + 4 * g + i) * 64 + col0 + c16] = Sr[kt][i];
  }
}

// ------------------------------------------------------------------ host side

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

bool dgda_chunk_supported(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                          const maba_tensor* gate, const maba_tensor* b) {
  if (!q || !k || !v || !gate || !b) return false;
  if (q->dtype != MABA_BF16 || k->dtype != MABA_BF16) return false;
  if (q->shape[3] != DK || v->shape[3] != DK) return false;
  if (q->stride[3] != 1 || k->stride[3] != 1) return false;
  if (gate->stride[3] != 0 || b->stride[3] != 0) return false;  // per-token decay and erase gate
  if (q->shape[2] > (int64_t)1 << 30) return false;
  for (const maba_tensor* t : {q, k}) {
    if (!aligned16(t->data)) return false;
    for (int d = 0; d < 3; ++d)
      if (t->shape[d] > 1 && (t->stride[d] % 8) != 0) return false;
  }
  return true;
}

static int nseg_for(int64_t L) {
  const int64_t nch = ceil_div(L, CH);
  return (int)ceil_div(nch > 0 ? nch : 1, CPS);
}

size_t dgda_chunk_workspace(int64_t BH, int64_t L) {
  const int64_t nseg = nseg_for(L);
  if (nseg <= 1) return 16;
  return (size_t)(BH * nseg * 64 * (128 + 64)) * sizeof(float);
}

int launch_dgda_chunk(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                      const maba_tensor* gate, int use_log, const maba_tensor* b,
                      const maba_tensor* w, const maba_tensor* s0, maba_tensor* out,
                      maba_tensor* sf, void* ws, size_t ws_bytes, hipStream_t stream) {
  const int64_t B = q->shape[0], H = q->shape[1], L = q->shape[2];
  const int64_t BH = B * H;
  ChunkArgs a;
  a.q = (const uint16_t*)q->data; a.qs0 = q->stride[0]; a.qs1 = q->stride[1]; a.qs2 = q->stride[2];
  a.k = (const uint16_t*)k->data; a.ks0 = k->stride[0]; a.ks1 = k->stride[1]; a.ks2 = k->stride[2];
  a.v = view4(v); a.gate = view4(gate); a.b = view4(b); a.w = view4(w); a.s0 = view4(s0);
  a.out = mview4(out); a.sf = mview4(sf);
  a.H = (int)H; a.L = (int)L;
  a.nchunks = (int)ceil_div(L, CH);
  a.nseg = nseg_for(L);
  a.use_log = use_log; a.has_s0 = s0 != nullptr;
  const size_t need = dgda_chunk_workspace(BH, L);
  if (ws_bytes < need) return fail(MABA_ERR_WORKSPACE, "dgda_prefill: workspace too small");
  a.agg = (float*)ws;
  a.sstart = a.agg + BH * a.nseg * 64 * 128;
  if (a.nseg > 1) {
    hipLaunchKernelGGL(dgda_chunk_kernel<true>, dim3((unsigned)(BH * a.nseg)), dim3(512), 0, stream, a);
    int rc = check_launch("dgda_prefill/aggregate");
    if (rc) return rc;
    hipLaunchKernelGGL(dgda_segment_scan_kernel, dim3((unsigned)(BH * 4)), dim3(64), 0, stream, a);
    rc = check_launch("dgda_prefill/scan");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(dgda_chunk_kernel<false>, dim3((unsigned)(BH * a.nseg)), dim3(256), 0, stream, a);
  return check_launch("dgda_prefill/output");
}

}  // namespace maba

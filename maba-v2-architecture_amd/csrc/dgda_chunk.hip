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
// With decays <= 1 every factor is <= 1, so nothing overflows; decays above one are
// taken as they are (the factors then grow as the recurrence's state does).
//
// Sequence parallelism (only B*H = 40 recurrences at the BASELINE shape, but
// 256 CUs): the (b,h)-major sequence of all B*H*nchunks chunks is cut into slots
// of U chunks, U = max(CPS, ceil(total / (2 * CUs))), so that the output pass runs
// exactly one wave of workgroups (two per CU) of equal length.  A segment is the
// part of one (b,h) sequence inside one slot; each (b,h) has up to nseg_max.
//   pass 1 (dgda_chunk_kernel<AGG>) runs every segment but the first of each (b,h)
//          from a zero state, carrying X = [N | M] (64 x 128): N is the segment's
//          state from S0 = 0, M its state transition (X starts as [0 | I], the M
//          half gets no input), so S_end = M S_start + N.
//   passes 2 and 3 (dgda_chunk_kernel<OUT>) run the segments for the outputs (and
//          the final state from the last segment), see the modes below.  A segment's
//          true start state is S_{s+1} = M_s S_s + N_s, and simply N_s wherever N_s
//          is already exact.
//
// Workgroup layout: wave w owns 16 columns of the carried state (pass 1: 8 waves
// over the 128 columns of [N | M]; pass 3: 4 waves over the 64 columns of S).
// Per chunk the workgroup stages k (and q) in LDS, builds L, A and the 16x16
// diagonal-block inverses T_II = (I + L_II)^-1 (one wave), then each wave runs
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
#include "dgda_common.h"

namespace maba {


constexpr int CH = 64;        // chunk length (tokens)
constexpr int DK = 64;        // key / value head size
constexpr int TPITCH = 20;    // bf16 row pitch of the 16x16 inverse blocks
constexpr int CPS = 16;       // chunks per segment
// The aggregate pass's bound (see chunk_segment): chunks probed, the log-decay at which the start
// state no longer counts, and the largest b |k|^2 taken as a contraction (2, less a margin for
// the rounding of the fp32 sums).
constexpr int ZC_PROBE = 4;
constexpr float ZC_LOG = -80.f;
constexpr float ZC_CONTRACT = 1.99f;

// Output-kernel modes.  Pass 1 records zc[s] for every segment s >= 1 of a (b,h):
// the number of chunks after which its transition M is exactly zero in fp32 (-1 if
// it never is); from there on the segment's state, and so its outputs, no longer
// depend on its start state.  OUT_ZERO (one workgroup per slot) runs segment 0 from
// the true initial state and every segment with zc[s] >= 0 from a zero start,
// writing all their outputs and their final states N_s (the true final state for
// segment 0); N_s is then exact wherever s = 0 or zc[s] >= 0.  OUT_FIX (one
// workgroup per segment s >= 1) re-runs the first zc[s] chunks of those segments
// from the true start state, and every segment whose M never vanished in full; it
// forms its start state itself from the last exact N_j and the maps (M, N) of the
// segments between.
// With fast decay zc[s] is 1 or 2, so the aggregate and fix-up passes shrink to a
// chunk or two per segment.  With one segment per (b,h) only OUT_ZERO runs.
constexpr int OUT_ZERO = 1, OUT_FIX = 2;

// Element strides are 32-bit (the host checks that they fit): the kernel arguments
// live in scalar registers for the whole kernel.
struct ChunkArgs {
  const uint16_t* q; int qs0, qs1, qs2;       // bf16 [B,H,L,64], channel stride 1
  const uint16_t* k; int ks0, ks1, ks2;
  const uint16_t* vp; int vs0, vs1, vs2;
  const float* gp; int gs0, gs1, gs2;         // log_alpha (use_log) or alpha, fp32, per token
  const float* bp; int bs0, bs1, bs2;         // erase gate b, fp32, per token
  const float* wp; int ws0, ws1, ws2, ws3;    // write gate w, fp32 (per token when ws3 == 0)
  View4 s0;
  int w_tok;                                  // write gate is per token (stride-0 channels)
  void* op; int os0, os1, os2, os3;           // output (bf16 or fp32, see OBF)
  MView4 sf;
  float* agg;      // [BH, nseg_max, 64, 128]
  int* zc;         // [BH, nseg_max]: chunks after which the segment's transition M is exactly zero, -1 if never
  int64_t U;       // chunks per slot
  int H, L, BH, nseg_max, nchunks, use_log, has_s0;
  int mode;        // output kernel: OUT_ZERO or OUT_FIX
};

__device__ __forceinline__ int seg_count(const ChunkArgs& a, int bh) { return seg_count_of(a.nchunks, a.U, bh); }
__device__ __forceinline__ void seg_range(const ChunkArgs& a, int bh, int k, int n, int& c0, int& c1) {
  seg_range_of(a.nchunks, a.U, bh, k, n, c0, c1);
}

// Lower-triangular 64x64 matrices are stored as their 10 lower 16x16 tiles
// (tile (I,J), J <= I, at index I(I+1)/2 + J), rows padded to TPITCH.
__device__ __forceinline__ int tri_tile(int I, int J) { return I * (I + 1) / 2 + J; }
constexpr int TILE_ELEMS = 16 * TPITCH;

// Columns 4g..4g+3 of row r of tile (I,J).
__device__ __forceinline__ i16x4 tri4(const short* base, int I, int J, int r, int g) {
  return *(const i16x4*)(base + tri_tile(I, J) * TILE_ELEMS + r * TPITCH + 4 * g);
}
// Permuted-K operand spanning tiles (I,J) and (I,J+1).
__device__ __forceinline__ i16x8 tri4x2(const short* base, int I, int J, int r, int g) {
  return cat8(tri4(base, I, J, r, g), tri4(base, I, J + 1, r, g));
}


// fp32 copies of the four diagonal 16x16 blocks of L (row pitch DPITCH floats).
constexpr int DPITCH = 20;
constexpr int DTILE_ELEMS = 16 * DPITCH;

// T_b = (I + N_b)^-1 for all four 16x16 diagonal blocks N_b = L_bb (strictly lower,
// fp32 copies, row pitch DPITCH) on one wave: lane 16b + j owns column j of block b
// and runs its forward substitution in registers, x_i = [i == j] - sum_{m<i} N_im x_m,
// with no cross-lane traffic (the 16 lanes of a block read the same rows of N).
// The result is stored transposed -- row j of TT_b is column j of T_b -- so that the
// solve reads T_b as an operand with the transposed LDS read.
__device__ __forceinline__ void diag_inverses(const float* LD, short* TH, short* TL, int lane) {
  const int b = lane >> 4, j = lane & 15;
  const float* n = LD + b * DTILE_ELEMS;
  float x[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    // four independent partial sums (one per column residue) keep the chain short
    float acc[4] = {(i == j) ? 1.f : 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (4 * q < i) {
        const f32x4 v = *(const f32x4*)(n + i * DPITCH + 4 * q);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (4 * q + r < i) acc[r] = fmaf(-v[r], x[4 * q + r], acc[r]);
      }
    }
    x[i] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  }
  short* th = TH + b * TILE_ELEMS + j * TPITCH;
  short* tl = TL + b * TILE_ELEMS + j * TPITCH;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    i16x4 hh, ll;
    split4(f32x4{x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]}, hh, ll);
    *(i16x4*)(th + 4 * q) = hh;
    *(i16x4*)(tl + 4 * q) = ll;
  }
}

// ------------------------------------------------------------------ shared memory

// Every member starts on a 16-byte boundary: the 8- and 16-byte LDS accesses and
// the transposed reads need naturally aligned addresses.
#define SM_ALIGN __attribute__((aligned(16)))
template <bool AGG>
struct ChunkSmem {
  SM_ALIGN short K[CH * PITCH];        // k rows (token-major)
  SM_ALIGN short V[CH * PITCH];        // v rows
  SM_ALIGN short Q[AGG ? 8 : CH * PITCH];
  SM_ALIGN short LH[10 * TILE_ELEMS];  // L hi/lo, strictly lower
  SM_ALIGN short LL[10 * TILE_ELEMS];
  SM_ALIGN short AH[AGG ? 8 : 10 * TILE_ELEMS];  // A hi/lo, lower incl. diagonal
  SM_ALIGN short AL[AGG ? 8 : 10 * TILE_ELEMS];
  SM_ALIGN short TH[4 * TILE_ELEMS];   // (I + L_II)^-1 hi/lo, stored transposed
  SM_ALIGN short TL[4 * TILE_ELEMS];
  SM_ALIGN float LD[4 * DTILE_ELEMS];  // L_II in fp32 for the inverses
  SM_ALIGN float lam2[CH];   // inclusive cumulative log-decay, in log2 units
  SM_ALIGN float rf[3][CH];  // 2^{lam2_i - lam2_{16J+15}}: row factors of the off-diagonal tiles (I,J)
  SM_ALIGN float cf[CH];     // 2^{lam2_{16J+15} - lam2_j}, J = j/16: their column factors
  SM_ALIGN float elam[CH];   // e^Lam
  SM_ALIGN float eend[CH];   // e^{Lam_63 - Lam}
  SM_ALIGN float beta[CH];
  SM_ALIGN float bel[CH];    // beta e^Lam
  SM_ALIGN float wtok[CH];
};

// ------------------------------------------------------------------ the chunk kernel

// The kernel's arguments read in place from the kernarg segment (see dgda_chunk_kernel).
typedef const __attribute__((address_space(4))) ChunkArgs KArgs;

// One segment: chunks [c_begin, c_end) of sequence bh, segment k of n.
template <bool AGG, bool WTOK, bool OBF>
__device__ __forceinline__ void chunk_segment(KArgs& a, ChunkSmem<AGG>& sm, int* s_mzero, int tid,
                                              int bh, int k, int n, int c_begin, int c_end) {
  constexpr int NW = AGG ? 8 : 4;
  constexpr int IPT = (CH * 8) / (NW * 64);  // 16-byte staging items per thread
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int bi = bh / a.H, hi = bh % a.H;
  const int64_t sidx = (int64_t)bh * a.nseg_max + k;
  const bool last = k == n - 1;
  if (!AGG && a.mode == OUT_ZERO && k > 0 && a.zc[sidx] < 0) return;  // M never vanished: OUT_FIX runs it in full
  if (!AGG && a.mode == OUT_FIX && a.zc[sidx] >= 0)
    c_end = c_begin + a.zc[sidx];                                     // only the chunks that see the start state
  // OUT_FIX (k >= 1): the start state is N_{k-1} when that is final (k - 1 = 0, or its M vanished)
  const bool pred_final = !AGG && a.mode == OUT_FIX && (k == 1 || a.zc[sidx - 1] >= 0);

  // Carried state slab: S[16kt + 4g + i][col0 + c16] in Sr[kt][i].  The source is
  // chosen once (uniform branches), so the slab's 16 loads issue back to back.
  f32x4 Sr[4];
  const int col0 = (wave & 3) * 16;
  const int col = col0 + c16;
  const bool is_m = AGG && wave >= 4;  // pass 1: M half of [N | M]
  auto fill = [&](auto load) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) Sr[kt][i] = load(16 * kt + 4 * g + i);
  };
  if (AGG) {
    fill([&](int r) { return (is_m && r == col) ? 1.f : 0.f; });
  } else if (k == 0 && a.has_s0) {
    const int64_t o = bi * a.s0.s0 + hi * a.s0.s1 + col * a.s0.s3, rs = a.s0.s2;
    if (a.s0.dt == MABA_F32) fill([&](int r) { return ((const float*)a.s0.p)[o + r * rs]; });
    else if (a.s0.dt == MABA_BF16) fill([&](int r) { return bf16_bits_to_f32(((const uint16_t*)a.s0.p)[o + r * rs]); });
    else fill([&](int r) { return __half2float(((const __half*)a.s0.p)[o + r * rs]); });
  } else if (k == 0 || a.mode == OUT_ZERO) {
    fill([&](int) { return 0.f; });
  } else if (pred_final) {
    const float* src = a.agg + (sidx - 1) * 64 * 128 + col;   // S_k = N_{k-1}
    fill([&](int r) { return src[r * 128]; });
  } else {
    // the predecessor's M did not vanish: start from the last exact final state N_j
    // (segment 0, or one whose M vanished) and apply the maps of the segments between
    const int* zc = a.zc + (int64_t)bh * a.nseg_max;
    int j = k - 1;
    while (j > 0 && zc[j] < 0) --j;
    const float* agg = a.agg + (int64_t)bh * a.nseg_max * 64 * 128;
    const float* src = agg + (int64_t)j * 64 * 128 + col;
    fill([&](int r) { return src[r * 128]; });
    for (int m = j + 1; m < k; ++m) apply_segment_map(agg + (int64_t)m * 64 * 128, Sr, col0, c16, g);
  }

  const uint16_t* qb = a.q + (int64_t)bi * a.qs0 + (int64_t)hi * a.qs1;
  const uint16_t* kb = a.k + (int64_t)bi * a.ks0 + (int64_t)hi * a.ks1;
  const uint16_t* vb = a.vp + (int64_t)bi * a.vs0 + (int64_t)hi * a.vs1;
  const float* gb = a.gp + (int64_t)bi * a.gs0 + (int64_t)hi * a.gs1;
  const float* bb = a.bp + (int64_t)bi * a.bs0 + (int64_t)hi * a.bs1;
  const float* wb = a.wp + (int64_t)bi * a.ws0 + (int64_t)hi * a.ws1 + (WTOK ? 0 : (int64_t)col * a.ws3);
  // output: this lane's column and rows 4g..4g+3 of a 16-row block, advanced per block
  // output (unit column stride): this lane writes token row c16 of each 16-row block,
  // columns col0 + 4g .. +3, as one 8- or 16-byte store
  const int64_t obase = (int64_t)bi * a.os0 + (int64_t)hi * a.os1 + (int64_t)c16 * a.os2 + col0 + 4 * g;

  // Output pass: wave roles rotate by two in the second half of the grid.  The two
  // workgroups of a CU place wave w on the same SIMD, so this pairs the diagonal-
  // inverse wave of one with a five-tile wave of the other, and the six-tile wave with
  // the wave that also forms the gates.
  const int rot = (!AGG && a.mode == OUT_ZERO && blockIdx.x >= gridDim.x / 2) ? 2 : 0;
  const int role = (wave + rot) & 3;
  const bool gate_wave = AGG ? wave == 0 : role == 2;   // forms the per-token gate arrays

  // ---- pass 1: a bound from the gates.  The segment's transition is M = prod_t (I - b_t k_t
  // k_t^T) alpha_t (per-token decay and erase gates); while every token has b_t |k_t|^2 <= 2
  // (and >= 0) each factor I - b_t k_t k_t^T is a contraction (its eigenvalues are 1 and
  // 1 - b_t |k_t|^2), so |M| <= exp(sum_t log alpha_t).  Once
  // that sum falls to ZC_LOG the start state adds less than e^ZC_LOG |S_start| to any later
  // state or output (e^-80 < 2e-35), and the zero-start pass's results from there on stand.
  // Wave 0 sums the log-decays of up to ZC_PROBE chunks (all their gate and key loads issued
  // at once) and checks b_t |k_t|^2 per token; when the bound is reached it records zc as the
  // chunks up to that point and the workgroup ends without a product.  Otherwise (slow decay,
  // or large erase gates or keys) the segment runs on [N | M] below, and zc records where M
  // became exactly zero, or -1.
  if constexpr (AGG) {
    if (wave == 0) {
      float la[ZC_PROBE], kk[ZC_PROBE], be[ZC_PROBE];
#pragma unroll
      for (int j = 0; j < ZC_PROBE; ++j) {
        const int t = (c_begin + j) * CH + lane;
        const bool in = c_begin + j < c_end && t < a.L;
        la[j] = in ? gb[(int64_t)(in ? t : 0) * a.gs2] : 0.f;
        be[j] = in ? bb[(int64_t)(in ? t : 0) * a.bs2] : 0.f;
        kk[j] = 0.f;
        i16x8 kv[8];
#pragma unroll
        for (int c8 = 0; c8 < 8; ++c8) {
          const i16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
          kv[c8] = in ? *(const i16x8*)(kb + (int64_t)(in ? t : 0) * a.ks2 + 8 * c8) : z;
        }
#pragma unroll
        for (int c8 = 0; c8 < 8; ++c8)
#pragma unroll
          for (int e = 0; e < 8; ++e) kk[j] = fmaf(bf16_val(kv[c8][e]), bf16_val(kv[c8][e]), kk[j]);
      }
      int zb = -1;
      float cum = 0.f;
#pragma unroll
      for (int j = 0; j < ZC_PROBE; ++j) {
        if (zb >= 0 || c_begin + j >= c_end) continue;
        float l = a.use_log ? la[j] : __logf(fmaxf(la[j], 1e-20f));
        // A decay above one raises the sum as it should; a NaN never satisfies the bound.
        l = (c_begin + j) * CH + lane < a.L ? l : 0.f;
        const float bk2 = be[j] * kk[j];
        if (__ballot(!(bk2 >= 0.f && bk2 <= ZC_CONTRACT)) != 0ull) break;   // a factor may expand
        cum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_incl_scan(l)), 63));
        if (cum <= ZC_LOG) zb = j + 1;
      }
      if (lane == 0) s_mzero[4] = zb;
    }
    lds_barrier();
    const int zb = s_mzero[4];
    if (zb >= 0) {
      if (tid == 0) a.zc[sidx] = zb;
      return;
    }
  }

  // ---- register prefetch of one chunk's k, v, q rows and per-token gates
  i16x8 pk[IPT], pv[IPT], pq[IPT];
  float pla = 0.f, pbe = 0.f, pwt = 0.f;
  auto prefetch = [&](int cc) {
    const int t0 = cc * CH;
#pragma unroll
    for (int it = 0; it < IPT; ++it) {
      const int i = tid + it * NW * 64;
      const int t = i >> 3, c8 = (i & 7) * 8;
      const i16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
      pk[it] = z; pv[it] = z; pq[it] = z;
      if (t0 + t < a.L) {
        pk[it] = *(const i16x8*)(kb + (int64_t)(t0 + t) * a.ks2 + c8);
        pv[it] = *(const i16x8*)(vb + (int64_t)(t0 + t) * a.vs2 + c8);
        if (!AGG) pq[it] = *(const i16x8*)(qb + (int64_t)(t0 + t) * a.qs2 + c8);
      }
    }
    if (gate_wave) {
      const int t = t0 + lane;
      pla = 0.f; pbe = 0.f; pwt = 0.f;
      if (t < a.L) {
        pla = gb[(int64_t)t * a.gs2];
        pbe = bb[(int64_t)t * a.bs2];
        if (WTOK) pwt = wb[(int64_t)t * a.ws2];
      }
    }
  };
  prefetch(c_begin);
  // Pass 1, M waves: once the wave's 64x16 slab of M is exactly zero it stays zero
  // (k M = 0, so v_e = 0, u = 0 and the update adds nothing), and the wave skips its
  // products for the rest of the segment while still joining every barrier.  With
  // fast decay e^{Lam_63} underflows within a chunk or two.
  bool idle = false;
  if (AGG && tid < 4) s_mzero[tid] = 0;   // pass 1: M slab w of the workgroup is exactly zero
  int c_stop = -1;            // pass 1: chunk at which M was found to be zero

  // Output pass: the hardware fills each CU with one workgroup from the first half of
  // the grid and then one from the second, and among equal priorities the older waves
  // issue first, so the two workgroups of a CU would finish far apart.  They take turns
  // at the higher wave priority from chunk to chunk instead.
  const int prio_phase = (!AGG && a.mode == OUT_ZERO && blockIdx.x >= gridDim.x / 2) ? 1 : 0;
  for (int c = c_begin; c < c_end; ++c) {
    const int t0 = c * CH;
    if (!AGG && a.mode == OUT_ZERO) {
      if ((c + prio_phase) & 1) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
    // per-channel write gate: this wave's 16 values, fetched before the staging barrier
    f32x4 wreg[4];
    if (!WTOK && !is_m) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = t0 + 16 * tt + 4 * g + i;
          wreg[tt][i] = t < a.L ? wb[(int64_t)t * a.ws2] : 0.f;
        }
    }
    lds_barrier();  // previous chunk is done with the shared buffers
    if (AGG && s_mzero[0] && s_mzero[1] && s_mzero[2] && s_mzero[3]) {  // workgroup-uniform
      c_stop = c;
      break;
    }
    // ---- stage the prefetched rows (k, v, q, k^T) and gates, then prefetch the next chunk
#pragma unroll
    for (int it = 0; it < IPT; ++it) {
      const int i = tid + it * NW * 64;
      const int t = i >> 3, c8 = (i & 7) * 8;
      *(i16x8*)(sm.K + t * PITCH + c8) = pk[it];
      *(i16x8*)(sm.V + t * PITCH + c8) = pv[it];
      if (!AGG) *(i16x8*)(sm.Q + t * PITCH + c8) = pq[it];
    }
    if (gate_wave) {   // one wave, lane = token
      float la = a.use_log ? pla : __logf(fmaxf(pla, 1e-20f));
      la = (t0 + lane < a.L) ? la : 0.f;
      const float s = wave_incl_scan(la);   // inclusive prefix sum of the log decay
      const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 63));
      const float el = __expf(s);
      const float l2 = s * 1.4426950408889634f;
      sm.lam2[lane] = l2;
      // Off-diagonal decay factors: for i in block I > J and j in block J,
      // 2^{l2_i - l2_j} = 2^{l2_i - r_J} 2^{r_J - l2_j} with r_J = l2 at token 16J + 15;
      // when no decay exceeds one, l2 does not increase and both factors are <= 1 (rows
      // i <= 16J + 15 never use rf[J]); decays above one give factors above one, as in the
      // recurrence.
      const float rJ[3] = {__int_as_float(__builtin_amdgcn_readlane(__float_as_int(l2), 15)),
                           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l2), 31)),
                           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l2), 47))};
      const float rown = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l2), 63));
      const int jb = lane >> 4;
      const float rj = jb == 0 ? rJ[0] : jb == 1 ? rJ[1] : jb == 2 ? rJ[2] : rown;
      sm.cf[lane] = __builtin_amdgcn_exp2f(rj - l2);
#pragma unroll
      for (int J = 0; J < 3; ++J) sm.rf[J][lane] = __builtin_amdgcn_exp2f(l2 - rJ[J]);
      sm.elam[lane] = el;
      sm.eend[lane] = __expf(last - s);
      sm.beta[lane] = pbe;
      sm.bel[lane] = pbe * el;
      sm.wtok[lane] = pwt;
    }
    if (c + 1 < c_end) prefetch(c + 1);
    lds_barrier();

    // ---- L = beta_i (k k^T) decay (strict lower) and A = (q k^T) decay (lower)
    // Tile (I,J) is computed as D = k_J x k_I^T (or k_J x q_I^T) so each lane holds
    // row 16I + c16 and columns 16J + 4g..+3: one 8-byte store into the tile.  Tile
    // index and kind are compile-time constants, so each wave's tile list is
    // straight-line code whose loads, products and exponentials interleave.
    // e^{Lam_i - Lam_j} = 2^{lam2_i - lam2_j}; off-diagonal tiles (I > J) hold only
    // i > j, diagonal tiles select j < i (L) or j <= i (A).
    auto build_tile = [&](auto tix_c, auto isa_c) {
      constexpr int TIX = decltype(tix_c)::value;
      constexpr bool ISA = decltype(isa_c)::value;
      constexpr int I = TIX < 1 ? 0 : TIX < 3 ? 1 : TIX < 6 ? 2 : 3;
      constexpr int J = TIX - I * (I + 1) / 2;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      const short* Bsrc = ISA ? sm.Q : sm.K;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const i16x8 av = lds8(sm.K, 16 * J + c16, 32 * p + 8 * g, PITCH);
        const i16x8 bv = lds8(Bsrc, 16 * I + c16, 32 * p + 8 * g, PITCH);
        acc = mma32(acc, av, bv);
      }
      const int i = 16 * I + c16;
      f32x4 val;
      if constexpr (I > J) {
        // off-diagonal: the factored decay, row factor (with -beta_i for L: off-diagonal
        // L tiles are stored negated, the solve accumulates -L_IJ u_J onto v_e_I) times
        // the column factors
        const float ri = ISA ? sm.rf[J][i] : -sm.beta[i] * sm.rf[J][i];
        const f32x4 cj = *(const f32x4*)(sm.cf + 16 * J + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) val[r] = (acc[r] * ri) * cj[r];
      } else {
        const float li = sm.lam2[i];
        const f32x4 lj = *(const f32x4*)(sm.lam2 + 16 * J + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * J + 4 * g + r;
          const float x = acc[r] * __builtin_amdgcn_exp2f(li - lj[r]);
          val[r] = (ISA ? j <= i : j < i) ? x : 0.f;
        }
        if (!ISA) val = val * sm.beta[i];
      }
      if (!ISA && I == J) {   // diagonal L tiles only feed the inverses, in fp32
        *(f32x4*)(sm.LD + I * DTILE_ELEMS + c16 * DPITCH + 4 * g) = val;
        return;
      }
      i16x4 h, l;
      split4(val, h, l);
      const int off = (I * (I + 1) / 2 + J) * TILE_ELEMS + c16 * TPITCH + 4 * g;
      *(i16x4*)((ISA ? sm.AH : sm.LH) + off) = h;
      *(i16x4*)((ISA ? sm.AL : sm.LL) + off) = l;
    };
    using std::integral_constant;
#define DGDA_TL(n) build_tile(integral_constant<int, n>{}, std::false_type{})
#define DGDA_TA(n) build_tile(integral_constant<int, n>{}, std::true_type{})
    // Output pass: the wave of role 3 builds the four diagonal L tiles (triangular
    // indices 0, 2, 5, 9) and inverts them at once -- its own LDS writes, read back in
    // order -- while the other roles build the off-diagonal L tiles (1, 3, 4, 6, 7, 8)
    // and the ten A tiles.  Aggregate pass: the eight waves share the ten L tiles and the
    // inverse runs after the barrier on wave 7, whose M slab is idle once it is zero.
    if constexpr (AGG) {
      switch (wave) {
        case 0: DGDA_TL(0); DGDA_TL(8); break;
        case 1: DGDA_TL(1); DGDA_TL(9); break;
        case 2: DGDA_TL(2); break;
        case 3: DGDA_TL(3); break;
        case 4: DGDA_TL(4); break;
        case 5: DGDA_TL(5); break;
        case 6: DGDA_TL(6); break;
        default: DGDA_TL(7); break;
      }
    } else {
      switch (role) {
        case 0: DGDA_TL(1); DGDA_TL(6); DGDA_TA(0); DGDA_TA(3); DGDA_TA(6); DGDA_TA(9); break;
        case 1: DGDA_TL(3); DGDA_TL(7); DGDA_TA(1); DGDA_TA(4); DGDA_TA(7); break;
        case 2: DGDA_TL(4); DGDA_TL(8); DGDA_TA(2); DGDA_TA(5); DGDA_TA(8); break;
        default:
          DGDA_TL(0); DGDA_TL(2); DGDA_TL(5); DGDA_TL(9);
          diag_inverses(sm.LD, sm.TH, sm.TL, lane);
          break;
      }
    }
#undef DGDA_TL
#undef DGDA_TA
    lds_barrier();

    // ---- state-dependent products: v_e = w*v - diag(beta e^Lam)(k S) and q S
    // (aggregate pass: overlapped with the inverses on wave 7)
    if (AGG && wave == NW - 1) diag_inverses(sm.LD, sm.TH, sm.TL, lane);
    i16x4 Sh[4], Sl[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) split4(Sr[kt], Sh[kt], Sl[kt]);
    f32x4 qsr[4];
    if (!AGG) {
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        f32x4 qs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          // operands swapped: lane (c16, g) gets (q S)[token 16I + c16][col0 + 4g .. +3]
          const i16x8 bv = lds4x2(sm.Q, 16 * I + c16, 32 * p + 4 * g, PITCH);
          qs = mma32(qs, cat8(Sh[2 * p], Sh[2 * p + 1]), bv);
          qs = mma32(qs, cat8(Sl[2 * p], Sl[2 * p + 1]), bv);
        }
        qsr[I] = qs;
      }
    }
    f32x4 u[4];
    if (!idle) {
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const i16x8 av = lds4x2(sm.K, 16 * tt + c16, 32 * p + 4 * g, PITCH);
        acc = mma32(acc, av, cat8(Sh[2 * p], Sh[2 * p + 1]));
        acc = mma32(acc, av, cat8(Sl[2 * p], Sl[2 * p + 1]));
      }
      // tokens 16tt + 4g .. +3 of this lane's column: gate products as one 16-byte read,
      // the v column fragment as one transposed read
      const f32x4 bel = *(const f32x4*)(sm.bel + 16 * tt + 4 * g);
      f32x4 y = {0.f, 0.f, 0.f, 0.f};
      if (!is_m) {
        const i16x4 vc = ldsT4(sm.V, 16 * tt, col0, c16, g, PITCH);
        const f32x4 wv = WTOK ? *(const f32x4*)(sm.wtok + 16 * tt + 4 * g) : wreg[tt];
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = wv[i] * bf16_val(vc[i]);
      }
      u[tt] = y - bel * acc;
    }
    }
    if (AGG) lds_barrier();   // the inverses run after the tile barrier only in the aggregate pass

    // ---- blocked forward substitution, u_I = T_II (v_e_I - sum_{J<I} L_IJ u_J): the
    // negated L tiles accumulate onto v_e_I itself; K=16 products never accumulate onto
    // a K=32 result, so I = 3 sums its two parts on the VALU
    i16x4 uh[4], ul[4];
    if (!idle) {
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 rhs = u[I];
      if (I >= 2) {  // J = 0,1 as one K = 32 step
        const i16x8 ah = tri4x2(sm.LH, I, 0, c16, g), al = tri4x2(sm.LL, I, 0, c16, g);
        const i16x8 bh8 = cat8(uh[0], uh[1]), bl8 = cat8(ul[0], ul[1]);
        rhs = mma32(rhs, ah, bh8);
        rhs = mma32(rhs, ah, bl8);
        rhs = mma32(rhs, al, bh8);
      }
      if (I == 1 || I == 3) {  // the remaining 16-wide step J = I-1
        const int J = I - 1;
        const i16x4 ah = tri4(sm.LH, I, J, c16, g), al = tri4(sm.LL, I, J, c16, g);
        f32x4 acc16 = I == 1 ? rhs : f32x4{0.f, 0.f, 0.f, 0.f};
        acc16 = mma16(acc16, ah, uh[J]);
        acc16 = mma16(acc16, ah, ul[J]);
        acc16 = mma16(acc16, al, uh[J]);
        rhs = I == 1 ? acc16 : rhs + acc16;
      }
      i16x4 rh, rl;
      split4(rhs, rh, rl);
      const i16x4 th = ldsT4(sm.TH + I * TILE_ELEMS, 0, 0, c16, g, TPITCH);   // T_I[c16][4g..4g+3]
      const i16x4 tl = ldsT4(sm.TL + I * TILE_ELEMS, 0, 0, c16, g, TPITCH);
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      x = mma16(x, th, rh);
      x = mma16(x, th, rl);
      x = mma16(x, tl, rh);
      u[I] = x;
      split4(x, uh[I], ul[I]);
    }
    }

    // ---- outputs: o = diag(e^Lam) (q S) + A u, computed transposed (u as the A
    // operand, the A tiles as the B operand) so that lane (c16, g) holds token
    // 16I + c16, columns col0 + 4g .. +3
    if (!AGG) {
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const int tl = 16 * I + c16;
        // the products accumulate onto e^Lam (q S); with a K=16 product after K=32 ones
        // (I = 2) the two parts are summed on the VALU (see the solve)
        f32x4 ov = sm.elam[tl] * qsr[I];
#pragma unroll
        for (int P = 0; P < 2; ++P) {  // J pairs (0,1), (2,3)
          if (2 * P + 1 <= I) {
            const i16x8 ah = tri4x2(sm.AH, I, 2 * P, c16, g), al = tri4x2(sm.AL, I, 2 * P, c16, g);
            const i16x8 bh8 = cat8(uh[2 * P], uh[2 * P + 1]), bl8 = cat8(ul[2 * P], ul[2 * P + 1]);
            ov = mma32(ov, bh8, ah);
            ov = mma32(ov, bl8, ah);
            ov = mma32(ov, bh8, al);
          }
        }
        if ((I & 1) == 0) {  // single J = I
          const i16x4 ah = tri4(sm.AH, I, I, c16, g), al = tri4(sm.AL, I, I, c16, g);
          f32x4 au16 = I == 0 ? ov : f32x4{0.f, 0.f, 0.f, 0.f};
          au16 = mma16(au16, uh[I], ah);
          au16 = mma16(au16, ul[I], ah);
          au16 = mma16(au16, uh[I], al);
          ov = I == 0 ? au16 : ov + au16;
        }
        if (t0 + tl < a.L) {
          const int64_t off = obase + (int64_t)(t0 + 16 * I) * a.os2;
          if (OBF) *(bf16x4*)((short*)a.op + off) = to_bf16x4(ov);
          else *(f32x4*)((float*)a.op + off) = ov;
        }
      }
    }

    // ---- state update: S = e^{Lam_63} S + k^T diag(e^{Lam_63 - Lam}) u
    if (idle) continue;
    i16x4 wh[4], wl[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const f32x4 x = u[tt] * *(const f32x4*)(sm.eend + 16 * tt + 4 * g);
      split4(x, wh[tt], wl[tt]);
    }
    const float gdec = sm.elam[CH - 1];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      f32x4 acc = Sr[kt] * gdec;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const i16x8 av = ldsT4x2(sm.K, 32 * p, 16 * kt, c16, g);
        acc = mma32(acc, av, cat8(wh[2 * p], wh[2 * p + 1]));
        acc = mma32(acc, av, cat8(wl[2 * p], wl[2 * p + 1]));
      }
      Sr[kt] = acc;
    }
    if (AGG && is_m) {
      bool nz = false;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) nz |= Sr[kt][i] != 0.f;
      idle = __ballot(nz) == 0ull;
      if (lane == 0) s_mzero[wave - 4] = idle;   // read after the next loop-top barrier
    }
  }

  // ---- segment results
  if (AGG) {
    if (tid == 0) a.zc[sidx] = c_stop >= 0 ? c_stop - c_begin : -1;
    if (c_stop < 0) {  // M never vanished: [N | M] for the fix-up pass
      float* dst = a.agg + sidx * 64 * 128;
      const int cc = (is_m ? 64 : 0) + col;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[(16 * kt + 4 * g + i) * 128 + cc] = Sr[kt][i];
    }
  } else if (a.mode == OUT_ZERO && !last) {  // N_k for the fix-up pass
    float* dst = a.agg + sidx * 64 * 128;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[(16 * kt + 4 * g + i) * 128 + col] = Sr[kt][i];
  } else if (last && !(a.mode == OUT_FIX && a.zc[sidx] >= 0)) {
    const int64_t o = bi * a.sf.s0 + hi * a.sf.s1 + col * a.sf.s3, rs = a.sf.s2;
    auto drain = [&](auto put) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) put(o + (16 * kt + 4 * g + i) * rs, Sr[kt][i]);
    };
    if (a.sf.dt == MABA_F32) drain([&](int64_t e, float v) { ((float*)a.sf.p)[e] = v; });
    else if (a.sf.dt == MABA_BF16) drain([&](int64_t e, float v) { ((uint16_t*)a.sf.p)[e] = f32_to_bf16_bits(v); });
    else drain([&](int64_t e, float v) { ((__half*)a.sf.p)[e] = __float2half(v); });
  }
}

template <bool AGG, bool WTOK, bool OBF>
__global__ __launch_bounds__(AGG ? 512 : 256, AGG ? 1 : 2) void dgda_chunk_kernel(ChunkArgs a) {
  __shared__ ChunkSmem<AGG> sm;
  __shared__ int s_mzero[5];   // [0, 4): the M slabs' zero flags; [4]: the bound's chunk count
  // Pass 1 and OUT_FIX: one workgroup per segment k >= 1.  OUT_ZERO: slot w covers
  // the chunks [U w, U w + U) of the (b,h)-major order, one segment per sequence it
  // touches.  Both walk the same loop so the segment body is inlined once.
  const bool per_segment = AGG || a.mode == OUT_FIX;
  const int64_t total = (int64_t)a.BH * a.nchunks;
  int64_t G = per_segment ? 0 : (int64_t)blockIdx.x * a.U;
  const int64_t Gend = per_segment ? 1 : min(G + a.U, total);
  while (G < Gend) {
    int bh, k, n, c0, c1;
    if (per_segment) {
      const int per = a.nseg_max - 1;
      bh = blockIdx.x / per;
      k = blockIdx.x % per + 1;
      n = seg_count(a, bh);
      if (k >= n) return;
      seg_range(a, bh, k, n, c0, c1);
      G = Gend;
    } else {
      bh = (int)(G / a.nchunks);
      const int64_t s = (int64_t)bh * a.nchunks;
      c0 = (int)(G - s);
      c1 = (int)(min(Gend, s + a.nchunks) - s);
      k = c0 == 0 ? 0 : (int)(blockIdx.x - s / a.U);
      n = seg_count(a, bh);
      G = s + c1;
    }
    // The thread index and the argument pointer pass through empty asm statements so
    // that nothing derived from them is hoisted out of this loop and held across the
    // segments: the segment body reads its arguments where it uses them (scalar loads
    // from the kernarg segment, where the single ChunkArgs argument sits at offset 0).
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    KArgs* ap = (KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    chunk_segment<AGG, WTOK, OBF>(*ap, sm, s_mzero, tid, bh, k, n, c0, c1);
  }
}

// ------------------------------------------------------------------ host side

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

bool dgda_chunk_strides_fit(const maba_tensor* t) {
  for (int d = 0; d < t->ndim; ++d)
    if (t->stride[d] < 0 || t->stride[d] > INT32_MAX) return false;
  return true;
}

bool dgda_chunk_supported(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                          const maba_tensor* gate, const maba_tensor* b) {
  if (!q || !k || !v || !gate || !b) return false;
  if (q->dtype != MABA_BF16 || k->dtype != MABA_BF16 || v->dtype != MABA_BF16) return false;
  if (q->shape[3] != DK || v->shape[3] != DK) return false;
  if (q->stride[3] != 1 || k->stride[3] != 1 || v->stride[3] != 1) return false;
  if (gate->stride[3] != 0 || b->stride[3] != 0) return false;  // per-token decay and erase gate
  if (gate->dtype != MABA_F32 || b->dtype != MABA_F32) return false;
  if (q->shape[2] > (int64_t)1 << 30) return false;
  for (const maba_tensor* t : {q, k, v}) {
    if (!aligned16(t->data)) return false;
    for (int d = 0; d < 3; ++d)
      if (t->shape[d] > 1 && (t->stride[d] % 8) != 0) return false;
  }
  for (const maba_tensor* t : {q, k, v, gate, b})
    if (!dgda_chunk_strides_fit(t)) return false;
  return true;
}

static SlotGeom chunk_geom(int64_t BH, int64_t L) {
  const int64_t nch = ceil_div(L, CH) > 0 ? ceil_div(L, CH) : 1;
  return slot_geom(BH, nch, CPS);
}

size_t dgda_chunk_workspace(int64_t BH, int64_t L) {
  const SlotGeom gm = chunk_geom(BH, L);
  if (gm.nseg_max <= 1) return 16;
  const int64_t nseg = gm.nseg_max;
  return (size_t)(BH * nseg * 64 * 128) * sizeof(float) + (size_t)(BH * nseg) * sizeof(int);
}

int launch_dgda_chunk(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                      const maba_tensor* gate, int use_log, const maba_tensor* b,
                      const maba_tensor* w, const maba_tensor* s0, maba_tensor* out,
                      maba_tensor* sf, void* ws, size_t ws_bytes, hipStream_t stream) {
  const int64_t B = q->shape[0], H = q->shape[1], L = q->shape[2];
  const int64_t BH = B * H;
  ChunkArgs a;
  // strides fit in int32 (dgda_chunk_supported and the caller check every operand)
  a.q = (const uint16_t*)q->data; a.qs0 = (int)q->stride[0]; a.qs1 = (int)q->stride[1]; a.qs2 = (int)q->stride[2];
  a.k = (const uint16_t*)k->data; a.ks0 = (int)k->stride[0]; a.ks1 = (int)k->stride[1]; a.ks2 = (int)k->stride[2];
  a.vp = (const uint16_t*)v->data; a.vs0 = (int)v->stride[0]; a.vs1 = (int)v->stride[1]; a.vs2 = (int)v->stride[2];
  a.gp = (const float*)gate->data; a.gs0 = (int)gate->stride[0]; a.gs1 = (int)gate->stride[1];
  a.gs2 = (int)gate->stride[2];
  a.bp = (const float*)b->data; a.bs0 = (int)b->stride[0]; a.bs1 = (int)b->stride[1]; a.bs2 = (int)b->stride[2];
  a.wp = (const float*)w->data; a.ws0 = (int)w->stride[0]; a.ws1 = (int)w->stride[1]; a.ws2 = (int)w->stride[2];
  a.ws3 = (int)w->stride[3];
  a.s0 = view4(s0);
  a.w_tok = w->stride[3] == 0;
  a.op = out->data; a.os0 = (int)out->stride[0]; a.os1 = (int)out->stride[1]; a.os2 = (int)out->stride[2];
  a.os3 = (int)out->stride[3];
  a.sf = mview4(sf);
  a.H = (int)H; a.L = (int)L; a.BH = (int)BH;
  a.nchunks = (int)(ceil_div(L, CH) > 0 ? ceil_div(L, CH) : 1);
  const SlotGeom gm = chunk_geom(BH, L);
  a.U = gm.U;
  a.nseg_max = gm.nseg_max;
  a.use_log = use_log; a.has_s0 = s0 != nullptr;
  const size_t need = dgda_chunk_workspace(BH, L);
  if (ws_bytes < need) return fail(MABA_ERR_WORKSPACE, "dgda_prefill: workspace too small");
  const int64_t nsegs = BH * a.nseg_max;
  a.agg = (float*)ws;
  a.zc = (int*)(a.agg + nsegs * 64 * 128);
  const bool obf = out->dtype == MABA_BF16;
  auto launch_out = [&](int mode) {
    a.mode = mode;
    const dim3 grid(mode == OUT_ZERO ? (unsigned)ceil_div(BH * a.nchunks, a.U) : (unsigned)(BH * (a.nseg_max - 1)));
    if (a.w_tok && obf) hipLaunchKernelGGL((dgda_chunk_kernel<false, true, true>), grid, dim3(256), 0, stream, a);
    else if (a.w_tok) hipLaunchKernelGGL((dgda_chunk_kernel<false, true, false>), grid, dim3(256), 0, stream, a);
    else if (obf) hipLaunchKernelGGL((dgda_chunk_kernel<false, false, true>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((dgda_chunk_kernel<false, false, false>), grid, dim3(256), 0, stream, a);
    return check_launch("dgda_prefill/output");
  };
  if (a.nseg_max == 1) {
    a.zc = nullptr;
    return launch_out(OUT_ZERO);
  }
  a.mode = OUT_ZERO;
  const dim3 agrid((unsigned)(BH * (a.nseg_max - 1)));
  if (a.w_tok) hipLaunchKernelGGL((dgda_chunk_kernel<true, true, true>), agrid, dim3(512), 0, stream, a);
  else hipLaunchKernelGGL((dgda_chunk_kernel<true, false, true>), agrid, dim3(512), 0, stream, a);
  int rc = check_launch("dgda_prefill/aggregate");
  if (rc) return rc;
  if ((rc = launch_out(OUT_ZERO))) return rc;
  return launch_out(OUT_FIX);
}

}  // namespace maba

// DGDA prefill for per-channel gates (decay, erase and write gates [B,H,L,d] with
// unit or zero channel stride): the layer's gate layout, and every head size the
// reference's GPU prefill takes (d_k, d_v in {32, 64, 128}, triton_dgda.py:389-396):
// the kernels are instantiated for d_k in {32, 64, 128} and d_v in {32, 64}; d_v = 128
// runs as two d_v = 64 calls over the two halves of the value columns (the recurrence
// is separable over value columns: every operation on them is column by column given
// the key-side quantities).  q, k, v in bf16, fp16 or fp32.
//
// Sub-chunks of SC = 16 tokens.  With Lam_i the inclusive cumulative log-decay of
// token i within the sub-chunk (a d_k-vector over key channels) and S the state at the
// sub-chunk start (reference math: cpu_dgda.py:101-146, common.py:229-268):
//   L_ij = sum_c (b*k)_ic k_jc e^{Lam_ic - Lam_jc}      i > j
//   A_ij = sum_c  q_ic    k_jc e^{Lam_ic - Lam_jc}      i >= j
//   u    = (I + L)^-1 (w*v - (b*k*e^Lam) S)
//   o    = (q*e^Lam) S + A u
//   S'   = diag(e^{Lam_15}) S + (k*e^{Lam_15 - Lam})^T u
// With decay gates a <= 1 every factor above is e^{<= 0}; gates above 1 (growth) are
// taken as the token recurrence takes them.  L and A are computed as
// (b*k*e^Lam)(k*e^{-Lam})^T and (q*e^Lam)(k*e^{-Lam})^T on MFMA when |Lam| <= 64 at every
// token and channel of the sub-chunk (so e^{+-Lam} stay far inside fp32), and pair by
// pair with exact exponentials on the VALU otherwise.  Products
// with fp32 operands split them into bf16 hi + lo (three MFMAs), so they carry ~16
// mantissa bits; the state stays in fp32 registers.
//
// MFMA layouts (16x16 tiles, lane (c16, g)): a result lane holds rows 4g..4g+3 of
// column c16.  The per-token vectors v_e, u and o of a wave's 16 state columns are in
// that layout (tokens 4g + i, column c16), which is the B-operand layout of the K = 16
// products T u, A u and (K_C^T) u, so they chain without data movement; the state slab
// Sr[kt] holds rows 16 kt + 4g + i of column c16 (the layout the segment map uses).
//
// Sequence parallelism, passes and modes: as the chunked path in dgda_chunk.hip (slots
// of U sub-chunks, aggregate [N | M] pass, zero-start and fix-up output passes).
//
// Fused layer prologue (PRO, d_k = d_v = 64; maba_hip_dgda_layer_prefill; reference layers/dgda.py:103-121,
// 186-207): the kernels read the layer's six bf16 projections instead of q, k, v and the
// gates, and form the op inputs in the staging step: the causal depthwise conv (kernel 4)
// + SiLU of q, k, v over [history, projections], the per-head L2 norm of k, the decay
// max(-softplus, -14) and the sigmoid erase and write gates, all in fp32 and never
// written back.  A stager lane loads the four conv taps of its token (tokens t-3 .. t,
// the earlier three mostly L1 hits from its neighbours' loads).  The key norm sums the
// 64 channels of a token over four waves: each stager wave leaves its partial sums in LDS
// before the loop-top barrier and the staging after it adds them.
#pragma once
#include "dgda_common.h"

namespace maba {

constexpr int SC = 16;             // tokens per sub-chunk
constexpr int SUB_MIN_U = 64;      // sub-chunks per slot at least (1,024 tokens)
constexpr int SUB_ZERO = 1, SUB_FIX = 2;
constexpr int TP = 20;             // bf16 row pitch of 16-column tiles
constexpr float SUB_MFMA_RANGE = 64.f;   // largest |Lam| within a sub-chunk on the MFMA path

struct SubArgs {
  const void* q; int qs0, qs1, qs2;         // [B,H,L,dk], channel stride 1 (16-bit or fp32, see F32IN)
  const void* k; int ks0, ks1, ks2;
  const void* vp; int vs0, vs1, vs2;
  // gates: fp32, or 16-bit in q's format (see G16); channel stride 0 or 1
  const void* gp; int gs0, gs1, gs2, gs3;   // log_alpha (use_log) or alpha
  const void* bp; int bs0, bs1, bs2, bs3;   // erase gate b
  const void* wp; int ws0, ws1, ws2, ws3;   // write gate w
  View4 s0;
  void* op; int os0, os1, os2;              // output [B,H,L,dv], channel stride 1 (bf16 or fp32, see OBF)
  MView4 sf;
  float* agg;      // [BH, nseg_max, dk, dv + dk]: [N | M] of segments whose M never vanished, N_k of the others
  int* zc;         // [BH, nseg_max]: sub-chunks after which the segment's M is exactly zero, -1 if never
  int64_t U;       // sub-chunks per slot
  int H, L, BH, nseg_max, nchunks, use_log, has_s0;
  int mode;        // output kernel: SUB_ZERO or SUB_FIX
  // fused prologue (PRO): the six bf16 projections [B, L, C] (q, k, v, decay, erase, write;
  // unit channel stride, head h at channels 64h ..), conv taps [C, 1, 4] (f32/bf16), the
  // bf16 conv history [B, C, 3] (null: zeros) and the key-norm eps
  const uint16_t* px[6]; int pxs0[6], pxs1[6];
  const void* cw[3]; int cwdt; int cwsc[3], cwst[3];
  const uint16_t* ph[3]; int phs0[3], phs1[3], phs2[3];
  float eps;
  int f16;         // 16-bit q, k, v are fp16 (else bf16)
  int of16;        // 16-bit output is fp16 (else bf16)
};
typedef const __attribute__((address_space(4))) SubArgs KSubArgs;

#define SM_ALIGN_SUB __attribute__((aligned(16)))
// fp32 rows of DK (or DV) channels are padded by 4 floats, bf16 rows of DK channels by 8
// (16-byte aligned rows that shift banks).
template <bool AGG, bool PRO, int DK, int DV>
struct SubSmem {
  static constexpr int FK = DK + 4, FV = DV + 4, PK = DK + 8;
  SM_ALIGN_SUB float Q[AGG ? 1 : SC][FK];
  SM_ALIGN_SUB float K[SC][FK];
  SM_ALIGN_SUB float BK[SC][FK];            // b * k
  SM_ALIGN_SUB float WV[SC][FV];            // w * v
  SM_ALIGN_SUB float LA[SC][FK];            // log decay, then the inclusive prefix Lam
  SM_ALIGN_SUB short QEh[AGG ? 8 : SC * PK], QEl[AGG ? 8 : SC * PK];   // q e^Lam
  SM_ALIGN_SUB short BKEh[SC * PK], BKEl[SC * PK];                     // b k e^Lam
  SM_ALIGN_SUB short KIh[SC * PK], KIl[SC * PK];                       // k e^-Lam
  SM_ALIGN_SUB short KCh[DK * TP], KCl[DK * TP];                       // (k e^{Lam_15 - Lam})^T
  SM_ALIGN_SUB short Th[SC * TP], Tl[SC * TP];                               // (I + L)^-1
  SM_ALIGN_SUB short Ah[AGG ? 8 : SC * TP], Al[AGG ? 8 : SC * TP];           // A (lower, with diagonal)
  SM_ALIGN_SUB float Lq[SC][4][4];                                            // L[i][p + 4 r] at [i][p][r]
  SM_ALIGN_SUB float elast[DK];                                               // e^{Lam_15}
  SM_ALIGN_SUB float nrm[PRO ? 2 : 1][4][16];   // fused prologue: |k|^2 partials [sub-chunk parity][stager wave][token]
  SM_ALIGN_SUB float cw[PRO ? 3 : 1][4][64];    // fused prologue: the head's conv taps [stream][tap][channel]
  int big[2];                               // some |Lam| exceeds SUB_MFMA_RANGE (by sub-chunk parity)
};

// Raw registers of four consecutive row elements (bf16 bits or fp32).  Prefetched rows
// stay raw until they are staged, so that no conversion waits for the loads.
template <bool F32IN>
using Raw4 = std::conditional_t<F32IN, f32x4, i16x4>;

template <bool F32IN>
__device__ __forceinline__ Raw4<F32IN> load_raw4(const void* base, int64_t off) {
  if constexpr (F32IN) return *(const f32x4*)((const float*)base + off);
  else return *(const i16x4*)((const uint16_t*)base + off);
}
template <bool F32IN>
__device__ __forceinline__ f32x4 raw_f32(Raw4<F32IN> r, bool f16) {
  if constexpr (F32IN) {
    return r;
  } else {
    if (f16) {
      auto h = [](short x) { return __half2float(__ushort_as_half((unsigned short)x)); };
      return f32x4{h(r[0]), h(r[1]), h(r[2]), h(r[3])};
    }
    return f32x4{bf16_val(r[0]), bf16_val(r[1]), bf16_val(r[2]), bf16_val(r[3])};
  }
}

// S <- M S + N for a segment map X = [N | M] (DK x (DV + DK) fp32, row-major: N in columns
// [0, DV), M in [DV, DV + DK)) on the slab Sr[kt][i] = S[16kt + 4g + i][col0 + c16] of one
// wave, with fp32 accuracy (M and S both split into bf16 hi/lo, three products).
template <int DK, int DV>
__device__ __forceinline__ void apply_map(const float* X, f32x4 (&Sr)[DK / 16], int col0, int c16, int g) {
  constexpr int NKT = DK / 16, AW = DV + DK;
  i16x4 Sh[NKT], Sl[NKT];
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt) split4(Sr[kt], Sh[kt], Sl[kt]);
#pragma unroll
  for (int mt = 0; mt < NKT; ++mt) {
    f32x4 acc;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = X[(16 * mt + 4 * g + i) * AW + col0 + c16];  // N
    const int row = 16 * mt + c16;
#pragma unroll
    for (int p = 0; p < DK / 32; ++p) {
      // A operand: M[row][32p + 4g..+3] and [32p + 16 + 4g..+3]
      const f32x4 m0 = *(const f32x4*)(X + row * AW + DV + 32 * p + 4 * g);
      const f32x4 m1 = *(const f32x4*)(X + row * AW + DV + 32 * p + 16 + 4 * g);
      i16x4 h0, l0, h1, l1;
      split4(m0, h0, l0);
      split4(m1, h1, l1);
      const i16x8 ah = cat8(h0, h1), al = cat8(l0, l1);
      const i16x8 bh8 = cat8(Sh[2 * p], Sh[2 * p + 1]), bl8 = cat8(Sl[2 * p], Sl[2 * p + 1]);
      acc = mma32(acc, ah, bh8);
      acc = mma32(acc, ah, bl8);
      acc = mma32(acc, al, bh8);
    }
    Sr[mt] = acc;
  }
}
// Four gate values of one token, channels c0 .. c0+3 at channel stride cs (0 or 1):
// four element loads, the same code for both strides (no branch, so the prefetched
// registers are not merged across paths, which would wait for the loads).  Raw fp32, or
// raw 16-bit (G16).
template <bool G16>
__device__ __forceinline__ Raw4<!G16> load_gate4(const void* base, int64_t off, int cs, int c0) {
  if constexpr (G16) {
    const uint16_t* row = (const uint16_t*)base + off;
    return i16x4{(short)row[c0 * cs], (short)row[(c0 + 1) * cs], (short)row[(c0 + 2) * cs], (short)row[(c0 + 3) * cs]};
  } else {
    const float* row = (const float*)base + off;
    return f32x4{row[c0 * cs], row[(c0 + 1) * cs], row[(c0 + 2) * cs], row[(c0 + 3) * cs]};
  }
}

// Inclusive prefix sum over each 16-lane DPP row (row_shr 1, 2, 4, 8; lanes shifted in
// from outside the row read zero).
__device__ __forceinline__ float row16_incl_scan(float x) {
  auto dpp = [](float v, auto ctrl_c) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), decltype(ctrl_c)::value, 0xf, 0xf, true));
  };
  using std::integral_constant;
  x += dpp(x, integral_constant<int, 0x111>{});
  x += dpp(x, integral_constant<int, 0x112>{});
  x += dpp(x, integral_constant<int, 0x114>{});
  x += dpp(x, integral_constant<int, 0x118>{});
  return x;
}

// One segment: sub-chunks [c_begin, c_end) of sequence bh, segment k of n.
template <bool AGG, bool F32IN, bool G16, bool OBF, bool PRO, int DK, int DV>
__device__ __forceinline__ void sub_segment(KSubArgs& a, SubSmem<AGG, PRO, DK, DV>& sm, int* s_mzero, int tid,
                                            int bh, int k, int n, int c_begin, int c_end) {
  static_assert(!PRO || (DK == 64 && DV == 64), "the fused prologue takes 64-channel heads");
  static_assert((DK == 32 || DK == 64 || DK == 128) && (DV == 32 || DV == 64), "head sizes");
  constexpr int NKT = DK / 16;                   // 16-row tiles of the key side
  constexpr int PK = SubSmem<AGG, PRO, DK, DV>::PK;
  constexpr int AW = DV + DK;                    // row length of a segment map [N | M]
  constexpr int NG = (DK > DV ? DK : DV) / 4;    // four-channel groups staged per token
  constexpr int NPASS = NG > 16 ? NG / 16 : 1;   // staging passes of the 256 stagers (d_k = 128: two)
  constexpr int NSTG = NG >= 16 ? 256 : 16 * NG; // stager threads
  constexpr int NOW = DV / 16;                   // waves holding state columns (aggregate pass: the N waves)
  constexpr int NMW = DK / 16;                   // aggregate pass: the M waves
  constexpr bool HAS_NOCOL = !AGG && DV < 64;    // output passes with d_v = 32: waves 2, 3 hold no columns
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int bi = bh / a.H, hi = bh % a.H;
  const int64_t sidx = (int64_t)bh * a.nseg_max + k;
  const bool last = k == n - 1;
  if (!AGG && a.mode == SUB_ZERO && k > 0 && a.zc[sidx] < 0) return;  // M never vanished: the fix-up runs it
  if (!AGG && a.mode == SUB_FIX && a.zc[sidx] >= 0) c_end = c_begin + a.zc[sidx];
  const bool pred_final = !AGG && a.mode == SUB_FIX && (k == 1 || a.zc[sidx - 1] >= 0);

  // ---- start state: Sr[kt][i] = S[16 kt + 4g + i][col0 + c16]
  f32x4 Sr[NKT];
  const bool is_m = AGG && wave >= NOW;        // aggregate pass: M part of [N | M]
  const bool nocol = HAS_NOCOL && wave >= NOW;
  const int col0 = 16 * (is_m ? wave - NOW : (nocol ? 0 : wave));
  const int col = col0 + c16;
  auto fill = [&](auto load) {
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) Sr[kt][i] = load(16 * kt + 4 * g + i);
  };
  if (AGG) {
    fill([&](int r) { return (is_m && r == col) ? 1.f : 0.f; });
  } else if (nocol) {
    fill([&](int) { return 0.f; });
  } else if (k == 0 && a.has_s0) {
    const int64_t o = bi * a.s0.s0 + hi * a.s0.s1 + col * a.s0.s3, rs = a.s0.s2;
    if (a.s0.dt == MABA_F32) fill([&](int r) { return ((const float*)a.s0.p)[o + r * rs]; });
    else if (a.s0.dt == MABA_BF16) fill([&](int r) { return bf16_bits_to_f32(((const uint16_t*)a.s0.p)[o + r * rs]); });
    else fill([&](int r) { return __half2float(((const __half*)a.s0.p)[o + r * rs]); });
  } else if (k == 0 || a.mode == SUB_ZERO) {
    fill([&](int) { return 0.f; });
  } else if (pred_final) {
    const float* src = a.agg + (sidx - 1) * DK * AW + col;   // S_k = N_{k-1}
    fill([&](int r) { return src[r * AW]; });
  } else {
    // the predecessor's M did not vanish: from the last exact N_j apply the maps of the
    // segments between
    const int* zc = a.zc + (int64_t)bh * a.nseg_max;
    int j = k - 1;
    while (j > 0 && zc[j] < 0) --j;
    const float* agg = a.agg + (int64_t)bh * a.nseg_max * DK * AW;
    const float* src = agg + (int64_t)j * DK * AW + col;
    fill([&](int r) { return src[r * AW]; });
    for (int m = j + 1; m < k; ++m) apply_map<DK, DV>(agg + (int64_t)m * DK * AW, Sr, col0, c16, g);
  }
  // the slab's loads complete here: inside the loop the compiler would otherwise count
  // them as pending and wait for every outstanding load (the prefetch) before using it
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(Sr[kt][i]));

  const int64_t qb = (int64_t)bi * a.qs0 + (int64_t)hi * a.qs1;
  const int64_t kb = (int64_t)bi * a.ks0 + (int64_t)hi * a.ks1;
  const int64_t vb = (int64_t)bi * a.vs0 + (int64_t)hi * a.vs1;
  const int64_t gb = (int64_t)bi * a.gs0 + (int64_t)hi * a.gs1;
  const int64_t bb = (int64_t)bi * a.bs0 + (int64_t)hi * a.bs1;
  const int64_t wb = (int64_t)bi * a.ws0 + (int64_t)hi * a.ws1;
  const int64_t obase = (int64_t)bi * a.os0 + (int64_t)hi * a.os1 + col;

  // ---- register prefetch of one sub-chunk's inputs: item (token st, channels c4..c4+3),
  // tokens along the 16 lanes of a DPP row; pass pp covers channel groups 16 pp .. 16 pp + 15
  // (key-side rows below d_k, value-side rows below d_v: both bounds fall on wave boundaries)
  const bool stager = tid < NSTG;
  const int st = tid & 15;
  const int c4 = (tid >> 4) * 4;                 // pass 0; pass pp adds 64 pp
  Raw4<F32IN> pq[NPASS] = {}, pk[NPASS] = {}, pv[NPASS] = {};
  Raw4<!G16> pg[NPASS] = {}, pb[NPASS] = {}, pw[NPASS] = {};
  // fused prologue: conv taps of tokens t-3 .. t (bf16 bits; taps before token 0 are
  // loaded at token 0 and replaced by the history in the first sub-chunk), the gate
  // projections and SiLU(conv k) of the staged token.  The head's conv weights go to LDS
  // once per segment (the previous segment's last reads of them were before its last
  // post-staging barrier).
  i16x4 tq[4] = {}, tk[4] = {}, tv[4] = {}, xg[3] = {};
  f32x4 kc = {};
  const int ch = hi * 64 + c4;   // the stager's first channel of the projection rows
  if constexpr (PRO) {
    for (int i = tid; i < 3 * 4 * 64; i += blockDim.x) {
      const int s = i >> 8, j = (i >> 6) & 3, cl = i & 63;
      sm.cw[s][j][cl] = load_elem(a.cw[s], a.cwdt, (int64_t)(hi * 64 + cl) * a.cwsc[s] + j * a.cwst[s]);
    }
    lds_barrier();
  }
  // row tr + st of projection s at the stager's channels: a uniform base pointer plus a
  // 32-bit lane offset, clamped to row 0 (rows before token 0 are replaced by the history)
  auto prow = [&](int s, int tr) {
    const uint16_t* base = a.px[s] + (int64_t)bi * a.pxs0[s];
    return *(const i16x4*)(base + max(st * a.pxs1[s] + ch + tr * a.pxs1[s], ch));
  };
  auto prefetch = [&](int cc) {
    const int tok = cc * SC + st;
    if (!stager || tok >= a.L) return;
    if constexpr (PRO) {
      const int t0 = cc * SC;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (!AGG) tq[j] = prow(0, t0 - 3 + j);
        tk[j] = prow(1, t0 - 3 + j);
        tv[j] = prow(2, t0 - 3 + j);
      }
#pragma unroll
      for (int s = 0; s < 3; ++s) xg[s] = prow(3 + s, t0);
      return;
    }
#pragma unroll
    for (int pp = 0; pp < NPASS; ++pp) {
      const int cp = c4 + 64 * pp;
      if (cp < DK) {
        pk[pp] = load_raw4<F32IN>(a.k, kb + (int64_t)tok * a.ks2 + cp);
        if (!AGG) pq[pp] = load_raw4<F32IN>(a.q, qb + (int64_t)tok * a.qs2 + cp);
        pg[pp] = load_gate4<G16>(a.gp, gb + (int64_t)tok * a.gs2, a.gs3, cp);
        pb[pp] = load_gate4<G16>(a.bp, bb + (int64_t)tok * a.bs2, a.bs3, cp);
      }
      if (cp < DV) {
        pv[pp] = load_raw4<F32IN>(a.vp, vb + (int64_t)tok * a.vs2 + cp);
        pw[pp] = load_gate4<G16>(a.wp, wb + (int64_t)tok * a.ws2, a.ws3, cp);
      }
    }
  };
  prefetch(c_begin);

  // outputs of a sub-chunk are stored during the next one's staging, before its prefetch:
  // vmcnt counts stores, and a store issued just before the staging's wait for the
  // prefetched rows would make that wait cover the store's latency
  f32x4 obuf = {0.f, 0.f, 0.f, 0.f};
  int ot0 = -1, ont = 0;
  auto flush = [&]() {
    if (AGG || ot0 < 0) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 4 * g + i;
      if (t < ont) {
        const int64_t off = obase + (int64_t)(ot0 + t) * a.os2;
        if (OBF) ((uint16_t*)a.op)[off] = a.of16 ? __half_as_ushort(__float2half(obuf[i])) : f32_to_bf16_bits(obuf[i]);
        else ((float*)a.op)[off] = obuf[i];
      }
    }
  };
  // fused prologue: SiLU(depthwise conv) of the stager's four channels of stream s from
  // the taps (oldest first)
  auto conv4 = [&](int s, const i16x4 (&t)[4]) {
    f32x4 w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = *(const f32x4*)&sm.cw[s][j][c4];
    f32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float acc = w[3][e] * bf16_val(t[3][e]);
      acc = fmaf(w[2][e], bf16_val(t[2][e]), acc);
      acc = fmaf(w[1][e], bf16_val(t[1][e]), acc);
      acc = fmaf(w[0][e], bf16_val(t[0][e]), acc);
      y[e] = pro_silu(acc);
    }
    return y;
  };
  // taps before token 0 (first sub-chunk of the sequence) come from the history, or are zero
  auto hist_taps = [&](int s, i16x4 (&t)[4]) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      if (st - 3 + j >= 0) continue;
      i16x4 h = {0, 0, 0, 0};
      if (a.ph[s]) {
        const uint16_t* hp = a.ph[s] + (int64_t)bi * a.phs0[s] + (int64_t)ch * a.phs1[s] + (int64_t)(st + j) * a.phs2[s];
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = (short)hp[(int64_t)e * a.phs1[s]];
      }
      t[j] = h;
    }
  };
  // before the loop-top barrier of sub-chunk cc: SiLU(conv k) of the prefetched taps and the
  // wave's |k|^2 partial per token (lanes 16 m + st hold channel groups 4 wave + m of token st)
  auto pre_norm = [&](int cc) {
    if constexpr (PRO) {
      if (!stager) return;
      if (cc == 0) {
        if (!AGG) hist_taps(0, tq);
        hist_taps(1, tk);
        hist_taps(2, tv);
      }
      kc = conv4(1, tk);
      float ss = kc[0] * kc[0] + kc[1] * kc[1] + kc[2] * kc[2] + kc[3] * kc[3];
      ss += __shfl_xor(ss, 16);
      ss += __shfl_xor(ss, 32);
      if (lane < 16) sm.nrm[cc & 1][wave][lane] = ss;
    }
  };

  bool idle = nocol;                     // aggregate pass, M waves: the slab is exactly zero
  if (AGG && tid < NMW) s_mzero[tid] = 0;
  if (tid == 0) sm.big[c_begin & 1] = 0;   // read after the first loop-top barrier
  int c_stop = -1;

  for (int c = c_begin; c < c_end; ++c) {
    const int t0 = c * SC;
    const int nt = min(SC, a.L - t0);
    pre_norm(c);
    lds_barrier();   // the previous sub-chunk is done with the shared buffers
    if (AGG) {
      bool allz = true;
#pragma unroll
      for (int m = 0; m < NMW; ++m) allz = allz && s_mzero[m] != 0;
      if (allz) {   // workgroup-uniform
        c_stop = c;
        break;
      }
    }
    // ---- (1) stage and scale.  The 16 lanes of a DPP row hold the 16 tokens of one
    // four-channel group, so the per-channel prefix Lam over the sub-chunk is a row scan
    // in registers.  Tokens past the end stage as zeros (no decay, no write).
    if (stager) {
      const bool on = st < nt;
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int pp = 0; pp < NPASS; ++pp) {
        const int cp = c4 + 64 * pp;
        f32x4 rk, rv, rq, rg, rb, rw;
        if constexpr (PRO) {
          const float n2 = (sm.nrm[c & 1][0][st] + sm.nrm[c & 1][1][st]) + (sm.nrm[c & 1][2][st] + sm.nrm[c & 1][3][st]);
          rk = kc * pro_knorm_inv(n2, a.eps);
          rv = conv4(2, tv);
          rq = AGG ? z : conv4(0, tq);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            rg[i] = pro_log_decay(bf16_val(xg[0][i]));
            rb[i] = pro_sigmoid(bf16_val(xg[1][i]));
            rw[i] = pro_sigmoid(bf16_val(xg[2][i]));
          }
        } else {
          const bool f16 = a.f16 != 0;
          rk = raw_f32<F32IN>(pk[pp], f16); rv = raw_f32<F32IN>(pv[pp], f16);
          rq = AGG ? z : raw_f32<F32IN>(pq[pp], f16);
          rg = raw_f32<!G16>(pg[pp], f16); rb = raw_f32<!G16>(pb[pp], f16); rw = raw_f32<!G16>(pw[pp], f16);
        }
        if (cp < DV) {
          f32x4 wv;
#pragma unroll
          for (int i = 0; i < 4; ++i) wv[i] = on ? rw[i] * rv[i] : 0.f;
          *(f32x4*)&sm.WV[st][cp] = wv;
        }
        if (cp >= DK) continue;
        const f32x4 kk = on ? rk : z;
        f32x4 la, bk, lam, l15;
        float mx = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float l = a.use_log ? rg[i] : __logf(fmaxf(rg[i], 1e-20f));
          la[i] = on ? l : 0.f;
          bk[i] = on ? rb[i] * rk[i] : 0.f;
          lam[i] = row16_incl_scan(la[i]);
          l15[i] = __shfl(lam[i], lane | 15);
          mx = fmaxf(mx, fabsf(lam[i]));
        }
        if (!(mx <= SUB_MFMA_RANGE)) sm.big[c & 1] = 1;   // benign race: every writer stores 1
        // fp32 rows for the exact pair-by-pair path
        *(f32x4*)&sm.K[st][cp] = kk;
        *(f32x4*)&sm.BK[st][cp] = bk;
        *(f32x4*)&sm.LA[st][cp] = lam;
        if (!AGG) *(f32x4*)&sm.Q[st][cp] = on ? rq : z;
        // scaled operands, split into bf16 hi + lo; e^{-Lam} is used only when |Lam| <= 64
        f32x4 e, ki, kcs, bke;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          e[i] = __expf(lam[i]);
          ki[i] = kk[i] * __expf(-lam[i]);
          kcs[i] = kk[i] * __expf(l15[i] - lam[i]);
          bke[i] = bk[i] * e[i];
        }
        if (st == SC - 1) *(f32x4*)&sm.elast[cp] = e;
        i16x4 h, l;
        split4(bke, h, l);
        *(i16x4*)(sm.BKEh + st * PK + cp) = h;
        *(i16x4*)(sm.BKEl + st * PK + cp) = l;
        split4(ki, h, l);
        *(i16x4*)(sm.KIh + st * PK + cp) = h;
        *(i16x4*)(sm.KIl + st * PK + cp) = l;
        if (!AGG) {
          split4((on ? rq : z) * e, h, l);
          *(i16x4*)(sm.QEh + st * PK + cp) = h;
          *(i16x4*)(sm.QEl + st * PK + cp) = l;
        }
        split4(kcs, h, l);   // transposed: row = channel, column = token
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sm.KCh[(cp + i) * TP + st] = h[i];
          sm.KCl[(cp + i) * TP + st] = l[i];
        }
      }
    }
    if (tid == 0) sm.big[(c + 1) & 1] = 0;   // last read in the previous sub-chunk
    flush();
    if (c + 1 < c_end) prefetch(c + 1);
    lds_barrier();
    const bool big = sm.big[c & 1] != 0;   // workgroup-uniform

    // ---- (4) L and its inverse (wave 0), A (wave 1); every wave: v_e and q S for its columns
    // tile of X (rows i) times KI^T (columns j): lane (c16, g) gets rows 4g + r of column j = c16
    auto tile_mfma = [&](const short* Xh, const short* Xl) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < DK / 32; ++p) {
        const i16x8 xh = lds8(Xh, c16, 32 * p + 8 * g, PK), xl = lds8(Xl, c16, 32 * p + 8 * g, PK);
        const i16x8 kh = lds8(sm.KIh, c16, 32 * p + 8 * g, PK), kl = lds8(sm.KIl, c16, 32 * p + 8 * g, PK);
        acc = mma32(acc, kh, xh);   // D[j][i]: rows of KI as A, rows of X as B
        acc = mma32(acc, kh, xl);
        acc = mma32(acc, kl, xh);
      }
      return acc;   // lane (c16, g), element r: X_i . KI_j with i = c16, j = 4g + r
    };
    if (big) {
      // strong decay: L and A pair by pair in fp32, exact exponentials (all 256 threads of
      // the first four waves, pair (i, j) = (t / 16, t % 16))
      if (tid < SC * SC) {
        const int i = tid >> 4, j = tid & 15;
        float lv = 0.f, av = 0.f;
        if (j <= i) {
          for (int cc = 0; cc < DK; ++cc) {
            const float d = __expf(sm.LA[i][cc] - sm.LA[j][cc]) * sm.K[j][cc];
            lv = fmaf(sm.BK[i][cc], d, lv);
            if (!AGG) av = fmaf(sm.Q[i][cc], d, av);
          }
        }
        sm.Lq[i][j & 3][j >> 2] = j < i ? lv : 0.f;
        if (!AGG) {
          const short hb = bf16_rn(av);
          sm.Ah[i * TP + j] = hb;
          sm.Al[i * TP + j] = bf16_rn(av - bf16_val(hb));
        }
      }
      lds_barrier();
    } else if (wave == 0) {
      const f32x4 d = tile_mfma(sm.BKEh, sm.BKEl);
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.Lq[c16][r][g] = (4 * g + r < c16) ? d[r] : 0.f;   // L[c16][4g + r]
    } else if (!AGG && wave == 1) {
      const f32x4 d = tile_mfma(sm.QEh, sm.QEl);
      f32x4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = (4 * g + r <= c16) ? d[r] : 0.f;
      i16x4 h, l;
      split4(v, h, l);
      *(i16x4*)(sm.Ah + c16 * TP + 4 * g) = h;   // row i = c16, columns j = 4g .. 4g + 3
      *(i16x4*)(sm.Al + c16 * TP + 4 * g) = l;
    }
    if (wave == 0) {
      // T = (I + L)^-1 by forward substitution, x_i = [i == j] - sum_{m<i} L_im x_m for
      // column j: the four lanes 4j .. 4j+3 split the sum by m mod 4 (lane p keeps x_m for
      // m = p, p + 4, ...) and add their parts with two quad DPP steps, so a step costs
      // four FMAs and two DPP adds.  L[i][m] = 0 for m >= i and x_m = 0 until computed,
      // so the products need no guards.  (Wave 0 reads its own LDS writes above in order.)
      const int jc = lane >> 2, p = lane & 3;
      auto qadd = [](float v, auto ctrl_c) {
        return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), decltype(ctrl_c)::value,
                                                              0xf, 0xf, false));
      };
      float xm[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < SC; ++i) {
        const f32x4 lv = *(const f32x4*)&sm.Lq[i][p][0];   // L[i][p + 4 r], r = 0..3
        float part = (p == 0 && i == jc) ? 1.f : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) part = fmaf(-lv[r], xm[r], part);
        part = qadd(part, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
        part = qadd(part, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
        if (p == (i & 3)) xm[i >> 2] = part;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {   // T[p + 4r][jc]
        const short hb = bf16_rn(xm[r]);
        sm.Th[(p + 4 * r) * TP + jc] = hb;
        sm.Tl[(p + 4 * r) * TP + jc] = bf16_rn(xm[r] - bf16_val(hb));
      }
    }
    // v_e = w*v - (b k e^Lam) S and q S: permuted K over the slab's row groups, lane
    // (c16, g) gets tokens 4g + i of column col
    i16x4 Sh[NKT], Sl[NKT];
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) split4(Sr[kt], Sh[kt], Sl[kt]);
    auto state_product = [&](const short* Xh, const short* Xl) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < DK / 32; ++p) {
        const i16x8 xh = lds4x2(Xh, c16, 32 * p + 4 * g, PK), xl = lds4x2(Xl, c16, 32 * p + 4 * g, PK);
        const i16x8 bh8 = cat8(Sh[2 * p], Sh[2 * p + 1]), bl8 = cat8(Sl[2 * p], Sl[2 * p + 1]);
        acc = mma32(acc, xh, bh8);
        acc = mma32(acc, xh, bl8);
        acc = mma32(acc, xl, bh8);
      }
      return acc;
    };
    f32x4 ve = {0.f, 0.f, 0.f, 0.f}, qs = ve;
    if (!idle) {
      ve = state_product(sm.BKEh, sm.BKEl);
#pragma unroll
      for (int i = 0; i < 4; ++i) ve[i] = (is_m ? 0.f : sm.WV[4 * g + i][col]) - ve[i];
    }
    if (!AGG && !idle) qs = state_product(sm.QEh, sm.QEl);
    lds_barrier();   // T (and A) are ready

    // ---- (5) u = T v_e, (6) o = q S + A u, (7) S' = diag(e^{Lam_15}) S + K_C^T u
    if (idle) continue;
    i16x4 vh, vl;
    split4(ve, vh, vl);
    f32x4 u = {0.f, 0.f, 0.f, 0.f};
    {
      const i16x4 th = lds4(sm.Th, c16, 4 * g, TP), tl = lds4(sm.Tl, c16, 4 * g, TP);   // T[c16][4g..]
      // D[m][n] = sum_k T[m][k] v_e[k][n]: A-operand rows of T, B-operand the v_e fragment
      u = mma16(u, th, vh);
      u = mma16(u, th, vl);
      u = mma16(u, tl, vh);
    }
    i16x4 uh, ul;
    split4(u, uh, ul);
    if (!AGG) {
      const i16x4 ah = lds4(sm.Ah, c16, 4 * g, TP), al = lds4(sm.Al, c16, 4 * g, TP);
      f32x4 o = qs;
      o = mma16(o, ah, uh);
      o = mma16(o, ah, ul);
      o = mma16(o, al, uh);
      obuf = o;
      ot0 = t0;
      ont = nt;
    }
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
      const f32x4 el = *(const f32x4*)(sm.elast + 16 * kt + 4 * g);
      f32x4 acc = Sr[kt] * el;
      const i16x4 kh = lds4(sm.KCh, 16 * kt + c16, 4 * g, TP), kl = lds4(sm.KCl, 16 * kt + c16, 4 * g, TP);
      acc = mma16(acc, kh, uh);
      acc = mma16(acc, kh, ul);
      acc = mma16(acc, kl, uh);
      Sr[kt] = acc;
    }
    if (AGG && is_m) {
      bool nz = false;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) nz |= Sr[kt][i] != 0.f;
      idle = __ballot(nz) == 0ull;
      if (lane == 0) s_mzero[wave - NOW] = idle;   // read after the next loop-top barrier
    }
  }

  flush();   // the last sub-chunk's outputs
  if (nocol) return;
  // ---- segment results
  auto drain = [&](auto put) {
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) put(16 * kt + 4 * g + i, Sr[kt][i]);
  };
  if (AGG) {
    if (tid == 0) a.zc[sidx] = c_stop >= 0 ? c_stop - c_begin : -1;
    if (c_stop < 0) {  // M never vanished: [N | M] for the fix-up pass
      float* dst = a.agg + sidx * DK * AW + (is_m ? DV : 0) + col;
      drain([&](int r, float v) { dst[r * AW] = v; });
    }
  } else if (a.mode == SUB_ZERO && !last) {  // N_k for the fix-up pass
    float* dst = a.agg + sidx * DK * AW + col;
    drain([&](int r, float v) { dst[r * AW] = v; });
  } else if (last && !(a.mode == SUB_FIX && a.zc[sidx] >= 0)) {
    const int64_t o = bi * a.sf.s0 + hi * a.sf.s1 + col * a.sf.s3, rs = a.sf.s2;
    if (a.sf.dt == MABA_F32) drain([&](int r, float v) { ((float*)a.sf.p)[o + r * rs] = v; });
    else if (a.sf.dt == MABA_BF16)
      drain([&](int r, float v) { ((uint16_t*)a.sf.p)[o + r * rs] = f32_to_bf16_bits(v); });
    else drain([&](int r, float v) { ((__half*)a.sf.p)[o + r * rs] = __float2half(v); });
  }
}

// Output passes: 256 threads (four waves).  Aggregate pass: one wave per 16 columns of
// [N | M], (d_v + d_k) / 16 waves.
template <bool AGG, bool F32IN, bool G16, bool OBF, bool PRO, int DK, int DV>
__global__ __launch_bounds__(AGG ? 4 * (DK + DV) : 256, AGG ? 1 : 2) void dgda_sub_kernel(SubArgs a) {
  __shared__ SubSmem<AGG, PRO, DK, DV> sm;
  __shared__ int s_mzero[DK / 16];
  // Aggregate and fix-up passes: one workgroup per segment k >= 1.  Output pass: slot
  // w covers the sub-chunks [U w, U w + U) of the (b,h)-major order, one segment per
  // sequence it touches.
  const bool per_segment = AGG || a.mode == SUB_FIX;
  const int64_t total = (int64_t)a.BH * a.nchunks;
  int64_t G = per_segment ? 0 : (int64_t)blockIdx.x * a.U;
  const int64_t Gend = per_segment ? 1 : min(G + a.U, total);
  while (G < Gend) {
    int bh, k, n, c0, c1;
    if (per_segment) {
      const int per = a.nseg_max - 1;
      bh = blockIdx.x / per;
      k = blockIdx.x % per + 1;
      n = seg_count_of(a.nchunks, a.U, bh);
      if (k >= n) return;
      seg_range_of(a.nchunks, a.U, bh, k, n, c0, c1);
      G = Gend;
    } else {
      bh = (int)(G / a.nchunks);
      const int64_t s = (int64_t)bh * a.nchunks;
      c0 = (int)(G - s);
      c1 = (int)(min(Gend, s + a.nchunks) - s);
      k = c0 == 0 ? 0 : (int)(blockIdx.x - s / a.U);
      n = seg_count_of(a.nchunks, a.U, bh);
      G = s + c1;
    }
    // the thread index and the argument pointer pass through empty asm statements so
    // that nothing derived from them is held across the segments
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    KSubArgs* ap = (KSubArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    sub_segment<AGG, F32IN, G16, OBF, PRO, DK, DV>(*ap, sm, s_mzero, tid, bh, k, n, c0, c1);
  }
}


// The aggregate, zero-start and fix-up passes (one zero-start pass when every sequence
// fits one slot).  PRO: the fused-prologue inputs (bf16 projections).  f32in: fp32 q, k,
// v; g16: 16-bit gates in q's format (only with 16-bit q, k, v); obf: 16-bit output.
// The caller has set the workspace pointers for d_k x (d_v + d_k) segment maps.
template <bool PRO, int DK, int DV>
int run_sub_passes(SubArgs& a, bool f32in, bool g16, bool obf, hipStream_t stream) {
#define MABA_SUB_K(AGG, F, G, O, P) dgda_sub_kernel<AGG, F, G, O, P, DK, DV>
  auto launch_out = [&](int mode) {
    a.mode = mode;
    const dim3 grid(mode == SUB_ZERO ? (unsigned)ceil_div((int64_t)a.BH * a.nchunks, a.U)
                                     : (unsigned)(a.BH * (a.nseg_max - 1)));
    if constexpr (PRO) {
      if (obf) hipLaunchKernelGGL((MABA_SUB_K(false, false, false, true, true)), grid, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((MABA_SUB_K(false, false, false, false, true)), grid, dim3(256), 0, stream, a);
    } else if (f32in) {
      if (obf) hipLaunchKernelGGL((MABA_SUB_K(false, true, false, true, false)), grid, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((MABA_SUB_K(false, true, false, false, false)), grid, dim3(256), 0, stream, a);
    } else if (g16) {
      if (obf) hipLaunchKernelGGL((MABA_SUB_K(false, false, true, true, false)), grid, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((MABA_SUB_K(false, false, true, false, false)), grid, dim3(256), 0, stream, a);
    } else {
      if (obf) hipLaunchKernelGGL((MABA_SUB_K(false, false, false, true, false)), grid, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((MABA_SUB_K(false, false, false, false, false)), grid, dim3(256), 0, stream, a);
    }
    return check_launch("dgda_prefill/sub-chunk output");
  };
  if (a.nseg_max == 1) {
    a.zc = nullptr;
    return launch_out(SUB_ZERO);
  }
  a.mode = SUB_ZERO;
  const dim3 agrid((unsigned)(a.BH * (a.nseg_max - 1))), ablock(4 * (DK + DV));
  if constexpr (PRO) hipLaunchKernelGGL((MABA_SUB_K(true, false, false, true, true)), agrid, ablock, 0, stream, a);
  else if (f32in) hipLaunchKernelGGL((MABA_SUB_K(true, true, false, true, false)), agrid, ablock, 0, stream, a);
  else if (g16) hipLaunchKernelGGL((MABA_SUB_K(true, false, true, true, false)), agrid, ablock, 0, stream, a);
  else hipLaunchKernelGGL((MABA_SUB_K(true, false, false, true, false)), agrid, ablock, 0, stream, a);
#undef MABA_SUB_K
  int rc = check_launch("dgda_prefill/sub-chunk aggregate");
  if (rc) return rc;
  if ((rc = launch_out(SUB_ZERO))) return rc;
  return launch_out(SUB_FIX);
}

// One translation unit per d_k instantiates the kernels (dgda_sub_k32.hip, dgda_sub.hip,
// dgda_sub_k128.hip), so that they compile in parallel; dv is 32 or 64.
int run_sub_k32(SubArgs& a, int dv, bool f32in, bool g16, bool obf, hipStream_t stream);
int run_sub_k64(SubArgs& a, int dv, bool f32in, bool g16, bool obf, hipStream_t stream);
int run_sub_k128(SubArgs& a, int dv, bool f32in, bool g16, bool obf, hipStream_t stream);

}  // namespace maba

// Sequence-parallel DGDA prefill for per-channel gates (the DGDA layer's layout:
// decay, erase and write gates [B,H,T,64] with unit channel stride), dk = dv = 64,
// q/k/v in bf16 or fp32.  The recurrence runs token by token, exactly as the
// reference writes it (maba_sparse/kernels/common.py:229-268):
//   S' = diag(a_t) S;   delta = w_t*v_t - S'^T (b_t*k_t);   S = S' + k_t delta^T;   o_t = S^T q_t
// with a_t = exp(log_alpha_t) or alpha_t, and no chunk algebra, so any gate values are
// handled exactly.  Parallelism comes from the slots and segments of the chunked
// path (dgda_chunk.hip): the (b,h)-major token sequence is cut into slots of U
// staging chunks, one output workgroup per slot, two per CU; an aggregate pass
// carries [N | M] per segment until M is exactly zero (zc), and a fix-up pass
// re-runs the first zc chunks of each segment from its true start state.
//
// Workgroup: wave w owns state columns 16(w&3)..+15 (aggregate pass: waves 4-7 carry
// M); lane (rg, cg) = (lane & 7, lane >> 3) holds rows 8 rg .. 8 rg + 7 of two adjacent
// columns.  Per token a wave does 64 VALU products on its slab and reduces the two
// dot products over the eight lanes of each column pair with three DPP steps.  The
// per-token vectors a, b*k, k, q and w*v are staged in LDS for TCH tokens at a time;
// a lane reads 8 rows of each (two 16-byte reads) and its two w*v entries, so the
// broadcast LDS reads per token stay at nine.
#include "dgda_common.h"

namespace maba {

#define SM_ALIGN_TOK __attribute__((aligned(16)))

constexpr int TCH = 32;         // tokens per staging chunk
constexpr int TOK_MIN_U = 32;   // staging chunks per slot at least (1,024 tokens)
constexpr int TOK_ZERO = 1, TOK_FIX = 2;

struct TokArgs {
  const void* q; int qs0, qs1, qs2;         // [B,H,L,64], channel stride 1 (bf16 or fp32, see F32IN)
  const void* k; int ks0, ks1, ks2;
  const void* vp; int vs0, vs1, vs2;
  const float* gp; int gs0, gs1, gs2, gs3;  // log_alpha (use_log) or alpha, fp32, channel stride 0 or 1
  const float* bp; int bs0, bs1, bs2, bs3;  // erase gate b, fp32, channel stride 0 or 1
  const float* wp; int ws0, ws1, ws2, ws3;  // write gate w, fp32, channel stride 0 or 1
  View4 s0;
  void* op; int os0, os1, os2;              // output [B,H,L,64], channel stride 1 (bf16 or fp32, see OBF)
  MView4 sf;
  float* agg;      // [BH, nseg_max, 64, 128]: [N | M] of segments whose M never vanished, N_k of the others
  int* zc;         // [BH, nseg_max]: chunks after which the segment's M is exactly zero, -1 if never
  int64_t U;       // staging chunks per slot
  int H, L, BH, nseg_max, nchunks, use_log, has_s0;
  int mode;        // output kernel: TOK_ZERO or TOK_FIX
};
typedef const __attribute__((address_space(4))) TokArgs KTokArgs;

template <bool AGG>
struct TokSmem {
  SM_ALIGN_TOK float A[TCH][64];    // decay a_t
  SM_ALIGN_TOK float BK[TCH][64];   // b_t * k_t
  SM_ALIGN_TOK float K[TCH][64];
  SM_ALIGN_TOK float Q[AGG ? 1 : TCH][64];
  SM_ALIGN_TOK float WV[TCH][64];   // w_t * v_t
};

// Sum over the eight lanes of a half-row (lanes 8m .. 8m+7): quad swaps of 1 and 2,
// then the half-row mirror, which pairs the two quads.
__device__ __forceinline__ float sum8_lanes(float x) {
  auto dpp = [](float v, auto ctrl_c) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), decltype(ctrl_c)::value, 0xf, 0xf, false));
  };
  using std::integral_constant;
  x += dpp(x, integral_constant<int, 0xB1>{});    // quad_perm [1,0,3,2]
  x += dpp(x, integral_constant<int, 0x4E>{});    // quad_perm [2,3,0,1]
  x += dpp(x, integral_constant<int, 0x141>{});   // row_half_mirror
  return x;
}

// Eight consecutive elements of a bf16 or fp32 row (16-byte aligned), as fp32.
template <bool F32IN>
__device__ __forceinline__ void load8(const void* base, int64_t off, float (&x)[8]) {
  if (F32IN) {
    const f32x4 a = *(const f32x4*)((const float*)base + off), b = *(const f32x4*)((const float*)base + off + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) { x[i] = a[i]; x[4 + i] = b[i]; }
  } else {
    const i16x8 h = *(const i16x8*)((const uint16_t*)base + off);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = bf16_bits_to_f32((uint16_t)h[i]);
  }
}
// Eight consecutive gate values of one token: vector loads for unit channel stride
// (16-byte aligned rows), one broadcast load for stride 0.
__device__ __forceinline__ void gate8(const float* row, int cs, int c0, float (&x)[8]) {
  if (cs == 0) {
    const float v = row[0];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = v;
  } else {
    const f32x4 a = *(const f32x4*)(row + c0), b = *(const f32x4*)(row + c0 + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) { x[i] = a[i]; x[4 + i] = b[i]; }
  }
}

// One segment: staging chunks [c_begin, c_end) of sequence bh, segment k of n.
// Lane (rg, cg) = (lane & 7, lane >> 3) holds S[8 rg + i][col0 + 2 cg + j], i < 8, j < 2.
template <bool AGG, bool F32IN, bool OBF>
__device__ __forceinline__ void tok_segment(KTokArgs& a, TokSmem<AGG>& sm, int* s_mzero, int tid,
                                            int bh, int k, int n, int c_begin, int c_end) {
  const int wave = tid >> 6, lane = tid & 63;
  const int rg = lane & 7, cg = lane >> 3;
  const int bi = bh / a.H, hi = bh % a.H;
  const int64_t sidx = (int64_t)bh * a.nseg_max + k;
  const bool last = k == n - 1;
  if (!AGG && a.mode == TOK_ZERO && k > 0 && a.zc[sidx] < 0) return;  // M never vanished: the fix-up runs it
  if (!AGG && a.mode == TOK_FIX && a.zc[sidx] >= 0) c_end = c_begin + a.zc[sidx];
  const bool pred_final = !AGG && a.mode == TOK_FIX && (k == 1 || a.zc[sidx - 1] >= 0);

  // ---- start state of the slab
  float S[8][2];
  const int col0 = (wave & 3) * 16;
  const int cA = col0 + 2 * cg;            // this lane's columns cA, cA + 1
  const bool is_m = AGG && wave >= 4;
  auto fill = [&](auto load) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) S[i][j] = load(8 * rg + i, cA + j);
  };
  if (AGG) {
    fill([&](int r, int c) { return (is_m && r == c) ? 1.f : 0.f; });
  } else if (k == 0 && a.has_s0) {
    const int64_t o = bi * a.s0.s0 + hi * a.s0.s1, rs = a.s0.s2, cs = a.s0.s3;
    if (a.s0.dt == MABA_F32) fill([&](int r, int c) { return ((const float*)a.s0.p)[o + r * rs + c * cs]; });
    else if (a.s0.dt == MABA_BF16)
      fill([&](int r, int c) { return bf16_bits_to_f32(((const uint16_t*)a.s0.p)[o + r * rs + c * cs]); });
    else fill([&](int r, int c) { return __half2float(((const __half*)a.s0.p)[o + r * rs + c * cs]); });
  } else if (k == 0 || a.mode == TOK_ZERO) {
    fill([&](int, int) { return 0.f; });
  } else if (pred_final) {
    const float* src = a.agg + (sidx - 1) * 64 * 128;   // S_k = N_{k-1}
    fill([&](int r, int c) { return src[r * 128 + c]; });
  } else {
    // the predecessor's M did not vanish: from the last exact N_j apply the maps of the
    // segments between on MFMA (accumulator-tile layout: lane (c16, g4) holds rows
    // 16 kt + 4 g4 + i of column col0 + c16), then move the slab to this layout through
    // a wave-private LDS region (the fix-up pass uses no LDS before its first chunk)
    const int c16 = lane & 15, g4 = lane >> 4;
    const int* zc = a.zc + (int64_t)bh * a.nseg_max;
    int j = k - 1;
    while (j > 0 && zc[j] < 0) --j;
    const float* agg = a.agg + (int64_t)bh * a.nseg_max * 64 * 128;
    f32x4 Sr[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) Sr[kt][i] = agg[(int64_t)j * 64 * 128 + (16 * kt + 4 * g4 + i) * 128 + col0 + c16];
    for (int m = j + 1; m < k; ++m) apply_segment_map(agg + (int64_t)m * 64 * 128, Sr, col0, c16, g4);
    static_assert(offsetof(TokSmem<AGG>, BK) == sizeof(sm.A) && 4 * 64 * 16 <= 2 * TCH * 64,
                  "the four output waves' [64][16] regions span A and BK");
    float* cv = &sm.A[0][0] + wave * 64 * 16;   // [64 rows][16 columns], inside A and BK
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) cv[(16 * kt + 4 * g4 + i) * 16 + c16] = Sr[kt][i];
    fill([&](int r, int c) { return cv[r * 16 + (c - col0)]; });
  }

  const int64_t qb = (int64_t)bi * a.qs0 + (int64_t)hi * a.qs1;
  const int64_t kb = (int64_t)bi * a.ks0 + (int64_t)hi * a.ks1;
  const int64_t vb = (int64_t)bi * a.vs0 + (int64_t)hi * a.vs1;
  const float* gb = a.gp + (int64_t)bi * a.gs0 + (int64_t)hi * a.gs1;
  const float* bb = a.bp + (int64_t)bi * a.bs0 + (int64_t)hi * a.bs1;
  const float* wb = a.wp + (int64_t)bi * a.ws0 + (int64_t)hi * a.ws1;

  bool idle = false;                       // aggregate pass, M waves: the slab is exactly zero
  if (AGG && tid < 4) s_mzero[tid] = 0;
  int c_stop = -1;
  float myo0 = 0.f, myo1 = 0.f;            // outputs of the token this lane stores (tokens t = rg mod 8)
  int myt = -1;

  // ---- register prefetch of one chunk's raw rows and gates: item (token t, 8-channel group)
  const int st = tid >> 3, sc8 = (tid & 7) * 8;   // this thread's staging item (threads < TCH * 8)
  const bool stager = tid < TCH * 8;
  float rk[8], rv[8], rq[8], rgt[8], rb[8], rw[8];
  auto prefetch = [&](int cc) {
    const int tok = cc * TCH + st;
    if (!stager || tok >= a.L) return;
    load8<F32IN>(a.k, kb + (int64_t)tok * a.ks2 + sc8, rk);
    load8<F32IN>(a.vp, vb + (int64_t)tok * a.vs2 + sc8, rv);
    if (!AGG) load8<F32IN>(a.q, qb + (int64_t)tok * a.qs2 + sc8, rq);
    gate8(gb + (int64_t)tok * a.gs2, a.gs3, sc8, rgt);
    gate8(bb + (int64_t)tok * a.bs2, a.bs3, sc8, rb);
    gate8(wb + (int64_t)tok * a.ws2, a.ws3, sc8, rw);
  };
  prefetch(c_begin);

  for (int c = c_begin; c < c_end; ++c) {
    const int t0 = c * TCH;
    const int nt = min(TCH, a.L - t0);
    lds_barrier();   // the previous chunk is done with the staged vectors
    if (AGG && s_mzero[0] && s_mzero[1] && s_mzero[2] && s_mzero[3]) {  // workgroup-uniform
      c_stop = c;
      break;
    }
    // ---- stage the prefetched item (tokens past the sequence are never read: nt bounds
    // the token loop), then prefetch the next chunk
    if (stager && st < nt) {
      float av[8], bkv[8], wvv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        av[i] = a.use_log ? __expf(rgt[i]) : rgt[i];
        bkv[i] = rb[i] * rk[i];
        wvv[i] = rw[i] * rv[i];
      }
      *(f32x4*)&sm.A[st][sc8] = f32x4{av[0], av[1], av[2], av[3]};
      *(f32x4*)&sm.A[st][sc8 + 4] = f32x4{av[4], av[5], av[6], av[7]};
      *(f32x4*)&sm.BK[st][sc8] = f32x4{bkv[0], bkv[1], bkv[2], bkv[3]};
      *(f32x4*)&sm.BK[st][sc8 + 4] = f32x4{bkv[4], bkv[5], bkv[6], bkv[7]};
      *(f32x4*)&sm.K[st][sc8] = f32x4{rk[0], rk[1], rk[2], rk[3]};
      *(f32x4*)&sm.K[st][sc8 + 4] = f32x4{rk[4], rk[5], rk[6], rk[7]};
      if (!AGG) {
        *(f32x4*)&sm.Q[st][sc8] = f32x4{rq[0], rq[1], rq[2], rq[3]};
        *(f32x4*)&sm.Q[st][sc8 + 4] = f32x4{rq[4], rq[5], rq[6], rq[7]};
      }
      *(f32x4*)&sm.WV[st][sc8] = f32x4{wvv[0], wvv[1], wvv[2], wvv[3]};
      *(f32x4*)&sm.WV[st][sc8 + 4] = f32x4{wvv[4], wvv[5], wvv[6], wvv[7]};
    }
    if (c + 1 < c_end) prefetch(c + 1);
    lds_barrier();
    if (idle) continue;

    // ---- tokens in sequence, two at a time: each token's vectors are read while the
    // previous one computes, alternating two register sets
    struct TokVec { f32x4 A[2], B[2], K[2], Q[2]; float W0, W1; };
    auto fetch = [&](int t, TokVec& v) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        v.A[h] = *(const f32x4*)&sm.A[t][8 * rg + 4 * h];
        v.B[h] = *(const f32x4*)&sm.BK[t][8 * rg + 4 * h];
        v.K[h] = *(const f32x4*)&sm.K[t][8 * rg + 4 * h];
        if (!AGG) v.Q[h] = *(const f32x4*)&sm.Q[t][8 * rg + 4 * h];
      }
      if (is_m) {
        v.W0 = 0.f; v.W1 = 0.f;
      } else {
        const float2 w2 = *(const float2*)&sm.WV[t][cA];
        v.W0 = w2.x; v.W1 = w2.y;
      }
    };
    auto token = [&](int t, const TokVec& v) {
      float p0 = 0.f, p1 = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float ai = v.A[i >> 2][i & 3], bi_ = v.B[i >> 2][i & 3];
        S[i][0] *= ai;
        S[i][1] *= ai;
        p0 = fmaf(S[i][0], bi_, p0);
        p1 = fmaf(S[i][1], bi_, p1);
      }
      const float d0 = v.W0 - sum8_lanes(p0), d1 = v.W1 - sum8_lanes(p1);
      float o0 = 0.f, o1 = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float ki = v.K[i >> 2][i & 3];
        S[i][0] = fmaf(ki, d0, S[i][0]);
        S[i][1] = fmaf(ki, d1, S[i][1]);
        if (!AGG) {
          const float qi = v.Q[i >> 2][i & 3];
          o0 = fmaf(S[i][0], qi, o0);
          o1 = fmaf(S[i][1], qi, o1);
        }
      }
      if (!AGG) {
        o0 = sum8_lanes(o0);
        o1 = sum8_lanes(o1);
        if ((t & 7) == rg) { myo0 = o0; myo1 = o1; myt = t0 + t; }
        if ((t & 7) == 7 || t == nt - 1) {   // every lane of a column pair has its token of the last eight
          if (myt >= 0) {
            const int64_t off = (int64_t)bi * a.os0 + (int64_t)hi * a.os1 + (int64_t)myt * a.os2 + cA;
            if (OBF) *(uint32_t*)((uint16_t*)a.op + off) = cvt_pk_bf16(myo0, myo1);
            else *(float2*)((float*)a.op + off) = make_float2(myo0, myo1);
          }
          myt = -1;
        }
      }
    };
    TokVec v0, v1;
    fetch(0, v0);
    for (int t = 0; t < nt; t += 2) {
      if (t + 1 < nt) fetch(t + 1, v1);
      token(t, v0);
      if (t + 1 < nt) {
        if (t + 2 < nt) fetch(t + 2, v0);
        token(t + 1, v1);
      }
    }
    if (AGG && is_m) {
      bool nz = false;
#pragma unroll
      for (int i = 0; i < 8; ++i) nz |= (S[i][0] != 0.f) | (S[i][1] != 0.f);
      idle = __ballot(nz) == 0ull;
      if (lane == 0) s_mzero[wave - 4] = idle;   // read after the next loop-top barrier
    }
  }

  // ---- segment results
  auto drain = [&](auto put) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) put(8 * rg + i, cA + j, S[i][j]);
  };
  if (AGG) {
    if (tid == 0) a.zc[sidx] = c_stop >= 0 ? c_stop - c_begin : -1;
    if (c_stop < 0) {  // M never vanished: [N | M] for the fix-up pass
      float* dst = a.agg + sidx * 64 * 128 + (is_m ? 64 : 0);
      drain([&](int r, int cc, float v) { dst[r * 128 + cc] = v; });
    }
  } else if (a.mode == TOK_ZERO && !last) {  // N_k for the fix-up pass
    float* dst = a.agg + sidx * 64 * 128;
    drain([&](int r, int cc, float v) { dst[r * 128 + cc] = v; });
  } else if (last && !(a.mode == TOK_FIX && a.zc[sidx] >= 0)) {
    const int64_t o = bi * a.sf.s0 + hi * a.sf.s1, rs = a.sf.s2, cs = a.sf.s3;
    if (a.sf.dt == MABA_F32) drain([&](int r, int cc, float v) { ((float*)a.sf.p)[o + r * rs + cc * cs] = v; });
    else if (a.sf.dt == MABA_BF16)
      drain([&](int r, int cc, float v) { ((uint16_t*)a.sf.p)[o + r * rs + cc * cs] = f32_to_bf16_bits(v); });
    else drain([&](int r, int cc, float v) { ((__half*)a.sf.p)[o + r * rs + cc * cs] = __float2half(v); });
  }
}

template <bool AGG, bool F32IN, bool OBF>
__global__ __launch_bounds__(AGG ? 512 : 256, AGG ? 1 : 2) void dgda_tok_kernel(TokArgs a) {
  __shared__ TokSmem<AGG> sm;
  __shared__ int s_mzero[4];
  // Aggregate and fix-up passes: one workgroup per segment k >= 1.  Output pass: slot
  // w covers the staging chunks [U w, U w + U) of the (b,h)-major order, one segment
  // per sequence it touches.
  const bool per_segment = AGG || a.mode == TOK_FIX;
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
    KTokArgs* ap = (KTokArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    tok_segment<AGG, F32IN, OBF>(*ap, sm, s_mzero, tid, bh, k, n, c0, c1);
  }
}

// ------------------------------------------------------------------ host side

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }
static bool fits32(const maba_tensor* t) {
  for (int d = 0; d < t->ndim; ++d)
    if (t->stride[d] < 0 || t->stride[d] > INT32_MAX) return false;
  return true;
}
// fp32 gate with channel stride 0 (per token) or 1 (per channel, 16-byte aligned rows)
static bool gate_ok(const maba_tensor* t) {
  if (!t || t->dtype != MABA_F32 || !fits32(t)) return false;
  if (t->stride[3] == 0) return true;
  if (t->stride[3] != 1 || !al16(t->data)) return false;
  for (int d = 0; d < 3; ++d)
    if (t->shape[d] > 1 && t->stride[d] % 4 != 0) return false;
  return true;
}

bool dgda_tok_supported(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                        const maba_tensor* gate, const maba_tensor* b, const maba_tensor* w,
                        const maba_tensor* out) {
  if (!q || !k || !v || !gate || !b) return false;
  if (q->shape[3] != 64 || v->shape[3] != 64) return false;
  const int dt = q->dtype;
  if ((dt != MABA_BF16 && dt != MABA_F32) || k->dtype != dt || v->dtype != dt) return false;
  const int vec = dt == MABA_BF16 ? 8 : 4;
  for (const maba_tensor* t : {q, k, v}) {
    if (t->stride[3] != 1 || !al16(t->data) || !fits32(t)) return false;
    for (int d = 0; d < 3; ++d)
      if (t->shape[d] > 1 && t->stride[d] % vec != 0) return false;
  }
  if (!gate_ok(gate) || !gate_ok(b)) return false;
  if (w && !gate_ok(w)) return false;
  // outputs go out as column pairs (4- or 8-byte stores)
  if (out && (out->stride[3] != 1 || !fits32(out) || (out->dtype != MABA_BF16 && out->dtype != MABA_F32) ||
              (uintptr_t)out->data % 8 != 0 || out->stride[0] % 2 != 0 || out->stride[1] % 2 != 0 ||
              out->stride[2] % 2 != 0))
    return false;
  return q->shape[2] <= ((int64_t)1 << 30);
}

static SlotGeom tok_geom(int64_t BH, int64_t L) {
  const int64_t nch = ceil_div(L, TCH) > 0 ? ceil_div(L, TCH) : 1;
  return slot_geom(BH, nch, TOK_MIN_U);
}

size_t dgda_tok_workspace(int64_t BH, int64_t L) {
  const SlotGeom gm = tok_geom(BH, L);
  if (gm.nseg_max <= 1) return 16;
  const int64_t nseg = gm.nseg_max;
  return (size_t)(BH * nseg * 64 * 128) * sizeof(float) + (size_t)(BH * nseg) * sizeof(int);
}

int launch_dgda_tok(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                    const maba_tensor* gate, int use_log, const maba_tensor* b,
                    const maba_tensor* w, const maba_tensor* s0, maba_tensor* out,
                    maba_tensor* sf, void* ws, size_t ws_bytes, hipStream_t stream) {
  const int64_t B = q->shape[0], H = q->shape[1], L = q->shape[2];
  const int64_t BH = B * H;
  TokArgs a;
  // strides fit in int32 (dgda_tok_supported checks every operand)
  a.q = q->data; a.qs0 = (int)q->stride[0]; a.qs1 = (int)q->stride[1]; a.qs2 = (int)q->stride[2];
  a.k = k->data; a.ks0 = (int)k->stride[0]; a.ks1 = (int)k->stride[1]; a.ks2 = (int)k->stride[2];
  a.vp = v->data; a.vs0 = (int)v->stride[0]; a.vs1 = (int)v->stride[1]; a.vs2 = (int)v->stride[2];
  a.gp = (const float*)gate->data; a.gs0 = (int)gate->stride[0]; a.gs1 = (int)gate->stride[1];
  a.gs2 = (int)gate->stride[2]; a.gs3 = (int)gate->stride[3];
  a.bp = (const float*)b->data; a.bs0 = (int)b->stride[0]; a.bs1 = (int)b->stride[1];
  a.bs2 = (int)b->stride[2]; a.bs3 = (int)b->stride[3];
  a.wp = (const float*)w->data; a.ws0 = (int)w->stride[0]; a.ws1 = (int)w->stride[1];
  a.ws2 = (int)w->stride[2]; a.ws3 = (int)w->stride[3];
  a.s0 = view4(s0);
  a.op = out->data; a.os0 = (int)out->stride[0]; a.os1 = (int)out->stride[1]; a.os2 = (int)out->stride[2];
  a.sf = mview4(sf);
  a.H = (int)H; a.L = (int)L; a.BH = (int)BH;
  a.nchunks = (int)(ceil_div(L, TCH) > 0 ? ceil_div(L, TCH) : 1);
  const SlotGeom gm = tok_geom(BH, L);
  a.U = gm.U;
  a.nseg_max = gm.nseg_max;
  a.use_log = use_log; a.has_s0 = s0 != nullptr;
  const size_t need = dgda_tok_workspace(BH, L);
  if (ws_bytes < need) return fail(MABA_ERR_WORKSPACE, "dgda_prefill: workspace too small");
  const int64_t nsegs = BH * a.nseg_max;
  a.agg = (float*)ws;
  a.zc = (int*)(a.agg + nsegs * 64 * 128);
  const bool f32in = q->dtype == MABA_F32, obf = out->dtype == MABA_BF16;
  auto launch_out = [&](int mode) {
    a.mode = mode;
    const dim3 grid(mode == TOK_ZERO ? (unsigned)ceil_div(BH * a.nchunks, a.U) : (unsigned)(BH * (a.nseg_max - 1)));
    if (f32in && obf) hipLaunchKernelGGL((dgda_tok_kernel<false, true, true>), grid, dim3(256), 0, stream, a);
    else if (f32in) hipLaunchKernelGGL((dgda_tok_kernel<false, true, false>), grid, dim3(256), 0, stream, a);
    else if (obf) hipLaunchKernelGGL((dgda_tok_kernel<false, false, true>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((dgda_tok_kernel<false, false, false>), grid, dim3(256), 0, stream, a);
    return check_launch("dgda_prefill/token output");
  };
  if (a.nseg_max == 1) {
    a.zc = nullptr;
    return launch_out(TOK_ZERO);
  }
  a.mode = TOK_ZERO;
  const dim3 agrid((unsigned)(BH * (a.nseg_max - 1)));
  if (f32in) hipLaunchKernelGGL((dgda_tok_kernel<true, true, true>), agrid, dim3(512), 0, stream, a);
  else hipLaunchKernelGGL((dgda_tok_kernel<true, false, true>), agrid, dim3(512), 0, stream, a);
  int rc = check_launch("dgda_prefill/token aggregate");
  if (rc) return rc;
  if ((rc = launch_out(TOK_ZERO))) return rc;
  return launch_out(TOK_FIX);
}

}  // namespace maba

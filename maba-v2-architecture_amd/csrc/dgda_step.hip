// DGDA single-token decode step (reference: maba_sparse/kernels/common.py:271-309,
// cpu_dgda.py:200-261).
//
//   S'    = diag(alpha) S
//   delta = w*v - (b*k)^T S'
//   S_new = S' + k delta^T
//   o     = S_new^T q
//
// One workgroup per (batch, head).  The [dk, dv] fp32 state is streamed once:
// each thread owns one column c and a contiguous run of rows, keeps its slice
// of S' in registers between the two reductions, and writes S_new once.  The
// kernel is HBM-bound on the state read + write (8*dk*dv bytes per head).
#include <initializer_list>

#include "dgda_common.h"

namespace maba {

struct StepArgs {
  View4 q, k, v, alpha, log_alpha, b, w, state;  // q..w are [B,H,d] (s2 = elem)
  MView4 out, new_state;
  int H, dk, dv;
  int has_state, use_log;
};

template <int DVP>
__global__ __launch_bounds__(256) void dgda_step_kernel(StepArgs a) {
  constexpr int RG = 256 / DVP;          // row groups
  constexpr int MAXR = 128 / RG;         // max rows per thread (dk <= 128)
  __shared__ float s_a[128], s_bk[128], s_k[128], s_q[128], s_wv[128];
  __shared__ float s_part[RG][DVP];

  const int bh = blockIdx.x;
  const int bi = bh / a.H, hi = bh % a.H;
  const int tid = threadIdx.x;
  const int dk = a.dk, dv = a.dv;

  for (int r = tid; r < dk; r += 256) {
    const float kk = a.k.at(bi, hi, r, 0);
    const float al = a.use_log ? __expf(a.log_alpha.at(bi, hi, r, 0)) : a.alpha.at(bi, hi, r, 0);
    s_a[r] = al;
    s_k[r] = kk;
    s_bk[r] = a.b.at(bi, hi, r, 0) * kk;
    s_q[r] = a.q.at(bi, hi, r, 0);
  }
  for (int c = tid; c < dv; c += 256) s_wv[c] = a.w.at(bi, hi, c, 0) * a.v.at(bi, hi, c, 0);
  __syncthreads();

  const int c = tid % DVP;
  const int rg = tid / DVP;
  const int rows_per = (dk + RG - 1) / RG;
  const int r0 = rg * rows_per;
  const bool col_ok = c < dv;

  float s[MAXR];
  float pred = 0.f;
#pragma unroll
  for (int i = 0; i < MAXR; ++i) {
    const int r = r0 + i;
    float x = 0.f;
    if (i < rows_per && r < dk && col_ok) {
      x = a.has_state ? a.state.at(bi, hi, r, c) : 0.f;
      x *= s_a[r];
      pred = fmaf(s_bk[r], x, pred);
    }
    s[i] = x;
  }
  s_part[rg][c] = pred;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int g = 0; g < RG; ++g) tot += s_part[g][c];
  const float delta = col_ok ? (s_wv[c] - tot) : 0.f;
  __syncthreads();

  float o = 0.f;
#pragma unroll
  for (int i = 0; i < MAXR; ++i) {
    const int r = r0 + i;
    if (i < rows_per && r < dk && col_ok) {
      const float sn = fmaf(s_k[r], delta, s[i]);
      a.new_state.put(bi, hi, r, c, sn);
      o = fmaf(s_q[r], sn, o);
    }
  }
  s_part[rg][c] = o;
  __syncthreads();
  if (rg == 0 && col_ok) {
    float t = 0.f;
#pragma unroll
    for (int g = 0; g < RG; ++g) t += s_part[g][c];
    a.out.put(bi, hi, c, 0, t);
  }
}

// Fast path for dk, dv in {32, 64, 128} with state rows of unit column stride (fp32 or bf16;
// contiguous rows unless dk = dv = 64), q/k/v of one dtype (bf16 or fp32) and fp32 gates: one
// 256-thread workgroup per (b, h), wave w owning state rows (dk/4) w .. (dk/4)(w+1) - 1 and
// lane c the state column c (and c + 64 when dv = 128).  Each lane issues its row loads at
// once and keeps them in registers; the per-row scalars (decay, b*k, k, q) are
// broadcast from the lane that loaded them with readlane, and the two column reductions
// over the rows (b k^T S' and q^T S_new) are summed per wave, then over the four waves in
// LDS in a fixed order.
struct StepFast {
  const void* q; const void* k; const void* v;
  int64_t qsb, qsh, qsd, ksb, ksh, ksd, vsb, vsh, vsd;
  const float* gate; int64_t gsb, gsh, gsd;   // log_alpha (use_log) or alpha
  const float* bb; int64_t bsb, bsh, bsd;
  const float* ww; int64_t wsb, wsh, wsd;
  const void* state; int64_t ssb, ssh; int ssr32;   // may be null (zero state); fp32 or bf16 (TS)
  void* nst; int64_t nsb, nsh; int nsr32;           // same dtype as the state; may alias it
  void* out; int odt; int64_t osb, osh, osd;
  int64_t BH;
  int H, use_log;
};

__device__ __forceinline__ float bcast(float x, int r) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), r));
}

template <typename T>
__device__ __forceinline__ float cvt(T x);
template <>
__device__ __forceinline__ float cvt<float>(float x) { return x; }
template <>
__device__ __forceinline__ float cvt<uint16_t>(uint16_t x) { return bf16_bits_to_f32(x); }

// Row offset i of a state slab: rows DV elements apart (CONTIG, the layout every caller
// uses: one base address and immediate offsets) or a run-time 32-bit row stride.
template <bool CONTIG, int DV = 64>
__device__ __forceinline__ int64_t row_at(int i, int rs) { return CONTIG ? (int64_t)(DV * i) : (int64_t)i * rs; }

// Head sizes of the fast step: d_k / 4 state rows per wave (four waves), step_nc columns per lane
// (lane c holds columns c and c + 64 when d_v = 128), step_nr row-scalar registers per lane (lane
// r holds the scalars of rows r and r + 64 when d_k = 128).
constexpr int step_nc(int dv) { return dv > 64 ? 2 : 1; }
constexpr int step_nr(int dk) { return dk > 64 ? 2 : 1; }

// The RPW = d_k / 4 rows of wave w's slab, S[RPW w + i][col + 64 j], from sp = &S[RPW w][col]
// (rs: row stride), as stored (converted by the caller once every load of the step is issued).
template <typename TS, bool CONTIG, int DK = 64, int DV = 64>
__device__ __forceinline__ void load_rows(TS (&s)[step_nc(DV)][DK / 4], const TS* sp, int rs) {
#pragma unroll
  for (int j = 0; j < step_nc(DV); ++j)
#pragma unroll
    for (int i = 0; i < DK / 4; ++i) s[j][i] = sp[row_at<CONTIG, DV>(i, rs) + 64 * j];
}

// Row r's scalar from the lane that holds it (r wave-uniform).
template <int NR>
__device__ __forceinline__ float row_scalar(const float (&x)[NR], int r) {
  if constexpr (NR == 1) return bcast(x[0], r);
  else return r < 64 ? bcast(x[0], r) : bcast(x[1], r - 64);
}

// The step on the rows of wave w (lane = column): s[j][i] holds S[RPW w + i][lane + 64 j] on
// entry; al, bk, kr, qr are the row scalars (register m: row 64 m + lane), vw[j] = w v of
// column lane + 64 j.  Writes the new state rows through np = &S_new[RPW w][lane] (row stride
// nrs; columns at or past d_v are not written) and returns o of the lane's columns (every
// wave).  Every state load of the caller precedes the first store, so S_new may alias S.
template <typename TS, bool CONTIG, int DK = 64, int DV = 64>
__device__ __forceinline__ void step_rows(float (&s)[step_nc(DV)][DK / 4],
                                          const float (&al)[step_nr(DK)],
                                          const float (&bk)[step_nr(DK)],
                                          const float (&kr)[step_nr(DK)],
                                          const float (&qr)[step_nr(DK)],
                                          const float (&vw)[step_nc(DV)], TS* np, int nrs,
                                          float (*s_red)[64 * step_nc(DV)],
                                          float (&o)[step_nc(DV)]) {
  constexpr int RPW = DK / 4, NC = step_nc(DV), NR = step_nr(DK);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const bool colok = DV >= 64 || lane < DV;
  float pred[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) pred[j] = 0.f;
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = RPW * wave + i;
    const float a_r = row_scalar<NR>(al, r), b_r = row_scalar<NR>(bk, r);
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      s[j][i] *= a_r;
      pred[j] = fmaf(b_r, s[j][i], pred[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < NC; ++j) s_red[wave][64 * j + lane] = pred[j];
  __syncthreads();
  float delta[NC], oo[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = 64 * j + lane;
    delta[j] = vw[j] - ((s_red[0][c] + s_red[1][c]) + (s_red[2][c] + s_red[3][c]));
    oo[j] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int r = RPW * wave + i;
    const float k_r = row_scalar<NR>(kr, r), q_r = row_scalar<NR>(qr, r);
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const float sn = fmaf(k_r, delta[j], s[j][i]);
      if (colok) {
        if constexpr (sizeof(TS) == 4) np[row_at<CONTIG, DV>(i, nrs) + 64 * j] = sn;
        else np[row_at<CONTIG, DV>(i, nrs) + 64 * j] = f32_to_bf16_bits(sn);
      }
      oo[j] = fmaf(q_r, sn, oo[j]);   // the fp32 state before its rounding, as the generic kernel
    }
  }
  __syncthreads();   // every wave has read s_red before it is reused
#pragma unroll
  for (int j = 0; j < NC; ++j) s_red[wave][64 * j + lane] = oo[j];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = 64 * j + lane;
    o[j] = (s_red[0][c] + s_red[1][c]) + (s_red[2][c] + s_red[3][c]);
  }
}

// T: dtype of q, k, v; TS: dtype of the state in and out (fp32 or bf16); HS: a state is
// given (else zeros); CONTIG: state rows d_v elements apart in and out; DK, DV in {32, 64,
// 128}.  The slab and the row scalars are all loaded before the first wait, so the step waits
// for one memory round trip (a run-time null test around the slab loads, or 64-bit strided
// addresses per row, made the compiler wait for the slab before it issued the scalars).
// With d_v = 32 the upper 32 lanes load column 31 again and store nothing; with d_k = 32
// lanes 32 .. 63 load the scalars of row 31 again (never broadcast).
template <typename T, typename TS, bool HS, bool CONTIG, int DK = 64, int DV = 64>
__global__ __launch_bounds__(256) void dgda_step_wave_kernel(StepFast a) {
  constexpr int RPW = DK / 4, NC = step_nc(DV), NR = step_nr(DK);
  __shared__ float s_red[4][64 * NC];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t bi = blockIdx.y, hi = blockIdx.x;   // grid (H, B): no division
  const int col = DV >= 64 ? lane : min(lane, DV - 1);
  TS raw[NC][RPW];
  if constexpr (HS)
    load_rows<TS, CONTIG, DK, DV>(raw, (const TS*)a.state + (bi * a.ssb + hi * a.ssh +
                                                               row_at<CONTIG, DV>(RPW * wave, a.ssr32) + col),
                                  a.ssr32);
  // lane r holds the row-r scalars (and row r + 64's); lane c holds w_c v_c (and column c +
  // 64's).  The (b, h) base is scalar and the lane's offset a 32-bit unsigned product (the host
  // checks that 127 * stride fits)
  T kx[NR], qx[NR];
  float gr[NR], br[NR];
#pragma unroll
  for (int m = 0; m < NR; ++m) {
    const uint32_t l = DK >= 64 ? (uint32_t)(lane + 64 * m) : (uint32_t)min(lane, DK - 1);
    kx[m] = ((const T*)a.k + (bi * a.ksb + hi * a.ksh))[l * (uint32_t)a.ksd];
    qx[m] = ((const T*)a.q + (bi * a.qsb + hi * a.qsh))[l * (uint32_t)a.qsd];
    gr[m] = (a.gate + (bi * a.gsb + hi * a.gsh))[l * (uint32_t)a.gsd];
    br[m] = (a.bb + (bi * a.bsb + hi * a.bsh))[l * (uint32_t)a.bsd];
  }
  T vx[NC];
  float wc[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const uint32_t c = (uint32_t)(col + 64 * j);
    vx[j] = ((const T*)a.v + (bi * a.vsb + hi * a.vsh))[c * (uint32_t)a.vsd];
    wc[j] = (a.ww + (bi * a.wsb + hi * a.wsh))[c * (uint32_t)a.wsd];
  }
  // every load above is issued before the first use waits (with 16-bit state rows the compiler
  // otherwise converts the first rows, and waits for them, before issuing the rest; with fp32
  // rows it issues them all and overlaps the first reduction with their arrival)
  if constexpr (sizeof(TS) == 2) __builtin_amdgcn_sched_barrier(0);
  float s[NC][RPW];
#pragma unroll
  for (int j = 0; j < NC; ++j)
#pragma unroll
    for (int i = 0; i < RPW; ++i) s[j][i] = HS ? cvt<TS>(raw[j][i]) : 0.f;
  float kr[NR], qr[NR], al[NR], bk[NR], vw[NC];
#pragma unroll
  for (int m = 0; m < NR; ++m) {
    kr[m] = cvt<T>(kx[m]);
    qr[m] = cvt<T>(qx[m]);
    al[m] = a.use_log ? __expf(gr[m]) : gr[m];
    bk[m] = br[m] * kr[m];
  }
#pragma unroll
  for (int j = 0; j < NC; ++j) vw[j] = wc[j] * cvt<T>(vx[j]);
  TS* np = (TS*)a.nst + (bi * a.nsb + hi * a.nsh + row_at<CONTIG, DV>(RPW * wave, a.nsr32) + lane);
  float o[NC];
  step_rows<TS, CONTIG, DK, DV>(s, al, bk, kr, qr, vw, np, a.nsr32, s_red, o);
  if (wave == 0) {
#pragma unroll
    for (int j = 0; j < NC; ++j)
      if (lane + 64 * j < DV) store_elem(a.out, a.odt, bi * a.osb + hi * a.osh + (lane + 64 * j) * a.osd, o[j]);
  }
}

// One decode token of the DGDA layer after its input projection, in one launch: the
// single-token prologue (layers/dgda.py:103-121, 186-207: causal depthwise conv + SiLU of
// q, k, v over the carried history, the key's head L2 norm, the decay, erase and write
// gates; the new history) followed by the step above, for one (b, h) per wave with
// lane = channel of the head, the layout of both parts.  q, k, v are rounded to bf16
// before the step and the gates kept in fp32, as the two separate launches store them,
// so the results equal theirs.  Every input of the wave (state column, projections,
// history) is read before its first store, so the state and the history update in place.
struct LayerStepArgs {
  const uint16_t* x[6]; int64_t xsb[6];                       // bf16 projection rows [B, C]
  const void* cw[3]; int cwdt; int64_t cwsc[3], cwst[3];      // conv taps [C, 1, 4]
  const uint16_t* hist[3]; int64_t hsb[3], hsc[3], hst[3];    // bf16 [B, C, 3] or null (zeros)
  uint16_t* nh[3]; int64_t nhsb[3], nhsc[3], nhst[3];         // bf16 new history (may alias hist)
  const void* state; int64_t ssb, ssh; int ssr32;             // [B, H, 64, 64] (TS) or null (zero)
  void* nst; int64_t nsb, nsh; int nsr32;                     // may alias state
  void* out; int odt; int64_t osb, osh, osd;                  // o [B, H, 64]
  int64_t BH;
  int H;
  float eps;
};

// TW: dtype of the conv taps; HS / HH: a state / a history is given (else zeros); CONTIG:
// state rows 64 elements apart (see dgda_step_wave_kernel).  The
// dtype and the presence of each input are compile-time, so the wave issues every load
// (state column, projections, taps, history) before it waits for the first: with a
// run-time dtype switch or a null test around a load, the compiler converts or merges
// each loaded value inside its branch and waits for that load alone, one memory round
// trip per tap.
template <typename TS, typename TW, bool HS, bool HH, bool CONTIG>
__global__ __launch_bounds__(256) void dgda_layer_step_kernel(LayerStepArgs a) {
  __shared__ float s_red[4][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t bi = blockIdx.y, hi = blockIdx.x;   // grid (H, B): no division
  const int64_t c = hi * 64 + lane;   // channel of the projection rows
  TS raw[1][16];
  if constexpr (HS)
    load_rows<TS, CONTIG>(raw, (const TS*)a.state + (bi * a.ssb + hi * a.ssh + row_at<CONTIG>(16 * wave, a.ssr32) + lane),
                          a.ssr32);
  // ---- prologue (as dgda_prologue_step_kernel); every wave forms all 64 channels
  uint16_t xr[6], hr[3][3];
  TW wr[3][4];
#pragma unroll
  for (int st = 0; st < 6; ++st) xr[st] = a.x[st][bi * a.xsb[st] + c];
#pragma unroll
  for (int st = 0; st < 3; ++st) {
#pragma unroll
    for (int j = 0; j < 4; ++j) wr[st][j] = ((const TW*)a.cw[st])[c * a.cwsc[st] + j * a.cwst[st]];
    if constexpr (HH) {
#pragma unroll
      for (int j = 0; j < 3; ++j) hr[st][j] = a.hist[st][bi * a.hsb[st] + c * a.hsc[st] + j * a.hst[st]];
    }
  }
  __builtin_amdgcn_sched_barrier(0);   // every load above is issued before the first use waits
  float s[1][16], x[6], w[3][4], h[3][3];
#pragma unroll
  for (int i = 0; i < 16; ++i) s[0][i] = HS ? cvt<TS>(raw[0][i]) : 0.f;
#pragma unroll
  for (int st = 0; st < 6; ++st) x[st] = bf16_bits_to_f32(xr[st]);
#pragma unroll
  for (int st = 0; st < 3; ++st) {
#pragma unroll
    for (int j = 0; j < 4; ++j) w[st][j] = cvt<TW>(wr[st][j]);
#pragma unroll
    for (int j = 0; j < 3; ++j) h[st][j] = HH ? bf16_bits_to_f32(hr[st][j]) : 0.f;
  }
  float y[3];
#pragma unroll
  for (int st = 0; st < 3; ++st) {
    float acc = w[st][3] * x[st];
    acc = fmaf(w[st][2], h[st][2], acc);
    acc = fmaf(w[st][1], h[st][1], acc);
    acc = fmaf(w[st][0], h[st][0], acc);
    y[st] = pro_silu(acc);
  }
  float ss = y[1] * y[1];
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) ss += __shfl_xor(ss, off);
  const float kinv = pro_knorm_inv(ss, a.eps);
  // lane r holds the row-r scalars of the step (q, k, decay, erase), lane c the column ones (v, write)
  const float qr = bf16_bits_to_f32(f32_to_bf16_bits(y[0]));
  const float kr = bf16_bits_to_f32(f32_to_bf16_bits(y[1] * kinv));
  const float vc = bf16_bits_to_f32(f32_to_bf16_bits(y[2]));
  const float gr = pro_log_decay(x[3]);
  const float br = pro_sigmoid(x[4]);
  const float wc = pro_sigmoid(x[5]);
  // ---- step (as dgda_step_wave_kernel with log_alpha).  Every wave's loads complete here,
  // before the step's first barrier, so no wave still reads the history when wave 0
  // overwrites it (in place) after the barriers below.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const float al[1] = {__expf(gr)}, bk[1] = {br * kr}, krr[1] = {kr}, qrr[1] = {qr}, vw[1] = {wc * vc};
  TS* np = (TS*)a.nst + (bi * a.nsb + hi * a.nsh + row_at<CONTIG>(16 * wave, a.nsr32) + lane);
  float ov[1];
  step_rows<TS, CONTIG>(s, al, bk, krr, qrr, vw, np, a.nsr32, s_red, ov);
  const float o = ov[0];
  if (wave == 0) {
#pragma unroll
    for (int st = 0; st < 3; ++st) {   // new history: the inputs of tokens -2, -1, 0
      uint16_t* nh = a.nh[st] + bi * a.nhsb[st] + c * a.nhsc[st];
      nh[0] = f32_to_bf16_bits(h[st][1]);
      nh[a.nhst[st]] = f32_to_bf16_bits(h[st][2]);
      nh[2 * a.nhst[st]] = f32_to_bf16_bits(x[st]);
    }
    store_elem(a.out, a.odt, bi * a.osb + hi * a.osh + lane * a.osd, o);
  }
}

}  // namespace maba

using namespace maba;

// The fast kernel for head sizes other than 64 x 64 (contiguous state rows): d_k, d_v in
// {32, 64, 128}, bf16 or fp32 q/k/v (bq), bf16 or fp32 state (sbf), a state given or not (hs).
template <int DK, int DV>
static void (*step_kernel_dims(bool bq, bool sbf, bool hs))(StepFast) {
#define MABA_STEP_SZ(T, TS) \
  return hs ? dgda_step_wave_kernel<T, TS, true, true, DK, DV> : dgda_step_wave_kernel<T, TS, false, true, DK, DV>
  if (bq) { if (sbf) MABA_STEP_SZ(uint16_t, uint16_t); MABA_STEP_SZ(uint16_t, float); }
  if (sbf) MABA_STEP_SZ(float, uint16_t);
  MABA_STEP_SZ(float, float);
#undef MABA_STEP_SZ
}
template <int DK>
static void (*step_kernel_dk(int64_t dv, bool bq, bool sbf, bool hs))(StepFast) {
  if (dv == 32) return step_kernel_dims<DK, 32>(bq, sbf, hs);
  if (dv == 64) return step_kernel_dims<DK, 64>(bq, sbf, hs);
  return step_kernel_dims<DK, 128>(bq, sbf, hs);
}
static void (*step_kernel_sized(int64_t dk, int64_t dv, bool bq, bool sbf, bool hs))(StepFast) {
  if (dk == 32) return step_kernel_dk<32>(dv, bq, sbf, hs);
  if (dk == 64) return step_kernel_dk<64>(dv, bq, sbf, hs);
  return step_kernel_dk<128>(dv, bq, sbf, hs);
}

// The fast kernel's per-lane offsets of the [B,H,d] operands are 32-bit unsigned products
// lane * stride (at most 127 * stride elements of up to 4 bytes).
static bool lane_strides_fit(std::initializer_list<const maba_tensor*> ts) {
  for (const maba_tensor* t : ts)
    if (t->stride[2] < 0 || t->stride[2] > ((int64_t)1 << 24)) return false;
  return true;
}

extern "C" int maba_hip_dgda_step(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                                  const maba_tensor* alpha, const maba_tensor* log_alpha,
                                  const maba_tensor* b, const maba_tensor* w,
                                  const maba_tensor* state, maba_tensor* out,
                                  maba_tensor* new_state, void* stream) {
  if (!q || q->ndim != 3) return fail(MABA_ERR_INVALID, "dgda_step: q must be [B,H,dk]");
  const int64_t B = q->shape[0], H = q->shape[1], dk = q->shape[2];
  if (!v || v->ndim != 3) return fail(MABA_ERR_INVALID, "dgda_step: v must be [B,H,dv]");
  const int64_t dv = v->shape[2];
  const int64_t sq[3] = {B, H, dk}, sv[3] = {B, H, dv}, ss[4] = {B, H, dk, dv};
  if (!expect_shape(q, "q", 3, sq) || !expect_shape(k, "k", 3, sq) || !expect_shape(v, "v", 3, sv) ||
      !expect_shape(b, "b", 3, sq) || !expect_shape(w, "w", 3, sv) ||
      !expect_shape(out, "out", 3, sv) || !expect_shape(new_state, "new_state", 4, ss))
    return MABA_ERR_INVALID;
  if (!alpha && !log_alpha) return fail(MABA_ERR_INVALID, "dgda_step: alpha or log_alpha required");
  if (log_alpha && !expect_shape(log_alpha, "log_alpha", 3, sq)) return MABA_ERR_INVALID;
  if (!log_alpha && !expect_shape(alpha, "alpha", 3, sq)) return MABA_ERR_INVALID;
  if (state && !expect_shape(state, "state", 4, ss)) return MABA_ERR_INVALID;
  const maba_tensor* all[] = {q, k, v, b, w, out, new_state, log_alpha ? log_alpha : alpha, state};
  for (const maba_tensor* t : all)
    if (t && !expect_float(t, "dgda_step")) return MABA_ERR_DTYPE;
  if (dk > 128 || dv > 128 || dk < 1 || dv < 1)
    return fail(MABA_ERR_UNSUPPORTED, "dgda_step: dk, dv must be in [1,128], got %lld, %lld",
                (long long)dk, (long long)dv);
  if (B * H == 0) return MABA_OK;

  StepArgs a;
  a.q = view4(q); a.k = view4(k); a.v = view4(v); a.b = view4(b); a.w = view4(w);
  a.alpha = view4(alpha); a.log_alpha = view4(log_alpha); a.state = view4(state);
  // [B,H,d] views: move the element stride to slot 2 so .at(b,h,i,0) indexes them.
  View4* vecs[] = {&a.q, &a.k, &a.v, &a.b, &a.w, &a.alpha, &a.log_alpha};
  for (View4* x : vecs) { x->s3 = 0; }
  a.q.s2 = q->stride[2]; a.k.s2 = k->stride[2]; a.v.s2 = v->stride[2];
  a.b.s2 = b->stride[2]; a.w.s2 = w->stride[2];
  if (alpha) a.alpha.s2 = alpha->stride[2];
  if (log_alpha) a.log_alpha.s2 = log_alpha->stride[2];
  a.out = mview4(out); a.out.s3 = 0;
  a.new_state = mview4(new_state);
  a.H = (int)H; a.dk = (int)dk; a.dv = (int)dv;
  a.has_state = state != nullptr;
  a.use_log = log_alpha != nullptr;

  hipStream_t s = (hipStream_t)stream;
  const maba_tensor* gate = log_alpha ? log_alpha : alpha;
  const bool qkv_same = q->dtype == k->dtype && q->dtype == v->dtype && (q->dtype == MABA_BF16 || q->dtype == MABA_F32);
  const int sdt = new_state->dtype;
  auto head_ok = [](int64_t d) { return d == 32 || d == 64 || d == 128; };
  // other head sizes than 64 take the fast kernel with contiguous state rows only
  const bool rows_contig = new_state->stride[2] == dv && (!state || state->stride[2] == dv);
  const bool fast = head_ok(dk) && head_ok(dv) && (dk == 64 && dv == 64 ? true : rows_contig) && qkv_same &&
                    gate->dtype == MABA_F32 && b->dtype == MABA_F32 &&
                    w->dtype == MABA_F32 && (sdt == MABA_F32 || sdt == MABA_BF16) && new_state->stride[3] == 1 &&
                    new_state->stride[2] <= INT32_MAX && B <= 65535 && lane_strides_fit({q, k, v, gate, b, w}) &&
                    (!state || (state->dtype == sdt && state->stride[3] == 1 && state->stride[2] <= INT32_MAX));
  if (fast) {
    StepFast f;
    f.q = q->data; f.qsb = q->stride[0]; f.qsh = q->stride[1]; f.qsd = q->stride[2];
    f.k = k->data; f.ksb = k->stride[0]; f.ksh = k->stride[1]; f.ksd = k->stride[2];
    f.v = v->data; f.vsb = v->stride[0]; f.vsh = v->stride[1]; f.vsd = v->stride[2];
    f.gate = (const float*)gate->data; f.gsb = gate->stride[0]; f.gsh = gate->stride[1]; f.gsd = gate->stride[2];
    f.bb = (const float*)b->data; f.bsb = b->stride[0]; f.bsh = b->stride[1]; f.bsd = b->stride[2];
    f.ww = (const float*)w->data; f.wsb = w->stride[0]; f.wsh = w->stride[1]; f.wsd = w->stride[2];
    f.state = state ? state->data : nullptr;
    f.ssb = state ? state->stride[0] : 0; f.ssh = state ? state->stride[1] : 0;
    f.ssr32 = state ? (int)state->stride[2] : (int)dv;
    f.nst = new_state->data; f.nsb = new_state->stride[0]; f.nsh = new_state->stride[1];
    f.nsr32 = (int)new_state->stride[2];
    f.out = out->data; f.odt = out->dtype; f.osb = out->stride[0]; f.osh = out->stride[1]; f.osd = out->stride[2];
    f.BH = B * H; f.H = (int)H; f.use_log = log_alpha != nullptr;
    const dim3 g4((unsigned)H, (unsigned)B);   // one workgroup per (b, h)
    const bool sbf = sdt == MABA_BF16, hs = state != nullptr, contig = f.ssr32 == dv && f.nsr32 == dv;
    void (*kern)(StepFast) = nullptr;
    if (dk == 64 && dv == 64) {
#define MABA_STEP_PICK(T, TS)                                                                          \
  kern = hs ? (contig ? dgda_step_wave_kernel<T, TS, true, true> : dgda_step_wave_kernel<T, TS, true, false>) \
            : (contig ? dgda_step_wave_kernel<T, TS, false, true> : dgda_step_wave_kernel<T, TS, false, false>)
      if (q->dtype == MABA_BF16) { if (sbf) MABA_STEP_PICK(uint16_t, uint16_t); else MABA_STEP_PICK(uint16_t, float); }
      else { if (sbf) MABA_STEP_PICK(float, uint16_t); else MABA_STEP_PICK(float, float); }
#undef MABA_STEP_PICK
    } else {
      kern = step_kernel_sized(dk, dv, q->dtype == MABA_BF16, sbf, hs);
    }
    hipLaunchKernelGGL(kern, g4, dim3(256), 0, s, f);
    return check_launch("dgda_step");
  }
  dim3 grid((unsigned)(B * H)), block(256);
  if (dv <= 32) hipLaunchKernelGGL(dgda_step_kernel<32>, grid, block, 0, s, a);
  else if (dv <= 64) hipLaunchKernelGGL(dgda_step_kernel<64>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(dgda_step_kernel<128>, grid, block, 0, s, a);
  return check_launch("dgda_step");
}

extern "C" int maba_hip_dgda_layer_step(const maba_tensor* const* xs, const maba_tensor* const* conv_w,
                                        const maba_tensor* const* hist, float eps, const maba_tensor* state,
                                        maba_tensor* out, maba_tensor* new_state, maba_tensor* const* new_hist,
                                        void* stream) {
  const char* who = "dgda_layer_step";
  if (!xs || !conv_w || !new_hist || !out || !new_state)
    return fail(MABA_ERR_INVALID, "%s: xs, conv_w and new_hist arrays, out and new_state required", who);
  if (out->ndim != 3 || out->shape[2] != 64)
    return fail(MABA_ERR_UNSUPPORTED, "%s: out must be [B,H,64] (64-channel heads)", who);
  const int64_t B = out->shape[0], H = out->shape[1], C = 64 * H;
  if (H < 1 || H > 16 || B > 65535) return fail(MABA_ERR_UNSUPPORTED, "%s: 1 <= H <= 16 and B <= 65535", who);
  if (out->dtype != MABA_F32 && out->dtype != MABA_BF16) return fail(MABA_ERR_DTYPE, "%s: out f32 or bf16", who);
  LayerStepArgs a;
  for (int st = 0; st < 6; ++st) {   // [B, C] or [B, 1, C] bf16 rows with unit channel stride
    const maba_tensor* t = xs[st];
    const bool ok = t && t->dtype == MABA_BF16 && t->shape[0] == B && t->shape[t->ndim - 1] == C &&
                    t->stride[t->ndim - 1] == 1 && (t->ndim == 2 || (t->ndim == 3 && t->shape[1] == 1));
    if (!ok) return fail(MABA_ERR_INVALID, "%s: projection %d must be bf16 [B,C] or [B,1,C], C = 64 H, unit channel stride", who, st);
    a.x[st] = (const uint16_t*)t->data;
    a.xsb[st] = t->stride[0];
  }
  for (int st = 0; st < 3; ++st) {
    const maba_tensor* w = conv_w[st];
    if (!w || w->ndim != 3 || w->shape[0] != C || w->shape[1] != 1 || w->shape[2] != 4 ||
        (w->dtype != MABA_F32 && w->dtype != MABA_BF16))
      return fail(MABA_ERR_INVALID, "%s: conv weight %d must be [C,1,4] f32/bf16", who, st);
    if (st > 0 && w->dtype != conv_w[0]->dtype) return fail(MABA_ERR_DTYPE, "%s: conv weights of one dtype", who);
    a.cw[st] = w->data; a.cwsc[st] = w->stride[0]; a.cwst[st] = w->stride[2];
    const int64_t hs[3] = {B, C, 3};
    const maba_tensor* hh = hist ? hist[st] : nullptr;   // no history array: zeros
    if (hh && (!expect_shape(hh, "hist", 3, hs) || hh->dtype != MABA_BF16))
      return fail(MABA_ERR_INVALID, "%s: history %d must be bf16 [B,C,3]", who, st);
    a.hist[st] = hh ? (const uint16_t*)hh->data : nullptr;
    a.hsb[st] = hh ? hh->stride[0] : 0; a.hsc[st] = hh ? hh->stride[1] : 0; a.hst[st] = hh ? hh->stride[2] : 0;
    maba_tensor* nh = new_hist[st];
    if (!nh || !expect_shape(nh, "new_hist", 3, hs) || nh->dtype != MABA_BF16)
      return fail(MABA_ERR_INVALID, "%s: new history %d must be bf16 [B,C,3]", who, st);
    a.nh[st] = (uint16_t*)nh->data; a.nhsb[st] = nh->stride[0]; a.nhsc[st] = nh->stride[1]; a.nhst[st] = nh->stride[2];
  }
  a.cwdt = conv_w[0]->dtype;
  const int nhist = (int)(a.hist[0] != nullptr) + (a.hist[1] != nullptr) + (a.hist[2] != nullptr);
  if (nhist != 0 && nhist != 3) return fail(MABA_ERR_INVALID, "%s: give all three histories or none", who);
  const int64_t ss4[4] = {B, H, 64, 64};
  if (!expect_shape(new_state, "new_state", 4, ss4) || new_state->stride[3] != 1 || new_state->stride[2] > INT32_MAX ||
      (new_state->dtype != MABA_F32 && new_state->dtype != MABA_BF16))
    return fail(MABA_ERR_INVALID, "%s: new_state must be f32/bf16 [B,H,64,64] with unit column stride", who);
  if (state && (!expect_shape(state, "state", 4, ss4) || state->stride[3] != 1 || state->stride[2] > INT32_MAX ||
                state->dtype != new_state->dtype))
    return fail(MABA_ERR_INVALID, "%s: state must match new_state", who);
  a.state = state ? state->data : nullptr;
  a.ssb = state ? state->stride[0] : 0; a.ssh = state ? state->stride[1] : 0; a.ssr32 = state ? (int)state->stride[2] : 64;
  a.nst = new_state->data; a.nsb = new_state->stride[0]; a.nsh = new_state->stride[1]; a.nsr32 = (int)new_state->stride[2];
  a.out = out->data; a.odt = out->dtype; a.osb = out->stride[0]; a.osh = out->stride[1]; a.osd = out->stride[2];
  a.BH = B * H; a.H = (int)H; a.eps = eps;
  if (B == 0) return MABA_OK;
  const dim3 g4((unsigned)H, (unsigned)B);   // one workgroup per (b, h)
  hipStream_t s = (hipStream_t)stream;
  const bool sb = new_state->dtype == MABA_BF16, wb = a.cwdt == MABA_BF16, hs = a.state != nullptr, hh = nhist == 3;
  const bool contig = a.ssr32 == 64 && a.nsr32 == 64;
  void (*k)(LayerStepArgs) = nullptr;
#define MABA_LS_PICK2(TS, TW, C)                                                                \
  k = hs ? (hh ? dgda_layer_step_kernel<TS, TW, true, true, C> : dgda_layer_step_kernel<TS, TW, true, false, C>) \
         : (hh ? dgda_layer_step_kernel<TS, TW, false, true, C> : dgda_layer_step_kernel<TS, TW, false, false, C>)
#define MABA_LS_PICK(TS, TW) do { if (contig) MABA_LS_PICK2(TS, TW, true); else MABA_LS_PICK2(TS, TW, false); } while (0)
  if (sb) { if (wb) MABA_LS_PICK(uint16_t, uint16_t); else MABA_LS_PICK(uint16_t, float); }
  else { if (wb) MABA_LS_PICK(float, uint16_t); else MABA_LS_PICK(float, float); }
#undef MABA_LS_PICK
#undef MABA_LS_PICK2
  hipLaunchKernelGGL(k, g4, dim3(256), 0, s, a);
  return check_launch(who);
}

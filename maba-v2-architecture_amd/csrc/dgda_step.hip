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

// Fast path for dk = dv = 64 with state rows of unit column stride (fp32 or bf16), q/k/v
// of one dtype (bf16 or fp32) and fp32 gates: one 256-thread workgroup per (b, h), wave w
// owning state rows 16w .. 16w+15 and lane c the state column c.  Each lane issues its 16
// row loads at once and keeps them in registers; the per-row scalars (decay, b*k, k, q) are
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

// Row offset i of a state slab: rows 64 elements apart (CONTIG, the layout every caller
// uses: one base address and immediate offsets) or a run-time 32-bit row stride.
template <bool CONTIG>
__device__ __forceinline__ int64_t row_at(int i, int rs) { return CONTIG ? (int64_t)(64 * i) : (int64_t)i * rs; }

// The 16 rows of wave w's slab, S[16w + i][lane], from sp = &S[16w][lane] (rs: row stride),
// as stored (converted by the caller once every load of the step is issued).
template <typename TS, bool CONTIG>
__device__ __forceinline__ void load_rows(TS (&s)[16], const TS* sp, int rs) {
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] = sp[row_at<CONTIG>(i, rs)];
}

// The step on the rows of wave w (lane = column): s[i] holds S[16w + i][lane] on entry;
// al, bk, kr, qr are the row scalars of row `lane`, vw = w_lane v_lane.  Writes the new state
// rows through np = &S_new[16w][lane] (row stride nrs) and returns o[lane] (every wave).
// Every state load of the caller precedes the first store, so S_new may alias S.
template <typename TS, bool CONTIG>
__device__ __forceinline__ float step_rows(float (&s)[16], float al, float bk, float kr, float qr, float vw,
                                           TS* np, int nrs, float (*s_red)[64]) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  float pred = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = 16 * wave + i;
    s[i] *= bcast(al, r);
    pred = fmaf(bcast(bk, r), s[i], pred);
  }
  s_red[wave][lane] = pred;
  __syncthreads();
  pred = (s_red[0][lane] + s_red[1][lane]) + (s_red[2][lane] + s_red[3][lane]);
  const float delta = vw - pred;
  float o = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = 16 * wave + i;
    const float sn = fmaf(bcast(kr, r), delta, s[i]);
    if constexpr (sizeof(TS) == 4) np[row_at<CONTIG>(i, nrs)] = sn;
    else np[row_at<CONTIG>(i, nrs)] = f32_to_bf16_bits(sn);
    o = fmaf(bcast(qr, r), sn, o);   // the fp32 state before its rounding, as the generic kernel
  }
  __syncthreads();   // every wave has read s_red before it is reused
  s_red[wave][lane] = o;
  __syncthreads();
  return (s_red[0][lane] + s_red[1][lane]) + (s_red[2][lane] + s_red[3][lane]);
}

// T: dtype of q, k, v; TS: dtype of the state in and out (fp32 or bf16); HS: a state is
// given (else zeros); CONTIG: state rows 64 elements apart in and out.  The slab and the row
// scalars are all loaded before the first wait, so the step waits for one memory round trip
// (a run-time null test around the slab loads, or 64-bit strided addresses per row, made the
// compiler wait for the slab before it issued the scalars).
template <typename T, typename TS, bool HS, bool CONTIG>
__global__ __launch_bounds__(256) void dgda_step_wave_kernel(StepFast a) {
  __shared__ float s_red[4][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t bi = blockIdx.y, hi = blockIdx.x;   // grid (H, B): no division
  TS raw[16];
  if constexpr (HS)
    load_rows<TS, CONTIG>(raw, (const TS*)a.state + (bi * a.ssb + hi * a.ssh + row_at<CONTIG>(16 * wave, a.ssr32) + lane),
                          a.ssr32);
  // lane r holds the row-r scalars; lane c holds w_c v_c.  The (b, h) base is scalar and the
  // lane's offset a 32-bit unsigned product (the host checks that 63 * stride fits)
  const uint32_t l = lane;
  const T kx = ((const T*)a.k + (bi * a.ksb + hi * a.ksh))[l * (uint32_t)a.ksd];
  const T qx = ((const T*)a.q + (bi * a.qsb + hi * a.qsh))[l * (uint32_t)a.qsd];
  const T vx = ((const T*)a.v + (bi * a.vsb + hi * a.vsh))[l * (uint32_t)a.vsd];
  const float gr = (a.gate + (bi * a.gsb + hi * a.gsh))[l * (uint32_t)a.gsd];
  const float br = (a.bb + (bi * a.bsb + hi * a.bsh))[l * (uint32_t)a.bsd];
  const float wc = (a.ww + (bi * a.wsb + hi * a.wsh))[l * (uint32_t)a.wsd];
  // every load above is issued before the first use waits (with 16-bit state rows the compiler
  // otherwise converts the first rows, and waits for them, before issuing the rest; with fp32
  // rows it issues them all and overlaps the first reduction with their arrival)
  if constexpr (sizeof(TS) == 2) __builtin_amdgcn_sched_barrier(0);
  float s[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] = HS ? cvt<TS>(raw[i]) : 0.f;
  const float kr = cvt<T>(kx), qr = cvt<T>(qx), vc = cvt<T>(vx);
  const float al = a.use_log ? __expf(gr) : gr;
  TS* np = (TS*)a.nst + (bi * a.nsb + hi * a.nsh + row_at<CONTIG>(16 * wave, a.nsr32) + lane);
  const float o = step_rows<TS, CONTIG>(s, al, br * kr, kr, qr, wc * vc, np, a.nsr32, s_red);
  if (wave == 0) store_elem(a.out, a.odt, bi * a.osb + hi * a.osh + lane * a.osd, o);
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
  TS raw[16];
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
  float s[16], x[6], w[3][4], h[3][3];
#pragma unroll
  for (int i = 0; i < 16; ++i) s[i] = HS ? cvt<TS>(raw[i]) : 0.f;
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
  const float al = __expf(gr);
  TS* np = (TS*)a.nst + (bi * a.nsb + hi * a.nsh + row_at<CONTIG>(16 * wave, a.nsr32) + lane);
  const float o = step_rows<TS, CONTIG>(s, al, br * kr, kr, qr, wc * vc, np, a.nsr32, s_red);
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

// The fast kernel's per-lane offsets of the [B,H,64] operands are 32-bit unsigned products
// lane * stride (at most 63 * stride elements of up to 4 bytes).
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
  const bool fast = dk == 64 && dv == 64 && qkv_same && gate->dtype == MABA_F32 && b->dtype == MABA_F32 &&
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
    f.ssr32 = state ? (int)state->stride[2] : 64;
    f.nst = new_state->data; f.nsb = new_state->stride[0]; f.nsh = new_state->stride[1];
    f.nsr32 = (int)new_state->stride[2];
    f.out = out->data; f.odt = out->dtype; f.osb = out->stride[0]; f.osh = out->stride[1]; f.osd = out->stride[2];
    f.BH = B * H; f.H = (int)H; f.use_log = log_alpha != nullptr;
    const dim3 g4((unsigned)H, (unsigned)B);   // one workgroup per (b, h)
    const bool sbf = sdt == MABA_BF16, hs = state != nullptr, contig = f.ssr32 == 64 && f.nsr32 == 64;
    void (*kern)(StepFast) = nullptr;
#define MABA_STEP_PICK(T, TS)                                                                          \
  kern = hs ? (contig ? dgda_step_wave_kernel<T, TS, true, true> : dgda_step_wave_kernel<T, TS, true, false>) \
            : (contig ? dgda_step_wave_kernel<T, TS, false, true> : dgda_step_wave_kernel<T, TS, false, false>)
    if (q->dtype == MABA_BF16) { if (sbf) MABA_STEP_PICK(uint16_t, uint16_t); else MABA_STEP_PICK(uint16_t, float); }
    else { if (sbf) MABA_STEP_PICK(float, uint16_t); else MABA_STEP_PICK(float, float); }
#undef MABA_STEP_PICK
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

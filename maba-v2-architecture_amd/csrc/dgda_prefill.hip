// DGDA prefill (reference: maba_sparse/kernels/common.py:229-268 for the math,
// cpu_dgda.py:33-197 for the chunked form, dispatcher.py:258-327 for the op).
//
// Two implementations sit behind maba_hip_dgda_prefill:
//
//  * dgda_prefill_seq_kernel -- general path for any gate layout (per-channel
//    decay), dk, dv <= 128 and any float dtypes: one workgroup per (b, h), one
//    thread per state column holding S[:, c] in registers, tokens in sequence.
//    Correct everywhere; latency-bound (about one token per microsecond).
//
//  * the chunked MFMA path (dgda_chunk.hip) for the per-token (scalar) decay
//    case with dk = dv = 64 and bf16 q/k/v -- the BASELINE configuration;
//  * the sub-chunk path (dgda_sub.h, dgda_sub*.hip) for per-channel or per-token gates
//    (the DGDA layer's layout) with dk, dv in {32, 64, 128} and bf16, fp16 or fp32
//    q/k/v: 16-token sub-chunks with exact per-channel decay, the state products on
//    MFMA, sequence-parallel like the above.
#include <algorithm>

#include "maba_common.h"

namespace maba {

struct SeqArgs {
  View4 q, k, v, gate, b, w, s0;  // gate = log_alpha (use_log) or alpha
  MView4 out, sf;
  int H, L, dk, dv;
  int use_log, has_s0;
};

constexpr int SEQ_TT = 16;  // tokens staged per LDS refill

template <int DKMAX>
__global__ __launch_bounds__(128) void dgda_prefill_seq_kernel(SeqArgs a) {
  __shared__ float s_a[SEQ_TT][DKMAX], s_bk[SEQ_TT][DKMAX], s_k[SEQ_TT][DKMAX], s_q[SEQ_TT][DKMAX];
  __shared__ float s_wv[SEQ_TT][128];
  const int bh = blockIdx.x;
  const int bi = bh / a.H, hi = bh % a.H;
  const int c = threadIdx.x;
  const int dk = a.dk, dv = a.dv;
  const bool col_ok = c < dv;
  float S[DKMAX];
#pragma unroll
  for (int r = 0; r < DKMAX; ++r) S[r] = (col_ok && r < dk && a.has_s0) ? a.s0.at(bi, hi, r, c) : 0.f;

  for (int t0 = 0; t0 < a.L; t0 += SEQ_TT) {
    const int nt = (a.L - t0) < SEQ_TT ? (a.L - t0) : SEQ_TT;
    __syncthreads();
    for (int i = threadIdx.x; i < SEQ_TT * DKMAX; i += blockDim.x) {
      const int tt = i / DKMAX, r = i % DKMAX;
      float al = 1.f, bk = 0.f, kk = 0.f, qq = 0.f;
      if (tt < nt && r < dk) {
        const int t = t0 + tt;
        const float g = a.gate.at(bi, hi, t, r);
        al = a.use_log ? __expf(g) : g;
        kk = a.k.at(bi, hi, t, r);
        bk = a.b.at(bi, hi, t, r) * kk;
        qq = a.q.at(bi, hi, t, r);
      }
      s_a[tt][r] = al; s_bk[tt][r] = bk; s_k[tt][r] = kk; s_q[tt][r] = qq;
    }
    for (int i = threadIdx.x; i < SEQ_TT * 128; i += blockDim.x) {
      const int tt = i / 128, e = i % 128;
      s_wv[tt][e] = (tt < nt && e < dv) ? a.w.at(bi, hi, t0 + tt, e) * a.v.at(bi, hi, t0 + tt, e) : 0.f;
    }
    __syncthreads();
    for (int tt = 0; tt < nt; ++tt) {
      float pred = 0.f;
#pragma unroll
      for (int r = 0; r < DKMAX; ++r) {
        S[r] *= s_a[tt][r];
        pred = fmaf(s_bk[tt][r], S[r], pred);
      }
      const float delta = s_wv[tt][c < 128 ? c : 0] - pred;
      float o = 0.f;
#pragma unroll
      for (int r = 0; r < DKMAX; ++r) {
        S[r] = fmaf(s_k[tt][r], delta, S[r]);
        o = fmaf(s_q[tt][r], S[r], o);
      }
      if (col_ok) a.out.put(bi, hi, t0 + tt, c, o);
    }
  }
  if (col_ok) {
#pragma unroll
    for (int r = 0; r < DKMAX; ++r)
      if (r < dk) a.sf.put(bi, hi, r, c, S[r]);
  }
}

int launch_dgda_seq(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                    const maba_tensor* gate, int use_log, const maba_tensor* b,
                    const maba_tensor* w, const maba_tensor* s0, maba_tensor* out,
                    maba_tensor* sf, hipStream_t stream) {
  const int64_t B = q->shape[0], H = q->shape[1], L = q->shape[2], dk = q->shape[3], dv = v->shape[3];
  if (dk > 128 || dv > 128)
    return fail(MABA_ERR_UNSUPPORTED, "dgda_prefill: dk, dv <= 128 required, got %lld, %lld",
                (long long)dk, (long long)dv);
  SeqArgs a;
  a.q = view4(q); a.k = view4(k); a.v = view4(v); a.gate = view4(gate);
  a.b = view4(b); a.w = view4(w); a.s0 = view4(s0);
  a.out = mview4(out); a.sf = mview4(sf);
  a.H = (int)H; a.L = (int)L; a.dk = (int)dk; a.dv = (int)dv;
  a.use_log = use_log; a.has_s0 = s0 != nullptr;
  dim3 grid((unsigned)(B * H)), block(dv <= 64 ? 64 : 128);
  if (dk <= 32) hipLaunchKernelGGL(dgda_prefill_seq_kernel<32>, grid, block, 0, stream, a);
  else if (dk <= 64) hipLaunchKernelGGL(dgda_prefill_seq_kernel<64>, grid, block, 0, stream, a);
  else hipLaunchKernelGGL(dgda_prefill_seq_kernel<128>, grid, block, 0, stream, a);
  return check_launch("dgda_prefill(seq)");
}

// Chunked MFMA path (dgda_chunk.hip).
bool dgda_chunk_strides_fit(const maba_tensor* t);
bool dgda_chunk_supported(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                          const maba_tensor* gate, const maba_tensor* b);
size_t dgda_chunk_workspace(int64_t BH, int64_t L);
int launch_dgda_chunk(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                      const maba_tensor* gate, int use_log, const maba_tensor* b,
                      const maba_tensor* w, const maba_tensor* s0, maba_tensor* out,
                      maba_tensor* sf, void* ws, size_t ws_bytes, hipStream_t stream);
// Sub-chunk path for per-channel gates (dgda_sub.hip).
bool dgda_sub_supported(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                        const maba_tensor* gate, const maba_tensor* b, const maba_tensor* w,
                        const maba_tensor* out);
size_t dgda_sub_workspace(int64_t BH, int64_t L, int64_t dk, int64_t dv);
int launch_dgda_sub(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                    const maba_tensor* gate, int use_log, const maba_tensor* b,
                    const maba_tensor* w, const maba_tensor* s0, maba_tensor* out,
                    maba_tensor* sf, void* ws, size_t ws_bytes, hipStream_t stream);
}  // namespace maba

using namespace maba;

extern "C" size_t maba_hip_dgda_prefill_workspace_size(const maba_tensor* q, const maba_tensor* v,
                                                      const maba_tensor* gate, const maba_tensor* b) {
  if (!q || q->ndim != 4 || !v || v->ndim != 4 || !gate || !b) return 0;
  // The call picks its path from every operand (k, w and out included), which this query
  // does not see.  Both workspace sizes depend only on the shapes, so the larger of those
  // of the paths that q, v and the gates admit is returned: the call's choice always fits.
  const int64_t BH = q->shape[0] * q->shape[1], L = q->shape[2];
  size_t n = 0;
  if (dgda_chunk_supported(q, q, v, gate, b)) n = dgda_chunk_workspace(BH, L);
  if (dgda_sub_supported(q, q, v, gate, b, nullptr, nullptr))
    n = std::max(n, dgda_sub_workspace(BH, L, q->shape[3], v->shape[3]));
  return n;
}

extern "C" int maba_hip_dgda_prefill(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                                     const maba_tensor* alpha, const maba_tensor* log_alpha,
                                     const maba_tensor* b, const maba_tensor* w,
                                     const maba_tensor* initial_state, maba_tensor* out,
                                     maba_tensor* final_state, int chunk_size, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  (void)chunk_size;
  if (!q || q->ndim != 4) return fail(MABA_ERR_INVALID, "dgda_prefill: q must be [B,H,L,dk]");
  if (!v || v->ndim != 4) return fail(MABA_ERR_INVALID, "dgda_prefill: v must be [B,H,L,dv]");
  const int64_t B = q->shape[0], H = q->shape[1], L = q->shape[2], dk = q->shape[3], dv = v->shape[3];
  const int64_t sq[4] = {B, H, L, dk}, sv[4] = {B, H, L, dv}, ss[4] = {B, H, dk, dv};
  if (!expect_shape(k, "k", 4, sq) || !expect_shape(v, "v", 4, sv) || !expect_shape(b, "b", 4, sq) ||
      !expect_shape(w, "w", 4, sv) || !expect_shape(out, "out", 4, sv) ||
      !expect_shape(final_state, "final_state", 4, ss))
    return MABA_ERR_INVALID;
  if (!alpha && !log_alpha) return fail(MABA_ERR_INVALID, "dgda_prefill: alpha or log_alpha required");
  const maba_tensor* gate = log_alpha ? log_alpha : alpha;
  if (!expect_shape(gate, log_alpha ? "log_alpha" : "alpha", 4, sq)) return MABA_ERR_INVALID;
  if (initial_state && !expect_shape(initial_state, "initial_state", 4, ss)) return MABA_ERR_INVALID;
  const maba_tensor* all[] = {q, k, v, b, w, gate, out, final_state, initial_state};
  for (const maba_tensor* t : all)
    if (t && !expect_float(t, "dgda_prefill")) return MABA_ERR_DTYPE;
  if (dk < 1 || dv < 1) return fail(MABA_ERR_INVALID, "dgda_prefill: empty head dims");
  if (B * H == 0) return MABA_OK;
  hipStream_t s = (hipStream_t)stream;
  // the chunked kernels store 4 consecutive output channels per lane (8 or 16 bytes)
  const bool out_vec = out->stride[3] == 1 && (uintptr_t)out->data % 16 == 0 && out->stride[0] % 4 == 0 &&
                       out->stride[1] % 4 == 0 && out->stride[2] % 4 == 0;
  if (dgda_chunk_supported(q, k, v, gate, b) && w->dtype == MABA_F32 &&
      (out->dtype == MABA_BF16 || out->dtype == MABA_F32) && out_vec && dgda_chunk_strides_fit(w) &&
      dgda_chunk_strides_fit(out)) {
    const size_t need = dgda_chunk_workspace(B * H, L);
    if (!workspace || workspace_bytes < need)
      return fail(MABA_ERR_WORKSPACE, "dgda_prefill: workspace of %zu bytes required", need);
    return launch_dgda_chunk(q, k, v, gate, log_alpha != nullptr, b, w, initial_state, out, final_state,
                             workspace, workspace_bytes, s);
  }
  if (dgda_sub_supported(q, k, v, gate, b, w, out)) {
    const size_t need = dgda_sub_workspace(B * H, L, dk, dv);
    if (!workspace || workspace_bytes < need)
      return fail(MABA_ERR_WORKSPACE, "dgda_prefill: workspace of %zu bytes required", need);
    return launch_dgda_sub(q, k, v, gate, log_alpha != nullptr, b, w, initial_state, out, final_state,
                           workspace, workspace_bytes, s);
  }
  return launch_dgda_seq(q, k, v, gate, log_alpha != nullptr, b, w, initial_state, out, final_state, s);
}

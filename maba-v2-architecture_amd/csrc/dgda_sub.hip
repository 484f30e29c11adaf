// Host side of the sub-chunk DGDA prefill for per-channel gates (kernels and their math
// in dgda_sub.h): operand checks, workspace sizing, the d_v = 128 split, the kernels for
// d_k = 64 and the fused layer prologue entry point (maba_hip_dgda_layer_prefill).
#include "dgda_sub.h"

namespace maba {

// ------------------------------------------------------------------ host side

static bool al16s(const void* p) { return ((uintptr_t)p & 15) == 0; }
static bool fits32s(const maba_tensor* t) {
  for (int d = 0; d < t->ndim; ++d)
    if (t->stride[d] < 0 || t->stride[d] > INT32_MAX) return false;
  return true;
}
// gate with channel stride 0 (per token) or 1 (per channel, 16-byte aligned rows), fp32 or
// (16-bit q, k, v) in q's dtype
static bool sub_gate_ok(const maba_tensor* t, int gdt) {
  if (!t || t->dtype != gdt || !fits32s(t)) return false;
  if (t->stride[3] == 0) return true;
  if (t->stride[3] != 1 || !al16s(t->data)) return false;
  for (int d = 0; d < 3; ++d)
    if (t->shape[d] > 1 && t->stride[d] % 4 != 0) return false;
  return true;
}

static bool sub_head_size(int64_t d) { return d == 32 || d == 64 || d == 128; }
static bool sub_io_dtype(int dt) { return dt == MABA_BF16 || dt == MABA_F16 || dt == MABA_F32; }

bool dgda_sub_supported(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                        const maba_tensor* gate, const maba_tensor* b, const maba_tensor* w,
                        const maba_tensor* out) {
  if (!q || !k || !v || !gate || !b) return false;
  if (!sub_head_size(q->shape[3]) || !sub_head_size(v->shape[3])) return false;
  const int dt = q->dtype;
  if (!sub_io_dtype(dt) || k->dtype != dt || v->dtype != dt) return false;
  for (const maba_tensor* t : {q, k, v}) {   // 4-element (8- or 16-byte) loads
    if (t->stride[3] != 1 || !al16s(t->data) || !fits32s(t)) return false;
    for (int d = 0; d < 3; ++d)
      if (t->shape[d] > 1 && t->stride[d] % 4 != 0) return false;
  }
  // the three gates share one dtype: fp32, or q's 16-bit dtype
  const int gdt = gate->dtype;
  if (gdt != MABA_F32 && (gdt != dt || dt == MABA_F32)) return false;
  if (!sub_gate_ok(gate, gdt) || !sub_gate_ok(b, gdt)) return false;
  if (w && !sub_gate_ok(w, gdt)) return false;
  if (out && (out->stride[3] != 1 || !fits32s(out) || !sub_io_dtype(out->dtype))) return false;
  return q->shape[2] <= ((int64_t)1 << 30);
}

static SlotGeom sub_geom(int64_t BH, int64_t L) {
  const int64_t nch = ceil_div(L, SC) > 0 ? ceil_div(L, SC) : 1;
  return slot_geom(BH, nch, SUB_MIN_U);
}

// d_v = 128 runs as two d_v = 64 calls, one after the other on the stream, which share
// the workspace.
static int64_t sub_dv_call(int64_t dv) { return dv == 128 ? 64 : dv; }

size_t dgda_sub_workspace(int64_t BH, int64_t L, int64_t dk, int64_t dv) {
  const SlotGeom gm = sub_geom(BH, L);
  if (gm.nseg_max <= 1) return 16;
  const int64_t nseg = gm.nseg_max;
  return (size_t)(BH * nseg * dk * (sub_dv_call(dv) + dk)) * sizeof(float) + (size_t)(BH * nseg) * sizeof(int);
}

static int64_t esz(int dt) { return dt == MABA_F32 ? 4 : 2; }

int launch_dgda_sub(const maba_tensor* q, const maba_tensor* k, const maba_tensor* v,
                    const maba_tensor* gate, int use_log, const maba_tensor* b,
                    const maba_tensor* w, const maba_tensor* s0, maba_tensor* out,
                    maba_tensor* sf, void* ws, size_t ws_bytes, hipStream_t stream) {
  const int64_t B = q->shape[0], H = q->shape[1], L = q->shape[2], dk = q->shape[3], dv = v->shape[3];
  const int64_t BH = B * H;
  SubArgs a = {};
  // strides fit in int32 (dgda_sub_supported checks every operand)
  a.q = q->data; a.qs0 = (int)q->stride[0]; a.qs1 = (int)q->stride[1]; a.qs2 = (int)q->stride[2];
  a.k = k->data; a.ks0 = (int)k->stride[0]; a.ks1 = (int)k->stride[1]; a.ks2 = (int)k->stride[2];
  a.vp = v->data; a.vs0 = (int)v->stride[0]; a.vs1 = (int)v->stride[1]; a.vs2 = (int)v->stride[2];
  a.gp = gate->data; a.gs0 = (int)gate->stride[0]; a.gs1 = (int)gate->stride[1];
  a.gs2 = (int)gate->stride[2]; a.gs3 = (int)gate->stride[3];
  a.bp = b->data; a.bs0 = (int)b->stride[0]; a.bs1 = (int)b->stride[1];
  a.bs2 = (int)b->stride[2]; a.bs3 = (int)b->stride[3];
  a.wp = w->data; a.ws0 = (int)w->stride[0]; a.ws1 = (int)w->stride[1];
  a.ws2 = (int)w->stride[2]; a.ws3 = (int)w->stride[3];
  a.s0 = view4(s0);
  a.op = out->data; a.os0 = (int)out->stride[0]; a.os1 = (int)out->stride[1]; a.os2 = (int)out->stride[2];
  a.sf = mview4(sf);
  a.H = (int)H; a.L = (int)L; a.BH = (int)BH;
  a.nchunks = (int)(ceil_div(L, SC) > 0 ? ceil_div(L, SC) : 1);
  const SlotGeom gm = sub_geom(BH, L);
  a.U = gm.U;
  a.nseg_max = gm.nseg_max;
  a.use_log = use_log; a.has_s0 = s0 != nullptr;
  a.f16 = q->dtype == MABA_F16; a.of16 = out->dtype == MABA_F16;
  const size_t need = dgda_sub_workspace(BH, L, dk, dv);
  if (ws_bytes < need) return fail(MABA_ERR_WORKSPACE, "dgda_prefill: workspace too small");
  const int64_t nsegs = BH * a.nseg_max, dvc = sub_dv_call(dv);
  a.agg = (float*)ws;
  a.zc = (int*)(a.agg + nsegs * dk * (dvc + dk));
  const bool f32in = q->dtype == MABA_F32, g16 = gate->dtype != MABA_F32, o16 = out->dtype != MABA_F32;
  auto run = [&](SubArgs& x) {
    if (dk == 32) return run_sub_k32(x, (int)dvc, f32in, g16, o16, stream);
    if (dk == 64) return run_sub_k64(x, (int)dvc, f32in, g16, o16, stream);
    return run_sub_k128(x, (int)dvc, f32in, g16, o16, stream);
  };
  if (dv != 128) return run(a);
  // the two halves of the value columns: v, w, the output and the states start 64
  // columns further in the second call
  for (int half = 0; half < 2; ++half) {
    SubArgs h = a;
    const int64_t c = 64 * half;
    h.vp = (const char*)v->data + c * esz(v->dtype);
    h.wp = (const char*)w->data + c * w->stride[3] * esz(w->dtype);
    h.op = (char*)out->data + c * esz(out->dtype);
    if (s0) h.s0.p = (const char*)s0->data + c * s0->stride[3] * esz(s0->dtype);
    h.sf.p = (char*)sf->data + c * sf->stride[3] * esz(sf->dtype);
    const int rc = run(h);
    if (rc) return rc;
  }
  return MABA_OK;
}

int run_sub_k64(SubArgs& a, int dv, bool f32in, bool g16, bool obf, hipStream_t stream) {
  return dv == 32 ? run_sub_passes<false, 64, 32>(a, f32in, g16, obf, stream)
                  : run_sub_passes<false, 64, 64>(a, f32in, g16, obf, stream);
}

}  // namespace maba

using namespace maba;

extern "C" size_t maba_hip_dgda_layer_prefill_workspace_size(int64_t B, int64_t H, int64_t L) {
  return dgda_sub_workspace(B * H, L, 64, 64);
}

extern "C" int maba_hip_dgda_layer_prefill(const maba_tensor* const* xs, const maba_tensor* const* conv_w,
                                           const maba_tensor* const* hist, float eps,
                                           const maba_tensor* initial_state, maba_tensor* out,
                                           maba_tensor* final_state, maba_tensor* const* new_hist, void* workspace,
                                           size_t workspace_bytes, void* stream) {
  if (!xs || !conv_w || !new_hist || !out || !final_state)
    return fail(MABA_ERR_INVALID, "dgda_layer_prefill: null argument");
  for (int s = 0; s < 6; ++s)
    if (!xs[s] || xs[s]->ndim != 3) return fail(MABA_ERR_INVALID, "dgda_layer_prefill: projection %d must be [B,L,C]", s);
  const int64_t B = xs[0]->shape[0], L = xs[0]->shape[1], C = xs[0]->shape[2];
  if (C % 64 != 0 || C == 0) return fail(MABA_ERR_UNSUPPORTED, "dgda_layer_prefill: C must be 64 * H");
  if (L < 1) return fail(MABA_ERR_INVALID, "dgda_layer_prefill: at least one token");
  if (L > ((int64_t)1 << 30)) return fail(MABA_ERR_UNSUPPORTED, "dgda_layer_prefill: L too large");
  const int64_t H = C / 64, BH = B * H;
  for (int s = 0; s < 6; ++s) {
    const maba_tensor* t = xs[s];
    if (t->shape[0] != B || t->shape[1] != L || t->shape[2] != C || t->dtype != MABA_BF16 || t->stride[2] != 1 ||
        ((uintptr_t)t->data & 7) || t->stride[0] % 4 || t->stride[1] % 4 || !fits32s(t))
      return fail(MABA_ERR_UNSUPPORTED, "dgda_layer_prefill: projections must be bf16 [B,L,C], unit channel "
                  "stride, 8-byte aligned rows");
    // the kernels address a sequence's rows with 32-bit offsets
    if ((L + SC) * t->stride[1] + C > INT32_MAX)
      return fail(MABA_ERR_UNSUPPORTED, "dgda_layer_prefill: L * row stride must stay below 2^31 elements");
  }
  const int64_t sw[3] = {C, 1, 4}, sh[3] = {B, C, 3};
  for (int s = 0; s < 3; ++s) {
    if (!expect_shape(conv_w[s], "conv weight", 3, sw) || !expect_float(conv_w[s], "conv weight"))
      return MABA_ERR_INVALID;
    if (conv_w[s]->dtype != conv_w[0]->dtype) return fail(MABA_ERR_DTYPE, "dgda_layer_prefill: conv weights differ in dtype");
    if (!fits32s(conv_w[s])) return fail(MABA_ERR_UNSUPPORTED, "dgda_layer_prefill: conv weight strides");
    if (hist) {
      if (!expect_shape(hist[s], "conv history", 3, sh)) return MABA_ERR_INVALID;
      if (hist[s]->dtype != MABA_BF16 || !fits32s(hist[s]))
        return fail(MABA_ERR_DTYPE, "dgda_layer_prefill: the conv history must be bf16");
    }
    if (!expect_shape(new_hist[s], "new conv history", 3, sh) || !expect_float(new_hist[s], "new conv history"))
      return MABA_ERR_INVALID;
  }
  const int64_t so[4] = {B, H, L, 64}, ss[4] = {B, H, 64, 64};
  if (!expect_shape(out, "out", 4, so) || !expect_shape(final_state, "final_state", 4, ss)) return MABA_ERR_INVALID;
  if (out->stride[3] != 1 || !fits32s(out) || (out->dtype != MABA_BF16 && out->dtype != MABA_F32))
    return fail(MABA_ERR_UNSUPPORTED, "dgda_layer_prefill: out must be f32/bf16 with unit channel stride");
  if (!expect_float(final_state, "final_state")) return MABA_ERR_DTYPE;
  if (initial_state && (!expect_shape(initial_state, "initial_state", 4, ss) || !expect_float(initial_state, "initial_state")))
    return MABA_ERR_INVALID;
  const size_t need = dgda_sub_workspace(BH, L, 64, 64);
  if (!workspace || workspace_bytes < need)
    return fail(MABA_ERR_WORKSPACE, "dgda_layer_prefill: workspace of %zu bytes required", need);
  if (B == 0) return MABA_OK;
  SubArgs a = {};
  for (int s = 0; s < 6; ++s) {
    a.px[s] = (const uint16_t*)xs[s]->data; a.pxs0[s] = (int)xs[s]->stride[0]; a.pxs1[s] = (int)xs[s]->stride[1];
  }
  a.cwdt = conv_w[0]->dtype;
  for (int s = 0; s < 3; ++s) {
    a.cw[s] = conv_w[s]->data; a.cwsc[s] = (int)conv_w[s]->stride[0]; a.cwst[s] = (int)conv_w[s]->stride[2];
    a.ph[s] = hist ? (const uint16_t*)hist[s]->data : nullptr;
    a.phs0[s] = hist ? (int)hist[s]->stride[0] : 0; a.phs1[s] = hist ? (int)hist[s]->stride[1] : 0;
    a.phs2[s] = hist ? (int)hist[s]->stride[2] : 0;
  }
  a.eps = eps;
  a.s0 = view4(initial_state);
  a.op = out->data; a.os0 = (int)out->stride[0]; a.os1 = (int)out->stride[1]; a.os2 = (int)out->stride[2];
  a.sf = mview4(final_state);
  a.H = (int)H; a.L = (int)L; a.BH = (int)BH;
  a.nchunks = (int)ceil_div(L, SC);
  const SlotGeom gm = sub_geom(BH, L);
  a.U = gm.U;
  a.nseg_max = gm.nseg_max;
  a.use_log = 1; a.has_s0 = initial_state != nullptr;
  const int64_t nsegs = BH * a.nseg_max;
  a.agg = (float*)workspace;
  a.zc = (int*)(a.agg + nsegs * 64 * 128);
  hipStream_t st = (hipStream_t)stream;
  const int rc = run_sub_passes<true, 64, 64>(a, false, false, out->dtype == MABA_BF16, st);
  if (rc) return rc;
  // after the passes, which read the old history: the new one may overwrite it in place
  return launch_dgda_new_history(xs, hist, new_hist, st);
}
